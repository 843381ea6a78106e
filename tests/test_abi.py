"""The C ABI library loads, exports every symbol include/fused_attn_hip.h declares, and
rejects invalid requests with status codes before touching a GPU.  CPU only: no call
here reaches a kernel launch."""
import ctypes
import os
import re

import pytest
import torch

from fused_attn import _hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fused_attn_hip.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fa_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_hip.library_path()):
        pytest.fail(f"{_hip.library_path()} is not built; run __graft_entry__.build()")
    return _hip.load_library()


def test_library_exports_every_declared_symbol(lib):
    names = _declared_functions()
    assert len(names) >= 8
    for name in names:
        assert hasattr(lib, name), name


def test_struct_layout_matches_header(lib):
    # fa_fwd_params: 4 pointers, 12 int64 strides, 6 int32 sizes, float, 3 int32,
    # 2 pointers, 2 int32, pointer + 2 int64, 2 pointers + 2 int64
    assert ctypes.sizeof(_hip.FwdParams) == 4 * 8 + 12 * 8 + 6 * 4 + 4 + 3 * 4 + 2 * 8 + 2 * 4 + 8 + 16 + 16 + 16
    assert _hip.FwdParams.cu_seqlens_q.offset % 8 == 0 and _hip.FwdParams.lse.offset % 8 == 0


def test_abi_version(lib):
    assert lib.fa_abi_version() == _hip.ABI_VERSION == 6


def test_choose_num_splits_known_answers(lib):
    assert lib.fa_choose_num_splits(1, 8, 32768, 1, 108) == 27
    assert lib.fa_choose_num_splits(64, 32, 32768, 1, 108) == 1
    assert lib.fa_choose_num_splits(1, 1, 512, 1, 108) == 2
    assert lib.fa_choose_num_splits(1, 1, 100000, 128, 108) == 1


def test_workspace_bytes(lib):
    # fp32 partials plus fp32 (max, sum) pairs per (row, partition)
    assert lib.fa_splitk_workspace_bytes(32, 32, 1, 128, 256) == 32 * 32 * 256 * (128 * 4 + 8)
    assert lib.fa_splitk_workspace_bytes(0, 32, 1, 128, 256) == 0


def _params(**over):
    p = _hip.FwdParams()
    # a plausible, aligned dense request; pointers are fake and never dereferenced
    p.q = p.k = p.v = p.o = 0x10000
    p.batch, p.heads_q, p.heads_kv, p.seqlen_q, p.seqlen_k, p.head_dim = 1, 4, 2, 16, 16, 64
    p.q_stride_b, p.q_stride_h, p.q_stride_n = 4 * 16 * 64, 16 * 64, 64
    p.k_stride_b, p.k_stride_h, p.k_stride_n = 2 * 16 * 64, 16 * 64, 64
    p.v_stride_b, p.v_stride_h, p.v_stride_n = 2 * 16 * 64, 16 * 64, 64
    p.o_stride_b, p.o_stride_h, p.o_stride_n = 4 * 16 * 64, 16 * 64, 64
    p.scale, p.dtype, p.kv_dtype = 0.125, _hip.BF16, _hip.BF16
    for k, v in over.items():
        setattr(p, k, v)
    return p


@pytest.mark.parametrize("over,code,msg", [
    (dict(head_dim=96), _hip.FA_ERR_UNSUPPORTED, "head_dim"),
    (dict(head_dim=48), _hip.FA_ERR_UNSUPPORTED, "head_dim"),
    (dict(dtype=_hip.F32, kv_dtype=_hip.F16), _hip.FA_ERR_INVALID_ARGUMENT, "k/v dtype"),
    (dict(heads_q=3), _hip.FA_ERR_INVALID_ARGUMENT, "multiple"),
    (dict(heads_kv=0), _hip.FA_ERR_INVALID_ARGUMENT, "non-negative"),
    (dict(kv_dtype=_hip.F16), _hip.FA_ERR_INVALID_ARGUMENT, "k/v dtype"),
    (dict(kv_dtype=_hip.FP8_E4M3), _hip.FA_ERR_INVALID_ARGUMENT, "k/v dtype"),
    (dict(q=0x10002), _hip.FA_ERR_INVALID_ARGUMENT, "aligned"),
    (dict(k_stride_n=60), _hip.FA_ERR_INVALID_ARGUMENT, "k/v strides"),
    (dict(q_stride_h=1020), _hip.FA_ERR_INVALID_ARGUMENT, "q strides"),
    (dict(o_stride_n=62), _hip.FA_ERR_INVALID_ARGUMENT, "o strides"),
    (dict(v=0), _hip.FA_ERR_INVALID_ARGUMENT, "non-NULL"),
    (dict(dtype=9), _hip.FA_ERR_INVALID_ARGUMENT, "unknown dtype"),
    (dict(scale=float("nan")), _hip.FA_ERR_INVALID_ARGUMENT, "NaN"),
    (dict(k_stride_n=1 << 24), _hip.FA_ERR_UNSUPPORTED, "token stride"),
    # 128-key tiles: 127 rows of a 16 MiB stride would overflow a signed 32-bit byte offset
    (dict(v_stride_n=1 << 23), _hip.FA_ERR_UNSUPPORTED, "token stride"),
])
def test_fwd_validation(lib, over, code, msg):
    p = _params(**over)
    assert lib.fa_attention_fwd(ctypes.byref(p), None) == code
    assert msg in lib.fa_last_error().decode()


def test_null_params(lib):
    assert lib.fa_attention_fwd(None, None) == _hip.FA_ERR_INVALID_ARGUMENT
    assert lib.fa_attention_varlen_fwd(None, None) == _hip.FA_ERR_INVALID_ARGUMENT
    assert lib.fa_attention_splitk(None, 128, None, 0, None) == _hip.FA_ERR_INVALID_ARGUMENT


def test_last_error_is_per_thread(lib):
    """fa_last_error() is thread-local: two threads that fail differently, in interleaved order, each
    read their own message (ctypes releases the GIL around the calls)."""
    import threading

    start = threading.Barrier(2)
    failed = threading.Barrier(2)
    seen = {}

    def worker(name, over, msg):
        p = _params(**over)
        start.wait()
        rc = lib.fa_attention_fwd(ctypes.byref(p), None)
        failed.wait()  # both threads have failed before either reads its message
        seen[name] = (rc, lib.fa_last_error().decode(), msg)

    threads = [threading.Thread(target=worker, args=("a", dict(head_dim=96), "head_dim")),
               threading.Thread(target=worker, args=("b", dict(q=0x10002), "aligned"))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    for name, (rc, text, msg) in seen.items():
        assert rc != _hip.FA_OK and msg in text, (name, text)


def test_empty_requests_succeed_without_launch(lib):
    assert lib.fa_attention_fwd(ctypes.byref(_params(batch=0)), None) == _hip.FA_OK
    assert lib.fa_attention_fwd(ctypes.byref(_params(seqlen_q=0)), None) == _hip.FA_OK
    assert lib.fa_last_error().decode() == ""


def test_varlen_validation(lib):
    p = _params()
    assert lib.fa_attention_varlen_fwd(ctypes.byref(p), None) == _hip.FA_ERR_INVALID_ARGUMENT
    assert "cu_seqlens" in lib.fa_last_error().decode()
    p = _params(cu_seqlens_q=0x20000, cu_seqlens_k=0x20000, max_seqlen_q=-1)
    assert lib.fa_attention_varlen_fwd(ctypes.byref(p), None) == _hip.FA_ERR_INVALID_ARGUMENT
    # LSE is accepted on the varlen path ([Hq, total_q]); a negative head stride is rejected
    p = _params(cu_seqlens_q=0x20000, cu_seqlens_k=0x20000, max_seqlen_q=8, max_seqlen_k=8, lse=0x30000,
                lse_stride_h=-1)
    assert lib.fa_attention_varlen_fwd(ctypes.byref(p), None) == _hip.FA_ERR_INVALID_ARGUMENT
    assert "LSE" in lib.fa_last_error().decode()


def test_splitk_validation(lib):
    p = _params()
    assert lib.fa_attention_splitk(ctypes.byref(p), 100, None, 0, None) == _hip.FA_ERR_INVALID_ARGUMENT
    assert "multiple of 64" in lib.fa_last_error().decode()
    assert lib.fa_attention_splitk(ctypes.byref(p), 0, None, 0, None) == _hip.FA_ERR_INVALID_ARGUMENT
    assert lib.fa_attention_splitk(ctypes.byref(p), 64, None, 0, None) == _hip.FA_ERR_WORKSPACE
    need = lib.fa_splitk_workspace_bytes(1, 4, 16, 64, 1)
    assert lib.fa_attention_splitk(ctypes.byref(p), 64, ctypes.c_void_p(0x40000), need - 4,
                                   None) == _hip.FA_ERR_WORKSPACE
    assert "need %d" % need in lib.fa_last_error().decode()
    assert lib.fa_attention_splitk(ctypes.byref(p), 64, ctypes.c_void_p(0x40004), need,
                                   None) == _hip.FA_ERR_WORKSPACE  # misaligned
    fp8 = _params(kv_dtype=_hip.FP8_E4M3, k_stride_n=64)
    assert lib.fa_attention_splitk(ctypes.byref(fp8), 64, ctypes.c_void_p(0x40000), need,
                                   None) == _hip.FA_ERR_INVALID_ARGUMENT
    assert "scale" in lib.fa_last_error().decode()
    fp8 = _params(kv_dtype=_hip.FP8_E4M3, k_stride_n=72, k_scale=0x50000, v_scale=0x50000)
    assert lib.fa_attention_splitk(ctypes.byref(fp8), 64, ctypes.c_void_p(0x40000), need,
                                   None) == _hip.FA_ERR_INVALID_ARGUMENT  # fp8 rows need 16-byte strides
    # the combine writes the optional LSE; a negative stride is rejected before launch
    p = _params(lse=0x30000, lse_stride_b=-1)
    assert lib.fa_attention_splitk(ctypes.byref(p), 64, ctypes.c_void_p(0x40000), need, None) == \
        _hip.FA_ERR_INVALID_ARGUMENT
    assert "LSE" in lib.fa_last_error().decode()
    # split-K keeps the MFMA shapes: fp32 and other head dims go to the prefill entry point
    p = _params(dtype=_hip.F32, kv_dtype=_hip.F32)
    assert lib.fa_attention_splitk(ctypes.byref(p), 64, ctypes.c_void_p(0x40000), need, None) == _hip.FA_ERR_UNSUPPORTED
    assert "dtype" in lib.fa_last_error().decode()
    p = _params(head_dim=32, q_stride_b=4 * 16 * 32, q_stride_h=16 * 32, q_stride_n=32)
    assert lib.fa_attention_splitk(ctypes.byref(p), 64, ctypes.c_void_p(0x40000), need, None) == _hip.FA_ERR_UNSUPPORTED
    assert "head_dim" in lib.fa_last_error().decode()


def test_make_params_marshals_strides():
    q = torch.empty(2, 64, 8, 128, dtype=torch.bfloat16).transpose(1, 2)  # [B,H,N,D] view of [B,N,H,D]
    k = torch.empty(2, 2, 64, 128, dtype=torch.bfloat16)
    o = torch.empty_like(q)
    p = _hip.make_params(q, k, k, o, True, 0.5)
    assert (p.q_stride_b, p.q_stride_h, p.q_stride_n) == (64 * 8 * 128, 128, 8 * 128)
    assert (p.k_stride_b, p.k_stride_h, p.k_stride_n) == (2 * 64 * 128, 64 * 128, 128)
    assert (p.o_stride_b, p.o_stride_h, p.o_stride_n) == q.stride()[:3]
    assert (p.batch, p.heads_q, p.heads_kv, p.seqlen_q, p.seqlen_k, p.head_dim) == (2, 8, 2, 64, 64, 128)
    assert p.causal == 1 and p.dtype == p.kv_dtype == _hip.BF16 and abs(p.scale - 0.5) < 1e-7
    assert p.lse is None and p.k_scale is None and p.v_scale is None and p.cu_seqlens_q is None
    # decode shape: size-1 dims are never stepped over and pass stride 0 (q's query dim, a K/V batch
    # of one broadcast over q's batch)
    qd = torch.empty(3, 8, 1, 64, dtype=torch.float16)
    kd = torch.empty(1, 2, 500, 64, dtype=torch.float16)
    od = torch.empty_like(qd)
    p = _hip.make_params(qd, kd, kd, od, False, 0.125)
    assert (p.q_stride_b, p.q_stride_h, p.q_stride_n) == (8 * 64, 64, 0)
    assert (p.k_stride_b, p.k_stride_h, p.k_stride_n) == (0, 500 * 64, 64)
    assert (p.batch, p.heads_q, p.heads_kv, p.seqlen_q, p.seqlen_k, p.head_dim) == (3, 8, 2, 1, 500, 64)
    assert p.causal == 0 and p.dtype == p.kv_dtype == _hip.F16 and p.max_seqlen_q == 0
    # varlen: token stride is dim 0, batch strides unused
    qv = torch.empty(100, 8, 64, dtype=torch.float16)
    kv = torch.empty(90, 2, 64, dtype=torch.float16)
    cu = torch.tensor([0, 40, 100], dtype=torch.int32)
    p = _hip.make_params(qv, kv, kv, qv, False, 1.0, cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=60,
                         max_seqlen_k=50)
    assert (p.q_stride_b, p.q_stride_h, p.q_stride_n) == (0, 64, 8 * 64)
    assert p.batch == 2 and p.max_seqlen_q == 60 and p.seqlen_k == 50 and p.dtype == _hip.F16


def test_aligned_view_copies_only_when_needed():
    t = torch.empty(2, 4, 16, 64, dtype=torch.bfloat16)
    assert _hip._aligned_view(t, 8, 16) is t
    odd = torch.randn(4 * 16 * 64 + 1).bfloat16()[1:].view(1, 4, 16, 64)
    c = _hip._aligned_view(odd, 8, 16)
    assert c is not odd and c.data_ptr() % 16 == 0 and torch.equal(c, odd)
    strided = torch.empty(1, 4, 16, 70, dtype=torch.bfloat16)[..., :64]
    assert _hip._aligned_view(strided, 8, 16).is_contiguous()


# ---- fa_quantize_kv_fp8 -----------------------------------------------------------------------


def _qparams(**over):
    p = _hip.QuantParams()
    # a plausible aligned request; pointers are fake, and every case below is rejected (or empty)
    # before a launch
    p.x, p.x8, p.scale = 0x10000, 0x20000, 0x30000
    p.batch, p.heads, p.seqlen, p.head_dim = 2, 4, 100, 64
    p.x_stride_b, p.x_stride_h, p.x_stride_n = 4 * 100 * 64, 100 * 64, 64
    p.dtype = _hip.BF16
    for k, v in over.items():
        setattr(p, k, v)
    return p


def test_quant_struct_layout(lib):
    # pointer, 3 int64 strides, 5 int32 (+4 padding), 2 pointers
    assert ctypes.sizeof(_hip.QuantParams) == 8 + 3 * 8 + 5 * 4 + 4 + 2 * 8
    assert _hip.QuantParams.x8.offset == 56


@pytest.mark.parametrize("over,code,msg", [
    (dict(head_dim=48), _hip.FA_ERR_UNSUPPORTED, "head_dim"),
    (dict(head_dim=512), _hip.FA_ERR_UNSUPPORTED, "head_dim"),
    (dict(dtype=_hip.FP8_E4M3), _hip.FA_ERR_UNSUPPORTED, "float32"),
    (dict(dtype=7), _hip.FA_ERR_UNSUPPORTED, "float32"),
    (dict(batch=-1), _hip.FA_ERR_INVALID_ARGUMENT, "non-negative"),
    (dict(seqlen=-5), _hip.FA_ERR_INVALID_ARGUMENT, "non-negative"),
    (dict(x=0), _hip.FA_ERR_INVALID_ARGUMENT, "non-NULL"),
    (dict(scale=0), _hip.FA_ERR_INVALID_ARGUMENT, "non-NULL"),
    (dict(x_stride_n=-64), _hip.FA_ERR_INVALID_ARGUMENT, "negative"),
    (dict(x_stride_n=68), _hip.FA_ERR_INVALID_ARGUMENT, "16 bytes"),
    (dict(x_stride_h=100 * 64 + 4), _hip.FA_ERR_INVALID_ARGUMENT, "16 bytes"),
    (dict(x=0x10008), _hip.FA_ERR_INVALID_ARGUMENT, "aligned"),
    (dict(x8=0x20008), _hip.FA_ERR_INVALID_ARGUMENT, "aligned"),
    (dict(scale=0x30002), _hip.FA_ERR_INVALID_ARGUMENT, "aligned"),
])
def test_quant_validation(lib, over, code, msg):
    p = _qparams(**over)
    assert lib.fa_quantize_kv_fp8(ctypes.byref(p), None) == code
    assert msg in lib.fa_last_error().decode()


def test_quant_fp32_rows_need_four_element_strides(lib):
    # fp32 vectors are 4 elements: a stride of 68 floats is 16-byte aligned, 66 is not
    assert lib.fa_quantize_kv_fp8(ctypes.byref(_qparams(dtype=_hip.F32, x_stride_n=66)), None) \
        == _hip.FA_ERR_INVALID_ARGUMENT
    assert lib.fa_quantize_kv_fp8(None, None) == _hip.FA_ERR_INVALID_ARGUMENT


def test_quant_empty_requests_succeed_without_launch(lib):
    for over in (dict(batch=0), dict(heads=0), dict(seqlen=0), dict(seqlen=0, x=0, x8=0, scale=0)):
        assert lib.fa_quantize_kv_fp8(ctypes.byref(_qparams(**over)), None) == _hip.FA_OK
        assert lib.fa_last_error().decode() == ""


# ---- fa_attention_paged_decode ------------------------------------------------------------------


def _paged(**over):
    kv = _hip.PagedKV()
    kv.block_table, kv.block_table_stride, kv.block_table_cols = 0x60000, 4, 4
    kv.page_size, kv.num_pages, kv.seqlens_k = 64, 16, 0x70000
    kv.k_page_stride = kv.v_page_stride = 2 * 64 * 64
    for k, v in over.items():
        setattr(kv, k, v)
    return kv


def _paged_call(lib, p=None, kv=None, split_len=128, ws=0x40000, ws_bytes=1 << 30):
    p = _params(seqlen_q=1, seqlen_k=200) if p is None else p
    kv = _paged() if kv is None else kv
    return lib.fa_attention_paged_decode(ctypes.byref(p), ctypes.byref(kv), split_len, ctypes.c_void_p(ws), ws_bytes,
                                         None)


def test_paged_struct_layout(lib):
    assert ctypes.sizeof(_hip.PagedKV) == 8 + 8 + 4 + 4 + 8 + 4 + 4 + 8 + 8
    assert _hip.PagedKV.k_page_stride.offset == 40


@pytest.mark.parametrize("kv_over,p_over,split,code,msg", [
    (dict(page_size=40), {}, 128, _hip.FA_ERR_INVALID_ARGUMENT, "multiple of 16"),
    (dict(page_size=0), {}, 128, _hip.FA_ERR_INVALID_ARGUMENT, "multiple of 16"),
    # beyond FA_MAX_PAGE_SIZE (2^24 keys): rejected before the page-slot magic number is derived
    (dict(page_size=(1 << 24) + 16), {}, 128, _hip.FA_ERR_INVALID_ARGUMENT, "at most 2^24"),
    (dict(page_size=(1 << 31) - 16), {}, 128, _hip.FA_ERR_INVALID_ARGUMENT, "at most 2^24"),
    (dict(num_pages=-1), {}, 128, _hip.FA_ERR_INVALID_ARGUMENT, "negative"),
    (dict(block_table_cols=3), {}, 128, _hip.FA_ERR_INVALID_ARGUMENT, "fewer pages"),
    (dict(block_table=0), {}, 128, _hip.FA_ERR_INVALID_ARGUMENT, "non-NULL"),
    (dict(seqlens_k=0), {}, 128, _hip.FA_ERR_INVALID_ARGUMENT, "non-NULL"),
    (dict(seqlens_k=0x70002), {}, 128, _hip.FA_ERR_INVALID_ARGUMENT, "aligned"),
    (dict(block_table_stride=2), dict(batch=2), 128, _hip.FA_ERR_INVALID_ARGUMENT, "overlap"),
    (dict(k_page_stride=2 * 64 * 64 + 4), {}, 128, _hip.FA_ERR_INVALID_ARGUMENT, "page strides"),
    (dict(v_page_stride=-8), {}, 128, _hip.FA_ERR_INVALID_ARGUMENT, "page strides"),
    ({}, {}, 100, _hip.FA_ERR_INVALID_ARGUMENT, "split_len"),
    # FP8 pools: 64-key scale blocks must not straddle pages; scales are required and their strides checked
    (dict(page_size=32), dict(kv_dtype=_hip.FP8_E4M3, k_scale=0x50000, v_scale=0x50000), 128,
     _hip.FA_ERR_INVALID_ARGUMENT, "multiple of 64"),
    ({}, dict(kv_dtype=_hip.FP8_E4M3), 128, _hip.FA_ERR_INVALID_ARGUMENT, "k_scale"),
    ({}, dict(kv_dtype=_hip.FP8_E4M3, k_scale=0x50000, v_scale=0x50000, scale_stride_b=-1), 128,
     _hip.FA_ERR_INVALID_ARGUMENT, "scale stride"),
    ({}, dict(lse=0x30000, lse_stride_h=-1), 128, _hip.FA_ERR_INVALID_ARGUMENT, "LSE"),
    ({}, dict(dtype=_hip.F32, kv_dtype=_hip.F32), 128, _hip.FA_ERR_UNSUPPORTED, "dtype"),
    ({}, dict(head_dim=32, q_stride_b=4 * 16 * 32, q_stride_h=16 * 32, q_stride_n=32), 128, _hip.FA_ERR_UNSUPPORTED,
     "head_dim"),
])
def test_paged_validation(lib, kv_over, p_over, split, code, msg):
    p = _params(seqlen_q=1, seqlen_k=200, **p_over)
    assert _paged_call(lib, p=p, kv=_paged(**kv_over), split_len=split) == code
    assert msg in lib.fa_last_error().decode()


def test_paged_workspace_and_null_params(lib):
    assert lib.fa_attention_paged_decode(None, ctypes.byref(_paged()), 128, None, 0, None) == _hip.FA_ERR_INVALID_ARGUMENT
    p = _params(seqlen_q=1, seqlen_k=200)
    assert lib.fa_attention_paged_decode(ctypes.byref(p), None, 128, None, 0, None) == _hip.FA_ERR_INVALID_ARGUMENT
    need = lib.fa_splitk_workspace_bytes(1, 4, 1, 64, 2)
    assert _paged_call(lib, ws_bytes=need - 4) == _hip.FA_ERR_WORKSPACE
    assert _paged_call(lib, ws=0x40004, ws_bytes=need) == _hip.FA_ERR_WORKSPACE
    # k_stride_b is ignored (keys come through the block table): a stride that the dense path
    # rejects does not matter here, so this request fails on the workspace only
    p = _params(seqlen_q=1, seqlen_k=200, k_stride_b=3)
    assert _paged_call(lib, p=p, ws_bytes=need - 4) == _hip.FA_ERR_WORKSPACE


def test_paged_split_spanning_too_many_pages_is_rejected(lib):
    # 32-key pages and 8256-key partitions: up to (8256 - 1) // 32 + 2 = 259 pages per workgroup
    p = _params(seqlen_q=1, seqlen_k=9000)
    kv = _paged(page_size=32, block_table_cols=282, block_table_stride=282, k_page_stride=2 * 32 * 64,
                v_page_stride=2 * 32 * 64)
    assert _paged_call(lib, p=p, kv=kv, split_len=8256) == _hip.FA_ERR_UNSUPPORTED
    assert "256 pages" in lib.fa_last_error().decode()


def test_paged_empty_requests_succeed_without_launch(lib):
    assert _paged_call(lib, p=_params(batch=0, seqlen_q=1, seqlen_k=200)) == _hip.FA_OK
    assert _paged_call(lib, p=_params(seqlen_q=0, seqlen_k=200)) == _hip.FA_OK


def test_views_with_token_strides_past_the_abi_bound_are_copied():
    """The C ABI rejects K/V token strides of 16 MiB or more; the Python layer hands such views to
    the kernels as contiguous copies instead, so callers never see that bound."""
    base = torch.zeros(2 * (1 << 23), dtype=torch.bfloat16)  # 32 MiB
    at_bound = base.as_strided((1, 1, 2, 64), (0, 0, 1 << 23, 1))  # [B, H, N, D], 16 MiB token stride
    below = base.as_strided((1, 1, 2, 64), (0, 0, (1 << 23) - 8, 1))
    packed = base.as_strided((2, 1, 64), (1 << 23, 0, 1))  # [T, H, D]
    for view in (at_bound, packed):
        out = _hip._aligned_view(view, 8, 16)
        assert out.data_ptr() != view.data_ptr() and out.is_contiguous() and torch.equal(out, view)
    assert _hip._aligned_view(below, 8, 16) is below
