"""The op stays a torch.library custom op with its fake kernel (reference: tests/test_torch_compile.py),
and the dispatch rules mirror the reference's (fused_attn/ops.py:56-73).  CPU only."""
import pytest
import torch

import fused_attn
from fused_attn import ops
from oracle import attention_oracle as orc


def test_fake_tensor_shape():
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        q = torch.empty(2, 8, 128, 64, dtype=torch.float16)
        k = torch.empty(2, 2, 128, 64, dtype=torch.float16)
        out = fused_attn.attention(q, k, k, causal=True)
    assert out.shape == (2, 8, 128, 64) and out.dtype == torch.float16


def test_opcheck():
    q, k, v = (torch.randn(1, 2, 16, 32) for _ in range(3))
    torch.library.opcheck(fused_attn.attention, (q, k, v, True, None))


def test_op_schema_matches_reference():
    schema = str(torch.ops.fused_attn.attention.default._schema)
    assert schema == ("fused_attn::attention(Tensor q, Tensor k, Tensor v, bool causal=False, "
                      "float? scale=None) -> Tensor")


def test_varlen_is_a_custom_op_with_fake():
    from torch._subclasses.fake_tensor import FakeTensorMode

    schema = str(torch.ops.fused_attn.attention_varlen.default._schema)
    assert schema == ("fused_attn::attention_varlen(Tensor q, Tensor k, Tensor v, Tensor cu_seqlens_q, "
                      "Tensor cu_seqlens_k, SymInt max_seqlen_q, SymInt max_seqlen_k, bool causal=False, "
                      "float? scale=None) -> Tensor")
    cu = torch.tensor([0, 3, 3, 10], dtype=torch.int32)
    with FakeTensorMode(allow_non_fake_inputs=True):
        q = torch.empty(10, 4, 32, dtype=torch.bfloat16)
        k = torch.empty(10, 2, 32, dtype=torch.bfloat16)
        out = fused_attn.attention_varlen(q, k, k, cu, cu, 7, 7, True)
    assert out.shape == (10, 4, 32) and out.dtype == torch.bfloat16
    q, k, v = torch.randn(10, 4, 32), torch.randn(10, 2, 32), torch.randn(10, 2, 32)
    torch.library.opcheck(fused_attn.attention_varlen, (q, k, v, cu, cu, 7, 7, True, None))


def test_torch_compile_no_graph_break():
    torch._dynamo.reset()

    def f(q, k, v):
        return fused_attn.attention(q, k, v, causal=True) * 2.0

    q, k, v = (torch.randn(1, 2, 16, 32) for _ in range(3))
    try:
        out = torch.compile(f, fullgraph=True)(q, k, v)
    except Exception as e:  # pragma: no cover - no C compiler for inductor on some images
        if "compiler" in str(e).lower() or "inductor" in str(e).lower():
            pytest.skip(f"inductor unavailable: {e}")
        raise
    torch.testing.assert_close(out, f(q, k, v), atol=1e-5, rtol=1e-5)


def test_cpu_tensors_use_reference_backend():
    q = torch.randn(1, 8, 1, 64)
    k = torch.randn(1, 2, 4096, 64)
    assert ops._pick_backend(q, k) == "reference"
    assert ops.is_decode_shaped(q, k)
    assert not ops.is_decode_shaped(torch.randn(1, 8, 17, 64), k)
    assert not ops.is_decode_shaped(q, torch.randn(1, 2, 2047, 64))
    assert "reference" in fused_attn.available_backends()


def test_backend_env_override(monkeypatch):
    q = torch.randn(1, 2, 4, 16)
    monkeypatch.setenv("FUSED_ATTN_BACKEND", "reference")
    assert ops._pick_backend(q) == "reference"
    for name in ("hip", "cuda_mma", "cuda", "triton", "splitk"):
        monkeypatch.setenv("FUSED_ATTN_BACKEND", name)
        assert ops._pick_backend(q) == "hip"
    monkeypatch.setenv("FUSED_ATTN_BACKEND", "bogus")
    with pytest.raises(ValueError):
        ops._pick_backend(q)


def test_hip_backend_on_cpu_tensors_fails_loudly(monkeypatch):
    monkeypatch.setenv("FUSED_ATTN_BACKEND", "hip")
    q = torch.randn(1, 2, 4, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError):
        fused_attn.attention(q, q, q)


def test_reference_backend_matches_oracle():
    torch.manual_seed(0)
    q, k, v = torch.randn(2, 8, 50, 64), torch.randn(2, 2, 70, 64), torch.randn(2, 2, 70, 64)
    for causal in (False, True):
        torch.testing.assert_close(fused_attn.attention(q, k, v, causal=causal),
                                   orc.attention(q, k, v, causal=causal), atol=1e-5, rtol=1e-5)
        torch.testing.assert_close(fused_attn.attention_reference(q, k, v, causal=causal, scale=0.2),
                                   orc.attention(q, k, v, causal=causal, scale=0.2), atol=1e-5, rtol=1e-5)
    qb = q.bfloat16()
    assert fused_attn.attention(qb, k.bfloat16(), v.bfloat16()).dtype == torch.bfloat16


@pytest.mark.parametrize("lens", [[5, 33, 70], [1, 1, 1], [128], [64, 0, 17]])
@pytest.mark.parametrize("causal", [False, True])
def test_varlen_reference_backend(lens, causal):
    torch.manual_seed(0)
    q, cu_q, max_q = fused_attn.pack_varlen([torch.randn(n, 8, 64) for n in lens])
    k, cu_k, max_k = fused_attn.pack_varlen([torch.randn(n, 2, 64) for n in lens])
    v, _, _ = fused_attn.pack_varlen([torch.randn(n, 2, 64) for n in lens])
    assert cu_q.dtype == torch.int32 and cu_q[0] == 0 and cu_q[-1] == sum(lens) and max_q == max(lens)
    out = fused_attn.attention_varlen(q, k, v, cu_q, cu_k, max_q, max_k, causal=causal)
    torch.testing.assert_close(out, orc.attention_varlen(q, k, v, cu_q, cu_k, causal=causal), atol=1e-5,
                               rtol=1e-5)


def test_package_fp8_quantiser_is_bit_identical_to_oracle():
    # CPU tensors take the torch chain, whose amax / 448.0 is a true division on the CPU
    torch.manual_seed(0)
    x = torch.randn(2, 3, 200, 64) * 2
    a8, as_ = fused_attn.quantize_kv_fp8(x)
    b8, bs = orc.quantize_kv_fp8(x, scale_div="true")
    assert torch.equal(a8.view(torch.uint8), b8.view(torch.uint8)) and torch.equal(as_, bs)
    torch.testing.assert_close(fused_attn.dequantize_kv_fp8(a8, as_), orc.dequantize_kv_fp8(b8, bs), atol=0, rtol=0)


def test_fp8_and_splitk_cpu_paths():
    torch.manual_seed(0)
    q = torch.randn(2, 4, 8, 64)
    k, v = torch.randn(2, 2, 300, 64), torch.randn(2, 2, 300, 64)
    k8, ks = fused_attn.quantize_kv_fp8(k)
    v8, vs = fused_attn.quantize_kv_fp8(v)
    out = fused_attn.attention_fp8(q.bfloat16(), k8, ks, v8, vs, causal=True)
    ref = orc.attention_fp8(q.bfloat16(), k8, ks, v8, vs, causal=True)
    assert out.dtype == torch.bfloat16 and (out.float() - ref).abs().max() < 1e-2
    torch.testing.assert_close(fused_attn.attention_splitk(q, k, v, causal=True, num_splits=3),
                               orc.attention(q, k, v, causal=True), atol=1e-5, rtol=1e-5)


def test_choose_num_splits_known_answers():
    # reference: tests/test_splitk_fp8.py:44-50
    assert fused_attn.choose_num_splits(1, 8, 32768, 1, num_sms=108) == 27
    assert fused_attn.choose_num_splits(64, 32, 32768, 1, num_sms=108) == 1
    assert fused_attn.choose_num_splits(1, 1, 512, 1, num_sms=108) == 2
    assert fused_attn.choose_num_splits(1, 1, 100000, 128, num_sms=108) == 1


def test_exports_match_reference_surface():
    for name in ("attention", "attention_varlen", "attention_reference", "attention_varlen_reference",
                 "available_backends", "pack_varlen", "attention_splitk_triton", "attention_fp8_triton",
                 "quantize_kv_fp8", "dequantize_kv_fp8"):
        assert callable(getattr(fused_attn, name)), name
    assert fused_attn.__version__ == "0.3.0"


def test_reference_import_paths():
    """The reference's callers import these module paths (benchmarks/bench_decode.py:47-48,
    tests/test_splitk_fp8.py:45); here they are HIP-backed."""
    from fused_attn.triton_fwd import attention_triton, attention_varlen_triton
    from fused_attn.triton_splitk import attention_splitk_triton, choose_num_splits

    assert choose_num_splits(1, 8, 32768, 1, num_sms=108) == 27
    q, k, v = torch.randn(1, 4, 9, 16), torch.randn(1, 2, 12, 16), torch.randn(1, 2, 12, 16)
    ref = orc.attention(q, k, v, causal=True)
    assert torch.allclose(attention_triton(q, k, v, causal=True), ref, atol=1e-5)
    assert torch.allclose(attention_splitk_triton(q, k, v, causal=True), ref, atol=1e-5)
    cu = torch.tensor([0, 9], dtype=torch.int32)
    out = attention_varlen_triton(q[0].transpose(0, 1), k[0].transpose(0, 1), v[0].transpose(0, 1), cu,
                                  torch.tensor([0, 12], dtype=torch.int32), 9, 12, causal=True)
    assert torch.allclose(out.transpose(0, 1), ref[0], atol=1e-5)


def test_attention_triton_cpu_lse_is_consistent_with_the_output():
    """exp(S - lse) are the softmax weights: they reproduce the oracle output and sum to 1 per row."""
    from fused_attn.triton_fwd import attention_triton

    torch.manual_seed(0)
    q, k, v = torch.randn(2, 4, 7, 16), torch.randn(2, 2, 11, 16), torch.randn(2, 2, 11, 16)
    o, lse = attention_triton(q, k, v, causal=True, return_lse=True)
    assert lse.shape == (2, 4, 7)
    kk, vv = orc.expand_kv(k, 2), orc.expand_kv(v, 2)
    s = torch.matmul(q, kk.transpose(-1, -2)) / 4.0
    s = s.masked_fill(~orc.causal_mask(7, 11), float("-inf"))
    p = torch.exp(s - lse[..., None])
    assert torch.allclose(p.sum(-1), torch.ones(2, 4, 7), atol=1e-5)
    assert torch.allclose(torch.matmul(p, vv), orc.attention(q, k, v, causal=True), atol=1e-5)


def test_paged_cpu_path_and_pool_builder():
    """fused_attn.attention_paged on CPU tensors (unfused per-sequence path) vs the oracle, and
    paged_from_dense's pools gather back to the dense keys."""
    gen = torch.Generator().manual_seed(5)
    k = torch.randn(3, 2, 200, 32, generator=gen)
    v = torch.randn(3, 2, 200, 32, generator=gen)
    q = torch.randn(3, 8, 2, 32, generator=gen)
    kc, vc, bt, lens = fused_attn.paged_from_dense(k, v, 64, seqlens=[200, 0, 77], extra_pages=2, generator=gen)
    assert kc.shape == (3 * 4 + 2, 2, 64, 32) and bt.shape == (3, 4) and bt.dtype == torch.int32
    from fused_attn.paged import gather_paged
    assert torch.equal(gather_paged(kc, bt, 200, 0), k[0])
    assert torch.equal(gather_paged(vc, bt, 77, 2), v[2, :, :77])
    for causal in (False, True):
        out = fused_attn.attention_paged(q, kc, vc, bt, lens, causal=causal)
        ref = orc.attention_paged(q, kc, vc, bt, lens, causal=causal)
        torch.testing.assert_close(out, ref, atol=1e-5, rtol=1e-5)
