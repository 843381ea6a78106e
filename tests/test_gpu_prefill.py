"""Dense prefill parity: the HIP MFMA kernel (through the public op and the C ABI) vs the fp32 oracle.

Mirrors the reference's kernel tests (tests/test_correctness.py:56-122,
tests/test_splitk_fp8.py:89-106) at the tolerances this build commits to."""
import math

import pytest
import torch

import fused_attn
from fused_attn import _hip, ops
from helpers import TOL, announce, max_err, randn
from oracle import attention_oracle as orc

pytestmark = pytest.mark.gpu

SHAPES = [
    (1, 1, 1, 64, 64),
    (2, 4, 4, 128, 128),
    (1, 8, 2, 100, 100),  # GQA 4:1, ragged tails
    (1, 4, 1, 37, 90),  # MQA, n_q < n_k (bottom-right causal)
    (1, 2, 2, 90, 40),  # n_q > n_k: leading rows see no key
    (3, 2, 2, 1, 257),  # single-token step below the split-K threshold
    (2, 8, 2, 333, 333),
    (1, 4, 1, 100, 500),
    (1, 2, 2, 500, 100),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("head_dim", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("b,h_q,h_kv,n_q,n_k", SHAPES)
def test_prefill_matches_oracle(b, h_q, h_kv, n_q, n_k, causal, head_dim, dtype):
    announce(f"prefill b={b} hq={h_q} hkv={h_kv} nq={n_q} nk={n_k} causal={causal} d={head_dim} {dtype}")
    torch.manual_seed(0)
    q = randn(b, h_q, n_q, head_dim, dtype=dtype)
    k = randn(b, h_kv, n_k, head_dim, dtype=dtype)
    v = randn(b, h_kv, n_k, head_dim, dtype=dtype)
    assert ops._pick_backend(q, k) == "hip" and ops._hip_kernel_for(q, k) == "fwd"
    out = fused_attn.attention(q, k, v, causal=causal)
    torch.cuda.synchronize()
    ref = orc.attention(q.cpu(), k.cpu(), v.cpu(), causal=causal)
    assert out.dtype == q.dtype and out.shape == q.shape
    assert not torch.isnan(out).any()
    assert max_err(out, ref) <= TOL[dtype]


def test_custom_scale_and_negative_scale():
    torch.manual_seed(0)
    q, k, v = (randn(1, 2, 64, 64, dtype=torch.bfloat16) for _ in range(3))
    for s in (0.05, -0.125):
        announce(f"scale={s}")
        out = fused_attn.attention(q, k, v, causal=True, scale=s)
        ref = orc.attention(q.cpu(), k.cpu(), v.cpu(), causal=True, scale=s)
        assert max_err(out, ref) <= TOL[torch.bfloat16]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_noncontiguous_bnhd_layout(dtype):
    """[B, N, H, D] storage (the usual HF layout) viewed as [B, H, N, D] (tests/test_correctness.py:97-106)."""
    announce(f"bnhd view {dtype}")
    torch.manual_seed(0)
    x = randn(2, 64, 3, 4, 64, dtype=dtype)
    q, k, v = (x[:, :, i].transpose(1, 2) for i in range(3))
    assert not q.is_contiguous()
    out = fused_attn.attention(q, k, v, causal=True)
    ref = orc.attention(q.cpu(), k.cpu(), v.cpu(), causal=True)
    # a contiguous [B,H,N,D] output, the strides of the op's fake (q.new_empty(q.shape))
    assert out.shape == q.shape and out.is_contiguous()
    assert max_err(out, ref) <= TOL[dtype]


def test_unaligned_views_are_copied_not_misread():
    announce("unaligned views")
    torch.manual_seed(0)
    base = randn(2 * 65 * 64 + 3, dtype=torch.bfloat16)
    q = base[3:].view(1, 2, 65, 64)[:, :, :64]  # data pointer 6 bytes past 16-byte alignment
    assert q.data_ptr() % 16 != 0
    k = randn(1, 2, 64, 64, dtype=torch.bfloat16)
    v = randn(1, 2, 64, 64, dtype=torch.bfloat16)
    out = fused_attn.attention(q, k, v)
    assert max_err(out, orc.attention(q.cpu(), k.cpu(), v.cpu())) <= TOL[torch.bfloat16]


@pytest.mark.parametrize("d", [128, 256])
@pytest.mark.parametrize("causal", [False, True])
def test_lse_output(causal, d):
    announce(f"lse causal={causal} d={d}")
    torch.manual_seed(0)
    q = randn(2, 8, 100, d, dtype=torch.bfloat16)
    k = randn(2, 2, 77, d, dtype=torch.bfloat16)
    v = randn(2, 2, 77, d, dtype=torch.bfloat16)
    out, lse = _hip.fwd(q, k, v, causal=causal, return_lse=True)
    qf, kf = q.float().cpu(), orc.expand_kv(k.float().cpu(), 4)
    s = torch.matmul(qf, kf.transpose(-1, -2)) / math.sqrt(d)
    if causal:
        s = s.masked_fill(~orc.causal_mask(100, 77), float("-inf"))
    ref = torch.logsumexp(s, dim=-1)
    got = lse.cpu()
    fin = torch.isfinite(ref)
    assert torch.equal(fin, torch.isfinite(got))  # rows without keys report -inf
    # l sums the bf16-rounded P that the MFMA consumes, so the LSE carries bf16-level
    # relative error in l: bound it by the bf16 resolution 2^-8
    assert (got[fin] - ref[fin]).abs().max().item() < 2.0 ** -8


def test_zero_sized_inputs():
    announce("zero-sized")
    q = torch.empty(0, 2, 16, 64, dtype=torch.bfloat16, device="cuda")
    k = torch.empty(0, 2, 16, 64, dtype=torch.bfloat16, device="cuda")
    assert fused_attn.attention(q, k, k).shape == q.shape
    q = torch.empty(1, 2, 0, 64, dtype=torch.bfloat16, device="cuda")
    k1 = randn(1, 2, 16, 64, dtype=torch.bfloat16)
    assert fused_attn.attention(q, k1, k1).shape == q.shape
    # n_k == 0: every row is empty -> zeros
    q = randn(1, 2, 8, 64, dtype=torch.bfloat16)
    kz = torch.empty(1, 2, 0, 64, dtype=torch.bfloat16, device="cuda")
    assert torch.all(fused_attn.attention(q, kz, kz) == 0)
    assert torch.all(fused_attn.attention(q, kz, kz, causal=True) == 0)


def test_unsupported_head_dim_raises_loudly():
    q = randn(1, 2, 16, 48, dtype=torch.bfloat16)  # fp32 goes to the generic kernel at D in {16, ..., 256}
    with pytest.raises(RuntimeError, match="unsupported"):
        _hip.fwd(q, q, q)


# ---- benchmark-sized workloads ------------------------------------------------------------------


@pytest.mark.parametrize("cfg", [
    dict(b=4, hq=32, hkv=8, n=4096, d=128, layout="bhnd"),
    dict(b=4, hq=16, hkv=16, n=4096, d=64, layout="bhnd"),
    dict(b=4, hq=16, hkv=16, n=4096, d=32, layout="bhnd"),
    dict(b=4, hq=16, hkv=16, n=4096, d=16, layout="bhnd"),
    dict(b=4, hq=32, hkv=8, n=4096, d=128, layout="bnhd"),
])
def test_benchmark_prefill_workloads(cfg):
    """Causal bf16 prefill at the benchmark sizes; oracle in fp32 on the GPU, per (batch, kv group)."""
    announce(f"benchmark prefill {cfg}")
    b, hq, hkv, n, d = cfg["b"], cfg["hq"], cfg["hkv"], cfg["n"], cfg["d"]
    gen = torch.Generator(device="cuda").manual_seed(0)
    if cfg["layout"] == "bnhd":
        q = randn(b, n, hq, d, dtype=torch.bfloat16, gen=gen).transpose(1, 2)
        k = randn(b, n, hkv, d, dtype=torch.bfloat16, gen=gen).transpose(1, 2)
        v = randn(b, n, hkv, d, dtype=torch.bfloat16, gen=gen).transpose(1, 2)
    else:
        q = randn(b, hq, n, d, dtype=torch.bfloat16, gen=gen)
        k = randn(b, hkv, n, d, dtype=torch.bfloat16, gen=gen)
        v = randn(b, hkv, n, d, dtype=torch.bfloat16, gen=gen)
    out = fused_attn.attention(q, k, v, causal=True)
    ref = orc.attention_chunked(q, k, v, causal=True)
    err = max_err(out, ref)
    print(f"max_abs_err={err:.3e}", flush=True)
    assert err <= TOL[torch.bfloat16]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_head_dim_256_views_varlen_and_decode_shapes(dtype):
    """D=256 on the MFMA kernel (32-key tiles, one wave per SIMD): the [B,N,H,D] view, a
    varlen batch with an empty sequence, and a decode-shaped call (split-K, and the prefill kernel on
    the same shape)."""
    announce(f"d=256 extra shapes {dtype}")
    torch.manual_seed(0)
    x = randn(2, 150, 3, 4, 256, dtype=dtype)
    q, k, v = (x[:, :, i].transpose(1, 2) for i in range(3))
    out = fused_attn.attention(q, k, v, causal=True)
    assert max_err(out, orc.attention(q.cpu(), k.cpu(), v.cpu(), causal=True)) <= TOL[dtype]
    lens = [37, 0, 300, 1]
    qv, cu, mx = fused_attn.pack_varlen([randn(n, 8, 256, dtype=dtype) for n in lens])
    kv, _, _ = fused_attn.pack_varlen([randn(n, 2, 256, dtype=dtype) for n in lens])
    vv, _, _ = fused_attn.pack_varlen([randn(n, 2, 256, dtype=dtype) for n in lens])
    out = fused_attn.attention_varlen(qv, kv, vv, cu, cu, mx, mx, causal=True)
    ref = orc.attention_varlen(qv.cpu(), kv.cpu(), vv.cpu(), cu.cpu(), cu.cpu(), causal=True)
    assert max_err(out, ref) <= TOL[dtype]
    q = randn(2, 8, 1, 256, dtype=dtype)
    k = randn(2, 2, 3000, 256, dtype=dtype)
    v = randn(2, 2, 3000, 256, dtype=dtype)
    assert ops._hip_kernel_for(q, k) == "splitk"
    out = fused_attn.attention(q, k, v)
    ref = orc.attention(q.cpu(), k.cpu(), v.cpu())
    assert max_err(out, ref) <= TOL[dtype]
    assert max_err(_hip.fwd(q, k, v), ref) <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("d", [16, 32])
def test_small_head_dims_views_varlen_and_decode_shapes(d, dtype):
    """D=32 and D=16 on the MFMA kernel (128-key tiles; at D=16 the V tile is padded to 32 columns):
    the [B,N,H,D] view, a varlen batch with an empty sequence, and a decode-shaped call (split-K
    does not take these head dims)."""
    announce(f"d={d} extra shapes {dtype}")
    torch.manual_seed(0)
    x = randn(2, 300, 3, 4, d, dtype=dtype)
    q, k, v = (x[:, :, i].transpose(1, 2) for i in range(3))
    out = fused_attn.attention(q, k, v, causal=True)
    assert max_err(out, orc.attention(q.cpu(), k.cpu(), v.cpu(), causal=True)) <= TOL[dtype]
    lens = [37, 0, 300, 1, 129]
    qv, cu, mx = fused_attn.pack_varlen([randn(n, 8, d, dtype=dtype) for n in lens])
    kv, _, _ = fused_attn.pack_varlen([randn(n, 2, d, dtype=dtype) for n in lens])
    vv, _, _ = fused_attn.pack_varlen([randn(n, 2, d, dtype=dtype) for n in lens])
    out = fused_attn.attention_varlen(qv, kv, vv, cu, cu, mx, mx, causal=True)
    ref = orc.attention_varlen(qv.cpu(), kv.cpu(), vv.cpu(), cu.cpu(), cu.cpu(), causal=True)
    assert max_err(out, ref) <= TOL[dtype]
    q = randn(2, 8, 1, d, dtype=dtype)
    k = randn(2, 2, 3000, d, dtype=dtype)
    v = randn(2, 2, 3000, d, dtype=dtype)
    assert ops._hip_kernel_for(q, k) == "fwd"
    assert max_err(fused_attn.attention(q, k, v), orc.attention(q.cpu(), k.cpu(), v.cpu())) <= TOL[dtype]


@pytest.mark.parametrize("causal", [False, True])
def test_long_context_prefill(causal):
    """N=16384 (128 query blocks per head, 256 key tiles): grid, schedule and tail at long context."""
    announce(f"long-context prefill causal={causal}")
    gen = torch.Generator(device="cuda").manual_seed(5)
    q = randn(1, 8, 16384, 128, dtype=torch.bfloat16, gen=gen)
    k = randn(1, 2, 16384, 128, dtype=torch.bfloat16, gen=gen)
    v = randn(1, 2, 16384, 128, dtype=torch.bfloat16, gen=gen)
    out = fused_attn.attention(q, k, v, causal=causal)
    ref = orc.attention_chunked(q, k, v, causal=causal, heads_per_chunk=1, rows_per_chunk=2048)
    err = max_err(out, ref)
    print(f"max_abs_err={err:.3e}", flush=True)
    assert err <= TOL[torch.bfloat16]


@pytest.mark.parametrize("n_q,n_k,causal", [(4200, 5000, True), (4096, 3000, True), (4100, 4100, False),
                                            (5000, 4200, True), (2048, 3000, False), (2500, 777, False),
                                            (4095, 4095, True)])
def test_eight_wave_blocks_ragged_and_offset(n_q, n_k, causal):
    """Dense D=128 with >= 4096 queries (>= 2048 without the causal mask) runs 256-query workgroups: a
    partial last block, bottom-right causal offsets both ways (rows that see no key when n_k < n_q) and
    the per-wave causal skip.  4095 causal queries stay on the 4-wave kernel, next to its limit."""
    announce(f"8-wave prefill nq={n_q} nk={n_k} causal={causal}")
    gen = torch.Generator(device="cuda").manual_seed(n_q + n_k)
    q = randn(1, 8, n_q, 128, dtype=torch.bfloat16, gen=gen)
    k = randn(1, 2, n_k, 128, dtype=torch.bfloat16, gen=gen)
    v = randn(1, 2, n_k, 128, dtype=torch.bfloat16, gen=gen)
    out = fused_attn.attention(q, k, v, causal=causal)
    ref = orc.attention_chunked(q, k, v, causal=causal, heads_per_chunk=2, rows_per_chunk=1024)
    assert not torch.isnan(out).any()
    assert max_err(out, ref) <= TOL[torch.bfloat16]


@pytest.mark.parametrize("n_q,n_k,causal", [(4200, 5000, True), (2500, 777, False)])
def test_eight_wave_blocks_fp16_with_lse(n_q, n_k, causal):
    """The 8-wave workgroups in fp16, with the LSE output: rows of a partial last block and rows that
    see no key (n_k < n_q) included."""
    announce(f"8-wave prefill fp16 + LSE nq={n_q} nk={n_k} causal={causal}")
    gen = torch.Generator(device="cuda").manual_seed(7 * n_q + n_k)
    q = randn(1, 8, n_q, 128, dtype=torch.float16, gen=gen)
    k = randn(1, 2, n_k, 128, dtype=torch.float16, gen=gen)
    v = randn(1, 2, n_k, 128, dtype=torch.float16, gen=gen)
    out, lse = _hip.fwd(q, k, v, causal=causal, return_lse=True)
    ref = orc.attention_chunked(q, k, v, causal=causal, heads_per_chunk=2, rows_per_chunk=1024)
    assert not torch.isnan(out).any()
    assert max_err(out, ref) <= TOL[torch.float16]
    # LSE against a float64 log-sum-exp of the same scores (rows with no key: -inf)
    qd, kd = q.double().cpu(), orc.expand_kv(k.double().cpu(), 4)
    s = torch.matmul(qd, kd.transpose(-1, -2)) / math.sqrt(128)
    if causal:
        s = s.masked_fill(~orc.causal_mask(n_q, n_k), float("-inf"))
    ref_lse = torch.logsumexp(s, dim=-1).float()
    got = lse.cpu()
    finite = torch.isfinite(ref_lse)
    assert torch.equal(finite, torch.isfinite(got))
    # l sums the fp16-rounded P (resolution 2^-11); bound the LSE error by 2^-9
    assert (got[finite] - ref_lse[finite]).abs().max().item() < 2.0 ** -9
