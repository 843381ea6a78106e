"""The fp32 kernels (the generic kernel at D=16, the fp32-MFMA kernel at D=32, 64, 128 and 256)
vs the fp32 oracle; the 16-bit cases in this matrix (D=16, 32, 256) run on the 16-bit MFMA kernel.

Mirrors the reference's fused-kernel matrix (tests/test_correctness.py:53-85): fp32 at
atol = rtol = 1e-4, fp16 / bf16 at the build's bars; plus its fp32 custom-scale and
[B, N, H, D] layout tests (tests/test_correctness.py:88-106), varlen and LSE."""
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
    (1, 2, 2, 90, 40),  # n_q > n_k: leading rows have no keys
    (3, 2, 2, 1, 257),  # single-token decode step
]


def _check(out, ref, dtype):
    if dtype == torch.float32:
        torch.testing.assert_close(out.cpu(), ref.cpu().float(), atol=1e-4, rtol=1e-4)
    else:
        assert max_err(out, ref) <= TOL[dtype]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dtype,d", [(torch.float32, 32), (torch.float32, 64), (torch.float32, 128),
                                     (torch.float32, 16), (torch.float32, 256), (torch.bfloat16, 16),
                                     (torch.bfloat16, 32), (torch.bfloat16, 256), (torch.float16, 32),
                                     (torch.float16, 256)])
def test_generic_matches_oracle(shape, causal, dtype, d):
    b, h_q, h_kv, n_q, n_k = shape
    announce(f"generic {shape} causal={causal} {dtype} d={d}")
    torch.manual_seed(0)
    q = randn(b, h_q, n_q, d, dtype=dtype)
    k = randn(b, h_kv, n_k, d, dtype=dtype)
    v = randn(b, h_kv, n_k, d, dtype=dtype)
    assert ops._hip_kernel_for(q, k) == "fwd"
    out = fused_attn.attention(q, k, v, causal=causal)
    assert out.shape == q.shape and out.dtype == dtype
    _check(out, orc.attention(q.cpu(), k.cpu(), v.cpu(), causal=causal), dtype)


def test_generic_custom_scale_fp32():
    announce("generic fp32 custom scale")
    torch.manual_seed(0)
    q, k, v = (randn(1, 2, 64, 64, dtype=torch.float32) for _ in range(3))
    for scale in (0.05, -0.3):
        out = fused_attn.attention(q, k, v, causal=True, scale=scale)
        _check(out, orc.attention(q.cpu(), k.cpu(), v.cpu(), causal=True, scale=scale), torch.float32)


def test_generic_noncontiguous_heads_fp32():
    """[B, N, H, D] storage viewed as [B, H, N, D] (reference: tests/test_correctness.py:97-106)."""
    announce("generic fp32 [B,N,H,D]")
    torch.manual_seed(0)
    x = torch.randn(2, 64, 3, 4, 64, device="cuda")
    q, k, v = (x[:, :, i].transpose(1, 2) for i in range(3))
    assert not q.is_contiguous()
    out = fused_attn.attention(q, k, v, causal=True)
    _check(out, orc.attention(q.cpu(), k.cpu(), v.cpu(), causal=True), torch.float32)


def test_generic_decode_shape_fp32_through_the_op():
    announce("generic fp32 decode shape")
    torch.manual_seed(0)
    q = randn(2, 8, 1, 128, dtype=torch.float32)
    k = randn(2, 2, 4096, 128, dtype=torch.float32)
    v = randn(2, 2, 4096, 128, dtype=torch.float32)
    out = fused_attn.attention(q, k, v)
    _check(out, orc.attention(q.cpu(), k.cpu(), v.cpu()), torch.float32)


@pytest.mark.parametrize("dtype,d", [(torch.float32, 64), (torch.bfloat16, 32), (torch.float32, 256)])
@pytest.mark.parametrize("causal", [False, True])
def test_generic_varlen(dtype, d, causal):
    announce(f"generic varlen {dtype} d={d} causal={causal}")
    torch.manual_seed(0)
    lens = [5, 0, 70, 1]
    qs = [randn(n, 4, d, dtype=dtype) for n in lens]
    ks = [randn(n, 2, d, dtype=dtype) for n in lens]
    vs = [randn(n, 2, d, dtype=dtype) for n in lens]
    q, cu_q, max_q = fused_attn.pack_varlen(qs)
    k, cu_k, max_k = fused_attn.pack_varlen(ks)
    v, _, _ = fused_attn.pack_varlen(vs)
    out = fused_attn.attention_varlen(q, k, v, cu_q, cu_k, max_q, max_k, causal=causal)
    ref = orc.attention_varlen(q.cpu(), k.cpu(), v.cpu(), cu_q.cpu(), cu_k.cpu(), causal=causal)
    _check(out, ref, dtype)


@pytest.mark.parametrize("d", [32, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_generic_lse_fp32(causal, d):
    """fp32 LSE on the fp32-MFMA kernel (D=32 and D=128)."""
    announce(f"fp32 lse causal={causal} d={d}")
    torch.manual_seed(0)
    q = randn(2, 4, 50, d, dtype=torch.float32)
    k = randn(2, 2, 40, d, dtype=torch.float32)
    out, lse = _hip.fwd(q, k, k, causal=causal, return_lse=True)
    s = torch.matmul(q.cpu(), orc.expand_kv(k.cpu(), 2).transpose(-1, -2)) / math.sqrt(d)
    if causal:
        s = s.masked_fill(~orc.causal_mask(50, 40), float("-inf"))
    ref = torch.logsumexp(s, dim=-1)
    got = lse.cpu()
    fin = torch.isfinite(ref)
    assert torch.equal(fin, torch.isfinite(got))
    assert (got[fin] - ref[fin]).abs().max().item() < 1e-4
