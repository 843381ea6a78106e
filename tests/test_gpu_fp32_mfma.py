"""The fp32-MFMA prefill kernel (fp32 Q/K/V, D = 32, 64, 128 and 256) vs the fp32 oracle at the reference's
fp32 bar, atol = rtol = 1e-4 (tests/test_correctness.py:53-85): several key tiles, ragged tails,
GQA/MQA, bottom-right causal alignment with rows that see no key, [B,N,H,D] views, negative scale,
packed sequences with empty ones, and a long causal sequence."""
import pytest
import torch

import fused_attn
from helpers import announce, randn
from oracle import attention_oracle as orc

pytestmark = pytest.mark.gpu

TOL = dict(atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("d", [32, 64, 128, 256])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("b,h_q,h_kv,n_q,n_k", [
    (1, 4, 4, 129, 129),   # one 128-query block plus one row, 5 key tiles
    (2, 8, 2, 300, 300),   # GQA 4:1, ragged tails
    (1, 4, 1, 100, 517),   # MQA, n_q < n_k
    (1, 2, 2, 517, 100),   # n_q > n_k: leading rows see no key
    (3, 2, 1, 31, 33),     # a tile and one key
])
def test_fp32_mfma_matches_oracle(b, h_q, h_kv, n_q, n_k, causal, d):
    announce(f"fp32 mfma b={b} hq={h_q} hkv={h_kv} nq={n_q} nk={n_k} causal={causal} d={d}")
    torch.manual_seed(0)
    q = randn(b, h_q, n_q, d, dtype=torch.float32)
    k = randn(b, h_kv, n_k, d, dtype=torch.float32)
    v = randn(b, h_kv, n_k, d, dtype=torch.float32)
    out = fused_attn.attention(q, k, v, causal=causal)
    torch.testing.assert_close(out.cpu(), orc.attention(q.cpu(), k.cpu(), v.cpu(), causal=causal), **TOL)


@pytest.mark.parametrize("d", [32, 64, 128, 256])
def test_fp32_mfma_views_and_scales(d):
    announce(f"fp32 mfma [B,N,H,D] view and scales d={d}")
    torch.manual_seed(1)
    x = randn(2, 200, 3, 4, d, dtype=torch.float32)
    q, k, v = (x[:, :, i].transpose(1, 2) for i in range(3))
    for scale in (None, 0.02, -0.1):
        out = fused_attn.attention(q, k, v, causal=True, scale=scale)
        torch.testing.assert_close(out.cpu(), orc.attention(q.cpu(), k.cpu(), v.cpu(), causal=True, scale=scale),
                                   **TOL)


@pytest.mark.parametrize("d", [32, 64, 128, 256])
@pytest.mark.parametrize("causal", [False, True])
def test_fp32_mfma_varlen(d, causal):
    announce(f"fp32 mfma varlen d={d} causal={causal}")
    torch.manual_seed(2)
    lens = [5, 0, 300, 1, 129, 0]
    q, cu, mx = fused_attn.pack_varlen([randn(n, 8, d, dtype=torch.float32) for n in lens])
    k, _, _ = fused_attn.pack_varlen([randn(n, 2, d, dtype=torch.float32) for n in lens])
    v, _, _ = fused_attn.pack_varlen([randn(n, 2, d, dtype=torch.float32) for n in lens])
    out = fused_attn.attention_varlen(q, k, v, cu, cu, mx, mx, causal=causal)
    ref = orc.attention_varlen(q.cpu(), k.cpu(), v.cpu(), cu.cpu(), cu.cpu(), causal=causal)
    torch.testing.assert_close(out.cpu(), ref, **TOL)


def test_fp32_mfma_long_causal():
    announce("fp32 mfma long causal N=2048 d=128")
    gen = torch.Generator(device="cuda").manual_seed(3)
    q = randn(1, 8, 2048, 128, dtype=torch.float32, gen=gen)
    k = randn(1, 2, 2048, 128, dtype=torch.float32, gen=gen)
    v = randn(1, 2, 2048, 128, dtype=torch.float32, gen=gen)
    out = fused_attn.attention(q, k, v, causal=True)
    ref = orc.attention_chunked(q, k, v, causal=True, heads_per_chunk=1, rows_per_chunk=512)
    torch.testing.assert_close(out, ref, **TOL)


def test_reference_cpu_configuration_on_the_gpu():
    """The reference's CPU-runnable case: dense causal MHA fp32 B=2 Hq=Hkv=4 N=256 D=64, seed 0,
    scale 1/sqrt(D), [B,H,N,D].  Runs on the fp32-MFMA kernel and matches the oracle at 1e-4."""
    announce("reference cpu configuration fp32 B=2 H=4 N=256 D=64")
    torch.manual_seed(0)
    q, k, v = (torch.randn(2, 4, 256, 64) for _ in range(3))
    out = fused_attn.attention(q.cuda(), k.cuda(), v.cuda(), causal=True)
    torch.testing.assert_close(out.cpu(), orc.attention(q, k, v, causal=True), **TOL)
    torch.testing.assert_close(out.cpu(), torch.from_numpy(orc.attention_f64(q, k, v, causal=True)).float(),
                               **TOL)
