"""Seeded random configurations for every HIP entry point, against the fp32 oracle.

Complements the fixed matrices of the other GPU tests (which follow the reference's
tests/test_correctness.py, test_varlen.py and test_splitk_fp8.py) with shapes no one
picked by hand: ragged lengths, every GQA ratio that divides the heads, both layouts,
custom and negative scales.  Each case is drawn from its own seed and named before
it runs.  The bar is the reference's assert_close(atol=tol, rtol=tol), since large
random scales produce outputs of magnitude ~4 (see helpers.close), and every case must also
meet the plain max-abs bar and prints its max-abs error (helpers.check_bars)."""
import math
import random

import pytest
import torch

import fused_attn
from fused_attn.triton_fwd import attention_triton
from helpers import FP8_TOL, TOL, announce, check_bars, randn
from oracle import attention_oracle as orc

pytestmark = pytest.mark.gpu

TOL32 = 1e-4


def _tol(dtype):
    return TOL32 if dtype == torch.float32 else TOL[dtype]


def _tensor(shape, dtype, bnhd):
    """[B, H, N, D] tensor, optionally as a view of [B, N, H, D] storage."""
    if not bnhd:
        return randn(*shape, dtype=dtype)
    b, h, n, d = shape
    return randn(b, n, h, d, dtype=dtype).transpose(1, 2)


@pytest.mark.parametrize("seed", range(48))
def test_fuzz_dense(seed):
    rng = random.Random(seed)
    dtype, d = rng.choice([(torch.bfloat16, 64), (torch.bfloat16, 128), (torch.float16, 64), (torch.float16, 128),
                           (torch.bfloat16, 32), (torch.float16, 256), (torch.float32, 64), (torch.float32, 16),
                           (torch.bfloat16, 16), (torch.float16, 32)])
    hkv = rng.choice([1, 2, 4])
    hq = hkv * rng.choice([1, 2, 4, 8])
    b = rng.randint(1, 3)
    n_q, n_k = rng.randint(1, 600), rng.randint(1, 600)
    causal = rng.random() < 0.6
    bnhd = rng.random() < 0.3
    scale = rng.choice([None, None, 0.07, -0.2])
    announce(f"fuzz dense seed={seed} {dtype} d={d} b={b} hq={hq} hkv={hkv} nq={n_q} nk={n_k} causal={causal} "
             f"bnhd={bnhd} scale={scale}")
    torch.manual_seed(seed)
    q = _tensor((b, hq, n_q, d), dtype, bnhd)
    k = _tensor((b, hkv, n_k, d), dtype, bnhd)
    v = _tensor((b, hkv, n_k, d), dtype, bnhd)
    out = fused_attn.attention(q, k, v, causal=causal, scale=scale)
    ref = orc.attention(q.cpu(), k.cpu(), v.cpu(), causal=causal, scale=scale)
    assert out.shape == q.shape and out.dtype == dtype
    check_bars(out, ref, _tol(dtype))


@pytest.mark.parametrize("seed", range(24))
def test_fuzz_dense_long(seed):
    """D=128 with 2048-5000 queries: the 256-query (8-wave) workgroups, with ragged last row
    blocks and key tiles, both layouts, custom and negative scales."""
    rng = random.Random(7000 + seed)
    dtype = rng.choice([torch.bfloat16, torch.float16])
    hkv = rng.choice([1, 2])
    hq = hkv * rng.choice([1, 2])
    causal = rng.random() < 0.5
    n_q = rng.randint(4096 if causal else 2048, 5000)
    n_k = rng.choice([rng.randint(1, 700), rng.randint(2000, 5000)])
    bnhd = rng.random() < 0.4
    scale = rng.choice([None, None, 0.05, -0.1])
    announce(f"fuzz dense long seed={seed} {dtype} hq={hq} hkv={hkv} nq={n_q} nk={n_k} causal={causal} "
             f"bnhd={bnhd} scale={scale}")
    torch.manual_seed(7000 + seed)
    q = _tensor((1, hq, n_q, 128), dtype, bnhd)
    k = _tensor((1, hkv, n_k, 128), dtype, bnhd)
    v = _tensor((1, hkv, n_k, 128), dtype, bnhd)
    out = fused_attn.attention(q, k, v, causal=causal, scale=scale)
    ref = orc.attention(q.cpu(), k.cpu(), v.cpu(), causal=causal, scale=scale)
    assert out.shape == q.shape and out.dtype == dtype
    check_bars(out, ref, _tol(dtype))


@pytest.mark.parametrize("seed", range(32))
def test_fuzz_splitk(seed):
    rng = random.Random(1000 + seed)
    dtype = rng.choice([torch.bfloat16, torch.float16])
    d = rng.choice([64, 128, 256])
    hkv = rng.choice([1, 2, 8])
    hq = hkv * rng.choice([1, 4, 8])
    b = rng.randint(1, 4)
    n_q = rng.randint(1, 16)
    n_k = rng.randint(1, 5000)
    split_len = 64 * rng.randint(1, 40)
    causal = rng.random() < 0.5
    announce(f"fuzz splitk seed={seed} {dtype} d={d} b={b} hq={hq} hkv={hkv} nq={n_q} nk={n_k} split={split_len} "
             f"causal={causal}")
    torch.manual_seed(seed)
    q = randn(b, hq, n_q, d, dtype=dtype)
    k = randn(b, hkv, n_k, d, dtype=dtype)
    v = randn(b, hkv, n_k, d, dtype=dtype)
    out = fused_attn.attention_splitk(q, k, v, causal=causal, split_len=split_len)
    ref = orc.attention(q.cpu(), k.cpu(), v.cpu(), causal=causal)
    check_bars(out, ref, TOL[dtype])


@pytest.mark.parametrize("seed", range(16))
def test_fuzz_fp8_splitk(seed):
    rng = random.Random(2000 + seed)
    d = rng.choice([64, 128, 256])
    hkv = rng.choice([1, 4])
    hq = hkv * rng.choice([1, 8])
    b = rng.randint(1, 3)
    n_q = rng.randint(1, 16)
    n_k = rng.randint(1, 3000)
    split_len = 64 * rng.randint(1, 24)
    announce(f"fuzz fp8 seed={seed} d={d} b={b} hq={hq} hkv={hkv} nq={n_q} nk={n_k} split={split_len}")
    torch.manual_seed(seed)
    q = randn(b, hq, n_q, d, dtype=torch.bfloat16)
    k8, ks = fused_attn.quantize_kv_fp8(randn(b, hkv, n_k, d))
    v8, vs = fused_attn.quantize_kv_fp8(randn(b, hkv, n_k, d))
    out = fused_attn.attention_fp8(q, k8, ks, v8, vs, split_len=split_len)
    ref = orc.attention_fp8(q.cpu(), k8.cpu(), ks.cpu(), v8.cpu(), vs.cpu())
    check_bars(out, ref, FP8_TOL)


@pytest.mark.parametrize("seed", range(24))
def test_fuzz_varlen(seed):
    rng = random.Random(3000 + seed)
    dtype, d = rng.choice([(torch.bfloat16, 128), (torch.float16, 64), (torch.bfloat16, 32), (torch.float32, 64)])
    hkv = rng.choice([1, 2, 4])
    hq = hkv * rng.choice([1, 2, 4])
    nseq = rng.randint(1, 9)
    lens_q = [rng.choice([0, 1, rng.randint(0, 400)]) for _ in range(nseq)]
    same = rng.random() < 0.5
    lens_k = list(lens_q) if same else [rng.randint(0, 400) for _ in range(nseq)]
    causal = rng.random() < 0.6
    announce(f"fuzz varlen seed={seed} {dtype} d={d} hq={hq} hkv={hkv} lens_q={lens_q} lens_k={lens_k} "
             f"causal={causal}")
    torch.manual_seed(seed)
    qs = [randn(n, hq, d, dtype=dtype) for n in lens_q]
    ks = [randn(n, hkv, d, dtype=dtype) for n in lens_k]
    vs = [randn(n, hkv, d, dtype=dtype) for n in lens_k]
    q, cu_q, max_q = fused_attn.pack_varlen(qs)
    k, cu_k, max_k = fused_attn.pack_varlen(ks)
    v, _, _ = fused_attn.pack_varlen(vs)
    out = fused_attn.attention_varlen(q, k, v, cu_q, cu_k, max_q, max_k, causal=causal)
    ref = orc.attention_varlen(q.cpu(), k.cpu(), v.cpu(), cu_q.cpu(), cu_k.cpu(), causal=causal)
    assert out.shape == q.shape
    check_bars(out, ref, _tol(dtype))


@pytest.mark.parametrize("seed", range(8))
def test_fuzz_varlen_long(seed):
    """Varlen D=128 batches whose longest sequence reaches the 256-query (8-wave) workgroups,
    beside empty, one-token and short sequences."""
    rng = random.Random(8000 + seed)
    dtype = rng.choice([torch.bfloat16, torch.float16])
    hkv = rng.choice([1, 2])
    hq = hkv * rng.choice([1, 2])
    causal = rng.random() < 0.5
    nseq = rng.randint(2, 5)
    lens_q = [rng.choice([0, 1, rng.randint(2, 700), rng.randint(700, 4600)]) for _ in range(nseq)]
    lens_q[rng.randrange(nseq)] = rng.randint(4096 if causal else 2048, 4600)
    same = rng.random() < 0.5
    lens_k = list(lens_q) if same else [rng.randint(0, 4600) for _ in range(nseq)]
    announce(f"fuzz varlen long seed={seed} {dtype} hq={hq} hkv={hkv} lens_q={lens_q} lens_k={lens_k} "
             f"causal={causal}")
    torch.manual_seed(8000 + seed)
    qs = [randn(n, hq, 128, dtype=dtype) for n in lens_q]
    ks = [randn(n, hkv, 128, dtype=dtype) for n in lens_k]
    vs = [randn(n, hkv, 128, dtype=dtype) for n in lens_k]
    q, cu_q, max_q = fused_attn.pack_varlen(qs)
    k, cu_k, max_k = fused_attn.pack_varlen(ks)
    v, _, _ = fused_attn.pack_varlen(vs)
    out = fused_attn.attention_varlen(q, k, v, cu_q, cu_k, max_q, max_k, causal=causal)
    ref = orc.attention_varlen(q.cpu(), k.cpu(), v.cpu(), cu_q.cpu(), cu_k.cpu(), causal=causal)
    assert out.shape == q.shape
    check_bars(out, ref, _tol(dtype))


@pytest.mark.parametrize("seed", range(16))
def test_fuzz_paged(seed):
    rng = random.Random(4000 + seed)
    dtype = rng.choice([torch.bfloat16, torch.float16])
    d = rng.choice([64, 128, 256])
    page = rng.choice([16, 32, 48, 64, 96, 128])
    hkv = rng.choice([1, 2, 4])
    hq = hkv * rng.choice([1, 4])
    b = rng.randint(1, 5)
    n_max = rng.randint(1, 2000)
    lens = [rng.randint(0, n_max) for _ in range(b)]
    n_q = rng.choice([1, 1, 3, 16])
    causal = n_q > 1 and rng.random() < 0.7
    split_len = 64 * rng.randint(1, 16)
    announce(f"fuzz paged seed={seed} {dtype} d={d} page={page} hq={hq} hkv={hkv} lens={lens} nq={n_q} "
             f"causal={causal} split={split_len}")
    gen = torch.Generator(device="cuda").manual_seed(seed)
    q = randn(b, hq, n_q, d, dtype=dtype, gen=gen)
    k = randn(b, hkv, n_max, d, dtype=dtype, gen=gen)
    v = randn(b, hkv, n_max, d, dtype=dtype, gen=gen)
    kc, vc, bt, sl = fused_attn.paged_from_dense(k, v, page, seqlens=lens, extra_pages=2,
                                                 generator=torch.Generator().manual_seed(seed))
    out = fused_attn.attention_paged(q, kc, vc, bt, sl, causal=causal, split_len=split_len)
    ref = orc.attention_paged(q, kc, vc, bt, sl, causal=causal)
    check_bars(out, ref, TOL[dtype])


def test_fuzz_lse_matches_logsumexp():
    """LSE of random dense calls against a float64 logsumexp of the scaled scores."""
    for seed in range(6):
        rng = random.Random(5000 + seed)
        dtype, d = rng.choice([(torch.bfloat16, 128), (torch.float16, 64), (torch.float32, 32)])
        n_q, n_k = rng.randint(1, 300), rng.randint(1, 300)
        causal = rng.random() < 0.5
        announce(f"fuzz lse seed={seed} {dtype} d={d} nq={n_q} nk={n_k} causal={causal}")
        torch.manual_seed(seed)
        q, k, v = randn(1, 2, n_q, d, dtype=dtype), randn(1, 2, n_k, d, dtype=dtype), randn(1, 2, n_k, d, dtype=dtype)
        _, lse = attention_triton(q, k, v, causal=causal, return_lse=True)
        s = torch.matmul(q.double().cpu(), k.double().cpu().transpose(-1, -2)) / math.sqrt(d)
        if causal:
            s = s.masked_fill(~orc.causal_mask(n_q, n_k), float("-inf"))
        ref = torch.logsumexp(s, dim=-1)
        got = lse.double().cpu()
        fin = torch.isfinite(ref)
        assert torch.equal(fin, torch.isfinite(got))
        bar = 1e-4 if dtype == torch.float32 else 2.0 ** -8
        assert (got[fin] - ref[fin]).abs().max().item() < bar
