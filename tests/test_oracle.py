"""Pins the oracle (oracle/attention_oracle.py) against library routines, an independent
float64 brute force, closed forms and the reference's own known answers.  CPU only."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention_oracle as orc


# ---- attention math ---------------------------------------------------------------------------


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("n", [1, 17, 128])
def test_oracle_matches_sdpa(n, causal):
    # reference: tests/test_correctness.py:32-39
    torch.manual_seed(0)
    q, k, v = (torch.randn(2, 4, n, 64) for _ in range(3))
    torch.testing.assert_close(orc.attention(q, k, v, causal=causal),
                               F.scaled_dot_product_attention(q, k, v, is_causal=causal), atol=1e-5, rtol=1e-5)


def test_oracle_gqa_equals_repeat_interleave_sdpa():
    # reference: tests/test_correctness.py:42-50
    torch.manual_seed(0)
    q = torch.randn(1, 8, 32, 64)
    k, v = torch.randn(1, 2, 32, 64), torch.randn(1, 2, 32, 64)
    exp = F.scaled_dot_product_attention(q, k.repeat_interleave(4, 1), v.repeat_interleave(4, 1), is_causal=True)
    torch.testing.assert_close(orc.attention(q, k, v, causal=True), exp, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("n_q,n_k", [(37, 90), (90, 40), (1, 257), (5, 5)])
def test_bottom_right_causal_matches_sdpa_with_explicit_mask(n_q, n_k):
    torch.manual_seed(1)
    q, k, v = torch.randn(1, 2, n_q, 32), torch.randn(1, 2, n_k, 32), torch.randn(1, 2, n_k, 32)
    i = torch.arange(n_q)[:, None]
    j = torch.arange(n_k)[None, :]
    mask = j <= i + (n_k - n_q)
    exp = F.scaled_dot_product_attention(q, k, v, attn_mask=mask)
    exp = torch.where(mask.any(-1)[None, None, :, None], exp, torch.zeros_like(exp))  # empty rows -> 0
    torch.testing.assert_close(orc.attention(q, k, v, causal=True), exp, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("shape", [(1, 4, 1, 37, 90, 16), (1, 2, 2, 9, 4, 8), (2, 4, 2, 13, 13, 32)])
def test_oracle_matches_float64_bruteforce(shape, causal):
    b, hq, hkv, nq, nk, d = shape
    torch.manual_seed(2)
    q, k, v = torch.randn(b, hq, nq, d), torch.randn(b, hkv, nk, d), torch.randn(b, hkv, nk, d)
    ref = orc.attention_f64(q, k, v, causal=causal, scale=0.3)
    np.testing.assert_allclose(orc.attention(q, k, v, causal=causal, scale=0.3).numpy(), ref, atol=2e-6, rtol=1e-5)


def test_closed_forms():
    torch.manual_seed(3)
    v = torch.randn(1, 1, 6, 8)
    k = torch.randn(1, 1, 6, 8)
    q = torch.randn(1, 1, 6, 8)
    out = orc.attention(q, k, v, causal=True)
    torch.testing.assert_close(out[0, 0, 0], v[0, 0, 0])  # first causal row sees only key 0
    # equal scores (zero queries) -> uniform weights -> running mean of the visible values
    out0 = orc.attention(torch.zeros_like(q), k, v, causal=True)
    means = torch.cumsum(v[0, 0], 0) / torch.arange(1, 7)[:, None]
    torch.testing.assert_close(out0[0, 0], means)
    # n_q > n_k: the first n_q - n_k rows see no key -> zeros
    outz = orc.attention(torch.randn(1, 1, 5, 8), k[:, :, :2], v[:, :, :2], causal=True)
    assert torch.all(outz[0, 0, :3] == 0) and torch.all(outz[0, 0, 3:].abs() > 0)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("shape", [(1, 4, 1, 37, 90, 16), (1, 2, 2, 9, 4, 8), (2, 4, 2, 13, 13, 32)])
def test_lse_matches_float64_bruteforce(shape, causal):
    b, hq, hkv, nq, nk, d = shape
    torch.manual_seed(5)
    q, k = torch.randn(b, hq, nq, d), torch.randn(b, hkv, nk, d)
    ref = orc.lse_f64(q, k, causal=causal, scale=0.3)
    got = orc.lse(q, k, causal=causal, scale=0.3).numpy()
    assert np.array_equal(np.isfinite(ref), np.isfinite(got))  # (9, 4) causal: 5 rows see no key
    fin = np.isfinite(ref)
    np.testing.assert_allclose(got[fin], ref[fin], atol=2e-6, rtol=1e-6)
    if causal and nq > nk:
        assert np.all(got[..., : nq - nk] == -np.inf)


def test_lse_closed_forms():
    torch.manual_seed(6)
    q, k = torch.randn(1, 1, 6, 8), torch.randn(1, 1, 6, 8)
    lse = orc.lse(q, k, causal=True, scale=0.5)
    # the first causal row sees only key 0: the LSE is its scaled score
    torch.testing.assert_close(lse[0, 0, 0], (q[0, 0, 0] @ k[0, 0, 0]) * 0.5)
    # zero queries: row i sees i + 1 equal (zero) scores -> ln(i + 1)
    lse0 = orc.lse(torch.zeros_like(q), k, causal=True)
    torch.testing.assert_close(lse0[0, 0], torch.log(torch.arange(1, 7, dtype=torch.float32)))


def test_chunked_equals_whole():
    torch.manual_seed(4)
    q, k, v = torch.randn(2, 8, 70, 32), torch.randn(2, 2, 90, 32), torch.randn(2, 2, 90, 32)
    for causal in (False, True):
        whole = orc.attention(q, k, v, causal=causal)
        for hpc, rpc in ((4, 0), (1, 16), (8, 7)):
            torch.testing.assert_close(orc.attention_chunked(q, k, v, causal=causal, heads_per_chunk=hpc,
                                                             rows_per_chunk=rpc), whole, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("lens_q,lens_k", [([5, 33, 70], [5, 33, 70]), ([64, 0, 17], [64, 0, 17]),
                                           ([8, 16], [40, 16]), ([0, 1, 3], [2, 1, 0])])
def test_varlen_oracle_matches_bruteforce(lens_q, lens_k):
    torch.manual_seed(5)
    hq, hkv, d = 4, 2, 16
    q = torch.randn(sum(lens_q), hq, d)
    k, v = torch.randn(sum(lens_k), hkv, d), torch.randn(sum(lens_k), hkv, d)
    cq = torch.tensor([0] + list(np.cumsum(lens_q)), dtype=torch.int32)
    ck = torch.tensor([0] + list(np.cumsum(lens_k)), dtype=torch.int32)
    out = orc.attention_varlen(q, k, v, cq, ck, causal=True)
    for i in range(len(lens_q)):
        qs = q[cq[i]:cq[i + 1]].transpose(0, 1)[None]
        if qs.shape[2] == 0:
            continue
        ks, vs = k[ck[i]:ck[i + 1]].transpose(0, 1)[None], v[ck[i]:ck[i + 1]].transpose(0, 1)[None]
        ref = orc.attention_f64(qs, ks, vs, causal=True)[0].transpose(1, 0, 2)
        np.testing.assert_allclose(out[cq[i]:cq[i + 1]].numpy(), ref, atol=2e-6, rtol=1e-5)
    assert not torch.isnan(out).any()  # every packed row belongs to a sequence and is written


# ---- FP8 ------------------------------------------------------------------------------------------


@pytest.mark.skipif(orc.FP8_DTYPE is None, reason="torch build lacks float8")
def test_e4m3fn_decode_table_matches_torch():
    codes = torch.arange(256, dtype=torch.uint8)
    got = codes.view(torch.float8_e4m3fn).float().tolist()
    for c in range(256):
        want = orc.e4m3fn_value(c)
        if math.isnan(want):
            assert math.isnan(got[c]), c
        else:
            assert got[c] == want, (c, got[c], want)


@pytest.mark.skipif(orc.FP8_DTYPE is None, reason="torch build lacks float8")
def test_fp8_roundtrip_bounds_and_scale_shape():
    # reference: tests/test_splitk_fp8.py:53-62
    torch.manual_seed(0)
    k = torch.randn(2, 2, 200, 64) * 3
    k8, ks = orc.quantize_kv_fp8(k)
    assert k8.dtype == torch.float8_e4m3fn and ks.shape == (2, 2, 4)
    kd = orc.dequantize_kv_fp8(k8, ks)
    assert ((kd - k).abs() / k.abs().clamp_min(1e-3)).median() < 0.08
    assert (kd - k).abs().max() / k.abs().max() < 0.07


def _e4m3_probe_values() -> np.ndarray:
    """Every finite code, every midpoint between neighbouring magnitudes and the fp32 values
    either side of it, the overflow boundary 464, fp32 subnormals, +-0, +-NaN, and a normal sample."""
    fin = np.array([v for v in (orc.e4m3fn_value(c) for c in range(256)) if not math.isnan(v)], dtype=np.float32)
    mag = np.unique(np.abs(fin)).astype(np.float64)
    mids = ((mag[1:] + mag[:-1]) / 2).astype(np.float32)
    special = np.array([0.0, 448.0, 449.0, 463.99997, 464.0, 464.00003, 480.0, 1e4, np.inf, 1e-40, 2.0 ** -10,
                        2.0 ** -10 * 1.0001, 2.0 ** -9 * 1.5, 2.0 ** -9 * 2.5, np.nan], dtype=np.float32)
    v = np.concatenate([fin, mids, np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(-np.inf)),
                        special])
    v = np.concatenate([v, -v, (np.random.default_rng(0).standard_normal(100000) * 60).astype(np.float32)])
    return v.astype(np.float32)


@pytest.mark.skipif(orc.FP8_DTYPE is None, reason="torch build lacks float8")
def test_e4m3fn_encoder_matches_torch_cast():
    v = _e4m3_probe_values()
    got = orc.e4m3fn_encode(v)
    want = torch.from_numpy(v).to(orc.FP8_DTYPE).view(torch.uint8).numpy()
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(float(v[i]), int(got[i]), int(want[i])) for i in bad[:8]]


def test_e4m3fn_encoder_rounds_to_nearest_even():
    # closed-form checks that do not go through torch: exact codes map to themselves, a midpoint
    # goes to the even neighbour, anything else to the nearer one
    for c in range(256):
        val = orc.e4m3fn_value(c)
        if not math.isnan(val):
            assert orc.e4m3fn_encode(np.float32(val)) == c
    assert orc.e4m3fn_encode(np.float32(1.0625)) == 0x38  # 1 + 1/16: tie of 1.0 (0x38) and 1.125 (0x39)
    assert orc.e4m3fn_encode(np.float32(1.1875)) == 0x3a  # tie of 1.125 (0x39) and 1.25 (0x3a)
    assert orc.e4m3fn_encode(np.float32(2.0 ** -10)) == 0x00  # half the smallest subnormal -> even (zero)
    assert orc.e4m3fn_encode(np.float32(3 * 2.0 ** -10)) == 0x02  # tie of codes 1 and 2
    assert orc.e4m3fn_encode(np.float32(464.0)) == 0x7e and orc.e4m3fn_encode(np.float32(465.0)) == 0x7f
    assert orc.e4m3fn_encode(np.float32(-0.0)) == 0x80 and orc.e4m3fn_encode(np.float32(-np.nan)) == 0xff
    v = (np.random.default_rng(1).standard_normal(20000) * 50).clip(-448, 448).astype(np.float32)
    dec = np.array([orc.e4m3fn_value(int(c)) for c in orc.e4m3fn_encode(v)])
    # within half a step: the step at |x| in [2^e, 2^(e+1)) is 2^(e-3), subnormal step 2^-9
    step = np.where(np.abs(v) < 2.0 ** -6, 2.0 ** -9, 2.0 ** (np.floor(np.log2(np.abs(v) + 1e-30)) - 3))
    assert np.all(np.abs(dec - v) <= step / 2 + 1e-12)


@pytest.mark.skipif(orc.FP8_DTYPE is None, reason="torch build lacks float8")
def test_fp8_quantiser_true_division_matches_torch_chain_on_cpu():
    """scale_div="true" is what the reference's chain gives on the CPU, bit for bit, including
    blocks that hold NaN, +-inf, zeros and a ragged last block."""
    torch.manual_seed(3)
    x = torch.randn(2, 3, 130, 32) * 5
    x[0, 1, 5, 3] = float("nan")
    x[1, 2, 100, 0] = float("inf")
    x[1, 0, 70, 7] = -float("inf")
    x[0, 0, 64:128] = 0.0
    x[1, 1, 3] = -0.0
    nblk = 3
    xf = torch.cat([x, x.new_zeros(2, 3, nblk * 64 - 130, 32)], dim=2).view(2, 3, nblk, 64, 32)
    scale = xf.abs().amax(dim=(-1, -2)).clamp_min(1e-12) / 448.0
    want8 = (xf / scale[..., None, None]).clamp(-448.0, 448.0).to(orc.FP8_DTYPE).view(2, 3, nblk * 64, 32)[:, :, :130]
    got8, got_s = orc.quantize_kv_fp8(x, scale_div="true")
    assert torch.equal(got8.view(torch.uint8), want8.contiguous().view(torch.uint8))
    assert torch.equal(got_s.nan_to_num(nan=-1.0), scale.nan_to_num(nan=-1.0))


def test_fp8_quantiser_reciprocal_scale_is_amax_times_float32_reciprocal():
    torch.manual_seed(4)
    x = torch.rand(1, 2, 256, 16) * 100
    _, s = orc.quantize_kv_fp8(x)
    amax = x.view(1, 2, 4, 64 * 16).abs().amax(-1).numpy().astype(np.float32)
    assert np.array_equal(s.numpy(), amax * (np.float32(1) / np.float32(448)))
    _, s_true = orc.quantize_kv_fp8(x, scale_div="true")
    assert np.array_equal(s_true.numpy(), amax / np.float32(448))


@pytest.mark.skipif(orc.FP8_DTYPE is None, reason="torch build lacks float8")
def test_fp8_scales_equal_blockwise_amax():
    torch.manual_seed(6)
    x = torch.randn(1, 2, 130, 16)
    _, s = orc.quantize_kv_fp8(x)
    xn = x.numpy()
    for h in range(2):
        for blk in range(3):
            amax = np.abs(xn[0, h, blk * 64:(blk + 1) * 64]).max()
            assert s[0, h, blk].item() == pytest.approx(amax / 448.0, rel=2.5e-7)
    # every quantised magnitude respects the E4M3 range and the block's scale
    x8, s = orc.quantize_kv_fp8(x)
    assert x8.float().abs().max() <= 448.0


@pytest.mark.skipif(orc.FP8_DTYPE is None, reason="torch build lacks float8")
def test_fp8_attention_accuracy_vs_fp32():
    # reference: tests/test_splitk_fp8.py:65-74
    torch.manual_seed(0)
    q = torch.randn(2, 4, 8, 64)
    k, v = torch.randn(2, 2, 300, 64), torch.randn(2, 2, 300, 64)
    k8, ks = orc.quantize_kv_fp8(k)
    v8, vs = orc.quantize_kv_fp8(v)
    ref = orc.attention(q, k, v, causal=True)
    out = orc.attention_fp8(q, k8, ks, v8, vs, causal=True)
    assert (out - ref).abs().max() < 5e-2


# ---- split-K --------------------------------------------------------------------------------------


def test_choose_num_splits_known_answers():
    # reference: tests/test_splitk_fp8.py:44-50
    assert orc.choose_num_splits(1, 8, 32768, 1, num_sms=108) == 27
    assert orc.choose_num_splits(64, 32, 32768, 1, num_sms=108) == 1
    assert orc.choose_num_splits(1, 1, 512, 1, num_sms=108) == 2
    assert orc.choose_num_splits(1, 1, 100000, 128, num_sms=108) == 1


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("split_len", [64, 128, 320, 4096])
def test_splitk_combine_is_exact(causal, split_len):
    torch.manual_seed(7)
    q, k, v = torch.randn(1, 4, 4, 32), torch.randn(1, 2, 777, 32), torch.randn(1, 2, 777, 32)
    o, m, l = orc.splitk_partials(q, k, v, causal, None, split_len)
    comb = orc.splitk_combine(o, m, l)
    np.testing.assert_allclose(comb, orc.attention_f64(q, k, v, causal=causal), atol=1e-12, rtol=1e-10)


def test_split_len_alignment():
    # reference: triton_splitk.py:153-154
    assert orc.split_len_for(1000, 3) == 384 and -(-1000 // 384) == 3
    assert orc.split_len_for(777, 8) == 128 and -(-777 // 128) == 7
    assert orc.split_len_for(2048, 1) == 2048


# ---- paged K/V ------------------------------------------------------------------------------------


def _scatter_pages(k, page_size, gen):
    """Dense [B, H, N, D] -> pool [P, H, page_size, D] in a shuffled page order, and its block table."""
    b, h, n, d = k.shape
    cols = -(-n // page_size)
    perm = torch.randperm(b * cols + 3, generator=gen)[:b * cols].view(b, cols)
    pool = torch.randn(b * cols + 3, h, page_size, d, generator=gen)  # unused pages hold garbage
    kp = torch.cat([k, k.new_zeros(b, h, cols * page_size - n, d)], dim=2)
    for bi in range(b):
        for c in range(cols):
            pool[perm[bi, c]] = kp[bi, :, c * page_size:(c + 1) * page_size]
    return pool, perm.to(torch.int32)


@pytest.mark.parametrize("causal", [False, True])
def test_paged_oracle_equals_dense_attention_on_the_scattered_keys(causal):
    gen = torch.Generator().manual_seed(11)
    b, hq, hkv, n, d, ps = 4, 4, 2, 150, 16, 32
    q = torch.randn(b, hq, 3, d, generator=gen)
    k = torch.randn(b, hkv, n, d, generator=gen)
    v = torch.randn(b, hkv, n, d, generator=gen)
    kpool, bt = _scatter_pages(k, ps, gen)
    vpool = torch.zeros_like(kpool)
    for bi in range(b):  # V scattered through the same table
        for c in range(bt.shape[1]):
            seg = v[bi, :, c * ps:(c + 1) * ps]
            vpool[bt[bi, c], :, :seg.shape[1]] = seg
    lens = torch.tensor([150, 0, 33, 64], dtype=torch.int32)
    got = orc.attention_paged(q, kpool, vpool, bt, lens, causal=causal)
    for bi, ln in enumerate(lens.tolist()):
        want = orc.attention(q[bi:bi + 1], k[bi:bi + 1, :, :ln], v[bi:bi + 1, :, :ln], causal=causal)
        torch.testing.assert_close(got[bi:bi + 1], want, atol=1e-6, rtol=1e-6)
    assert torch.all(got[1] == 0)  # no keys -> zeros


@pytest.mark.parametrize("causal", [False, True])
def test_paged_fp8_oracle_equals_dense_fp8_attention(causal):
    """Pages of 64*m keys start on 64-key scale blocks, so scattering a dense FP8 cache's bytes and
    block scales into shuffled pages must reproduce the dense FP8 oracle exactly, per sequence."""
    gen = torch.Generator().manual_seed(13)
    b, hq, hkv, n, d, ps = 3, 4, 2, 200, 16, 128
    q = torch.randn(b, hq, 2, d, generator=gen)
    k8, ks = orc.quantize_kv_fp8(torch.randn(b, hkv, n, d, generator=gen) * 3)
    v8, vs = orc.quantize_kv_fp8(torch.randn(b, hkv, n, d, generator=gen) * 0.01)
    cols, bpp = -(-n // ps), ps // 64
    perm = torch.randperm(b * cols + 2, generator=gen)[:b * cols].view(b, cols)
    npages = b * cols + 2

    def scatter(x8, sc):
        pool = torch.zeros(npages, hkv, ps, d, dtype=torch.uint8)
        spool = torch.rand(npages, hkv, bpp, generator=gen) + 5.0  # unused pages: garbage scales
        xb = torch.cat([x8.view(torch.uint8), torch.zeros(b, hkv, cols * ps - n, d, dtype=torch.uint8)], dim=2)
        scp = torch.cat([sc, torch.zeros(b, hkv, cols * bpp - sc.shape[-1])], dim=2)
        for bi in range(b):
            for c in range(cols):
                pool[perm[bi, c]] = xb[bi, :, c * ps:(c + 1) * ps]
                spool[perm[bi, c]] = scp[bi, :, c * bpp:(c + 1) * bpp]
        return pool.view(x8.dtype), spool

    k8p, ksp = scatter(k8, ks)
    v8p, vsp = scatter(v8, vs)
    lens = torch.tensor([200, 0, 129], dtype=torch.int32)
    got = orc.attention_paged_fp8(q, k8p, ksp, v8p, vsp, perm.to(torch.int32), lens, causal=causal)
    for bi, ln in enumerate(lens.tolist()):
        want = orc.attention(q[bi:bi + 1], orc.dequantize_kv_fp8(k8, ks)[bi:bi + 1, :, :ln],
                             orc.dequantize_kv_fp8(v8, vs)[bi:bi + 1, :, :ln], causal=causal)
        assert torch.equal(got[bi:bi + 1], want)
    assert torch.all(got[1] == 0)


def test_paged_oracle_out_of_pool_pages_read_as_zero_keys():
    gen = torch.Generator().manual_seed(12)
    k = torch.randn(1, 1, 96, 8, generator=gen)
    kpool, bt = _scatter_pages(k, 32, gen)
    bad = bt.clone()
    bad[0, 1] = kpool.shape[0] + 7
    got = orc.paged_gather(kpool, bad, 96, 0)
    want = k[0].clone()
    want[:, 32:64] = 0
    assert torch.equal(got, want)
    bad[0, 2] = -1
    assert torch.all(orc.paged_gather(kpool, bad, 96, 0)[:, 64:] == 0)
