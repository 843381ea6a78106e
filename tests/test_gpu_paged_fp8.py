"""FP8 (e4m3fn) paged K/V pools on the HIP split-K kernel.

The reference's FP8 decode path (fused_attn/fp8.py:59-147) reads a dense cache; paged K/V is
its roadmap item (README.md:224) with no reference code.  An FP8 pool here is what
``quantize_kv_fp8`` writes for a [num_pages, Hkv, page_size, D] cache: e4m3fn bytes plus fp32
64-key block scales [num_pages, Hkv, page_size / 64].  Two checks, as for 16-bit pools: the fp32
oracle on each sequence's dequantised gathered keys (the reference's FP8 bar, 5e-2, judged on the
dequantised K/V as tests/test_splitk_fp8.py:85 does), and bit equality with the dense FP8 split-K
kernel on the same bytes, scales and partitions."""
import pytest
import torch

import fused_attn
from helpers import FP8_TOL, announce, max_err, randn
from oracle import attention_oracle as orc

pytestmark = pytest.mark.gpu


def _fp8_dense_and_paged(b, hq, hkv, nq, n, d, page, dtype, lens=None, seed=0, extra=3, v_mag=None):
    gen = torch.Generator(device="cuda").manual_seed(seed)
    q = randn(b, hq, nq, d, dtype=dtype, gen=gen)
    k = randn(b, hkv, n, d, gen=gen)
    v = randn(b, hkv, n, d, gen=gen)
    if v_mag is not None:  # per-64-key-block magnitudes of V (block scales far apart)
        nblk = -(-n // 64)
        mags = v_mag[torch.arange(b * hkv * nblk, device="cuda") % len(v_mag)].view(b, hkv, nblk)
        v = v * mags.repeat_interleave(64, dim=-1)[..., :n, None]
    k8, ks = fused_attn.quantize_kv_fp8(k)
    v8, vs = fused_attn.quantize_kv_fp8(v)
    cpu_gen = torch.Generator().manual_seed(seed)
    pools = fused_attn.paged_from_dense_fp8(k8, ks, v8, vs, page, seqlens=lens, extra_pages=extra, generator=cpu_gen)
    return q, (k8, ks, v8, vs), pools


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("page", [64, 128, 256])
@pytest.mark.parametrize("nq,causal", [(1, False), (4, True), (20, True)])
def test_paged_fp8_matches_oracle(dtype, d, page, nq, causal):
    announce(f"paged fp8 oracle {dtype} d={d} page={page} nq={nq} causal={causal}")
    lens = [300, 0, 1000, 64]
    q, _, (kc, vc, ksp, vsp, bt, sl) = _fp8_dense_and_paged(4, 8, 2, nq, 1000, d, page, dtype, lens=lens)
    out = fused_attn.attention_paged(q, kc, vc, bt, sl, causal=causal, max_seqlen_k=1000, split_len=128,
                                     k_scale=ksp, v_scale=vsp)
    torch.cuda.synchronize()
    ref = orc.attention_paged_fp8(q, kc.cpu(), ksp.cpu(), vc.cpu(), vsp.cpu(), bt, sl, causal=causal)
    assert out.shape == q.shape and out.dtype == dtype and not torch.isnan(out).any()
    err = max_err(out, ref)
    print(f"max_abs_err={err:.3e}", flush=True)
    assert err <= FP8_TOL
    assert torch.all(out[1] == 0)  # zero-length sequence


@pytest.mark.parametrize("split_len", [64, 128, 512, None])
@pytest.mark.parametrize("nq,causal", [(1, False), (16, True), (20, True)])  # 1, 2 and 4 waves
def test_paged_fp8_is_bit_identical_to_dense_fp8(split_len, nq, causal):
    """Equal lengths, pages on 64-key blocks: the paged kernel equals the dense FP8 split-K kernel
    bit for bit (same bytes, same block scales, same partitions)."""
    announce(f"paged fp8 == dense fp8 split_len={split_len} nq={nq} causal={causal}")
    q, (k8, ks, v8, vs), (kc, vc, ksp, vsp, bt, sl) = _fp8_dense_and_paged(3, 16, 4, nq, 777, 128, 128,
                                                                           torch.bfloat16)
    sk = split_len or fused_attn.ops.default_split_len(nq, 777, 3, 4, 4)
    dense = fused_attn.attention_fp8(q, k8, ks, v8, vs, causal=causal, split_len=sk)
    paged = fused_attn.attention_paged(q, kc, vc, bt, sl, causal=causal, split_len=sk, k_scale=ksp, v_scale=vsp)
    assert torch.equal(dense, paged)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_paged_fp8_block_scales_far_apart(dtype):
    """V blocks of magnitudes 1e-3 .. 1e3 (block scales six decades apart): the per-workgroup V
    reference scale taken over the pages must equal the dense kernel's, and the result must meet the
    bar relative to the output's own magnitude."""
    announce(f"paged fp8 far-apart scales {dtype}")
    mags = torch.tensor([1e-3, 1.0, 1e3, 0.05, 30.0], device="cuda")
    q, (k8, ks, v8, vs), (kc, vc, ksp, vsp, bt, sl) = _fp8_dense_and_paged(2, 8, 2, 1, 2048, 128, 256, dtype,
                                                                           v_mag=mags)
    dense = fused_attn.attention_fp8(q, k8, ks, v8, vs, split_len=512)
    paged = fused_attn.attention_paged(q, kc, vc, bt, sl, split_len=512, k_scale=ksp, v_scale=vsp)
    assert torch.equal(dense, paged)
    ref = orc.attention_paged_fp8(q, kc.cpu(), ksp.cpu(), vc.cpu(), vsp.cpu(), bt, sl)
    err = (paged.float().cpu() - ref).abs().max().item()
    mag = ref.abs().max().item()
    print(f"max_abs_err={err:.3e} (|ref| max {mag:.3e})", flush=True)
    assert err <= FP8_TOL * max(1.0, mag) * 2 ** -3


def test_paged_fp8_ragged_lengths_bit_identical_per_sequence():
    announce("paged fp8 ragged per-sequence")
    lens = [1, 129, 640, 0, 1000, 64, 65]
    q, (k8, ks, v8, vs), (kc, vc, ksp, vsp, bt, sl) = _fp8_dense_and_paged(len(lens), 8, 8, 1, 1000, 64, 64,
                                                                           torch.float16, lens=lens)
    paged = fused_attn.attention_paged(q, kc, vc, bt, sl, split_len=128, k_scale=ksp, v_scale=vsp)
    for b, n in enumerate(lens):
        if n == 0:
            assert torch.all(paged[b] == 0)
            continue
        nb = -(-n // 64)
        dense = fused_attn.attention_fp8(q[b:b + 1], k8[b:b + 1, :, :n].contiguous(), ks[b:b + 1, :, :nb].contiguous(),
                                         v8[b:b + 1, :, :n].contiguous(), vs[b:b + 1, :, :nb].contiguous(),
                                         split_len=128)
        assert torch.equal(dense, paged[b:b + 1]), b


def test_paged_fp8_out_of_pool_entries_read_as_zero_keys():
    announce("paged fp8 out-of-pool entries")
    q, _, (kc, vc, ksp, vsp, bt, sl) = _fp8_dense_and_paged(2, 4, 2, 1, 512, 64, 128, torch.bfloat16)
    bad = bt.clone()
    bad[0, 1] = kc.shape[0] + 100
    bad[1, 3] = -5
    out = fused_attn.attention_paged(q, kc, vc, bad, sl, split_len=128, k_scale=ksp, v_scale=vsp)
    ref = orc.attention_paged_fp8(q, kc.cpu(), ksp.cpu(), vc.cpu(), vsp.cpu(), bad, sl)
    assert max_err(out, ref) <= FP8_TOL


def test_paged_fp8_pool_views_and_scale_dtypes():
    """A [num_pages, page_size, Hkv, D] pool passed as a transposed view, and fp16 scales, give the
    same bits."""
    announce("paged fp8 pool views")
    q, _, (kc, vc, ksp, vsp, bt, sl) = _fp8_dense_and_paged(2, 8, 2, 1, 500, 128, 64, torch.bfloat16)
    ref = fused_attn.attention_paged(q, kc, vc, bt, sl, split_len=128, k_scale=ksp, v_scale=vsp)
    kc_t = kc.view(torch.uint8).transpose(1, 2).contiguous().transpose(1, 2).view(kc.dtype)
    vc_t = vc.view(torch.uint8).transpose(1, 2).contiguous().transpose(1, 2).view(vc.dtype)
    assert not kc_t.is_contiguous()
    assert torch.equal(fused_attn.attention_paged(q, kc_t, vc_t, bt, sl, split_len=128, k_scale=ksp, v_scale=vsp),
                       ref)
    # scales that are exactly representable in fp16 convert back to the same fp32 words
    k16, v16 = ksp.half(), vsp.half()
    ref16 = fused_attn.attention_paged(q, kc, vc, bt, sl, split_len=128, k_scale=k16.float(), v_scale=v16.float())
    assert torch.equal(fused_attn.attention_paged(q, kc, vc, bt, sl, split_len=128, k_scale=k16, v_scale=v16), ref16)


def test_paged_fp8_decode_cache_bit_identical_to_dense():
    """A large FP8 cache (B=4 Hq=64 Hkv=8, 65536 keys in 64-key pages, shuffled): the paged kernel
    equals the dense FP8 kernel at 128-key and at the default partitions."""
    announce("paged fp8 decode cache B=4 Hq=64 Hkv=8 n_k=65536")
    b, hq, hkv, n, d = 4, 64, 8, 65536, 128
    gen = torch.Generator(device="cuda").manual_seed(7)
    q = randn(b, hq, 1, d, dtype=torch.bfloat16, gen=gen)
    k8, ks = fused_attn.quantize_kv_fp8(randn(b, hkv, n, d, dtype=torch.bfloat16, gen=gen))
    v8, vs = fused_attn.quantize_kv_fp8(randn(b, hkv, n, d, dtype=torch.bfloat16, gen=gen))
    kc, vc, ksp, vsp, bt, sl = fused_attn.paged_from_dense_fp8(k8, ks, v8, vs, 64,
                                                               generator=torch.Generator().manual_seed(7))
    for split_len in (128, fused_attn.ops.default_split_len(1, n, b, hkv, hq // hkv)):
        dense = fused_attn.attention_fp8(q, k8, ks, v8, vs, split_len=split_len)
        paged = fused_attn.attention_paged(q, kc, vc, bt, sl, split_len=split_len, k_scale=ksp, v_scale=vsp)
        assert torch.equal(dense, paged), split_len
