"""FP8 E4M3 KV-cache attention on the HIP split-K kernel vs the fp32 oracle run on the
dequantised K/V (reference: tests/test_splitk_fp8.py:77-86)."""
import pytest
import torch

import fused_attn
from helpers import FP8_TOL, announce, max_err, randn
from oracle import attention_oracle as orc

pytestmark = pytest.mark.gpu


def test_fp8_kernel_matches_dequantized_oracle_prefill_shaped():
    """The reference's own GPU case: n_q=128, causal, fp16 q."""
    announce("fp8 reference case")
    torch.manual_seed(0)
    q = randn(2, 8, 128, 64, dtype=torch.float16)
    k, v = randn(2, 2, 1024, 64), randn(2, 2, 1024, 64)
    k8, ks = fused_attn.quantize_kv_fp8(k)
    v8, vs = fused_attn.quantize_kv_fp8(v)
    out = fused_attn.attention_fp8_triton(q, k8, ks, v8, vs, causal=True)
    ref = orc.attention_fp8(q.cpu(), k8.cpu(), ks.cpu(), v8.cpu(), vs.cpu(), causal=True)
    assert out.dtype == q.dtype
    assert max_err(out, ref) <= FP8_TOL


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("b,h_q,h_kv,n_q,n_k,d", [(2, 8, 2, 1, 1000, 128), (1, 4, 4, 3, 4096, 64),
                                                  (3, 16, 2, 16, 2100, 128), (1, 4, 1, 200, 333, 128),
                                                  (2, 8, 2, 4, 1300, 256)])
@pytest.mark.parametrize("split_len", [None, 64, 256])
def test_fp8_matches_oracle(b, h_q, h_kv, n_q, n_k, d, causal, dtype, split_len):
    announce(f"fp8 b={b} hq={h_q} hkv={h_kv} nq={n_q} nk={n_k} d={d} causal={causal} {dtype} split={split_len}")
    torch.manual_seed(0)
    q = randn(b, h_q, n_q, d, dtype=dtype)
    k, v = randn(b, h_kv, n_k, d), randn(b, h_kv, n_k, d)
    k8, ks = fused_attn.quantize_kv_fp8(k)
    v8, vs = fused_attn.quantize_kv_fp8(v)
    out = fused_attn.attention_fp8(q, k8, ks, v8, vs, causal=causal, split_len=split_len)
    ref = orc.attention_fp8(q.cpu(), k8.cpu(), ks.cpu(), v8.cpu(), vs.cpu(), causal=causal)
    assert max_err(out, ref) <= FP8_TOL


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fp8_decode_is_exact_for_every_code(dtype):
    """One key: the output row is exactly the decoded V row times its power-of-two scale.
    Covers all 254 finite E4M3 codes through the in-kernel conversion."""
    announce(f"fp8 all codes {dtype}")
    codes = torch.arange(256, dtype=torch.uint8)
    codes[codes == 0x7F] = 0
    codes[codes == 0xFF] = 0
    v8 = codes.view(torch.float8_e4m3fn).reshape(1, 2, 1, 128).cuda()
    k8 = torch.zeros_like(v8)
    ks = torch.ones(1, 2, 1, device="cuda")
    vs = torch.tensor([[[0.25], [2.0]]], device="cuda")
    q = randn(1, 2, 1, 128, dtype=dtype)
    out = fused_attn.attention_fp8(q, k8, ks, v8, vs)
    want = (v8.float() * vs[..., None]).to(dtype)
    assert torch.equal(out, want)


@pytest.mark.parametrize("split_len", [128, None])
def test_benchmark_fp8_decode_workload(split_len):
    """B=16, Hq=64, Hkv=8, n_q=1, n_k=65536, D=128; K/V N(0,1) fp32 quantised per 64-key block.
    At 128-key partitions and at the op's default partitions (4096 keys here), the path a caller
    of attention_fp8 without split_len takes."""
    announce(f"benchmark fp8 decode split={split_len}")
    gen = torch.Generator(device="cuda").manual_seed(0)
    q = randn(16, 64, 1, 128, dtype=torch.bfloat16, gen=gen)
    k8, ks = fused_attn.quantize_kv_fp8(randn(16, 8, 65536, 128, gen=gen))
    v8, vs = fused_attn.quantize_kv_fp8(randn(16, 8, 65536, 128, gen=gen))
    out = fused_attn.attention_fp8(q, k8, ks, v8, vs, split_len=split_len)
    ref = torch.empty(16, 64, 1, 128, device="cuda")
    for bi in range(16):  # oracle per batch element on the dequantised cache
        ref[bi:bi + 1] = orc.attention_fp8(q[bi:bi + 1], k8[bi:bi + 1], ks[bi:bi + 1], v8[bi:bi + 1],
                                           vs[bi:bi + 1])
    err = max_err(out, ref)
    print(f"max_abs_err={err:.3e}", flush=True)
    assert err <= FP8_TOL


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("vmag", ["small", "large", "mixed"])
@pytest.mark.parametrize("split_len", [128, 2048])
def test_fp8_value_magnitudes_keep_relative_accuracy(vmag, dtype, split_len):
    """V caches of small (1e-3) and large (1e3) magnitude, and both in alternating 64-key blocks.  The kernel
    rounds P times a V scale ratio of at most 2 to q's 16-bit type (the accumulator is kept in units of a
    recent block's V scale, restored in fp32 at the end), so with fp16 q small V blocks do not fall into
    fp16's subnormal range.  Checked by the error relative to the output's magnitude, against the oracle
    on the dequantised cache (the absolute 5e-2 bar cannot see a relative loss on outputs of size 1e-3)."""
    announce(f"fp8 magnitudes {vmag} {dtype} split={split_len}")
    torch.manual_seed(7)
    b, hq, hkv, nq, nk, d = 2, 8, 2, 4, 4000, 128
    q = randn(b, hq, nq, d, dtype=dtype)
    k = randn(b, hkv, nk, d)
    v = randn(b, hkv, nk, d)
    if vmag == "small":
        v = v * 1e-3
    elif vmag == "large":
        v = v * 1e3
    else:  # blocks of 64 keys alternate between 1e-3 and 1e3
        blk = (torch.arange(nk, device=v.device) // 64) % 2
        v = v * torch.where(blk == 0, 1e-3, 1e3)[None, None, :, None]
    k8, ks = fused_attn.quantize_kv_fp8(k)
    v8, vs = fused_attn.quantize_kv_fp8(v)
    out = fused_attn.attention_fp8(q, k8, ks, v8, vs, causal=True, split_len=split_len)
    ref = orc.attention_fp8(q.cpu(), k8.cpu(), ks.cpu(), v8.cpu(), vs.cpu(), causal=True).to(out.device)
    rel = ((out.float() - ref).abs().max() / ref.abs().max()).item()
    print(f"{vmag} {dtype}: max relative error {rel:.3e}", flush=True)
    assert torch.isfinite(out).all()
    assert rel <= 1e-2


def test_fp8_lse_matches_oracle_on_dequantized_keys():
    announce("fp8 lse")
    torch.manual_seed(8)
    q = randn(2, 8, 3, 128, dtype=torch.bfloat16)
    k8, ks = fused_attn.quantize_kv_fp8(randn(2, 2, 1500, 128))
    v8, vs = fused_attn.quantize_kv_fp8(randn(2, 2, 1500, 128))
    out, lse = fused_attn.attention_fp8(q, k8, ks, v8, vs, causal=True, split_len=256, return_lse=True)
    kd = orc.dequantize_kv_fp8(k8.cpu(), ks.cpu())
    ref = orc.lse(q.cpu(), kd, causal=True).to(lse.device)
    assert (lse - ref).abs().max().item() < 2.0 ** -8
    assert max_err(out, orc.attention_fp8(q.cpu(), k8.cpu(), ks.cpu(), v8.cpu(), vs.cpu(), causal=True)) <= FP8_TOL


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("n_q", [1, 16])
@pytest.mark.parametrize("split_len", [128, 2048, None])
def test_fp8_small_v_blocks_carrying_the_attention_beside_large_v_blocks(dtype, n_q, split_len):
    """64-key blocks alternate between V of magnitude 1e-3 and 1e3, and the keys of the large-V blocks
    score about 28 below the others, so the small-V blocks carry the output while a large-V block
    (1e6 times the scale) shares every partition and workgroup.  A kernel that folded a ratio to the
    largest V scale of its keys into P before P's 16-bit rounding would push P times 1e-6 into fp16's
    subnormal range here; the reference multiplies each block's P*V by v_scale in fp32 (fp8.py:116).
    Checked at a relative bar against the oracle on the dequantised cache."""
    announce(f"fp8 small-V blocks beside large-V blocks {dtype} n_q={n_q} split={split_len}")
    gen = torch.Generator(device="cuda").manual_seed(41)
    b, hq, hkv, nk, d = 2, 16, 2, 4096, 128
    g = hq // hkv
    # every query row of a kv group leans along that group's unit direction u (q.u = 8 +- 1), and the
    # keys of the large-V blocks point along -40 u: their scores sit near -28, the others' near 0
    u = randn(b, hkv, 1, d, gen=gen)
    u = u / u.norm(dim=-1, keepdim=True)
    q = (randn(b, hkv, g * n_q, d, gen=gen) + 8.0 * u).view(b, hq, n_q, d)
    k = randn(b, hkv, nk, d, gen=gen)
    v = randn(b, hkv, nk, d, gen=gen)
    large = ((torch.arange(nk, device="cuda") // 64) % 2 == 1)[None, None, :, None]
    k = torch.where(large, -40.0 * u + 0.1 * k, k)
    v = v * torch.where(large, 1e3, 1e-3)
    q = q.to(dtype)
    k8, ks = fused_attn.quantize_kv_fp8(k)
    v8, vs = fused_attn.quantize_kv_fp8(v)
    out = fused_attn.attention_fp8(q, k8, ks, v8, vs, split_len=split_len)
    ref = orc.attention_fp8(q, k8, ks, v8, vs)
    # the small-V blocks carry the output: it is of their magnitude, not the large blocks'
    assert ref.abs().max().item() < 1e-2
    rel = ((out.float() - ref).abs().max() / ref.abs().max()).item()
    print(f"max relative error {rel:.3e} |ref|max={ref.abs().max().item():.3e}", flush=True)
    assert torch.isfinite(out).all()
    assert rel <= 1e-2
