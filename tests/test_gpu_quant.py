"""The fused HIP FP8 KV quantiser vs the reference's torch chain on the GPU, bit for bit.

The reference quantises with a torch op chain (fused_attn/fp8.py:31-45); its bytes and
scales on the GPU are the target.  The same inputs also go through the numpy oracle
(reciprocal scale, table-driven e4m3fn rounding), which pins the chain independently."""
import numpy as np
import pytest
import torch

import fused_attn
from fused_attn import _hip, fp8
from helpers import FP8_TOL, announce, max_err, randn
from oracle import attention_oracle as orc

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(orc.FP8_DTYPE is None, reason="torch build lacks float8")]


def _bytes(x8: torch.Tensor) -> torch.Tensor:
    return x8.view(torch.uint8).cpu()


def _same_scales(a: torch.Tensor, b: torch.Tensor) -> bool:
    a, b = a.cpu(), b.cpu()
    return torch.equal(a.isnan(), b.isnan()) and torch.equal(a.nan_to_num(nan=0.0), b.nan_to_num(nan=0.0))


def _check_against_chain_and_oracle(x: torch.Tensor, oracle: bool = True):
    got8, got_s = _hip.quantize_kv_fp8(x)
    torch.cuda.synchronize()
    want8, want_s = fp8._quantize_kv_fp8_torch(x)  # the reference's chain, on the GPU
    assert got8.dtype == orc.FP8_DTYPE and got8.shape == x.shape and got8.is_contiguous()
    assert got_s.dtype == torch.float32 and got_s.shape == want_s.shape
    assert _same_scales(got_s, want_s)
    gb, wb = _bytes(got8), _bytes(want8)
    bad = (gb != wb).nonzero()
    assert bad.numel() == 0, f"{bad.shape[0]} bytes differ, first at {bad[0].tolist()}"
    if oracle:
        # the oracle runs on the host, whose invalid operations (inf / inf) make NaNs of the
        # other sign: compare NaN codes (S.1111.111) without their sign bit
        o8, o_s = orc.quantize_kv_fp8(x.cpu())
        assert _same_scales(got_s, o_s)
        ob = _bytes(o8)
        nan_g, nan_o = (gb & 0x7F) == 0x7F, (ob & 0x7F) == 0x7F
        assert torch.equal(nan_g, nan_o) and torch.equal(gb[~nan_g], ob[~nan_o])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("d", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("n", [1, 63, 64, 65, 200])
def test_quantiser_bits_equal_torch_chain(dtype, d, n):
    announce(f"quantize {dtype} d={d} n={n}")
    gen = torch.Generator(device="cuda").manual_seed(d * 1000 + n)
    x = (randn(2, 3, n, d, gen=gen) * 4).to(dtype)
    _check_against_chain_and_oracle(x)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_quantiser_special_values(dtype):
    """NaN, +-inf, -0, all-zero blocks, values that become e4m3 subnormals, and exact rounding
    ties: a block whose amax is 448 has scale 448 * fl(1/448) == 1, so x / scale == x and
    every midpoint between neighbouring e4m3 values reaches the conversion unchanged."""
    announce(f"quantize special values {dtype}")
    d = 64
    x = torch.randn(1, 2, 6 * 64, d) * 3
    x[0, 0, 5, 3] = float("nan")  # block 0 of head 0: NaN everywhere
    x[0, 0, 64 + 7, 0] = float("inf")  # block 1: inf/inf = NaN at that element, finite/inf = +-0
    x[0, 0, 128 + 9, 1] = -float("inf")
    x[0, 0, 192:256] = 0.0  # block 3: all zeros -> scale 1e-12 / 448
    x[0, 0, 200, 5] = -0.0
    x[0, 0, 256:320] *= 1e-3  # block 4: tiny values, many e4m3 subnormals after scaling
    # head 1: blocks whose amax is 448 hold the e4m3 midpoints (and their neighbours) that the
    # dtype represents exactly
    fin = np.array([orc.e4m3fn_value(c) for c in range(0x7f)], dtype=np.float64)
    mids = (fin[1:] + fin[:-1]) / 2
    vals = np.concatenate([fin, mids, -fin, -mids]).astype(np.float32)
    t = torch.from_numpy(vals).to(dtype)
    vals = t[t.float() == torch.from_numpy(vals)].float()  # drop what the dtype would round
    if dtype == torch.float32:  # fp32 also carries the neighbours of each midpoint
        m = torch.from_numpy(mids.astype(np.float32))
        vals = torch.cat([vals, torch.nextafter(m, m + 1), torch.nextafter(m, m - 1)])
    per_block = 64 * d - 1
    nb = 5
    flat = torch.zeros(nb * 64 * d)
    for b in range(nb):
        chunk = vals[b * per_block:(b + 1) * per_block]
        flat[b * 64 * d] = 448.0
        flat[b * 64 * d + 1:b * 64 * d + 1 + chunk.numel()] = chunk
    assert vals.numel() <= nb * per_block
    x[0, 1, :nb * 64] = flat.view(nb * 64, d)
    x = x.to(dtype).cuda()
    _check_against_chain_and_oracle(x)
    s = _hip.quantize_kv_fp8(x)[1].cpu()
    assert torch.isnan(s[0, 0, 0]) and torch.all(s[0, 1, :nb] == 1.0)


def test_quantiser_strided_views():
    announce("quantize strided views")
    torch.manual_seed(0)
    base = randn(2, 100, 4, 128, dtype=torch.bfloat16)  # [B, N, H, D] storage
    x = base.transpose(1, 2)
    assert not x.is_contiguous()
    _check_against_chain_and_oracle(x)
    odd = randn(2 * 4 * 70 * 64 + 3, dtype=torch.float16)[3:].view(2, 4, 70, 64)  # 6 bytes off alignment
    assert odd.data_ptr() % 16 != 0
    _check_against_chain_and_oracle(odd)
    padded = randn(1, 2, 90, 80, dtype=torch.float32)[..., :64]  # row stride 80 floats
    _check_against_chain_and_oracle(padded)


def test_quantiser_routing_and_empty_inputs(monkeypatch):
    announce("quantize routing")
    x = randn(1, 2, 0, 64, dtype=torch.bfloat16)
    x8, s = fused_attn.quantize_kv_fp8(x)
    assert x8.shape == (1, 2, 0, 64) and s.shape == (1, 2, 0)
    x = randn(0, 2, 10, 64, dtype=torch.bfloat16)
    assert fused_attn.quantize_kv_fp8(x)[1].shape == (0, 2, 1)
    # GPU tensors take the HIP kernel; the forced reference backend takes the torch chain
    calls = []
    real = _hip.quantize_kv_fp8
    monkeypatch.setattr(_hip, "quantize_kv_fp8", lambda t: calls.append(1) or real(t))
    x = randn(1, 2, 70, 64, dtype=torch.bfloat16)
    a8, a_s = fused_attn.quantize_kv_fp8(x)
    assert calls == [1]
    monkeypatch.setenv("FUSED_ATTN_BACKEND", "reference")
    b8, b_s = fused_attn.quantize_kv_fp8(x)
    assert calls == [1]
    assert torch.equal(_bytes(a8), _bytes(b8)) and _same_scales(a_s, b_s)
    # a head dim the kernel does not take uses the chain on the GPU
    monkeypatch.delenv("FUSED_ATTN_BACKEND")
    y = randn(1, 1, 70, 48, dtype=torch.bfloat16)
    assert fused_attn.quantize_kv_fp8(y)[0].shape == y.shape and calls == [1]


def test_quantiser_decode_cache_size_and_attention():
    """The decode cache size (B=16, Hkv=8, N=65536, D=128, bf16) bit for bit, then FP8 attention
    over the HIP-quantised cache within the FP8 bar of the oracle."""
    announce("quantize decode cache 16x8x65536x128")
    gen = torch.Generator(device="cuda").manual_seed(0)
    k = randn(16, 8, 65536, 128, dtype=torch.bfloat16, gen=gen)
    _check_against_chain_and_oracle(k, oracle=False)
    v = randn(4, 8, 4096, 128, dtype=torch.bfloat16, gen=gen)
    kk = randn(4, 8, 4096, 128, dtype=torch.bfloat16, gen=gen)
    q = randn(4, 32, 1, 128, dtype=torch.bfloat16, gen=gen)
    k8, ks = fused_attn.quantize_kv_fp8(kk)
    v8, vs = fused_attn.quantize_kv_fp8(v)
    out = fused_attn.attention_fp8(q, k8, ks, v8, vs)
    ref = orc.attention_fp8(q.cpu(), k8.cpu(), ks.cpu(), v8.cpu(), vs.cpu())
    assert max_err(out, ref) <= FP8_TOL
