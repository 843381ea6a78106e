"""ORACLE — test infrastructure, not product code.

A restatement of the reference's attention algorithm used only to check the
HIP kernels.  Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
CPU-baseline leg may import it, and only as the checker (or the timed CPU
baseline), never as the path that produces the library's results.

Two independent formulations, so that each pins the other:

* torch fp32 (runs on any device; chunked variants for large shapes) following
  the reference's op order: fused_attn/reference.py:16-95,
  fused_attn/fp8.py:26-56, fused_attn/triton_splitk.py:90-137,153-154;
* numpy float64 brute force (explicit per-row loops, no matmul library), used
  on small inputs only;
* the FP8 quantiser in numpy float32 with a table-driven e4m3fn encoder.

How each function is pinned (checked in tests/test_oracle.py):
  attention            vs torch.nn.functional.scaled_dot_product_attention
                       (non-causal and square causal), vs SDPA with an explicit
                       bottom-right mask, vs the float64 brute force, and vs
                       closed forms (one visible key -> that value row; no
                       visible key -> zeros; equal scores -> mean of V).
  expand_kv / GQA      vs repeat_interleave + SDPA (tests/test_correctness.py:42-50
                       in the reference).
  lse                  vs the float64 brute force lse_f64 (-inf rows included), and closed
                       forms: one visible key -> its scaled score; n equal scores -> s + ln n.
  attention_varlen     vs per-sequence dense attention and the brute force,
                       including zero-length sequences.
  e4m3fn_encode        vs torch's float8_e4m3fn cast on every code, every
                       midpoint between neighbouring codes and its fp32
                       neighbours, subnormals, +-0, NaN and values past 448;
                       every encoded byte decodes (closed form) to within half
                       a step of its input.
  quantize_kv_fp8      vs the reference's torch chain on the CPU bit for bit
                       (scale_div="true"), vs the reference's round-trip bounds
                       and scale shape (tests/test_splitk_fp8.py:53-62), and
                       vs a per-block recomputation of the scales.
  splitk_* / combine   vs unsplit attention (the combine is an exact identity,
                       triton_splitk.py:11-16), for several split lengths.
  choose_num_splits    known answers 27, 1, 2, 1 (tests/test_splitk_fp8.py:44-50).
  attention_paged      vs dense attention on the K/V that were scattered into randomly
                       ordered pages (ragged lengths, zero-length sequences, causal), and a
                       page index outside the pool contributes zero keys.

tests/test_oracle_mutants.py plants plausible mistakes in copies of this module (mask offsets,
dropped scale, swapped operands, wrong head mapping, rounding rules, constants, combine terms)
and checks that the pins above fail on each of them.
"""
from __future__ import annotations

import math
from typing import Optional

import numpy as np
import torch

LOG2E = 1.4426950408889634
QBLOCK = 64
E4M3_MAX = 448.0
FP8_DTYPE = getattr(torch, "float8_e4m3fn", None)


# ---------------------------------------------------------------------------------------------
# dense / varlen attention, torch fp32 (fused_attn/reference.py:16-95)
# ---------------------------------------------------------------------------------------------


def expand_kv(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    """[B, Hkv, N, D] -> [B, Hkv*n_rep, N, D], q-head h reads kv-head h // n_rep (reference.py:16-21)."""
    return x if n_rep == 1 else torch.repeat_interleave(x, n_rep, dim=1)


def causal_mask(n_q: int, n_k: int, device=None) -> torch.Tensor:
    """True where key j is visible to query i: j <= i + (n_k - n_q) (reference.py:24-33)."""
    i = torch.arange(n_q, device=device).view(-1, 1)
    j = torch.arange(n_k, device=device).view(1, -1)
    return (j - i) <= (n_k - n_q)


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False,
              scale: Optional[float] = None, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """fp32 attention in the reference's op order (reference.py:36-62).

    Returns fp32 unless ``out_dtype`` is given (the reference casts to q.dtype;
    the kernels are judged against the fp32 result before that cast)."""
    h_q, n_q, d = q.shape[1], q.shape[2], q.shape[3]
    h_kv, n_k = k.shape[1], k.shape[2]
    assert h_q % h_kv == 0
    qf, kf, vf = q.float(), expand_kv(k.float(), h_q // h_kv), expand_kv(v.float(), h_q // h_kv)
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    s = torch.matmul(qf, kf.transpose(-1, -2)) * scale
    if causal:
        s = s.masked_fill(~causal_mask(n_q, n_k, device=s.device), float("-inf"))
    p = torch.nan_to_num(torch.softmax(s, dim=-1), nan=0.0)
    o = torch.matmul(p, vf)
    return o if out_dtype is None else o.to(out_dtype)


def lse(q: torch.Tensor, k: torch.Tensor, causal: bool = False, scale: Optional[float] = None) -> torch.Tensor:
    """Natural-log sum of exp of the scaled scores, fp32 [B, Hq, Nq]: the log of the softmax
    denominator of ``attention`` (the quantity the reference's Triton kernel writes with
    WRITE_LSE, fused_attn/triton_fwd.py:169-172).  Rows with no visible key give -inf."""
    h_q, n_q, d = q.shape[1], q.shape[2], q.shape[3]
    h_kv, n_k = k.shape[1], k.shape[2]
    kf = expand_kv(k.float(), h_q // h_kv)
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    s = torch.matmul(q.float(), kf.transpose(-1, -2)) * scale
    if causal:
        s = s.masked_fill(~causal_mask(n_q, n_k, device=s.device), float("-inf"))
    return torch.logsumexp(s, dim=-1)


def attention_chunked(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False,
                      scale: Optional[float] = None, heads_per_chunk: int = 0,
                      rows_per_chunk: int = 0) -> torch.Tensor:
    """``attention`` evaluated per (batch, kv-head group[, query rows]) to bound the score-matrix memory.

    Attention is independent per batch element and per query row, so the result
    equals ``attention`` on the whole tensors (up to matmul blocking order)."""
    b, h_q, n_q, d = q.shape
    h_kv, n_k = k.shape[1], k.shape[2]
    g = h_q // h_kv
    heads_per_chunk = heads_per_chunk or g
    rows_per_chunk = rows_per_chunk or n_q
    out = torch.empty((b, h_q, n_q, d), dtype=torch.float32, device=q.device)
    for bi in range(b):
        for h0 in range(0, h_q, heads_per_chunk):
            h1 = min(h_q, h0 + heads_per_chunk)
            kv0, kv1 = h0 // g, (h1 - 1) // g + 1
            kk, vv = k[bi:bi + 1, kv0:kv1], v[bi:bi + 1, kv0:kv1]
            for r0 in range(0, n_q, rows_per_chunk):
                r1 = min(n_q, r0 + rows_per_chunk)
                qq = q[bi:bi + 1, h0:h1, r0:r1]
                # rows r0..r1 of an n_q-row causal problem: keep the bottom-right alignment by
                # giving the slice its true row offset through the key range it may see
                if causal:
                    qpad_rows = n_q - r1  # rows after the slice
                    # queries r0..r1 see keys j <= i + (n_k - n_q); as a standalone problem with
                    # n_q' = r1 - r0 rows they need n_k' = n_k - qpad_rows keys for the same alignment
                    n_k_eff = n_k - qpad_rows
                    if n_k_eff <= 0:
                        out[bi, h0:h1, r0:r1] = 0.0
                        continue
                    kk2, vv2 = kk[:, :, :n_k_eff], vv[:, :, :n_k_eff]
                else:
                    kk2, vv2 = kk, vv
                # expand the kv heads of this head range to the q heads
                rep_idx = torch.arange(h0, h1, device=q.device) // g - kv0
                ke = kk2[:, rep_idx]
                ve = vv2[:, rep_idx]
                out[bi, h0:h1, r0:r1] = attention(qq, ke, ve, causal=causal, scale=scale)[0]
    return out


def attention_varlen(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens_q: torch.Tensor,
                     cu_seqlens_k: torch.Tensor, causal: bool = False, scale: Optional[float] = None,
                     fill: float = float("nan")) -> torch.Tensor:
    """Packed layout, per-sequence dense attention (reference.py:65-95); fp32 result.

    Rows outside every sequence keep ``fill``; zero-length sequences write nothing."""
    out = torch.full(q.shape, fill, dtype=torch.float32, device=q.device)
    cq, ck = cu_seqlens_q.tolist(), cu_seqlens_k.tolist()
    for i in range(len(cq) - 1):
        if cq[i + 1] == cq[i]:
            continue
        qs = q[cq[i]:cq[i + 1]].transpose(0, 1).unsqueeze(0)
        ks = k[ck[i]:ck[i + 1]].transpose(0, 1).unsqueeze(0)
        vs = v[ck[i]:ck[i + 1]].transpose(0, 1).unsqueeze(0)
        out[cq[i]:cq[i + 1]] = attention_chunked(qs, ks, vs, causal=causal, scale=scale)[0].transpose(0, 1)
    return out


# ---------------------------------------------------------------------------------------------
# float64 brute force (independent of torch.matmul / softmax)
# ---------------------------------------------------------------------------------------------


def attention_f64(q, k, v, causal: bool = False, scale: Optional[float] = None) -> np.ndarray:
    """Per-row float64 loops.  q [B,Hq,Nq,D], k/v [B,Hkv,Nk,D] (numpy or torch) -> float64 numpy."""
    q, k, v = (np.asarray(t.float().cpu() if isinstance(t, torch.Tensor) else t, dtype=np.float64) for t in (q, k, v))
    b, h_q, n_q, d = q.shape
    h_kv, n_k = k.shape[1], k.shape[2]
    g = h_q // h_kv
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    out = np.zeros((b, h_q, n_q, d))
    for bi in range(b):
        for h in range(h_q):
            kk, vv = k[bi, h // g], v[bi, h // g]
            for i in range(n_q):
                last = n_k if not causal else min(n_k, i + (n_k - n_q) + 1)
                if last <= 0:
                    continue  # no visible key: zeros
                s = np.array([float(np.dot(q[bi, h, i], kk[j])) * scale for j in range(last)])
                w = np.exp(s - s.max())
                out[bi, h, i] = (w[:, None] * vv[:last]).sum(0) / w.sum()
    return out


def lse_f64(q, k, causal: bool = False, scale: Optional[float] = None) -> np.ndarray:
    """Per-row float64 loops: max + log(sum exp(s - max)) over the visible keys, -inf without any."""
    q, k = (np.asarray(t.float().cpu() if isinstance(t, torch.Tensor) else t, dtype=np.float64) for t in (q, k))
    b, h_q, n_q, d = q.shape
    h_kv, n_k = k.shape[1], k.shape[2]
    g = h_q // h_kv
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    out = np.full((b, h_q, n_q), -np.inf)
    for bi in range(b):
        for h in range(h_q):
            kk = k[bi, h // g]
            for i in range(n_q):
                last = n_k if not causal else min(n_k, i + (n_k - n_q) + 1)
                if last <= 0:
                    continue
                s = np.array([float(np.dot(q[bi, h, i], kk[j])) * scale for j in range(last)])
                out[bi, h, i] = s.max() + math.log(float(np.exp(s - s.max()).sum()))
    return out


# ---------------------------------------------------------------------------------------------
# FP8 E4M3 KV cache (fused_attn/fp8.py:26-56)
# ---------------------------------------------------------------------------------------------


def e4m3fn_value(code: int) -> float:
    """Closed-form OCP E4M3 (fn) decode: bias 7, 3 mantissa bits, S.1111.111 = NaN, no infinities."""
    s, e, m = (code >> 7) & 1, (code >> 3) & 15, code & 7
    if e == 15 and m == 7:
        return float("nan")
    mag = math.ldexp(m / 8.0, -6) if e == 0 else math.ldexp(1.0 + m / 8.0, e - 7)
    return -mag if s else mag


_E4M3_POS = None  # magnitudes of the 127 finite non-negative e4m3fn codes 0x00..0x7e, ascending


def e4m3fn_encode(x: np.ndarray) -> np.ndarray:
    """fp32 -> e4m3fn bytes by nearest representable value, ties to the even code; |x| beyond
    the largest finite value (448) rounds to it up to 464 and is NaN past that
    (non-saturating, as torch's cast); NaN -> S.1111.111 with x's sign.

    Built from the closed-form decoder ``e4m3fn_value`` (a table lookup, not the bit tricks of
    a production converter), so it checks torch's cast rather than restating it."""
    global _E4M3_POS
    if _E4M3_POS is None:
        _E4M3_POS = np.array([e4m3fn_value(c) for c in range(0x7f)], dtype=np.float64)
    xf = np.asarray(x, dtype=np.float32)
    mag = np.abs(xf).astype(np.float64).ravel()
    hi = np.clip(np.searchsorted(_E4M3_POS, mag, side="left"), 1, 0x7e)  # table[hi-1] < mag <= table[hi]
    lo = hi - 1
    d_lo, d_hi = mag - _E4M3_POS[lo], _E4M3_POS[hi] - mag
    code = np.where(d_lo < d_hi, lo, np.where(d_hi < d_lo, hi, np.where(lo % 2 == 0, lo, hi)))
    code = np.where(mag == 0, 0, code)
    # above 448 the next step, 480, would be the odd code S.1111.111 (NaN): up to the midpoint
    # 464 (a tie goes to the even code) the value rounds to 448, past it to NaN
    code = np.where(mag > 448.0, np.where(mag <= 464.0, 0x7e, 0x7f), code)
    code = np.where(np.isnan(mag), 0x7f, code).astype(np.uint8)
    sign = (np.signbit(xf.ravel())).astype(np.uint8) << 7
    return (code | sign).reshape(xf.shape)


def quantize_kv_fp8(x: torch.Tensor, qblock: int = QBLOCK, scale_div: str = "reciprocal"):
    """Per (b, kv-head, qblock keys) amax/448 scale; (x/scale).clamp(+-448) -> e4m3fn (fp8.py:31-45).

    numpy float32 throughout.  ``scale_div`` is how torch evaluates ``amax / 448.0`` (a tensor
    divided by a Python scalar, fp8.py:43): on the GPU as a multiply by the float32 reciprocal
    ("reciprocal"), on the CPU as a true division ("true").  Everything else is the same on
    both devices: correctly rounded x / scale, NaN-propagating amax and clamps, and the
    cast rounding to nearest even."""
    b, h, n, d = x.shape
    nblk = -(-n // qblock)
    xf = np.zeros((b, h, nblk * qblock, d), dtype=np.float32)
    xf[:, :, :n] = x.detach().float().cpu().numpy()
    blk = xf.reshape(b, h, nblk, qblock, d)
    a = np.abs(blk).reshape(b, h, nblk, -1)
    amax = np.where(np.isnan(a).any(axis=-1), np.float32(np.nan), np.nanmax(a, axis=-1, initial=0.0))
    amax = np.where(np.isnan(amax), amax, np.maximum(amax, np.float32(1e-12))).astype(np.float32)
    if scale_div == "reciprocal":
        scale = amax * (np.float32(1.0) / np.float32(E4M3_MAX))
    elif scale_div == "true":
        scale = amax / np.float32(E4M3_MAX)
    else:
        raise ValueError(scale_div)
    scale = scale.astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        y = (blk / scale[..., None, None]).astype(np.float32)
    y = np.where(np.isnan(y), y, np.clip(y, -E4M3_MAX, E4M3_MAX)).astype(np.float32)
    codes = e4m3fn_encode(y).reshape(b, h, nblk * qblock, d)[:, :, :n]
    x8 = torch.from_numpy(np.ascontiguousarray(codes))
    if FP8_DTYPE is not None:
        x8 = x8.view(FP8_DTYPE)
    return x8, torch.from_numpy(np.ascontiguousarray(scale))


def dequantize_kv_fp8(x8: torch.Tensor, scale: torch.Tensor, qblock: int = QBLOCK) -> torch.Tensor:
    """x8.float() * scale of its 64-key block (fp8.py:48-56)."""
    n = x8.shape[2]
    per_key = scale.repeat_interleave(qblock, dim=-1)[..., :n]
    return x8.float() * per_key[..., None]


def attention_fp8(q, k8, k_scale, v8, v_scale, causal: bool = False, scale: Optional[float] = None):
    """FP8-KV attention judged against the fp32 oracle on the dequantised K/V (tests/test_splitk_fp8.py:85)."""
    return attention(q.float(), dequantize_kv_fp8(k8, k_scale), dequantize_kv_fp8(v8, v_scale), causal=causal,
                     scale=scale)


# ---------------------------------------------------------------------------------------------
# paged (block-table) K/V: the reference's roadmap item (README.md:224), defined here as dense
# attention over each sequence's keys gathered through its block table
# ---------------------------------------------------------------------------------------------


def paged_gather(cache: torch.Tensor, block_table: torch.Tensor, seqlen: int, b: int, num_pages=None):
    """Keys 0..seqlen-1 of sequence b from a [num_pages, H, page_size, D] pool, one key at a time
    (key n is row n % page_size of page block_table[b, n // page_size]); a page index outside
    [0, num_pages) contributes zero keys."""
    num_pages = cache.shape[0] if num_pages is None else num_pages
    page_size = cache.shape[2]
    out = cache.new_zeros(cache.shape[1], seqlen, cache.shape[3])
    bt = block_table.cpu()
    for n in range(seqlen):
        pg = int(bt[b, n // page_size])
        if 0 <= pg < num_pages:
            out[:, n] = cache[pg, :, n % page_size]
    return out


def attention_paged(q, k_cache, v_cache, block_table, seqlens_k, causal: bool = False, scale: Optional[float] = None):
    """Per sequence: gather its keys, then the dense oracle with bottom-right causal alignment."""
    out = torch.zeros(q.shape, dtype=torch.float32)
    for b, n in enumerate(seqlens_k.cpu().tolist()):
        k = paged_gather(k_cache.cpu().float(), block_table, n, b)[None]
        v = paged_gather(v_cache.cpu().float(), block_table, n, b)[None]
        out[b:b + 1] = attention(q[b:b + 1].cpu().float(), k, v, causal=causal, scale=scale)
    return out


def attention_paged_fp8(q, k8_pool, k_scale_pool, v8_pool, v_scale_pool, block_table, seqlens_k,
                        causal: bool = False, scale: Optional[float] = None):
    """FP8 paged pools: each page dequantised with its own 64-key block scales (a pool is a
    [num_pages, H, page_size, D] cache to fp8.py:48-56), then the paged oracle.  The reference
    judges FP8 attention against the fp32 oracle on the dequantised K/V
    (tests/test_splitk_fp8.py:85); its roadmap's paged K/V (README.md:224) has no code."""
    return attention_paged(q, dequantize_kv_fp8(k8_pool, k_scale_pool), dequantize_kv_fp8(v8_pool, v_scale_pool),
                           block_table, seqlens_k, causal=causal, scale=scale)


# ---------------------------------------------------------------------------------------------
# split-K (fused_attn/triton_splitk.py)
# ---------------------------------------------------------------------------------------------


def choose_num_splits(batch: int, heads: int, seqlen_k: int, seqlen_q: int, num_sms: int = 108) -> int:
    """triton_splitk.py:130-137."""
    if seqlen_q > 64:
        return 1
    want = max(1, (2 * num_sms) // max(batch * heads, 1))
    return int(min(want, max(1, seqlen_k // 256), 64))


def split_len_for(n_k: int, num_splits: int, block: int = 64) -> int:
    """Split length rounded up to whole blocks (triton_splitk.py:153-154)."""
    per = -(-max(n_k, 1) // max(1, num_splits))
    return -(-per // block) * block


def splitk_partials(q, k, v, causal: bool, scale: Optional[float], split_len: int):
    """float64 partials per split: un-normalised O_s, and log2-domain m_s, l_s (triton_splitk.py:29-96).

    Returns (o [B,Hq,S,Nq,D], m [B,Hq,S,Nq], l [B,Hq,S,Nq]) as numpy float64."""
    q, k, v = (np.asarray(t.float().cpu(), dtype=np.float64) for t in (q, k, v))
    b, h_q, n_q, d = q.shape
    h_kv, n_k = k.shape[1], k.shape[2]
    g = h_q // h_kv
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    n_split = max(1, -(-n_k // split_len))
    o = np.zeros((b, h_q, n_split, n_q, d))
    m = np.full((b, h_q, n_split, n_q), -np.inf)
    l = np.zeros((b, h_q, n_split, n_q))
    for bi in range(b):
        for h in range(h_q):
            s_all = q[bi, h] @ k[bi, h // g].T * (scale * LOG2E)  # [Nq, Nk], log2 domain
            if causal:
                i = np.arange(n_q)[:, None]
                j = np.arange(n_k)[None, :]
                s_all = np.where(j <= i + (n_k - n_q), s_all, -np.inf)
            for si in range(n_split):
                lo, hi = si * split_len, min(n_k, (si + 1) * split_len)
                s = s_all[:, lo:hi]
                if s.shape[1] == 0:
                    continue
                mx = s.max(axis=1)
                ms = np.where(np.isneginf(mx), 0.0, mx)
                p = np.exp2(s - ms[:, None])
                m[bi, h, si] = mx
                l[bi, h, si] = p.sum(1)
                o[bi, h, si] = p @ v[bi, h // g, lo:hi]
    return o, m, l


def splitk_combine(o, m, l) -> np.ndarray:
    """O = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s, 0 when the sum is 0 (triton_splitk.py:99-127)."""
    mx = m.max(axis=2, keepdims=True)
    ms = np.where(np.isneginf(mx), 0.0, mx)
    w = np.exp2(m - ms)  # [B,Hq,S,Nq]
    lt = (w * l).sum(axis=2)
    num = (w[..., None] * o).sum(axis=2)
    return num / np.where(lt == 0.0, 1.0, lt)[..., None]


def attn_flops(b: int, h: int, n: int, d: int, causal: bool) -> float:
    """QK^T and PV at 2 FLOP per MAC, halved when causal (benchmarks/bench.py:44-46)."""
    f = 4.0 * b * h * n * n * d
    return f / 2 if causal else f
