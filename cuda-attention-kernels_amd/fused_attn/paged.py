"""Paged (block-table) K/V cache for decode.

The reference lists paged K/V for its decode kernels as a roadmap item
(README.md:224) and has no interface for it; this module gives it the split-K
decode semantics of ``attention_splitk_triton`` (fused_attn/triton_splitk.py:140-181)
applied to each sequence's keys, gathered through a block table:

    k_cache, v_cache   [num_pages, Hkv, page_size, D]  (any strides with unit D stride;
                       a [num_pages, page_size, Hkv, D] pool passes as .transpose(1, 2))
    block_table        int32 [B, pages_per_seq]: sequence b's key n is in page
                       block_table[b, n // page_size] at offset n % page_size
    seqlens_k          int32 [B]: keys per sequence (ragged; 0 allowed)

    o = attention_paged(q, k_cache, v_cache, block_table, seqlens_k)   # q, o [B, Hq, n_q, D]

FP8 pools (float8_e4m3fn) hold the bytes ``quantize_kv_fp8`` writes for a
[num_pages, Hkv, page_size, D] pool and take its block scales, fp32
[num_pages, Hkv, page_size / 64], as ``k_scale`` / ``v_scale`` (page_size a multiple of 64):
the semantics of ``attention_fp8_triton`` (fused_attn/fp8.py:125-147) on each sequence's
gathered keys.

``causal`` aligns each sequence's queries to the end of its own keys (bottom-right, as
the dense op).  On the GPU this runs the split-K HIP kernel in its paged mode; page_size
must be a multiple of 16 (64 for FP8 pools).  CPU tensors, or ``FUSED_ATTN_BACKEND=reference``, gather the
pages and run the unfused reference per sequence.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from . import _hip
from .fp8 import FP8_DTYPE, QBLOCK, dequantize_kv_fp8
from .ops import _pick_backend, default_split_len
from .reference import attention_reference, lse_reference


def gather_paged(cache: torch.Tensor, block_table: torch.Tensor, seqlen: int, b: int) -> torch.Tensor:
    """Sequence ``b``'s first ``seqlen`` keys as a dense [Hkv, seqlen, D] tensor."""
    page_size = cache.shape[2]
    npg = -(-seqlen // page_size)
    pages = block_table[b, :npg].long().to(cache.device)
    return cache[pages].permute(1, 0, 2, 3).reshape(cache.shape[1], npg * page_size, cache.shape[3])[:, :seqlen]


def attention_paged_reference(q, k_cache, v_cache, block_table, seqlens_k, causal: bool = False,
                              scale: Optional[float] = None, return_lse: bool = False):
    """Unfused path: gather each sequence's pages, then ``attention_reference`` on it."""
    out = torch.empty_like(q)
    lse = torch.empty(q.shape[:3], dtype=torch.float32, device=q.device) if return_lse else None
    lens = seqlens_k.tolist()
    for b, n in enumerate(lens):
        k = gather_paged(k_cache, block_table, n, b)[None]
        v = gather_paged(v_cache, block_table, n, b)[None]
        out[b:b + 1] = attention_reference(q[b:b + 1], k, v, causal=causal, scale=scale)
        if return_lse:
            lse[b:b + 1] = lse_reference(q[b:b + 1], k, causal=causal, scale=scale)
    return (out, lse) if return_lse else out


def attention_paged(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, block_table: torch.Tensor,
                    seqlens_k: torch.Tensor, causal: bool = False, scale: Optional[float] = None,
                    max_seqlen_k: Optional[int] = None, split_len: Optional[int] = None, return_lse: bool = False,
                    k_scale: Optional[torch.Tensor] = None, v_scale: Optional[torch.Tensor] = None):
    """Decode attention over a paged K/V cache.  ``max_seqlen_k`` (the largest entry of
    ``seqlens_k``) sizes the grid; when omitted it is read from ``seqlens_k`` (a device sync).
    FP8 pools take their per-page block scales ``k_scale`` / ``v_scale``.
    With ``return_lse`` also returns the natural-log LSE, fp32 [B, H_q, N_q]."""
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
    fp8 = FP8_DTYPE is not None and k_cache.dtype == FP8_DTYPE
    if not q.is_cuda or _pick_backend(q) != "hip":
        if fp8:
            if k_scale is None or v_scale is None:
                raise RuntimeError("FP8 pools need k_scale and v_scale")
            if k_cache.shape[2] % QBLOCK:
                raise RuntimeError(f"FP8 pools need page_size a multiple of {QBLOCK}")
            k_cache, v_cache = dequantize_kv_fp8(k_cache, k_scale), dequantize_kv_fp8(v_cache, v_scale)
        return attention_paged_reference(q, k_cache, v_cache, block_table, seqlens_k, causal=causal, scale=scale,
                                         return_lse=return_lse)
    if max_seqlen_k is None:
        max_seqlen_k = int(seqlens_k.max().item()) if seqlens_k.numel() else 0
    if split_len is None:
        b, hq, nq, _ = q.shape
        hkv = k_cache.shape[1]
        split_len = default_split_len(nq, max_seqlen_k, b, hkv, hq // hkv)
        # a partition may span at most 256 pages of the block table
        page_size = k_cache.shape[2]
        split_len = min(split_len, max(64, (254 * page_size) // 64 * 64))
    return _hip.paged_decode(q, k_cache, v_cache, block_table, seqlens_k, max_seqlen_k, causal=causal, scale=scale,
                             split_len=split_len, return_lse=return_lse, k_scale=k_scale if fp8 else None,
                             v_scale=v_scale if fp8 else None)


def paged_from_dense(k: torch.Tensor, v: torch.Tensor, page_size: int, seqlens: Optional[list] = None,
                     extra_pages: int = 0, generator: Optional[torch.Generator] = None):
    """Scatter dense K/V [B, Hkv, N, D] into pools of ``page_size``-key pages in a random page order.

    Returns (k_cache, v_cache, block_table int32 [B, ceil(N/page_size)], seqlens_k int32 [B]); sequence b
    keeps its first ``seqlens[b]`` keys (default N).  ``extra_pages`` unused pages are added to the pools."""
    b, hkv, n, d = k.shape
    cols = -(-n // page_size)
    seqlens = [n] * b if seqlens is None else list(seqlens)
    num_pages = b * cols + extra_pages
    perm = torch.randperm(num_pages, generator=generator, device="cpu")[:b * cols].view(b, cols)
    pad = cols * page_size - n
    kp = torch.nn.functional.pad(k, (0, 0, 0, pad)) if pad else k
    vp = torch.nn.functional.pad(v, (0, 0, 0, pad)) if pad else v
    k_cache = torch.zeros(num_pages, hkv, page_size, d, dtype=k.dtype, device=k.device)
    v_cache = torch.zeros_like(k_cache)
    idx = perm.reshape(-1).to(k.device)
    k_cache[idx] = kp.view(b, hkv, cols, page_size, d).permute(0, 2, 1, 3, 4).reshape(b * cols, hkv, page_size, d)
    v_cache[idx] = vp.view(b, hkv, cols, page_size, d).permute(0, 2, 1, 3, 4).reshape(b * cols, hkv, page_size, d)
    block_table = perm.to(torch.int32).to(k.device)
    seqlens_k = torch.tensor(seqlens, dtype=torch.int32, device=k.device)
    return k_cache, v_cache, block_table, seqlens_k


def paged_from_dense_fp8(k8: torch.Tensor, k_scale: torch.Tensor, v8: torch.Tensor, v_scale: torch.Tensor,
                         page_size: int, seqlens: Optional[list] = None, extra_pages: int = 0,
                         generator: Optional[torch.Generator] = None):
    """Scatter a dense FP8 cache (``quantize_kv_fp8`` output: e4m3fn [B, Hkv, N, D] and fp32 block
    scales [B, Hkv, ceil(N/64)]) into pools of ``page_size``-key pages (a multiple of 64) in a random
    page order, with each page's block scales alongside.

    Returns (k_cache, v_cache, k_scale_pool, v_scale_pool, block_table, seqlens_k): pools
    [num_pages, Hkv, page_size, D] e4m3fn, scale pools fp32 [num_pages, Hkv, page_size / 64], an int32
    [B, ceil(N/page_size)] block table and int32 [B] lengths.  Because pages start on 64-key blocks,
    page p's scales are exactly the dense scales of the blocks it holds, so the pools describe the same
    keys bit for bit.  ``extra_pages`` unused (zero) pages are added."""
    if page_size % QBLOCK:
        raise ValueError(f"page_size must be a multiple of {QBLOCK}")
    b, hkv, n, d = k8.shape
    cols = -(-n // page_size)
    bpp = page_size // QBLOCK
    seqlens = [n] * b if seqlens is None else list(seqlens)
    num_pages = b * cols + extra_pages
    perm = torch.randperm(num_pages, generator=generator, device="cpu")[:b * cols].view(b, cols)
    idx = perm.reshape(-1).to(k8.device)

    def pages(x8):
        xb = x8.view(torch.uint8)
        pad = cols * page_size - n
        xb = torch.nn.functional.pad(xb, (0, 0, 0, pad)) if pad else xb
        pool = torch.zeros(num_pages, hkv, page_size, d, dtype=torch.uint8, device=x8.device)
        pool[idx] = xb.reshape(b, hkv, cols, page_size, d).permute(0, 2, 1, 3, 4).reshape(b * cols, hkv, page_size, d)
        return pool.view(x8.dtype)

    def scale_pages(sc):
        pad = cols * bpp - sc.shape[-1]
        sc = torch.nn.functional.pad(sc.float(), (0, pad)) if pad else sc.float()
        pool = torch.zeros(num_pages, hkv, bpp, dtype=torch.float32, device=sc.device)
        pool[idx] = sc.reshape(b, hkv, cols, bpp).permute(0, 2, 1, 3).reshape(b * cols, hkv, bpp)
        return pool

    block_table = perm.to(torch.int32).to(k8.device)
    seqlens_k = torch.tensor(seqlens, dtype=torch.int32, device=k8.device)
    return pages(k8), pages(v8), scale_pages(k_scale), scale_pages(v_scale), block_table, seqlens_k
