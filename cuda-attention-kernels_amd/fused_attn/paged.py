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

``causal`` aligns each sequence's queries to the end of its own keys (bottom-right, as
the dense op).  On the GPU this runs the split-K HIP kernel in its paged mode; page_size
must be a multiple of 32.  CPU tensors, or ``FUSED_ATTN_BACKEND=reference``, gather the
pages and run the unfused reference per sequence.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from . import _hip
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
                    max_seqlen_k: Optional[int] = None, split_len: Optional[int] = None, return_lse: bool = False):
    """Decode attention over a paged K/V cache.  ``max_seqlen_k`` (the largest entry of
    ``seqlens_k``) sizes the grid; when omitted it is read from ``seqlens_k`` (a device sync).
    With ``return_lse`` also returns the natural-log LSE, fp32 [B, H_q, N_q]."""
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
    if not q.is_cuda or _pick_backend(q) != "hip":
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
                             split_len=split_len, return_lse=return_lse)


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
