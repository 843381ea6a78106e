"""Split-K attention ("flash-decoding") for long-context decode.

Decode contributes one or a few query rows per request, so a one-pass kernel
has too few workgroups to stream a long K/V cache at full HBM bandwidth.  The
keys are cut into partitions of ``split_len`` keys (a multiple of 64); each
partition runs the online-softmax loop and writes an fp32 partial output
normalised by its own row sum (Ô_s = O_s / l_s, a convex combination of V rows)
plus its log2-domain (max, sum); a combine kernel merges them exactly:

    m = max_s m_s,   l = sum_s 2^(m_s - m) l_s,   O = sum_s 2^(m_s - m) l_s Ô_s / l

which is the reference's merge of un-normalised partials O_s = l_s Ô_s
(reference: fused_attn/triton_splitk.py:1-16,90-127).  On MI355X one workgroup
covers a (batch, kv-head, partition): all Hq/Hkv query heads that share the
kv-head are rows of the same tile, so the K/V cache is read once from HBM.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from . import _hip
from .reference import attention_reference, lse_reference


def choose_num_splits(batch: int, heads: int, seqlen_k: int, seqlen_q: int, num_sms: int = 108) -> int:
    """Enough splits for ~2 programs per compute unit, each covering >= 256 keys (triton_splitk.py:130-137)."""
    if seqlen_q > 64:
        return 1  # prefill-sized queries already fill the GPU
    programs = batch * heads
    want = max(1, (2 * num_sms) // max(programs, 1))
    cap = max(1, seqlen_k // 256)
    return int(min(want, cap, 64))


def attention_splitk(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    causal: bool = False,
    scale: Optional[float] = None,
    num_splits: Optional[int] = None,
    split_len: Optional[int] = None,
    return_lse: bool = False,
):
    """Split-K attention (reference signature: triton_splitk.py:140-143, plus ``split_len`` and
    ``return_lse``, which also returns the natural-log LSE fp32 [B, H_q, N_q] from the combine:
    the quantity chunked or cascaded decode merges further).

    ``num_splits`` is honoured as in the reference: each partition gets
    ``ceil(ceil(n_k / num_splits) / 64) * 64`` keys.  ``split_len`` (a multiple
    of 64) sets the partition size directly.  With neither, ``ops.default_split_len``
    chooses it (partitions as long as possible while the grid keeps about
    SPLITK_TARGET_WGS workgroups).  CPU tensors use the unfused reference.
    """
    d = q.shape[-1]
    n_k = k.shape[-2]
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    if not q.is_cuda:
        o = attention_reference(q, k, v, causal=causal, scale=scale)
        return (o, lse_reference(q, k, causal=causal, scale=scale)) if return_lse else o
    if split_len is None:
        if num_splits is not None:
            split_len = _hip.split_len_for(n_k, num_splits)
        else:
            from .ops import default_split_len

            split_len = default_split_len(q.shape[-2], n_k, q.shape[0], k.shape[1], q.shape[1] // k.shape[1])
    return _hip.splitk(q, k, v, causal=causal, scale=scale, split_len=int(split_len), return_lse=return_lse)


# The reference exported the Triton entry under this name (fused_attn/__init__.py:5-9).
attention_splitk_triton = attention_splitk
