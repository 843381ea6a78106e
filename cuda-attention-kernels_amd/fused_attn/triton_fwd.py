"""The reference's ``fused_attn.triton_fwd`` entry points, HIP-backed (no Triton).

Callers of the reference import ``attention_triton`` / ``attention_varlen_triton``
from this module path (e.g. benchmarks/bench_decode.py:47); both keep their
signatures (fused_attn/triton_fwd.py:225-233, 268-279) and run the gfx950 prefill
kernel.  ``autotune`` is accepted and ignored: the kernel has one tuned shape per
head dim.  ``attention_varlen_triton`` additionally takes ``return_lse`` (natural-log
LSE as fp32 [H_q, total_q]), which the reference's varlen path did not offer.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _hip
from .reference import attention_reference, attention_varlen_reference, lse_reference


def attention_triton(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    causal: bool = False,
    scale: Optional[float] = None,
    return_lse: bool = False,
    autotune: Optional[bool] = None,
):
    """Dense layout: q [B, H_q, N_q, D]; k, v [B, H_kv, N_k, D].  Returns o, or (o, lse [B, H_q, N_q])."""
    del autotune
    if not q.is_cuda:
        o = attention_reference(q, k, v, causal=causal, scale=scale)
        if not return_lse:
            return o
        return o, lse_reference(q, k, causal=causal, scale=scale)
    return _hip.fwd(q, k, v, causal=causal, scale=scale, return_lse=return_lse)


def attention_varlen_triton(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    max_seqlen_q: int,
    max_seqlen_k: int,
    causal: bool = False,
    scale: Optional[float] = None,
    autotune: Optional[bool] = None,
    return_lse: bool = False,
):
    """Packed layout: q [total_q, H_q, D]; k, v [total_k, H_kv, D]."""
    del autotune
    if not q.is_cuda:
        if return_lse:
            raise RuntimeError("return_lse on the varlen path needs GPU tensors")
        return attention_varlen_reference(q, k, v, cu_seqlens_q, cu_seqlens_k, causal=causal, scale=scale)
    return _hip.varlen_fwd(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, causal=causal,
                           scale=scale, return_lse=return_lse)
