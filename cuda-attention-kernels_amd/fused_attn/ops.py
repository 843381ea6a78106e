"""Public op and backend dispatch.

``fused_attn.attention`` is the ``torch.library`` custom op of the reference
(fused_attn/ops.py:76-104), same name, schema, defaults and fake kernel, so
``torch.compile(fullgraph=True)`` still traces it and it shows up by name in
profiler traces.

Dispatch is ``hip`` or ``reference`` (the reference's five backends,
ops.py:34-73, collapse into these two):

* GPU tensors go to the HIP backend (``_hip``): MFMA FA2 prefill, or split-K
  flash-decoding for decode-shaped calls (at most 16 queries against at least
  2048 keys, ops.py:36-37,63-66).  If the HIP library cannot run on the device
  the call raises; it never falls back silently.
* CPU tensors, or ``FUSED_ATTN_BACKEND=reference``, use the unfused PyTorch
  path in ``reference.py``.

``FUSED_ATTN_BACKEND`` also accepts the reference's GPU backend names
(``cuda_mma``, ``cuda``, ``triton`` -> ``hip``; ``splitk`` -> ``hip`` with the
split-K kernel forced) so existing environments keep working.
"""
from __future__ import annotations

import math
import os
from typing import Optional

import torch

from . import _hip
from .reference import attention_reference, attention_varlen_reference

BACKENDS = ("hip", "reference")
_ALIASES = {"cuda_mma": "hip", "cuda": "hip", "triton": "hip", "splitk": "hip"}
SPLITK_MAX_Q = 16  # decode-shaped: few query rows ...
SPLITK_MIN_K = 2048  # ... against a long context
DEFAULT_SPLIT_KEYS = 128  # smallest split-K partition chosen by default (keys, a multiple of 64)
MAX_SPLIT_KEYS = 4096  # largest
SPLITK_TARGET_WGS = 2048  # default partitions make about this many split-K workgroups


def available_backends() -> list[str]:
    out = []
    if _hip.available():
        out.append("hip")
    out.append("reference")
    return out


def _forced_backend() -> Optional[str]:
    forced = os.environ.get("FUSED_ATTN_BACKEND")
    if not forced:
        return None
    if forced not in BACKENDS and forced not in _ALIASES:
        raise ValueError(f"unknown backend {forced!r}; expected one of {BACKENDS} "
                         f"(or a reference name {tuple(_ALIASES)})")
    return forced


def _pick_backend(q: torch.Tensor, k: Optional[torch.Tensor] = None) -> str:
    """``hip`` for GPU tensors, ``reference`` otherwise or when forced (reference: ops.py:56-73)."""
    forced = _forced_backend()
    if forced is not None:
        return _ALIASES.get(forced, forced)
    return "hip" if q.is_cuda else "reference"


def is_decode_shaped(q: torch.Tensor, k: Optional[torch.Tensor]) -> bool:
    """Few queries against a long context: the split-K regime (ops.py:63)."""
    return k is not None and q.shape[-2] <= SPLITK_MAX_Q and k.shape[-2] >= SPLITK_MIN_K


SPLITK_DTYPES = (torch.float16, torch.bfloat16)  # the split-K kernel: 16-bit Q with D in {64, 128, 256}
SPLITK_HEAD_DIMS = (64, 128, 256)


def _hip_kernel_for(q: torch.Tensor, k: torch.Tensor) -> str:
    """Which HIP kernel family serves this call: ``splitk`` or ``fwd``.

    fp32 and head dims other than 64 / 128 / 256 always take ``fwd``, whose MFMA or generic
    kernel covers them (the reference's Triton path likewise served every shape).
    """
    if q.dtype not in SPLITK_DTYPES or q.shape[-1] not in SPLITK_HEAD_DIMS:
        return "fwd"
    if os.environ.get("FUSED_ATTN_BACKEND") == "splitk" or is_decode_shaped(q, k):
        return "splitk"
    return "fwd"


@torch.library.custom_op("fused_attn::attention", mutates_args=())
def attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    causal: bool = False,
    scale: Optional[float] = None,
) -> torch.Tensor:
    """Fused scaled-dot-product attention.

    q: [B, H_q, N_q, D]; k, v: [B, H_kv, N_k, D] with H_q % H_kv == 0.
    Returns [B, H_q, N_q, D] in q's dtype.
    """
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
    if _pick_backend(q, k) == "hip":
        if _hip_kernel_for(q, k) == "splitk":
            return _hip.splitk(q, k, v, causal=causal, scale=scale,
                               split_len=default_split_len(q.shape[-2], k.shape[-2], q.shape[0], k.shape[1],
                                                           q.shape[1] // k.shape[1]))
        return _hip.fwd(q, k, v, causal=causal, scale=scale)
    return attention_reference(q, k, v, causal=causal, scale=scale)


@attention.register_fake
def _attention_fake(q, k, v, causal=False, scale=None):
    return q.new_empty(q.shape)


def default_split_len(seqlen_q: int, seqlen_k: int, batch: int = 1, heads_kv: int = 1, group: int = 1) -> int:
    """Keys per split-K partition when the caller does not choose one.

    A split-K workgroup streams one partition of one (batch, kv-head) for up to 128
    (q-head, query) rows, so the grid has batch * heads_kv * row_blocks * partitions
    workgroups.  Partitions are made as long as possible while the grid keeps about
    SPLITK_TARGET_WGS workgroups: longer partitions write fewer partials and
    spend less per workgroup (on MI355X, B=32 Hkv=8 n_k=32768 D=128 bf16 decode moves
    5.6 TB/s at 128-key partitions, 6.0 at 512, 6.5 at 2048 and 6.65 at 4096).
    """
    rows = group * seqlen_q
    row_blocks = -(-rows // 128)
    items = max(1, batch * heads_kv * row_blocks)
    parts = max(1, -(-SPLITK_TARGET_WGS // items))
    keys = -(-max(seqlen_k, 1) // parts)
    keys = -(-keys // 64) * 64
    return int(min(max(keys, DEFAULT_SPLIT_KEYS), MAX_SPLIT_KEYS))


@torch.library.custom_op("fused_attn::attention_varlen", mutates_args=())
def attention_varlen(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    max_seqlen_q: int,
    max_seqlen_k: int,
    causal: bool = False,
    scale: Optional[float] = None,
) -> torch.Tensor:
    """Packed/ragged attention. q: [total_q, H_q, D]; k, v: [total_k, H_kv, D] (reference: ops.py:107-124).

    Same signature as the reference's plain function, registered as a custom op with a
    fake so that ``torch.compile(fullgraph=True)`` traces it like ``attention``.  On GPU
    tensors it runs the HIP kernel in varlen mode (the reference ran its Python
    reference loop whenever its CUDA extension was built, ops.py:119-124).
    """
    if _pick_backend(q) == "hip":
        return _hip.varlen_fwd(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, causal=causal,
                               scale=scale)
    return attention_varlen_reference(q, k, v, cu_seqlens_q, cu_seqlens_k, causal=causal, scale=scale)


@attention_varlen.register_fake
def _attention_varlen_fake(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, causal=False,
                           scale=None):
    return q.new_empty(q.shape)


def pack_varlen(tensors: list[torch.Tensor]):
    """[[N_i, H, D], ...] -> (packed [sum N_i, H, D], int32 cu_seqlens [n+1] starting at 0, max N_i)
    (reference: ops.py:127-132)."""
    lens = [t.shape[0] for t in tensors]
    dev = tensors[0].device
    cu = torch.zeros(len(lens) + 1, dtype=torch.int32, device=dev)
    cu[1:] = torch.cumsum(torch.tensor(lens, device=dev), 0)
    return torch.cat(tensors, 0), cu, max(lens)
