"""FP8 (OCP E4M3, ``torch.float8_e4m3fn``) KV cache.

Decode is bound by reading K/V, so an FP8 cache halves the bytes streamed from
HBM.  Values are scaled per (batch, kv-head, block of ``QBLOCK`` keys): each
block is divided by absmax/448 before the cast (fused_attn/fp8.py:26-45).

    k8, ks = quantize_kv_fp8(k)          # [B,Hkv,N,D] float8_e4m3fn, [B,Hkv,ceil(N/64)] fp32
    v8, vs = quantize_kv_fp8(v)
    o = attention_fp8(q, k8, ks, v8, vs, causal=True)

On the GPU the quantiser is one fused HIP kernel (one workgroup per 64-key
block) whose bytes and scales are bit-identical to the reference's torch chain on
the GPU; CPU tensors, or ``FUSED_ATTN_BACKEND=reference``, run that torch chain.
The dequantiser is the reference's torch chain.  ``attention_fp8`` runs the
HIP split-K kernel, which keeps K/V 8-bit in LDS and widens each E4M3 element
exactly to q's 16-bit type as it reads an MFMA operand, and multiplies the score
block by ``scale * k_scale``.  For V it keeps the fp32 accumulator in units of a
recent block's ``v_scale`` (v_cur): a block whose scale is within a factor 2 of
v_cur folds ``v_scale / v_cur`` into P before P's 16-bit rounding, any other
block first rescales the accumulator to its own scale, and v_cur multiplies the
result in fp32.  This is the reference's ``P.V * v_scale`` per block
(fp8.py:116) up to fp32 rounding, with P never scaled by more than 2.  Any
number of queries is accepted (prefill-shaped calls too).
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from . import _hip
from .ops import _pick_backend
from .reference import attention_reference, lse_reference

QBLOCK = 64  # keys per scale
E4M3_MAX = 448.0
FP8_DTYPE = getattr(torch, "float8_e4m3fn", None)


def quantize_kv_fp8(x: torch.Tensor, qblock: int = QBLOCK) -> tuple[torch.Tensor, torch.Tensor]:
    """x [B, Hkv, N, D] (any float dtype) -> (float8_e4m3fn, same shape; fp32 scales [B, Hkv, ceil(N/qblock)]).

    GPU tensors of fp32/fp16/bf16 with D in {16, 32, 64, 128, 256} go to the fused HIP kernel
    (it raises if the library or device is unusable); other shapes and CPU tensors take the
    reference's torch chain (fused_attn/fp8.py:31-45)."""
    assert FP8_DTYPE is not None, "this torch build has no float8_e4m3fn"
    if (x.is_cuda and qblock == QBLOCK and _pick_backend(x) == "hip" and x.dim() == 4
            and x.dtype in (torch.float32, torch.float16, torch.bfloat16) and x.shape[-1] in _hip.QUANT_HEAD_DIMS):
        return _hip.quantize_kv_fp8(x)
    return _quantize_kv_fp8_torch(x, qblock)


def _quantize_kv_fp8_torch(x: torch.Tensor, qblock: int = QBLOCK) -> tuple[torch.Tensor, torch.Tensor]:
    """The reference's torch op chain (fused_attn/fp8.py:31-45), on x's device."""
    b, h, n, d = x.shape
    nblk = -(-n // qblock)
    xf = x.float()
    pad = nblk * qblock - n
    if pad:
        xf = torch.nn.functional.pad(xf, (0, 0, 0, pad))
    blocks = xf.view(b, h, nblk, qblock, d)
    scale = blocks.abs().amax(dim=(-1, -2)).clamp_min(1e-12) / E4M3_MAX  # [B, Hkv, nblk]
    scaled = (blocks / scale[..., None, None]).clamp(-E4M3_MAX, E4M3_MAX)
    x8 = scaled.to(FP8_DTYPE).view(b, h, nblk * qblock, d)[:, :, :n].contiguous()
    return x8, scale.contiguous()


def dequantize_kv_fp8(x8: torch.Tensor, scale: torch.Tensor, qblock: int = QBLOCK) -> torch.Tensor:
    """Inverse of ``quantize_kv_fp8`` up to rounding: fp32 [B, Hkv, N, D] (fused_attn/fp8.py:48-56)."""
    b, h, n, d = x8.shape
    nblk = scale.shape[-1]
    xf = x8.float()
    pad = nblk * qblock - n
    if pad:
        xf = torch.nn.functional.pad(xf, (0, 0, 0, pad))
    out = xf.view(b, h, nblk, qblock, d) * scale[..., None, None]
    return out.view(b, h, nblk * qblock, d)[:, :, :n]


def attention_fp8(
    q: torch.Tensor,
    k8: torch.Tensor,
    k_scale: torch.Tensor,
    v8: torch.Tensor,
    v_scale: torch.Tensor,
    causal: bool = False,
    scale: Optional[float] = None,
    split_len: Optional[int] = None,
    return_lse: bool = False,
):
    """Attention over an FP8 K/V cache (reference signature: fused_attn/fp8.py:125-128, plus ``split_len``
    and ``return_lse``: the natural-log LSE fp32 [B, H_q, N_q] of the scores on the dequantised keys)."""
    assert q.dtype in (torch.float16, torch.bfloat16), \
        "Q must be fp16/bf16 (FP8 is converted to Q's dtype for the MFMA)"
    assert k8.dtype == FP8_DTYPE and v8.dtype == FP8_DTYPE
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
    if not q.is_cuda:
        kd = dequantize_kv_fp8(k8, k_scale)
        o = attention_reference(q, kd, dequantize_kv_fp8(v8, v_scale), causal=causal, scale=scale)
        return (o, lse_reference(q, kd, causal=causal, scale=scale)) if return_lse else o
    if split_len is None:
        if q.shape[-2] <= 16:  # decode-shaped: partitions sized for the grid (ops.default_split_len)
            from .ops import default_split_len

            split_len = default_split_len(q.shape[-2], k8.shape[-2], q.shape[0], k8.shape[1], q.shape[1] // k8.shape[1])
        else:  # prefill-shaped: one partition, as the reference's single-pass kernel (fp8.py:136-145)
            split_len = max(QBLOCK, -(-k8.shape[-2] // QBLOCK) * QBLOCK)
    return _hip.splitk(q, k8, v8, causal=causal, scale=scale, split_len=int(split_len), k_scale=k_scale,
                       v_scale=v_scale, return_lse=return_lse)


# The reference exported the Triton entry under this name (fused_attn/__init__.py:5-9).
attention_fp8_triton = attention_fp8
