"""Unfused PyTorch attention: the ``reference`` backend of the op.

This is the public, user-callable unfused path that the reference package
exports (fused_attn/reference.py:1-95).  It runs on any device with plain torch
ops, materialises the full score matrix, and is the backend the op uses for
CPU tensors or when ``FUSED_ATTN_BACKEND=reference``.  It keeps the
reference's operation order (fp32 upcast, GQA head sharing, scale, bottom-right
causal mask, softmax, NaN rows -> 0, P V, cast back) because its outputs define
the op's results on those paths.
"""
from __future__ import annotations

import math
from typing import Optional

import torch


def _expand_kv(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    """[B, Hkv, N, D] -> [B, Hkv*n_rep, N, D]; q-head h reads kv-head h // n_rep (reference.py:16-21)."""
    if n_rep == 1:
        return x
    b, h, n, d = x.shape
    return x.unsqueeze(2).expand(b, h, n_rep, n, d).reshape(b, h * n_rep, n, d)


def causal_mask(seqlen_q: int, seqlen_k: int, device=None) -> torch.Tensor:
    """Boolean [seqlen_q, seqlen_k], True where key j is visible to query i: j <= i + (seqlen_k - seqlen_q).

    Bottom-right alignment (reference.py:24-33): the last query sees every key.
    """
    rows = torch.arange(seqlen_q, device=device).unsqueeze(1)
    cols = torch.arange(seqlen_k, device=device).unsqueeze(0)
    return cols <= rows + (seqlen_k - seqlen_q)


def attention_reference(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    causal: bool = False,
    scale: Optional[float] = None,
    upcast: bool = True,
) -> torch.Tensor:
    """q [B, Hq, Nq, D]; k, v [B, Hkv, Nk, D] -> [B, Hq, Nq, D] in q's dtype (reference.py:36-62)."""
    assert q.dim() == 4 and k.dim() == 4 and v.dim() == 4
    _, h_q, n_q, d = q.shape
    h_kv, n_k = k.shape[1], k.shape[2]
    assert h_q % h_kv == 0, "H_q must be a multiple of H_kv"
    out_dtype = q.dtype
    if upcast:
        q, k, v = q.float(), k.float(), v.float()
    rep = h_q // h_kv
    k, v = _expand_kv(k, rep), _expand_kv(v, rep)
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    s = torch.matmul(q, k.transpose(-1, -2)) * scale
    if causal:
        s = s.masked_fill(~causal_mask(n_q, n_k, device=q.device), float("-inf"))
    p = torch.softmax(s, dim=-1)
    p = torch.nan_to_num(p, nan=0.0)  # a row with no visible key is all -inf -> NaN -> 0
    return torch.matmul(p, v).to(out_dtype)


def attention_varlen_reference(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    causal: bool = False,
    scale: Optional[float] = None,
) -> torch.Tensor:
    """Packed layout: q [Tq, Hq, D]; k, v [Tk, Hkv, D]; cu_seqlens int32 [nseq+1] (reference.py:65-95).

    Sequences with no queries are skipped; every other query row is written.
    """
    assert q.dim() == 3
    out = torch.empty_like(q)
    bounds_q = cu_seqlens_q.tolist()
    bounds_k = cu_seqlens_k.tolist()
    for i in range(len(bounds_q) - 1):
        q0, q1 = bounds_q[i], bounds_q[i + 1]
        k0, k1 = bounds_k[i], bounds_k[i + 1]
        if q1 == q0:
            continue
        o = attention_reference(
            q[q0:q1].transpose(0, 1).unsqueeze(0),
            k[k0:k1].transpose(0, 1).unsqueeze(0),
            v[k0:k1].transpose(0, 1).unsqueeze(0),
            causal=causal,
            scale=scale,
        )
        out[q0:q1] = o[0].transpose(0, 1)
    return out


def lse_reference(q: torch.Tensor, k: torch.Tensor, causal: bool = False, scale: Optional[float] = None) -> torch.Tensor:
    """Natural-log LSE of the unfused scores [B, H_q, N_q] (the softmax denominator of
    ``attention_reference``, in log form, as the Triton kernel's WRITE_LSE output,
    fused_attn/triton_fwd.py:169-172); rows without a visible key are -inf."""
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
    g = q.shape[1] // k.shape[1]
    kk = k.float().repeat_interleave(g, dim=1)
    s = torch.matmul(q.float(), kk.transpose(-1, -2)) * scale
    if causal:
        n_q, n_k = q.shape[-2], k.shape[-2]
        i = torch.arange(n_q, device=q.device)[:, None]
        j = torch.arange(n_k, device=q.device)[None, :]
        s = s.masked_fill(j > i + (n_k - n_q), float("-inf"))
    return torch.logsumexp(s, dim=-1)
