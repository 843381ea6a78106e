"""ctypes binding of ``libfused_attn_hip.so`` (the C ABI in ``include/fused_attn_hip.h``).

This module replaces the reference's compiled pybind extension ``fused_attn._C``
(csrc/bindings.cpp:90-96).  It turns torch tensors into the plain pointers,
element strides and sizes of ``fa_fwd_params``, allocates every output and
workspace with the torch caching allocator on the tensors' device, enqueues the
kernels on the current stream and maps ``fa_status`` codes to ``RuntimeError``
(the reference's TORCH_CHECK failures surfaced as RuntimeError too,
csrc/bindings.cpp:35-50).

There is no fallback here: if the library is missing or the device is not a
gfx950 GPU, every entry point raises.
"""
from __future__ import annotations

import contextlib
import ctypes
import math
import os
import threading
from typing import Optional

import torch

LIB_NAME = "libfused_attn_hip.so"
ABI_VERSION = 6

# fa_dtype codes
F16, BF16, F32, FP8_E4M3 = 0, 1, 2, 3
_DTYPE_CODE = {torch.float16: F16, torch.bfloat16: BF16, torch.float32: F32}
_FP8 = getattr(torch, "float8_e4m3fn", None)
if _FP8 is not None:
    _DTYPE_CODE[_FP8] = FP8_E4M3

FA_OK, FA_ERR_INVALID_ARGUMENT, FA_ERR_UNSUPPORTED, FA_ERR_WORKSPACE, FA_ERR_HIP = range(5)
_STATUS_NAME = {
    FA_ERR_INVALID_ARGUMENT: "invalid argument",
    FA_ERR_UNSUPPORTED: "unsupported",
    FA_ERR_WORKSPACE: "workspace",
    FA_ERR_HIP: "HIP error",
}

FP8_QBLOCK = 64  # keys per FP8 scale block; split-K partitions are multiples of it


class FwdParams(ctypes.Structure):
    """Mirror of ``fa_fwd_params`` (include/fused_attn_hip.h)."""

    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("q_stride_b", ctypes.c_int64),
        ("q_stride_h", ctypes.c_int64),
        ("q_stride_n", ctypes.c_int64),
        ("k_stride_b", ctypes.c_int64),
        ("k_stride_h", ctypes.c_int64),
        ("k_stride_n", ctypes.c_int64),
        ("v_stride_b", ctypes.c_int64),
        ("v_stride_h", ctypes.c_int64),
        ("v_stride_n", ctypes.c_int64),
        ("o_stride_b", ctypes.c_int64),
        ("o_stride_h", ctypes.c_int64),
        ("o_stride_n", ctypes.c_int64),
        ("batch", ctypes.c_int32),
        ("heads_q", ctypes.c_int32),
        ("heads_kv", ctypes.c_int32),
        ("seqlen_q", ctypes.c_int32),
        ("seqlen_k", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("causal", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("kv_dtype", ctypes.c_int32),
        ("cu_seqlens_q", ctypes.c_void_p),
        ("cu_seqlens_k", ctypes.c_void_p),
        ("max_seqlen_q", ctypes.c_int32),
        ("max_seqlen_k", ctypes.c_int32),
        ("lse", ctypes.c_void_p),
        ("lse_stride_b", ctypes.c_int64),
        ("lse_stride_h", ctypes.c_int64),
        ("k_scale", ctypes.c_void_p),
        ("v_scale", ctypes.c_void_p),
        ("scale_stride_b", ctypes.c_int64),
        ("scale_stride_h", ctypes.c_int64),
    ]


class QuantParams(ctypes.Structure):
    """Mirror of ``fa_quant_params`` (include/fused_attn_hip.h)."""

    _fields_ = [
        ("x", ctypes.c_void_p),
        ("x_stride_b", ctypes.c_int64),
        ("x_stride_h", ctypes.c_int64),
        ("x_stride_n", ctypes.c_int64),
        ("batch", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("seqlen", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("x8", ctypes.c_void_p),
        ("scale", ctypes.c_void_p),
    ]


class PagedKV(ctypes.Structure):
    """Mirror of ``fa_paged_kv`` (include/fused_attn_hip.h)."""

    _fields_ = [
        ("block_table", ctypes.c_void_p),
        ("block_table_stride", ctypes.c_int64),
        ("block_table_cols", ctypes.c_int32),
        ("page_size", ctypes.c_int32),
        ("seqlens_k", ctypes.c_void_p),
        ("num_pages", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("k_page_stride", ctypes.c_int64),
        ("v_page_stride", ctypes.c_int64),
    ]


_lib = None
_lib_error: Optional[str] = None
_lock = threading.Lock()


def library_path() -> str:
    """``$FUSED_ATTN_HIP_LIB`` if set, else the in-tree build next to this file."""
    return os.environ.get("FUSED_ATTN_HIP_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)


def _bind(lib: ctypes.CDLL) -> None:
    P = ctypes.POINTER(FwdParams)
    lib.fa_attention_fwd.argtypes = [P, ctypes.c_void_p]
    lib.fa_attention_fwd.restype = ctypes.c_int
    lib.fa_attention_varlen_fwd.argtypes = [P, ctypes.c_void_p]
    lib.fa_attention_varlen_fwd.restype = ctypes.c_int
    lib.fa_splitk_workspace_bytes.argtypes = [ctypes.c_int32] * 5
    lib.fa_splitk_workspace_bytes.restype = ctypes.c_size_t
    lib.fa_attention_splitk.argtypes = [P, ctypes.c_int32, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    lib.fa_attention_splitk.restype = ctypes.c_int
    lib.fa_attention_splitk_noalloc.argtypes = [P, ctypes.c_int32, ctypes.c_void_p]
    lib.fa_attention_splitk_noalloc.restype = ctypes.c_int
    lib.fa_choose_num_splits.argtypes = [ctypes.c_int32] * 5
    lib.fa_choose_num_splits.restype = ctypes.c_int32
    lib.fa_attention_paged_decode.argtypes = [P, ctypes.POINTER(PagedKV), ctypes.c_int32, ctypes.c_void_p,
                                              ctypes.c_size_t, ctypes.c_void_p]
    lib.fa_attention_paged_decode.restype = ctypes.c_int
    lib.fa_quantize_kv_fp8.argtypes = [ctypes.POINTER(QuantParams), ctypes.c_void_p]
    lib.fa_quantize_kv_fp8.restype = ctypes.c_int
    lib.fa_device_supported.argtypes = [ctypes.c_int32]
    lib.fa_device_supported.restype = ctypes.c_int32
    lib.fa_last_error.argtypes = []
    lib.fa_last_error.restype = ctypes.c_char_p
    lib.fa_abi_version.argtypes = []
    lib.fa_abi_version.restype = ctypes.c_int32


def load_library() -> ctypes.CDLL:
    """Load and bind the shared library once; raise RuntimeError if it is unusable."""
    global _lib, _lib_error
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not os.path.exists(path):
            _lib_error = f"{path} not found: build it with `python -c 'import __graft_entry__ as g; g.build()'`"
            raise RuntimeError(f"fused_attn HIP backend unavailable: {_lib_error}")
        try:
            lib = ctypes.CDLL(path)
            _bind(lib)
        except OSError as e:
            _lib_error = str(e)
            raise RuntimeError(f"fused_attn HIP backend unavailable: {e}") from e
        got = lib.fa_abi_version()
        if got != ABI_VERSION:
            _lib_error = f"ABI version mismatch: library {got}, bindings {ABI_VERSION}"
            raise RuntimeError(f"fused_attn HIP backend unavailable: {_lib_error}")
        _lib = lib
        return lib


def library_loaded() -> bool:
    try:
        load_library()
        return True
    except RuntimeError:
        return False


_device_ok: dict[int, bool] = {}


def device_supported(device: torch.device | int | None = None) -> bool:
    """True when the library loads and ``device`` is a gfx950 GPU (has_tensor_core_kernel analogue)."""
    if isinstance(device, torch.device) and device.index is not None:
        ok = _device_ok.get(device.index)  # per-call fast path: the answer is fixed per device
        if ok is not None:
            return ok
    if not torch.cuda.is_available():
        return False
    if device is None:
        idx = torch.cuda.current_device()
    elif isinstance(device, int):
        idx = device
    else:
        idx = torch.device(device).index
        idx = torch.cuda.current_device() if idx is None else idx
    if idx not in _device_ok:
        try:
            _device_ok[idx] = bool(load_library().fa_device_supported(idx))
        except RuntimeError:
            _device_ok[idx] = False
    return _device_ok[idx]


def available() -> bool:
    return device_supported()


def _check(status: int, what: str) -> None:
    if status != FA_OK:
        msg = load_library().fa_last_error().decode(errors="replace")
        raise RuntimeError(f"fused_attn HIP {what} failed ({_STATUS_NAME.get(status, status)}): {msg}")


# ----------------------------------------------------------------------------------------------
# tensor preparation
# ----------------------------------------------------------------------------------------------


TOKEN_STRIDE_LIMIT_BYTES = 1 << 24  # the C ABI's bound on K/V token strides


def _aligned_view(t: torch.Tensor, vec_elems: int, base_align: int) -> torch.Tensor:
    """``t`` itself when its D stride is 1 and its pointer/other strides allow the kernels'
    vector accesses, else a contiguous copy (the kernels never see an unaligned view)."""
    # (fast path: a contiguous tensor's strides are multiples of its last size)
    if (t.is_contiguous() and t.dim() >= 3 and t.size(-1) % vec_elems == 0 and t.data_ptr() % base_align == 0
            and t.stride(2 if t.dim() == 4 else 0) * t.element_size() < TOKEN_STRIDE_LIMIT_BYTES):
        return t
    ok = t.stride(-1) == 1 and t.data_ptr() % base_align == 0
    if ok:
        for i in range(t.dim() - 1):
            if t.size(i) > 1 and t.stride(i) % vec_elems != 0:
                ok = False
                break
    # The kernels address up to 128 K/V rows from a tile start with 32-bit byte offsets, and the
    # C ABI rejects token strides of 16 MiB or more: such a view is copied too.  The token dim is
    # 2 of [B, H, N, D] and 0 of a packed [T, H, D].
    tok = 2 if t.dim() == 4 else 0
    if ok and t.dim() >= 3 and t.size(tok) > 1 and t.stride(tok) * t.element_size() >= TOKEN_STRIDE_LIMIT_BYTES:
        ok = False
    # clone, not contiguous(): an already-contiguous view at an unaligned offset must be copied too
    return t if ok else t.clone(memory_format=torch.contiguous_format)


def _check_qkv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, layout: str, kv_fp8: bool = False) -> None:
    """Reject q/k/v that do not describe one attention problem before anything is launched
    (the reference's check_inputs, csrc/bindings.cpp:35-44, and _check, triton_fwd.py:217-222):
    the kernels take head_dim and the batch from q and the K/V dtype, lengths and heads from k,
    so a V of another shape or dtype, or a K of another head_dim, would be read out of bounds.

    layout: "dense" q [B,Hq,Nq,D], k/v [B or 1,Hkv,Nk,D]; "varlen" q [Tq,Hq,D], k/v [Tk,Hkv,D];
    "paged" q [B,Hq,Nq,D], k/v pools [P,Hkv,page,D]."""
    nd = 3 if layout == "varlen" else 4
    if q.dim() != nd or k.dim() != nd or v.dim() != nd:
        raise RuntimeError(f"expected {nd}-D q, k and v for the {layout} layout, got "
                           f"{tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    if k.shape != v.shape:
        raise RuntimeError(f"k and v must have the same shape, got {tuple(k.shape)} and {tuple(v.shape)}")
    if k.dtype != v.dtype:
        raise RuntimeError(f"k and v must have the same dtype, got {k.dtype} and {v.dtype}")
    if kv_fp8:
        if k.dtype != _FP8:
            raise RuntimeError(f"FP8 K/V must be float8_e4m3fn, got {k.dtype}")
    elif q.dtype != k.dtype:
        raise RuntimeError(f"q/k/v dtypes must match, got {q.dtype} and {k.dtype}")
    if q.shape[-1] != k.shape[-1]:
        raise RuntimeError(f"q and k must have the same head_dim, got {q.shape[-1]} and {k.shape[-1]}")
    hq, hkv = q.shape[-2 if layout == "varlen" else 1], k.shape[-2 if layout == "varlen" else 1]
    if hkv == 0 or hq % hkv != 0:
        raise RuntimeError(f"H_q ({hq}) must be a multiple of H_kv ({hkv})")
    if layout == "dense" and k.shape[0] not in (q.shape[0], 1):
        raise RuntimeError(f"k/v batch ({k.shape[0]}) must equal q's ({q.shape[0]}) or be 1")


def _prep_qkv(q, k, v, kv_fp8: bool = False):
    q = _aligned_view(q, 8, 16)
    kv_vec = 16 if kv_fp8 else 8
    k = _aligned_view(k, kv_vec, 16)
    v = _aligned_view(v, kv_vec, 16)
    return q, k, v


def _new_output(q: torch.Tensor) -> torch.Tensor:
    """A contiguous output of q's shape and dtype, whatever q's strides.

    The custom ops' fake kernels return ``q.new_empty(q.shape)`` (fused_attn/ops.py:102-104), which
    is contiguous, and Inductor checks a custom op's real output against the fake's strides.  The
    reference's ``torch::empty_like`` (csrc/bindings.cpp:56) keeps a ``[B,N,H,D]`` view's strides
    instead, so a compiled graph fed such a view would fail that check; a contiguous output keeps
    eager and compiled calls alike.  The kernels write through the output's strides either way."""
    return torch.empty(q.shape, dtype=q.dtype, device=q.device)


def _check_out(out: torch.Tensor, q: torch.Tensor) -> None:
    """A caller-provided output must be what the kernels write: q's shape, dtype and device, unit
    D stride, 8-byte aligned with 8-byte strides (the C ABI's rule for o).  Checked before anything
    is launched, since a smaller buffer would be written past its end."""
    if tuple(out.shape) != tuple(q.shape):
        raise RuntimeError(f"out must have q's shape {tuple(q.shape)}, got {tuple(out.shape)}")
    if out.dtype != q.dtype:
        raise RuntimeError(f"out must have q's dtype {q.dtype}, got {out.dtype}")
    if out.device != q.device:
        raise RuntimeError(f"out must be on {q.device}, got {out.device}")
    vec = 8 // out.element_size()
    if out.numel() and (out.stride(-1) != 1 or out.data_ptr() % 8
                        or any(out.size(i) > 1 and out.stride(i) % vec for i in range(out.dim() - 1))):
        raise RuntimeError("out needs a unit D stride, an 8-byte aligned start and strides of whole 8-byte words")


def _check_lse_out(lse: torch.Tensor, shape: tuple, device: torch.device) -> None:
    """A caller-provided LSE: fp32 of the given shape on the device, unit stride along the last dim
    (the kernels write it through its first two strides)."""
    if tuple(lse.shape) != tuple(shape):
        raise RuntimeError(f"lse must have shape {tuple(shape)}, got {tuple(lse.shape)}")
    if lse.dtype != torch.float32:
        raise RuntimeError(f"lse must be float32, got {lse.dtype}")
    if lse.device != device:
        raise RuntimeError(f"lse must be on {device}, got {lse.device}")
    if lse.numel() and (lse.size(-1) > 1 and lse.stride(-1) != 1 or lse.stride(0) < 0 or lse.stride(1) < 0):
        raise RuntimeError("lse needs a unit stride along its last dim")


def _stride(t: torch.Tensor, i: int) -> int:
    # a size-1 dim is never stepped over; its stride is irrelevant and passed as 0
    return t.stride(i) if t.size(i) > 1 else 0


def make_params(q, k, v, o, causal: bool, scale: float, *, kv_dtype=None, lse=None, k_scale=None, v_scale=None,
                cu_seqlens_q=None, cu_seqlens_k=None, max_seqlen_q=0, max_seqlen_k=0) -> FwdParams:
    """Fill ``fa_fwd_params`` from tensors.  Dense: q/o [B,Hq,Nq,D], k/v [B,Hkv,Nk,D].
    Varlen: q/o [Tq,Hq,D], k/v [Tk,Hkv,D] with int32 cu_seqlens of length batch+1."""
    if cu_seqlens_q is None:
        # one positional constructor call (filled in C) instead of a Python attribute set per field
        qz, kz, vz, oz = q.shape, k.shape, v.shape, o.shape
        qs, ks, vs, os_ = q.stride(), k.stride(), v.stride(), o.stride()
        p = FwdParams(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
            qs[0] if qz[0] > 1 else 0, qs[1] if qz[1] > 1 else 0, qs[2] if qz[2] > 1 else 0,
            ks[0] if kz[0] > 1 else 0, ks[1] if kz[1] > 1 else 0, ks[2] if kz[2] > 1 else 0,
            vs[0] if vz[0] > 1 else 0, vs[1] if vz[1] > 1 else 0, vs[2] if vz[2] > 1 else 0,
            os_[0] if oz[0] > 1 else 0, os_[1] if oz[1] > 1 else 0, os_[2] if oz[2] > 1 else 0,
            qz[0], qz[1], kz[1], qz[2], kz[2], qz[3])
    else:
        p = FwdParams()
        p.q, p.k, p.v, p.o = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr()
        p.q_stride_b = p.k_stride_b = p.v_stride_b = p.o_stride_b = 0
        p.q_stride_h, p.q_stride_n = _stride(q, 1), _stride(q, 0)
        p.k_stride_h, p.k_stride_n = _stride(k, 1), _stride(k, 0)
        p.v_stride_h, p.v_stride_n = _stride(v, 1), _stride(v, 0)
        p.o_stride_h, p.o_stride_n = _stride(o, 1), _stride(o, 0)
        p.batch = cu_seqlens_q.numel() - 1
        p.heads_q, p.head_dim = q.shape[1], q.shape[2]
        p.heads_kv = k.shape[1]
        p.seqlen_q, p.seqlen_k = int(max_seqlen_q), int(max_seqlen_k)
        p.cu_seqlens_q, p.cu_seqlens_k = cu_seqlens_q.data_ptr(), cu_seqlens_k.data_ptr()
        p.max_seqlen_q, p.max_seqlen_k = int(max_seqlen_q), int(max_seqlen_k)
    p.scale = float(scale)
    p.causal = 1 if causal else 0
    p.dtype = _DTYPE_CODE.get(q.dtype, -1)
    p.kv_dtype = _DTYPE_CODE.get(k.dtype if kv_dtype is None else kv_dtype, -1)
    if lse is not None:
        p.lse = lse.data_ptr()
        p.lse_stride_b, p.lse_stride_h = lse.stride(0), lse.stride(1)
    if k_scale is not None:
        p.k_scale, p.v_scale = k_scale.data_ptr(), v_scale.data_ptr()
        p.scale_stride_b, p.scale_stride_h = k_scale.stride(0), k_scale.stride(1)
    return p


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(t: torch.Tensor) -> int:
    """Handle of the current stream of t's device: the stream the op's work goes on."""
    if _raw_stream is not None:
        return _raw_stream(t.device.index)
    return torch.cuda.current_stream(t.device).cuda_stream


_SAME_DEVICE = contextlib.nullcontext()


def _on_device(dev: torch.device):
    """``torch.cuda.device(dev)``, or no device switch at all when ``dev`` is already current."""
    return _SAME_DEVICE if torch.cuda.current_device() == dev.index else torch.cuda.device(dev)


def _require_gpu(*ts: torch.Tensor) -> None:
    dev = ts[0].device
    if dev.type != "cuda":
        raise RuntimeError("fused_attn HIP backend needs GPU tensors")
    for t in ts[1:]:
        if t.device != dev:
            raise RuntimeError(f"all tensors must be on {dev}, got {t.device}")
    if not device_supported(dev):
        raise RuntimeError(
            f"fused_attn HIP backend unavailable on {dev}: "
            + (_lib_error or "device is not a gfx950 GPU (set FUSED_ATTN_BACKEND=reference to run the unfused path)"))


# ----------------------------------------------------------------------------------------------
# entry points
# ----------------------------------------------------------------------------------------------


def fwd(q, k, v, causal: bool = False, scale: Optional[float] = None, return_lse: bool = False,
        out: Optional[torch.Tensor] = None):
    """Dense FA2 forward.  q [B,Hq,Nq,D]; k, v [B,Hkv,Nk,D]; returns o (and natural-log LSE [B,Hq,Nq])."""
    _check_qkv(q, k, v, "dense")
    if out is not None:
        _check_out(out, q)
    _require_gpu(q, k, v)
    lib = load_library()
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
    q, k, v = _prep_qkv(q, k, v)
    o = _new_output(q) if out is None else out
    lse = torch.empty(q.shape[:3], dtype=torch.float32, device=q.device) if return_lse else None
    p = make_params(q, k, v, o, causal, scale, lse=lse)
    with _on_device(q.device):
        _check(lib.fa_attention_fwd(ctypes.byref(p), ctypes.c_void_p(_stream(q))), "attention_fwd")
    return (o, lse) if return_lse else o


def varlen_fwd(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q: int, max_seqlen_k: int, causal: bool = False,
               scale: Optional[float] = None, out: Optional[torch.Tensor] = None, return_lse: bool = False):
    """Packed varlen forward.  q [Tq,Hq,D]; k, v [Tk,Hkv,D]; cu_seqlens int32 [nseq+1] on the GPU.

    With ``return_lse`` also returns the natural-log LSE as fp32 [Hq, Tq]; rows of tokens outside every
    sequence are left unwritten (like the output rows)."""
    _check_qkv(q, k, v, "varlen")
    if out is not None:
        _check_out(out, q)
    _require_gpu(q, k, v, cu_seqlens_q, cu_seqlens_k)
    if cu_seqlens_q.dtype != torch.int32 or cu_seqlens_k.dtype != torch.int32:
        raise RuntimeError("cu_seqlens must be int32")
    if cu_seqlens_q.numel() != cu_seqlens_k.numel():
        raise RuntimeError("cu_seqlens_q and cu_seqlens_k must have the same length")
    lib = load_library()
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
    q, k, v = _prep_qkv(q, k, v)
    cu_q, cu_k = cu_seqlens_q.contiguous(), cu_seqlens_k.contiguous()
    o = _new_output(q) if out is None else out
    lse = torch.empty((q.shape[1], q.shape[0]), dtype=torch.float32, device=q.device) if return_lse else None
    p = make_params(q, k, v, o, causal, scale, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, max_seqlen_q=max_seqlen_q,
                    max_seqlen_k=max_seqlen_k)
    if lse is not None:  # [Hq, Tq]: head stride Tq, unit token stride
        p.lse = lse.data_ptr()
        p.lse_stride_b, p.lse_stride_h = 0, lse.stride(0)
    with _on_device(q.device):
        _check(lib.fa_attention_varlen_fwd(ctypes.byref(p), ctypes.c_void_p(_stream(q))), "attention_varlen_fwd")
    return (o, lse) if return_lse else o


def _check_fp8_scales(k: torch.Tensor, k_scale, v_scale) -> None:
    """FP8 block scales must be [B_k, Hkv, ceil(Nk / 64)] floats on k's device
    (fused_attn/fp8.py:31-45): the kernel indexes them by (batch, kv-head, 64-key block)."""
    if k_scale is None or v_scale is None:
        raise RuntimeError("FP8 K/V needs k_scale and v_scale")
    want = (k.shape[0], k.shape[1], -(-k.shape[2] // FP8_QBLOCK))
    for name, t in (("k_scale", k_scale), ("v_scale", v_scale)):
        if tuple(t.shape) != want:
            raise RuntimeError(f"{name} must have shape {want} (per 64-key block of k), got {tuple(t.shape)}")
        if not t.is_floating_point() or t.dtype == _FP8:
            raise RuntimeError(f"{name} must be a float tensor, got {t.dtype}")
        if t.device != k.device:
            raise RuntimeError(f"{name} must be on {k.device}, got {t.device}")


def _prep_fp8_scales(k: torch.Tensor, k_scale, v_scale):
    """FP8 block scales as the kernel reads them: fp32 with unit stride along the blocks and the
    same strides for both.  Scales of another float dtype are converted: the kernel reads raw
    fp32 words."""
    if k_scale.dtype != torch.float32 or k_scale.stride(-1) != 1:
        k_scale = k_scale.to(torch.float32).contiguous()
    if v_scale.dtype != torch.float32 or v_scale.stride(-1) != 1:
        v_scale = v_scale.to(torch.float32).contiguous()
    if k_scale.stride() != v_scale.stride():
        k_scale, v_scale = k_scale.contiguous(), v_scale.contiguous()
    return k_scale, v_scale


def split_len_for(seqlen_k: int, num_splits: int, block: int = FP8_QBLOCK) -> int:
    """Split length rounded up to whole ``block``-key tiles (triton_splitk.py:153-154)."""
    num_splits = max(1, int(num_splits))
    per = -(-max(seqlen_k, 1) // num_splits)
    return -(-per // block) * block


def splitk(q, k, v, causal: bool = False, scale: Optional[float] = None, split_len: int = 128,
           k_scale: Optional[torch.Tensor] = None, v_scale: Optional[torch.Tensor] = None,
           workspace: Optional[torch.Tensor] = None, return_lse: bool = False):
    """Split-K flash-decoding + LSE combine.  k/v may be float8_e4m3fn with per-64-key fp32 scales.
    With ``return_lse`` also returns the natural-log LSE, fp32 [B, Hq, Nq] (-inf for rows without keys)."""
    fp8 = _FP8 is not None and k.dtype == _FP8
    _check_qkv(q, k, v, "dense", kv_fp8=fp8)
    if fp8:
        _check_fp8_scales(k, k_scale, v_scale)
    _require_gpu(q, k, v)
    lib = load_library()
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
    q, k, v = _prep_qkv(q, k, v, kv_fp8=fp8)
    if fp8:
        k_scale, v_scale = _prep_fp8_scales(k, k_scale, v_scale)
    o = _new_output(q)
    b, hq, nq, d = q.shape
    nk = k.shape[2]
    splits = -(-nk // split_len) if nk > 0 else 1
    need = lib.fa_splitk_workspace_bytes(b, hq, nq, d, splits)
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(max(need, 16) // 4 + 4, dtype=torch.float32, device=q.device)
    lse = torch.empty((b, hq, nq), dtype=torch.float32, device=q.device) if return_lse else None
    p = make_params(q, k, v, o, causal, scale, k_scale=k_scale if fp8 else None, v_scale=v_scale if fp8 else None,
                    lse=lse)
    with _on_device(q.device):
        _check(lib.fa_attention_splitk(ctypes.byref(p), int(split_len), ctypes.c_void_p(workspace.data_ptr()),
                                       workspace.numel() * workspace.element_size(),
                                       ctypes.c_void_p(_stream(q))), "attention_splitk")
    return (o, lse) if return_lse else o


SPLITK_NOALLOC_MAX_BYTES = 64 << 20  # FA_SPLITK_NOALLOC_MAX_BYTES


def splitk_noalloc(q, k, v, causal: bool = False, scale: Optional[float] = None, split_len: int = 128,
                   k_scale: Optional[torch.Tensor] = None, v_scale: Optional[torch.Tensor] = None,
                   out: Optional[torch.Tensor] = None, return_lse: bool = False,
                   lse: Optional[torch.Tensor] = None):
    """``splitk`` through fa_attention_splitk_noalloc: the library uses its own static per-GPU workspace
    (at most SPLITK_NOALLOC_MAX_BYTES) and allocates nothing; calls overlapping on one GPU race.

    A call that must allocate nothing passes ``out`` ([B,Hq,Nq,D] in q's dtype) and, for the LSE,
    ``lse`` (fp32 [B,Hq,Nq], implies ``return_lse``), with q/k/v (and FP8 scales) already in the
    kernels' layout (unit D stride, 16-byte aligned rows), so that nothing is copied either.  Both are
    checked against q before anything is launched.  Without them they are allocated here."""
    fp8 = _FP8 is not None and k.dtype == _FP8
    _check_qkv(q, k, v, "dense", kv_fp8=fp8)
    if out is not None:
        _check_out(out, q)
    if lse is not None:
        _check_lse_out(lse, q.shape[:3], q.device)
        return_lse = True
    if fp8:
        _check_fp8_scales(k, k_scale, v_scale)
    _require_gpu(q, k, v)
    lib = load_library()
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
    q, k, v = _prep_qkv(q, k, v, kv_fp8=fp8)
    if fp8:
        k_scale, v_scale = _prep_fp8_scales(k, k_scale, v_scale)
    o = _new_output(q) if out is None else out
    if return_lse and lse is None:
        lse = torch.empty(q.shape[:3], dtype=torch.float32, device=q.device)
    p = make_params(q, k, v, o, causal, scale, k_scale=k_scale if fp8 else None, v_scale=v_scale if fp8 else None,
                    lse=lse)
    with _on_device(q.device):
        _check(lib.fa_attention_splitk_noalloc(ctypes.byref(p), int(split_len), ctypes.c_void_p(_stream(q))),
               "attention_splitk_noalloc")
    return (o, lse) if return_lse else o


def _check_paged_fp8_scales(k_cache: torch.Tensor, k_scale, v_scale) -> None:
    """FP8 pools carry 64-key block scales per page, [num_pages, Hkv, page_size / 64] floats on
    the pools' device: the kernel indexes them by (page, kv-head, block inside the page)."""
    if k_scale is None or v_scale is None:
        raise RuntimeError("FP8 pools need k_scale and v_scale")
    if k_cache.shape[2] % FP8_QBLOCK:
        raise RuntimeError(f"FP8 pools need page_size a multiple of {FP8_QBLOCK}, got {k_cache.shape[2]}")
    want = (k_cache.shape[0], k_cache.shape[1], k_cache.shape[2] // FP8_QBLOCK)
    for name, t in (("k_scale", k_scale), ("v_scale", v_scale)):
        if tuple(t.shape) != want:
            raise RuntimeError(f"{name} must have shape {want} (per page, kv-head and 64-key block), "
                               f"got {tuple(t.shape)}")
        if not t.is_floating_point() or t.dtype == _FP8:
            raise RuntimeError(f"{name} must be a float tensor, got {t.dtype}")
        if t.device != k_cache.device:
            raise RuntimeError(f"{name} must be on {k_cache.device}, got {t.device}")


def paged_decode(q, k_cache, v_cache, block_table, seqlens_k, max_seqlen_k: int, causal: bool = False,
                 scale: Optional[float] = None, split_len: int = 128, workspace: Optional[torch.Tensor] = None,
                 return_lse: bool = False, k_scale: Optional[torch.Tensor] = None,
                 v_scale: Optional[torch.Tensor] = None):
    """Split-K decode over a paged cache.  q [B,Hq,Nq,D]; k_cache/v_cache [num_pages, Hkv, page_size, D]
    (any strides with unit D stride); block_table int32 [B, cols]; seqlens_k int32 [B], both on the GPU.
    FP8 pools (float8_e4m3fn) take their block scales k_scale/v_scale [num_pages, Hkv, page_size / 64].
    With ``return_lse`` also returns the natural-log LSE, fp32 [B, Hq, Nq]."""
    if k_cache.shape != v_cache.shape or k_cache.dim() != 4:
        raise RuntimeError("k_cache and v_cache must both be [num_pages, Hkv, page_size, D]")
    fp8 = k_cache.dtype == _FP8
    _check_qkv(q, k_cache, v_cache, "paged", kv_fp8=fp8)
    if fp8:
        _check_paged_fp8_scales(k_cache, k_scale, v_scale)
    _require_gpu(q, k_cache, v_cache, block_table, seqlens_k)
    if block_table.dtype != torch.int32 or seqlens_k.dtype != torch.int32:
        raise RuntimeError("block_table and seqlens_k must be int32")
    if block_table.dim() != 2 or seqlens_k.dim() != 1 or block_table.shape[0] != q.shape[0] \
            or seqlens_k.shape[0] != q.shape[0]:
        raise RuntimeError("block_table must be [B, pages] and seqlens_k [B] for q's batch B")
    lib = load_library()
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
    q, k_cache, v_cache = _prep_qkv(q, k_cache, v_cache, kv_fp8=fp8)
    if fp8:
        k_scale, v_scale = _prep_fp8_scales(k_cache, k_scale, v_scale)
    bt = block_table if block_table.stride(-1) == 1 else block_table.contiguous()
    sl = seqlens_k.contiguous()
    o = _new_output(q)
    b, hq, nq, d = q.shape
    max_k = int(max_seqlen_k)
    splits = -(-max_k // split_len) if max_k > 0 else 1
    need = lib.fa_splitk_workspace_bytes(b, hq, nq, d, splits)
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(max(need, 16) // 4 + 4, dtype=torch.float32, device=q.device)
    lse = torch.empty((b, hq, nq), dtype=torch.float32, device=q.device) if return_lse else None
    p = make_params(q, k_cache, v_cache, o, causal, scale, lse=lse, k_scale=k_scale if fp8 else None,
                    v_scale=v_scale if fp8 else None)
    p.seqlen_k = max_k
    p.k_stride_b = p.v_stride_b = 0
    kv = PagedKV()
    kv.block_table, kv.block_table_stride, kv.block_table_cols = bt.data_ptr(), bt.stride(0), bt.shape[1]
    kv.page_size, kv.num_pages = k_cache.shape[2], k_cache.shape[0]
    kv.seqlens_k = sl.data_ptr()
    kv.k_page_stride, kv.v_page_stride = _stride(k_cache, 0), _stride(v_cache, 0)
    with _on_device(q.device):
        _check(lib.fa_attention_paged_decode(ctypes.byref(p), ctypes.byref(kv), int(split_len),
                                             ctypes.c_void_p(workspace.data_ptr()),
                                             workspace.numel() * workspace.element_size(),
                                             ctypes.c_void_p(_stream(q))), "attention_paged_decode")
    return (o, lse) if return_lse else o


def choose_num_splits(batch: int, heads: int, seqlen_k: int, seqlen_q: int, num_cus: int) -> int:
    return int(load_library().fa_choose_num_splits(batch, heads, seqlen_k, seqlen_q, num_cus))


def workspace_bytes(batch: int, heads_q: int, seqlen_q: int, head_dim: int, num_splits: int) -> int:
    return int(load_library().fa_splitk_workspace_bytes(batch, heads_q, seqlen_q, head_dim, num_splits))


QUANT_HEAD_DIMS = (16, 32, 64, 128, 256)


def quantize_kv_fp8(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Fused FP8 KV quantiser.  x [B,Hkv,N,D] fp32/fp16/bf16 on the GPU -> (float8_e4m3fn
    [B,Hkv,N,D] contiguous, fp32 scales [B,Hkv,ceil(N/64)]), bit-identical to the reference's
    torch chain on the GPU (fused_attn/fp8.py:31-45)."""
    _require_gpu(x)
    if _FP8 is None:
        raise RuntimeError("this torch build has no float8_e4m3fn")
    if x.dim() != 4:
        raise RuntimeError(f"x must be [B, H, N, D], got {tuple(x.shape)}")
    lib = load_library()
    x = _aligned_view(x, 16 // x.element_size(), 16)
    b, h, n, d = x.shape
    nblk = -(-n // FP8_QBLOCK)
    x8 = torch.empty((b, h, n, d), dtype=_FP8, device=x.device)
    scale = torch.empty((b, h, nblk), dtype=torch.float32, device=x.device)
    p = QuantParams()
    p.x, p.x8, p.scale = x.data_ptr(), x8.data_ptr(), scale.data_ptr()
    p.x_stride_b, p.x_stride_h, p.x_stride_n = _stride(x, 0), _stride(x, 1), _stride(x, 2)
    p.batch, p.heads, p.seqlen, p.head_dim = b, h, n, d
    p.dtype = _DTYPE_CODE.get(x.dtype, -1) if x.dtype != _FP8 else -1
    with _on_device(x.device):
        _check(lib.fa_quantize_kv_fp8(ctypes.byref(p), ctypes.c_void_p(_stream(x))), "quantize_kv_fp8")
    return x8, scale
