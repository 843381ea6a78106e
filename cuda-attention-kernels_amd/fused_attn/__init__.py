"""fused_attn: fused multi-head attention for LLM inference on AMD MI355X (gfx950 HIP kernels).

Same public surface as the reference package (fused_attn/__init__.py:2-23):
the ``fused_attn::attention`` custom op, ``attention_varlen``, the unfused
reference, split-K decode and the FP8 KV-cache path.  The ``*_triton`` names
are kept as aliases of the HIP-backed functions.
"""
from .fp8 import attention_fp8, attention_fp8_triton, dequantize_kv_fp8, quantize_kv_fp8
from .ops import attention, attention_varlen, available_backends, pack_varlen
from .paged import attention_paged, attention_paged_reference, paged_from_dense, paged_from_dense_fp8
from .reference import attention_reference, attention_varlen_reference
from .splitk import attention_splitk, attention_splitk_triton, choose_num_splits

__all__ = [
    "attention",
    "attention_varlen",
    "attention_reference",
    "attention_varlen_reference",
    "available_backends",
    "pack_varlen",
    "attention_splitk",
    "attention_splitk_triton",
    "attention_fp8",
    "attention_fp8_triton",
    "quantize_kv_fp8",
    "dequantize_kv_fp8",
    "choose_num_splits",
    "attention_paged",
    "attention_paged_reference",
    "paged_from_dense",
    "paged_from_dense_fp8",
]
__version__ = "0.3.0"
