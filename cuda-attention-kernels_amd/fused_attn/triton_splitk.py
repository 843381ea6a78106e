"""The reference's ``fused_attn.triton_splitk`` entry points, HIP-backed (no Triton).

Callers import ``attention_splitk_triton`` and ``choose_num_splits`` from this module
path (benchmarks/bench_decode.py:48, tests/test_splitk_fp8.py:45); they are the
HIP split-K functions of ``fused_attn.splitk`` under the reference's names.
"""
from .splitk import attention_splitk, attention_splitk_triton, choose_num_splits

__all__ = ["attention_splitk", "attention_splitk_triton", "choose_num_splits"]
