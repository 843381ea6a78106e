"""The oracle's pins catch plausible mistakes.  CPU only.

Each case plants one mistake (a wrong mask offset, a dropped term, a transposed or swapped
operand, a wrong index, a wrong rounding rule or constant) in a copy of
oracle/attention_oracle.py, loads the copy as its own module, and runs the pin tests of
tests/test_oracle.py against it: every pin named for the mistake must fail.  The same pins
run against the real oracle in the same way and must pass, so a failure of a mutant comes from
the planted mistake and not from the harness.
"""
import inspect
import types

import pytest

import test_oracle as pins
from oracle import attention_oracle as orc

_SOURCE = inspect.getsource(orc)


def _mutant(func: str, old: str, new: str) -> types.ModuleType:
    """A fresh copy of the oracle module with ``old`` replaced by ``new`` once, inside ``func``."""
    fsrc = inspect.getsource(getattr(orc, func))
    assert _SOURCE.count(fsrc) == 1 and fsrc.count(old) == 1, (func, old)
    mod = types.ModuleType(f"attention_oracle_mutant_{func}")
    exec(compile(_SOURCE.replace(fsrc, fsrc.replace(old, new)), mod.__name__, "exec"), mod.__dict__)
    return mod


# (pin test, keyword arguments): the pins of tests/test_oracle.py that each mistake must fail
SDPA_NONCAUSAL = (pins.test_oracle_matches_sdpa, dict(n=17, causal=False))
SDPA_CAUSAL = (pins.test_oracle_matches_sdpa, dict(n=17, causal=True))
GQA = (pins.test_oracle_gqa_equals_repeat_interleave_sdpa, {})
BOTTOM_RIGHT = (pins.test_bottom_right_causal_matches_sdpa_with_explicit_mask, dict(n_q=37, n_k=90))
MORE_Q_THAN_K = (pins.test_bottom_right_causal_matches_sdpa_with_explicit_mask, dict(n_q=90, n_k=40))
BRUTE_RECT = (pins.test_oracle_matches_float64_bruteforce, dict(shape=(1, 4, 1, 37, 90, 16), causal=True))
BRUTE_GQA = (pins.test_oracle_matches_float64_bruteforce, dict(shape=(2, 4, 2, 13, 13, 32), causal=False))
CLOSED = (pins.test_closed_forms, {})
VARLEN_RAGGED = (pins.test_varlen_oracle_matches_bruteforce, dict(lens_q=[8, 16], lens_k=[40, 16]))
VARLEN_EMPTY_K = (pins.test_varlen_oracle_matches_bruteforce, dict(lens_q=[0, 1, 3], lens_k=[2, 1, 0]))
DECODE_TABLE = (pins.test_e4m3fn_decode_table_matches_torch, {})
ENC_TORCH = (pins.test_e4m3fn_encoder_matches_torch_cast, {})
ENC_RNE = (pins.test_e4m3fn_encoder_rounds_to_nearest_even, {})
QUANT_CHAIN = (pins.test_fp8_quantiser_true_division_matches_torch_chain_on_cpu, {})
QUANT_RECIP = (pins.test_fp8_quantiser_reciprocal_scale_is_amax_times_float32_reciprocal, {})
QUANT_AMAX = (pins.test_fp8_scales_equal_blockwise_amax, {})
QUANT_ROUNDTRIP = (pins.test_fp8_roundtrip_bounds_and_scale_shape, {})
FP8_ATTN = (pins.test_fp8_attention_accuracy_vs_fp32, {})
COMBINE = (pins.test_splitk_combine_is_exact, dict(causal=False, split_len=64))
COMBINE_CAUSAL = (pins.test_splitk_combine_is_exact, dict(causal=True, split_len=128))
SPLITS_KAT = (pins.test_choose_num_splits_known_answers, {})
SPLIT_LEN = (pins.test_split_len_alignment, {})
PAGED = (pins.test_paged_oracle_equals_dense_attention_on_the_scattered_keys, dict(causal=True))
LSE_BRUTE = (pins.test_lse_matches_float64_bruteforce, dict(shape=(1, 2, 2, 9, 4, 8), causal=True))
LSE_BRUTE_GQA = (pins.test_lse_matches_float64_bruteforce, dict(shape=(2, 4, 2, 13, 13, 32), causal=False))
LSE_CLOSED = (pins.test_lse_closed_forms, {})
PAGED_OOB = (pins.test_paged_oracle_out_of_pool_pages_read_as_zero_keys, {})
PAGED_FP8 = (pins.test_paged_fp8_oracle_equals_dense_fp8_attention, dict(causal=False))

MUTANTS = {
    # causal mask and its bottom-right alignment (reference.py:24-33)
    "top_left_causal_mask": ("causal_mask", "<= (n_k - n_q)", "<= 0", [BOTTOM_RIGHT, BRUTE_RECT]),
    "causal_mask_off_by_one": ("causal_mask", "<= (n_k - n_q)", "< (n_k - n_q)", [SDPA_CAUSAL, CLOSED]),
    "bruteforce_window_off_by_one": ("attention_f64", "(n_k - n_q) + 1)", "(n_k - n_q))", [BRUTE_RECT]),
    # scores, softmax and the value product (reference.py:36-62)
    "scale_dropped": ("attention", "kf.transpose(-1, -2)) * scale", "kf.transpose(-1, -2))",
                      [SDPA_NONCAUSAL, BRUTE_GQA]),
    "default_scale_1_over_d": ("attention", "1.0 / math.sqrt(d) if", "1.0 / d if", [SDPA_NONCAUSAL]),
    "softmax_over_queries": ("attention", "torch.softmax(s, dim=-1)", "torch.softmax(s, dim=-2)",
                             [SDPA_NONCAUSAL, BRUTE_GQA]),
    "keys_in_place_of_values": ("attention", "torch.matmul(p, vf)", "torch.matmul(p, kf)",
                                [SDPA_NONCAUSAL, BRUTE_GQA]),
    "empty_rows_left_nan": ("attention", "torch.nan_to_num(torch.softmax(s, dim=-1), nan=0.0)",
                            "torch.softmax(s, dim=-1)", [MORE_Q_THAN_K, CLOSED]),
    # natural-log LSE of the scores (triton_fwd.py:169-172)
    "lse_scale_dropped": ("lse", "kf.transpose(-1, -2)) * scale", "kf.transpose(-1, -2))",
                          [LSE_BRUTE_GQA, LSE_CLOSED]),
    "lse_base_2": ("lse", "torch.logsumexp(s, dim=-1)", "torch.logsumexp(s, dim=-1) / math.log(2.0)",
                   [LSE_BRUTE_GQA, LSE_CLOSED]),
    "lse_top_left_mask": ("lse", "~causal_mask(n_q, n_k, device=s.device)", "~causal_mask(n_q, n_q, device=s.device)[:, :n_k]",
                          [LSE_BRUTE]),
    # GQA head mapping (reference.py:16-21): q-head h reads kv-head h // g, not h % Hkv
    "gqa_heads_modulo": ("expand_kv", "torch.repeat_interleave(x, n_rep, dim=1)", "x.repeat(1, n_rep, 1, 1)",
                         [GQA, BRUTE_GQA]),
    # packed sequences (reference.py:65-95)
    "varlen_keys_at_query_offsets": ("attention_varlen", "cu_seqlens_k.tolist()", "cu_seqlens_q.tolist()",
                                     [VARLEN_RAGGED]),
    "varlen_skips_keyless_sequences": ("attention_varlen", "if cq[i + 1] == cq[i]:",
                                       "if cq[i + 1] == cq[i] or ck[i + 1] == ck[i]:", [VARLEN_EMPTY_K]),
    # e4m3fn decode and encode (fp8.py:26-45)
    "e4m3_bias_8": ("e4m3fn_value", "e - 7)", "e - 8)", [DECODE_TABLE]),
    "e4m3_ties_toward_zero": ("e4m3fn_encode", "np.where(lo % 2 == 0, lo, hi)", "lo", [ENC_TORCH, ENC_RNE]),
    "e4m3_ties_away_from_zero": ("e4m3fn_encode", "np.where(lo % 2 == 0, lo, hi)", "hi", [ENC_TORCH, ENC_RNE]),
    "e4m3_overflow_tie_to_nan": ("e4m3fn_encode", "mag <= 464.0", "mag < 464.0", [ENC_TORCH, ENC_RNE]),
    "e4m3_saturating": ("e4m3fn_encode", "np.where(mag <= 464.0, 0x7e, 0x7f)", "0x7e", [ENC_TORCH, ENC_RNE]),
    # block scales (fp8.py:31-45) and dequantisation (fp8.py:48-56)
    "scale_amax_over_447": ("quantize_kv_fp8", "amax / np.float32(E4M3_MAX)", "amax / np.float32(447.0)",
                            [QUANT_CHAIN, QUANT_RECIP]),
    "reciprocal_scale_amax_over_447": ("quantize_kv_fp8", "np.float32(1.0) / np.float32(E4M3_MAX)",
                                       "np.float32(1.0) / np.float32(447.0)", [QUANT_RECIP, QUANT_AMAX]),
    "amax_ignores_nan": ("quantize_kv_fp8",
                         "np.where(np.isnan(a).any(axis=-1), np.float32(np.nan), np.nanmax(a, axis=-1, initial=0.0))",
                         "np.nanmax(a, axis=-1, initial=0.0)", [QUANT_CHAIN]),
    "dequant_scale_blocks_cycled": ("dequantize_kv_fp8", "scale.repeat_interleave(qblock, dim=-1)",
                                    "scale.repeat(1, 1, qblock)", [QUANT_ROUNDTRIP, FP8_ATTN]),
    # split-K partials and the log-sum-exp combine (triton_splitk.py:29-127)
    "combine_without_rescale": ("splitk_combine", "np.exp2(m - ms)", "np.ones_like(m)", [COMBINE, COMBINE_CAUSAL]),
    "combine_natural_exp": ("splitk_combine", "np.exp2(m - ms)", "np.exp(m - ms)", [COMBINE, COMBINE_CAUSAL]),
    "partials_top_left_mask": ("splitk_partials", "j <= i + (n_k - n_q)", "j <= i", [COMBINE_CAUSAL]),
    "partials_natural_exp": ("splitk_partials", "np.exp2(s - ms[:, None])", "np.exp(s - ms[:, None])",
                             [COMBINE, COMBINE_CAUSAL]),
    # split heuristics (triton_splitk.py:130-137, 153-154)
    "num_splits_one_per_sm": ("choose_num_splits", "(2 * num_sms)", "num_sms", [SPLITS_KAT]),
    "num_splits_per_128_keys": ("choose_num_splits", "seqlen_k // 256", "seqlen_k // 128", [SPLITS_KAT]),
    "split_len_rounded_down": ("split_len_for", "-(-per // block) * block", "(per // block) * block", [SPLIT_LEN]),
    # paged gather
    "page_row_from_page_number": ("paged_gather", "cache[pg, :, n % page_size]", "cache[pg, :, n // page_size]",
                                  [PAGED]),
    "negative_page_wraps": ("paged_gather", "if 0 <= pg < num_pages:", "if pg < num_pages:", [PAGED_OOB]),
    # FP8 pools: each pool dequantised with its own scales
    "paged_fp8_scales_swapped": ("attention_paged_fp8", "dequantize_kv_fp8(k8_pool, k_scale_pool)",
                                 "dequantize_kv_fp8(k8_pool, v_scale_pool)", [PAGED_FP8]),
}


def _run(pin, module, monkeypatch):
    fn, kwargs = pin
    with monkeypatch.context() as m:
        m.setattr(pins, "orc", module)
        fn(**kwargs)


@pytest.mark.parametrize("name", sorted(MUTANTS))
def test_pins_fail_on_planted_mistake(name, monkeypatch):
    func, old, new, caught_by = MUTANTS[name]
    if any("fp8" in p[0].__name__ or "e4m3" in p[0].__name__ for p in caught_by) and orc.FP8_DTYPE is None:
        pytest.skip("torch build lacks float8")
    mod = _mutant(func, old, new)
    for pin in caught_by:
        with pytest.raises(AssertionError):
            _run(pin, mod, monkeypatch)


def test_pins_pass_on_the_unchanged_copy(monkeypatch):
    """The harness itself changes nothing: a copy of the oracle loaded the same way passes every pin."""
    mod = _mutant("attention", "torch.matmul(p, vf)", "torch.matmul(p, vf)")
    used = {(p[0].__name__, repr(sorted(p[1].items()))): p for *_, cb in MUTANTS.values() for p in cb}
    for pin in used.values():
        if orc.FP8_DTYPE is None and ("fp8" in pin[0].__name__ or "e4m3" in pin[0].__name__):
            continue
        _run(pin, mod, monkeypatch)
