"""Benchmark of the fused attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-decode]

One step = one call of ``fused_attn.attention`` on the causal GQA prefill
workload B=4, Hq=32, Hkv=8, N=4096, D=128, bf16, [B,H,N,D], q/k/v ~ N(0,1)
(the workload the headline metric is quoted on).  Inputs are resident in HBM
before timing starts.  Printed as ONE JSON line:

* ``value``: prefill TFLOP/s = 4*B*Hq*N^2*D/2 / (wall time per step)
  (FLOP convention of benchmarks/bench.py:44-46 in the reference).
* ``roofline``: the prefill kernel's algorithmic FLOPs / its average duration
  from HIP events recorded around every launch on the launch stream, against
  the 2516.6 TFLOP/s dense bf16 MFMA peak (256 CU x 4096 FLOP/clk x 2.4 GHz).
  ``traffic`` is HBM bytes per launch from the rocprofv3 FETCH_SIZE/WRITE_SIZE
  summary committed under profiles/ (null if absent).
* ``decode``: split-K flash-decoding B=32, Hq=32, Hkv=8, n_q=1, n_k=32768,
  D=128 bf16 with 128-key partitions; GB/s = (K+V+Q+O bytes) / time per call,
  against 8 TB/s.  Also the n_q=16 causal spec-decode shape and the FP8 KV
  cache (B=16, Hq=64, Hkv=8, n_k=65536).
* ``cpu_baseline``: the unfused fp32 oracle on the host cores, timed over the
  whole prefill workload one (batch, kv-head group) slice at a time; ``cpu_config0``
  times it in full on the reference's CPU configuration (fp32 B=2 H=4 N=256 D=64
  causal, 2 warm-up + 3 timed calls, benchmarks/bench.py:54-61 in the reference).
* ``max_abs_err`` beside every timed attention workload: against the unfused fp32
  reference backend (fused_attn/reference.py) on one (batch, kv-head group) slice of
  the timed call's output, as the reference's benchmark records it
  (benchmarks/bench.py:87,110-114).
* ``context``: torch's scaled_dot_product_attention on the same GPU and workload
  (flash or memory-efficient backend), and the single-pass prefill kernel on the
  decode shape (benchmarks/bench_decode.py:41-65 in the reference).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "cuda-attention-kernels_amd"))

MFMA_BF16_PEAK_TFLOPS = 2516.6
MFMA_FP32_PEAK_TFLOPS = 157.3  # dense fp32 MFMA peak of MI355X
HBM_PEAK_GBS = 8000.0
PREFILL = dict(b=4, hq=32, hkv=8, n=4096, d=128)
DECODE = dict(b=32, hq=32, hkv=8, nk=32768, d=128)
FP8_DECODE = dict(b=16, hq=64, hkv=8, nk=65536, d=128)
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "prefill_bf16_causal_b4_h32_n4096_d128_traffic.txt")


def attn_flops(b, h, n, d, causal):
    f = 4.0 * b * h * n * n * d
    return f / 2 if causal else f


WARMUP_MIN_S = 0.2  # untimed warm-up per workload: at least this long, and at least `warmup` calls
FIRST_WARMUP_MIN_S = 1.0  # the same for the first timed workload of the process
_warmed = [False]


def _time_calls(fn, steps, warmup):
    """Wall time per call (synchronised both sides) and mean per-launch duration from HIP events.

    Before the timed region the workload runs untimed for ``warmup`` calls and at least
    WARMUP_MIN_S seconds, FIRST_WARMUP_MIN_S for the process's first workload (the reference's
    benchmark warms up by time too: triton's do_bench, benchmarks/bench.py:49-53).  An MI355X takes
    a fraction of a second of load to settle: the causal prefill workload, timed first in a fresh
    process, measured 942-948 TFLOP/s after 0.2 s of warm-up and 1031-1044 after 0.5, 1 or 2 s (the
    same as every later round of it in that process)."""
    import torch

    t_end = time.perf_counter() + (WARMUP_MIN_S if _warmed[0] else FIRST_WARMUP_MIN_S)
    _warmed[0] = True
    done = 0
    while done < warmup or time.perf_counter() < t_end:
        fn()
        done += 1
        if done % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        starts[i].record()
        fn()
        ends[i].record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    ev = sum(s.elapsed_time(e) for s, e in zip(starts, ends)) / steps / 1e3
    return wall, ev


def _ref_err(out, q, k, v, causal, scale=None):
    """max |out - ref| against the unfused fp32 reference backend (fused_attn/reference.py) on the same
    inputs (the reference benchmark's max_abs_err, benchmarks/bench.py:87,110-114)."""
    from fused_attn.reference import attention_reference

    ref = attention_reference(q.float(), k.float(), v.float(), causal=causal, scale=scale)
    return round((out.float() - ref).abs().max().item(), 6)


def _slice_err(out, q, k, v, causal):
    """_ref_err on the first (batch, kv-head group) slice of a [B, H, N, D] call."""
    g = q.shape[1] // k.shape[1]
    return _ref_err(out[:1, :g], q[:1, :g], k[:1, :1], v[:1, :1], causal)


def _batch0_err(out, q, k, v, causal):
    """_ref_err on batch element 0 of a [B, H, N, D] call (every head)."""
    return _ref_err(out[:1], q[:1], k[:1], v[:1], causal)


def _traffic_bytes():
    try:
        text = open(TRAFFIC_FILE).read()
    except OSError:
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", text)
    return float(m.group(1)) if m else None


PREFILL_SETS = 3  # input sets the timed prefill calls rotate through (3 x 335.5 MB > the 256 MiB MALL)


def bench_prefill(steps, warmup, with_sdpa=True):
    """The headline prefill workload; calls rotate through PREFILL_SETS input sets so that no call
    finds its inputs left in the memory-side cache by the previous one."""
    import torch

    import fused_attn

    c = PREFILL
    g = torch.Generator(device="cuda").manual_seed(0)
    sets = []
    for _ in range(PREFILL_SETS):
        q = torch.randn(c["b"], c["hq"], c["n"], c["d"], device="cuda", generator=g).bfloat16()
        k = torch.randn(c["b"], c["hkv"], c["n"], c["d"], device="cuda", generator=g).bfloat16()
        v = torch.randn(c["b"], c["hkv"], c["n"], c["d"], device="cuda", generator=g).bfloat16()
        sets.append((q, k, v))
    q, k, v = sets[0]
    out = fused_attn.attention(q, k, v, causal=True)
    err = _slice_err(out, q, k, v, True)
    del out
    turn = [0]

    def step():
        q, k, v = sets[turn[0] % PREFILL_SETS]
        turn[0] += 1
        return fused_attn.attention(q, k, v, causal=True)

    wall, ev = _time_calls(step, steps, warmup)
    flops = attn_flops(c["b"], c["hq"], c["n"], c["d"], True)
    sdpa = bench_sdpa(sets[0], steps, warmup, flops) if with_sdpa else None
    del sets
    torch.cuda.empty_cache()
    return flops, wall, ev, err, sdpa


def bench_sdpa(qkv, steps, warmup, flops):
    """Context: torch's scaled_dot_product_attention on the same workload and GPU (the reference benchmark's
    torch.sdpa line, benchmarks/bench.py:94-96), restricted to its flash and memory-efficient backends;
    GQA through enable_gqa.  None when neither backend takes the call."""
    import torch
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    q, k, v = qkv
    for be in (SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION):
        try:
            with sdpa_kernel(be):
                fn = lambda: F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True)  # noqa: E731
                out = fn()
                err = _slice_err(out, q, k, v, True)
                del out
                wall, ev = _time_calls(fn, steps, warmup)
        except RuntimeError as e:
            last = f"{type(e).__name__}: {str(e)[:120]}"
            continue
        return {"workload": "torch.nn.functional.scaled_dot_product_attention, same prefill workload (context)",
                "backend": str(be).split(".")[-1], "ms": round(wall * 1e3, 4), "ms_events": round(ev * 1e3, 4),
                "TFLOP_s": round(flops / wall / 1e12, 1), "TFLOP_s_events": round(flops / ev / 1e12, 1),
                "max_abs_err": err}
    return {"workload": "torch sdpa", "skipped": last}


def bench_prefill_extras(steps, warmup):
    """The other prefill configurations (D=64 MHA, the [B,N,H,D] view, the 16-sequence varlen batch), and D=16, 32 and 256."""
    import torch

    import fused_attn

    res = {}
    g = torch.Generator(device="cuda").manual_seed(0)

    def entry(name, workload, fn, flops, err_fn=None):
        out = fn()
        err = err_fn(out) if err_fn is not None else _slice_err(out, q, k, v, True)
        del out
        wall, ev = _time_calls(fn, steps, warmup)
        res[name] = {"workload": workload, "ms": round(wall * 1e3, 4), "ms_events": round(ev * 1e3, 4),
                     "TFLOP_s": round(flops / wall / 1e12, 1),
                     "TFLOP_s_events": round(flops / ev / 1e12, 1),
                     "mfma_frac": round(flops / ev / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4), "max_abs_err": err}

    q = torch.randn(4, 16, 4096, 64, device="cuda", generator=g).bfloat16()
    k = torch.randn(4, 16, 4096, 64, device="cuda", generator=g).bfloat16()
    v = torch.randn(4, 16, 4096, 64, device="cuda", generator=g).bfloat16()
    entry("prefill_d64_mha", "causal MHA prefill B=4 Hq=Hkv=16 N=4096 D=64 bf16",
          lambda: fused_attn.attention(q, k, v, causal=True), attn_flops(4, 16, 4096, 64, True))
    q = torch.randn(4, 16, 4096, 32, device="cuda", generator=g).bfloat16()
    k = torch.randn(4, 16, 4096, 32, device="cuda", generator=g).bfloat16()
    v = torch.randn(4, 16, 4096, 32, device="cuda", generator=g).bfloat16()
    entry("prefill_d32_mha", "causal MHA prefill B=4 Hq=Hkv=16 N=4096 D=32 bf16",
          lambda: fused_attn.attention(q, k, v, causal=True), attn_flops(4, 16, 4096, 32, True))
    q, k, v = (x[..., :16].contiguous() for x in (q, k, v))
    entry("prefill_d16_mha", "causal MHA prefill B=4 Hq=Hkv=16 N=4096 D=16 bf16",
          lambda: fused_attn.attention(q, k, v, causal=True), attn_flops(4, 16, 4096, 16, True))
    q = torch.randn(2, 16, 4096, 256, device="cuda", generator=g).bfloat16()
    k = torch.randn(2, 4, 4096, 256, device="cuda", generator=g).bfloat16()
    v = torch.randn(2, 4, 4096, 256, device="cuda", generator=g).bfloat16()
    entry("prefill_d256_gqa", "causal GQA prefill B=2 Hq=16 Hkv=4 N=4096 D=256 bf16",
          lambda: fused_attn.attention(q, k, v, causal=True), attn_flops(2, 16, 4096, 256, True))
    c = PREFILL
    q = torch.randn(c["b"], c["hq"], c["n"], c["d"], device="cuda", generator=g)
    k = torch.randn(c["b"], c["hkv"], c["n"], c["d"], device="cuda", generator=g)
    v = torch.randn(c["b"], c["hkv"], c["n"], c["d"], device="cuda", generator=g)
    flops = attn_flops(c["b"], c["hq"], c["n"], c["d"], True)
    entry("prefill_fp32", f"causal GQA prefill B={c['b']} Hq={c['hq']} Hkv={c['hkv']} N={c['n']} D={c['d']} fp32",
          lambda: fused_attn.attention(q, k, v, causal=True), flops)
    res["prefill_fp32"]["mfma_fp32_frac"] = round(flops / (res["prefill_fp32"]["ms_events"] * 1e-3) / 1e12
                                                  / MFMA_FP32_PEAK_TFLOPS, 4)
    q = torch.randn(c["b"], c["n"], c["hq"], c["d"], device="cuda", generator=g).bfloat16().transpose(1, 2)
    k = torch.randn(c["b"], c["n"], c["hkv"], c["d"], device="cuda", generator=g).bfloat16().transpose(1, 2)
    v = torch.randn(c["b"], c["n"], c["hkv"], c["d"], device="cuda", generator=g).bfloat16().transpose(1, 2)
    entry("prefill_bnhd_view", f"causal GQA prefill B={c['b']} Hq={c['hq']} Hkv={c['hkv']} N={c['n']} D={c['d']} bf16, "
          "[B,N,H,D] storage viewed as [B,H,N,D]",
          lambda: fused_attn.attention(q, k, v, causal=True), attn_flops(c["b"], c["hq"], c["n"], c["d"], True))
    lens = torch.randint(0, 4097, (16,), generator=torch.Generator().manual_seed(0)).tolist()
    lens[0], lens[1] = 0, 1
    total = sum(lens)
    q = torch.randn(total, 32, 128, device="cuda", generator=g).bfloat16()
    k = torch.randn(total, 8, 128, device="cuda", generator=g).bfloat16()
    v = torch.randn(total, 8, 128, device="cuda", generator=g).bfloat16()
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32, device="cuda")
    mx = max(lens)
    def varlen_err(out):  # the two longest sequences, per sequence against the reference backend
        errs = []
        for i in sorted(range(len(lens)), key=lambda i: -lens[i])[:2]:
            s, e = int(cu[i]), int(cu[i + 1])
            seq = [x[s:e].transpose(0, 1)[None] for x in (q, k, v)]
            errs.append(_ref_err(out[s:e].transpose(0, 1)[None], *seq, True))
        return max(errs)

    entry("varlen_prefill", f"varlen causal prefill, 16 sequences (lengths U[0,4096] by seed 0, one 0, one 1; "
          f"{total} tokens) Hq=32 Hkv=8 D=128 bf16",
          lambda: fused_attn.attention_varlen(q, k, v, cu, cu, mx, mx, causal=True),
          sum(attn_flops(1, 32, n, 128, True) for n in lens), err_fn=varlen_err)
    return res


def bench_decode(steps, warmup, only_128=False):
    import torch

    import fused_attn

    res = {}
    c = DECODE
    g = torch.Generator(device="cuda").manual_seed(0)
    k = torch.randn(c["b"], c["hkv"], c["nk"], c["d"], device="cuda", generator=g).bfloat16()
    v = torch.randn(c["b"], c["hkv"], c["nk"], c["d"], device="cuda", generator=g).bfloat16()
    cases = ((1, False, 128),) if only_128 else ((1, False, 128), (16, True, 128), (1, False, None), (16, True, None))
    for nq, causal, split in cases:
        q = torch.randn(c["b"], c["hq"], nq, c["d"], device="cuda", generator=g).bfloat16()
        fn = lambda: fused_attn.attention_splitk(q, k, v, causal=causal, split_len=split)  # noqa: E731
        err = _batch0_err(fn(), q, k, v, causal)
        wall, ev = _time_calls(fn, steps, warmup)
        nbytes = 2 * k.numel() * 2 + 2 * q.numel() * 2
        key = ("decode" if nq == 1 else "spec_decode_nq16") + ("" if split else "_default_split")
        keys = split or fused_attn.ops.default_split_len(nq, c["nk"], c["b"], c["hkv"], c["hq"] // c["hkv"])
        res[key] = {
            "workload": f"split-K B={c['b']} Hq={c['hq']} Hkv={c['hkv']} n_q={nq} n_k={c['nk']} D={c['d']} bf16"
                        f"{' causal' if causal else ''}, {keys}-key partitions + LSE combine"
                        f"{'' if split else ' (default partition policy)'}",
            "ms": round(wall * 1e3, 4), "GB_s": round(nbytes / wall / 1e9, 1),
            "GB_s_events": round(nbytes / ev / 1e9, 1), "bytes": nbytes,
            "hbm_frac": round(nbytes / wall / 1e9 / HBM_PEAK_GBS, 4),
            "hbm_frac_events": round(nbytes / ev / 1e9 / HBM_PEAK_GBS, 4), "max_abs_err": err,
        }
    if only_128:
        return res
    # context: the single-pass prefill kernel on the n_q = 1 decode shape (the reference's bench_decode
    # prints single-pass beside split-K and FP8 per context length, benchmarks/bench_decode.py:41-65)
    q = torch.randn(c["b"], c["hq"], 1, c["d"], device="cuda", generator=g).bfloat16()
    fn = lambda: fused_attn._hip.fwd(q, k, v)  # noqa: E731
    err = _batch0_err(fn(), q, k, v, False)
    wall, ev = _time_calls(fn, max(3, steps // 4), warmup)
    nbytes = 2 * k.numel() * 2 + 2 * q.numel() * 2
    res["single_pass_decode"] = {
        "workload": f"single-pass prefill kernel on the decode shape B={c['b']} Hq={c['hq']} Hkv={c['hkv']} n_q=1 "
                    f"n_k={c['nk']} D={c['d']} bf16 (context: no key split)",
        "ms": round(wall * 1e3, 4), "GB_s": round(nbytes / wall / 1e9, 1),
        "GB_s_events": round(nbytes / ev / 1e9, 1), "bytes": nbytes,
        "hbm_frac": round(nbytes / wall / 1e9 / HBM_PEAK_GBS, 4),
            "hbm_frac_events": round(nbytes / ev / 1e9 / HBM_PEAK_GBS, 4), "max_abs_err": err,
    }
    res.update(bench_paged(k, v, steps, warmup, g))
    res.update(bench_paged(k, v, steps, warmup, g, page_size=16, splits=(128,), suffix="_16key_pages"))
    del k, v
    torch.cuda.empty_cache()
    c = FP8_DECODE
    q = torch.randn(c["b"], c["hq"], 1, c["d"], device="cuda", generator=g).bfloat16()
    k8, ks = fused_attn.quantize_kv_fp8(torch.randn(c["b"], c["hkv"], c["nk"], c["d"], device="cuda", generator=g))
    v8, vs = fused_attn.quantize_kv_fp8(torch.randn(c["b"], c["hkv"], c["nk"], c["d"], device="cuda", generator=g))
    torch.cuda.empty_cache()
    from fused_attn.fp8 import dequantize_kv_fp8

    kd0, vd0 = dequantize_kv_fp8(k8[:1], ks[:1]), dequantize_kv_fp8(v8[:1], vs[:1])
    for split in (128, None):
        fn = lambda: fused_attn.attention_fp8(q, k8, ks, v8, vs, split_len=split)  # noqa: E731
        err = _ref_err(fn()[:1], q[:1], kd0, vd0, False)  # against the reference on the dequantised cache
        wall, ev = _time_calls(fn, steps, warmup)
        nbytes = 2 * k8.numel() + 2 * ks.numel() * 4 + 2 * q.numel() * 2
        keys = split or fused_attn.ops.default_split_len(1, c["nk"], c["b"], c["hkv"], c["hq"] // c["hkv"])
        res["fp8_decode" + ("" if split else "_default_split")] = {
            "workload": f"FP8-KV split-K B={c['b']} Hq={c['hq']} Hkv={c['hkv']} n_q=1 n_k={c['nk']} D={c['d']}, "
                        f"e4m3fn + fp32 per-64-key scales, {keys}-key partitions"
                        f"{'' if split else ' (default partition policy)'}",
            "ms": round(wall * 1e3, 4), "GB_s": round(nbytes / wall / 1e9, 1),
            "GB_s_events": round(nbytes / ev / 1e9, 1), "bytes": nbytes,
            "hbm_frac": round(nbytes / wall / 1e9 / HBM_PEAK_GBS, 4),
            "hbm_frac_events": round(nbytes / ev / 1e9 / HBM_PEAK_GBS, 4), "max_abs_err": err,
        }
    # the same FP8 cache scattered into a shuffled pool of 64-key pages with per-page block scales
    kc, vc, ksp, vsp, bt, sl = fused_attn.paged_from_dense_fp8(k8, ks, v8, vs, 64,
                                                               generator=torch.Generator().manual_seed(0))
    for split in (128, None):
        keys = split or fused_attn.ops.default_split_len(1, c["nk"], c["b"], c["hkv"], c["hq"] // c["hkv"])
        fn = lambda: fused_attn.attention_paged(q, kc, vc, bt, sl, max_seqlen_k=c["nk"], split_len=keys,  # noqa: E731
                                                k_scale=ksp, v_scale=vsp)
        err = _ref_err(fn()[:1], q[:1], kd0, vd0, False)
        wall, ev = _time_calls(fn, steps, warmup)
        nbytes = 2 * kc.numel() + 2 * ksp.numel() * 4 + 2 * q.numel() * 2 + bt.numel() * 4
        res["paged_fp8_decode" + ("" if split else "_default_split")] = {
            "workload": f"paged FP8-KV split-K B={c['b']} Hq={c['hq']} Hkv={c['hkv']} n_q=1 n_k={c['nk']} D={c['d']}, "
                        f"64-key e4m3fn pages in shuffled order with per-page fp32 block scales, {keys}-key partitions"
                        f"{'' if split else ' (default partition policy)'}",
            "ms": round(wall * 1e3, 4), "GB_s": round(nbytes / wall / 1e9, 1),
            "GB_s_events": round(nbytes / ev / 1e9, 1), "bytes": nbytes,
            "hbm_frac": round(nbytes / wall / 1e9 / HBM_PEAK_GBS, 4),
            "hbm_frac_events": round(nbytes / ev / 1e9 / HBM_PEAK_GBS, 4), "max_abs_err": err,
        }
    del q, k8, ks, v8, vs, kd0, vd0, kc, vc, ksp, vsp
    torch.cuda.empty_cache()
    res.update(bench_decode_d256(steps, warmup, g))
    return res


DECODE_SWEEP = dict(b=1, hq=32, hkv=8, d=128, ctx=(4096, 16384, 65536))
PREFILL_SWEEP = dict(b=2, hq=32, hkv=8, d=128, n=(2048, 8192, 16384))


def bench_decode_sweep(steps, warmup):
    """Single-sequence decode across context lengths (the reference's decode benchmark,
    benchmarks/bench_decode.py:30-65: batch 1, Hq=32, Hkv=8, D=128, one fp16 query, causal, contexts
    4096/16384/65536): the single-pass prefill kernel, split-K with the reference's split heuristic
    (choose_num_splits over the GPU's 256 CUs), split-K with attention_splitk's default partitions, and
    the FP8 KV cache at its default partitions.  GB/s counts each variant's own K/V (+ scale) bytes."""
    import torch

    import fused_attn
    from fused_attn.fp8 import dequantize_kv_fp8
    from fused_attn.triton_fwd import attention_triton

    c = DECODE_SWEEP
    g = torch.Generator(device="cuda").manual_seed(0)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    res = {}
    for n in c["ctx"]:
        q = torch.randn(c["b"], c["hq"], 1, c["d"], device="cuda", generator=g).half()
        k = torch.randn(c["b"], c["hkv"], n, c["d"], device="cuda", generator=g).half()
        v = torch.randn(c["b"], c["hkv"], n, c["d"], device="cuda", generator=g).half()
        k8, ks = fused_attn.quantize_kv_fp8(k)
        v8, vs = fused_attn.quantize_kv_fp8(v)
        kd, vd = dequantize_kv_fp8(k8, ks), dequantize_kv_fp8(v8, vs)
        kv16 = 2 * k.numel() * 2
        kv8 = 2 * k8.numel() + 2 * ks.numel() * 4
        splits = fused_attn.choose_num_splits(c["b"], c["hq"], n, 1, cus)
        default = fused_attn.ops.default_split_len(1, n, c["b"], c["hkv"], c["hq"] // c["hkv"])
        variants = (
            ("single_pass", "single-pass prefill kernel (no key split)",
             lambda: attention_triton(q, k, v, causal=True), kv16, (k, v)),
            ("splitk_ref_heuristic", f"split-K, {splits} splits (the reference's choose_num_splits over {cus} CUs)",
             lambda: fused_attn.attention_splitk(q, k, v, causal=True, num_splits=splits), kv16, (k, v)),
            # called as the reference's benchmark calls its split-K function (bench_decode.py:53-54), not
            # through the custom op, whose dispatch adds host time the other rows do not pay
            ("splitk_default", f"split-K, {default}-key partitions (attention_splitk's default policy)",
             lambda: fused_attn.attention_splitk(q, k, v, causal=True), kv16, (k, v)),
            ("fp8_kv", "FP8-KV split-K (e4m3fn + fp32 per-64-key scales), default partitions",
             lambda: fused_attn.attention_fp8(q, k8, ks, v8, vs, causal=True), kv8, (kd, vd)),
        )
        row = {}
        for name, what, fn, nbytes, (kr, vr) in variants:
            err = _ref_err(fn(), q, kr, vr, True)
            wall, ev = _time_calls(fn, steps, warmup)
            row[name] = {"workload": what, "ms": round(wall * 1e3, 4), "ms_events": round(ev * 1e3, 4),
                         "GB_s": round(nbytes / wall / 1e9, 1), "bytes": nbytes,
                         "hbm_frac": round(nbytes / wall / 1e9 / HBM_PEAK_GBS, 4), "max_abs_err": err}
        res[f"ctx{n}"] = row
        del q, k, v, k8, ks, v8, vs, kd, vd
        torch.cuda.empty_cache()
    return {"workload": f"decode B={c['b']} Hq={c['hq']} Hkv={c['hkv']} n_q=1 D={c['d']} fp16 causal, contexts "
                        f"{'/'.join(map(str, c['ctx']))}", **res}


def bench_prefill_sweep(steps, warmup):
    """The reference README's prefill table shape (README.md:167-175, filled by benchmarks/bench.py:64-127):
    causal bf16 B=2 Hq=32 Hkv=8 D=128 at N = 2048, 8192, 16384."""
    import torch

    import fused_attn

    c = PREFILL_SWEEP
    g = torch.Generator(device="cuda").manual_seed(0)
    res = {}
    for n in c["n"]:
        q = torch.randn(c["b"], c["hq"], n, c["d"], device="cuda", generator=g).bfloat16()
        k = torch.randn(c["b"], c["hkv"], n, c["d"], device="cuda", generator=g).bfloat16()
        v = torch.randn(c["b"], c["hkv"], n, c["d"], device="cuda", generator=g).bfloat16()
        fn = lambda: fused_attn.attention(q, k, v, causal=True)  # noqa: E731
        err = _slice_err(fn(), q, k, v, True)
        wall, ev = _time_calls(fn, steps, warmup)
        flops = attn_flops(c["b"], c["hq"], n, c["d"], True)
        res[f"N{n}"] = {"ms": round(wall * 1e3, 4), "ms_events": round(ev * 1e3, 4),
                        "TFLOP_s": round(flops / wall / 1e12, 1), "TFLOP_s_events": round(flops / ev / 1e12, 1),
                        "mfma_frac": round(flops / wall / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4), "max_abs_err": err}
        del q, k, v
        torch.cuda.empty_cache()
    return {"workload": f"causal prefill B={c['b']} Hq={c['hq']} Hkv={c['hkv']} D={c['d']} bf16, "
                        f"N={'/'.join(map(str, c['n']))}", **res}


def bench_decode_d256(steps, warmup, g):
    """Split-K decode at head dim 256: B=8 Hq=32 Hkv=8 n_k=32768 bf16 (2.147 GB of K+V), 128-key partitions."""
    import torch

    import fused_attn

    b, hq, hkv, nk, d = 8, 32, 8, 32768, 256
    k = torch.randn(b, hkv, nk, d, device="cuda", generator=g).bfloat16()
    v = torch.randn(b, hkv, nk, d, device="cuda", generator=g).bfloat16()
    q = torch.randn(b, hq, 1, d, device="cuda", generator=g).bfloat16()
    fn = lambda: fused_attn.attention_splitk(q, k, v, split_len=128)  # noqa: E731
    err = _batch0_err(fn(), q, k, v, False)
    wall, ev = _time_calls(fn, steps, warmup)
    nbytes = 2 * k.numel() * 2 + 2 * q.numel() * 2
    res = {"decode_d256": {"max_abs_err": err,
        "workload": f"split-K B={b} Hq={hq} Hkv={hkv} n_q=1 n_k={nk} D={d} bf16, 128-key partitions + LSE combine",
        "ms": round(wall * 1e3, 4), "GB_s": round(nbytes / wall / 1e9, 1),
        "GB_s_events": round(nbytes / ev / 1e9, 1), "bytes": nbytes,
        "hbm_frac": round(nbytes / wall / 1e9 / HBM_PEAK_GBS, 4),
            "hbm_frac_events": round(nbytes / ev / 1e9 / HBM_PEAK_GBS, 4),
    }}
    del q, k, v
    torch.cuda.empty_cache()
    return res


def bench_paged(k, v, steps, warmup, g, page_size=64, splits=(128, None), suffix=""):
    """Split-K decode over the same K/V scattered into a shuffled pool of `page_size`-key pages."""
    import torch

    import fused_attn

    c = DECODE
    kc, vc, bt, sl = fused_attn.paged_from_dense(k, v, page_size, generator=torch.Generator().manual_seed(0))
    q = torch.randn(c["b"], c["hq"], 1, c["d"], device="cuda", generator=g).bfloat16()
    res = {}
    for split in splits:
        keys = split or fused_attn.ops.default_split_len(1, c["nk"], c["b"], c["hkv"], c["hq"] // c["hkv"])
        keys = min(keys, max(64, (254 * page_size) // 64 * 64))  # as the op caps it for small pages
        fn = lambda: fused_attn.attention_paged(q, kc, vc, bt, sl, max_seqlen_k=c["nk"], split_len=keys)  # noqa: E731
        err = _batch0_err(fn(), q, k, v, False)  # the pool holds the dense K/V, shuffled into pages
        wall, ev = _time_calls(fn, steps, warmup)
        nbytes = 2 * kc.numel() * 2 + 2 * q.numel() * 2 + bt.numel() * 4
        res["paged_decode" + suffix + ("" if split else "_default_split")] = {
            "workload": f"paged split-K B={c['b']} Hq={c['hq']} Hkv={c['hkv']} n_q=1 n_k={c['nk']} D={c['d']} bf16, "
                        f"{page_size}-key pages in shuffled order, {keys}-key partitions + LSE combine"
                        f"{'' if split else ' (default partition policy)'}",
            "ms": round(wall * 1e3, 4), "GB_s": round(nbytes / wall / 1e9, 1),
            "GB_s_events": round(nbytes / ev / 1e9, 1), "bytes": nbytes,
            "hbm_frac": round(nbytes / wall / 1e9 / HBM_PEAK_GBS, 4),
            "hbm_frac_events": round(nbytes / ev / 1e9 / HBM_PEAK_GBS, 4), "max_abs_err": err,
        }
    return res


def bench_quantize(steps, warmup):
    """The fused FP8 KV quantiser over one K cache of the FP8 decode workload (bf16 in, e4m3fn + scales out)."""
    import torch

    import fused_attn

    c = FP8_DECODE
    g = torch.Generator(device="cuda").manual_seed(0)
    x = torch.randn(c["b"], c["hkv"], c["nk"], c["d"], device="cuda", generator=g).bfloat16()
    # correctness beside the timing: bytes and scales of batch element 0 against the reference's torch chain
    from fused_attn.fp8 import _quantize_kv_fp8_torch

    x8, sc = fused_attn.quantize_kv_fp8(x)
    r8, rs = _quantize_kv_fp8_torch(x[:1])
    mismatches = int((x8[:1].view(torch.uint8) != r8.view(torch.uint8)).sum().item()) + \
        int((sc[:1] != rs).sum().item())
    del x8, sc, r8, rs
    wall, ev = _time_calls(lambda: fused_attn.quantize_kv_fp8(x), steps, warmup)
    nblk = -(-c["nk"] // 64)
    nbytes = x.numel() * 2 + x.numel() + c["b"] * c["hkv"] * nblk * 4
    return {
        "workload": f"FP8 KV quantiser B={c['b']} Hkv={c['hkv']} N={c['nk']} D={c['d']}: bf16 -> e4m3fn + fp32 "
                    "per-64-key scales",
        "kernel": "quantize_kv_fp8_kernel<bf16,128>",
        "ms": round(wall * 1e3, 4), "GB_s": round(nbytes / wall / 1e9, 1),
        "GB_s_events": round(nbytes / ev / 1e9, 1), "bytes": nbytes,
        "hbm_frac": round(nbytes / wall / 1e9 / HBM_PEAK_GBS, 4),
            "hbm_frac_events": round(nbytes / ev / 1e9 / HBM_PEAK_GBS, 4),
        "mismatches_vs_torch_chain": mismatches,
    }


def cpu_config0():
    """The reference's CPU configuration in full: dense causal MHA fp32 B=2 Hq=Hkv=4 n_q=n_k=256 D=64,
    q/k/v ~ N(0,1) from torch.manual_seed(0), through the fp32 oracle on the host cores; 2 warm-up and 3
    timed calls, as the reference times its CPU path (benchmarks/bench.py:54-61)."""
    import torch

    sys.path.insert(0, ROOT)
    from oracle import attention_oracle as orc

    torch.set_num_threads(int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)))
    torch.manual_seed(0)
    q, k, v = (torch.randn(2, 4, 256, 64) for _ in range(3))
    for _ in range(2):
        orc.attention(q, k, v, causal=True)
    t0 = time.perf_counter()
    for _ in range(3):
        orc.attention(q, k, v, causal=True)
    dt = (time.perf_counter() - t0) / 3
    flops = attn_flops(2, 4, 256, 64, True)
    return {"workload": "causal MHA fp32 B=2 Hq=Hkv=4 n_q=n_k=256 D=64 (the reference's CPU configuration), "
                        "unfused fp32 oracle, 2 warm-up + 3 timed calls",
            "ms": round(dt * 1e3, 4), "TFLOP_s": round(flops / dt / 1e12, 6), "cores": torch.get_num_threads(),
            "kind": "port"}


def cpu_baseline(passes=3):
    """The fp32 oracle on host cores over the whole prefill workload, one (batch, kv-head group) slice
    at a time (the unfused oracle materialises a [G, N, N] fp32 score matrix per slice)."""
    import torch

    sys.path.insert(0, ROOT)
    from oracle import attention_oracle as orc

    torch.set_num_threads(int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)))
    c = PREFILL
    g = c["hq"] // c["hkv"]
    n_slices = c["b"] * c["hkv"]
    gen = torch.Generator().manual_seed(0)
    slices = [(torch.randn(1, g, c["n"], c["d"], generator=gen).bfloat16(),
               torch.randn(1, 1, c["n"], c["d"], generator=gen).bfloat16(),
               torch.randn(1, 1, c["n"], c["d"], generator=gen).bfloat16()) for _ in range(n_slices)]
    orc.attention(*slices[0], causal=True)  # warm-up
    t0 = time.perf_counter()
    for _ in range(passes):
        for q, k, v in slices:
            orc.attention(q, k, v, causal=True)
    dt = (time.perf_counter() - t0) / passes
    flops = attn_flops(c["b"], c["hq"], c["n"], c["d"], True)
    return {
        "value": round(flops / dt / 1e12, 5), "unit": "TFLOP/s", "cores": torch.get_num_threads(), "kind": "port",
        "sample": f"unfused fp32 oracle over the whole prefill workload (B={c['b']} Hq={c['hq']} Hkv={c['hkv']} "
                  f"N={c['n']} D={c['d']} causal, bf16 inputs), one of its {n_slices} (batch, kv-head group) slices "
                  f"at a time; {passes} timed passes after one warm-up slice, {dt:.2f} s per pass",
        "ms_per_step": round(dt * 1e3, 1),
    }


def copy_calibration(steps, warmup, nbytes=1 << 30):
    """A plain device copy of known size: the yardstick for the PMC byte counters (FETCH_SIZE, WRITE_SIZE)."""
    import torch

    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    wall, ev = _time_calls(lambda: dst.copy_(src), steps, warmup)
    return wall, ev, nbytes


def run_only(which, steps, warmup):
    if which == "prefill":
        flops, wall, ev, _, _ = bench_prefill(steps, warmup, with_sdpa=False)
        print(f"prefill: {flops / ev / 1e12:.1f} TFLOP/s kernel, {ev * 1e3:.4f} ms", flush=True)
    elif which == "prefill_other":
        print(json.dumps(bench_prefill_extras(steps, warmup)), flush=True)
    elif which == "prefill_sweep":
        print(json.dumps(bench_prefill_sweep(steps, warmup)), flush=True)
    elif which == "decode_sweep":
        print(json.dumps(bench_decode_sweep(steps, warmup)), flush=True)
    elif which == "quantize":
        print(json.dumps(bench_quantize(steps, warmup)), flush=True)
    elif which == "mfma_ceiling":
        print(json.dumps(bench_mfma_ceiling(steps, warmup)), flush=True)
    elif which in ("decode", "decode128"):
        print(json.dumps(bench_decode(steps, warmup, only_128=which == "decode128")), flush=True)
    else:
        wall, ev, nbytes = copy_calibration(steps, warmup)
        print(f"copy {nbytes} B: {ev * 1e3:.4f} ms, {2 * nbytes / ev / 1e9:.1f} GB/s read+write", flush=True)


CEILING_ITERS = 4000  # rounds of four MFMAs per wave: about 0.6 ms per launch, like the prefill kernel


def bench_mfma_ceiling(steps, warmup, prefill_tflops=None):
    """What the matrix cores sustain on this board: the probe kernel of fa_ceiling.hip (libfa_probe.so)
    streams independent v_mfma_f32_32x32x16_bf16 on register operands of random bf16 data, eight waves
    per CU as the 8-wave prefill kernel runs, with no memory, LDS or vector work.  Timed like the other
    workloads; its rate is the practical ceiling for the prefill loop's matrix work (the board's clock
    under MFMA load included), beside the spec peak that roofline.frac uses."""
    import ctypes

    import torch

    lib = ctypes.CDLL(os.path.join(ROOT, "cuda-attention-kernels_amd", "fused_attn", "libfa_probe.so"))
    lib.fa_probe_mfma_ceiling.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_void_p]
    lib.fa_probe_data_elems.restype = ctypes.c_int
    g = torch.Generator(device="cuda").manual_seed(0)
    data = torch.randn(lib.fa_probe_data_elems(), device="cuda", generator=g).bfloat16()
    grid = torch.cuda.get_device_properties(0).multi_processor_count
    out = torch.empty(grid * 512, dtype=torch.float32, device="cuda")

    def launch():
        rc = lib.fa_probe_mfma_ceiling(ctypes.c_void_p(data.data_ptr()), ctypes.c_void_p(out.data_ptr()), grid,
                                       CEILING_ITERS, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        if rc != 0:
            raise RuntimeError(f"mfma ceiling probe launch failed ({rc})")

    wall, ev = _time_calls(launch, steps, warmup)
    flops = float(grid) * 8 * CEILING_ITERS * 4 * (2 * 32 * 32 * 16)
    tflops = flops / ev / 1e12
    res = {"workload": f"v_mfma_f32_32x32x16_bf16 only, register operands of random bf16 data, {grid} workgroups "
                       f"of 8 waves (one per CU), {CEILING_ITERS} x 4 MFMAs per wave",
           "TFLOP_s": round(tflops, 1), "ms": round(ev * 1e3, 4), "frac_of_peak": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4)}
    if prefill_tflops is not None:
        res["prefill_frac_of_ceiling"] = round(prefill_tflops / tflops, 4)
    return res


def main():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--no-decode", action="store_true")
    p.add_argument("--only", choices=["prefill", "prefill_other", "prefill_sweep", "decode", "decode128",
                                      "decode_sweep", "quantize", "copy", "mfma_ceiling"],
                   default=None,
                   help="run one workload without the JSON line (for profiler runs)")
    a = p.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: the attention kernels run on a single MI355X "
              "(multi-GPU sharding is a design note, not part of this build).", file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    if a.only is not None:
        run_only(a.only, a.steps, a.warmup)
        return
    flops, wall, ev, err, sdpa = bench_prefill(a.steps, a.warmup)
    achieved = flops / ev / 1e12
    c = PREFILL
    line = {
        "metric": "prefill TFLOP/s bf16 causal N=4096 D=128; split-K decode achieved HBM GB/s",
        "value": round(flops / wall / 1e12, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "warmup_min_s_per_workload": WARMUP_MIN_S,
        "warmup_min_s_first_workload": FIRST_WARMUP_MIN_S,
        "ms_per_step": round(wall * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": f"synthetic: q/k/v ~ N(0,1) from a seeded generator, cast to bf16, resident in HBM; the timed "
                f"calls rotate through {PREFILL_SETS} input sets",
        "max_abs_err": err,
        "config": {"workload": f"causal GQA prefill B={c['b']} Hq={c['hq']} Hkv={c['hkv']} N={c['n']} D={c['d']} "
                               "bf16 [B,H,N,D]", "batch": c["b"], "heads_q": c["hq"], "heads_kv": c["hkv"],
                   "seq_len": c["n"], "head_dim": c["d"], "causal": True, "parallelism": "single-gpu"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": MFMA_BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4),
                     "traffic": _traffic_bytes(), "kernel": "attn_fwd_kernel<128,BF16,8>",
                     "kernel_ms": round(ev * 1e3, 4)},
    }
    line["context"] = {"sdpa": sdpa}
    try:  # a measurement aid beside the headline: its absence must not cost the bench line
        line["mfma_ceiling"] = bench_mfma_ceiling(max(5, a.steps // 2), max(2, a.warmup), prefill_tflops=achieved)
    except (OSError, RuntimeError) as e:
        line["mfma_ceiling"] = {"error": str(e)}
    line["prefill_other"] = bench_prefill_extras(max(5, a.steps // 2), max(2, a.warmup))
    line["prefill_sweep"] = bench_prefill_sweep(max(5, a.steps // 2), max(2, a.warmup))
    if not a.no_decode:
        line["decode"] = bench_decode(max(5, a.steps), max(2, a.warmup))
        line["decode_sweep"] = bench_decode_sweep(max(5, a.steps), max(2, a.warmup))
        line["quantize"] = bench_quantize(max(5, a.steps), max(2, a.warmup))
    if not a.no_cpu:
        line["cpu_baseline"] = cpu_baseline()
        line["cpu_config0"] = cpu_config0()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
