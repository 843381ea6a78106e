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
  whole prefill workload one (batch, kv-head group) slice at a time.
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


def _time_calls(fn, steps, warmup):
    """Wall time per call (synchronised both sides) and mean per-launch duration from HIP events.

    Before the timed region the workload runs untimed for ``warmup`` calls and at least
    WARMUP_MIN_S seconds (the reference's benchmark warms up by time too: triton's do_bench,
    benchmarks/bench.py:49-53).  MI355X clocks take some tens of milliseconds of load to
    settle; a cold first workload measured ~15% slow after 5 calls."""
    import torch

    t_end = time.perf_counter() + WARMUP_MIN_S
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


def _traffic_bytes():
    try:
        text = open(TRAFFIC_FILE).read()
    except OSError:
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", text)
    return float(m.group(1)) if m else None


def bench_prefill(steps, warmup):
    import torch

    import fused_attn

    c = PREFILL
    g = torch.Generator(device="cuda").manual_seed(0)
    q = torch.randn(c["b"], c["hq"], c["n"], c["d"], device="cuda", generator=g).bfloat16()
    k = torch.randn(c["b"], c["hkv"], c["n"], c["d"], device="cuda", generator=g).bfloat16()
    v = torch.randn(c["b"], c["hkv"], c["n"], c["d"], device="cuda", generator=g).bfloat16()
    out = fused_attn.attention(q, k, v, causal=True)
    assert not torch.isnan(out).any()
    wall, ev = _time_calls(lambda: fused_attn.attention(q, k, v, causal=True), steps, warmup)
    flops = attn_flops(c["b"], c["hq"], c["n"], c["d"], True)
    return flops, wall, ev


def bench_prefill_extras(steps, warmup):
    """The other prefill configurations (D=64 MHA, the [B,N,H,D] view, the 16-sequence varlen batch), and D=16, 32 and 256."""
    import torch

    import fused_attn

    res = {}
    g = torch.Generator(device="cuda").manual_seed(0)

    def entry(name, workload, fn, flops):
        out = fn()
        assert not torch.isnan(out).any()
        wall, ev = _time_calls(fn, steps, warmup)
        res[name] = {"workload": workload, "ms": round(wall * 1e3, 4), "ms_events": round(ev * 1e3, 4),
                     "TFLOP_s": round(flops / wall / 1e12, 1),
                     "TFLOP_s_events": round(flops / ev / 1e12, 1),
                     "mfma_frac": round(flops / ev / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4)}

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
    entry("varlen_prefill", f"varlen causal prefill, 16 sequences (lengths U[0,4096] by seed 0, one 0, one 1; "
          f"{total} tokens) Hq=32 Hkv=8 D=128 bf16",
          lambda: fused_attn.attention_varlen(q, k, v, cu, cu, mx, mx, causal=True),
          sum(attn_flops(1, 32, n, 128, True) for n in lens))
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
            "hbm_frac": round(nbytes / ev / 1e9 / HBM_PEAK_GBS, 4),
        }
    if only_128:
        return res
    res.update(bench_paged(k, v, steps, warmup, g))
    del k, v
    torch.cuda.empty_cache()
    c = FP8_DECODE
    q = torch.randn(c["b"], c["hq"], 1, c["d"], device="cuda", generator=g).bfloat16()
    k8, ks = fused_attn.quantize_kv_fp8(torch.randn(c["b"], c["hkv"], c["nk"], c["d"], device="cuda", generator=g))
    v8, vs = fused_attn.quantize_kv_fp8(torch.randn(c["b"], c["hkv"], c["nk"], c["d"], device="cuda", generator=g))
    torch.cuda.empty_cache()
    for split in (128, None):
        fn = lambda: fused_attn.attention_fp8(q, k8, ks, v8, vs, split_len=split)  # noqa: E731
        wall, ev = _time_calls(fn, steps, warmup)
        nbytes = 2 * k8.numel() + 2 * ks.numel() * 4 + 2 * q.numel() * 2
        keys = split or fused_attn.ops.default_split_len(1, c["nk"], c["b"], c["hkv"], c["hq"] // c["hkv"])
        res["fp8_decode" + ("" if split else "_default_split")] = {
            "workload": f"FP8-KV split-K B={c['b']} Hq={c['hq']} Hkv={c['hkv']} n_q=1 n_k={c['nk']} D={c['d']}, "
                        f"e4m3fn + fp32 per-64-key scales, {keys}-key partitions"
                        f"{'' if split else ' (default partition policy)'}",
            "ms": round(wall * 1e3, 4), "GB_s": round(nbytes / wall / 1e9, 1),
            "GB_s_events": round(nbytes / ev / 1e9, 1), "bytes": nbytes,
            "hbm_frac": round(nbytes / ev / 1e9 / HBM_PEAK_GBS, 4),
        }
    del q, k8, ks, v8, vs
    torch.cuda.empty_cache()
    res.update(bench_decode_d256(steps, warmup, g))
    return res


def bench_decode_d256(steps, warmup, g):
    """Split-K decode at head dim 256: B=8 Hq=32 Hkv=8 n_k=32768 bf16 (2.147 GB of K+V), 128-key partitions."""
    import torch

    import fused_attn

    b, hq, hkv, nk, d = 8, 32, 8, 32768, 256
    k = torch.randn(b, hkv, nk, d, device="cuda", generator=g).bfloat16()
    v = torch.randn(b, hkv, nk, d, device="cuda", generator=g).bfloat16()
    q = torch.randn(b, hq, 1, d, device="cuda", generator=g).bfloat16()
    fn = lambda: fused_attn.attention_splitk(q, k, v, split_len=128)  # noqa: E731
    wall, ev = _time_calls(fn, steps, warmup)
    nbytes = 2 * k.numel() * 2 + 2 * q.numel() * 2
    res = {"decode_d256": {
        "workload": f"split-K B={b} Hq={hq} Hkv={hkv} n_q=1 n_k={nk} D={d} bf16, 128-key partitions + LSE combine",
        "ms": round(wall * 1e3, 4), "GB_s": round(nbytes / wall / 1e9, 1),
        "GB_s_events": round(nbytes / ev / 1e9, 1), "bytes": nbytes,
        "hbm_frac": round(nbytes / ev / 1e9 / HBM_PEAK_GBS, 4),
    }}
    del q, k, v
    torch.cuda.empty_cache()
    return res


def bench_paged(k, v, steps, warmup, g, page_size=64):
    """Split-K decode over the same K/V scattered into a shuffled pool of 64-key pages."""
    import torch

    import fused_attn

    c = DECODE
    kc, vc, bt, sl = fused_attn.paged_from_dense(k, v, page_size, generator=torch.Generator().manual_seed(0))
    q = torch.randn(c["b"], c["hq"], 1, c["d"], device="cuda", generator=g).bfloat16()
    res = {}
    for split in (128, None):
        keys = split or fused_attn.ops.default_split_len(1, c["nk"], c["b"], c["hkv"], c["hq"] // c["hkv"])
        fn = lambda: fused_attn.attention_paged(q, kc, vc, bt, sl, max_seqlen_k=c["nk"], split_len=keys)  # noqa: E731
        wall, ev = _time_calls(fn, steps, warmup)
        nbytes = 2 * kc.numel() * 2 + 2 * q.numel() * 2 + bt.numel() * 4
        res["paged_decode" + ("" if split else "_default_split")] = {
            "workload": f"paged split-K B={c['b']} Hq={c['hq']} Hkv={c['hkv']} n_q=1 n_k={c['nk']} D={c['d']} bf16, "
                        f"{page_size}-key pages in shuffled order, {keys}-key partitions + LSE combine"
                        f"{'' if split else ' (default partition policy)'}",
            "ms": round(wall * 1e3, 4), "GB_s": round(nbytes / wall / 1e9, 1),
            "GB_s_events": round(nbytes / ev / 1e9, 1), "bytes": nbytes,
            "hbm_frac": round(nbytes / ev / 1e9 / HBM_PEAK_GBS, 4),
        }
    return res


def bench_quantize(steps, warmup):
    """The fused FP8 KV quantiser over one K cache of the FP8 decode workload (bf16 in, e4m3fn + scales out)."""
    import torch

    import fused_attn

    c = FP8_DECODE
    g = torch.Generator(device="cuda").manual_seed(0)
    x = torch.randn(c["b"], c["hkv"], c["nk"], c["d"], device="cuda", generator=g).bfloat16()
    wall, ev = _time_calls(lambda: fused_attn.quantize_kv_fp8(x), steps, warmup)
    nblk = -(-c["nk"] // 64)
    nbytes = x.numel() * 2 + x.numel() + c["b"] * c["hkv"] * nblk * 4
    return {
        "workload": f"FP8 KV quantiser B={c['b']} Hkv={c['hkv']} N={c['nk']} D={c['d']}: bf16 -> e4m3fn + fp32 "
                    "per-64-key scales",
        "kernel": "quantize_kv_fp8_kernel<bf16,128>",
        "ms": round(wall * 1e3, 4), "GB_s": round(nbytes / wall / 1e9, 1),
        "GB_s_events": round(nbytes / ev / 1e9, 1), "bytes": nbytes,
        "hbm_frac": round(nbytes / ev / 1e9 / HBM_PEAK_GBS, 4),
    }


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
        flops, wall, ev = bench_prefill(steps, warmup)
        print(f"prefill: {flops / ev / 1e12:.1f} TFLOP/s kernel, {ev * 1e3:.4f} ms", flush=True)
    elif which == "quantize":
        print(json.dumps(bench_quantize(steps, warmup)), flush=True)
    elif which in ("decode", "decode128"):
        print(json.dumps(bench_decode(steps, warmup, only_128=which == "decode128")), flush=True)
    else:
        wall, ev, nbytes = copy_calibration(steps, warmup)
        print(f"copy {nbytes} B: {ev * 1e3:.4f} ms, {2 * nbytes / ev / 1e9:.1f} GB/s read+write", flush=True)


def main():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--no-decode", action="store_true")
    p.add_argument("--only", choices=["prefill", "decode", "decode128", "quantize", "copy"], default=None,
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
    flops, wall, ev = bench_prefill(a.steps, a.warmup)
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
        "ms_per_step": round(wall * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: q/k/v ~ N(0,1) from a seeded generator, cast to bf16, resident in HBM",
        "config": {"workload": f"causal GQA prefill B={c['b']} Hq={c['hq']} Hkv={c['hkv']} N={c['n']} D={c['d']} "
                               "bf16 [B,H,N,D]", "batch": c["b"], "heads_q": c["hq"], "heads_kv": c["hkv"],
                   "seq_len": c["n"], "head_dim": c["d"], "causal": True, "parallelism": "single-gpu"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": MFMA_BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4),
                     "traffic": _traffic_bytes(), "kernel": "attn_fwd_kernel<128,BF16,8>",
                     "kernel_ms": round(ev * 1e3, 4)},
    }
    line["prefill_other"] = bench_prefill_extras(max(5, a.steps // 2), max(2, a.warmup))
    if not a.no_decode:
        line["decode"] = bench_decode(max(5, a.steps), max(2, a.warmup))
        line["quantize"] = bench_quantize(max(5, a.steps), max(2, a.warmup))
    if not a.no_cpu:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
