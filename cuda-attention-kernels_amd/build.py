"""Build ``fused_attn/libfused_attn_hip.so`` (and the measurement probe ``fused_attn/libfa_probe.so``)
for gfx950 with hipcc.

    python cuda-attention-kernels_amd/build.py          # or __graft_entry__.build()

Each source compiles to an object under ``_build/`` at the repository root, in
parallel, then one shared library is linked next to ``fused_attn/_hip.py`` (the
ctypes loader looks there).  hipcc cross-compiles for gfx950 without a GPU.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD_DIR = os.path.join(ROOT, "_build")
LIB_OUT = os.path.join(HERE, "fused_attn", "libfused_attn_hip.so")
SOURCES = ["fa_prefill.hip", "fa_prefill_f32.hip", "fa_splitk.hip", "fa_generic.hip", "fa_quant.hip", "fa_abi.cpp"]
# the matrix-core ceiling probe bench.py times beside the prefill workload: a library of its own
PROBE_SOURCES = ["fa_ceiling.hip"]
PROBE_OUT = os.path.join(HERE, "fused_attn", "libfa_probe.so")
ARCH = os.environ.get("FUSED_ATTN_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    # no packed-fp32 VALU instructions anywhere in the device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in (r.stdout + r.stderr).splitlines() if noise not in line)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    cmds = []

    def objects(sources):
        objs = []
        for src in sources:
            obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
            cmds.append([HIPCC, *COMMON, "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj])
            objs.append(obj)
        return objs

    libs = [(LIB_OUT, objects(SOURCES)), (PROBE_OUT, objects(PROBE_SOURCES))]
    with ThreadPoolExecutor(max_workers=len(cmds)) as ex:
        list(ex.map(_run, cmds))
    for out, objs in libs:
        tmp = out + ".tmp"
        _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp])
        os.replace(tmp, out)
        if verbose:
            print(f"built {out}")
    return LIB_OUT


if __name__ == "__main__":
    build(verbose=True)
