"""The matrix-core ceiling probe (csrc/fa_ceiling.hip, fused_attn/libfa_probe.so) that bench.py times
beside the prefill workload.  Its rate is only meaningful if every counted MFMA is executed: each lane's
four accumulators take the same product every round, so after n rounds they hold n times the first
round's values, and each workgroup's output is the sum of its lanes' accumulators (a permutation of
them across threads).  Checked for n = 1, 2 and 8 against n = 1, in fp32."""
import ctypes
import os

import pytest
import torch

from helpers import announce

pytestmark = pytest.mark.gpu

PROBE = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "cuda-attention-kernels_amd",
                     "fused_attn", "libfa_probe.so")


def _run(lib, data, grid, iters):
    out = torch.full((grid * 512,), float("nan"), dtype=torch.float32, device="cuda")
    rc = lib.fa_probe_mfma_ceiling(ctypes.c_void_p(data.data_ptr()), ctypes.c_void_p(out.data_ptr()), grid, iters,
                                   ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0
    torch.cuda.synchronize()
    return out


def test_probe_accumulates_every_round():
    announce("mfma ceiling probe linearity")
    lib = ctypes.CDLL(PROBE)
    lib.fa_probe_mfma_ceiling.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_void_p]
    lib.fa_probe_data_elems.restype = ctypes.c_int
    g = torch.Generator(device="cuda").manual_seed(5)
    # small integers: every product and partial sum is exact in fp32, so the comparison is exact
    data = torch.randint(-3, 4, (lib.fa_probe_data_elems(),), device="cuda", generator=g).bfloat16()
    grid = 4
    one = _run(lib, data, grid, 1)
    assert torch.isfinite(one).all() and one.abs().sum() > 0
    for n in (2, 8):
        assert torch.equal(_run(lib, data, grid, n), one * n), n
    # invalid requests are refused before a launch
    assert lib.fa_probe_mfma_ceiling(ctypes.c_void_p(data.data_ptr()), None, grid, 1, None) != 0
    assert lib.fa_probe_mfma_ceiling(ctypes.c_void_p(data.data_ptr()), ctypes.c_void_p(1), 0, 1, None) != 0
