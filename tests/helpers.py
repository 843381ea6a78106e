"""Shared helpers for the parity tests."""
import sys

import torch

# max-abs error bars against the fp32 oracle
TOL = {torch.bfloat16: 2e-2, torch.float16: 5e-3}
FP8_TOL = 5e-2


def max_err(out: torch.Tensor, ref: torch.Tensor) -> float:
    return (out.float() - ref.float().to(out.device)).abs().max().item() if out.numel() else 0.0


def announce(msg: str) -> None:
    """Name the case before GPU work starts, flushed, so a crash still identifies it."""
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def randn(*shape, dtype=torch.float32, device="cuda", gen=None):
    return torch.randn(*shape, dtype=torch.float32, device=device, generator=gen).to(dtype)
