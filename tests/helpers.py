"""Shared helpers for the parity tests."""
import sys

import torch

# max-abs error bars against the fp32 oracle
TOL = {torch.bfloat16: 2e-2, torch.float16: 5e-3}
FP8_TOL = 5e-2


def max_err(out: torch.Tensor, ref: torch.Tensor) -> float:
    return (out.float() - ref.float().to(out.device)).abs().max().item() if out.numel() else 0.0


def close(out: torch.Tensor, ref: torch.Tensor, tol: float) -> bool:
    """The reference's bar, torch.testing.assert_close(atol=tol, rtol=tol) (tests/test_correctness.py:84-85,
    tests/test_splitk_fp8.py:29): |out - ref| <= tol + tol * |ref| everywhere.  max_err <= tol (used by
    the fixed-case tests) is stricter; with large softmax scales the output follows single V rows of
    magnitude ~4, where one bf16 ulp (0.031) already exceeds an absolute 2e-2."""
    if not out.numel():
        return True
    r = ref.float().to(out.device)
    return bool(((out.float() - r).abs() <= tol + tol * r.abs()).all().item())


def check_bars(out: torch.Tensor, ref: torch.Tensor, tol: float) -> float:
    """Assert both bars, the reference's (close) and the plain max-abs one (max_err <= tol), and print the
    max-abs error beside the output's magnitude.  Returns the max-abs error."""
    err = max_err(out, ref)
    mag = ref.float().abs().max().item() if ref.numel() else 0.0
    print(f"max_abs_err={err:.3e} |ref|max={mag:.3e} bar={tol:g}", flush=True)
    assert close(out, ref, tol), err
    assert err <= tol, (err, mag)
    return err


def announce(msg: str) -> None:
    """Name the case before GPU work starts, flushed, so a crash still identifies it."""
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def randn(*shape, dtype=torch.float32, device="cuda", gen=None):
    return torch.randn(*shape, dtype=torch.float32, device=device, generator=gen).to(dtype)
