"""Shared helpers for the attention tests."""

import sys

import torch

from oracle.eager_attention import max_abs


def announce(msg: str) -> None:
    """Print and flush the case about to run on the GPU, so a crash names it."""
    print(f"[case] {msg}", file=sys.stderr, flush=True)


def assert_close_abs(name: str, got: torch.Tensor, want: torch.Tensor, tol: float, ctx: str = ""):
    err = max_abs(got, want)
    assert err <= tol, f"{name}: max|err| = {err:.3e} > {tol:.1e} {ctx}"
    return err
