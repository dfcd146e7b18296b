"""Shared helpers for the parity tests: seeded CPU inputs, tolerances, error stats."""

from __future__ import annotations

import sys

import torch

# bf16 gate from the attention path's contract: against the reference math run
# in fp32 on the same (bf16-valued) inputs, max-abs <= 2e-2, mean-abs <= 2e-3.
BF16_MAX_ABS = 2e-2
BF16_MEAN_ABS = 2e-3


def say(msg: str) -> None:
    """Name the GPU case about to run (flushed, so a crash still shows it)."""
    print(f"[case] {msg}", file=sys.stderr, flush=True)


def randn(*shape, seed: int, dtype=torch.float32, scale: float = 1.0) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def err_stats(got: torch.Tensor, ref: torch.Tensor):
    d = (got.detach().float().cpu() - ref.detach().float().cpu()).abs()
    return float(d.max()), float(d.mean())


def assert_bf16_close(got, ref, what: str = "", max_abs: float = BF16_MAX_ABS,
                      mean_abs: float = BF16_MEAN_ABS) -> None:
    mx, mean = err_stats(got, ref)
    assert mx <= max_abs and mean <= mean_abs, f"{what}: max-abs {mx:.3e} mean-abs {mean:.3e}"
