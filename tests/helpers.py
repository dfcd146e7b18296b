"""Shared helpers for the parity tests: seeded CPU inputs, tolerances, error stats."""

from __future__ import annotations

import sys

import torch

# bf16 gate from the attention path's contract: against the reference math run
# in fp32 on the same (bf16-valued) inputs, max-abs <= 2e-2, mean-abs <= 2e-3.
BF16_MAX_ABS = 2e-2
BF16_MEAN_ABS = 2e-3
# fp32 gate: fp32 inputs keep fp32 arithmetic (the reference's SDPA runs in the
# input dtype), so only summation order and the exp2 / rsqrt instructions'
# last-bit rounding separate the kernels from the fp32 oracle.
FP32_MAX_ABS = 1e-5
FP32_MEAN_ABS = 1e-6


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


def assert_fp32_close(got, ref, what: str = "", max_abs: float = FP32_MAX_ABS,
                      mean_abs: float = FP32_MEAN_ABS) -> None:
    assert got.dtype == torch.float32, f"{what}: expected an fp32 result, got {got.dtype}"
    mx, mean = err_stats(got, ref)
    assert mx <= max_abs and mean <= mean_abs, f"{what}: max-abs {mx:.3e} mean-abs {mean:.3e} (fp32 gate)"


def assert_close_for(dtype, got, ref, what: str = "") -> None:
    """The gate of the input dtype: fp32 inputs at the fp32 gate, bf16 at the bf16 one."""
    if dtype == torch.float32:
        assert_fp32_close(got, ref, what)
    else:
        assert_bf16_close(got, ref, what)
