"""Shared helpers for the GPU parity tests (HIP path vs the CPU fp64 oracle)."""

from __future__ import annotations

import json
import os
import sys

import torch

DIL = (1, 3, 5)
DEV = "cuda"

# Tolerances (stated once, used by every GPU parity test).
#   fp32 filter ops: exact fp32 FMAs vs fp64 -> tight
#   fp32 fused generator: 3 x bf16 products per fp32 product (~2^-16 rel.)
#   bf16/fp16: output rounding (2^-9 rel.) plus rounding of generated taps
TOL = {
    "filter": {torch.float32: (2e-5, 2e-5), torch.bfloat16: (2e-2, 1e-2), torch.float16: (4e-3, 2e-3)},
    "gen_fwd": {torch.float32: (2e-4, 1e-4), torch.bfloat16: (3e-2, 2e-2), torch.float16: (1e-2, 5e-3)},
    "gen_bwd": {torch.float32: (3e-3, 3e-3), torch.bfloat16: (1e-1, 5e-2), torch.float16: (3e-2, 2e-2)},
    # module level: the reference's bounds (fp32 fwd 2e-3, bwd 3e-3; bf16 fwd 3e-2)
    "module_fwd": {torch.float32: (2e-3, 2e-3), torch.bfloat16: (3e-2, 3e-2), torch.float16: (1e-2, 1e-2)},
    "module_bwd": {torch.float32: (3e-3, 3e-3), torch.bfloat16: (1e-1, 1e-1), torch.float16: (3e-2, 3e-2)},
}


# Bounds on the module output: maximum absolute error against the float64
# oracle, for every kernel size: fp32 2e-3 and bf16 3e-2 as stated for the
# target shapes, fp16 1e-2.  (The reference's own model tolerance is looser:
# gpu_bench.py:48-53, fp32 3e-3 at K >= 5, bf16 5e-2.)
MAX_ABS_OUT = {torch.float32: 2e-3, torch.bfloat16: 3e-2, torch.float16: 1e-2}


def max_abs_bound(dtype, kernel_size: int) -> float:
    return MAX_ABS_OUT[dtype]


def bf16_ulp(t: torch.Tensor) -> torch.Tensor:
    """One bf16 rounding step at |t| (8 significant bits): 2^(floor(log2|t|) - 7)."""
    e = torch.floor(torch.log2(t.abs().clamp_min(2.0**-126)))
    return torch.exp2(e - 7)


def assert_bf16_oracle(actual: torch.Tensor, expected_bf16: torch.Tensor, bound: float,
                       what: str) -> dict:
    """The bf16 bound against the oracle run in bf16 (gpu_validate.py:29):
    every element within `bound`, or within one bf16 rounding step of the
    oracle's value -- two results rounded to bf16 independently land one
    step apart wherever the exact value lies between them (0.03125 for
    outputs in [4, 8)).  Returns the max abs difference and how many
    elements needed the one-step allowance."""
    a = actual.detach().double().cpu()
    e = expected_bf16.detach().double().cpu()
    assert a.shape == e.shape, f"{what}: shape {tuple(a.shape)} != {tuple(e.shape)}"
    d = (a - e).abs()
    allowed = torch.clamp(bf16_ulp(e), min=bound)
    bad = d > allowed
    if bool(bad.any()):
        idx = int(torch.argmax((d - allowed).flatten()))
        raise AssertionError(
            f"{what}: {int(bad.sum())} elements beyond max({bound}, one bf16 step) of the bf16 "
            f"oracle; worst: actual={a.flatten()[idx].item():.6g} "
            f"oracle_bf16={e.flatten()[idx].item():.6g}")
    return {"max_abs": d.max().item(), "one_step_elements": int((d > bound).sum()),
            "ref_max_abs": e.abs().max().item()}


def error_stats(actual: torch.Tensor, expected: torch.Tensor) -> dict:
    """Max abs error, RMSE and the expected tensor's max magnitude, in float64."""
    a = actual.detach().double().cpu()
    e = expected.detach().double().cpu()
    d = a - e
    return {
        "max_abs": d.abs().max().item(),
        "rmse": d.square().mean().sqrt().item(),
        "ref_max_abs": e.abs().max().item(),
    }


def record_errors(case: str, errors: dict) -> None:
    """Appends one JSON line {case, errors} to $DDPM_ERROR_LOG when it is set
    (the measured error table of the parity tests)."""
    path = os.environ.get("DDPM_ERROR_LOG")
    if not path:
        return
    with open(path, "a") as f:
        f.write(json.dumps({"case": case, "errors": errors}) + "\n")


def assert_max_abs(actual: torch.Tensor, expected: torch.Tensor, bound: float, what: str) -> dict:
    stats = error_stats(actual, expected)
    assert actual.shape == expected.shape, f"{what}: shape {tuple(actual.shape)} != {tuple(expected.shape)}"
    assert stats["max_abs"] <= bound, f"{what}: max abs error {stats['max_abs']:.3e} > {bound:.1e}"
    return stats


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def assert_close(actual: torch.Tensor, expected: torch.Tensor, atol: float, rtol: float, what: str):
    a = actual.detach().double().cpu()
    e = expected.detach().double().cpu()
    assert a.shape == e.shape, f"{what}: shape {tuple(a.shape)} != {tuple(e.shape)}"
    diff = (a - e).abs()
    bound = atol + rtol * e.abs()
    bad = diff > bound
    if bool(bad.any()):
        idx = int(torch.argmax((diff - bound).flatten()))
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{a.numel()} elements out of tolerance "
            f"(atol={atol}, rtol={rtol}); max|diff|={diff.max().item():.3e}; "
            f"worst flat index {idx}: actual={a.flatten()[idx].item():.6g} "
            f"expected={e.flatten()[idx].item():.6g}"
        )
    return diff.max().item()


def randn(shape, seed, dtype=torch.float32, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g, dtype=torch.float64) * scale).to(dtype)


def default_generator_params(c: int, k: int, seed: int, dtype):
    """Default-initialised 1x1 generator conv parameters (seeded), on the CPU."""
    torch.manual_seed(seed)
    conv = torch.nn.Conv2d(c, 3 * c * k * k, 1)
    return conv.weight.detach().to(dtype), conv.bias.detach().to(dtype)
