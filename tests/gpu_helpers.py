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
# oracle.  K <= 3: fp32 2e-3 and bf16 3e-2 as stated for the target shapes;
# K >= 5: the reference's own model tolerance (gpu_bench.py:48-53: fp32 3e-3,
# bf16 5e-2); fp16 1e-2.
MAX_ABS_OUT = {torch.float32: 2e-3, torch.bfloat16: 3e-2, torch.float16: 1e-2}
MAX_ABS_OUT_K5 = {torch.float32: 3e-3, torch.bfloat16: 5e-2, torch.float16: 1e-2}


def max_abs_bound(dtype, kernel_size: int) -> float:
    return (MAX_ABS_OUT_K5 if kernel_size >= 5 else MAX_ABS_OUT)[dtype]


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
