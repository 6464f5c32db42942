"""Module-level GPU parity: the drop-in DDPM on the MI355X vs the oracle
(UnfoldDDPM, float64 on the CPU) with identical weights and inputs.

Mirrors the reference's GPU validation (gpu_validate.py:39-103): B=2, C=24,
H=15, W=17 (non-power-of-two channels, non-square map), K in {1,3,5},
fp32 and bf16, forced fused and forced materialized training; output, dx, dy
and every generator/fuse parameter gradient.  Tolerances: output maximum
absolute error against the float64 oracle fp32 2e-3, bf16 3e-2, fp16 1e-2
(every K); bf16 outputs also against the oracle run in bf16, as the
reference validates (gpu_validate.py:29): within 3e-2 or one bf16 rounding
step of it; fp32 gradients 3e-3 (relative to each gradient's max), bf16
gradients 1e-1.
"""

import pytest
import torch

from dynamicconvolutionoperator_amd import DDPM
from oracle.unfold_ref import UnfoldDDPM
from tests.gpu_helpers import (DEV, TOL, assert_bf16_oracle, assert_close, assert_max_abs,
                               error_stats, max_abs_bound, record_errors, say)

pytestmark = pytest.mark.gpu


def make_models(channels, kernel_size, dtype, **kwargs):
    torch.manual_seed(123)
    reference = UnfoldDDPM(channels, kernel_size)
    candidate = DDPM(channels, kernel_size, **kwargs)
    candidate.load_state_dict(reference.state_dict())
    # oracle in float64 on the CPU from the dtype-rounded parameters
    reference = reference.to(dtype).double()
    return reference, candidate.to(DEV).to(dtype)


def bf16_oracle(channels, kernel_size):
    """The oracle with make_models' weights, run in bf16 on the CPU (the
    reference's validation runs its Unfold model in the tested dtype,
    gpu_validate.py:29)."""
    torch.manual_seed(123)
    return UnfoldDDPM(channels, kernel_size).to(torch.bfloat16)


def check_bf16_output(actual, x, y, channels, kernel_size, errors):
    """Asserts a bf16 module output against the bf16-run oracle and records
    the difference beside the float64 figure."""
    with torch.no_grad():
        expected = bf16_oracle(channels, kernel_size)(x.cpu(), y.cpu())
    errors["out_vs_bf16_oracle"] = assert_bf16_oracle(actual, expected,
                                                      max_abs_bound(torch.bfloat16, kernel_size),
                                                      "out vs bf16 oracle")


def check_training(channels, h, w, kernel_size, dtype, fused, n=2, seed=456):
    ref, cand = make_models(channels, kernel_size, dtype, fused_generator_training=fused)
    ref.train()
    cand.train()
    torch.manual_seed(seed)
    x = torch.randn(n, channels, h, w).to(dtype)
    y = torch.randn_like(x)
    x_ref = x.double().requires_grad_()
    y_ref = y.double().requires_grad_()
    x_new = x.to(DEV).requires_grad_()
    y_new = y.to(DEV).requires_grad_()
    expected = ref(x_ref, y_ref)
    actual = cand(x_new, y_new)
    e_grads = torch.autograd.grad(expected.square().mean(), (x_ref, y_ref, *ref.parameters()))
    a_grads = torch.autograd.grad(actual.float().square().mean(), (x_new, y_new, *cand.parameters()))
    out_stats = assert_max_abs(actual, expected, max_abs_bound(dtype, kernel_size), "out")
    errors = {"out": out_stats}
    if dtype == torch.bfloat16:
        check_bf16_output(actual, x, y, channels, kernel_size, errors)
    atol, rtol = TOL["module_bwd"][dtype]
    names = ["dx", "dy", "d generator.weight", "d generator.bias", "d fuse.weight", "d fuse.bias"]
    for name, a, e in zip(names, a_grads, e_grads):
        scale = e.abs().max().item()
        errors[name] = error_stats(a, e)
        assert_close(a, e, atol * scale, rtol, name)
    record_errors(f"train N={n} C={channels} {h}x{w} K={kernel_size} {str(dtype)[6:]} "
                  f"{'fused' if fused else 'materialized'}", errors)
    return out_stats["max_abs"]


@pytest.mark.parametrize("kernel_size", [1, 3, 5])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("fused", [True, False])
def test_training_matches_oracle_nonaligned(kernel_size, dtype, fused):
    say(f"module training K={kernel_size} dtype={dtype} fused={fused}")
    check_training(24, 15, 17, kernel_size, dtype, fused)


@pytest.mark.parametrize("kernel_size", [1, 3, 5])
def test_fused_inference_matches_oracle(kernel_size):
    say(f"module fused inference K={kernel_size}")
    ref, cand = make_models(16, kernel_size, torch.float32)
    ref.eval()
    cand.eval()
    torch.manual_seed(789)
    x = torch.randn(2, 16, 15, 17)
    y = torch.randn_like(x)
    with torch.inference_mode():
        expected = ref(x.double(), y.double())
        actual = cand(x.to(DEV), y.to(DEV))
    stats = assert_max_abs(actual, expected, max_abs_bound(torch.float32, kernel_size),
                           "fused inference out")
    record_errors(f"infer N=2 C=16 15x17 K={kernel_size} float32", {"out": stats})


def test_c32_48x48_inference_on_gpu():
    """The CPU plumbing configuration (C=32, K=3, 48x48, fp32 inference) on the
    HIP path: fused generator route against the float64 oracle."""
    say("module inference C=32 48x48 K=3 fp32 (HIP path)")
    ref, cand = make_models(32, 3, torch.float32)
    ref.eval()
    cand.eval()
    torch.manual_seed(456)
    x = torch.randn(1, 32, 48, 48)
    y = torch.randn_like(x)
    with torch.inference_mode():
        expected = ref(x.double(), y.double())
        actual = cand(x.to(DEV), y.to(DEV))
    stats = assert_max_abs(actual, expected, max_abs_bound(torch.float32, 3), "C32 48x48 out")
    record_errors("infer N=1 C=32 48x48 K=3 float32", {"out": stats})


@pytest.mark.parametrize("channels", [96, 128])
@pytest.mark.parametrize("fused", [True, False])
def test_training_wide_channels(channels, fused):
    """More than 64 channels, on both routing requests (fp32, small map)."""
    say(f"module training C={channels} fused={fused}")
    check_training(channels, 12, 20, 3, torch.float32, fused, n=1, seed=457)


def test_autocast_bf16_uses_materialized_route():
    ref, cand = make_models(8, 3, torch.float32)
    torch.manual_seed(7)
    x = torch.randn(1, 8, 12, 16)
    y = torch.randn_like(x)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        out = cand(x.to(DEV), y.to(DEV))
    assert out.dtype == torch.bfloat16
    with torch.no_grad():
        expected = ref(x.double(), y.double())
    assert_close(out, expected, 5e-2, 5e-2, "autocast out")


def test_autocast_fp16_uses_materialized_route():
    """fp16 autocast: the generator conv runs in fp16, the HIP filter takes fp32 x
    with fp16 kernels and returns fp16, as the reference's mixed path does."""
    ref, cand = make_models(8, 3, torch.float32)
    torch.manual_seed(8)
    x = torch.randn(1, 8, 12, 16)
    y = torch.randn_like(x)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.float16):
        out = cand(x.to(DEV), y.to(DEV))
    assert out.dtype == torch.float16
    with torch.no_grad():
        expected = ref(x.double(), y.double())
    assert_close(out, expected, 1e-2, 1e-2, "autocast fp16 out")


def test_module_runs_native_library():
    """The module's GPU route goes through libddpm_hip.so (no torch fallback)."""
    import dynamicconvolutionoperator_amd._lib as lib
    import dynamicconvolutionoperator_amd.ops as ops

    calls = []
    real = ops._launch_generator_dynamic_cat

    def spy(*a, **k):
        calls.append(1)
        return real(*a, **k)

    ops._launch_generator_dynamic_cat = spy
    try:
        _, cand = make_models(8, 3, torch.float32)
        with torch.no_grad():
            cand(torch.randn(1, 8, 9, 9, device=DEV), torch.randn(1, 8, 9, 9, device=DEV))
    finally:
        ops._launch_generator_dynamic_cat = real
    assert calls and lib.available()
