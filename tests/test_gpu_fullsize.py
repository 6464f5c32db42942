"""Parity at the benchmark shapes (B=1, C=64).

* 256x256 fused recompute training, fp32 and bf16, against the float64 CPU
  oracle (forward and all gradients);
* 128x128 fused inference, fp32;
* K=5 128x128 bf16 inference on the fused and the materialized route (output
  also against the oracle run in bf16), fp32 fused inference, bf16 and fp32
  materialized training;
* size-independent adjoint identities of the fused operator at 256x256:
  the fused op is linear in x and affine in y, W and b, so
  <F(x + v) - F(x), g> = <v, dX(g)> and likewise for y, W and b; both sides
  come from the HIP kernels alone and are reduced in float64.
"""

import pytest
import torch

from dynamicconvolutionoperator_amd import ops
from tests.gpu_helpers import (DEV, DIL, assert_max_abs, default_generator_params, max_abs_bound,
                               randn, record_errors, say)
from tests.test_gpu_module import check_bf16_output, check_training, make_models

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_training_256_fused(dtype):
    say(f"full-size training 256x256 C=64 K=3 dtype={dtype}")
    check_training(64, 256, 256, 3, dtype, fused=True, n=1, seed=21)


def test_inference_128_fused_fp32():
    say("full-size fused inference 128x128 C=64 K=3 fp32")
    ref, cand = make_models(64, 3, torch.float32)
    ref.eval()
    cand.eval()
    torch.manual_seed(20)
    x = torch.randn(1, 64, 128, 128)
    y = torch.randn_like(x)
    with torch.inference_mode():
        expected = ref(x.double(), y.double())
        actual = cand(x.to(DEV), y.to(DEV))
    stats = assert_max_abs(actual, expected, max_abs_bound(torch.float32, 3), "out 128 fp32")
    record_errors("infer N=1 C=64 128x128 K=3 float32 fused", {"out": stats})


@pytest.mark.parametrize("route", ["fused", "materialized"])
def test_k5_128_bf16_inference(route):
    """K=5 128x128 bf16 inference on the fused forward (the module's default,
    as the reference's) and on the materialized route
    (fused_generator_inference=False)."""
    say(f"full-size K=5 128x128 bf16 inference, {route} route")
    ref, cand = make_models(64, 5, torch.bfloat16,
                            fused_generator_inference=route == "fused")
    ref.eval()
    cand.eval()
    torch.manual_seed(22)
    x = torch.randn(1, 64, 128, 128).to(torch.bfloat16)
    y = torch.randn_like(x)
    with torch.inference_mode():
        expected = ref(x.double(), y.double())
        actual = cand(x.to(DEV), y.to(DEV))
    errors = {"out": assert_max_abs(actual, expected, max_abs_bound(torch.bfloat16, 5),
                                    "out K5 bf16")}
    check_bf16_output(actual, x, y, 64, 5, errors)
    record_errors(f"infer N=1 C=64 128x128 K=5 bfloat16 {route}", errors)


def test_k5_128_fp32_inference_fused():
    """K=5 128x128 fp32 inference on the fused forward (pair-plane concat)."""
    say("full-size K=5 128x128 fp32 fused inference")
    ref, cand = make_models(64, 5, torch.float32)
    ref.eval()
    cand.eval()
    torch.manual_seed(25)
    x = torch.randn(1, 64, 128, 128)
    y = torch.randn_like(x)
    with torch.inference_mode():
        expected = ref(x.double(), y.double())
        actual = cand(x.to(DEV), y.to(DEV))
    stats = assert_max_abs(actual, expected, max_abs_bound(torch.float32, 5), "out K5 fp32")
    record_errors("infer N=1 C=64 128x128 K=5 float32 fused", {"out": stats})


def test_k5_128_bf16_materialized_training():
    say("full-size K=5 128x128 bf16 materialized training")
    check_training(64, 128, 128, 5, torch.bfloat16, fused=False, n=1, seed=23)


def test_k5_128_fp32_materialized_training():
    """The materialized route's fp32 backward: the generator convolution's
    weight / bias and input gradients run as split-bf16 MFMA kernels."""
    say("full-size K=5 128x128 fp32 materialized training")
    check_training(64, 128, 128, 5, torch.float32, fused=False, n=1, seed=24)


def _dot(a, b):
    return (a.double() * b.double()).sum().item()


def test_adjoint_identities_256_fp32():
    say("adjoint identities 256x256 C=64 K=3 fp32")
    shape = (1, 64, 256, 256)
    x = randn(shape, 70).to(DEV)
    y = randn(shape, 71).to(DEV)
    wt, b = default_generator_params(64, 3, 72, torch.float32)
    wt, b = wt.to(DEV), b.to(DEV)
    g = randn((1, 256, 256, 256), 73).to(DEV)
    vx, vy = randn(shape, 74).to(DEV), randn(shape, 75).to(DEV)
    vw = randn(tuple(wt.shape), 76, scale=0.1).to(DEV)
    vb = randn(tuple(b.shape), 77, scale=0.1).to(DEV)

    xs, ys, ws, bs = (t.clone().requires_grad_() for t in (x, y, wt, b))
    ops.fused_generator_dynamic_cat(xs, ys, ws, bs, 3, DIL).backward(g)
    with torch.no_grad():
        f0 = ops.fused_generator_dynamic_cat(x, y, wt, b, 3, DIL)
        checks = {
            "x": (ops.fused_generator_dynamic_cat(x + vx, y, wt, b, 3, DIL), vx, xs.grad),
            "y": (ops.fused_generator_dynamic_cat(x, y + vy, wt, b, 3, DIL), vy, ys.grad),
            "W": (ops.fused_generator_dynamic_cat(x, y, wt + vw, b, 3, DIL), vw, ws.grad),
            "b": (ops.fused_generator_dynamic_cat(x, y, wt, b + vb, 3, DIL), vb, bs.grad),
        }
    for name, (f1, v, grad) in checks.items():
        lhs = _dot(f1 - f0, g)
        rhs = _dot(v, grad)
        say(f"  adjoint {name}: lhs={lhs:.6e} rhs={rhs:.6e}")
        assert abs(lhs - rhs) <= 1e-4 * max(abs(lhs), abs(rhs)) + 1e-2, name


def test_filter_adjoint_and_linearity_256():
    say("materialized filter adjoint 256x256 C=64 K=3 fp32")
    shape = (1, 64, 256, 256)
    x = randn(shape, 80).to(DEV)
    k = randn((1, 3, 64, 9, 256, 256), 81).to(DEV)
    g = randn((1, 256, 256, 256), 82).to(DEV)
    v = randn(shape, 83).to(DEV)
    vk = randn(tuple(k.shape), 84).to(DEV)
    xs, ks = x.clone().requires_grad_(), k.clone().requires_grad_()
    ops.fused_dynamic_cat(xs, ks, 3, DIL).backward(g)
    with torch.no_grad():
        fx = ops.fused_dynamic_cat(v, k, 3, DIL)
        fk = ops.fused_dynamic_cat(x, vk, 3, DIL)
        lin = ops.fused_dynamic_cat(x + v, k, 3, DIL) - ops.fused_dynamic_cat(x, k, 3, DIL) - fx
    lhs, rhs = _dot(fx, g), _dot(v, xs.grad)
    assert abs(lhs - rhs) <= 1e-5 * abs(lhs) + 1e-2
    lhs, rhs = _dot(fk[:, 64:], g[:, 64:]), _dot(vk, ks.grad)
    assert abs(lhs - rhs) <= 1e-5 * abs(lhs) + 1e-2
    assert lin.abs().max().item() < 1e-4
