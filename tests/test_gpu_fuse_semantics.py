"""The module's ``self.fuse`` / ``self.generator`` semantics on the GPU route,
and the fused training step's peak temporary memory.

The reference ends every forward with ``self.fuse(cat)`` (triton_impl.py:392)
and the materialized route calls ``self.generator(y)`` (:340-347), so hooks,
weight reparametrisations and convolution attributes of those submodules take
effect.  The HIP kernels stand in for them only while they are the
constructor's plain convolutions; these tests change the submodules the ways
users do and compare against the float64 oracle changed the same way:

* a forward pre-hook that negates the concat, and a forward hook, on ``fuse``;
* ``torch.nn.utils.weight_norm`` (a forward pre-hook) on ``fuse``: the g / v
  gradients match the oracle's;
* ``torch.nn.utils.parametrizations.weight_norm`` on ``fuse`` (no hook: the
  HIP kernels read the parametrised weight, autograd reaches g / v);
* ``fuse`` replaced by a reflect-padded convolution;
* a forward hook on ``generator`` on the materialized route.
"""

import warnings

import pytest
import torch
from torch import nn

from dynamicconvolutionoperator_amd import DDPM
from oracle.unfold_ref import UnfoldDDPM
from tests.gpu_helpers import DEV, TOL, assert_close, assert_max_abs, max_abs_bound, say

pytestmark = pytest.mark.gpu


def _pair(channels, kernel_size, dtype, edit, **kwargs):
    """Oracle (float64, CPU) and module (GPU, dtype) with the same weights,
    both changed by `edit(module)`; the oracle's parameters are the
    dtype-rounded ones."""
    torch.manual_seed(123)
    ref = UnfoldDDPM(channels, kernel_size)
    cand = DDPM(channels, kernel_size, **kwargs)
    cand.load_state_dict(ref.state_dict())
    ref = ref.to(dtype).double()
    cand = cand.to(DEV).to(dtype)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore", FutureWarning)
        edit(ref)
        edit(cand)
    return ref, cand


def _compare(ref, cand, dtype, kernel_size, shape, seed=5):
    """Output and every named parameter's gradient (plus dx, dy) of a
    training step against the oracle."""
    torch.manual_seed(seed)
    x = torch.randn(*shape).to(dtype)
    y = torch.randn_like(x)
    xr, yr = x.double().requires_grad_(), y.double().requires_grad_()
    xg, yg = x.to(DEV).requires_grad_(), y.to(DEV).requires_grad_()
    expected = ref(xr, yr)
    actual = cand(xg, yg)
    assert_max_abs(actual, expected, max_abs_bound(dtype, kernel_size), "out")
    rnames = [n for n, _ in ref.named_parameters()]
    cnames = [n for n, _ in cand.named_parameters()]
    assert rnames == cnames
    e = torch.autograd.grad(expected.square().mean(), (xr, yr, *ref.parameters()))
    a = torch.autograd.grad(actual.float().square().mean(), (xg, yg, *cand.parameters()))
    atol, rtol = TOL["module_bwd"][dtype]
    for name, ga, ge in zip(["dx", "dy", *cnames], a, e):
        assert_close(ga, ge, atol * ge.abs().max().item(), rtol, f"d {name}")
    return actual


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_fuse_forward_hooks_fire(dtype):
    """A pre-hook that negates the concat (exact in every dtype) and a
    forward hook that counts calls: the GPU route runs both, as calling
    self.fuse does."""
    say(f"fuse hooks dtype={dtype}")
    calls = []

    def edit(m):
        m.fuse.register_forward_pre_hook(lambda mod, args: (-args[0],))
        m.fuse.register_forward_hook(lambda mod, args, out: calls.append(out.shape))

    ref, cand = _pair(16, 3, dtype, edit, fused_generator_training=True)
    _compare(ref, cand, dtype, 3, (2, 16, 15, 17))
    assert len(calls) == 2  # one oracle forward, one module forward
    assert not cand._hip_fuse()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_fuse_weight_norm_hook(dtype):
    """torch.nn.utils.weight_norm recomputes fuse.weight from g and v in a
    forward pre-hook: training reaches g and v as on the oracle."""
    say(f"fuse weight_norm (hook) dtype={dtype}")

    def edit(m):
        torch.nn.utils.weight_norm(m.fuse)

    ref, cand = _pair(16, 3, dtype, edit, fused_generator_training=True)
    assert not cand._hip_fuse()
    _compare(ref, cand, dtype, 3, (2, 16, 15, 17))


def test_fuse_weight_norm_parametrization_runs_hip():
    """parametrizations.weight_norm: no hook, so the HIP fuse convolution runs
    on the parametrised weight and autograd carries its gradient to
    original0 / original1 (fp32: the pair-plane route)."""
    say("fuse parametrizations.weight_norm fp32")

    def edit(m):
        torch.nn.utils.parametrizations.weight_norm(m.fuse)

    ref, cand = _pair(16, 3, torch.float32, edit, fused_generator_training=True)
    assert cand._hip_fuse()
    _compare(ref, cand, torch.float32, 3, (2, 16, 15, 17))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_fuse_reflect_padding(dtype):
    """fuse replaced by a reflect-padded convolution: the result is the
    reflect-padded convolution's, not the zero-padded one's."""
    say(f"fuse padding_mode=reflect dtype={dtype}")

    def edit(m):
        conv = nn.Conv2d(64, 16, 3, padding=1, padding_mode="reflect").to(m.fuse.weight)
        with torch.no_grad():
            conv.weight.copy_(m.fuse.weight)
            conv.bias.copy_(m.fuse.bias)
        m.fuse = conv

    ref, cand = _pair(16, 3, dtype, edit, fused_generator_training=True)
    assert not cand._hip_fuse()
    out = _compare(ref, cand, dtype, 3, (2, 16, 15, 17))
    # and it differs from the zero-padded convolution at the border
    torch.manual_seed(123)
    plain = DDPM(16, 3, fused_generator_training=True).to(DEV).to(dtype)
    plain.generator.load_state_dict(cand.generator.state_dict())
    plain.fuse.load_state_dict(cand.fuse.state_dict())
    torch.manual_seed(5)
    x = torch.randn(2, 16, 15, 17).to(dtype)
    y = torch.randn_like(x)
    with torch.no_grad():
        zero_padded = plain(x.to(DEV), y.to(DEV))
    assert (zero_padded[..., 0, :] - out.detach()[..., 0, :]).abs().max().item() > 1e-3


def test_generator_hook_on_materialized_route():
    """The materialized route calls self.generator(y) when the generator
    carries a hook (here one that halves the generated kernels)."""
    say("generator forward hook, materialized route K=5 fp32")
    calls = []

    def edit(m):
        def hook(mod, args, out):
            calls.append(1)
            return out * 0.5
        m.generator.register_forward_hook(hook)

    ref, cand = _pair(16, 5, torch.float32, edit, fused_generator_training=False)
    _compare(ref, cand, torch.float32, 5, (1, 16, 12, 20))
    assert len(calls) == 2


def test_fused_training_peak_memory_256_fp32():
    """Peak temporary memory of the fp32 fused training step at B1 C64 K3
    256x256, measured as gpu_memory_bench.py:47-76 does (warm-up, gradients
    released, reset peak, baseline, one step): at most 180 MiB, under 10% of
    the Unfold route's 1825 MiB (the pair-plane concat is released before the
    generator's backward allocates its buffers)."""
    say("peak temporary memory, fused fp32 training 256x256 C=64")
    torch.manual_seed(21)
    module = DDPM(64, 3).to(DEV).train()
    x = torch.randn(1, 64, 256, 256, device=DEV, requires_grad=True)
    y = torch.randn(1, 64, 256, 256, device=DEV, requires_grad=True)

    def step():
        module.zero_grad(set_to_none=True)
        x.grad = None
        y.grad = None
        module(x, y).square().mean().backward()

    for _ in range(2):
        step()
    torch.cuda.synchronize()
    module.zero_grad(set_to_none=True)
    x.grad = None
    y.grad = None
    torch.cuda.empty_cache()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    step()
    torch.cuda.synchronize()
    peak_mib = (torch.cuda.max_memory_allocated() - base) / 2**20
    say(f"  peak temporary memory {peak_mib:.1f} MiB")
    assert peak_mib <= 180.0, f"peak temporary memory {peak_mib:.1f} MiB"
