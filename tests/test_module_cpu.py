"""CPU tests of the drop-in module, restating the reference's own unit tests
(test_triton_impl.py:9-65) against the oracle, plus the config with C=32,
48x48 (CPU inference plumbing)."""

import pytest
import torch

from dynamicconvolutionoperator_amd import DDPM
from oracle.unfold_ref import UnfoldDDPM


def _models(channels, kernel_size, max_generated_bytes=0):
    torch.manual_seed(123)
    reference = UnfoldDDPM(channels, kernel_size)
    candidate = DDPM(
        channels,
        kernel_size,
        spatial_tile_size=11,  # tile boundaries that do not divide H*W
        max_generated_bytes=max_generated_bytes,
        recompute=True,
    )
    candidate.load_state_dict(reference.state_dict())
    return reference, candidate


@pytest.mark.parametrize("kernel_size", [1, 3, 5])
def test_forward_matches_unfold_across_tile_boundaries(kernel_size):
    reference, candidate = _models(3, kernel_size)
    x = torch.randn(2, 3, 5, 7)
    y = torch.randn_like(x)
    with torch.no_grad():
        expected = reference(x, y)
        actual = candidate(x, y)
    torch.testing.assert_close(actual, expected, atol=2e-6, rtol=2e-5)


@pytest.mark.parametrize("budget", [0, 1024**3])
def test_backward_matches_unfold_with_recomputation(budget):
    reference, candidate = _models(4, 3, budget)
    x_ref = torch.randn(2, 4, 5, 7, requires_grad=True)
    y_ref = torch.randn_like(x_ref, requires_grad=True)
    x_new = x_ref.detach().clone().requires_grad_()
    y_new = y_ref.detach().clone().requires_grad_()
    expected = reference(x_ref, y_ref)
    actual = candidate(x_new, y_new)
    expected_grads = torch.autograd.grad(expected.square().mean(), (x_ref, y_ref, *reference.parameters()))
    actual_grads = torch.autograd.grad(actual.square().mean(), (x_new, y_new, *candidate.parameters()))
    torch.testing.assert_close(actual, expected, atol=2e-6, rtol=2e-5)
    for a, e in zip(actual_grads, expected_grads):
        torch.testing.assert_close(a, e, atol=3e-6, rtol=3e-5)


def test_native_shifted_view_backward_matches_unfold():
    """Inference-time module (eval) with grad: the shifted-view custom backward."""
    reference, candidate = _models(3, 3, 1024**3)
    candidate.eval()
    x_ref = torch.randn(1, 3, 6, 9, requires_grad=True)
    y_ref = torch.randn_like(x_ref, requires_grad=True)
    x_new = x_ref.detach().clone().requires_grad_()
    y_new = y_ref.detach().clone().requires_grad_()
    e = torch.autograd.grad(reference(x_ref, y_ref).sum(), (x_ref, y_ref))
    a = torch.autograd.grad(candidate(x_new, y_new).sum(), (x_new, y_new))
    for ai, ei in zip(a, e):
        torch.testing.assert_close(ai, ei, atol=3e-6, rtol=3e-5)


def test_cpu_inference_c32_48x48():
    """C=32, K=3, B=1, 48x48 fp32 inference (the shifted-view CPU route)."""
    torch.manual_seed(123)
    reference = UnfoldDDPM(32, 3)
    candidate = DDPM(32, 3)
    candidate.load_state_dict(reference.state_dict())
    torch.manual_seed(456)
    x = torch.randn(1, 32, 48, 48)
    y = torch.randn_like(x)
    with torch.no_grad():
        torch.testing.assert_close(candidate(x, y), reference(x, y), atol=2e-5, rtol=2e-5)


def test_rejects_invalid_shapes():
    model = DDPM(4, 3)
    with pytest.raises(ValueError, match="identical shapes"):
        model(torch.randn(1, 4, 5, 5), torch.randn(1, 4, 4, 5))
    with pytest.raises(ValueError, match="NCHW"):
        model(torch.randn(4, 5, 5), torch.randn(4, 5, 5))
    with pytest.raises(ValueError, match="expected 4 channels"):
        model(torch.randn(1, 3, 5, 5), torch.randn(1, 3, 5, 5))


def test_rejects_even_kernel_and_bad_dim():
    with pytest.raises(ValueError, match="positive odd"):
        DDPM(4, 2)
    with pytest.raises(ValueError, match="dim must be positive"):
        DDPM(0, 3)


def test_state_dict_and_parameter_order_match_reference():
    torch.manual_seed(5)
    ref = UnfoldDDPM(6, 3)
    torch.manual_seed(5)
    new = DDPM(6, 3)
    assert list(new.state_dict()) == ["generator.weight", "generator.bias", "fuse.weight", "fuse.bias"]
    for a, b in zip(new.parameters(), ref.parameters()):
        assert torch.equal(a, b)  # same seeded default init (generator created first)
    assert new.dilations == (1, 3, 5)
