"""Pins the oracle before anything is checked against it.

Each check is chosen so that a plausible mistake in the oracle (transposed
taps, swapped branch/channel order in the generator rows, wrong dilation sign,
missing zero padding, a dropped term in the backward) fails at least one:
integer known-answer vectors from a self-contained loop script, closed forms,
autograd through the Unfold graph, the adjoint identity, and agreement of two
independent restatements (torch Unfold and loop-level C).
"""

import numpy as np
import pytest
import torch

from oracle import c_oracle
from oracle import unfold_ref as ref

DIL = (1, 3, 5)


def t64(a):
    return torch.tensor(a, dtype=torch.float64)


# ---------------------------------------------------------------- known answers
def test_kat_filter_forward_and_backward(kat_cases):
    for case in (c for c in kat_cases if c["kind"] == "filter"):
        K = case["K"]
        x, k, g = t64(case["x"]), t64(case["kernels"]), t64(case["grad_out"])
        out = ref.dynamic_cat(x, k, K)
        assert torch.equal(out, t64(case["out"])), f"torch fwd K={K}"
        dx, dk = ref.dynamic_cat_backward(x, k, g, K)
        assert torch.equal(dx, t64(case["grad_x"])), f"torch dx K={K}"
        assert torch.equal(dk, t64(case["grad_kernels"])), f"torch dk K={K}"
        np.testing.assert_array_equal(c_oracle.dynamic_cat(x.numpy(), k.numpy(), K), case["out"])
        cdx, cdk = c_oracle.dynamic_cat_backward(x.numpy(), k.numpy(), g.numpy(), K)
        np.testing.assert_array_equal(cdx, case["grad_x"])
        np.testing.assert_array_equal(cdk, case["grad_kernels"])


def test_kat_generator_forward_and_backward(kat_cases):
    for case in (c for c in kat_cases if c["kind"] == "generator"):
        K, C = case["K"], case["C"]
        x, y, g = t64(case["x"]), t64(case["y"]), t64(case["grad_out"])
        w = t64(case["weight"]).reshape(3 * C * K * K, C, 1, 1)
        b = t64(case["bias"])
        out = ref.generator_dynamic_cat(x, y, w, b, K)
        assert torch.equal(out, t64(case["out"])), f"torch gen fwd K={K}"
        dx, dy, dw, db = ref.generator_dynamic_cat_backward(x, y, w, b, g, K)
        assert torch.equal(dx, t64(case["grad_x"]))
        assert torch.equal(dy, t64(case["grad_y"]))
        assert torch.equal(dw.reshape(-1, C), t64(case["grad_weight"]))
        assert torch.equal(db, t64(case["grad_bias"]))
        np.testing.assert_array_equal(
            c_oracle.generator_dynamic_cat(x.numpy(), y.numpy(), w.numpy(), b.numpy(), K), case["out"]
        )
        cdx, cdy, cdw, cdb = c_oracle.generator_dynamic_cat_backward(
            x.numpy(), y.numpy(), w.numpy(), b.numpy(), g.numpy(), K
        )
        np.testing.assert_array_equal(cdx, case["grad_x"])
        np.testing.assert_array_equal(cdy, case["grad_y"])
        np.testing.assert_array_equal(cdw.reshape(-1, C), case["grad_weight"])
        np.testing.assert_array_equal(cdb, case["grad_bias"])


# ---------------------------------------------------------------- closed forms
@pytest.mark.parametrize("K", [1, 3, 5])
def test_identity_channels_are_x(K):
    g = torch.Generator().manual_seed(0)
    x = torch.randn(2, 3, 6, 9, generator=g, dtype=torch.float64)
    k = torch.randn(2, 3, 3, K * K, 6, 9, generator=g, dtype=torch.float64)
    assert torch.equal(ref.dynamic_cat(x, k, K)[:, :3], x)


def test_k1_is_elementwise_product_for_every_dilation():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(2, 4, 5, 7, generator=g, dtype=torch.float64)
    k = torch.randn(2, 3, 4, 1, 5, 7, generator=g, dtype=torch.float64)
    out = ref.dynamic_cat(x, k, 1)
    for b in range(3):
        assert torch.allclose(out[:, 4 * (b + 1) : 4 * (b + 2)], k[:, b, :, 0] * x, rtol=0, atol=0)


def test_zero_kernels_give_zero_branches():
    x = torch.randn(1, 2, 8, 8, dtype=torch.float64)
    k = torch.zeros(1, 3, 2, 9, 8, 8, dtype=torch.float64)
    assert torch.count_nonzero(ref.dynamic_cat(x, k, 3)[:, 2:]) == 0


@pytest.mark.parametrize("ki,kj", [(0, 0), (0, 2), (2, 1), (1, 1)])
def test_one_hot_kernel_is_zero_padded_shift(ki, kj):
    K, H, W = 3, 9, 13
    x = torch.arange(H * W, dtype=torch.float64).reshape(1, 1, H, W) + 1
    k = torch.zeros(1, 3, 1, 9, H, W, dtype=torch.float64)
    k[:, :, :, ki * K + kj] = 1
    out = ref.dynamic_cat(x, k, K)
    for b, d in enumerate(DIL):
        dh, dw = (ki - 1) * d, (kj - 1) * d
        expect = torch.zeros(H, W, dtype=torch.float64)
        for h in range(H):
            for w in range(W):
                if 0 <= h + dh < H and 0 <= w + dw < W:
                    expect[h, w] = x[0, 0, h + dh, w + dw]
        assert torch.equal(out[0, 1 + b], expect), (b, d)


# ---------------------------------------------------------------- backward
@pytest.mark.parametrize("K", [1, 3, 5])
def test_closed_form_backward_matches_autograd(K):
    g = torch.Generator().manual_seed(2 + K)
    n, c, h, w = 2, 3, 7, 10
    x = torch.randn(n, c, h, w, generator=g, dtype=torch.float64, requires_grad=True)
    y = torch.randn(n, c, h, w, generator=g, dtype=torch.float64, requires_grad=True)
    wt = torch.randn(3 * c * K * K, c, 1, 1, generator=g, dtype=torch.float64, requires_grad=True)
    b = torch.randn(3 * c * K * K, generator=g, dtype=torch.float64, requires_grad=True)
    go = torch.randn(n, 4 * c, h, w, generator=g, dtype=torch.float64)
    out = ref.generator_dynamic_cat(x, y, wt, b, K)
    auto = torch.autograd.grad(out, (x, y, wt, b), go)
    closed = ref.generator_dynamic_cat_backward(x.detach(), y.detach(), wt.detach(), b.detach(), go, K)
    for a, cf in zip(auto, closed):
        torch.testing.assert_close(cf, a, rtol=1e-12, atol=1e-12)


def test_adjoint_identity_filter():
    g = torch.Generator().manual_seed(7)
    x = torch.randn(1, 4, 11, 9, generator=g, dtype=torch.float64)
    k = torch.randn(1, 3, 4, 9, 11, 9, generator=g, dtype=torch.float64)
    go = torch.randn(1, 16, 11, 9, generator=g, dtype=torch.float64)
    vx = torch.randn_like(x)
    vk = torch.randn_like(k)
    dx, dk = ref.dynamic_cat_backward(x, k, go, 3)
    # out is linear in x for fixed k and linear in k for fixed x
    lhs_x = (ref.dynamic_cat(vx, k, 3) * go).sum()
    lhs_k = (ref.dynamic_cat(x, vk, 3)[:, 4:] * go[:, 4:]).sum()
    torch.testing.assert_close(lhs_x, (vx * dx).sum(), rtol=1e-12, atol=1e-10)
    torch.testing.assert_close(lhs_k, (vk * dk).sum(), rtol=1e-12, atol=1e-10)


# ---------------------------------------------------------------- two restatements agree
@pytest.mark.parametrize("K", [1, 3, 5])
def test_torch_and_c_restatements_agree(K):
    g = torch.Generator().manual_seed(30 + K)
    n, c, h, w = 2, 5, 13, 21
    x = torch.randn(n, c, h, w, generator=g, dtype=torch.float64)
    y = torch.randn(n, c, h, w, generator=g, dtype=torch.float64)
    wt = torch.randn(3 * c * K * K, c, 1, 1, generator=g, dtype=torch.float64) * 0.3
    b = torch.randn(3 * c * K * K, generator=g, dtype=torch.float64)
    go = torch.randn(n, 4 * c, h, w, generator=g, dtype=torch.float64)
    out_t = ref.generator_dynamic_cat(x, y, wt, b, K).numpy()
    out_c = c_oracle.generator_dynamic_cat(x.numpy(), y.numpy(), wt.numpy(), b.numpy(), K)
    np.testing.assert_allclose(out_c, out_t, rtol=1e-12, atol=1e-11)
    grads_t = ref.generator_dynamic_cat_backward(x, y, wt, b, go, K)
    grads_c = c_oracle.generator_dynamic_cat_backward(
        x.numpy(), y.numpy(), wt.numpy(), b.numpy(), go.numpy(), K
    )
    for gt, gc in zip(grads_t, grads_c):
        np.testing.assert_allclose(gc, gt.numpy(), rtol=1e-11, atol=1e-10)


def test_unfold_module_matches_functional_form():
    torch.manual_seed(123)
    m = ref.UnfoldDDPM(6, 3).double()
    x = torch.randn(2, 6, 9, 10, dtype=torch.float64)
    y = torch.randn_like(x)
    cat = ref.generator_dynamic_cat(x, y, m.generator.weight, m.generator.bias, 3)
    torch.testing.assert_close(m(x, y), m.fuse(cat), rtol=0, atol=0)
    assert list(m.state_dict()) == ["generator.weight", "generator.bias", "fuse.weight", "fuse.bias"]
