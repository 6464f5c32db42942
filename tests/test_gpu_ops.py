"""Operator-level parity of the HIP kernels with the oracle (GPU).

Every entry point of libddpm_hip.so is called through the drop-in operators
(fused_dynamic_cat, fused_generator_dynamic_cat) on seeded inputs and compared
with the CPU float64 oracle computed from the same (dtype-rounded) inputs.
"""

import pytest
import torch

from dynamicconvolutionoperator_amd import ops
from oracle import unfold_ref as ref
from tests.gpu_helpers import DEV, DIL, TOL, assert_close, default_generator_params, randn, say

pytestmark = pytest.mark.gpu

SHAPES = [
    (2, 24, 15, 17),  # non-aligned channels and width (scalar path)
    (1, 16, 16, 32),  # W % 4 == 0 (vector path), C = 16
    (1, 64, 20, 64),  # C = 64, several tiles
    (1, 10, 12, 40),  # C % 4 != 0: element-wise tails of the weight-gradient stores
]


def t(case, key, dtype=torch.float32):
    return torch.tensor(case[key], dtype=torch.float64).to(dtype)


# ---------------------------------------------------------------- known answers (exact)
def test_kat_filter_exact(kat_cases):
    for case in (c for c in kat_cases if c["kind"] == "filter"):
        K = case["K"]
        say(f"kat filter K={K} shape=({case['N']},{case['C']},{case['H']},{case['W']})")
        x = t(case, "x").to(DEV).requires_grad_()
        k = t(case, "kernels").to(DEV).requires_grad_()
        out = ops.fused_dynamic_cat(x, k, K, DIL)
        assert torch.equal(out.cpu().double(), t(case, "out", torch.float64))
        out.backward(t(case, "grad_out").to(DEV))
        assert torch.equal(x.grad.cpu().double(), t(case, "grad_x", torch.float64))
        assert torch.equal(k.grad.cpu().double(), t(case, "grad_kernels", torch.float64))


def test_kat_generator_exact(kat_cases):
    for case in (c for c in kat_cases if c["kind"] == "generator"):
        K, C = case["K"], case["C"]
        say(f"kat generator K={K} shape=({case['N']},{C},{case['H']},{case['W']})")
        x = t(case, "x").to(DEV).requires_grad_()
        y = t(case, "y").to(DEV).requires_grad_()
        w = t(case, "weight").reshape(3 * C * K * K, C, 1, 1).to(DEV).requires_grad_()
        b = t(case, "bias").to(DEV).requires_grad_()
        out = ops.fused_generator_dynamic_cat(x, y, w, b, K, DIL)
        assert torch.equal(out.detach().cpu().double(), t(case, "out", torch.float64))
        out.backward(t(case, "grad_out").to(DEV))
        assert torch.equal(x.grad.cpu().double(), t(case, "grad_x", torch.float64))
        assert torch.equal(y.grad.cpu().double(), t(case, "grad_y", torch.float64))
        assert torch.equal(w.grad.reshape(-1, C).cpu().double(), t(case, "grad_weight", torch.float64))
        assert torch.equal(b.grad.cpu().double(), t(case, "grad_bias", torch.float64))


# ---------------------------------------------------------------- materialized filter
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("K", [1, 3, 5])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_filter_matches_oracle(shape, K, dtype):
    n, c, h, w = shape
    say(f"filter shape={shape} K={K} dtype={dtype}")
    x = randn(shape, 10, dtype)
    k = randn((n, 3, c, K * K, h, w), 11, dtype)
    g = randn((n, 4 * c, h, w), 12, dtype)
    xd = x.to(DEV).requires_grad_()
    kd = k.to(DEV).requires_grad_()
    out = ops.fused_dynamic_cat(xd, kd, K, DIL)
    assert out.dtype == dtype
    out.backward(g.to(DEV))
    atol, rtol = TOL["filter"][dtype]
    x64, k64, g64 = x.double(), k.double(), g.double()
    assert_close(out, ref.dynamic_cat(x64, k64, K), atol, rtol, "filter out")
    dx, dk = ref.dynamic_cat_backward(x64, k64, g64, K)
    assert_close(xd.grad, dx, atol, rtol, "filter dx")
    assert_close(kd.grad, dk, atol, rtol, "filter dk")


@pytest.mark.parametrize("w", [20, 32])  # W % 8 != 0 / == 0 (16-byte kernel chunks in dX)
def test_filter_mixed_dtypes_autocast_layout(w):
    """x fp32 with bf16 kernels (the autocast case): out and dK in bf16, dX in fp32."""
    n, c, h, K = 1, 8, 12, 3
    x = randn((n, c, h, w), 20, torch.float32)
    k = randn((n, 3, c, K * K, h, w), 21, torch.bfloat16)
    g = randn((n, 4 * c, h, w), 22, torch.bfloat16)
    xd = x.to(DEV).requires_grad_()
    kd = k.to(DEV).requires_grad_()
    out = ops.fused_dynamic_cat(xd, kd, K, DIL)
    assert out.dtype == torch.bfloat16
    out.backward(g.to(DEV))
    assert xd.grad.dtype == torch.float32 and kd.grad.dtype == torch.bfloat16
    assert_close(out, ref.dynamic_cat(x.double(), k.double(), K), 2e-2, 1e-2, "mixed out")
    dx, dk = ref.dynamic_cat_backward(x.double(), k.double(), g.double(), K)
    assert_close(xd.grad, dx, 2e-4, 1e-4, "mixed dx")
    assert_close(kd.grad, dk, 2e-2, 1e-2, "mixed dk")


# ---------------------------------------------------------------- fused generator
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("K", [1, 3])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_generator_matches_oracle(shape, K, dtype):
    n, c, h, w = shape
    say(f"generator shape={shape} K={K} dtype={dtype}")
    x = randn(shape, 30, dtype)
    y = randn(shape, 31, dtype)
    wt, b = default_generator_params(c, K, 32, dtype)
    g = randn((n, 4 * c, h, w), 33, dtype)
    xd, yd = x.to(DEV).requires_grad_(), y.to(DEV).requires_grad_()
    wd, bd = wt.to(DEV).requires_grad_(), b.to(DEV).requires_grad_()
    out = ops.fused_generator_dynamic_cat(xd, yd, wd, bd, K, DIL)
    assert out.dtype == dtype
    out.backward(g.to(DEV))

    x64, y64, w64, b64, g64 = (v.double() for v in (x, y, wt, b, g))
    kern = ref.generated_kernels(y64, w64, b64, K)
    if dtype != torch.float32:
        kern = kern.to(dtype).double()  # the generated taps are rounded to the input dtype
    atol, rtol = TOL["gen_fwd"][dtype]
    assert_close(out, ref.dynamic_cat(x64, kern, K), atol, rtol, "gen out")
    dx, dy, dw, db = ref.generator_dynamic_cat_backward(x64, y64, w64, b64, g64, K)
    atol, rtol = TOL["gen_bwd"][dtype]
    # gradient magnitudes scale with the number of summed terms; compare relative to the max
    for name, a, e in (("dx", xd.grad, dx), ("dy", yd.grad, dy), ("dw", wd.grad, dw), ("db", bd.grad, db)):
        scale = max(1.0, e.abs().max().item())
        assert_close(a, e, atol * scale, rtol, f"gen {name}")


@pytest.mark.parametrize(
    "shape",
    [
        (1, 72, 13, 21),   # 65..96 channels: four K steps, the last one partly zero
        (2, 128, 16, 40),  # the largest fused channel count, W % 4 == 0
    ],
)
@pytest.mark.parametrize("K", [1, 3])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_generator_wide_channels_match_oracle(shape, K, dtype):
    """65..128 channels on the fused kernels: 32-column tiles, dY and dW over two
    halves of the output / input channels."""
    n, c, h, w = shape
    say(f"generator wide shape={shape} K={K} dtype={dtype}")
    assert ops.generator_supported(c, K, DIL)
    x = randn(shape, 38, dtype)
    y = randn(shape, 39, dtype)
    wt, b = default_generator_params(c, K, 40, dtype)
    g = randn((n, 4 * c, h, w), 41, dtype)
    xd, yd = x.to(DEV).requires_grad_(), y.to(DEV).requires_grad_()
    wd, bd = wt.to(DEV).requires_grad_(), b.to(DEV).requires_grad_()
    out = ops.fused_generator_dynamic_cat(xd, yd, wd, bd, K, DIL)
    out.backward(g.to(DEV))
    x64, y64, w64, b64, g64 = (v.double() for v in (x, y, wt, b, g))
    kern = ref.generated_kernels(y64, w64, b64, K)
    if dtype != torch.float32:
        kern = kern.to(dtype).double()
    atol, rtol = TOL["gen_fwd"][dtype]
    assert_close(out, ref.dynamic_cat(x64, kern, K), atol, rtol, "gen out")
    dx, dy, dw, db = ref.generator_dynamic_cat_backward(x64, y64, w64, b64, g64, K)
    atol, rtol = TOL["gen_bwd"][dtype]
    for name, a, e in (("dx", xd.grad, dx), ("dy", yd.grad, dy), ("dw", wd.grad, dw), ("db", bd.grad, db)):
        scale = max(1.0, e.abs().max().item())
        assert_close(a, e, atol * scale, rtol, f"gen {name}")


@pytest.mark.parametrize(
    "shape,dil",
    [
        ((2, 24, 15, 17), (1, 3, 5)),   # non-aligned channels and width
        ((1, 40, 37, 45), (1, 3, 5)),   # W % 4 != 0, several tiles
        ((1, 24, 36, 72), (1, 3, 5)),   # W % 4 == 0 (vector halo staging)
        ((1, 64, 32, 64), (2, 4, 6)),   # the largest K = 5 halo (radius 12)
        ((1, 96, 20, 36), (1, 3, 5)),   # 65..128 channels: four K steps
    ],
)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_generator_forward_k5_matches_oracle(shape, dil, dtype):
    """The fused forward at K = 5 (inference: no gradient needed), as the
    reference fuses inference at any K (triton_impl.py:317-338)."""
    n, c, h, w = shape
    say(f"generator forward K=5 shape={shape} dil={dil} dtype={dtype}")
    assert ops.generator_supported(c, 5, dil, forward_only=True)
    assert not ops.generator_supported(c, 5, dil)
    x = randn(shape, 50, dtype)
    y = randn(shape, 51, dtype)
    wt, b = default_generator_params(c, 5, 52, dtype)
    calls = []
    real = ops._launch_generator_dynamic_cat

    def spy(*a, **k):
        calls.append(1)
        return real(*a, **k)

    ops._launch_generator_dynamic_cat = spy
    try:
        with torch.no_grad():
            out = ops.fused_generator_dynamic_cat(x.to(DEV), y.to(DEV), wt.to(DEV), b.to(DEV), 5, dil)
    finally:
        ops._launch_generator_dynamic_cat = real
    assert calls, "K = 5 inference did not take the fused forward"
    assert out.dtype == dtype
    x64, y64, w64, b64 = (v.double() for v in (x, y, wt, b))
    kern = ref.generated_kernels(y64, w64, b64, 5)
    if dtype != torch.float32:
        kern = kern.to(dtype).double()
    atol, rtol = TOL["gen_fwd"][dtype]
    assert_close(out, ref.dynamic_cat(x64, kern, 5, dil), atol, rtol, "gen K5 out")


def test_generator_k5_with_grad_materializes():
    """With gradients needed, K = 5 keeps the materialized route (the fused
    backward covers K <= 3), with the fused forward's result."""
    shape = (1, 16, 12, 20)
    x = randn(shape, 53).to(DEV)
    y = randn(shape, 54).to(DEV)
    wt, b = default_generator_params(16, 5, 55, torch.float32)
    wt, b = wt.to(DEV), b.to(DEV)
    with torch.no_grad():
        fused = ops.fused_generator_dynamic_cat(x, y, wt, b, 5, DIL)
    xs = x.clone().requires_grad_()
    out = ops.fused_generator_dynamic_cat(xs, y, wt, b, 5, DIL)
    assert out.grad_fn is not None and "DynamicCat" in type(out.grad_fn).__name__
    assert "Generator" not in type(out.grad_fn).__name__
    assert_close(out, fused.cpu().double(), 2e-4, 1e-4, "materialized vs fused K5")


@pytest.mark.parametrize(
    "K,dil,fused",
    [
        (3, (2, 7, 8), True),    # largest dilation the fused kernels stage
        (3, (1, 2, 6), True),    # halo radius 6 (partial rows shifted by 2)
        (3, (4, 1, 1), True),    # halo radius 4 (no shift)
        (1, (1, 12, 20), True),  # a 1x1 tap ignores the dilation
        (3, (1, 3, 9), False),   # beyond the fused halo: materialized route
    ],
)
@pytest.mark.parametrize("shape", [(1, 40, 37, 45), (1, 24, 36, 72)])  # W % 4 != 0 / == 0
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_generator_dilation_sets(K, dil, fused, shape, dtype):
    n, c, h, w = shape
    say(f"generator dilations={dil} K={K} dtype={dtype}")
    assert ops.generator_supported(c, K, dil) == fused
    x = randn(shape, 34, dtype)
    y = randn(shape, 35, dtype)
    wt, b = default_generator_params(c, K, 36, dtype)
    g = randn((n, 4 * c, h, w), 37, dtype)
    xd, yd = x.to(DEV).requires_grad_(), y.to(DEV).requires_grad_()
    wd, bd = wt.to(DEV).requires_grad_(), b.to(DEV).requires_grad_()
    out = ops.fused_generator_dynamic_cat(xd, yd, wd, bd, K, dil)
    out.backward(g.to(DEV))
    x64, y64, w64, b64, g64 = (v.double() for v in (x, y, wt, b, g))
    kern = ref.generated_kernels(y64, w64, b64, K)
    if dtype != torch.float32:
        kern = kern.to(dtype).double()
    atol, rtol = TOL["gen_fwd"][dtype]
    assert_close(out, ref.dynamic_cat(x64, kern, K, dil), atol, rtol, "gen out")
    dx, dy, dw, db = ref.generator_dynamic_cat_backward(x64, y64, w64, b64, g64, K, dil)
    atol, rtol = TOL["gen_bwd"][dtype]
    for name, a, e in (("dx", xd.grad, dx), ("dy", yd.grad, dy), ("dw", wd.grad, dw), ("db", bd.grad, db)):
        scale = max(1.0, e.abs().max().item())
        assert_close(a, e, atol * scale, rtol, f"gen {name}")


# ---------------------------------------------------------------- generator 1x1 conv (materialized route)
@pytest.mark.parametrize(
    "shape,K",
    [
        ((2, 24, 15, 17), 5),  # H*W % 4 != 0: element-wise stores
        ((1, 20, 16, 16), 3),  # C % 8 != 0: element-wise weight loads
        ((1, 64, 32, 32), 5),  # the K = 5 configuration's channel count
        ((1, 128, 8, 12), 1),  # the largest C, four 32-channel K steps
        # weight / bias gradients summed over split partials (one workgroup
        # per 64 rows and pixel range, partials reduced in split order):
        ((2, 64, 48, 64), 5),  # 6 splits of pixel steps spanning both images
        ((3, 8, 40, 40), 5),   # C = 8: one channel block, 5 (2-byte) / 10 (fp32) splits
        ((2, 24, 45, 37), 3),  # odd H*W: element-wise operand loads, 4 splits
        ((1, 128, 32, 64), 3),  # C = 128: 64-pixel steps, 4 splits
        ((1, 8, 16, 24), 3),   # 216 rows o: dY in one o split, written directly
    ],
)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_generator_kernels_match_oracle(shape, K, dtype):
    n, c, h, w = shape
    say(f"generator kernels shape={shape} K={K} dtype={dtype}")
    y = randn(shape, 70, dtype)
    wt, b = default_generator_params(c, K, 71, dtype)
    g = randn((n, 3 * c * K * K, h, w), 72, dtype)
    yd, wd, bd = (t.to(DEV).requires_grad_() for t in (y, wt, b))
    assert ops.generator_kernels_supported(yd, wd, bd)
    out = ops.generator_kernels(yd, wd, bd, K)
    assert out.dtype == dtype and tuple(out.shape) == (n, 3 * c * K * K, h, w)
    out.backward(g.to(DEV))
    y64, w64, b64, g64 = (t.double().requires_grad_() for t in (y, wt, b, g))
    e = ref.generated_kernels(y64, w64, b64, K).reshape(n, -1, h, w)
    atol, rtol = TOL["gen_fwd"][dtype]
    assert_close(out, e, atol, rtol, "generator kernels")
    dy, dw, db = torch.autograd.grad(e, (y64, w64, b64), g64.detach())
    atol, rtol = TOL["gen_bwd"][dtype]
    for name, a, ex in (("dy", yd.grad, dy), ("dw", wd.grad, dw), ("db", bd.grad, db)):
        scale = max(1.0, ex.abs().max().item())
        assert_close(a, ex, atol * scale, rtol, f"generator kernels {name}")


def test_generator_kernels_weight_gradient_deterministic_and_empty():
    """Split partials are summed in a fixed order: two backward passes agree
    bit for bit.  An empty batch gives zero weight / bias gradients."""
    c, K = 64, 5
    say("generator kernels weight gradient determinism")
    wt, b = default_generator_params(c, K, 74, torch.float32)
    y = randn((2, c, 48, 64), 75).to(DEV)
    g = randn((2, 3 * c * K * K, 48, 64), 76).to(DEV)
    grads = []
    for _ in range(2):
        wd, bd = (t.to(DEV).requires_grad_() for t in (wt, b))
        ops.generator_kernels(y, wd, bd, K).backward(g)
        grads.append((wd.grad.clone(), bd.grad.clone()))
    assert torch.equal(grads[0][0], grads[1][0]) and torch.equal(grads[0][1], grads[1][1])
    say("generator kernels empty batch")
    wd, bd = (t.to(DEV).requires_grad_() for t in (wt, b))
    y0 = torch.zeros((0, c, 8, 8), device=DEV, requires_grad=True)
    ops.generator_kernels(y0, wd, bd, K).sum().backward()
    assert torch.count_nonzero(wd.grad) == 0 and torch.count_nonzero(bd.grad) == 0


def test_generator_inference_has_no_autograd_graph():
    x = randn((1, 8, 9, 16), 40).to(DEV)
    y = randn((1, 8, 9, 16), 41).to(DEV)
    wt, b = default_generator_params(8, 3, 42, torch.float32)
    with torch.no_grad():
        out = ops.fused_generator_dynamic_cat(x, y, wt.to(DEV), b.to(DEV), 3, DIL)
    assert out.grad_fn is None
    with torch.inference_mode():
        out2 = ops.fused_generator_dynamic_cat(x, y, wt.to(DEV), b.to(DEV), 3, DIL)
    assert torch.equal(out, out2)


@pytest.mark.parametrize(
    "shape",
    [
        # steps = row segments of 128 columns; at most 16 splits of at least 4 steps
        (2, 32, 40, 64),     # 80 steps -> 16 splits of 5
        (1, 24, 4, 17),      # 4 steps -> one split writes the gradients directly
        (1, 10, 3, 20),      # C % 4 != 0, direct
        (1, 10, 24, 40),     # C % 4 != 0, 24 steps -> 6 splits, scalar split reduction
        (2, 64, 128, 136),   # 512 steps -> 16 splits, a partial 128-column block per row
        (1, 24, 150, 130),   # W % 8 != 0 (element-wise y / gradient copies), 16 splits
        (1, 96, 40, 64),     # two input-channel halves (the second partly zero), 10 splits
        (1, 128, 4, 20),     # two halves, one split writes the gradients directly
    ],
)
def test_generator_weight_gradient_splits(shape):
    n, c, h, w = shape
    say(f"weight gradient shape={shape}")
    x = randn(shape, 50)
    y = randn(shape, 51)
    wt, b = default_generator_params(c, 3, 52, torch.float32)
    g = randn((n, 4 * c, h, w), 53)
    wd, bd = wt.to(DEV).requires_grad_(), b.to(DEV).requires_grad_()
    out = ops.fused_generator_dynamic_cat(x.to(DEV), y.to(DEV), wd, bd, 3, DIL)
    out.backward(g.to(DEV))
    _, _, dw, db = ref.generator_dynamic_cat_backward(x.double(), y.double(), wt.double(), b.double(), g.double(), 3)
    assert_close(wd.grad, dw, 3e-3 * dw.abs().max().item(), 3e-3, "split dw")
    assert_close(bd.grad, db, 3e-3 * db.abs().max().item(), 3e-3, "split db")


def test_deterministic_backward():
    shape = (1, 64, 64, 64)
    x = randn(shape, 60).to(DEV)
    y = randn(shape, 61).to(DEV)
    wt, b = default_generator_params(64, 3, 62, torch.float32)
    g = randn((1, 256, 64, 64), 63).to(DEV)
    grads = []
    for _ in range(2):
        wd, bd = wt.to(DEV).requires_grad_(), b.to(DEV).requires_grad_()
        xd, yd = x.clone().requires_grad_(), y.clone().requires_grad_()
        ops.fused_generator_dynamic_cat(xd, yd, wd, bd, 3, DIL).backward(g)
        grads.append([v.grad.clone() for v in (xd, yd, wd, bd)])
    for a, b2 in zip(*grads):
        assert torch.equal(a, b2)
