"""The fp32 pair-plane concat (dtype code 3) through the C-ABI, and the fused
module op built on it.

* ddpm_gen_fwd with dtype 3 writes the concat as bf16 (hi, lo) pair planes:
  bit for bit a host split of the plain fp32 concat (hi = the top 16 bits of
  each fp32 pattern, lo = the remainder rounded to nearest even by torch's
  float -> bfloat16 conversion; per 32-plane chunk, plane j < 16 = the hi
  halves of channels 2j (low 16 bits) and 2j + 1, plane 16 + j their lo
  halves).
* ddpm_fuse_conv_fwd with dtype 3 feeds the MFMA the operands the fp32 path
  splits itself, in another channel order within each 32-plane chunk:
  against float64 F.conv2d at the fuse convolution's fp32 tolerance.
* ddpm_fuse_conv_bwd_weight with dtype 3 keeps each MFMA row's channel and
  the pixel order: bit-identical to the plain fp32 call.
* ops.fused_ddpm against fuse_conv3x3(fused_generator_dynamic_cat(...)):
  the output within the fp32 fuse-convolution tolerance, every gradient
  bit-identical (the concat gradient does not depend on how the concat is
  stored).

Shapes: 4-column vector stores (W % 4 == 0) and element-wise stores (15 x
17), C = 16 / 48 / 64 (a channel block starting mid-chunk), K = 1 and 3, the
256 x 256 C = 64 workload, and C % 16 != 0 refused by ddpm_gen_fwd.
"""

import ctypes

import pytest
import torch
import torch.nn.functional as F

from dynamicconvolutionoperator_amd import _lib, ops
from tests.gpu_helpers import DEV, DIL, assert_close, default_generator_params, randn, say

pytestmark = pytest.mark.gpu

PAIRS = 3
FP32_CONV_TOL = 2e-5  # the fuse convolution's fp32 bound against float64 (relative to max |ref|)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _pair_planes(cat: torch.Tensor) -> torch.Tensor:
    """Host split of an fp32 NCHW concat into pair planes, as uint32 bit
    patterns held in int64."""
    n, ci, h, w = cat.shape
    cat = cat.detach().cpu().contiguous()
    bits = cat.view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    hi = bits >> 16
    top = bits & 0xFFFF0000
    hi_f = torch.where(top >= 2**31, top - 2**32, top).to(torch.int32).view(torch.float32)
    lo = (cat - hi_f).to(torch.bfloat16).view(torch.int16).to(torch.int64) & 0xFFFF
    hi = hi.reshape(n, ci // 32, 16, 2, h, w)
    lo = lo.reshape(n, ci // 32, 16, 2, h, w)
    words = torch.cat([hi[:, :, :, 0] | (hi[:, :, :, 1] << 16), lo[:, :, :, 0] | (lo[:, :, :, 1] << 16)], 2)
    return words.reshape(n, ci, h, w)


def _as_device_words(words: torch.Tensor) -> torch.Tensor:
    """int64-held uint32 patterns -> an fp32 device tensor with those bits."""
    w32 = torch.where(words >= 2**31, words - 2**32, words).to(torch.int32)
    return w32.view(torch.float32).to(DEV)


def _words(t: torch.Tensor) -> torch.Tensor:
    return t.detach().cpu().contiguous().view(torch.int32).to(torch.int64) & 0xFFFFFFFF


def _gen_fwd(x, y, wt, b, k, dt):
    n, c, h, w = x.shape
    out = torch.full((n, 4 * c, h, w), float("nan"), device=DEV)
    rc = _lib.load().ddpm_gen_fwd(_ptr(x), _ptr(y), _ptr(wt), _ptr(b), _ptr(out), n, c, h, w, k, *DIL, dt,
                                  _stream())
    return rc, out


GEN_CASES = [((1, 64, 64, 64), 3), ((2, 16, 20, 36), 3), ((1, 32, 40, 56), 1), ((1, 48, 15, 17), 3),
             ((1, 64, 256, 256), 3)]


@pytest.mark.parametrize("shape,k", GEN_CASES)
def test_gen_fwd_pair_planes_are_the_split_concat(shape, k):
    say(f"gen_fwd pair planes shape={shape} K={k}")
    n, c, h, w = shape
    seed = 1500 + c + w
    x = randn(shape, seed).to(DEV)
    y = randn(shape, seed + 1).to(DEV)
    wt, b = (t.to(DEV) for t in default_generator_params(c, k, seed + 2, torch.float32))
    rc, plain = _gen_fwd(x, y, wt, b, k, 0)
    assert rc == 0, rc
    rc, pairs = _gen_fwd(x, y, wt, b, k, PAIRS)
    assert rc == 0, rc
    torch.cuda.synchronize()
    assert not torch.isnan(plain).any()
    got, want = _words(pairs), _pair_planes(plain)
    bad = int((got != want).sum())
    assert bad == 0, f"{bad}/{got.numel()} pair-plane words differ from the host split"


def test_gen_fwd_pair_planes_need_whole_chunks():
    say("gen_fwd pair planes C=24 refused")
    shape = (1, 24, 8, 8)
    x = randn(shape, 1).to(DEV)
    wt, b = (t.to(DEV) for t in default_generator_params(24, 3, 2, torch.float32))
    rc, _ = _gen_fwd(x, x, wt, b, 3, PAIRS)
    assert rc == _lib.STATUS_UNSUPPORTED


CONV_CASES = [(2, 24, 15, 17), (1, 16, 12, 40), (1, 32, 19, 96), (1, 64, 128, 128), (1, 64, 256, 256)]


@pytest.mark.parametrize("shape", CONV_CASES)
def test_fuse_conv_reads_pair_planes(shape):
    say(f"fuse conv pair planes shape={shape}")
    lib = _lib.load()
    n, c, h, w = shape
    seed = 1600 + c + w
    cat = randn((n, 4 * c, h, w), seed)
    torch.manual_seed(seed + 1)
    conv = torch.nn.Conv2d(4 * c, c, 3, 1, 1)
    wt = conv.weight.detach().float()
    b = conv.bias.detach().float()
    g = randn((n, c, h, w), seed + 2)
    ref = F.conv2d(cat.double(), wt.double(), b.double(), padding=1)
    pc = _as_device_words(_pair_planes(cat))
    cd, wd, bd, gd = (t.to(DEV) for t in (cat, wt, b, g))
    ws_bytes = int(lib.ddpm_fuse_conv_workspace_bytes(n, c, h, w, PAIRS))
    assert ws_bytes == int(lib.ddpm_fuse_conv_workspace_bytes(n, c, h, w, 0))
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=DEV)
    out = torch.full((n, c, h, w), float("nan"), device=DEV)
    rc = lib.ddpm_fuse_conv_fwd(_ptr(pc), _ptr(wd), _ptr(bd), _ptr(out), _ptr(ws), ws_bytes, n, c, h, w, PAIRS,
                                _stream())
    assert rc == 0, rc
    torch.cuda.synchronize()
    scale = ref.abs().max().item()
    assert_close(out, ref, FP32_CONV_TOL * scale, FP32_CONV_TOL, f"fwd pairs {shape}")

    # weight / bias gradients: bit-identical to the plain fp32 call
    wsw_bytes = int(lib.ddpm_fuse_conv_bwd_weight_workspace_bytes(n, c, h, w, PAIRS))
    grads = []
    for src, dt in ((cd, 0), (pc, PAIRS)):
        gw = torch.full_like(wd, float("nan"))
        gb = torch.full_like(bd, float("nan"))
        wsw = torch.empty(max(wsw_bytes, 16), dtype=torch.uint8, device=DEV)
        rc = lib.ddpm_fuse_conv_bwd_weight(_ptr(src), _ptr(gd), _ptr(gw), _ptr(gb), _ptr(wsw), wsw_bytes,
                                           n, c, h, w, dt, _stream())
        assert rc == 0, rc
        torch.cuda.synchronize()
        grads.append((gw, gb))
    assert not torch.isnan(grads[0][0]).any()
    for name, a, e in (("d weight", grads[1][0], grads[0][0]), ("d bias", grads[1][1], grads[0][1])):
        assert torch.equal(a, e), f"{name} {shape}: max|diff| {(a - e).abs().max().item():.3e}"


FUSED_CASES = [((1, 64, 64, 64), 3), ((2, 16, 20, 36), 3), ((1, 48, 15, 17), 3), ((1, 32, 40, 56), 1)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape,k", FUSED_CASES)
def test_fused_ddpm_matches_the_separate_ops(shape, k, dtype):
    """fp32 (pair-plane concat): the output within the fuse convolution's
    tolerance, every gradient bit-identical; bf16 (plain concat, the same
    kernels as the separate ops): the output too bit-identical."""
    say(f"fused_ddpm shape={shape} K={k} dtype={dtype}")
    n, c, h, w = shape
    seed = 1700 + c + w
    x0 = randn(shape, seed).to(dtype)
    y0 = randn(shape, seed + 1).to(dtype)
    gw0, gb0 = default_generator_params(c, k, seed + 2, dtype)
    torch.manual_seed(seed + 3)
    conv = torch.nn.Conv2d(4 * c, c, 3, 1, 1)
    fw0, fb0 = conv.weight.detach().to(dtype), conv.bias.detach().to(dtype)
    gout = randn((n, c, h, w), seed + 4).to(dtype).to(DEV)
    runs = []
    for fused in (False, True):
        leaves = [t.to(DEV).requires_grad_() for t in (x0, y0, gw0, gb0, fw0, fb0)]
        x, y, gw, gb, fw, fb = leaves
        assert ops.fused_ddpm_supported(x, y, gw, gb, fw, fb, k, DIL)
        if fused:
            out = ops.fused_ddpm(x, y, gw, gb, fw, fb, k, DIL)
        else:
            out = ops.fuse_conv3x3(ops.fused_generator_dynamic_cat(x, y, gw, gb, k, DIL), fw, fb)
        grads = torch.autograd.grad(out, leaves, gout)
        torch.cuda.synchronize()
        runs.append((out.detach(), grads))
    (o_sep, g_sep), (o_fused, g_fused) = runs
    if dtype == torch.float32:
        scale = o_sep.abs().max().item()
        assert_close(o_fused, o_sep, FP32_CONV_TOL * scale, FP32_CONV_TOL, f"out {shape}")
    else:
        assert torch.equal(o_fused, o_sep), f"out {shape} {dtype}"
    names = ("dx", "dy", "d gen weight", "d gen bias", "d fuse weight", "d fuse bias")
    for name, a, e in zip(names, g_fused, g_sep):
        assert torch.equal(a, e), f"{name} {shape}: max|diff| {(a - e).abs().max().item():.3e}"

    # inference (no autograd graph) gives the training forward's output
    with torch.no_grad():
        args = [t.to(DEV) for t in (x0, y0, gw0, gb0, fw0, fb0)]
        o_inf = ops.fused_ddpm(*args, k, DIL)
    assert torch.equal(o_inf, o_fused)


def test_fused_ddpm_partial_gradients():
    """Only the fuse convolution's parameters, or only x, require grad."""
    say("fused_ddpm partial gradients")
    shape, k = (1, 16, 24, 32), 3
    c = shape[1]
    x0, y0 = randn(shape, 1800).to(DEV), randn(shape, 1801).to(DEV)
    gw0, gb0 = (t.to(DEV) for t in default_generator_params(c, k, 1802, torch.float32))
    torch.manual_seed(1803)
    conv = torch.nn.Conv2d(4 * c, c, 3, 1, 1).to(DEV)
    fw0, fb0 = conv.weight.detach(), conv.bias.detach()
    gout = randn(shape, 1804).to(DEV)
    full = [t.clone().requires_grad_() for t in (x0, y0, gw0, gb0, fw0, fb0)]
    all_grads = torch.autograd.grad(ops.fused_ddpm(*full, k, DIL), full, gout)
    for want in ((4, 5), (0,)):
        leaves = [t.clone().requires_grad_(i in want) for i, t in enumerate((x0, y0, gw0, gb0, fw0, fb0))]
        out = ops.fused_ddpm(*leaves, k, DIL)
        got = torch.autograd.grad(out, [leaves[i] for i in want], gout)
        for i, gr in zip(want, got):
            assert torch.equal(gr, all_grads[i]), f"leaf {i}"


@pytest.mark.parametrize("shape", [(1, 64, 256, 256), (2, 16, 20, 36), (1, 48, 15, 17)])
def test_fuse_conv_combined_backward_reads_pair_planes(shape):
    """ddpm_fuse_conv_bwd with a pair-plane concat (dtype 3; grad_out and
    weight plain fp32): bit-identical to ddpm_fuse_conv_bwd_data plus
    ddpm_fuse_conv_bwd_weight on the plain fp32 concat."""
    from tests.test_gpu_fuse_conv import _fuse_conv_bwd_calls

    say(f"fuse conv combined backward pair planes shape={shape}")
    n, c, h, w = shape
    seed = 1700 + c + w
    cat = randn((n, 4 * c, h, w), seed)
    torch.manual_seed(seed + 1)
    wt = torch.nn.Conv2d(4 * c, c, 3, 1, 1).weight.detach().float().to(DEV)
    g = randn((n, c, h, w), seed + 2).to(DEV)
    sep = _fuse_conv_bwd_calls(cat.to(DEV), wt, g, 0, False)
    com = _fuse_conv_bwd_calls(_as_device_words(_pair_planes(cat)), wt, g, PAIRS, True)
    for name, a, e in zip(("d cat", "d weight", "d bias"), com, sep):
        assert not torch.isnan(e).any(), f"{name} {shape}"
        assert torch.equal(a, e), f"{name} {shape}: max|diff| {(a - e).abs().max().item():.3e}"


def _gen_fwd_conv(x, y, gw, gb, fw, fb, k, code, packed):
    """The concat and the fuse convolution's output through the C-ABI:
    ddpm_gen_fwd + ddpm_fuse_conv_fwd, or ddpm_gen_fwd_pack +
    ddpm_fuse_conv_fwd_packed (outputs and workspace started as NaN / 0xff)."""
    lib = _lib.load()
    n, c, h, w = x.shape
    cat = torch.full((n, 4 * c, h, w), float("nan"), dtype=x.dtype, device=DEV)
    out = torch.full((n, c, h, w), float("nan"), dtype=x.dtype, device=DEV)
    nb = int(lib.ddpm_fuse_conv_workspace_bytes(n, c, h, w, code))
    ws = torch.full((max(nb, 16),), 255, dtype=torch.uint8, device=DEV)
    if packed:
        rc = lib.ddpm_gen_fwd_pack(_ptr(x), _ptr(y), _ptr(gw), _ptr(gb), _ptr(cat), _ptr(fw), _ptr(ws), nb,
                                   n, c, h, w, k, *DIL, code, _stream())
        assert rc == 0, rc
        rc = lib.ddpm_fuse_conv_fwd_packed(_ptr(cat), _ptr(fb), _ptr(out), _ptr(ws), nb, n, c, h, w, code,
                                           _stream())
        assert rc == 0, rc
    else:
        rc = lib.ddpm_gen_fwd(_ptr(x), _ptr(y), _ptr(gw), _ptr(gb), _ptr(cat), n, c, h, w, k, *DIL, code,
                              _stream())
        assert rc == 0, rc
        rc = lib.ddpm_fuse_conv_fwd(_ptr(cat), _ptr(fw), _ptr(fb), _ptr(out), _ptr(ws), nb, n, c, h, w, code,
                                    _stream())
        assert rc == 0, rc
    torch.cuda.synchronize()
    return cat, out


@pytest.mark.parametrize("code", [0, 1, 2, PAIRS])
@pytest.mark.parametrize("shape,k", [((1, 64, 256, 256), 3), ((1, 64, 128, 128), 3), ((2, 16, 20, 36), 3),
                                     ((1, 48, 15, 17), 1), ((1, 32, 40, 56), 5), ((1, 128, 32, 64), 3)])
def test_gen_fwd_pack_is_gen_fwd_then_fuse_conv_fwd(shape, k, code):
    """ddpm_gen_fwd_pack (the generator's workgroups packing the fuse
    convolution's weight) + ddpm_fuse_conv_fwd_packed: concat and output bit
    for bit those of ddpm_gen_fwd + ddpm_fuse_conv_fwd, in every dtype code
    (2-byte K = 3 at C <= 64: the tap-pair generator kernel), with the 128x128
    forward's input-plane splits, element-wise rows and C = 128."""
    n, c, h, w = shape
    if code == PAIRS and c % 16 != 0:
        pytest.skip("pair planes need C % 16 == 0")
    say(f"gen_fwd_pack shape={shape} k={k} code={code}")
    dt = {0: torch.float32, 1: torch.bfloat16, 2: torch.float16, PAIRS: torch.float32}[code]
    x = randn(shape, 1800 + c + w)
    y = randn(shape, 1801 + c + w)
    gw, gb = default_generator_params(c, k, 1802 + c, torch.float32)
    torch.manual_seed(1803 + c)
    conv = torch.nn.Conv2d(4 * c, c, 3, 1, 1)
    x, y, gw, gb, fw, fb = (t.detach().to(dt).to(DEV).contiguous()
                            for t in (x, y, gw, gb, conv.weight, conv.bias))
    a = _gen_fwd_conv(x, y, gw, gb, fw, fb, k, code, False)
    b = _gen_fwd_conv(x, y, gw, gb, fw, fb, k, code, True)
    for name, u, v in zip(("concat", "out"), b, a):
        if code == PAIRS and name == "concat":
            u, v = _words(u), _words(v)
        else:
            assert not torch.isnan(v).any(), f"{name} {shape}"
        assert torch.equal(u, v), f"{name} {shape} k={k} code={code}"
