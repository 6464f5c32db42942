"""Host-side tests (no GPU): the C-ABI library loads and exports every symbol
declared in include/ddpm_hip.h, argument validation needs no device, the
routing rules mirror the reference's (triton_impl.py:311-329), and GPU
tensors never fall back to the CPU branch."""

import os
import re

import pytest
import torch

import dynamicconvolutionoperator_amd as dco
from dynamicconvolutionoperator_amd import _lib, module

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_symbols():
    text = open(os.path.join(ROOT, "include", "ddpm_hip.h")).read()
    return sorted(set(re.findall(r"^\w[\w\s\*]*?\b(ddpm_\w+)\s*\(", text, re.M)))


def test_header_declares_the_bound_symbols():
    assert _declared_symbols() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _declared_symbols():
        assert hasattr(lib, name), name


def test_host_only_queries():
    lib = _lib.load()
    assert lib.ddpm_abi_version() == _lib.ABI_VERSION == 7
    assert b"invalid argument" in lib.ddpm_status_string(10001)
    assert lib.ddpm_gen_supported(64, 3, 5) == 1
    # up to 128 channels (four 32-channel K steps, 32-column tiles above 64)
    assert lib.ddpm_gen_supported(65, 3, 5) == 1
    assert lib.ddpm_gen_supported(128, 3, 5) == 1
    assert lib.ddpm_gen_supported(128, 3, 8) == 1
    assert lib.ddpm_gen_supported(129, 3, 5) == 0
    assert lib.ddpm_gen_supported(129, 1, 1) == 0
    assert lib.ddpm_gen_supported(64, 5, 5) == 0
    # the backward kernels stage a column halo of 8 pixels; 1x1 taps ignore dilation
    assert lib.ddpm_gen_supported(64, 3, 8) == 1
    assert lib.ddpm_gen_supported(64, 3, 9) == 0
    assert lib.ddpm_gen_supported(64, 1, 50) == 1
    # the forward alone (inference): K = 5, and larger halos, as far as the
    # LDS holds the halo tile of a 32-column tile
    assert lib.ddpm_gen_fwd_supported(64, 3, 5) == 1
    assert lib.ddpm_gen_fwd_supported(64, 5, 5) == 1
    assert lib.ddpm_gen_fwd_supported(128, 5, 5) == 1
    assert lib.ddpm_gen_fwd_supported(64, 5, 6) == 1
    assert lib.ddpm_gen_fwd_supported(64, 5, 7) == 0
    assert lib.ddpm_gen_fwd_supported(64, 3, 9) == 1
    assert lib.ddpm_gen_fwd_supported(64, 3, 12) == 1
    assert lib.ddpm_gen_fwd_supported(64, 3, 13) == 0
    assert lib.ddpm_gen_fwd_supported(64, 7, 1) == 0
    assert lib.ddpm_gen_fwd_supported(129, 5, 5) == 0
    assert lib.ddpm_gen_fwd_supported(64, 1, 50) == 1
    # at most 16 splits of 27 (branch, tap) x C x (C + 1) fp32 partials, at least
    # 4 steps (row segments of 128 columns) each: 16 at 256x256; the same
    # for every dtype (fp32 y is split into bf16 hi / lo while it is staged)
    ysplit = lambda n, c, h, w: n * c * h * w * 4  # noqa: E731  (generator GEMM's y planes)
    part = 16 * 27 * 64 * 65 * 4
    assert lib.ddpm_gen_bwd_w_workspace_bytes(1, 64, 256, 256, 3, 0) == part
    assert lib.ddpm_gen_bwd_w_workspace_bytes(1, 64, 256, 256, 3, 1) == part
    assert lib.ddpm_gen_bwd_w_workspace_bytes(1, 64, 256, 256, 3, 7) == 0  # invalid dtype
    # 30 steps at 4 per split: 8 splits
    assert lib.ddpm_gen_bwd_w_workspace_bytes(2, 24, 15, 17, 3, 0) == 8 * 27 * 24 * 25 * 4
    # 4 steps or fewer: one split writes the gradients directly
    assert lib.ddpm_gen_bwd_w_workspace_bytes(1, 24, 4, 17, 3, 0) == 0
    assert lib.ddpm_gen_bwd_w_workspace_bytes(1, 24, 4, 17, 3, 2) == 0
    # dX partials: 16x64 tiles (4 x 16 of them) x 4 channel blocks x 16 channels x
    # the 16+2R rows of the halo tile, R = 5, each padded from 64+2R = 74 columns
    # (shifted by 3 so that tile columns sit 16-byte aligned) to 80 ...
    assert lib.ddpm_gen_bwd_x_workspace_bytes(1, 64, 256, 256, 3, 1, 3, 5) == 64 * 4 * 16 * 26 * 80 * 4
    # ... and 16x32 tiles when the R = 8 accumulator tile does not fit the LDS
    assert lib.ddpm_gen_bwd_x_workspace_bytes(1, 64, 256, 256, 3, 1, 3, 8) == 128 * 4 * 16 * 32 * 48 * 4
    assert lib.ddpm_gen_bwd_x_workspace_bytes(1, 64, 256, 256, 5, 1, 3, 5) == 0  # unsupported
    # above 64 channels always 16x32 tiles (8 x 16 of them), 8 channel blocks; R = 5:
    # 32+2R = 42 columns padded (shift 3) to 48
    assert lib.ddpm_gen_bwd_x_workspace_bytes(1, 128, 256, 256, 3, 1, 3, 5) == 128 * 8 * 16 * 26 * 48 * 4
    assert lib.ddpm_gen_bwd_x_workspace_bytes(1, 129, 256, 256, 3, 1, 3, 5) == 0  # unsupported
    # dY's packed weight: [output-channel halves][3 branches][32-channel chunks][K*K]
    # [16-channel blocks per half][hi, lo][64 lanes] x 16 bytes
    assert lib.ddpm_gen_bwd_y_workspace_bytes(64, 3) == 1 * 3 * 2 * 9 * 4 * 2 * 64 * 16
    assert lib.ddpm_gen_bwd_y_workspace_bytes(96, 3) == 2 * 3 * 3 * 9 * 4 * 2 * 64 * 16
    assert lib.ddpm_gen_bwd_y_workspace_bytes(128, 3) == 2 * 3 * 4 * 9 * 4 * 2 * 64 * 16
    assert lib.ddpm_gen_bwd_y_workspace_bytes(129, 3) == 0
    # the weight gradient at 128 channels: the same 16 splits of C x (C + 1) partials
    assert lib.ddpm_gen_bwd_w_workspace_bytes(1, 128, 256, 256, 3, 1) == 16 * 27 * 128 * 129 * 4
    # generator convolution weight gradient at 128x128, C = 64, K = 5: 4800 rows in
    # 75 tiles of 64, 6 splits (450 workgroups for 512 slots) of (4800 x 64 + 4800)
    # fp32 partials, then the bf16 hi / lo planes of an fp32 y
    assert lib.ddpm_gen_kernels_bwd_w_workspace_bytes(1, 64, 128, 128, 5) == (
        6 * (4800 * 64 + 4800) * 4 + ysplit(1, 64, 128, 128))
    # 32x32: 16 steps of 64 pixels at 8 per workgroup give the most partials (2 splits)
    assert lib.ddpm_gen_kernels_bwd_w_workspace_bytes(1, 64, 32, 32, 5) == (
        2 * (4800 * 64 + 4800) * 4 + ysplit(1, 64, 32, 32))
    # 8 steps of 32 pixels (4x64) or fewer: one split, no partials
    assert lib.ddpm_gen_kernels_bwd_w_workspace_bytes(1, 64, 4, 64, 5) == ysplit(1, 64, 4, 64)
    assert lib.ddpm_gen_kernels_bwd_w_workspace_bytes(1, 129, 32, 32, 5) == 0  # unsupported
    # its input gradient: 150 chunks of 32 rows packed as fp32 hi / lo fragments
    # (2 KB per chunk and 16-channel block), then 4 o splits of fp32 dY partials
    # (128 pixel tiles x 4 = 512 workgroups)
    assert lib.ddpm_gen_kernels_bwd_y_workspace_bytes(1, 64, 128, 128, 5) == (
        150 * 4 * 2 * 1024 + 4 * 64 * 128 * 128 * 4)


def test_entry_points_validate_arguments_before_touching_the_device():
    lib = _lib.load()
    null = None
    # even kernel size / bad dtype / null pointers are rejected host-side
    assert lib.ddpm_filter_fwd(null, null, null, 1, 1, 4, 4, 2, 1, 3, 5, 0, 0, null) == 10001
    assert lib.ddpm_filter_fwd(null, null, null, 1, 1, 4, 4, 3, 1, 3, 5, 7, 0, null) == 10001
    assert lib.ddpm_filter_fwd(null, null, null, 1, 1, 4, 4, 3, 1, 3, 5, 0, 0, null) == 10001
    assert lib.ddpm_gen_fwd(null, null, null, null, null, 1, 129, 4, 4, 3, 1, 3, 5, 0, null) == 10002
    assert lib.ddpm_gen_fwd(null, null, null, null, null, 1, 128, 4, 4, 3, 1, 3, 5, 0, null) == 10001
    assert lib.ddpm_gen_bwd_w(null, null, null, null, null, null, 0, 1, 64, 256, 256, 3, 1, 3, 5, 0, null) != 0
    # the generator 1x1 convolution: even kernel size, more than 128 channels
    assert lib.ddpm_gen_kernels(null, null, null, null, 1, 64, 8, 8, 4, 1, null) == 10001
    assert lib.ddpm_gen_kernels(null, null, null, null, 1, 129, 8, 8, 5, 1, null) == 10002
    assert lib.ddpm_gen_kernels(null, null, null, null, 1, 64, 8, 8, 5, 1, null) == 10001
    # its weight gradient: even kernel size, more than 128 channels, null outputs
    assert lib.ddpm_gen_kernels_bwd_w(null, null, null, null, null, 0, 1, 64, 8, 8, 4, 1, null) == 10001
    assert lib.ddpm_gen_kernels_bwd_w(null, null, null, null, null, 0, 1, 129, 8, 8, 5, 1, null) == 10002
    assert lib.ddpm_gen_kernels_bwd_w(null, null, null, null, null, 0, 1, 64, 8, 8, 5, 1, null) == 10001
    assert lib.ddpm_gen_kernels_bwd_y(null, null, null, null, 0, 1, 64, 8, 8, 4, 1, null) == 10001
    assert lib.ddpm_gen_kernels_bwd_y(null, null, null, null, 0, 1, 129, 8, 8, 5, 1, null) == 10002
    assert lib.ddpm_gen_kernels_bwd_y(null, null, null, null, 0, 0, 64, 8, 8, 5, 1, null) == 0
    # empty tensors are a no-op
    assert lib.ddpm_filter_fwd(null, null, null, 0, 4, 4, 4, 3, 1, 3, 5, 0, 0, null) == 0
    assert lib.ddpm_gen_kernels(null, null, null, null, 0, 64, 8, 8, 5, 1, null) == 0
    # dtype code 3 (fp32 pair-plane concat): whole 32-plane chunks only, and
    # only where an entry point documents it
    assert lib.ddpm_gen_fwd(null, null, null, null, null, 1, 24, 4, 4, 3, 1, 3, 5, 3, null) == 10002
    assert lib.ddpm_gen_fwd(null, null, null, null, null, 1, 32, 4, 4, 3, 1, 3, 5, 3, null) == 10001
    assert lib.ddpm_fuse_conv_fwd(null, null, null, null, null, 0, 1, 12, 4, 4, 3, null) == 10002
    assert lib.ddpm_fuse_conv_bwd_weight(null, null, null, null, null, 0, 1, 12, 4, 4, 3, null) == 10002
    assert lib.ddpm_fuse_conv_workspace_bytes(1, 64, 32, 32, 3) == lib.ddpm_fuse_conv_workspace_bytes(1, 64, 32, 32, 0)
    assert lib.ddpm_filter_fwd(null, null, null, 1, 1, 4, 4, 3, 1, 3, 5, 3, 3, null) == 10001


def test_fused_ddpm_takes_rocm_tensors_of_one_dtype_only():
    """ops.fused_ddpm (the module's fused route with the HIP fuse
    convolution) is refused for CPU tensors and mixed dtypes; the module's
    CPU branch never reaches it."""
    from dynamicconvolutionoperator_amd import ops

    c, k = 16, 3
    x = torch.randn(1, c, 8, 8)
    gw, gb = torch.randn(3 * c * k * k, c, 1, 1), torch.randn(3 * c * k * k)
    fw, fb = torch.randn(c, 4 * c, 3, 3), torch.randn(c)
    assert not ops.fused_ddpm_supported(x, x, gw, gb, fw, fb, k, (1, 3, 5))
    assert not ops.fused_ddpm_supported(x.bfloat16(), x.bfloat16(), gw, gb, fw, fb, k, (1, 3, 5))
    with pytest.raises(ValueError):
        ops.fused_ddpm(x, x, gw, gb, fw, fb, k, (1, 3, 5))
    m = module.DDPM(c, k)
    assert m(x, x).shape == x.shape


class _FakeTensor:
    def __init__(self, shape, dtype=torch.float32):
        self.shape = shape
        self.dtype = dtype
        self.device = torch.device("cpu")


@pytest.mark.parametrize(
    "tokens_shape, dtype, k, flag, grad, autocast, expect",
    [
        ((1, 64, 256, 256), torch.float32, 3, None, True, False, "fused"),  # > 16384 tokens
        ((1, 64, 128, 128), torch.float32, 3, None, True, False, "fused"),  # == 16384, fp32
        ((1, 64, 128, 128), torch.bfloat16, 3, None, True, False, "materialized"),  # == 16384 bf16
        ((1, 64, 64, 64), torch.float32, 3, None, True, False, "materialized"),  # small, training
        ((1, 64, 64, 64), torch.float32, 3, None, False, False, "fused"),  # inference
        ((1, 64, 64, 64), torch.float32, 3, True, True, False, "fused"),  # forced fused
        ((1, 64, 256, 256), torch.float32, 3, False, True, False, "materialized"),  # forced off
        ((1, 64, 256, 256), torch.float32, 5, True, True, False, "materialized"),  # K > 3
        ((1, 64, 256, 256), torch.float32, 5, None, False, False, "fused"),  # K = 5 inference
        ((1, 64, 256, 256), torch.float32, 7, None, False, False, "materialized"),  # K = 7 inference
        ((1, 64, 256, 256), torch.float32, 3, None, False, True, "materialized"),  # autocast
    ],
)
def test_routing_rules(monkeypatch, tokens_shape, dtype, k, flag, grad, autocast, expect):
    c = tokens_shape[1]
    m = module.DDPM(c, k, fused_generator_training=flag).to(dtype)
    x = _FakeTensor(tokens_shape, dtype)
    monkeypatch.setattr(torch, "is_autocast_enabled", lambda *a, **k: autocast)

    def supported(ch, ks, dil, *shape_dtype, forward_only=False):
        return ch <= 64 and (ks <= 3 or (forward_only and ks == 5))

    with torch.set_grad_enabled(grad):
        assert m._route(x, x, supported) == expect


def test_routing_dtype_mismatch_materializes():
    m = module.DDPM(8, 3)  # fp32 parameters
    x = _FakeTensor((1, 8, 64, 64), torch.bfloat16)
    with torch.no_grad():
        assert m._route(x, x, lambda *a, **k: True) == "materialized"


def test_routing_respects_the_fused_kernels_offset_bound():
    """One image's planes past 2^31 - 1 bytes take the materialized route
    instead of failing inside the fused kernels (ops.generator_supported)."""
    from dynamicconvolutionoperator_amd import ops

    m = module.DDPM(64, 3, fused_generator_training=True)
    small = _FakeTensor((1, 64, 256, 256))
    huge = _FakeTensor((1, 64, 2900, 2900))  # 64 x 2900^2 x 4 B = 2.15 GB per image
    with torch.no_grad():
        assert m._route(small, small, ops.generator_supported) == "fused"
        assert m._route(huge, huge, ops.generator_supported) == "materialized"
    # in bf16 the same image is half the bytes and stays fused
    assert ops.generator_supported(64, 3, (1, 3, 5), huge.shape, torch.bfloat16)


class _FakeParam:
    def __init__(self, shape, dtype=torch.float32):
        self.shape = shape
        self.dtype = dtype


@pytest.mark.parametrize(
    "c, k, hw, dtype, expect",
    [
        (64, 5, 128, torch.float32, True),
        (64, 5, 384, torch.float32, False),  # 4800 planes x 384^2 x 4 B = 2.83 GB per image
        (64, 5, 384, torch.bfloat16, True),  # 1.42 GB
        (128, 3, 512, torch.float32, False),  # 3456 x 512^2 x 4 B = 3.6 GB
        (128, 5, 256, torch.float32, False),
        (129, 3, 32, torch.float32, False),  # more than 128 channels
    ],
)
def test_generator_kernels_supported_bounds(c, k, hw, dtype, expect):
    from dynamicconvolutionoperator_amd import ops

    o = 3 * c * k * k
    y = _FakeTensor((1, c, hw, hw), dtype)
    y.ndim = 4
    assert ops.generator_kernels_supported(y, _FakeParam((o, c, 1, 1), dtype),
                                           _FakeParam((o,), dtype)) is expect


def test_gpu_tensors_fail_loudly_without_the_library(monkeypatch):
    """A missing library must raise for device tensors, never fall back."""

    def missing():
        raise _lib.HipLibraryError("libddpm_hip.so is not built")

    monkeypatch.setattr(module, "_load_hip_ops", missing)
    m = module.DDPM(4, 3)

    x = torch.randn(1, 4, 5, 5)
    # DDPM.forward routes on x.is_cuda; emulate a device tensor's routing
    monkeypatch.setattr(torch.Tensor, "is_cuda", property(lambda self: True))
    with pytest.raises(_lib.HipLibraryError):
        m(x, x.clone())


def test_public_api_names():
    for name in ("DDPM", "fused_dynamic_cat", "fused_generator_dynamic_cat"):
        assert hasattr(dco, name)


def test_plain_conv_guard():
    """The HIP kernels stand in for self.fuse / self.generator only while they
    are the constructor's plain convolutions without hooks; otherwise the
    module calls them, as the reference does (triton_impl.py:340-347, 392)."""
    import warnings

    from torch import nn
    from torch.nn.utils import parametrizations

    m = module.DDPM(8, 3)
    assert m._hip_fuse() and module.plain_conv(m.generator, 1)
    m.fuse_conv_backend = "library"
    assert not m._hip_fuse()
    m.fuse_conv_backend = "hip"
    # attributes of the convolution
    for kwargs in ({"padding": 1, "padding_mode": "reflect"}, {"padding": 1, "padding_mode": "circular"},
                   {"padding": 2, "dilation": 2}, {"padding": 1, "stride": 2},
                   {"padding": 1, "groups": 4}, {"padding": 0}, {"padding": "same"}):
        m.fuse = nn.Conv2d(32, 8, 3, **kwargs)
        assert not m._hip_fuse(), kwargs
    m.fuse = nn.Conv2d(32, 8, 3, 1, 1)
    assert m._hip_fuse()
    # hooks on the module
    h = m.fuse.register_forward_hook(lambda *a: None)
    assert not m._hip_fuse()
    h.remove()
    h = m.fuse.register_forward_pre_hook(lambda *a: None)
    assert not m._hip_fuse()
    h.remove()
    h = m.fuse.register_full_backward_hook(lambda *a: None)
    assert not m._hip_fuse()
    h.remove()
    assert m._hip_fuse()
    # global module hooks
    h = nn.modules.module.register_module_forward_hook(lambda *a: None)
    try:
        assert not m._hip_fuse()
    finally:
        h.remove()
    # weight_norm: the old API is a forward pre-hook, the parametrization is not
    with warnings.catch_warnings():
        warnings.simplefilter("ignore", FutureWarning)
        torch.nn.utils.weight_norm(m.fuse)
    assert not m._hip_fuse()
    m.fuse = parametrizations.weight_norm(nn.Conv2d(32, 8, 3, 1, 1))
    assert m._hip_fuse()

    # a subclass with its own forward, or another module entirely
    class Scaled(nn.Conv2d):
        def forward(self, t):
            return super().forward(t) * 2

    m.fuse = Scaled(32, 8, 3, 1, 1)
    assert not m._hip_fuse()
    m.fuse = nn.Sequential(nn.Conv2d(32, 8, 3, 1, 1))
    assert not m._hip_fuse()
    # the generator on the materialized route
    m.generator.register_forward_hook(lambda *a: None)
    assert not module.plain_conv(m.generator, 1)
    assert not module.plain_conv(nn.Conv2d(8, 216, 3, padding=1), 1)
    assert module.plain_conv(nn.Conv2d(8, 216, 1), 1)


def test_bench_prices_every_step_entry_point():
    """bench.py's roofline can pick any fused-route entry point the training
    step calls: each has its algorithmic bytes and flops (the materialized
    route's are priced only where bench times them alone)."""
    import sys

    sys.path.insert(0, ROOT)
    import bench

    step = [n for n in bench.timed_entry_points(_lib.SIGNATURES)
            if not n.startswith(("ddpm_gen_kernels", "ddpm_gen_bwd_y_noalloc"))]
    assert "ddpm_fuse_conv_bwd" in step and "ddpm_gen_fwd_pack" in step
    for name in step:
        nbytes, flops = bench.work_per_launch(name, 4)
        assert nbytes > 0, name
