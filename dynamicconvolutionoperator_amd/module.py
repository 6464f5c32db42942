"""Drop-in ``DDPM`` module (Dynamic Dilated Pyramid Module, HDFNet ECCV 2020).

Same constructor, attributes, parameter order, state-dict keys, input checks,
error messages and routing as the reference's module (triton_impl.py:247-392),
with the GPU route backed by HIP kernels for gfx950:

* ROCm ("cuda") tensors -> :meth:`DDPM._cuda_cat`, which picks the fused
  generator route (generator + filter + concat in one kernel; recompute
  backward) or the materialized route (1x1 generator conv, then the HIP
  dynamic filter) with the reference's rules (triton_impl.py:311-348).
  If the HIP library is missing it raises instead of falling back.
* CPU tensors -> the reference's CPU branch (triton_impl.py:353-391).

The final 3x3 ``fuse`` convolution is a plain ``nn.Conv2d`` (its parameters and
state-dict keys are the reference's); on ROCm tensors its forward and
gradients run as HIP MFMA kernels while ``self.fuse`` is that convolution
unmodified (3x3, stride 1, zero padding 1, no dilation or groups, no hooks);
anything else -- hooks such as the old ``weight_norm`` / ``spectral_norm``,
another ``padding_mode``, a replaced module -- is honoured by calling
``self.fuse(cat)`` as the reference always does (triton_impl.py:392).
``fuse_conv_backend = "library"`` selects MIOpen through ``self.fuse`` always.
The materialized route likewise calls ``self.generator(y)`` unless the
generator is the constructor's unmodified 1x1 convolution
(triton_impl.py:340-347).  On the fused route with the HIP fuse
convolution, generator, filter, concat and fuse convolution run as one pair
of autograd ops (``ops.fused_ddpm``) whose generator launch also packs the
fuse weight; an fp32 concat (C % 16 == 0) is stored as bf16 pair planes,
already split the way the fuse convolution's fp32 MFMA products need it.
"""

from __future__ import annotations

import functools

import torch
from torch import nn
from torch.nn.modules import module as _torch_module

from . import _cpu

_DEFAULT_DILATIONS = (1, 3, 5)


@functools.lru_cache(maxsize=1)
def _load_hip_ops():
    """Lazily bind the HIP operators (counterpart of triton_impl.py:23-33).

    Unlike the reference, a missing library is an error for GPU tensors, not
    a silent fallback: HipLibraryError propagates to the caller.
    """
    from . import _lib, ops

    _lib.load()
    return (ops.fused_dynamic_cat, ops.fused_generator_dynamic_cat, ops.generator_supported,
            ops._generate, ops.fuse_conv3x3, ops._fused_ddpm_checked, ops.fused_ddpm_supported)


def _module_hooks_set(m: nn.Module) -> bool:
    """Whether calling ``m`` would run a hook: its own forward / backward
    hooks or the global module hooks."""
    g = _torch_module
    return bool(
        m._forward_hooks or m._forward_pre_hooks or m._backward_hooks or m._backward_pre_hooks
        or g._global_forward_hooks or g._global_forward_pre_hooks
        or g._global_backward_hooks or g._global_backward_pre_hooks
    )


def plain_conv(m: nn.Module, kernel_size: int) -> bool:
    """Whether ``m`` computes exactly ``F.conv2d(t, m.weight, m.bias,
    padding=kernel_size // 2)``, so a kernel may run that convolution from
    ``m.weight`` / ``m.bias`` in place of calling ``m``: an ``nn.Conv2d``
    whose forward is Conv2d's own (parametrized weights, as from
    ``torch.nn.utils.parametrizations``, qualify: ``m.weight`` evaluates
    them), a square ``kernel_size`` kernel, stride 1, zero padding of
    ``kernel_size // 2``, no dilation or groups, and no hooks."""
    if not isinstance(m, nn.Conv2d) or m.transposed:
        return False
    cls = type(m)
    if cls.forward is not nn.Conv2d.forward or cls._conv_forward is not nn.Conv2d._conv_forward:
        return False
    pad = kernel_size // 2
    if (m.kernel_size != (kernel_size, kernel_size) or m.stride != (1, 1)
            or m.padding != (pad, pad) or m.dilation != (1, 1) or m.groups != 1
            or m.padding_mode != "zeros"):
        return False
    return not _module_hooks_set(m)


def _check_inputs(x: torch.Tensor, y: torch.Tensor, channels: int) -> None:
    if x.ndim != 4 or y.ndim != 4:
        raise ValueError(f"x and y must be NCHW tensors, got {x.shape=} and {y.shape=}")
    if x.shape != y.shape:
        raise ValueError(f"x and y must have identical shapes, got {x.shape=} and {y.shape=}")
    if x.shape[1] != channels:
        raise ValueError(f"expected {channels} channels, got {x.shape[1]}")
    if x.device != y.device:
        raise ValueError(f"x and y must be on the same device, got {x.device} and {y.device}")


class DDPM(nn.Module):
    """Dynamic Dilated Pyramid Module with HIP fast paths.

    Args:
        dim: Input/output channel count.
        kernel_size: Odd dynamic depthwise kernel size.
        spatial_tile_size: CPU streaming tile in pixels (``0`` = all pixels).
        max_generated_bytes: CPU only - materialize the dynamic kernels while
            they fit this byte budget, else stream tiles (``0`` = always stream).
        recompute: CPU streaming - recompute generated tiles in backward.
        fused_generator_inference: fuse generator + filter when gradients are
            disabled.
        fused_generator_training: recompute-based fused training for K <= 3.
            ``None`` fuses above 16384 spatial tokens and at exactly 16384 for
            FP32; ``True`` always; ``False`` never.
    """

    def __init__(
        self,
        dim: int,
        kernel_size: int = 3,
        *,
        spatial_tile_size: int = 4096,
        max_generated_bytes: int = 256 * 1024**2,
        recompute: bool = True,
        fused_generator_inference: bool = True,
        fused_generator_training: bool | None = None,
    ) -> None:
        super().__init__()
        if kernel_size < 1 or kernel_size % 2 == 0:
            raise ValueError(f"kernel_size must be a positive odd integer, got {kernel_size}")
        if dim < 1:
            raise ValueError(f"dim must be positive, got {dim}")
        self.dim = dim
        self.kernel_size = kernel_size
        self.spatial_tile_size = spatial_tile_size
        self.max_generated_bytes = max_generated_bytes
        self.recompute = recompute
        self.fused_generator_inference = fused_generator_inference
        self.fused_generator_training = fused_generator_training
        self.dilations = _DEFAULT_DILATIONS
        # the 3x3 fuse convolution on ROCm tensors: "hip" runs it as this
        # library's MFMA kernels (same Conv2d parameters), "library" calls
        # self.fuse (MIOpen), as the reference calls cuDNN
        self.fuse_conv_backend = "hip"
        # creation order (generator, then fuse) fixes the seeded default init
        self.generator = nn.Conv2d(dim, 3 * dim * kernel_size**2, 1)
        self.fuse = nn.Conv2d(4 * dim, dim, 3, 1, 1)
        self._cpu_unfolds = nn.ModuleList(
            nn.Unfold(kernel_size, d, padding=kernel_size // 2 * d, stride=1) for d in self.dilations
        )

    # ------------------------------------------------------------------ GPU
    def _route(self, x: torch.Tensor, y: torch.Tensor, gen_supported) -> str:
        """Returns "fused" or "materialized" with the reference's rules
        (triton_impl.py:311-329); shapes outside the fused kernels' coverage
        (``ops.generator_supported``: the forward's alone without grad, where
        K = 5 is fused as the reference fuses inference at any K) use the
        materialized route."""
        tokens = x.shape[0] * x.shape[2] * x.shape[3]
        requested = self.fused_generator_training
        if requested is None:
            requested = tokens > 16384 or (tokens == 16384 and x.dtype == torch.float32)
        grad = torch.is_grad_enabled()
        fuse_training = grad and requested and self.kernel_size <= 3
        bias = self.generator.bias
        can_fuse = (
            (self.fused_generator_inference or fuse_training)
            and (not grad or fuse_training)
            and not torch.is_autocast_enabled(x.device.type)
            and x.dtype == y.dtype == self.generator.weight.dtype
            and bias is not None
            and bias.dtype == x.dtype
            and gen_supported(self.dim, self.kernel_size, self.dilations, x.shape, x.dtype,
                              forward_only=not grad)
        )
        return "fused" if can_fuse else "materialized"

    def _cuda_cat(self, x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
        fused_dynamic_cat, fused_generator_dynamic_cat, gen_supported, generate = _load_hip_ops()[:4]
        if self._route(x, y, gen_supported) == "fused":
            return fused_generator_dynamic_cat(
                x, y, self.generator.weight, self.generator.bias, self.kernel_size, self.dilations
            )
        # the generator 1x1 convolution: the HIP MFMA kernel where it applies;
        # under autocast the Conv2d runs in the autocast dtype, as the
        # reference's does (the filter's output dtype follows the kernels')
        if torch.is_autocast_enabled(y.device.type) or not plain_conv(self.generator, 1):
            kernels = self.generator(y)
        else:
            kernels = generate(y, self.generator.weight, self.generator.bias, self.kernel_size)
        kernels = kernels.reshape(
            x.shape[0], len(self.dilations), self.dim, self.kernel_size**2, x.shape[2], x.shape[3]
        )
        return fused_dynamic_cat(x, kernels, self.kernel_size, self.dilations)

    # ------------------------------------------------------------------ CPU
    def _cpu_cat(self, x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
        generated_bytes = (
            x.shape[0] * len(self.dilations) * self.dim * self.kernel_size**2
            * x.shape[2] * x.shape[3] * x.element_size()
        )
        if 0 < generated_bytes <= self.max_generated_bytes:
            kernels = self.generator(y).reshape(
                x.shape[0], len(self.dilations), self.dim, self.kernel_size**2, x.shape[2], x.shape[3]
            )
            if self.training and torch.is_grad_enabled():
                return _cpu.cpu_training_dynamic_cat(x, kernels, self.kernel_size, self._cpu_unfolds)
            return _cpu.native_dynamic_cat(x, kernels, self.kernel_size, self.dilations)
        return _cpu.streaming_generator_dynamic_cat(
            x,
            y,
            self.generator.weight,
            self.generator.bias,
            self.kernel_size,
            self.dilations,
            self.spatial_tile_size,
            self.recompute and self.training,
        )

    def _hip_fuse(self) -> bool:
        """Whether the HIP kernels may stand in for ``self.fuse``: the "hip"
        backend and ``self.fuse`` the plain 3x3 zero-padded convolution
        without hooks (:func:`plain_conv`); otherwise ``self.fuse`` is called,
        as the reference does (triton_impl.py:392)."""
        return self.fuse_conv_backend == "hip" and plain_conv(self.fuse, 3)

    def _cuda_fuse(self, cat_out: torch.Tensor) -> torch.Tensor:
        """The fuse convolution of a ROCm concat: the HIP kernels where
        :meth:`_hip_fuse` allows and autocast is off, else ``self.fuse``
        (under autocast the Conv2d runs in the autocast dtype, as the
        reference's does)."""
        if self._hip_fuse() and not torch.is_autocast_enabled(cat_out.device.type):
            fuse_conv3x3 = _load_hip_ops()[4]
            return fuse_conv3x3(cat_out, self.fuse.weight, self.fuse.bias)
        return self.fuse(cat_out)

    def _cuda_pairs(self, x: torch.Tensor, y: torch.Tensor) -> torch.Tensor | None:
        """The fused route with the HIP fuse convolution: generator, filter,
        concat and fuse convolution as one pair of ops (``ops.fused_ddpm``:
        the generator's launch also packs the fuse weight; an fp32 concat is
        stored as bf16 pair planes); ``None`` where it does not apply."""
        if not self._hip_fuse():
            return None
        ops = _load_hip_ops()
        fused_ddpm, supported = ops[5], ops[6]
        args = (x, y, self.generator.weight, self.generator.bias, self.fuse.weight, self.fuse.bias,
                self.kernel_size, self.dilations)
        if not supported(*args) or self._route(x, y, ops[2]) != "fused":
            return None
        return fused_ddpm(*args)  # the arguments as checked just now

    def forward(self, x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
        _check_inputs(x, y, self.dim)
        if x.is_cuda:
            out = self._cuda_pairs(x, y)
            if out is not None:
                return out
            return self._cuda_fuse(self._cuda_cat(x, y))
        elif x.device.type == "cpu":
            cat_out = self._cpu_cat(x, y)
        else:
            raise ValueError(f"unsupported device {x.device}")
        return self.fuse(cat_out)


__all__ = ["DDPM", "plain_conv"]
