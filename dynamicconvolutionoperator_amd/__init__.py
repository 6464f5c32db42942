"""MI355X-native DDPM hot path (Dynamic Dilated Pyramid Module, HDFNet ECCV 2020).

Public API (drop-in for the reference's triton_impl / _triton_kernels):

* :class:`DDPM` - ``DDPM(dim, kernel_size=3, *, spatial_tile_size=4096,
  max_generated_bytes=256 MiB, recompute=True, fused_generator_inference=True,
  fused_generator_training=None)``; ``module(x, y) -> [N, C, H, W]``.
* :func:`fused_dynamic_cat` - ``(x, kernels, kernel_size, dilations)``.
* :func:`fused_generator_dynamic_cat` - ``(x, y, weight, bias, kernel_size,
  dilations)``.

GPU work runs in hand-written HIP kernels for gfx950 loaded from the in-tree
``libddpm_hip.so`` (build with ``python -m dynamicconvolutionoperator_amd.build``).
"""

from .module import DDPM
from ._cpu import native_dynamic_cat_from_kernels


def fused_dynamic_cat(x, kernels, kernel_size, dilations):
    from .ops import fused_dynamic_cat as _f

    return _f(x, kernels, kernel_size, dilations)


def fused_generator_dynamic_cat(x, y, weight, bias, kernel_size, dilations):
    from .ops import fused_generator_dynamic_cat as _f

    return _f(x, y, weight, bias, kernel_size, dilations)


__all__ = ["DDPM", "fused_dynamic_cat", "fused_generator_dynamic_cat", "native_dynamic_cat_from_kernels"]
