"""CPU-device branch of the drop-in ``DDPM`` (tensors that live on the host).

Mirrors the reference's CPU paths (triton_impl.py:47-244) so that a CPU user
of the reference sees the same routing and numerics:

* :func:`native_dynamic_cat_from_kernels` - shifted views of the zero-padded x
  instead of Unfold (triton_impl.py:47-70);
* :class:`NativeDynamicCat` - its custom backward with one unfold (dK) and one
  fold (dX) per dilation (triton_impl.py:73-132);
* :func:`cpu_training_dynamic_cat` - the Unfold path used for CPU training
  (triton_impl.py:146-166);
* :func:`streaming_generator_dynamic_cat` - generate and consume the dynamic
  kernels one spatial tile at a time, with per-tile checkpointing when
  training (triton_impl.py:169-244).

These functions are only reached for CPU tensors; GPU tensors go through the
HIP operators and never fall back here.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn
from torch.utils.checkpoint import checkpoint


def native_dynamic_cat_from_kernels(
    x: torch.Tensor, kernels: torch.Tensor, kernel_size: int, dilations: tuple[int, int, int]
) -> torch.Tensor:
    """``[x, d0, d1, d2]`` by summing shifted windows of the padded x."""
    _, _, h, w = x.shape
    r = kernel_size // 2
    halo = r * max(dilations)
    xp = F.pad(x, (halo, halo, halo, halo))
    branches = [x]
    for b, d in enumerate(dilations):
        acc = torch.zeros_like(x)
        for ki in range(kernel_size):
            top = halo + (ki - r) * d
            for kj in range(kernel_size):
                left = halo + (kj - r) * d
                window = xp[:, :, top : top + h, left : left + w]
                acc = acc + window * kernels[:, b, :, ki * kernel_size + kj]
        branches.append(acc)
    return torch.cat(branches, dim=1)


class NativeDynamicCat(torch.autograd.Function):
    """Shifted-view forward; backward with one unfold and one fold per dilation."""

    @staticmethod
    def forward(ctx, x, kernels, kernel_size, dilations):
        ctx.save_for_backward(x, kernels)
        ctx.kernel_size = kernel_size
        ctx.dilations = dilations
        return native_dynamic_cat_from_kernels(x, kernels, kernel_size, dilations)

    @staticmethod
    def backward(ctx, grad_out):
        x, kernels = ctx.saved_tensors
        k = ctx.kernel_size
        n, c, h, w = x.shape
        kk = k * k
        r = k // 2
        grad_x = grad_out[:, :c].contiguous()
        grad_k = []
        for b, d in enumerate(ctx.dilations):
            g = grad_out[:, (b + 1) * c : (b + 2) * c].contiguous()
            cols = F.unfold(x, kernel_size=k, dilation=d, padding=r * d).view(n, c, kk, h, w)
            grad_k.append(cols * g.unsqueeze(2))
            contrib = (kernels[:, b] * g.unsqueeze(2)).reshape(n, c * kk, h * w)
            grad_x = grad_x + F.fold(contrib, (h, w), kernel_size=k, dilation=d, padding=r * d)
        return grad_x, torch.stack(grad_k, dim=1), None, None


def native_dynamic_cat(x, kernels, kernel_size, dilations):
    if torch.is_grad_enabled() and (x.requires_grad or kernels.requires_grad):
        return NativeDynamicCat.apply(x, kernels, kernel_size, dilations)
    return native_dynamic_cat_from_kernels(x, kernels, kernel_size, dilations)


def cpu_training_dynamic_cat(
    x: torch.Tensor, kernels: torch.Tensor, kernel_size: int, unfolds: nn.ModuleList
) -> torch.Tensor:
    """Unfold path; oneDNN's unfold backward keeps its columns (faster CPU training)."""
    n, c, h, w = x.shape
    branches = [x]
    for kern, unfold in zip(kernels.unbind(dim=1), unfolds):
        cols = unfold(x).view(n, c, kernel_size * kernel_size, h, w)
        branches.append((cols * kern).sum(2))
    return torch.cat(branches, dim=1)


def streaming_generator_dynamic_cat(
    x: torch.Tensor,
    y: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor,
    kernel_size: int,
    dilations: tuple[int, int, int],
    tile_size: int,
    recompute: bool,
) -> torch.Tensor:
    """Generate and consume the dynamic kernels ``tile_size`` pixels at a time.

    Temporary kernel storage is O(N * tile * 3 * C * K^2); with ``recompute``
    and grad enabled each tile is checkpointed, so backward regenerates it.
    """
    n, c, h, w = x.shape
    hw = h * w
    kk = kernel_size * kernel_size
    r = kernel_size // 2
    halo = r * max(dilations)
    xp = F.pad(x, (halo, halo, halo, halo))
    tokens = y.flatten(2).transpose(1, 2)  # [N, HW, C]
    w2 = weight[:, :, 0, 0]
    tile = hw if tile_size <= 0 else min(tile_size, hw)
    per_branch: list[list[torch.Tensor]] = [[] for _ in dilations]

    for start in range(0, hw, tile):
        stop = min(start + tile, hw)
        pos = torch.arange(start, stop, device=x.device)
        rows = torch.div(pos, w, rounding_mode="floor")
        cols = pos.remainder(w)

        def one_tile(y_tile, x_pad, gen_w, gen_b, rows=rows, cols=cols, length=stop - start):
            gen = F.linear(y_tile, gen_w, gen_b).view(n, length, len(dilations), c, kk)
            outs = []
            for b, d in enumerate(dilations):
                acc = torch.zeros((n, length, c), dtype=x.dtype, device=x.device)
                for ki in range(kernel_size):
                    hi = rows + halo + (ki - r) * d
                    for kj in range(kernel_size):
                        wi = cols + halo + (kj - r) * d
                        acc = acc + x_pad[:, :, hi, wi].transpose(1, 2) * gen[:, :, b, :, ki * kernel_size + kj]
                outs.append(acc)
            return tuple(outs)

        args = (tokens[:, start:stop], xp, w2, bias)
        if recompute and torch.is_grad_enabled():
            outs = checkpoint(one_tile, *args, use_reentrant=False)
        else:
            outs = one_tile(*args)
        for b, t in enumerate(outs):
            per_branch[b].append(t)

    branches = [x]
    for tiles in per_branch:
        branches.append(torch.cat(tiles, dim=1).transpose(1, 2).reshape(n, c, h, w))
    return torch.cat(branches, dim=1)
