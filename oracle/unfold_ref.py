"""Torch restatement of the reference's Unfold oracle and its closed-form backward.

Test infrastructure only (see ``oracle/__init__.py``).

Reference files followed (cited as file:line of lartpang/DynamicConvolutionOperator):
* ``UnfoldDDPM`` / ``DepthDCOp``  -> unfold_impl.py:5-42
* ``dynamic_cat``                 -> unfold_impl.py:35-42 and gpu_bench.py:56-67
* ``generator``                   -> unfold_impl.py:15,23 (1x1 conv, rows o=(b*C+c)*K^2+tap)
* ``dynamic_cat_backward``        -> triton_impl.py:94-132 (unfold for dK, fold for dX)
* ``generator_dynamic_cat_backward`` -> _triton_kernels.py:430-811 (dX gather, dY = W^T dK,
                                    dW = dK y^T, db = sum dK)
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

DILATIONS = (1, 3, 5)


class DepthDCOp(nn.Module):
    """Dilated dynamic depthwise op through ``nn.Unfold`` (unfold_impl.py:32-42)."""

    def __init__(self, kernel_size: int, dilation: int = 1):
        super().__init__()
        self.unfold = nn.Unfold(
            kernel_size, dilation, padding=kernel_size // 2 * dilation, stride=1
        )

    def forward(self, x: torch.Tensor, kernel: torch.Tensor) -> torch.Tensor:
        n, c, h, w = x.shape
        patches = self.unfold(x).reshape(n, c, -1, h, w)
        return (patches * kernel).sum(2)


class UnfoldDDPM(nn.Module):
    """The reference's math oracle (unfold_impl.py:5-29).

    Parameters are created generator-first, then fuse, so a seeded default
    init matches the drop-in module's, and state-dict keys are
    ``generator.{weight,bias}`` and ``fuse.{weight,bias}``.
    """

    def __init__(self, dim: int, kernel_size: int = 3):
        super().__init__()
        self.kernel_size = kernel_size
        self.generator = nn.Conv2d(dim, 3 * dim * kernel_size**2, 1)
        self.branch_1 = DepthDCOp(kernel_size, 1)
        self.branch_3 = DepthDCOp(kernel_size, 3)
        self.branch_5 = DepthDCOp(kernel_size, 5)
        self.fuse = nn.Conv2d(4 * dim, dim, 3, 1, 1)

    def dynamic_cat(self, x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
        n, c, h, w = x.shape
        kernels = self.generator(y).reshape(n, 3, c, self.kernel_size**2, h, w)
        k1, k3, k5 = kernels.unbind(dim=1)
        return torch.cat(
            (x, self.branch_1(x, k1), self.branch_3(x, k3), self.branch_5(x, k5)), dim=1
        )

    def forward(self, x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
        return self.fuse(self.dynamic_cat(x, y))


def _patches(x: torch.Tensor, kernel_size: int, dilation: int) -> torch.Tensor:
    n, c, h, w = x.shape
    return F.unfold(
        x, kernel_size=kernel_size, dilation=dilation, padding=kernel_size // 2 * dilation
    ).view(n, c, kernel_size * kernel_size, h, w)


def dynamic_cat(
    x: torch.Tensor, kernels: torch.Tensor, kernel_size: int, dilations=DILATIONS
) -> torch.Tensor:
    """``[x, d1, d3, d5]`` from materialized kernels ``[N,3,C,K^2,H,W]``.

    out_b[n,c,h,w] = sum_{ki,kj} k[n,b,c,ki*K+kj,h,w] * x[n,c,h+(ki-r)d_b,w+(kj-r)d_b]
    with zero padding (unfold_impl.py:35-42; gpu_bench.py:56-67).
    """
    branches = [x]
    for b, d in enumerate(dilations):
        branches.append((_patches(x, kernel_size, d) * kernels[:, b]).sum(2))
    return torch.cat(branches, dim=1)


def generator(y: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    """1x1 conv ``C -> 3*C*K^2`` (unfold_impl.py:15,23)."""
    return F.conv2d(y, weight, bias)


def generated_kernels(
    y: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, kernel_size: int
) -> torch.Tensor:
    n, c, h, w = y.shape
    return generator(y, weight, bias).reshape(n, 3, c, kernel_size**2, h, w)


def generator_dynamic_cat(
    x: torch.Tensor,
    y: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor,
    kernel_size: int,
    dilations=DILATIONS,
) -> torch.Tensor:
    return dynamic_cat(x, generated_kernels(y, weight, bias, kernel_size), kernel_size, dilations)


def dynamic_cat_backward(
    x: torch.Tensor,
    kernels: torch.Tensor,
    grad_out: torch.Tensor,
    kernel_size: int,
    dilations=DILATIONS,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Closed-form (dX, dK) of ``dynamic_cat`` (triton_impl.py:94-132).

    dK_b = unfold_b(x) * gO_b ; dX = gO_x + sum_b fold_b(k_b * gO_b).
    """
    n, c, h, w = x.shape
    kk = kernel_size * kernel_size
    r = kernel_size // 2
    grad_x = grad_out[:, :c].clone()
    dks = []
    for b, d in enumerate(dilations):
        g = grad_out[:, (b + 1) * c : (b + 2) * c]
        dks.append(_patches(x, kernel_size, d) * g.unsqueeze(2))
        weighted = (kernels[:, b] * g.unsqueeze(2)).reshape(n, c * kk, h * w)
        grad_x = grad_x + F.fold(
            weighted, (h, w), kernel_size=kernel_size, dilation=d, padding=r * d
        )
    return grad_x, torch.stack(dks, dim=1)


def generator_dynamic_cat_backward(
    x: torch.Tensor,
    y: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor,
    grad_out: torch.Tensor,
    kernel_size: int,
    dilations=DILATIONS,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Closed-form (dX, dY, dW, db) of the generator + dynamic filter + concat.

    gen = W y + b;  dK = unfold(x) * gO_b  (dL/dgen);
    dX = gO_x + sum_b fold_b(gen_b * gO_b);  dY = W^T dK;
    dW = sum_tokens dK y^T;  db = sum_tokens dK   (_triton_kernels.py:430-811).
    """
    n, c, h, w = x.shape
    kernels = generated_kernels(y, weight, bias, kernel_size)
    grad_x, dk = dynamic_cat_backward(x, kernels, grad_out, kernel_size, dilations)
    g_rows = weight.shape[0]
    dk_rows = dk.reshape(n, g_rows, h * w)  # row o = (b*C + c)*K^2 + tap
    w2 = weight.reshape(g_rows, c)
    grad_y = torch.einsum("oi,nop->nip", w2, dk_rows).reshape(n, c, h, w)
    y_tok = y.reshape(n, c, h * w)
    grad_w = torch.einsum("nop,nip->oi", dk_rows, y_tok).reshape(weight.shape)
    grad_b = dk_rows.sum(dim=(0, 2))
    return grad_x, grad_y, grad_w, grad_b
