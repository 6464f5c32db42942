"""Operator-level API: ``fused_dynamic_cat`` and ``fused_generator_dynamic_cat``.

Drop-in counterparts of the reference's operators
(_triton_kernels.py:814-870 and :873-1065): same arguments, same output
dtype rules and the same autograd outputs, backed by hand-written HIP kernels
for gfx950 through the C-ABI in ``libddpm_hip.so``.

* ``fused_dynamic_cat(x, kernels, kernel_size, dilations)`` -> ``[N, 4C, H, W]``
  in ``kernels.dtype``; backward returns ``(dX, dK, None, None)``.
* ``fused_generator_dynamic_cat(x, y, weight, bias, kernel_size, dilations)``
  -> ``[N, 4C, H, W]`` in ``x.dtype``; backward recomputes the generator and
  returns ``(dX, dY, dW, db, None, None)``; only ``x, y, weight, bias`` are
  saved.

All tensors are allocated by torch (so ``max_memory_allocated`` sees them);
kernels run asynchronously on the current stream.  Tensors must be on a ROCm
("cuda") device; nothing here runs on the CPU.
"""

from __future__ import annotations

import contextlib
import functools

import torch

from . import _lib

_DTYPES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}
# dtype code of an fp32 concat stored as bf16 (hi, lo) pair planes: per
# 32-plane chunk, plane j < 16 holds the hi halves of channels (2j, 2j+1) and
# plane 16 + j their lo halves (hi = the top 16 bits of the fp32 pattern, lo =
# the remainder rounded to nearest even)
_PAIR_PLANES = 3


def _dt(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}; expected float32, bfloat16 or float16") from None


def _ptr(t: torch.Tensor) -> int:
    """t's device address for a ``void*`` argument (ctypes converts the int
    through the function's argtypes; no c_void_p object per pointer)."""
    return t.data_ptr()


# The current device and the raw handle of its current stream straight from
# torch's C layer: torch.cuda.current_stream() builds a Stream object per
# call (about 10 us of host time inside a backward, several calls per step).
_current_device = getattr(torch._C, "_cuda_getDevice", None) or torch.cuda.current_device
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None) or (
    lambda idx: torch.cuda.current_stream(idx).cuda_stream)


def _stream(t: torch.Tensor) -> int:
    """The current stream of t's device, as the C-ABI's hipStream_t (an int
    for the ``void*`` argument)."""
    idx = t.device.index
    return _raw_stream(_current_device() if idx is None else idx)


def _on(device: torch.device):
    """Device guard for a launch: a no-op when `device` is already current
    (the usual case)."""
    if device.index is None or device.index == _current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(device)


@functools.lru_cache(maxsize=512)
def _ws_bytes(query: str, *args) -> int:
    """Workspace bytes from a C-ABI ``*_workspace_bytes`` query (a pure
    function of its arguments, so each shape is asked once)."""
    return int(getattr(_lib.load(), query)(*args))


def _as(t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """t in `dtype`, contiguous (no torch call when it already is)."""
    if t.dtype != dtype:
        t = t.to(dtype)
    return t if t.is_contiguous() else t.contiguous()


def _require_device(*tensors: torch.Tensor) -> None:
    dev = tensors[0].device
    if dev.type != "cuda":
        raise ValueError(f"HIP operators need tensors on a ROCm device, got {dev}")
    for t in tensors[1:]:
        if t.device != dev:
            raise ValueError(f"all tensors must be on {dev}, got {t.device}")


def _check_dilations(dilations) -> tuple[int, int, int]:
    d = tuple(int(v) for v in dilations)
    if len(d) != 3 or min(d) < 1:
        raise ValueError(f"dilations must be three positive integers, got {dilations}")
    return d


def _check_kernel_size(kernel_size: int) -> int:
    k = int(kernel_size)
    if k < 1 or k % 2 == 0:
        raise ValueError(f"kernel_size must be a positive odd integer, got {kernel_size}")
    return k


# ---------------------------------------------------------------------------
# Materialized path: kernels given as [N, 3, C, K*K, H, W]
# ---------------------------------------------------------------------------
def _check_filter_inputs(x: torch.Tensor, kernels: torch.Tensor, k: int) -> None:
    if x.ndim != 4:
        raise ValueError(f"x must be NCHW, got shape {tuple(x.shape)}")
    n, c, h, w = x.shape
    if tuple(kernels.shape) != (n, 3, c, k * k, h, w):
        raise ValueError(
            f"kernels must have shape {(n, 3, c, k * k, h, w)}, got {tuple(kernels.shape)}"
        )
    _require_device(x, kernels)
    _dt(x)
    _dt(kernels)


def _filter_call(fn_name: str, a, b, out, x_shape, k, dil, x_dtype: int, k_dtype: int):
    lib = _lib.load()
    n, c, h, w = x_shape
    with _on(out.device):
        code = getattr(lib, fn_name)(
            _ptr(a), _ptr(b), _ptr(out), n, c, h, w, k, dil[0], dil[1], dil[2], x_dtype, k_dtype,
            _stream(out),
        )
    _lib.check(code, fn_name)


class _DynamicCat(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, kernels, kernel_size, dilations):
        k = _check_kernel_size(kernel_size)
        dil = _check_dilations(dilations)
        x = x.contiguous()
        kernels = kernels.contiguous()
        _check_filter_inputs(x, kernels, k)
        n, c, h, w = x.shape
        out = torch.empty((n, 4 * c, h, w), dtype=kernels.dtype, device=x.device)
        _filter_call("ddpm_filter_fwd", x, kernels, out, x.shape, k, dil, _dt(x), _dt(kernels))
        ctx.save_for_backward(x, kernels)
        ctx.kernel_size = k
        ctx.dilations = dil
        return out

    @staticmethod
    def backward(ctx, grad_out):
        x, kernels = ctx.saved_tensors
        grad_out = _as(grad_out, kernels.dtype)
        grad_x = grad_k = None
        if ctx.needs_input_grad[0]:
            grad_x = torch.empty_like(x)
            _filter_call("ddpm_filter_bwd_x", grad_out, kernels, grad_x, x.shape, ctx.kernel_size,
                         ctx.dilations, _dt(x), _dt(kernels))
        if ctx.needs_input_grad[1]:
            grad_k = torch.empty_like(kernels)
            _filter_call("ddpm_filter_bwd_k", x, grad_out, grad_k, x.shape, ctx.kernel_size,
                         ctx.dilations, _dt(x), _dt(kernels))
        return grad_x, grad_k, None, None


def fused_dynamic_cat(x, kernels, kernel_size, dilations):
    """``[x, d0, d1, d2]`` from materialized dynamic kernels (_triton_kernels.py:869-870)."""
    return _DynamicCat.apply(x, kernels, kernel_size, dilations)


# ---------------------------------------------------------------------------
# Fused generator path
# ---------------------------------------------------------------------------
# The fused kernels address one image's [C][H][W] planes with 32-bit byte offsets.
_FUSED_MAX_IMAGE_BYTES = 2**31 - 1


@functools.lru_cache(maxsize=256)
def _gen_query(forward_only: bool, channels: int, kernel_size: int, max_dilation: int) -> bool:
    """The library's coverage query (a pure function of its arguments, asked
    once per configuration: the module checks it on every call)."""
    lib = _lib.load()
    query = lib.ddpm_gen_fwd_supported if forward_only else lib.ddpm_gen_supported
    return bool(query(channels, kernel_size, max_dilation))


def generator_supported(channels: int, kernel_size: int, dilations=(1, 3, 5), shape=None,
                        dtype=None, forward_only: bool = False) -> bool:
    """Whether the fused generator kernels handle this configuration and,
    given ``shape`` ``[N, C, H, W]`` and ``dtype``, whether one image's planes
    fit their 32-bit offsets.  ``forward_only``: the forward alone (inference:
    ``ddpm_gen_fwd_supported``, K in {1, 3, 5}); else forward and recompute
    backward (``ddpm_gen_supported``, K in {1, 3})."""
    if not _gen_query(bool(forward_only), int(channels), int(kernel_size), int(max(dilations))):
        return False
    if shape is not None:
        esize = (dtype if dtype is not None else torch.float32).itemsize
        if int(shape[1]) * int(shape[2]) * int(shape[3]) * esize > _FUSED_MAX_IMAGE_BYTES:
            return False
    return True


def _check_generator_inputs(x, y, weight, bias, k: int) -> None:
    if x.ndim != 4 or y.shape != x.shape:
        raise ValueError(f"x and y must be NCHW tensors of identical shapes, got {x.shape} and {y.shape}")
    n, c, h, w = x.shape
    g = 3 * c * k * k
    if weight.numel() != g * c or weight.shape[0] != g:
        raise ValueError(f"weight must have shape {(g, c, 1, 1)}, got {tuple(weight.shape)}")
    if bias is None or tuple(bias.shape) != (g,):
        raise ValueError(f"bias must have shape {(g,)}")
    _require_device(x, y, weight, bias)
    if not (x.dtype == y.dtype == weight.dtype == bias.dtype):
        raise TypeError("x, y, weight and bias must share one dtype on the fused generator path")
    _dt(x)


def _launch_generator_dynamic_cat(x, y, weight, bias, k, dil):
    x = x.contiguous()
    y = y.contiguous()
    weight = weight.contiguous()
    bias = bias.contiguous()
    _check_generator_inputs(x, y, weight, bias, k)
    n, c, h, w = x.shape
    out = torch.empty((n, 4 * c, h, w), dtype=x.dtype, device=x.device)
    lib = _lib.load()
    with _on(x.device):
        code = lib.ddpm_gen_fwd(
            _ptr(x), _ptr(y), _ptr(weight), _ptr(bias), _ptr(out), n, c, h, w, k, *dil, _dt(x),
            _stream(x),
        )
    _lib.check(code, "ddpm_gen_fwd")
    return out


class _GeneratorDynamicCat(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, y, weight, bias, k, dil):
        # k and dil as fused_generator_dynamic_cat checked them
        x = x.contiguous()
        y = y.contiguous()
        weight = weight.contiguous()
        bias = bias.contiguous()
        out = _launch_generator_dynamic_cat(x, y, weight, bias, k, dil)
        ctx.save_for_backward(x, y, weight, bias)
        ctx.kernel_size = k
        ctx.dilations = dil
        return out

    @staticmethod
    def backward(ctx, grad_out):
        x, y, weight, bias = ctx.saved_tensors
        grads = _generator_backward(x, y, weight, bias, _as(grad_out, x.dtype), ctx.kernel_size,
                                    ctx.dilations, ctx.needs_input_grad[:4])
        return (*grads, None, None)


def _align256(nbytes: int) -> int:
    return (nbytes + 255) // 256 * 256


def _generator_backward(x, y, weight, bias, grad_out, k, dil, needs):
    """The four gradients of the fused generator op (``None`` where
    ``needs`` says no): one ``ddpm_gen_bwd`` call when all are needed, else
    the combined dX / dW call or the separate entry points."""
    n, c, h, w = x.shape
    lib = _lib.load()
    dt = _dt(x)
    stream = _stream(x)
    grad_x = grad_y = grad_w = grad_b = None
    need_x, need_y = needs[0], needs[1]
    need_wb = needs[2] or needs[3]
    combined = need_x and need_y and need_wb

    def alloc_y():
        wsy_bytes = _ws_bytes("ddpm_gen_bwd_y_workspace_bytes", c, k)
        return (torch.empty_like(y), torch.empty(wsy_bytes, dtype=torch.uint8, device=x.device),
                wsy_bytes)

    with _on(x.device):
        if combined:
            # one call: dY's weight packing and dX's halo reduction run on
            # the CUs dW leaves free; its three workspaces share one
            # allocation (256-byte aligned parts)
            grad_x = torch.empty_like(x)
            grad_y = torch.empty_like(y)
            grad_w = torch.empty_like(weight)
            grad_b = torch.empty_like(bias)
            wsx_bytes = _ws_bytes("ddpm_gen_bwd_x_workspace_bytes", n, c, h, w, k, *dil)
            ws_bytes = _ws_bytes("ddpm_gen_bwd_w_workspace_bytes", n, c, h, w, k, dt)
            wsy_bytes = _ws_bytes("ddpm_gen_bwd_y_workspace_bytes", c, k)
            oy = _align256(wsx_bytes)
            ow = oy + _align256(wsy_bytes)
            wsall = torch.empty(ow + max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
            base = wsall.data_ptr()
            _lib.check(
                lib.ddpm_gen_bwd(_ptr(x), _ptr(y), _ptr(weight), _ptr(bias), _ptr(grad_out),
                                 _ptr(grad_x), _ptr(grad_y), _ptr(grad_w), _ptr(grad_b),
                                 base, wsx_bytes, base + oy, wsy_bytes, base + ow, ws_bytes,
                                 n, c, h, w, k, *dil, dt, stream),
                "ddpm_gen_bwd",
            )
            del wsall
            if not needs[2]:
                grad_w = None
            if not needs[3]:
                grad_b = None
            return grad_x, grad_y, grad_w, grad_b
        if need_x:
            grad_x = torch.empty_like(x)
            wsx_bytes = _ws_bytes("ddpm_gen_bwd_x_workspace_bytes", n, c, h, w, k, *dil)
            wsx = torch.empty(wsx_bytes, dtype=torch.uint8, device=x.device)
        if need_wb:
            grad_w = torch.empty_like(weight)
            grad_b = torch.empty_like(bias)
            ws_bytes = _ws_bytes("ddpm_gen_bwd_w_workspace_bytes", n, c, h, w, k, dt)
            ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
        y_pending = need_y
        if need_x and need_wb:
            # one call: dX's halo reduction runs on the CUs dW leaves free
            _lib.check(
                lib.ddpm_gen_bwd_xw(_ptr(x), _ptr(y), _ptr(weight), _ptr(bias), _ptr(grad_out),
                                    _ptr(grad_x), _ptr(grad_w), _ptr(grad_b), _ptr(wsx),
                                    wsx_bytes, _ptr(ws), ws_bytes, n, c, h, w, k, *dil, dt,
                                    stream),
                "ddpm_gen_bwd_xw",
            )
        elif need_x:
            _lib.check(
                lib.ddpm_gen_bwd_x(_ptr(y), _ptr(weight), _ptr(bias), _ptr(grad_out),
                                   _ptr(grad_x), _ptr(wsx), wsx_bytes, n, c, h, w, k, *dil,
                                   dt, stream),
                "ddpm_gen_bwd_x",
            )
        elif need_wb:
            _lib.check(
                lib.ddpm_gen_bwd_w(_ptr(x), _ptr(y), _ptr(grad_out), _ptr(grad_w),
                                   _ptr(grad_b), _ptr(ws), ws_bytes, n, c, h, w, k, *dil, dt,
                                   stream),
                "ddpm_gen_bwd_w",
            )
        if need_x:
            del wsx
        if need_wb:
            del ws
            if not needs[2]:
                grad_w = None
            if not needs[3]:
                grad_b = None
        if y_pending:
            # allocated once the dX and dW workspaces are released
            grad_y, wsy, wsy_bytes = alloc_y()
            _lib.check(
                lib.ddpm_gen_bwd_y(_ptr(x), _ptr(weight), _ptr(grad_out), _ptr(grad_y),
                                   _ptr(wsy), wsy_bytes, n, c, h, w, k, *dil, dt, stream),
                "ddpm_gen_bwd_y",
            )
    return grad_x, grad_y, grad_w, grad_b


# ---------------------------------------------------------------------------
# Generator 1x1 convolution of the materialized route
# ---------------------------------------------------------------------------
GENERATOR_KERNELS_MAX_CHANNELS = 128  # ddpm_gen_kernels keeps y's K operand in registers


def generator_kernels_supported(y, weight, bias) -> bool:
    """Whether ``ddpm_gen_kernels`` (and its backward) computes this generator
    convolution: one dtype for y, weight and bias, at most 128 channels, and
    one image's generated planes within the kernels' 32-bit offsets
    (``ddpm_gen_kernels_supported``)."""
    if bias is None or y.dtype not in _DTYPES or not (y.dtype == weight.dtype == bias.dtype):
        return False
    if y.ndim != 4 or y.shape[1] > GENERATOR_KERNELS_MAX_CHANNELS:
        return False
    o, c = weight.shape[0], y.shape[1]
    k2, rem = divmod(o, 3 * c)
    k = int(round(k2 ** 0.5))
    if rem or k * k != k2:
        return False
    n, _, h, w = y.shape
    return bool(_lib.load().ddpm_gen_kernels_supported(n, c, h, w, k, _DTYPES[y.dtype]))


class _GeneratorKernels(torch.autograd.Function):
    """``kernels = conv2d(y, weight, bias)`` for the 1x1 generator, as
    ``[N, 3CK², H, W]`` in y's dtype (the reference's ``self.generator(y)``,
    triton_impl.py:340-347).  Forward: one HIP MFMA kernel with the bias and
    the output rounding fused.  Backward: dW and db in one HIP kernel that
    reads dK once (``ddpm_gen_kernels_bwd_w``), dY = Wᵀ·dK in another
    (``ddpm_gen_kernels_bwd_y``)."""

    @staticmethod
    def forward(ctx, y, weight, bias, kernel_size):
        k = _check_kernel_size(kernel_size)
        y = y.contiguous()
        n, c, h, w = y.shape
        o = 3 * c * k * k
        if tuple(weight.shape) not in ((o, c, 1, 1), (o, c)) or tuple(bias.shape) != (o,):
            raise ValueError(
                f"generator weight / bias must be [{o}, {c}, 1, 1] / [{o}], got "
                f"{tuple(weight.shape)} / {tuple(bias.shape)}"
            )
        _require_device(y, weight, bias)
        w2 = weight.reshape(o, c).contiguous()
        b = bias.contiguous()
        out = torch.empty((n, o, h, w), dtype=y.dtype, device=y.device)
        lib = _lib.load()
        with _on(y.device):
            code = lib.ddpm_gen_kernels(_ptr(y), _ptr(w2), _ptr(b), _ptr(out), n, c, h, w, k, _dt(y),
                                        _stream(y))
        _lib.check(code, "ddpm_gen_kernels")
        ctx.save_for_backward(y, w2)
        ctx.weight_shape = tuple(weight.shape)
        ctx.kernel_size = k
        return out

    @staticmethod
    def backward(ctx, grad):
        y, w2 = ctx.saved_tensors
        n, c, h, w = y.shape
        o = w2.shape[0]
        g = grad.to(y.dtype).contiguous().view(n, o, h * w)
        grad_y = grad_w = grad_b = None
        if ctx.needs_input_grad[0]:
            grad_y = _generator_kernels_input_grad(w2, g, n, c, h, w, ctx.kernel_size)
        if ctx.needs_input_grad[1] or ctx.needs_input_grad[2]:
            k = ctx.kernel_size
            lib = _lib.load()
            gw = torch.empty((o, c), dtype=y.dtype, device=y.device)
            gb = torch.empty((o,), dtype=y.dtype, device=y.device)
            with _on(y.device):
                ws_bytes = _ws_bytes("ddpm_gen_kernels_bwd_w_workspace_bytes", n, c, h, w, k)
                ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=y.device)
                code = lib.ddpm_gen_kernels_bwd_w(_ptr(y), _ptr(g), _ptr(gw), _ptr(gb), _ptr(ws),
                                                  ws_bytes, n, c, h, w, k, _dt(y), _stream(y))
            _lib.check(code, "ddpm_gen_kernels_bwd_w")
            if ctx.needs_input_grad[1]:
                grad_w = gw.reshape(ctx.weight_shape)
            if ctx.needs_input_grad[2]:
                grad_b = gb
        return grad_y, grad_w, grad_b, None


def _generator_kernels_input_grad(w2, g, n, c, h, w, k):
    """dY = Wᵀ·dK of the generator convolution through ``ddpm_gen_kernels_bwd_y``
    (every shape :func:`generator_kernels_supported` accepts)."""
    lib = _lib.load()
    grad_y = torch.empty((n, c, h, w), dtype=g.dtype, device=g.device)
    with _on(g.device):
        ws_bytes = _ws_bytes("ddpm_gen_kernels_bwd_y_workspace_bytes", n, c, h, w, k)
        ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=g.device)
        code = lib.ddpm_gen_kernels_bwd_y(_ptr(w2), _ptr(g), _ptr(grad_y), _ptr(ws), ws_bytes, n, c, h,
                                          w, k, _dt(g), _stream(g))
    _lib.check(code, "ddpm_gen_kernels_bwd_y")
    return grad_y


def generator_kernels(y, weight, bias, kernel_size):
    """The 1x1 generator convolution ``[N, 3CK², H, W]`` of the materialized
    route through ``ddpm_gen_kernels`` (shapes and dtypes of
    :func:`generator_kernels_supported`)."""
    return _GeneratorKernels.apply(y, weight, bias, kernel_size)


def _generate(y, weight, bias, k):
    if generator_kernels_supported(y, weight, bias):
        return generator_kernels(y, weight, bias, k)
    return torch.nn.functional.conv2d(y, weight, bias)


def _materialized_generator_dynamic_cat(x, y, weight, bias, k, dil):
    n, c, h, w = x.shape
    kernels = _generate(y, weight, bias, k).reshape(n, 3, c, k * k, h, w)
    return fused_dynamic_cat(x, kernels, k, dil)


def fused_generator_dynamic_cat(x, y, weight, bias, kernel_size, dilations):
    """Generator + dynamic filter + concat (_triton_kernels.py:1056-1065).

    Uses the autograd Function when grad is enabled and any input requires
    grad, else a single forward launch (which also takes K = 5).  Shapes
    outside the fused kernels' coverage (:func:`generator_supported`) run the
    generator as a 1x1 convolution and the HIP materialized filter, with the
    same result and autograd outputs.
    """
    k = _check_kernel_size(kernel_size)
    dil = _check_dilations(dilations)
    needs_grad = torch.is_grad_enabled() and any(t.requires_grad for t in (x, y, weight, bias))
    if not generator_supported(x.shape[1], k, dil, x.shape, x.dtype, forward_only=not needs_grad):
        return _materialized_generator_dynamic_cat(x, y, weight, bias, k, dil)
    if needs_grad:
        return _GeneratorDynamicCat.apply(x, y, weight, bias, k, dil)
    return _launch_generator_dynamic_cat(x, y, weight, bias, k, dil)


# ---------------------------------------------------------------------------
# The 3x3 fuse convolution
# ---------------------------------------------------------------------------
def fuse_conv_supported(cat, weight, bias) -> bool:
    """Whether the HIP fuse convolution takes this call: Conv2d(4C -> C, 3,
    padding 1) weights, one dtype for the concat, weight and bias, a ROCm
    device, and one image's planes within 32-bit byte offsets."""
    if cat.ndim != 4 or weight.ndim != 4 or cat.dtype not in _DTYPES:
        return False
    n, ci, h, w = cat.shape
    c = weight.shape[0]
    if tuple(weight.shape) != (c, ci, 3, 3) or ci != 4 * c:
        return False
    if weight.dtype != cat.dtype or (bias is not None and bias.dtype != cat.dtype):
        return False
    if cat.device.type != "cuda" or weight.device != cat.device:
        return False
    return ci * h * w * cat.element_size() <= 2**31 - 1


def _fuse_conv_workspace(n, c, h, w, dt, device):
    nbytes = _ws_bytes("ddpm_fuse_conv_workspace_bytes", n, c, h, w, dt)
    return torch.empty(max(nbytes, 16), dtype=torch.uint8, device=device), nbytes


def _fuse_conv_forward(cat, weight, bias, cat_code):
    """``ddpm_fuse_conv_fwd`` of a contiguous concat; ``cat_code`` is the
    concat's dtype code (3: fp32 pair planes)."""
    n, ci, h, w = cat.shape
    c = weight.shape[0]
    out = torch.empty((n, c, h, w), dtype=weight.dtype, device=cat.device)
    lib = _lib.load()
    with _on(cat.device):
        ws, nbytes = _fuse_conv_workspace(n, c, h, w, cat_code, cat.device)
        code = lib.ddpm_fuse_conv_fwd(_ptr(cat), _ptr(weight),
                                      _ptr(bias.contiguous()) if bias is not None else None,
                                      _ptr(out), _ptr(ws), nbytes, n, c, h, w, cat_code, _stream(cat))
    _lib.check(code, "ddpm_fuse_conv_fwd")
    return out


def _fuse_conv_backward(cat, weight, has_bias, grad_out, needs, cat_code):
    """Gradients of the fuse convolution for the concat (plain layout), the
    weight and the bias, ``None`` where ``needs`` says no.  ``cat_code`` 3
    reads a pair-plane concat in the weight gradient (its input gradient is a
    plain fp32 concat)."""
    n, ci, h, w = cat.shape
    c = weight.shape[0]
    dt = _dt(weight)
    grad_cat = grad_w = grad_b = None
    lib = _lib.load()
    need_w = needs[1]
    need_b = has_bias and needs[2]
    data_bytes = _ws_bytes("ddpm_fuse_conv_workspace_bytes", n, c, h, w, dt) if needs[0] else 0
    weight_bytes = (_ws_bytes("ddpm_fuse_conv_bwd_weight_workspace_bytes", n, c, h, w, cat_code)
                    if need_w or need_b else 0)
    if needs[0] and (need_w or need_b):
        # all gradients in one call (two launches); its two workspaces live at once
        off = _align256(data_bytes)
        ws = torch.empty(max(off + weight_bytes, 16), dtype=torch.uint8, device=cat.device)
        grad_cat = torch.empty((n, ci, h, w), dtype=weight.dtype, device=cat.device)
        gw = torch.empty_like(weight)
        gb = torch.empty((c,), dtype=weight.dtype, device=cat.device)
        with _on(cat.device):
            code = lib.ddpm_fuse_conv_bwd(_ptr(cat), _ptr(weight), _ptr(grad_out), _ptr(grad_cat),
                                          _ptr(gw), _ptr(gb), _ptr(ws), data_bytes,
                                          _ptr(ws) + off, weight_bytes, n, c, h, w, cat_code,
                                          _stream(cat))
        if code != _lib.STATUS_UNSUPPORTED:
            _lib.check(code, "ddpm_fuse_conv_bwd")
            return grad_cat, gw if need_w else None, gb if need_b else None
        grad_cat = None  # a part the combined call does not take: the two calls below
    # one workspace serves both calls (they run in order on one stream)
    ws = torch.empty(max(data_bytes, weight_bytes, 16), dtype=torch.uint8, device=cat.device)
    if needs[0]:
        grad_cat = torch.empty((n, ci, h, w), dtype=weight.dtype, device=cat.device)
        with _on(cat.device):
            code = lib.ddpm_fuse_conv_bwd_data(_ptr(grad_out), _ptr(weight), _ptr(grad_cat),
                                               _ptr(ws), data_bytes, n, c, h, w, dt, _stream(cat))
        _lib.check(code, "ddpm_fuse_conv_bwd_data")
    if need_w or need_b:
        gw = torch.empty_like(weight)
        gb = torch.empty((c,), dtype=weight.dtype, device=cat.device)
        with _on(cat.device):
            code = lib.ddpm_fuse_conv_bwd_weight(_ptr(cat), _ptr(grad_out), _ptr(gw), _ptr(gb),
                                                 _ptr(ws), weight_bytes, n, c, h, w, cat_code,
                                                 _stream(cat))
        if code == _lib.STATUS_UNSUPPORTED and cat_code != _PAIR_PLANES:
            _, gw, gb = torch.ops.aten.convolution_backward(
                grad_out, cat, weight, [c] if has_bias else None, [1, 1], [1, 1], [1, 1],
                False, [0, 0], 1, [False, need_w, need_b])
        else:
            _lib.check(code, "ddpm_fuse_conv_bwd_weight")
        grad_w = gw if need_w else None
        grad_b = gb if need_b else None
    return grad_cat, grad_w, grad_b


class _FuseConv3x3(torch.autograd.Function):
    """``F.conv2d(cat, weight, bias, padding=1)`` for the DDPM fuse
    convolution as HIP MFMA kernels: forward and input gradient
    (``ddpm_fuse_conv_fwd`` / ``_bwd_data``, implicit GEMMs over the input
    planes), weight and bias gradients (``ddpm_fuse_conv_bwd_weight``, a
    split pixel reduction; more than 128 output channels use the library's
    backward-filter convolution)."""

    @staticmethod
    def forward(ctx, cat, weight, bias):
        cat = cat.contiguous()
        weight = weight.contiguous()
        out = _fuse_conv_forward(cat, weight, bias, _dt(cat))
        ctx.save_for_backward(cat, weight)
        ctx.has_bias = bias is not None
        return out

    @staticmethod
    def backward(ctx, grad_out):
        cat, weight = ctx.saved_tensors
        return _fuse_conv_backward(cat, weight, ctx.has_bias, _as(grad_out, cat.dtype),
                                   ctx.needs_input_grad, _dt(cat))


def fuse_conv3x3(cat, weight, bias=None):
    """The DDPM fuse convolution ``Conv2d(4C -> C, 3, padding=1)`` on the HIP
    path (shapes of :func:`fuse_conv_supported`), else the library one."""
    if fuse_conv_supported(cat, weight, bias):
        return _FuseConv3x3.apply(cat, weight, bias)
    return torch.nn.functional.conv2d(cat, weight, bias, padding=1)


# ---------------------------------------------------------------------------
# Generator + filter + concat + fuse convolution, fp32 concat in pair planes
# ---------------------------------------------------------------------------
def fused_ddpm_supported(x, y, gen_weight, gen_bias, fuse_weight, fuse_bias, kernel_size,
                         dilations) -> bool:
    """Whether :func:`fused_ddpm` takes this call: one dtype (fp32, bf16 or
    fp16) throughout, a ROCm device, the fused generator kernels' coverage
    (:func:`generator_supported`; the forward's alone when no gradient is
    needed), for fp32 C % 16 == 0 (whole 32-plane chunks of the pair-plane
    concat), the HIP fuse convolution's coverage and weight shapes of
    DDPM(C, K)."""
    if x.dtype not in _DTYPES or x.ndim != 4 or not x.is_cuda:
        return False
    n, c, h, w = x.shape
    k = int(kernel_size)
    if (x.dtype == torch.float32 and c % 16 != 0) or tuple(y.shape) != tuple(x.shape) \
            or y.device != x.device:
        return False
    g = 3 * c * k * k
    if gen_bias is None or tuple(gen_weight.shape) != (g, c, 1, 1) or tuple(gen_bias.shape) != (g,):
        return False
    if tuple(fuse_weight.shape) != (c, 4 * c, 3, 3):
        return False
    if fuse_bias is not None and tuple(fuse_bias.shape) != (c,):
        return False
    tensors = (y, gen_weight, gen_bias, fuse_weight, fuse_bias)
    if any(t is not None and (t.dtype != x.dtype or t.device != x.device) for t in tensors):
        return False
    needs_grad = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad for t in (x, *tensors))
    if not generator_supported(c, k, dilations, x.shape, x.dtype, forward_only=not needs_grad):
        return False
    return 4 * c * h * w * x.element_size() <= 2**31 - 1


def _cat_code(dtype: torch.dtype) -> int:
    """The concat's dtype code on the fused_ddpm route: fp32 pair planes, else
    the plain dtype."""
    return _PAIR_PLANES if dtype == torch.float32 else _DTYPES[dtype]


def _concat_pack(x, y, gen_weight, gen_bias, fuse_weight, k, dil):
    """ddpm_gen_fwd_pack: the concat (fp32 as pair planes) and, in the fuse
    convolution's workspace, its packed weight (returned with it)."""
    n, c, h, w = x.shape
    code = _cat_code(x.dtype)
    cat = torch.empty((n, 4 * c, h, w), dtype=x.dtype, device=x.device)
    lib = _lib.load()
    with _on(x.device):
        ws, nbytes = _fuse_conv_workspace(n, c, h, w, code, x.device)
        rc = lib.ddpm_gen_fwd_pack(_ptr(x), _ptr(y), _ptr(gen_weight), _ptr(gen_bias), _ptr(cat),
                                   _ptr(fuse_weight), _ptr(ws), nbytes, n, c, h, w, k, *dil, code,
                                   _stream(x))
    _lib.check(rc, "ddpm_gen_fwd_pack")
    return cat, ws


def _fuse_conv_forward_packed(cat, ws, fuse_bias):
    """ddpm_fuse_conv_fwd_packed over a concat of :func:`_concat_pack` whose
    workspace ``ws`` holds the packed weight."""
    n, ci, h, w = cat.shape
    c = ci // 4
    out = torch.empty((n, c, h, w), dtype=cat.dtype, device=cat.device)
    lib = _lib.load()
    with _on(cat.device):
        rc = lib.ddpm_fuse_conv_fwd_packed(_ptr(cat), _ptr(fuse_bias) if fuse_bias is not None else None,
                                           _ptr(out), _ptr(ws), ws.numel(), n, c, h, w,
                                           _cat_code(cat.dtype), _stream(cat))
    _lib.check(rc, "ddpm_fuse_conv_fwd_packed")
    return out


class _GeneratorConcat(torch.autograd.Function):
    """Generator + filter + concat, an fp32 concat written as pair planes
    (an encoding only :class:`_FuseConvOfConcat` reads; the gradient arriving
    for it is the plain fp32 gradient of the concat values), so the backward
    is the generator op's (recompute from x, y, W, b).  The same launch packs
    the fuse convolution's weight into the forward workspace it returns
    beside the concat (no gradient)."""

    @staticmethod
    def forward(ctx, x, y, gen_weight, gen_bias, fuse_weight, kernel_size, dilations):
        cat, ws = _concat_pack(x, y, gen_weight, gen_bias, fuse_weight, kernel_size, dilations)
        ctx.save_for_backward(x, y, gen_weight, gen_bias)
        ctx.kernel_size = kernel_size
        ctx.dilations = dilations
        ctx.mark_non_differentiable(ws)
        # no zero-filled gradient for the workspace output (a fill kernel per step)
        ctx.set_materialize_grads(False)
        return cat, ws

    @staticmethod
    def backward(ctx, grad_cat, grad_ws):
        if grad_cat is None:
            return (None,) * 7
        x, y, gen_weight, gen_bias = ctx.saved_tensors
        grads = _generator_backward(x, y, gen_weight, gen_bias, _as(grad_cat, x.dtype),
                                    ctx.kernel_size, ctx.dilations, ctx.needs_input_grad[:4])
        return (*grads, None, None, None)


class _FuseConvOfConcat(torch.autograd.Function):
    """The fuse convolution of a :class:`_GeneratorConcat` concat (fp32:
    forward and weight / bias gradients read the pair planes; the input
    gradient is a plain fp32 concat gradient).  A node of its own, so
    autograd releases the saved concat as soon as this backward has run,
    before the generator's backward allocates its buffers."""

    @staticmethod
    def forward(ctx, cat, ws, fuse_weight, fuse_bias):
        # ws: the forward's workspace, holding the packed weight (_GeneratorConcat)
        out = _fuse_conv_forward_packed(cat, ws, fuse_bias)
        ctx.save_for_backward(cat, fuse_weight)
        ctx.has_bias = fuse_bias is not None
        return out

    @staticmethod
    def backward(ctx, grad_out):
        cat, fuse_weight = ctx.saved_tensors
        grads = _fuse_conv_backward(cat, fuse_weight, ctx.has_bias, _as(grad_out, cat.dtype),
                                    (ctx.needs_input_grad[0], *ctx.needs_input_grad[2:]),
                                    _cat_code(cat.dtype))
        return grads[0], None, grads[1], grads[2]


def fused_ddpm(x, y, gen_weight, gen_bias, fuse_weight, fuse_bias, kernel_size, dilations):
    """``fuse_conv3x3(fused_generator_dynamic_cat(x, y, ...), fuse_weight,
    fuse_bias)`` for shapes of :func:`fused_ddpm_supported`, the generator's
    launch also packing the fuse convolution's weight.  fp32 keeps the concat
    in pair planes between the two (the result differs from the separate ops
    only by the fuse convolution's summation order); bf16 / fp16 give the
    separate ops' results bit for bit."""
    k = _check_kernel_size(kernel_size)
    dil = _check_dilations(dilations)
    if not fused_ddpm_supported(x, y, gen_weight, gen_bias, fuse_weight, fuse_bias, k, dil):
        raise ValueError("fused_ddpm: shapes or dtypes outside fused_ddpm_supported")
    return _fused_ddpm_checked(x, y, gen_weight, gen_bias, fuse_weight, fuse_bias, k, dil)


def _fused_ddpm_checked(x, y, gen_weight, gen_bias, fuse_weight, fuse_bias, k, dil):
    """:func:`fused_ddpm` for arguments :func:`fused_ddpm_supported` has
    accepted (k an int, dil a tuple of three ints)."""
    x, y = x.contiguous(), y.contiguous()
    gen_weight, gen_bias = gen_weight.contiguous(), gen_bias.contiguous()
    fuse_weight = fuse_weight.contiguous()
    fuse_bias = fuse_bias.contiguous() if fuse_bias is not None else None
    tensors = (x, y, gen_weight, gen_bias, fuse_weight, fuse_bias)
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in tensors):
        cat, ws = _GeneratorConcat.apply(x, y, gen_weight, gen_bias, fuse_weight, k, dil)
        return _FuseConvOfConcat.apply(cat, ws, fuse_weight, fuse_bias)
    cat, ws = _concat_pack(x, y, gen_weight, gen_bias, fuse_weight, k, dil)
    return _fuse_conv_forward_packed(cat, ws, fuse_bias)


__all__ = [
    "fuse_conv3x3",
    "fused_ddpm",
    "fused_ddpm_supported",
    "fuse_conv_supported",
    "fused_dynamic_cat",
    "fused_generator_dynamic_cat",
    "generator_supported",
    "generator_kernels",
    "generator_kernels_supported",
]
