"""ctypes wrapper of ``ddpm_oracle.c`` (float64 numpy in, float64 numpy out).

Test infrastructure only.  Build with ``make -C oracle`` (``__graft_entry__.build``
does it).  Every function mirrors one C entry point; see that file for the
reference lines each follows.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libddpm_oracle.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        p = ctypes.c_void_p
        i = ctypes.c_int
        lib.oracle_dynamic_cat_fwd.argtypes = [p, p, p, i, i, i, i, i, i, i, i]
        lib.oracle_dynamic_cat_bwd.argtypes = [p, p, p, p, p, i, i, i, i, i, i, i, i]
        lib.oracle_generator.argtypes = [p, p, p, p, i, i, i, ctypes.c_int64]
        lib.oracle_generator_bwd.argtypes = [p, p, p, p, p, p, i, i, i, ctypes.c_int64]
        _lib = lib
    return _lib


def _f64(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float64))


def _ptr(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data)


def dynamic_cat(x, kernels, kernel_size: int, dilations=(1, 3, 5)) -> np.ndarray:
    x = _f64(x)
    k = _f64(kernels)
    n, c, h, w = x.shape
    out = np.empty((n, 4 * c, h, w), dtype=np.float64)
    _load().oracle_dynamic_cat_fwd(_ptr(x), _ptr(k), _ptr(out), n, c, h, w, kernel_size, *dilations)
    return out


def dynamic_cat_backward(x, kernels, grad_out, kernel_size: int, dilations=(1, 3, 5)):
    x = _f64(x)
    k = _f64(kernels)
    g = _f64(grad_out)
    n, c, h, w = x.shape
    dx = np.empty_like(x)
    dk = np.empty_like(k)
    _load().oracle_dynamic_cat_bwd(
        _ptr(x), _ptr(k), _ptr(g), _ptr(dx), _ptr(dk), n, c, h, w, kernel_size, *dilations
    )
    return dx, dk


def generator(y, weight, bias) -> np.ndarray:
    y = _f64(y)
    w2 = _f64(weight).reshape(weight.shape[0], -1)
    b = _f64(bias)
    n, c, h, w = y.shape
    g = w2.shape[0]
    gen = np.empty((n, g, h, w), dtype=np.float64)
    _load().oracle_generator(_ptr(y), _ptr(w2), _ptr(b), _ptr(gen), n, c, g, h * w)
    return gen


def generator_dynamic_cat(x, y, weight, bias, kernel_size: int, dilations=(1, 3, 5)):
    n, c, h, w = np.shape(x)
    gen = generator(y, weight, bias).reshape(n, 3, c, kernel_size**2, h, w)
    return dynamic_cat(x, gen, kernel_size, dilations)


def generator_dynamic_cat_backward(x, y, weight, bias, grad_out, kernel_size: int, dilations=(1, 3, 5)):
    y64 = _f64(y)
    n, c, h, w = y64.shape
    gen = generator(y64, weight, bias).reshape(n, 3, c, kernel_size**2, h, w)
    dx, dk = dynamic_cat_backward(x, gen, grad_out, kernel_size, dilations)
    w2 = _f64(weight).reshape(weight.shape[0], -1)
    g = w2.shape[0]
    dy = np.empty_like(y64)
    dw = np.empty_like(w2)
    db = np.empty(g, dtype=np.float64)
    dk = np.ascontiguousarray(dk.reshape(n, g, h, w))
    _load().oracle_generator_bwd(_ptr(y64), _ptr(w2), _ptr(dk), _ptr(dy), _ptr(dw), _ptr(db), n, c, g, h * w)
    return dx, dy, dw.reshape(np.shape(weight)), db
