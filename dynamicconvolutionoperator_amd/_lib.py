"""ctypes binding of ``libddpm_hip.so`` (the C-ABI declared in include/ddpm_hip.h).

The library is built in-tree by ``dynamicconvolutionoperator_amd.build``.  It
is loaded after ``torch`` so that it binds to the HIP runtime torch already
loaded (both carry the soname ``libamdhip64.so.7``); pointers and streams
passed from torch are then valid in the library.

There is no silent fallback: :func:`load` raises :class:`HipLibraryError`
when the library is missing or does not load, and GPU callers let it
propagate.
"""

from __future__ import annotations

import ctypes
import functools
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libddpm_hip.so")

# C-ABI symbols and their signatures (argument types, result type).
_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_FILTER_ARGS = [_P, _P, _P, _L, _L, _L, _L, _I, _I, _I, _I, _I, _I, _P]
SIGNATURES: dict[str, tuple[list, type]] = {
    "ddpm_abi_version": ([], _I),
    "ddpm_status_string": ([_I], ctypes.c_char_p),
    "ddpm_gen_supported": ([_L, _I, _I], _I),
    "ddpm_gen_fwd_supported": ([_L, _I, _I], _I),
    "ddpm_gen_kernels_supported": ([_L, _L, _L, _L, _I, _I], _I),
    "ddpm_gen_kernels": ([_P, _P, _P, _P, _L, _L, _L, _L, _I, _I, _P], _I),
    "ddpm_gen_kernels_bwd_w_workspace_bytes": ([_L, _L, _L, _L, _I], _L),
    "ddpm_gen_kernels_bwd_y_workspace_bytes": ([_L, _L, _L, _L, _I], _L),
    "ddpm_gen_kernels_bwd_y": ([_P, _P, _P, _P, _L, _L, _L, _L, _L, _I, _I, _P], _I),
    "ddpm_gen_kernels_bwd_w": ([_P, _P, _P, _P, _P, _L, _L, _L, _L, _L, _I, _I, _P], _I),
    "ddpm_filter_fwd": (_FILTER_ARGS, _I),
    "ddpm_filter_bwd_x": (_FILTER_ARGS, _I),
    "ddpm_filter_bwd_k": (_FILTER_ARGS, _I),
    "ddpm_gen_fwd": ([_P, _P, _P, _P, _P, _L, _L, _L, _L, _I, _I, _I, _I, _I, _P], _I),
    "ddpm_gen_bwd_x_workspace_bytes": ([_L, _L, _L, _L, _I, _I, _I, _I], _L),
    "ddpm_gen_bwd_x": ([_P, _P, _P, _P, _P, _P, _L, _L, _L, _L, _L, _I, _I, _I, _I, _I, _P], _I),
    "ddpm_gen_bwd_y_workspace_bytes": ([_L, _I], _L),
    "ddpm_gen_bwd_y": ([_P, _P, _P, _P, _P, _L, _L, _L, _L, _L, _I, _I, _I, _I, _I, _P], _I),
    "ddpm_gen_bwd_y_noalloc": ([_P, _P, _P, _P, _L, _L, _L, _L, _I, _I, _I, _I, _I, _P], _I),
    "ddpm_gen_bwd_y_noalloc_scratch_bytes": ([], _L),
    "ddpm_gen_bwd_w_workspace_bytes": ([_L, _L, _L, _L, _I, _I], _L),
    "ddpm_fuse_conv_workspace_bytes": ([_L, _L, _L, _L, _I], _L),
    "ddpm_fuse_conv_fwd": ([_P, _P, _P, _P, _P, _L, _L, _L, _L, _L, _I, _P], _I),
    "ddpm_fuse_conv_bwd_data": ([_P, _P, _P, _P, _L, _L, _L, _L, _L, _I, _P], _I),
    "ddpm_fuse_conv_bwd_weight_workspace_bytes": ([_L, _L, _L, _L, _I], _L),
    "ddpm_fuse_conv_bwd_weight": ([_P, _P, _P, _P, _P, _L, _L, _L, _L, _L, _I, _P], _I),
    "ddpm_fuse_conv_bwd": ([_P, _P, _P, _P, _P, _P, _P, _L, _P, _L, _L, _L, _L, _L, _I, _P], _I),
    "ddpm_gen_fwd_pack": ([_P, _P, _P, _P, _P, _P, _P, _L, _L, _L, _L, _L, _I, _I, _I, _I, _I, _P],
                          _I),
    "ddpm_fuse_conv_fwd_packed": ([_P, _P, _P, _P, _L, _L, _L, _L, _L, _I, _P], _I),
    "ddpm_gen_bwd_w": ([_P, _P, _P, _P, _P, _P, _L, _L, _L, _L, _L, _I, _I, _I, _I, _I, _P], _I),
    "ddpm_gen_bwd_xw": ([_P, _P, _P, _P, _P, _P, _P, _P, _P, _L, _P, _L, _L, _L, _L, _L, _I, _I, _I,
                         _I, _I, _P], _I),
    "ddpm_gen_bwd": ([_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _L, _P, _L, _P, _L, _L, _L, _L, _L, _I,
                      _I, _I, _I, _I, _P], _I),
}


ABI_VERSION = 7  # include/ddpm_hip.h


class HipLibraryError(RuntimeError):
    """The HIP library is missing or failed to load."""


@functools.lru_cache(maxsize=1)
def load() -> ctypes.CDLL:
    """Load and bind ``libddpm_hip.so``; raise :class:`HipLibraryError` if impossible."""
    import torch  # noqa: F401  (binds the library to torch's HIP runtime)

    if not os.path.exists(LIB_PATH):
        raise HipLibraryError(
            f"{LIB_PATH} is not built; run `python -m dynamicconvolutionoperator_amd.build`"
        )
    try:
        lib = ctypes.CDLL(LIB_PATH)
    except OSError as exc:  # pragma: no cover - depends on the environment
        raise HipLibraryError(f"failed to load {LIB_PATH}: {exc}") from exc
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    if lib.ddpm_abi_version() != ABI_VERSION:
        raise HipLibraryError("libddpm_hip.so ABI version mismatch; rebuild it")
    return lib


def available() -> bool:
    try:
        load()
        return True
    except HipLibraryError:
        return False


STATUS_UNSUPPORTED = 10002


def check(code: int, what: str) -> None:
    """Raise on a non-zero status from a C-ABI call."""
    if code != 0:
        msg = load().ddpm_status_string(code).decode()
        if code in (10001,):
            raise ValueError(f"{what}: {msg}")
        raise RuntimeError(f"{what} failed (status {code}): {msg}")
