"""The no-allocation dY entry point against the workspace one.

``ddpm_gen_bwd_y_noalloc`` runs the kernels of ``ddpm_gen_bwd_y`` with the
packed weight in the library's fixed device buffer instead of a caller
workspace, so its result must be bit-identical.  Two calls in a row, the
second on a smaller input (the buffer keeps the first call's contents), then
a 2-byte dtype; both entry points are called through the C-ABI.
"""

import ctypes

import pytest
import torch

from dynamicconvolutionoperator_amd import _lib
from tests.gpu_helpers import DEV, DIL, default_generator_params, randn, say

pytestmark = pytest.mark.gpu

_DT = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _bind(lib):
    return lib.ddpm_gen_bwd_y_noalloc, lib.ddpm_gen_bwd_y_noalloc_scratch_bytes


def _both(lib, noalloc, shape, k, dtype, seed):
    n, c, h, w = shape
    x = randn(shape, seed).to(dtype).to(DEV)
    go = randn((n, 4 * c, h, w), seed + 1).to(dtype).to(DEV)
    wt, _ = default_generator_params(c, k, seed + 2, dtype)
    wt = wt.reshape(3 * c * k * k, c).contiguous().to(DEV)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    dims = (n, c, h, w, k, *DIL, _DT[dtype])
    ws_bytes = int(lib.ddpm_gen_bwd_y_workspace_bytes(c, k))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    ref = torch.full_like(x, float("nan"))
    out = torch.full_like(x, float("nan"))
    rc = lib.ddpm_gen_bwd_y(_ptr(x), _ptr(wt), _ptr(go), _ptr(ref), _ptr(ws), ws_bytes, *dims, stream)
    assert rc == 0, lib.ddpm_status_string(rc)
    rc = noalloc(_ptr(x), _ptr(wt), _ptr(go), _ptr(out), *dims, stream)
    assert rc == 0, lib.ddpm_status_string(rc)
    torch.cuda.synchronize()
    return ref, out


def test_noalloc_bwd_y_matches_workspace_entry_point():
    lib = _lib.load()
    noalloc, scratch_bytes = _bind(lib)
    # the fixed buffer covers the largest packed weight the fused kernels take
    assert scratch_bytes() >= lib.ddpm_gen_bwd_y_workspace_bytes(128, 3)
    cases = [
        ((1, 128, 16, 40), 3, torch.float32),  # the largest packed weight
        ((1, 64, 48, 96), 3, torch.float32),
        ((2, 24, 15, 17), 3, torch.float32),  # smaller: the buffer holds the last call's weight
        ((1, 40, 20, 32), 1, torch.bfloat16),
    ]
    for i, (shape, k, dtype) in enumerate(cases):
        say(f"no-alloc dY call {i}: shape={shape} K={k} dtype={dtype}")
        ref, out = _both(lib, noalloc, shape, k, dtype, 600 + 10 * i)
        assert not torch.isnan(ref).any()
        assert torch.equal(out, ref), f"call {i}: max diff {(out.float() - ref.float()).abs().max().item()}"


def test_noalloc_bwd_y_validates_before_launching():
    lib = _lib.load()
    noalloc, _ = _bind(lib)
    null = None
    # even kernel size, bad dtype, null pointers: rejected on the host
    assert noalloc(null, null, null, null, 1, 8, 4, 4, 2, 1, 3, 5, 0, null) == 10001
    assert noalloc(null, null, null, null, 1, 8, 4, 4, 3, 1, 3, 5, 7, null) == 10001
    assert noalloc(null, null, null, null, 1, 8, 4, 4, 3, 1, 3, 5, 0, null) == 10001
    # an empty batch is a no-op
    assert noalloc(null, null, null, null, 0, 8, 4, 4, 3, 1, 3, 5, 0, null) == 0
