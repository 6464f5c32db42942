"""ddpm_gen_bwd_xw against ddpm_gen_bwd_x + ddpm_gen_bwd_w, through the C-ABI.

The combined entry point runs the same kernels -- the dX tile kernel, the
weight-gradient partial kernel and its split reduction -- but performs dX's
halo reduction in helper workgroups of the weight-gradient launch (on the
CUs its at most 16 x 3 x channel-block workgroups leave free), or as its own
kernel where fewer than a quarter of the CUs are free.  Every result must be
bit-identical to the two separate calls.  Shapes: 256x256 C=64 (64 helper
workgroups), C=16 (most of the grid is helpers), C=128 (two input-channel
halves fill the CUs: separate reduction kernel), W % 4 != 0 (one column per
item), K=1 (256-thread workgroups), and an empty batch.
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


def _run(shape, k, dtype, seed):
    lib = _lib.load()
    n, c, h, w = shape
    dt = _DT[dtype]
    x = randn(shape, seed).to(dtype).to(DEV)
    y = randn(shape, seed + 1).to(dtype).to(DEV)
    wt, b = default_generator_params(c, k, seed + 2, dtype)
    wt, b = wt.to(DEV), b.to(DEV)
    g = randn((n, 4 * c, h, w), seed + 3).to(dtype).to(DEV)
    wsx_bytes = int(lib.ddpm_gen_bwd_x_workspace_bytes(n, c, h, w, k, *DIL))
    ws_bytes = int(lib.ddpm_gen_bwd_w_workspace_bytes(n, c, h, w, k, dt))
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    outs = []
    for combined in (False, True):
        gx = torch.full_like(x, float("nan"))
        gw = torch.full_like(wt, float("nan"))
        gb = torch.full_like(b, float("nan"))
        wsx = torch.empty(max(wsx_bytes, 16), dtype=torch.uint8, device=DEV)
        ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=DEV)
        if combined:
            rc = lib.ddpm_gen_bwd_xw(_ptr(x), _ptr(y), _ptr(wt), _ptr(b), _ptr(g), _ptr(gx), _ptr(gw),
                                     _ptr(gb), _ptr(wsx), wsx_bytes, _ptr(ws), ws_bytes, n, c, h, w, k,
                                     *DIL, dt, stream)
            assert rc == 0, lib.ddpm_status_string(rc).decode()
        else:
            rc = lib.ddpm_gen_bwd_x(_ptr(y), _ptr(wt), _ptr(b), _ptr(g), _ptr(gx), _ptr(wsx), wsx_bytes,
                                    n, c, h, w, k, *DIL, dt, stream)
            assert rc == 0, rc
            rc = lib.ddpm_gen_bwd_w(_ptr(x), _ptr(y), _ptr(g), _ptr(gw), _ptr(gb), _ptr(ws), ws_bytes,
                                    n, c, h, w, k, *DIL, dt, stream)
            assert rc == 0, rc
        torch.cuda.synchronize()
        outs.append((gx, gw, gb))
    return outs


@pytest.mark.parametrize(
    "shape,k,dtype",
    [
        ((1, 64, 256, 256), 3, torch.float32),
        ((1, 64, 256, 256), 3, torch.bfloat16),
        ((2, 16, 20, 36), 3, torch.float32),
        ((1, 128, 24, 40), 3, torch.bfloat16),
        ((1, 24, 15, 17), 3, torch.float32),
        ((1, 32, 40, 56), 1, torch.bfloat16),
    ],
)
def test_bwd_xw_matches_separate_calls(shape, k, dtype):
    say(f"bwd_xw shape={shape} K={k} {dtype}")
    (sx, sw, sb), (cx, cw, cb) = _run(shape, k, dtype, 1200 + shape[1] + shape[3])
    for name, a, e in (("dx", cx, sx), ("dw", cw, sw), ("db", cb, sb)):
        assert not torch.isnan(e).any(), f"{name}: separate calls left unwritten entries"
        assert torch.equal(a, e), f"{name}: max|diff| {(a.float() - e.float()).abs().max().item():.3e}"


def test_bwd_xw_empty_batch_launches_nothing():
    say("bwd_xw empty batch")
    lib = _lib.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    null = ctypes.c_void_p(0)
    rc = lib.ddpm_gen_bwd_xw(null, null, null, null, null, null, null, null, null, 0, null, 0,
                             0, 16, 8, 8, 3, *DIL, 0, stream)
    assert rc == 0
