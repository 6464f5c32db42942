#!/usr/bin/env python3
"""Benchmark of the DDPM hot path on one MI355X.

Headline workload (``value``): one fused recompute training step of the
drop-in DDPM module -- forward and backward of ``module(x, y).square().mean()``
-- at B=1, C=64, K=3, H=W=256, fp32, synthetic N(0,1) inputs and seeded
default-init weights.  This is the configuration on which the reference
quotes its absolute fused training time (3.66 ms on an RTX 5090,
README.md:161-162).

Also reported on the same line: bf16 training, fused inference (fp32/bf16),
the materialized dynamic filter's HBM bandwidth at 256x256 (the
"dyn-filter HBM TB/s" part of the metric), peak temporary memory of the fused
step vs the Unfold route, the Unfold route's GPU step time, a roofline entry
for the dominant HIP kernel of the step (HIP events around each launch on its
stream, inside the timed region) and a CPU baseline (the Unfold oracle
restatement timed on the host cores).

Usage: python bench.py [--gpus 1] [--steps 50] [--warmup 10]
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

METRIC = "DDPM fwd & fwd+bwd ms, B1 C64 K3 256² fp32/bf16; dyn-filter HBM TB/s"
REFERENCE_TRAIN_MS = 3.66  # fused training step, 256x256 fp32, RTX 5090 (README.md:161-162)
HBM_PEAK_GBS = 8000.0
BF16_DENSE_TFLOPS = 2500.0
B, C, K, H, W = 1, 64, 3, 256, 256
DIL = (1, 3, 5)


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--quick", action="store_true", help="skip the secondary measurements")
    p.add_argument(
        "--kernel",
        help="comma-separated C-ABI entry points (or 'copy') to run alone at the headline "
        "shape, for rocprofv3 counter runs; no timing line is printed",
    )
    p.add_argument("--dtype", choices=("f32", "bf16"), default="f32", help="with --kernel")
    p.add_argument("--reps", type=int, default=3, help="launches per entry point with --kernel")
    return p.parse_args()


# --------------------------------------------------------------------------- helpers
def make_inputs(dtype, seed=21, grad=True):
    import torch

    torch.manual_seed(seed)
    x = torch.randn(B, C, H, W, device="cuda", dtype=dtype, requires_grad=grad)
    y = torch.randn(B, C, H, W, device="cuda", dtype=dtype, requires_grad=grad)
    return x, y


def make_module(dtype, fused=True):
    import torch

    from dynamicconvolutionoperator_amd import DDPM

    torch.manual_seed(21)
    return DDPM(C, K, fused_generator_training=fused).cuda().to(dtype).train()


def train_step(module, x, y):
    module.zero_grad(set_to_none=True)
    x.grad = None
    y.grad = None
    module(x, y).square().mean().backward()


def progress(msg):
    """One line per finished measurement on stderr (stdout carries only the JSON line)."""
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_loop(fn, steps, warmup):
    """Mean ms per call: warmup, sync, then `steps` calls bracketed by syncs."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


class LaunchTimer:
    """Brackets every call of the named C-ABI entry points with HIP events.

    Every entry point takes the stream it launches on as its last argument
    (the operators pass the current stream); the events are recorded on that
    stream, so each (start, end) pair spans exactly that entry point's
    kernels, also for a caller that launches on a stream of its own.
    """

    def __init__(self, lib, names):
        import torch

        self.torch = torch
        self.records = {n: [] for n in names}
        self.active = False
        self.streams = {}
        for name in names:
            real = getattr(lib, name)

            def wrapper(*args, _real=real, _name=name):
                if not self.active:
                    return _real(*args)
                stream = self._stream(args[-1])
                start = torch.cuda.Event(enable_timing=True)
                end = torch.cuda.Event(enable_timing=True)
                start.record(stream)
                rc = _real(*args)
                end.record(stream)
                self.records[_name].append((start, end))
                return rc

            setattr(lib, name, wrapper)

    def _stream(self, handle):
        """torch stream object for a raw hipStream_t argument."""
        ptr = handle.value if hasattr(handle, "value") else handle
        ptr = int(ptr or 0)
        stream = self.streams.get(ptr)
        if stream is None:
            current = self.torch.cuda.current_stream()
            if ptr == current.cuda_stream:
                stream = current
            else:
                stream = self.torch.cuda.ExternalStream(ptr)
            self.streams[ptr] = stream
        return stream

    def mean_ms(self):
        out = {}
        for name, recs in self.records.items():
            if recs:
                out[name] = sum(s.elapsed_time(e) for s, e in recs) / len(recs)
        return out

    def counts(self):
        return {n: len(r) for n, r in self.records.items() if r}


def work_per_launch(name, esize):
    """Algorithmic work of one launch at the headline shape: (bytes, flops)."""
    E = B * C * H * W
    G = 3 * C * K * K
    gemm = 2.0 * B * H * W * C * G  # the generator contraction C -> 3CK^2
    table = {
        "ddpm_gen_fwd": ((6 * E + G * (C + 1)) * esize, gemm),  # x, y in; cat (4E) out
        "ddpm_gen_bwd_x": ((6 * E + G * (C + 1)) * esize, gemm),  # y, gO (4E) in; dX out
        "ddpm_gen_bwd_y": ((5 * E + G * C) * esize, gemm),  # x, gO branches (3E) in; dY out
        "ddpm_gen_bwd_w": ((5 * E) * esize + G * (C + 1) * esize, gemm),  # x, y, gO branches in
        "ddpm_filter_fwd": ((3 * K * K + 5) * E * esize, 0.0),
        "ddpm_filter_bwd_x": ((3 * K * K + 5) * E * esize, 0.0),
        "ddpm_filter_bwd_k": ((3 * K * K + 4) * E * esize, 0.0),
    }
    return table[name]


def load_traffic(kernel_entry, dtype_name):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE),
    committed under profiles/; None when no measurement exists."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    try:
        with open(path) as f:
            data = json.load(f)
        return data[f"{kernel_entry}:{dtype_name}"]["hbm_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


# --------------------------------------------------------------------------- measurements
def filter_bandwidth(dtype, repeats=30):
    """Materialized dynamic filter forward at 256x256, rotating two buffer sets
    (2 x 537 MB for fp32) so repeats do not run out of the 256 MB MALL."""
    import torch

    from dynamicconvolutionoperator_amd import ops

    sets = []
    for s in range(2):
        g = torch.Generator(device="cuda").manual_seed(10 + s)
        x = torch.randn(B, C, H, W, device="cuda", dtype=dtype, generator=g)
        k = torch.randn(B, 3, C, K * K, H, W, device="cuda", dtype=dtype, generator=g)
        sets.append((x, k))
    with torch.inference_mode():
        for i in range(4):
            ops.fused_dynamic_cat(*sets[i % 2], K, DIL)
        torch.cuda.synchronize()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(repeats)]
        for i in range(repeats):
            ev[i][0].record()
            ops.fused_dynamic_cat(*sets[i % 2], K, DIL)
            ev[i][1].record()
        torch.cuda.synchronize()
    ms = sum(s.elapsed_time(e) for s, e in ev) / repeats
    esize = torch.empty((), dtype=dtype).element_size()
    nbytes = (3 * K * K + 5) * B * C * H * W * esize
    del sets
    torch.cuda.empty_cache()
    return {"ms": ms, "bytes": nbytes, "GB/s": nbytes / ms / 1e6, "frac_of_8TBps": nbytes / ms / 1e6 / HBM_PEAK_GBS}


def unfold_route_step(params, x, y):
    """The reference's Unfold route (unfold_impl.py:21-42) with the module's
    parameters, used here only as the GPU memory/time baseline."""
    import torch
    import torch.nn.functional as F

    gw, gb, fw, fb = params
    n, c, h, w = x.shape
    kernels = F.conv2d(y, gw, gb).reshape(n, 3, c, K * K, h, w)
    outs = [x]
    for b, d in enumerate(DIL):
        cols = F.unfold(x, K, dilation=d, padding=K // 2 * d).reshape(n, c, K * K, h, w)
        outs.append((cols * kernels[:, b]).sum(2))
    return F.conv2d(torch.cat(outs, 1), fw, fb, padding=1)


def peak_temp_mib(step):
    import torch

    for _ in range(2):
        step()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    step()
    torch.cuda.synchronize()
    return (torch.cuda.max_memory_allocated() - base) / 2**20


def cpu_baseline(budget_s=20.0):
    """The Unfold oracle restatement (fp32, torch on the host cores) running the
    same training step; a bounded number of steps (about `budget_s` seconds)."""
    import torch

    from oracle.unfold_ref import UnfoldDDPM

    # the host's CPU share: OMP_NUM_THREADS when the environment sets it
    threads = int(os.environ.get("OMP_NUM_THREADS") or 0) or os.cpu_count() or 1
    torch.set_num_threads(threads)
    torch.manual_seed(21)
    model = UnfoldDDPM(C, K).train()
    x = torch.randn(B, C, H, W, requires_grad=True)
    y = torch.randn(B, C, H, W, requires_grad=True)

    def step():
        model.zero_grad(set_to_none=True)
        x.grad = None
        y.grad = None
        model(x, y).square().mean().backward()

    t0 = time.perf_counter()
    step()  # warm-up (allocations, oneDNN primitive creation)
    first = time.perf_counter() - t0
    n = max(1, min(20, int(budget_s / max(first, 1e-3))))
    t0 = time.perf_counter()
    for _ in range(n):
        step()
    ms = (time.perf_counter() - t0) * 1e3 / n
    cpu = platform.processor() or "cpu"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": ms,
        "unit": "ms per training step",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"{n} timed steps (after 1 warm-up) of the full B1 C64 K3 256x256 fp32 "
        f"Unfold-route training step on {cpu}",
    }


# --------------------------------------------------------------------------- kernel mode
COPY_BYTES = 2**30  # 'copy': a plain 1 GiB device copy (4x the MALL; reads and writes this many bytes)


def kernel_mode(args):
    """Launches the named entry points `reps` times each at B1 C64 K3 256x256
    (dilations 1/3/5) on seeded inputs, and 'copy' as a plain device copy of
    COPY_BYTES, so that rocprofv3 --pmc can read each kernel's HBM counters
    (FETCH_SIZE / WRITE_SIZE) and the copy calibrates them."""
    import ctypes

    import torch

    from dynamicconvolutionoperator_amd import _lib

    lib = _lib.load()
    dt = {"f32": torch.float32, "bf16": torch.bfloat16}[args.dtype]
    code = 0 if dt == torch.float32 else 1
    ptr = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    g = torch.Generator(device="cuda").manual_seed(1)
    rnd = lambda *shape: torch.randn(*shape, device="cuda", generator=g).to(dt)  # noqa: E731
    x, y = rnd(B, C, H, W), rnd(B, C, H, W)
    go = rnd(B, 4 * C, H, W)
    wt, bs = rnd(3 * C * K * K, C) * 0.1, rnd(3 * C * K * K) * 0.1
    kern = rnd(B, 3, C, K * K, H, W)
    out = torch.empty(B, 4 * C, H, W, device="cuda", dtype=dt)
    dx, dy, dk = torch.empty_like(x), torch.empty_like(y), torch.empty_like(kern)
    dw, db = torch.empty_like(wt), torch.empty_like(bs)
    wsb = max(int(lib.ddpm_gen_bwd_w_workspace_bytes(B, C, H, W, K)),
              int(lib.ddpm_gen_bwd_y_workspace_bytes(C, K)),
              int(lib.ddpm_gen_bwd_x_workspace_bytes(B, C, H, W, K, *DIL)), 1)
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    shp = (B, C, H, W, K, *DIL)
    calls = {
        "ddpm_gen_fwd": lambda: lib.ddpm_gen_fwd(ptr(x), ptr(y), ptr(wt), ptr(bs), ptr(out), *shp, code, s),
        "ddpm_gen_bwd_x": lambda: lib.ddpm_gen_bwd_x(ptr(y), ptr(wt), ptr(bs), ptr(go), ptr(dx), ptr(ws), wsb,
                                                     *shp, code, s),
        "ddpm_gen_bwd_y": lambda: lib.ddpm_gen_bwd_y(ptr(x), ptr(wt), ptr(go), ptr(dy), ptr(ws), wsb, *shp,
                                                     code, s),
        "ddpm_gen_bwd_w": lambda: lib.ddpm_gen_bwd_w(ptr(x), ptr(y), ptr(go), ptr(dw), ptr(db), ptr(ws), wsb,
                                                     *shp, code, s),
        "ddpm_filter_fwd": lambda: lib.ddpm_filter_fwd(ptr(x), ptr(kern), ptr(out), *shp, code, code, s),
        "ddpm_filter_bwd_x": lambda: lib.ddpm_filter_bwd_x(ptr(go), ptr(kern), ptr(dx), *shp, code, code, s),
        "ddpm_filter_bwd_k": lambda: lib.ddpm_filter_bwd_k(ptr(x), ptr(go), ptr(dk), *shp, code, code, s),
        "copy": lambda: (dst.copy_(src), 0)[1],
    }
    names = args.kernel.split(",")
    for name in names:
        if name not in calls:
            raise SystemExit(f"unknown --kernel {name}; choose from {', '.join(calls)}")
    for name in names:
        for _ in range(args.reps):
            rc = calls[name]()
            if rc:
                raise SystemExit(f"{name} failed with status {rc}")
        torch.cuda.synchronize()
        print(f"ran {name} x{args.reps} ({args.dtype})", flush=True)


# --------------------------------------------------------------------------- main
def main():
    args = parse_args()
    if args.gpus != 1:
        print(
            f"bench.py runs on one GPU only (got --gpus {args.gpus}); the DDPM hot path has no "
            "multi-GPU component in this build.",
            file=sys.stderr,
        )
        sys.exit(2)

    import torch

    from dynamicconvolutionoperator_amd import _lib

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    if args.kernel:
        kernel_mode(args)
        return
    lib = _lib.load()
    entries = [n for n in _lib.SIGNATURES if n.startswith(("ddpm_gen_fwd", "ddpm_gen_bwd_x", "ddpm_gen_bwd_y", "ddpm_gen_bwd_w", "ddpm_filter_"))]
    entries = [n for n in entries if not n.endswith("_workspace_bytes")]
    timer = LaunchTimer(lib, entries)

    # ---- headline: fp32 fused recompute training step
    module = make_module(torch.float32)
    x, y = make_inputs(torch.float32)
    for _ in range(args.warmup):
        train_step(module, x, y)
    torch.cuda.synchronize()
    timer.active = True
    t0 = time.perf_counter()
    for _ in range(args.steps):
        train_step(module, x, y)
    torch.cuda.synchronize()
    train_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    timer.active = False
    per_entry = timer.mean_ms()
    counts = timer.counts()
    step_share = {n: per_entry[n] * counts[n] / args.steps for n in per_entry}
    dominant = max(step_share, key=step_share.get)
    nbytes, flops = work_per_launch(dominant, 4)
    dom_ms = per_entry[dominant]
    if flops > 0:
        # fp32 operands run as three bf16 MFMA products: ceiling = bf16 dense peak / 3
        peak = BF16_DENSE_TFLOPS / 3.0
        achieved = flops / dom_ms / 1e9
        roofline = {"bound": "mfma", "achieved": achieved, "peak": peak, "unit": "TFLOP/s",
                    "frac": achieved / peak}
    else:
        achieved = nbytes / dom_ms / 1e6
        roofline = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": achieved / HBM_PEAK_GBS}
    roofline.update({
        "traffic": load_traffic(dominant, "f32"),
        "kernel": dominant,
        "kernel_ms": dom_ms,
        "algorithmic_bytes": nbytes,
        "algorithmic_flops": flops,
        "hbm_GB/s_algorithmic": nbytes / dom_ms / 1e6,
    })
    kernels = {
        n: {"ms": per_entry[n], "launches_per_step": counts[n] // args.steps,
            "share_of_step_ms": step_share[n]}
        for n in per_entry
    }
    del module, x, y
    torch.cuda.empty_cache()
    progress(f"fp32 training step {train_ms:.3f} ms")

    extra = {"kernels_fp32_train": kernels}
    if not args.quick:
        # ---- bf16 training, inference
        module = make_module(torch.bfloat16)
        x, y = make_inputs(torch.bfloat16)
        extra["train_ms_bf16"] = time_loop(lambda: train_step(module, x, y), args.steps, args.warmup)
        module.eval()
        with torch.inference_mode():
            extra["infer_ms_bf16"] = time_loop(lambda: module(x, y), args.steps, args.warmup)
        del module, x, y
        module = make_module(torch.float32).eval()
        x, y = make_inputs(torch.float32, grad=False)
        with torch.inference_mode():
            extra["infer_ms_fp32"] = time_loop(lambda: module(x, y), args.steps, args.warmup)
        del module, x, y
        torch.cuda.empty_cache()

        progress("bf16 training and inference done")
        # ---- dynamic filter bandwidth (materialized path)
        extra["filter_fwd_fp32"] = filter_bandwidth(torch.float32)
        extra["filter_fwd_bf16"] = filter_bandwidth(torch.bfloat16)

        progress("filter bandwidth done")
        # ---- peak temporary memory and Unfold-route time (GPU)
        for name, dtype in (("fp32", torch.float32), ("bf16", torch.bfloat16)):
            module = make_module(dtype)
            x, y = make_inputs(dtype)
            fused_mib = peak_temp_mib(lambda: train_step(module, x, y))
            params = [p for p in module.parameters()]

            def unfold_step():
                for p in params:
                    p.grad = None
                x.grad = None
                y.grad = None
                unfold_route_step(params, x, y).square().mean().backward()

            unfold_mib = peak_temp_mib(unfold_step)
            extra[f"peak_temp_mib_{name}"] = {"fused": fused_mib, "unfold": unfold_mib,
                                              "fused_over_unfold": fused_mib / unfold_mib}
            extra[f"unfold_route_train_ms_{name}"] = time_loop(unfold_step, 10, 3)
            del module, x, y, params
            torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu_baseline:
        progress("CPU baseline (about 20 s)")
        cpu = cpu_baseline()

    result = {
        "metric": METRIC,
        "value": train_ms,
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": train_ms,
        "higher_is_better": False,
        "scaling": "weak",
        # time-like metric: value / reference (RTX 5090, README.md:161-162); < 1 is faster
        "vs_baseline": train_ms / REFERENCE_TRAIN_MS,
        "dtype": "f32",
        "data": "synthetic N(0,1) inputs, seeded default-init weights",
        "config": {
            "workload": "DDPM fused recompute training step (fwd+bwd of out.square().mean()), "
            "B1 C64 K3 256x256, dilations 1/3/5",
            "global_batch": B,
            "channels": C,
            "kernel_size": K,
            "height": H,
            "width": W,
            "route": "fused generator (HIP) + 3x3 fuse conv (MIOpen)",
            "parallelism": "single GPU",
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
        "device": torch.cuda.get_device_name(0),
        "extra": extra,
    }
    print(json.dumps(result))


if __name__ == "__main__":
    main()
