"""Write integer known-answer vectors for the DDPM path into ``ddpm_kat.json``.

Self-contained on purpose: it imports neither torch, the oracle, nor the
product.  Each expected value is computed by plain nested loops straight from
the definition (unfold_impl.py:15-42; backward by the chain rule):

  gen[n][o][h][w]  = sum_i W[o][i] * y[n][i][h][w] + b[o],  o = (b*C + c)*K*K + ki*K + kj
  out_b[n][c][h][w] = sum_{ki,kj} k[n][b][c][ki*K+kj][h][w] * x[n][c][h+(ki-r)d_b][w+(kj-r)d_b]
                      (zero outside the image), cat = [x, out_0, out_1, out_2]
  dK[n][b][c][t][h][w] = g_b[n][c][h][w] * x[n][c][h+(ki-r)d][w+(kj-r)d]
  dX[n][c][q] = g_x[n][c][q] + sum_{b,t} k[n][b][c][t][q-off] * g_b[n][c][q-off]
  dY = W^T dK, dW = sum dK y^T, db = sum dK

Inputs are small integers, so every expected value is an exact integer in
float32: a test may compare with zero tolerance.  Cases are non-square, use
C>1 and N>1 so that transposed taps, swapped branch/channel order in the
generator rows, a wrong dilation sign or a missing boundary zero each change
the answer.

Run:  python tests/golden/make_golden.py   (rewrites ddpm_kat.json)
"""

from __future__ import annotations

import json
import os
import random

DIL = (1, 3, 5)


def rnd_ints(rng, shape, lo, hi):
    if len(shape) == 1:
        return [rng.randint(lo, hi) for _ in range(shape[0])]
    return [rnd_ints(rng, shape[1:], lo, hi) for _ in range(shape[0])]


def zeros(shape):
    if len(shape) == 1:
        return [0] * shape[0]
    return [zeros(shape[1:]) for _ in range(shape[0])]


def filter_fwd(x, k, K):
    N, C, H, W = len(x), len(x[0]), len(x[0][0]), len(x[0][0][0])
    r = K // 2
    out = zeros((N, 4 * C, H, W))
    for n in range(N):
        for c in range(C):
            for h in range(H):
                for w in range(W):
                    out[n][c][h][w] = x[n][c][h][w]
            for b, d in enumerate(DIL):
                for h in range(H):
                    for w in range(W):
                        acc = 0
                        for ki in range(K):
                            for kj in range(K):
                                hh, ww = h + (ki - r) * d, w + (kj - r) * d
                                if 0 <= hh < H and 0 <= ww < W:
                                    acc += k[n][b][c][ki * K + kj][h][w] * x[n][c][hh][ww]
                        out[n][(b + 1) * C + c][h][w] = acc
    return out


def filter_bwd(x, k, g, K):
    N, C, H, W = len(x), len(x[0]), len(x[0][0]), len(x[0][0][0])
    r = K // 2
    dx = [[[list(g[n][c][h]) for h in range(H)] for c in range(C)] for n in range(N)]
    dk = zeros((N, 3, C, K * K, H, W))
    for n in range(N):
        for b, d in enumerate(DIL):
            for c in range(C):
                gb = g[n][(b + 1) * C + c]
                for h in range(H):
                    for w in range(W):
                        for ki in range(K):
                            for kj in range(K):
                                hh, ww = h + (ki - r) * d, w + (kj - r) * d
                                if 0 <= hh < H and 0 <= ww < W:
                                    t = ki * K + kj
                                    dk[n][b][c][t][h][w] = gb[h][w] * x[n][c][hh][ww]
                                    dx[n][c][hh][ww] += k[n][b][c][t][h][w] * gb[h][w]
    return dx, dk


def generator(y, wt, bias, K):
    N, C, H, W = len(y), len(y[0]), len(y[0][0]), len(y[0][0][0])
    KK = K * K
    k = zeros((N, 3, C, KK, H, W))
    for n in range(N):
        for b in range(3):
            for c in range(C):
                for t in range(KK):
                    o = (b * C + c) * KK + t
                    for h in range(H):
                        for w in range(W):
                            k[n][b][c][t][h][w] = bias[o] + sum(
                                wt[o][i] * y[n][i][h][w] for i in range(C)
                            )
    return k


def generator_bwd(y, wt, dk, K):
    N, C, H, W = len(y), len(y[0]), len(y[0][0]), len(y[0][0][0])
    KK = K * K
    G = 3 * C * KK
    dy = zeros((N, C, H, W))
    dw = zeros((G, C))
    db = [0] * G
    for n in range(N):
        for b in range(3):
            for c in range(C):
                for t in range(KK):
                    o = (b * C + c) * KK + t
                    for h in range(H):
                        for w in range(W):
                            v = dk[n][b][c][t][h][w]
                            db[o] += v
                            for i in range(C):
                                dw[o][i] += v * y[n][i][h][w]
                                dy[n][i][h][w] += wt[o][i] * v
    return dy, dw, db


def filter_case(seed, N, C, H, W, K):
    rng = random.Random(seed)
    x = rnd_ints(rng, (N, C, H, W), -4, 4)
    k = rnd_ints(rng, (N, 3, C, K * K, H, W), -3, 3)
    g = rnd_ints(rng, (N, 4 * C, H, W), -3, 3)
    out = filter_fwd(x, k, K)
    dx, dk = filter_bwd(x, k, g, K)
    return {
        "kind": "filter", "N": N, "C": C, "H": H, "W": W, "K": K, "dilations": list(DIL),
        "x": x, "kernels": k, "grad_out": g, "out": out, "grad_x": dx, "grad_kernels": dk,
    }


def generator_case(seed, N, C, H, W, K):
    rng = random.Random(seed)
    G = 3 * C * K * K
    x = rnd_ints(rng, (N, C, H, W), -3, 3)
    y = rnd_ints(rng, (N, C, H, W), -2, 2)
    wt = rnd_ints(rng, (G, C), -2, 2)
    bias = rnd_ints(rng, (G,), -2, 2)
    g = rnd_ints(rng, (N, 4 * C, H, W), -2, 2)
    k = generator(y, wt, bias, K)
    out = filter_fwd(x, k, K)
    dx, dk = filter_bwd(x, k, g, K)
    dy, dw, db = generator_bwd(y, wt, dk, K)
    return {
        "kind": "generator", "N": N, "C": C, "H": H, "W": W, "K": K, "dilations": list(DIL),
        "x": x, "y": y, "weight": wt, "bias": bias, "grad_out": g, "out": out,
        "grad_x": dx, "grad_y": dy, "grad_weight": dw, "grad_bias": db,
    }


def main():
    cases = [
        filter_case(11, 1, 2, 5, 7, 3),
        filter_case(12, 2, 1, 3, 4, 1),
        filter_case(13, 1, 1, 6, 11, 5),
        generator_case(21, 1, 2, 4, 6, 3),
        generator_case(22, 2, 3, 3, 5, 1),
        generator_case(23, 1, 2, 7, 6, 3),
    ]
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ddpm_kat.json")
    with open(path, "w") as f:
        json.dump({"generated_by": "tests/golden/make_golden.py", "cases": cases}, f, separators=(",", ":"))
    print(f"wrote {len(cases)} cases to {path}")


if __name__ == "__main__":
    main()
