/*
 * Loop-level double-precision restatement of the DDPM hot path.
 *
 * Test infrastructure only: the reference the HIP kernels are tested against,
 * and a second, independent restatement that pins the torch Unfold oracle.  Nothing in the
 * product library links or loads this file.
 *
 * Layouts (all contiguous, NCHW-style):
 *   x, y      [N][C][H][W]
 *   kernels   [N][3][C][K*K][H][W]                  (unfold_impl.py:23)
 *   weight    [3*C*K*K][C]  row o = (b*C + c)*K*K + tap, tap = ki*K + kj
 *   bias      [3*C*K*K]
 *   cat       [N][4*C][H][W] = [x, d1, d3, d5]      (unfold_impl.py:29)
 * Neighbour of (h,w) for tap (ki,kj) at dilation d: (h+(ki-r)d, w+(kj-r)d),
 * r = K/2, zero outside the image (unfold padding K//2*d, unfold_impl.py:35-37).
 */
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#define IDX4(n, c, h, w, C, H, W) ((((int64_t)(n) * (C) + (c)) * (H) + (h)) * (W) + (w))

static int dil_of(int b, int d0, int d1, int d2) { return b == 0 ? d0 : (b == 1 ? d1 : d2); }

/* unfold_impl.py:35-42 (DepthDCOp.forward) for the three dilations + concat. */
void oracle_dynamic_cat_fwd(const double* x, const double* k, double* out, int N, int C, int H,
                            int W, int K, int d0, int d1, int d2) {
  const int r = K / 2, KK = K * K;
  const int64_t HW = (int64_t)H * W;
#pragma omp parallel for collapse(2) schedule(static)
  for (int n = 0; n < N; ++n)
    for (int c = 0; c < C; ++c) {
      const double* xp = x + ((int64_t)n * C + c) * HW;
      double* o0 = out + ((int64_t)n * 4 * C + c) * HW;
      memcpy(o0, xp, sizeof(double) * HW);
      for (int b = 0; b < 3; ++b) {
        const int d = dil_of(b, d0, d1, d2);
        const double* kp = k + (((int64_t)n * 3 + b) * C + c) * KK * HW;
        double* ob = out + ((int64_t)n * 4 * C + (int64_t)(b + 1) * C + c) * HW;
        for (int h = 0; h < H; ++h)
          for (int w = 0; w < W; ++w) {
            double acc = 0.0;
            for (int ki = 0; ki < K; ++ki)
              for (int kj = 0; kj < K; ++kj) {
                const int hh = h + (ki - r) * d, ww = w + (kj - r) * d;
                if (hh < 0 || hh >= H || ww < 0 || ww >= W) continue;
                acc += kp[(int64_t)(ki * K + kj) * HW + (int64_t)h * W + w] * xp[(int64_t)hh * W + ww];
              }
            ob[(int64_t)h * W + w] = acc;
          }
      }
    }
}

/* Adjoint of the above (triton_impl.py:94-132): dX by explicit scatter, dK by product. */
void oracle_dynamic_cat_bwd(const double* x, const double* k, const double* g, double* dx,
                            double* dk, int N, int C, int H, int W, int K, int d0, int d1, int d2) {
  const int r = K / 2, KK = K * K;
  const int64_t HW = (int64_t)H * W;
#pragma omp parallel for collapse(2) schedule(static)
  for (int n = 0; n < N; ++n)
    for (int c = 0; c < C; ++c) {
      const double* xp = x + ((int64_t)n * C + c) * HW;
      double* dxp = dx + ((int64_t)n * C + c) * HW;
      memcpy(dxp, g + ((int64_t)n * 4 * C + c) * HW, sizeof(double) * HW);
      for (int b = 0; b < 3; ++b) {
        const int d = dil_of(b, d0, d1, d2);
        const double* kp = k + (((int64_t)n * 3 + b) * C + c) * KK * HW;
        double* dkp = dk + (((int64_t)n * 3 + b) * C + c) * KK * HW;
        const double* gb = g + ((int64_t)n * 4 * C + (int64_t)(b + 1) * C + c) * HW;
        for (int h = 0; h < H; ++h)
          for (int w = 0; w < W; ++w) {
            const int64_t p = (int64_t)h * W + w;
            for (int ki = 0; ki < K; ++ki)
              for (int kj = 0; kj < K; ++kj) {
                const int64_t t = (int64_t)(ki * K + kj) * HW + p;
                const int hh = h + (ki - r) * d, ww = w + (kj - r) * d;
                if (hh < 0 || hh >= H || ww < 0 || ww >= W) {
                  dkp[t] = 0.0;
                  continue;
                }
                const int64_t q = (int64_t)hh * W + ww;
                dkp[t] = gb[p] * xp[q];
                dxp[q] += kp[t] * gb[p];
              }
          }
      }
    }
}

/* 1x1 conv generator (unfold_impl.py:15,23): gen[n][o][p] = sum_i W[o][i] y[n][i][p] + b[o]. */
void oracle_generator(const double* y, const double* wt, const double* bias, double* gen, int N,
                      int C, int G, int64_t HW) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int n = 0; n < N; ++n)
    for (int o = 0; o < G; ++o) {
      double* gp = gen + ((int64_t)n * G + o) * HW;
      for (int64_t p = 0; p < HW; ++p) gp[p] = bias[o];
      for (int i = 0; i < C; ++i) {
        const double wv = wt[(int64_t)o * C + i];
        const double* yp = y + ((int64_t)n * C + i) * HW;
        for (int64_t p = 0; p < HW; ++p) gp[p] += wv * yp[p];
      }
    }
}

/* Parameter / input gradients of the generator given dK = dL/dgen
 * (_triton_kernels.py:534-811): dY = W^T dK, dW = sum_p dK y^T, db = sum_p dK. */
void oracle_generator_bwd(const double* y, const double* wt, const double* dk, double* dy,
                          double* dw, double* db, int N, int C, int G, int64_t HW) {
#pragma omp parallel for schedule(static)
  for (int o = 0; o < G; ++o) {
    double bacc = 0.0;
    for (int n = 0; n < N; ++n) {
      const double* dkp = dk + ((int64_t)n * G + o) * HW;
      for (int64_t p = 0; p < HW; ++p) bacc += dkp[p];
    }
    db[o] = bacc;
    for (int i = 0; i < C; ++i) {
      double acc = 0.0;
      for (int n = 0; n < N; ++n) {
        const double* dkp = dk + ((int64_t)n * G + o) * HW;
        const double* yp = y + ((int64_t)n * C + i) * HW;
        for (int64_t p = 0; p < HW; ++p) acc += dkp[p] * yp[p];
      }
      dw[(int64_t)o * C + i] = acc;
    }
  }
#pragma omp parallel for collapse(2) schedule(static)
  for (int n = 0; n < N; ++n)
    for (int i = 0; i < C; ++i) {
      double* dyp = dy + ((int64_t)n * C + i) * HW;
      for (int64_t p = 0; p < HW; ++p) dyp[p] = 0.0;
      for (int o = 0; o < G; ++o) {
        const double wv = wt[(int64_t)o * C + i];
        const double* dkp = dk + ((int64_t)n * G + o) * HW;
        for (int64_t p = 0; p < HW; ++p) dyp[p] += wv * dkp[p];
      }
    }
}
