// Fused recompute backward of generator + dynamic dilated filter + concat.
//
// Counterparts of _generator_dynamic_cat_bwd_x / _bwd_y /
// _bwd_weight_partial / _bwd_weight_reduce (_triton_kernels.py:430-811,
// launched at :927-1053).  Nothing but x, y, W, b and grad_cat is read; the
// dynamic kernels and their gradient dK = dL/dgen are formed on chip only.
//
//   gen[(b,c,t), p] = W[(b,c,t), :] . y[:, p] + bias[(b,c,t)]
//   dK[(b,c,t), p]  = gO_b[c, p] * x[c, p + off(b,t)]
//   dX[c, q]  = gO_x[c, q] + sum_{b,t} q(gen[(b,c,t), q - off]) * gO_b[c, q - off]
//   dY[i, p]  = sum_{b,c,t} W[(b,c,t), i] * dK[(b,c,t), p]
//   dW[o, i]  = sum_p dK[o, p] * y[i, p],   db[o] = sum_p dK[o, p]
//
// All products run on v_mfma_f32_16x16x32_{bf16,f16}; fp32 operands as three
// bf16 products (relative error ~2^-16 per product, fp32 accumulation).

#include "gen_common.h"
#include <type_traits>

namespace ddpm {

constexpr int kBwdThreads = 256;
constexpr int kBwdRPW = 1;                 // tile rows per wave
constexpr int kBwdCPW = 2;                 // 16-pixel column blocks per wave
constexpr int kBwdTH = 4 * kBwdRPW;
constexpr int kBwdTW = 16 * kBwdCPW;
constexpr int kBwdNB = kBwdRPW * kBwdCPW;

template <typename T>
__device__ __forceinline__ void load_row8(const T* __restrict__ p, bool row_ok, int k0, int C,
                                          bool vec, float (&v)[8]) {
  if (row_ok && vec && k0 + 8 <= C) {
    if constexpr (sizeof(T) == 4) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(p + k0);
      const f32x4 b = *reinterpret_cast<const f32x4*>(p + k0 + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] = a[e];
        v[4 + e] = b[e];
      }
    } else {
      typedef T T8 __attribute__((ext_vector_type(8)));
      const T8 a = *reinterpret_cast<const T8*>(p + k0);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = to_f(a[e]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (row_ok && k0 + e < C) ? to_f(p[k0 + e]) : 0.f;
  }
}

// ---------------------------------------------------------------------------
// dX: per output tile (4 rows x 32 cols), all channels.  For each (b, tap) the
// generator is recomputed at the gathered source pixels q - off (y operand
// loaded at the shifted pixels), rounded like the forward, multiplied by the
// branch gradient at the same source pixels and accumulated.
// ---------------------------------------------------------------------------
template <typename T, int KS, int MB>
__global__ __launch_bounds__(kBwdThreads) void gen_bwd_x_kernel(const T* __restrict__ y,
                                                                  const T* __restrict__ wt,
                                                                  const T* __restrict__ bias,
                                                                  const T* __restrict__ gout,
                                                                  T* __restrict__ gx, GenGeom g) {
  typedef Mma<T> M;
  typedef typename M::V V;
  constexpr int KK = KS * KS;
  constexpr int r = KS / 2;
  constexpr int KSTEPS = (MB + 1) / 2;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  float* __restrict__ bs = reinterpret_cast<float*>(smem);  // [3][KK][C]

  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int tile = bid % g.tiles;
  const int n = bid / g.tiles;
  const int ty = tile / g.tiles_w, tx = tile - ty * g.tiles_w;
  const int h0 = ty * kBwdTH, w0 = tx * kBwdTW;
  const int C = g.C;
  const int64_t HW = (int64_t)g.H * g.W;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int col16 = lane & 15, quad = lane >> 4;

  for (int idx = tid; idx < 3 * KK * MB * 16; idx += kBwdThreads) {
    const int m = idx % (MB * 16), bt = idx / (MB * 16);
    const int b = bt / KK, t = bt - b * KK;
    bs[idx] = m < C ? to_f(bias[(int64_t)(b * C + m) * KK + t]) : 0.f;
  }
  __syncthreads();

  const T* __restrict__ go = gout + (int64_t)n * 4 * C * HW;
  const T* __restrict__ yn = y + (int64_t)n * C * HW;
  const bool wvec = g.wvec != 0;

  f32x4 acc[kBwdNB][MB];
#pragma unroll
  for (int blk = 0; blk < kBwdNB; ++blk) {
    const int gh = h0 + wave * kBwdRPW + blk / kBwdCPW;
    const int gw = w0 + (blk % kBwdCPW) * 16 + col16;
    const bool ok = gh < g.H && gw < g.W;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int ch = mb * 16 + 4 * quad + e;
        acc[blk][mb][e] = (ok && ch < C) ? to_f(go[(int64_t)ch * HW + (int64_t)gh * g.W + gw]) : 0.f;
      }
  }

  // Flattened (branch, tap) loop with the weight rows of the next step
  // prefetched into registers.
  float wnext[MB][KSTEPS][8];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk)
      load_row8<T>(wt + (int64_t)(mb * 16 + col16) * KK * C, mb * 16 + col16 < C, 32 * kk + 8 * quad,
                   C, wvec, wnext[mb][kk]);
#pragma unroll 1
  for (int bt = 0; bt < 3 * KK; ++bt) {
    const int b = bt / KK, t = bt - b * KK;
    const int ki = t / KS, kj = t - ki * KS;
    const int d = dil_of(b, g.d0, g.d1, g.d2);
    const int dh = (ki - r) * d, dw = (kj - r) * d;
    const T* __restrict__ gob = go + (int64_t)(b + 1) * C * HW;
    V afrag[MB][KSTEPS][M::P];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int kk = 0; kk < KSTEPS; ++kk) M::pack(wnext[mb][kk], afrag[mb][kk]);
    if (bt + 1 < 3 * KK) {
      const int b1 = (bt + 1) / KK, t1 = (bt + 1) - b1 * KK;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const int crow = mb * 16 + col16;
        const T* __restrict__ wrow = wt + ((int64_t)(b1 * C + crow) * KK + t1) * C;
#pragma unroll
        for (int kk = 0; kk < KSTEPS; ++kk)
          load_row8<T>(wrow, crow < C, 32 * kk + 8 * quad, C, wvec, wnext[mb][kk]);
      }
    }
#pragma unroll
    for (int blk = 0; blk < kBwdNB; ++blk) {
      const int sh = h0 + wave * kBwdRPW + blk / kBwdCPW - dh;
      const int sw = w0 + (blk % kBwdCPW) * 16 + col16 - dw;
      const bool ok = (unsigned)sh < (unsigned)g.H && (unsigned)sw < (unsigned)g.W;
      const int64_t sp = (int64_t)sh * g.W + sw;
      V bfrag[KSTEPS][M::P];
#pragma unroll
      for (int kk = 0; kk < KSTEPS; ++kk) {
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int i = 32 * kk + 8 * quad + e;
          v[e] = (ok && i < C) ? to_f(yn[(int64_t)i * HW + sp]) : 0.f;
        }
        M::pack(v, bfrag[kk]);
      }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        f32x4 dacc = *reinterpret_cast<const f32x4*>(bs + bt * (MB * 16) + mb * 16 + 4 * quad);
#pragma unroll
        for (int kk = 0; kk < KSTEPS; ++kk) dacc = M::mac(afrag[mb][kk], bfrag[kk], dacc);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int ch = mb * 16 + 4 * quad + e;
          const float gv = (ok && ch < C) ? to_f(gob[(int64_t)ch * HW + sp]) : 0.f;
          acc[blk][mb][e] = fmaf(quant<T>(dacc[e]), gv, acc[blk][mb][e]);
        }
      }
    }
  }

#pragma unroll
  for (int blk = 0; blk < kBwdNB; ++blk) {
    const int gh = h0 + wave * kBwdRPW + blk / kBwdCPW;
    const int gw = w0 + (blk % kBwdCPW) * 16 + col16;
    if (gh < g.H && gw < g.W) {
      T* __restrict__ xo = gx + (int64_t)n * C * HW + (int64_t)gh * g.W + gw;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int ch = mb * 16 + 4 * quad + e;
          if (ch < C) xo[(int64_t)ch * HW] = from_f<T>(acc[blk][mb][e]);
        }
    }
  }
}

// ---------------------------------------------------------------------------
// dY: M = input channels i (all MB blocks), N = 16 pixels, K = output
// channels c for each (b, tap).  B operand dK = gO_b[c,p] * x[c, p+off] is
// formed in registers; the A operand W_bt^T is staged per (b, tap) in LDS,
// pre-split into MFMA parts and shared by the 4 waves.
// ---------------------------------------------------------------------------
template <typename T, int KS, int MB>
__global__ __launch_bounds__(kBwdThreads) void gen_bwd_y_kernel(const T* __restrict__ x,
                                                                  const T* __restrict__ wt,
                                                                  const T* __restrict__ gout,
                                                                  T* __restrict__ gy, GenGeom g) {
  typedef Mma<T> M;
  typedef typename M::V V;
  typedef typename M::E E;
  constexpr int KK = KS * KS;
  constexpr int r = KS / 2;
  constexpr int KSTEPS = (MB + 1) / 2;
  constexpr int CP = KSTEPS * 32;  // padded K extent
  constexpr int LSTR = CP + 8;     // LDS row stride (elements), keeps 16 B alignment
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  // [2 buffers][P parts][MB*16 rows i][LSTR cols c]
  E* __restrict__ ws = reinterpret_cast<E*>(smem);
  constexpr int PART = MB * 16 * LSTR;

  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int tile = bid % g.tiles;
  const int n = bid / g.tiles;
  const int ty = tile / g.tiles_w, tx = tile - ty * g.tiles_w;
  const int h0 = ty * kBwdTH, w0 = tx * kBwdTW;
  const int C = g.C;
  const int64_t HW = (int64_t)g.H * g.W;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int col16 = lane & 15, quad = lane >> 4;
  const T* __restrict__ xn = x + (int64_t)n * C * HW;
  const T* __restrict__ go = gout + (int64_t)n * 4 * C * HW;

  // Stage W_bt^T (rows i, cols c), split into MFMA parts, into buffer `buf`.
  auto stage = [&](int bt, int buf) {
    const int b = bt / KK, t = bt - b * KK;
    E* __restrict__ dst = ws + buf * (M::P * PART);
    for (int idx = tid; idx < MB * 16 * CP; idx += kBwdThreads) {
      const int i = idx % (MB * 16), c = idx / (MB * 16);  // coalesced over i
      float v = 0.f;
      if (i < C && c < C) v = to_f(wt[((int64_t)(b * C + c) * KK + t) * C + i]);
      if constexpr (M::P == 2) {
        const bf16 h = (bf16)v;
        dst[i * LSTR + c] = h;
        dst[PART + i * LSTR + c] = (bf16)(v - (float)h);
      } else {
        dst[i * LSTR + c] = (E)v;
      }
    }
  };

  f32x4 acc[kBwdNB][MB];
#pragma unroll
  for (int blk = 0; blk < kBwdNB; ++blk)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[blk][mb] = f32x4{0.f, 0.f, 0.f, 0.f};

  stage(0, 0);
  for (int b = 0; b < 3; ++b) {
    const int d = dil_of(b, g.d0, g.d1, g.d2);
    const T* __restrict__ gob = go + (int64_t)(b + 1) * C * HW;
    // branch gradient at this wave's pixels for the lane's K slots (c)
    float gv[kBwdNB][KSTEPS][8];
#pragma unroll
    for (int blk = 0; blk < kBwdNB; ++blk) {
      const int gh = h0 + wave * kBwdRPW + blk / kBwdCPW;
      const int gw = w0 + (blk % kBwdCPW) * 16 + col16;
      const bool ok = gh < g.H && gw < g.W;
#pragma unroll
      for (int kk = 0; kk < KSTEPS; ++kk)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int c = 32 * kk + 8 * quad + e;
          gv[blk][kk][e] =
              (ok && c < C) ? to_f(gob[(int64_t)c * HW + (int64_t)gh * g.W + gw]) : 0.f;
        }
    }
    for (int t = 0; t < KK; ++t) {
      const int bt = b * KK + t;
      const int buf = bt & 1;
      __syncthreads();  // buffer buf complete; buffer buf^1 free
      if (bt + 1 < 3 * KK) stage(bt + 1, buf ^ 1);
      const int ki = t / KS, kj = t % KS;
      const int dh = (ki - r) * d, dw = (kj - r) * d;
      const E* __restrict__ src = ws + buf * (M::P * PART);
#pragma unroll
      for (int blk = 0; blk < kBwdNB; ++blk) {
        const int gh = h0 + wave * kBwdRPW + blk / kBwdCPW;
        const int gw = w0 + (blk % kBwdCPW) * 16 + col16;
        const int nh = gh + dh, nw = gw + dw;
        const bool ok = gh < g.H && gw < g.W && (unsigned)nh < (unsigned)g.H &&
                        (unsigned)nw < (unsigned)g.W;
        const int64_t np = (int64_t)nh * g.W + nw;
        V bfrag[KSTEPS][M::P];
#pragma unroll
        for (int kk = 0; kk < KSTEPS; ++kk) {
          float v[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int c = 32 * kk + 8 * quad + e;
            v[e] = (ok && c < C) ? gv[blk][kk][e] * to_f(xn[(int64_t)c * HW + np]) : 0.f;
          }
          M::pack(v, bfrag[kk]);
        }
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
          for (int kk = 0; kk < KSTEPS; ++kk) {
            V a[M::P];
#pragma unroll
            for (int pp = 0; pp < M::P; ++pp)
              a[pp] = *reinterpret_cast<const V*>(src + pp * PART + (mb * 16 + col16) * LSTR +
                                                  32 * kk + 8 * quad);
            acc[blk][mb] = M::mac(a, bfrag[kk], acc[blk][mb]);
          }
        }
      }
    }
  }

#pragma unroll
  for (int blk = 0; blk < kBwdNB; ++blk) {
    const int gh = h0 + wave * kBwdRPW + blk / kBwdCPW;
    const int gw = w0 + (blk % kBwdCPW) * 16 + col16;
    if (gh < g.H && gw < g.W) {
      T* __restrict__ yo = gy + (int64_t)n * C * HW + (int64_t)gh * g.W + gw;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = mb * 16 + 4 * quad + e;
          if (i < C) yo[(int64_t)i * HW] = from_f<T>(acc[blk][mb][e]);
        }
    }
  }
}

// ---------------------------------------------------------------------------
// dW / db partial: one workgroup per (branch*tap, split); its 4 waves take
// interleaved 32-token steps of the split and are reduced through LDS in a
// fixed order at the end (deterministic, no atomics).  M = output channels c,
// N = input channels i, K = tokens.
// ---------------------------------------------------------------------------
struct WGradGeom {
  int N, C, H, W, K;
  int d0, d1, d2;
  int splits;
  int tokens_per_split;  // multiple of 32
  int64_t tokens;        // N*H*W
  int direct;            // write grad_weight/grad_bias directly (splits == 1)
  int fast;              // W % 8 == 0: 8-token runs stay inside one image row
};

template <typename T, int KS, int MB, bool FAST>
__global__ __launch_bounds__(kBwdThreads) void gen_bwd_w_partial_kernel(
    const T* __restrict__ x, const T* __restrict__ y, const T* __restrict__ gout,
    float* __restrict__ pw, float* __restrict__ pb, T* __restrict__ dw_out, T* __restrict__ db_out,
    WGradGeom g) {
  typedef Mma<T> M;
  typedef typename M::V V;
  constexpr int KK = KS * KS;
  constexpr int r = KS / 2;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  float* __restrict__ red = reinterpret_cast<float*>(smem);  // [MB*16][MB*16 + 1] + [4][MB*16]

  const int bt = blockIdx.x;      // branch * KK + tap
  const int split = blockIdx.y;
  const int b = bt / KK, t = bt - b * KK;
  const int ki = t / KS, kj = t % KS;
  const int d = dil_of(b, g.d0, g.d1, g.d2);
  const int dh = (ki - r) * d, dw = (kj - r) * d;
  const int C = g.C;
  const int64_t HW = (int64_t)g.H * g.W;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int col16 = lane & 15, quad = lane >> 4;

  f32x4 acc[MB][MB];
#pragma unroll
  for (int mc = 0; mc < MB; ++mc)
#pragma unroll
    for (int mi = 0; mi < MB; ++mi) acc[mc][mi] = f32x4{0.f, 0.f, 0.f, 0.f};
  float bacc[MB];
#pragma unroll
  for (int mc = 0; mc < MB; ++mc) bacc[mc] = 0.f;

  const int64_t tbeg = (int64_t)split * g.tokens_per_split;
  int64_t tend = tbeg + g.tokens_per_split;
  if (tend > g.tokens) tend = g.tokens;

  for (int64_t t0 = tbeg + 32 * wave; t0 < tend; t0 += 32 * 4) {
    const int64_t tk = t0 + 8 * quad;  // first of this lane's 8 tokens
    float yv[MB][8];
    float dk[MB][8];
    if constexpr (FAST) {
      // 8 tokens inside one row: n, h fixed, w .. w+7 (W % 8 == 0, tk % 8 == 0)
      const bool any = tk < tend;
      const int64_t nn = any ? tk / HW : 0;
      const int64_t p = tk - nn * HW;
      const int hh = (int)(p / g.W), ww = (int)(p - (int64_t)hh * g.W);
      const int nh = hh + dh;
      const bool nh_ok = any && (unsigned)nh < (unsigned)g.H;
      const T* __restrict__ yb = y + nn * C * HW + p;
      const T* __restrict__ gb = gout + (nn * 4 * C + (int64_t)(b + 1) * C) * HW + p;
      const T* __restrict__ xb = x + nn * C * HW + (int64_t)nh * g.W;
#pragma unroll
      for (int m = 0; m < MB; ++m) {
        const int ch = m * 16 + col16;  // row c for A, col i for B (same lane index)
        const bool ch_ok = any && ch < C;
        if (ch_ok) {
          VecIO<T, 8>::load(yb + (int64_t)ch * HW, yv[m]);
          float gv[8];
          VecIO<T, 8>::load(gb + (int64_t)ch * HW, gv);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int nw = ww + e + dw;
            const float xv =
                (nh_ok && (unsigned)nw < (unsigned)g.W) ? to_f(xb[(int64_t)ch * HW + nw]) : 0.f;
            dk[m][e] = gv[e] * xv;
          }
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            yv[m][e] = 0.f;
            dk[m][e] = 0.f;
          }
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int64_t tt = tk + e;
        const bool ok = tt < tend;
        const int64_t nn = ok ? tt / HW : 0;
        const int64_t p = tt - nn * HW;
        const int hh = (int)(p / g.W), ww = (int)(p - (int64_t)hh * g.W);
        const int nh = hh + dh, nw = ww + dw;
        const bool nok = ok && (unsigned)nh < (unsigned)g.H && (unsigned)nw < (unsigned)g.W;
#pragma unroll
        for (int m = 0; m < MB; ++m) {
          const int ch = m * 16 + col16;
          const bool cok = ok && ch < C;
          yv[m][e] = cok ? to_f(y[(nn * C + ch) * HW + p]) : 0.f;
          const float gv =
              cok ? to_f(gout[(nn * 4 * C + (int64_t)(b + 1) * C + ch) * HW + p]) : 0.f;
          const float xv = (cok && nok) ? to_f(x[(nn * C + ch) * HW + (int64_t)nh * g.W + nw]) : 0.f;
          dk[m][e] = gv * xv;
        }
      }
    }
    V afr[MB][M::P], bfr[MB][M::P];
#pragma unroll
    for (int m = 0; m < MB; ++m) {
      M::pack(dk[m], afr[m]);
      M::pack(yv[m], bfr[m]);
      // db uses the operand-precision dK, like the weight gradient
#pragma unroll
      for (int e = 0; e < 8; ++e) bacc[m] += quant<T>(dk[m][e]);
    }
#pragma unroll
    for (int mc = 0; mc < MB; ++mc)
#pragma unroll
      for (int mi = 0; mi < MB; ++mi) acc[mc][mi] = M::mac(afr[mc], bfr[mi], acc[mc][mi]);
  }

  // ---- deterministic reduction of the 4 waves (fixed order 0,1,2,3)
  constexpr int NO = MB * 16;
  constexpr int RS = NO + 1;
  float* __restrict__ rb = red + NO * RS;  // bias partials [4 waves][4 quads][NO]
#pragma unroll
  for (int m = 0; m < MB; ++m) rb[(wave * 4 + quad) * NO + m * 16 + col16] = bacc[m];
  for (int w = 0; w < 4; ++w) {
    if (wave == w) {
#pragma unroll
      for (int mc = 0; mc < MB; ++mc)
#pragma unroll
        for (int mi = 0; mi < MB; ++mi)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int c = mc * 16 + 4 * quad + e, i = mi * 16 + col16;
            float* dst = red + c * RS + i;
            *dst = (w == 0 ? 0.f : *dst) + acc[mc][mi][e];
          }
    }
    __syncthreads();
  }
  // write out: NO x NO weights + NO biases
  for (int idx = tid; idx < NO * NO; idx += kBwdThreads) {
    const int c = idx / NO, i = idx - c * NO;
    if (c >= C || i >= C) continue;
    const float v = red[c * RS + i];
    if (g.direct)
      dw_out[((int64_t)(b * C + c) * KK + t) * C + i] = from_f<T>(v);
    else
      pw[(((int64_t)split * 3 * KK + bt) * C + c) * C + i] = v;
  }
  for (int c = tid; c < NO; c += kBwdThreads) {
    if (c >= C) continue;
    float v = 0.f;
    for (int w = 0; w < 16; ++w) v += rb[w * NO + c];
    if (g.direct)
      db_out[(int64_t)(b * C + c) * KK + t] = from_f<T>(v);
    else
      pb[((int64_t)split * 3 * KK + bt) * C + c] = v;
  }
}

// Fixed-order sum of the split partials, written in Conv2d parameter layout.
template <typename T>
__global__ __launch_bounds__(256) void gen_bwd_w_reduce_kernel(const float* __restrict__ pw,
                                                                 const float* __restrict__ pb,
                                                                 T* __restrict__ dw_out,
                                                                 T* __restrict__ db_out, int C,
                                                                 int KK, int splits) {
  const int64_t per = (int64_t)3 * KK * C * C;
  const int64_t perb = (int64_t)3 * KK * C;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx < per) {
    float v = 0.f;
    for (int s = 0; s < splits; ++s) v += pw[s * per + idx];
    // idx = (bt*C + c)*C + i  ->  row o = (b*C + c)*KK + t
    const int64_t i = idx % C;
    const int64_t c = (idx / C) % C;
    const int64_t bt = idx / ((int64_t)C * C);
    const int64_t b = bt / KK, t = bt % KK;
    dw_out[((b * C + c) * KK + t) * C + i] = from_f<T>(v);
  } else if (idx < per + perb) {
    const int64_t j = idx - per;
    float v = 0.f;
    for (int s = 0; s < splits; ++s) v += pb[s * perb + j];
    const int64_t c = j % C, bt = j / C;
    const int64_t b = bt / KK, t = bt % KK;
    db_out[(b * C + c) * KK + t] = from_f<T>(v);
  }
}

namespace {

template <typename F>
int with_type(int dt, F&& f) {
  switch (dt) {
    case kF32:
      return f(float());
    case kBF16:
      return f(bf16());
    case kF16:
      return f(f16());
    default:
      return kBadArgument;
  }
}

template <typename F>
int with_mb(int mb, F&& f) {
  switch (mb) {
    case 1:
      return f(std::integral_constant<int, 1>());
    case 2:
      return f(std::integral_constant<int, 2>());
    case 3:
      return f(std::integral_constant<int, 3>());
    case 4:
      return f(std::integral_constant<int, 4>());
    default:
      return kUnsupported;
  }
}

template <typename F>
int with_ks(int k, F&& f) {
  if (k == 1) return f(std::integral_constant<int, 1>());
  if (k == 3) return f(std::integral_constant<int, 3>());
  return kUnsupported;
}

int bwd_geom(GenGeom& g, int64_t n, int64_t c, int64_t h, int64_t w, int k, int d0, int d1,
             int d2) {
  const int st = gen_make_geom(g, n, c, h, w, k, d0, d1, d2);
  if (st != kOk) return st;
  // the backward kernels tile 4 rows x 32 cols
  g.tiles_w = (int)((w + kBwdTW - 1) / kBwdTW);
  g.tiles = g.tiles_w * (int)((h + kBwdTH - 1) / kBwdTH);
  return kOk;
}

void wgrad_geom(WGradGeom& g, int64_t n, int64_t c, int64_t h, int64_t w, int k, int d0, int d1,
                int d2) {
  g.N = (int)n;
  g.C = (int)c;
  g.H = (int)h;
  g.W = (int)w;
  g.K = k;
  g.d0 = d0;
  g.d1 = d1;
  g.d2 = d2;
  g.tokens = n * h * w;
  // At most 16 fp32 partials; about 2048 tokens per split below that.
  int64_t splits = (g.tokens + 2047) / 2048;
  if (splits < 1) splits = 1;
  if (splits > 16) splits = 16;
  g.splits = (int)splits;
  int64_t tps = (g.tokens + splits - 1) / splits;
  tps = (tps + 127) / 128 * 128;  // 4 waves x 32-token steps
  g.tokens_per_split = (int)tps;
  g.direct = splits == 1;
  g.fast = (w % 8) == 0;
}

}  // namespace
}  // namespace ddpm

using namespace ddpm;

extern "C" int ddpm_gen_bwd_x(const void* y, const void* weight, const void* bias,
                              const void* grad_out, void* grad_x, int64_t n, int64_t c, int64_t h,
                              int64_t w, int kernel_size, int d0, int d1, int d2, int dtype,
                              hipStream_t stream) {
  if (dtype < kF32 || dtype > kF16) return kBadArgument;
  GenGeom g;
  int st = bwd_geom(g, n, c, h, w, kernel_size, d0, d1, d2);
  if (st != kOk) return st;
  if (n == 0 || c == 0 || h == 0 || w == 0) return kOk;
  if (!y || !weight || !bias || !grad_out || !grad_x) return kBadArgument;
  g.wvec = ((uintptr_t)weight % 16 == 0) && (c % 8 == 0);
  const int mb = (int)((c + 15) / 16);
  return with_type(dtype, [&](auto tag) {
    using T = decltype(tag);
    return with_ks(kernel_size, [&](auto ks) {
      constexpr int KS = decltype(ks)::value;
      return with_mb(mb, [&](auto mbc) {
        constexpr int MB = decltype(mbc)::value;
        const size_t lds = (size_t)3 * KS * KS * MB * 16 * sizeof(float);
        hipLaunchKernelGGL((gen_bwd_x_kernel<T, KS, MB>), dim3((unsigned)((int64_t)g.N * g.tiles)),
                           dim3(kBwdThreads), lds, stream, (const T*)y, (const T*)weight,
                           (const T*)bias, (const T*)grad_out, (T*)grad_x, g);
        return (int)hipGetLastError();
      });
    });
  });
}

extern "C" int ddpm_gen_bwd_y(const void* x, const void* weight, const void* grad_out,
                              void* grad_y, int64_t n, int64_t c, int64_t h, int64_t w,
                              int kernel_size, int d0, int d1, int d2, int dtype,
                              hipStream_t stream) {
  if (dtype < kF32 || dtype > kF16) return kBadArgument;
  GenGeom g;
  int st = bwd_geom(g, n, c, h, w, kernel_size, d0, d1, d2);
  if (st != kOk) return st;
  if (n == 0 || c == 0 || h == 0 || w == 0) return kOk;
  if (!x || !weight || !grad_out || !grad_y) return kBadArgument;
  const int mb = (int)((c + 15) / 16);
  return with_type(dtype, [&](auto tag) {
    using T = decltype(tag);
    return with_ks(kernel_size, [&](auto ks) {
      constexpr int KS = decltype(ks)::value;
      return with_mb(mb, [&](auto mbc) {
        constexpr int MB = decltype(mbc)::value;
        constexpr int KSTEPS = (MB + 1) / 2;
        constexpr int LSTR = KSTEPS * 32 + 8;
        const size_t lds = (size_t)2 * Mma<T>::P * MB * 16 * LSTR * 2;
        hipLaunchKernelGGL((gen_bwd_y_kernel<T, KS, MB>), dim3((unsigned)((int64_t)g.N * g.tiles)),
                           dim3(kBwdThreads), lds, stream, (const T*)x, (const T*)weight,
                           (const T*)grad_out, (T*)grad_y, g);
        return (int)hipGetLastError();
      });
    });
  });
}

extern "C" int64_t ddpm_gen_bwd_w_workspace_bytes(int64_t n, int64_t c, int64_t h, int64_t w,
                                                  int kernel_size) {
  if (n <= 0 || c <= 0 || h <= 0 || w <= 0 || kernel_size < 1) return 0;
  WGradGeom g;
  wgrad_geom(g, n, c, h, w, kernel_size, 1, 1, 1);
  if (g.direct) return 0;
  const int64_t kk = (int64_t)kernel_size * kernel_size;
  return (int64_t)g.splits * 3 * kk * c * (c + 1) * (int64_t)sizeof(float);
}

extern "C" int ddpm_gen_bwd_w(const void* x, const void* y, const void* grad_out,
                              void* grad_weight, void* grad_bias, void* workspace,
                              int64_t workspace_bytes, int64_t n, int64_t c, int64_t h, int64_t w,
                              int kernel_size, int d0, int d1, int d2, int dtype,
                              hipStream_t stream) {
  if (dtype < kF32 || dtype > kF16) return kBadArgument;
  GenGeom gg;
  int st = gen_make_geom(gg, n, c, h, w, kernel_size, d0, d1, d2);
  if (st != kOk) return st;
  if (n == 0 || c == 0 || h == 0 || w == 0) return kOk;
  if (!x || !y || !grad_out || !grad_weight || !grad_bias) return kBadArgument;
  WGradGeom g;
  wgrad_geom(g, n, c, h, w, kernel_size, d0, d1, d2);
  const int64_t need = ddpm_gen_bwd_w_workspace_bytes(n, c, h, w, kernel_size);
  if (need > 0 && (!workspace || workspace_bytes < need)) return kWorkspaceTooSmall;
  if (g.fast && (((uintptr_t)x | (uintptr_t)y | (uintptr_t)grad_out) % (8 * (dtype == kF32 ? 4 : 2))))
    g.fast = 0;
  const int mb = (int)((c + 15) / 16);
  const int kk = kernel_size * kernel_size;
  float* pw = (float*)workspace;
  float* pb = pw ? pw + (int64_t)g.splits * 3 * kk * c * c : nullptr;
  return with_type(dtype, [&](auto tag) {
    using T = decltype(tag);
    return with_ks(kernel_size, [&](auto ks) {
      constexpr int KS = decltype(ks)::value;
      return with_mb(mb, [&](auto mbc) {
        constexpr int MB = decltype(mbc)::value;
        constexpr int NO = MB * 16;
        const size_t lds = (size_t)(NO * (NO + 1) + 16 * NO) * sizeof(float);
        const dim3 grid(3 * KS * KS, g.splits);
        if (g.fast)
          hipLaunchKernelGGL((gen_bwd_w_partial_kernel<T, KS, MB, true>), grid, dim3(kBwdThreads),
                             lds, stream, (const T*)x, (const T*)y, (const T*)grad_out, pw, pb,
                             (T*)grad_weight, (T*)grad_bias, g);
        else
          hipLaunchKernelGGL((gen_bwd_w_partial_kernel<T, KS, MB, false>), grid,
                             dim3(kBwdThreads), lds, stream, (const T*)x, (const T*)y,
                             (const T*)grad_out, pw, pb, (T*)grad_weight, (T*)grad_bias, g);
        int e = (int)hipGetLastError();
        if (e != 0 || g.direct) return e;
        const int64_t total = (int64_t)3 * kk * c * c + (int64_t)3 * kk * c;
        hipLaunchKernelGGL((gen_bwd_w_reduce_kernel<T>), dim3((unsigned)((total + 255) / 256)),
                           dim3(256), 0, stream, pw, pb, (T*)grad_weight, (T*)grad_bias, (int)c,
                           kk, g.splits);
        return (int)hipGetLastError();
      });
    });
  });
}
