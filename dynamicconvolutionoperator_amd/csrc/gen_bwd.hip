// Fused recompute backward of generator + dynamic dilated filter + concat.
//
// Counterpart of _generator_dynamic_cat_bwd_x (_triton_kernels.py:430-531,
// launched at :944-961); the y and weight gradients live in gen_bwd_y.hip and
// gen_bwd_w.hip.  Nothing but y, W, b and grad_cat is read; the dynamic
// kernels are recomputed on chip only.
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
