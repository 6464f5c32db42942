// Materialized dynamic dilated depthwise filter: forward, dX and dK.
//
// Counterparts of the reference's _dynamic_cat_fwd / _dynamic_cat_bwd_x /
// _dynamic_cat_bwd_k (_triton_kernels.py:21-254), redesigned for CDNA4:
//   * one workgroup = one (n, c) plane x one spatial tile of TH rows x TW cols;
//   * the x (or branch-gradient) tile plus a halo of R = (K/2)*max(d) is staged
//     once in LDS, so all three dilations read neighbours from LDS, zero padded;
//   * the 3*K*K kernel planes stream through with VEC-wide coalesced loads
//     (16 B per lane for fp32 when W % 4 == 0), FP32 accumulation;
//   * outputs [x, d0, d1, d2] are written directly (no Unfold buffers).
// All three kernels move HBM bytes proportional to (3K^2 + 5) planes and are
// bandwidth bound.

#include "ddpm_common.h"

namespace ddpm {

struct FilterGeom {
  int N, C, H, W, K;
  int d0, d1, d2;
  int R;         // halo radius
  int tpr_log2;  // log2(threads per tile row)
  int TH, TW;    // tile rows / cols
  int tiles_w, tiles;
  int LH, LW;    // LDS tile rows / cols (TH + 2R, TW + 2R)
};

constexpr int kFilterThreads = 256;
constexpr int kFilterMaxPasses = 4;  // tile height = rows per pass * passes

// Stage plane[h0-R : h0+TH+R, w0-R : w0+TW+R] into LDS as fp32, zero outside
// the image.  One wave per LDS row, lanes over columns (coalesced).
template <typename T>
__device__ __forceinline__ void stage_tile(float* __restrict__ s, const T* __restrict__ plane,
                                           const FilterGeom& g, int h0, int w0) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  for (int i = wave; i < g.LH; i += kFilterThreads / 64) {
    const int gh = h0 - g.R + i;
    const bool row_ok = (unsigned)gh < (unsigned)g.H;
    const T* __restrict__ src = plane + (int64_t)gh * g.W;
    float* __restrict__ dst = s + i * g.LW;
    for (int j = lane; j < g.LW; j += 64) {
      const int gw = w0 - g.R + j;
      float v = 0.f;
      if (row_ok && (unsigned)gw < (unsigned)g.W) v = to_f(src[gw]);
      dst[j] = v;
    }
  }
}

template <typename TX, typename TK, int KS, int VEC>
__global__ __launch_bounds__(kFilterThreads) void filter_fwd_kernel(const TX* __restrict__ x,
                                                                      const TK* __restrict__ kern,
                                                                      TK* __restrict__ out,
                                                                      FilterGeom g) {
  extern __shared__ float xs[];
  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int plane = bid / g.tiles;
  const int tile = bid - plane * g.tiles;
  const int n = plane / g.C, c = plane - n * g.C;
  const int ty = tile / g.tiles_w, tx = tile - ty * g.tiles_w;
  const int h0 = ty * g.TH, w0 = tx * g.TW;
  const int64_t HW = (int64_t)g.H * g.W;

  stage_tile<TX>(xs, x + (int64_t)plane * HW, g, h0, w0);
  __syncthreads();

  const int K = KS > 0 ? KS : g.K;
  const int KK = K * K, r = K / 2;
  const int64_t bstride = (int64_t)g.C * KK * HW;
  const TK* __restrict__ kp = kern + ((int64_t)n * 3 * g.C + c) * KK * HW;
  TK* __restrict__ op = out + ((int64_t)n * 4 * g.C + c) * HW;
  const int64_t ostride = (int64_t)g.C * HW;

  const int tpr = 1 << g.tpr_log2;
  const int tcol = (threadIdx.x & (tpr - 1)) * VEC;
  const int rpp = kFilterThreads >> g.tpr_log2;
  const int gw = w0 + tcol;
  if (gw >= g.W) return;  // no barrier below
  for (int trow = threadIdx.x >> g.tpr_log2; trow < g.TH; trow += rpp) {
    const int gh = h0 + trow;
    if (gh >= g.H) break;
    const int64_t p = (int64_t)gh * g.W + gw;
    const float* __restrict__ xc = xs + (trow + g.R) * g.LW + tcol + g.R;
    float acc[3][VEC];
#pragma unroll
    for (int b = 0; b < 3; ++b)
#pragma unroll
      for (int v = 0; v < VEC; ++v) acc[b][v] = 0.f;
#pragma unroll
    for (int b = 0; b < 3; ++b) {
      const int d = dil_of(b, g.d0, g.d1, g.d2);
      const TK* __restrict__ kb = kp + b * bstride + p;
#pragma unroll
      for (int ki = 0; ki < (KS > 0 ? KS : 1); ++ki) {
        for (int kir = (KS > 0 ? ki : 0); kir < (KS > 0 ? ki + 1 : K); ++kir) {
          const float* __restrict__ xr = xc + (kir - r) * d * g.LW;
#pragma unroll
          for (int kj = 0; kj < (KS > 0 ? KS : 1); ++kj) {
            for (int kjr = (KS > 0 ? kj : 0); kjr < (KS > 0 ? kj + 1 : K); ++kjr) {
              float kv[VEC];
              VecIO<TK, VEC>::load(kb + (int64_t)(kir * K + kjr) * HW, kv);
              const float* __restrict__ xq = xr + (kjr - r) * d;
#pragma unroll
              for (int v = 0; v < VEC; ++v) acc[b][v] = fmaf(kv[v], xq[v], acc[b][v]);
            }
          }
        }
      }
    }
    float xv[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) xv[v] = xc[v];
    VecIO<TK, VEC>::store(op + p, xv);
#pragma unroll
    for (int b = 0; b < 3; ++b) VecIO<TK, VEC>::store(op + (b + 1) * ostride + p, acc[b]);
  }
}

template <typename TX, typename TK, int KS, int VEC>
__global__ __launch_bounds__(kFilterThreads) void filter_bwd_k_kernel(const TX* __restrict__ x,
                                                                        const TK* __restrict__ gout,
                                                                        TK* __restrict__ gk,
                                                                        FilterGeom g) {
  extern __shared__ float xs[];
  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int plane = bid / g.tiles;
  const int tile = bid - plane * g.tiles;
  const int n = plane / g.C, c = plane - n * g.C;
  const int ty = tile / g.tiles_w, tx = tile - ty * g.tiles_w;
  const int h0 = ty * g.TH, w0 = tx * g.TW;
  const int64_t HW = (int64_t)g.H * g.W;

  stage_tile<TX>(xs, x + (int64_t)plane * HW, g, h0, w0);
  __syncthreads();

  const int K = KS > 0 ? KS : g.K;
  const int KK = K * K, r = K / 2;
  const int64_t bstride = (int64_t)g.C * KK * HW;
  TK* __restrict__ kp = gk + ((int64_t)n * 3 * g.C + c) * KK * HW;
  const TK* __restrict__ gp = gout + ((int64_t)n * 4 * g.C + c) * HW;
  const int64_t gstride = (int64_t)g.C * HW;

  const int tpr = 1 << g.tpr_log2;
  const int tcol = (threadIdx.x & (tpr - 1)) * VEC;
  const int rpp = kFilterThreads >> g.tpr_log2;
  const int gw = w0 + tcol;
  if (gw >= g.W) return;
  for (int trow = threadIdx.x >> g.tpr_log2; trow < g.TH; trow += rpp) {
    const int gh = h0 + trow;
    if (gh >= g.H) break;
    const int64_t p = (int64_t)gh * g.W + gw;
    const float* __restrict__ xc = xs + (trow + g.R) * g.LW + tcol + g.R;
    float go[3][VEC];
#pragma unroll
    for (int b = 0; b < 3; ++b) VecIO<TK, VEC>::load(gp + (b + 1) * gstride + p, go[b]);
#pragma unroll
    for (int b = 0; b < 3; ++b) {
      const int d = dil_of(b, g.d0, g.d1, g.d2);
      TK* __restrict__ kb = kp + b * bstride + p;
#pragma unroll
      for (int ki = 0; ki < (KS > 0 ? KS : 1); ++ki) {
        for (int kir = (KS > 0 ? ki : 0); kir < (KS > 0 ? ki + 1 : K); ++kir) {
          const float* __restrict__ xr = xc + (kir - r) * d * g.LW;
#pragma unroll
          for (int kj = 0; kj < (KS > 0 ? KS : 1); ++kj) {
            for (int kjr = (KS > 0 ? kj : 0); kjr < (KS > 0 ? kj + 1 : K); ++kjr) {
              const float* __restrict__ xq = xr + (kjr - r) * d;
              float prod[VEC];
#pragma unroll
              for (int v = 0; v < VEC; ++v) prod[v] = go[b][v] * xq[v];
              VecIO<TK, VEC>::store(kb + (int64_t)(kir * K + kjr) * HW, prod);
            }
          }
        }
      }
    }
  }
}

// dX[c,q] = gO_x[c,q] + sum_b sum_tap k_b[c,tap,q-off] * gO_b[c,q-off]   (gather form)
// The three branch-gradient tiles (+halo) are staged together in LDS; the
// kernel planes are gathered at the shifted source pixels.
template <typename TX, typename TK, int KS, int VEC>
__global__ __launch_bounds__(kFilterThreads) void filter_bwd_x_kernel(const TK* __restrict__ gout,
                                                                        const TK* __restrict__ kern,
                                                                        TX* __restrict__ gx,
                                                                        FilterGeom g) {
  extern __shared__ float gs[];
  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int plane = bid / g.tiles;
  const int tile = bid - plane * g.tiles;
  const int n = plane / g.C, c = plane - n * g.C;
  const int ty = tile / g.tiles_w, tx = tile - ty * g.tiles_w;
  const int h0 = ty * g.TH, w0 = tx * g.TW;
  const int64_t HW = (int64_t)g.H * g.W;

  const int K = KS > 0 ? KS : g.K;
  const int KK = K * K, r = K / 2;
  const int64_t bstride = (int64_t)g.C * KK * HW;
  const TK* __restrict__ kp = kern + ((int64_t)n * 3 * g.C + c) * KK * HW;
  const TK* __restrict__ gp = gout + ((int64_t)n * 4 * g.C + c) * HW;
  const int64_t gstride = (int64_t)g.C * HW;
  const int lplane = g.LH * g.LW;

#pragma unroll
  for (int b = 0; b < 3; ++b) stage_tile<TK>(gs + b * lplane, gp + (b + 1) * gstride, g, h0, w0);
  __syncthreads();

  const int tpr = 1 << g.tpr_log2;
  const int tcol = (threadIdx.x & (tpr - 1)) * VEC;
  const int rpp = kFilterThreads >> g.tpr_log2;
  const int gw = w0 + tcol;
  if (gw >= g.W) return;
  TX* __restrict__ xo = gx + (int64_t)plane * HW;
  for (int trow = threadIdx.x >> g.tpr_log2; trow < g.TH; trow += rpp) {
    const int gh = h0 + trow;
    if (gh >= g.H) break;
    const int64_t p = (int64_t)gh * g.W + gw;
    float acc[VEC];
    VecIO<TK, VEC>::load(gp + p, acc);
#pragma unroll
    for (int b = 0; b < 3; ++b) {
      const int d = dil_of(b, g.d0, g.d1, g.d2);
      const TK* __restrict__ kb = kp + b * bstride;
      const float* __restrict__ gc = gs + b * lplane + (trow + g.R) * g.LW + tcol + g.R;
#pragma unroll
      for (int ki = 0; ki < (KS > 0 ? KS : 1); ++ki) {
        for (int kir = (KS > 0 ? ki : 0); kir < (KS > 0 ? ki + 1 : K); ++kir) {
          const int sh = gh - (kir - r) * d;  // source row of the gathered term
          const bool sh_ok = (unsigned)sh < (unsigned)g.H;
          const float* __restrict__ gr = gc - (kir - r) * d * g.LW;
#pragma unroll
          for (int kj = 0; kj < (KS > 0 ? KS : 1); ++kj) {
            for (int kjr = (KS > 0 ? kj : 0); kjr < (KS > 0 ? kj + 1 : K); ++kjr) {
              const int dw = (kjr - r) * d;
              const TK* __restrict__ kt = kb + (int64_t)(kir * K + kjr) * HW + (int64_t)sh * g.W;
#pragma unroll
              for (int v = 0; v < VEC; ++v) {
                const int sw = gw + v - dw;
                float kv = 0.f;
                if (sh_ok && (unsigned)sw < (unsigned)g.W) kv = to_f(kt[sw]);
                acc[v] = fmaf(kv, gr[v - dw], acc[v]);
              }
            }
          }
        }
      }
    }
    VecIO<TX, VEC>::store(xo + p, acc);
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
namespace {

int pow2ceil(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}
int ilog2(int v) {
  int l = 0;
  while ((1 << l) < v) ++l;
  return l;
}

constexpr size_t kFilterMaxLds = 64 * 1024;

int make_geom(FilterGeom& g, int64_t n, int64_t c, int64_t h, int64_t w, int k, int d0, int d1,
              int d2, int vec, int lds_planes) {
  if (n < 0 || c < 0 || h < 0 || w < 0) return kBadArgument;
  if (k < 1 || (k % 2) == 0 || d0 < 1 || d1 < 1 || d2 < 1) return kBadArgument;
  if (c > (1 << 24) || h > (1 << 20) || w > (1 << 20) || h * w > (int64_t)1 << 31) return kUnsupported;
  g.N = (int)n;
  g.C = (int)c;
  g.H = (int)h;
  g.W = (int)w;
  g.K = k;
  g.d0 = d0;
  g.d1 = d1;
  g.d2 = d2;
  int dmax = d0 > d1 ? d0 : d1;
  dmax = dmax > d2 ? dmax : d2;
  g.R = (k / 2) * dmax;
  const int tpc = (int)((w + vec - 1) / vec);
  int tpr = pow2ceil(tpc);
  if (tpr > 64) tpr = 64;
  g.tpr_log2 = ilog2(tpr);
  g.TW = tpr * vec;
  const int rpp = kFilterThreads / tpr;
  int passes = 16 / rpp;
  if (passes < 1) passes = 1;
  if (passes > kFilterMaxPasses) passes = kFilterMaxPasses;
  // Do not make tiles taller than the image needs.
  while (passes > 1 && rpp * (passes - 1) >= h) --passes;
  for (;;) {
    g.TH = rpp * passes;
    g.LH = g.TH + 2 * g.R;
    g.LW = g.TW + 2 * g.R;
    if ((size_t)lds_planes * g.LH * g.LW * sizeof(float) <= kFilterMaxLds) break;
    if (passes == 1) return kUnsupported;
    --passes;
  }
  g.tiles_w = (int)((w + g.TW - 1) / g.TW);
  const int tiles_h = (int)((h + g.TH - 1) / g.TH);
  g.tiles = g.tiles_w * tiles_h;
  if ((int64_t)g.tiles * n * c > 0x7fffffffLL) return kUnsupported;
  return kOk;
}

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

enum class FilterOp { kFwd, kBwdX, kBwdK };

template <typename TX, typename TK, int KS, int VEC>
void launch_one(FilterOp op, const void* a, const void* b, void* o, const FilterGeom& g,
                hipStream_t stream) {
  const dim3 grid((unsigned)((int64_t)g.tiles * g.N * g.C));
  const dim3 block(kFilterThreads);
  const size_t lds = (size_t)(op == FilterOp::kBwdX ? 3 : 1) * g.LH * g.LW * sizeof(float);
  switch (op) {
    case FilterOp::kFwd:
      hipLaunchKernelGGL((filter_fwd_kernel<TX, TK, KS, VEC>), grid, block, lds, stream,
                         (const TX*)a, (const TK*)b, (TK*)o, g);
      break;
    case FilterOp::kBwdK:
      hipLaunchKernelGGL((filter_bwd_k_kernel<TX, TK, KS, VEC>), grid, block, lds, stream,
                         (const TX*)a, (const TK*)b, (TK*)o, g);
      break;
    case FilterOp::kBwdX:
      hipLaunchKernelGGL((filter_bwd_x_kernel<TX, TK, KS, VEC>), grid, block, lds, stream,
                         (const TK*)a, (const TK*)b, (TX*)o, g);
      break;
  }
}

template <typename TX, typename TK>
void launch_typed(FilterOp op, const void* a, const void* b, void* o, const FilterGeom& g, int vec,
                  hipStream_t stream) {
  if (vec == 4) {
    switch (g.K) {
      case 1:
        return launch_one<TX, TK, 1, 4>(op, a, b, o, g, stream);
      default:
        return launch_one<TX, TK, 3, 4>(op, a, b, o, g, stream);
    }
  }
  switch (g.K) {
    case 1:
      return launch_one<TX, TK, 1, 1>(op, a, b, o, g, stream);
    case 3:
      return launch_one<TX, TK, 3, 1>(op, a, b, o, g, stream);
    case 5:
      return launch_one<TX, TK, 5, 1>(op, a, b, o, g, stream);
    case 7:
      return launch_one<TX, TK, 7, 1>(op, a, b, o, g, stream);
    default:
      return launch_one<TX, TK, 0, 1>(op, a, b, o, g, stream);
  }
}

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

size_t esize(int dt) { return dt == kF32 ? 4 : 2; }

int run_filter(FilterOp op, const void* a, const void* b, void* o, int64_t n, int64_t c, int64_t h,
               int64_t w, int k, int d0, int d1, int d2, int x_dtype, int k_dtype,
               hipStream_t stream) {
  if (x_dtype < kF32 || x_dtype > kF16 || k_dtype < kF32 || k_dtype > kF16) return kBadArgument;
  if (n == 0 || c == 0 || h == 0 || w == 0) return kOk;
  if (!a || !b || !o) return kBadArgument;
  // 4-wide vectors need W % 4 == 0 (so rows start aligned) and aligned bases
  // for the streamed kernel / gradient / output planes; K <= 3 keeps the
  // per-thread tap registers bounded.
  const size_t kv = 4 * esize(k_dtype), xv = 4 * esize(x_dtype);
  bool vec4 = (w % 4 == 0) && k <= 3;
  switch (op) {
    case FilterOp::kFwd:
      vec4 = vec4 && aligned(b, kv) && aligned(o, kv);
      break;
    case FilterOp::kBwdK:
      vec4 = vec4 && aligned(b, kv) && aligned(o, kv);
      break;
    case FilterOp::kBwdX:
      vec4 = vec4 && aligned(a, kv) && aligned(o, xv);
      break;
  }
  const int vec = vec4 ? 4 : 1;
  FilterGeom g;
  int st = make_geom(g, n, c, h, w, k, d0, d1, d2, vec, op == FilterOp::kBwdX ? 3 : 1);
  if (st != kOk) return st;
  st = with_type(x_dtype, [&](auto tx) {
    using TX = decltype(tx);
    return with_type(k_dtype, [&](auto tk) {
      using TK = decltype(tk);
      launch_typed<TX, TK>(op, a, b, o, g, vec, stream);
      return (int)kOk;
    });
  });
  if (st != kOk) return st;
  return (int)hipGetLastError();
}

}  // namespace
}  // namespace ddpm

using namespace ddpm;

extern "C" int ddpm_filter_fwd(const void* x, const void* kernels, void* out, int64_t n, int64_t c,
                               int64_t h, int64_t w, int kernel_size, int d0, int d1, int d2,
                               int x_dtype, int k_dtype, hipStream_t stream) {
  return run_filter(FilterOp::kFwd, x, kernels, out, n, c, h, w, kernel_size, d0, d1, d2, x_dtype,
                    k_dtype, stream);
}

extern "C" int ddpm_filter_bwd_x(const void* grad_out, const void* kernels, void* grad_x, int64_t n,
                                 int64_t c, int64_t h, int64_t w, int kernel_size, int d0, int d1,
                                 int d2, int x_dtype, int k_dtype, hipStream_t stream) {
  return run_filter(FilterOp::kBwdX, grad_out, kernels, grad_x, n, c, h, w, kernel_size, d0, d1, d2,
                    x_dtype, k_dtype, stream);
}

extern "C" int ddpm_filter_bwd_k(const void* x, const void* grad_out, void* grad_kernels, int64_t n,
                                 int64_t c, int64_t h, int64_t w, int kernel_size, int d0, int d1,
                                 int d2, int x_dtype, int k_dtype, hipStream_t stream) {
  return run_filter(FilterOp::kBwdK, x, grad_out, grad_kernels, n, c, h, w, kernel_size, d0, d1, d2,
                    x_dtype, k_dtype, stream);
}
