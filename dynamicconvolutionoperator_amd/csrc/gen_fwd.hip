// Fused kernel generator + dynamic dilated filter + concat, forward.
//
// Counterpart of the reference's _generator_dynamic_cat_fwd
// (_triton_kernels.py:268-420, launched at :873-908), redesigned for CDNA4:
//
//   gen[(b,c,tap), p] = sum_i W[(b,c,tap), i] * y[i, p] + bias[(b,c,tap)]
//   out_b[c, p]       = sum_tap q(gen[(b,c,tap), p]) * x[c, p + off(b,tap)]
//   cat               = [x, out_0, out_1, out_2]
//
// q() rounds the generated tap to the input dtype (bf16/f16), as the
// reference does before consuming it (_triton_kernels.py:332-335).
//
// Work decomposition: one workgroup = (image n, 16-channel block, spatial
// tile of TH=8 rows x TW=32 cols).  The generator is an MFMA GEMM with the
// 16 output channels of one (branch, tap) as M, 16 pixels as N and the input
// channels as K (v_mfma_f32_16x16x32_{bf16,f16}; fp32 runs as three bf16
// products).  The y operand of each wave's 4 pixel blocks stays in registers
// for all 3*K*K (branch, tap) products; the generated taps stay in the MFMA
// result registers and are multiplied against the x halo tile held in LDS
// (channel-innermost, swizzled), so no dynamic kernel ever reaches HBM.

#include "gen_common.h"

namespace ddpm {

constexpr int kGenThreads = 256;
constexpr int kGenRPW = 2;                 // tile rows per wave
constexpr int kGenCPW = 2;                 // 16-pixel column blocks per wave
constexpr int kGenTH = 4 * kGenRPW;        // tile rows
constexpr int kGenTW = 16 * kGenCPW;       // tile cols
constexpr int kGenNB = kGenRPW * kGenCPW;  // pixel blocks per wave

// LDS swizzle of the 4-channel groups inside one pixel (conflict-free reads
// of 4 consecutive channels by 16 consecutive pixels).
template <typename T>
__device__ __forceinline__ int gen_swz(int pix) {
  return sizeof(T) == 4 ? ((pix >> 1) & 3) : ((pix >> 2) & 3);
}

// Loads 8 consecutive weights W[o][k0 .. k0+7] as fp32 (zero past C or for
// rows beyond C output channels).
template <typename T>
__device__ __forceinline__ void load_w8(const T* __restrict__ wt, int64_t o, bool row_ok, int k0,
                                        int C, bool wvec, float (&v)[8]) {
  const T* __restrict__ p = wt + o * C + k0;
  if (row_ok && wvec && k0 + 8 <= C) {
    if constexpr (sizeof(T) == 4) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(p);
      const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] = a[e];
        v[4 + e] = b[e];
      }
    } else {
      typedef T T8 __attribute__((ext_vector_type(8)));
      const T8 a = *reinterpret_cast<const T8*>(p);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = to_f(a[e]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (row_ok && k0 + e < C) ? to_f(p[e]) : 0.f;
  }
}

template <typename T, int KS, int KSTEPS>
__global__ __launch_bounds__(kGenThreads) void gen_fwd_kernel(const T* __restrict__ x,
                                                                const T* __restrict__ y,
                                                                const T* __restrict__ wt,
                                                                const T* __restrict__ bias,
                                                                T* __restrict__ out, GenGeom g) {
  typedef Mma<T> M;
  typedef typename M::V V;
  typedef T T4 __attribute__((ext_vector_type(4)));
  constexpr int KK = KS * KS;
  constexpr int r = KS / 2;

  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int npix = g.LH * g.LW;
  T4* __restrict__ xs = reinterpret_cast<T4*>(smem);                    // [npix][4 groups]
  float* __restrict__ bs = reinterpret_cast<float*>(smem + (size_t)npix * 4 * sizeof(T4));  // [3][KK][16]

  // Block -> (n, tile, channel block), channel block fastest.
  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int cb = bid % g.cblocks;
  const int nt = bid / g.cblocks;
  const int tile = nt % g.tiles;
  const int n = nt / g.tiles;
  const int ty = tile / g.tiles_w, tx = tile - ty * g.tiles_w;
  const int h0 = ty * kGenTH, w0 = tx * kGenTW;
  const int C = g.C;
  const int64_t HW = (int64_t)g.H * g.W;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int col16 = lane & 15, quad = lane >> 4;
  const int c0 = cb * 16;

  // ---- stage x tile (+halo, zero padded) for this channel block; copy the
  //      interior to the identity channels of the output.
  for (int grp = 0; grp < 4; ++grp) {
    for (int pix = tid; pix < npix; pix += kGenThreads) {
      const int i = pix / g.LW, j = pix - i * g.LW;
      const int gh = h0 - g.R + i, gw = w0 - g.R + j;
      const bool in_img = (unsigned)gh < (unsigned)g.H && (unsigned)gw < (unsigned)g.W;
      const bool interior = i >= g.R && i < g.R + kGenTH && j >= g.R && j < g.R + kGenTW;
      T4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int ch = c0 + 4 * grp + e;
        T val = (T)0.f;
        if (in_img && ch < C) {
          const int64_t off = ((int64_t)n * C + ch) * HW + (int64_t)gh * g.W + gw;
          val = x[off];
          if (interior) out[((int64_t)n * 4 * C + ch) * HW + (int64_t)gh * g.W + gw] = val;
        }
        v[e] = val;
      }
      xs[pix * 4 + (grp ^ gen_swz<T>(pix))] = v;
    }
  }
  // ---- bias rows of this channel block, [branch][tap][16]
  for (int idx = tid; idx < 3 * KK * 16; idx += kGenThreads) {
    const int m = idx & 15, bt = idx >> 4;
    const int b = bt / KK, t = bt - b * KK;
    const int ch = c0 + m;
    bs[idx] = ch < C ? to_f(bias[(int64_t)(b * C + ch) * KK + t]) : 0.f;
  }

  // ---- y operand (unshifted pixels) for this wave's pixel blocks
  V bfrag[kGenNB][KSTEPS][M::P];
#pragma unroll
  for (int blk = 0; blk < kGenNB; ++blk) {
    const int gh = h0 + wave * kGenRPW + blk / kGenCPW;
    const int gw = w0 + (blk % kGenCPW) * 16 + col16;
    const bool ok = gh < g.H && gw < g.W;
    const T* __restrict__ yp = y + (int64_t)n * C * HW + (int64_t)gh * g.W + gw;
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) {
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int i = 32 * kk + 8 * quad + e;
        v[e] = (ok && i < C) ? to_f(yp[(int64_t)i * HW]) : 0.f;
      }
      M::pack(v, bfrag[blk][kk]);
    }
  }
  __syncthreads();

  const int crow = c0 + col16;  // channel of this lane's A-fragment row
  const bool crow_ok = crow < C;
  const bool wvec = g.wvec != 0;

  // Flattened (branch, tap) loop; the weight rows of step bt+1 are fetched
  // while step bt runs its MFMAs and epilogue.
  float wnext[KSTEPS][8];
#pragma unroll
  for (int kk = 0; kk < KSTEPS; ++kk)
    load_w8<T>(wt, (int64_t)crow * KK, crow_ok, 32 * kk + 8 * quad, C, wvec, wnext[kk]);
  f32x4 acc[kGenNB];
#pragma unroll 1
  for (int bt = 0; bt < 3 * KK; ++bt) {
    const int b = bt / KK, t = bt - b * KK;
    const int ki = t / KS, kj = t - ki * KS;
    const int d = dil_of(b, g.d0, g.d1, g.d2);
    if (t == 0) {
#pragma unroll
      for (int blk = 0; blk < kGenNB; ++blk) acc[blk] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    V afrag[KSTEPS][M::P];
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) M::pack(wnext[kk], afrag[kk]);
    if (bt + 1 < 3 * KK) {
      const int b1 = (bt + 1) / KK, t1 = (bt + 1) - b1 * KK;
      const int64_t o1 = (int64_t)(b1 * C + crow) * KK + t1;
#pragma unroll
      for (int kk = 0; kk < KSTEPS; ++kk)
        load_w8<T>(wt, o1, crow_ok, 32 * kk + 8 * quad, C, wvec, wnext[kk]);
    }
    const f32x4 binit = *reinterpret_cast<const f32x4*>(bs + bt * 16 + 4 * quad);
    const int dh = (ki - r) * d, dw = (kj - r) * d;
#pragma unroll
    for (int blk = 0; blk < kGenNB; ++blk) {
      f32x4 dacc = binit;
#pragma unroll
      for (int kk = 0; kk < KSTEPS; ++kk) dacc = M::mac(afrag[kk], bfrag[blk][kk], dacc);
      const int lrow = wave * kGenRPW + blk / kGenCPW + g.R + dh;
      const int lcol = (blk % kGenCPW) * 16 + col16 + g.R + dw;
      const int pix = lrow * g.LW + lcol;
      const T4 xv = xs[pix * 4 + (quad ^ gen_swz<T>(pix))];
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[blk][e] = fmaf(quant<T>(dacc[e]), to_f(xv[e]), acc[blk][e]);
    }
    if (t == KK - 1) {
      // ---- store branch b
#pragma unroll
      for (int blk = 0; blk < kGenNB; ++blk) {
        const int gh = h0 + wave * kGenRPW + blk / kGenCPW;
        const int gw = w0 + (blk % kGenCPW) * 16 + col16;
        if (gh < g.H && gw < g.W) {
          T* __restrict__ op = out + ((int64_t)n * 4 * C + (int64_t)(b + 1) * C) * HW +
                               (int64_t)gh * g.W + gw;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int ch = c0 + 4 * quad + e;
            if (ch < C) op[(int64_t)ch * HW] = from_f<T>(acc[blk][e]);
          }
        }
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

}  // namespace

// Shared with gen_bwd.hip.
int gen_make_geom(GenGeom& g, int64_t n, int64_t c, int64_t h, int64_t w, int k, int d0, int d1,
                  int d2) {
  if (n < 0 || c < 0 || h < 0 || w < 0) return kBadArgument;
  if (k < 1 || (k % 2) == 0 || d0 < 1 || d1 < 1 || d2 < 1) return kBadArgument;
  if (k > 3 || c > 64) return kUnsupported;
  if (h > (1 << 20) || w > (1 << 20) || h * w > ((int64_t)1 << 31)) return kUnsupported;
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
  g.cblocks = (int)((c + 15) / 16);
  g.tiles_w = (int)((w + kGenTW - 1) / kGenTW);
  g.tiles = g.tiles_w * (int)((h + kGenTH - 1) / kGenTH);
  g.LH = kGenTH + 2 * g.R;
  g.LW = kGenTW + 2 * g.R;
  g.wvec = 0;
  // fp32 halo tile + bias rows must fit the 64 KB a workgroup may allocate
  if ((size_t)g.LH * g.LW * 16 * sizeof(float) + 3 * k * k * 16 * sizeof(float) > 64 * 1024)
    return kUnsupported;
  if ((int64_t)g.tiles * g.cblocks * n > 0x7fffffffLL) return kUnsupported;
  return kOk;
}

}  // namespace ddpm

using namespace ddpm;

extern "C" int ddpm_gen_fwd(const void* x, const void* y, const void* weight, const void* bias,
                            void* out, int64_t n, int64_t c, int64_t h, int64_t w, int kernel_size,
                            int d0, int d1, int d2, int dtype, hipStream_t stream) {
  if (dtype < kF32 || dtype > kF16) return kBadArgument;
  GenGeom g;
  int st = gen_make_geom(g, n, c, h, w, kernel_size, d0, d1, d2);
  if (st != kOk) return st;
  if (n == 0 || c == 0 || h == 0 || w == 0) return kOk;
  if (!x || !y || !weight || !bias || !out) return kBadArgument;
  g.wvec = ((uintptr_t)weight % 16 == 0) && (c % 8 == 0);
  return with_type(dtype, [&](auto tag) {
    using T = decltype(tag);
    const size_t lds = (size_t)g.LH * g.LW * 16 * sizeof(T) + 3 * kernel_size * kernel_size * 16 * 4;
    const dim3 grid((unsigned)((int64_t)g.N * g.tiles * g.cblocks));
    const dim3 block(kGenThreads);
    const int ksteps = (int)((c + 31) / 32);
    if (kernel_size == 1) {
      if (ksteps == 1)
        hipLaunchKernelGGL((gen_fwd_kernel<T, 1, 1>), grid, block, lds, stream, (const T*)x,
                           (const T*)y, (const T*)weight, (const T*)bias, (T*)out, g);
      else
        hipLaunchKernelGGL((gen_fwd_kernel<T, 1, 2>), grid, block, lds, stream, (const T*)x,
                           (const T*)y, (const T*)weight, (const T*)bias, (T*)out, g);
    } else {
      if (ksteps == 1)
        hipLaunchKernelGGL((gen_fwd_kernel<T, 3, 1>), grid, block, lds, stream, (const T*)x,
                           (const T*)y, (const T*)weight, (const T*)bias, (T*)out, g);
      else
        hipLaunchKernelGGL((gen_fwd_kernel<T, 3, 2>), grid, block, lds, stream, (const T*)x,
                           (const T*)y, (const T*)weight, (const T*)bias, (T*)out, g);
    }
    return (int)hipGetLastError();
  });
}
