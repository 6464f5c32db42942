// Gradient with respect to x of the fused op (recompute backward).
//
// Counterpart of _generator_dynamic_cat_bwd_x (_triton_kernels.py:430-531,
// launched at :944-961):
//
//   gen[(b,c,t), p] = sum_i W[(b,c,t), i] * y[i, p] + bias[(b,c,t)]
//   dX[c, q] = gO_x[c, q] + sum_{b,t} q(gen[(b,c,t), q - off(b,t)]) * gO_b[c, q - off(b,t)]
//
// q() rounds a generated tap to bf16/f16 as the forward does
// (_triton_kernels.py:512-515).  The generator is recomputed at the gathered
// source pixels q - off with v_mfma_f32_16x16x32_{bf16,f16} (M = c, N =
// pixels, K = i; fp32 runs as three bf16 products).  Two small packing
// kernels prepare the operands once per call, in a caller-provided workspace:
//   * y transposed to channel-innermost ([n][h][w][part][CP], 16-bit,
//     CP = C rounded up to 32) and, for fp32, split into bf16 hi/lo, so the
//     B fragment of 8 channels at one pixel is a single 16-byte load;
//   * the weight in A-fragment order (split for fp32), one 16 KB slice per
//     (branch, tap) at C = 64, which the workgroup copies global -> LDS one tap
//     ahead and shares among its waves.
// One workgroup covers 4 rows x 32 columns (a wave per row, two 16-pixel
// blocks per wave) and all C output channels.

#include "gen_common.h"
#include <type_traits>

namespace ddpm {

constexpr int kXtRows = 4;                  // tile rows, one wave each
constexpr int kXtCols = 32;                 // tile columns, two blocks per wave
constexpr int kXtThreads = 64 * kXtRows;

struct XGeom {
  int N, C, H, W;
  int d0, d1, d2;
  int tiles_w, tiles;
  int cp;       // channels per pixel in the transposed y (C rounded up to 32)
  int parts;    // 2 for fp32 (hi, lo), 1 for 2-byte types
};

// ---- y -> yT[n][h][w][part][cp] (16-bit), via an LDS transpose of 64-pixel
//      row segments
template <typename T>
__global__ __launch_bounds__(256) void gen_ytrans_kernel(const T* __restrict__ y,
                                                         uint16_t* __restrict__ yt, int C, int H,
                                                         int W, int cp) {
  constexpr int P = Mma<T>::P;
  __shared__ float s[64][65];  // [channel][pixel]
  const int segs = (W + 63) / 64;
  const int row = blockIdx.x / segs;  // n*H + h
  const int w0 = (blockIdx.x - row * segs) * 64;
  const int n = row / H, h = row - n * H;
  const int64_t HW = (int64_t)H * W;
  for (int c0 = 0; c0 < cp; c0 += 64) {
    __syncthreads();
    for (int idx = threadIdx.x; idx < 64 * 64; idx += 256) {
      const int c = idx >> 6, j = idx & 63;
      const int ch = c0 + c, w = w0 + j;
      s[c][j] = (ch < C && w < W) ? to_f(y[((int64_t)n * C + ch) * HW + (int64_t)h * W + w]) : 0.f;
    }
    __syncthreads();
    const int groups = (cp - c0 < 64 ? cp - c0 : 64) / 8;
    for (int item = threadIdx.x; item < 64 * groups; item += 256) {
      const int gq = item % groups, j = item / groups;
      const int w = w0 + j;
      if (w >= W) continue;
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = s[8 * gq + e][j];
      typename Mma<T>::V o[P];
      Mma<T>::pack(v, o);
      u32x4* dst = reinterpret_cast<u32x4*>(yt + ((int64_t)row * W + w) * P * cp + c0 + 8 * gq);
#pragma unroll
      for (int part = 0; part < P; ++part)
        dst[(int64_t)part * cp / 8] = __builtin_bit_cast(u32x4, o[part]);
    }
  }
}

// ---- weight in A-fragment order: 16-byte units [b][t][cb][kk][part][lane],
//      lane (c = cb*16 + (lane & 15), q = lane >> 4) holding
//      W[(b*C + c)*KK + t][kk*32 + 8*q + e], e = 0..7
template <typename T, int KS, int MB>
__global__ __launch_bounds__(256) void gen_pack_w_kernel(const T* __restrict__ wt,
                                                         uint32_t* __restrict__ pk, int C, int nk) {
  constexpr int KK = KS * KS;
  constexpr int P = Mma<T>::P;
  const int total = 3 * KK * MB * nk * 64;
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int lane = idx & 63;
  int rest = idx >> 6;
  const int kk = rest % nk;
  rest /= nk;
  const int cb = rest % MB;
  const int bt = rest / MB;
  const int b = bt / KK, t = bt - b * KK;
  const int c = cb * 16 + (lane & 15), q = lane >> 4;
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int i = kk * 32 + 8 * q + e;
    v[e] = (c < C && i < C) ? to_f(wt[((int64_t)(b * C + c) * KK + t) * C + i]) : 0.f;
  }
  typename Mma<T>::V o[P];
  Mma<T>::pack(v, o);
  u32x4* __restrict__ dst = reinterpret_cast<u32x4*>(pk);
  const int64_t unit = ((int64_t)((bt * MB + cb) * nk + kk) * P) * 64 + lane;
#pragma unroll
  for (int part = 0; part < P; ++part) dst[unit + part * 64] = __builtin_bit_cast(u32x4, o[part]);
}

// CF: C == MB*16, every channel row of the last 16-channel block exists.
template <typename T, int KS, int MB, bool CF>
__global__ __launch_bounds__(kXtThreads) void gen_bwd_x_kernel(const uint16_t* __restrict__ yt,
                                                               const uint32_t* __restrict__ pk,
                                                               const T* __restrict__ bias,
                                                               const T* __restrict__ gout,
                                                               T* __restrict__ gx, XGeom g) {
  typedef Mma<T> M;
  typedef typename M::V V;
  constexpr int KK = KS * KS;
  constexpr int r = KS / 2;
  constexpr int P = M::P;
  constexpr int NK = (MB + 1) / 2;               // 32-channel K steps
  constexpr int AU = MB * NK * P * 64;           // 16-byte units per tap
  constexpr int E = (int)sizeof(T);
  extern __shared__ __attribute__((aligned(16))) uint32_t xsm[];
  uint32_t* __restrict__ abuf = xsm;                                   // [2][AU*4]
  float* __restrict__ bs = reinterpret_cast<float*>(xsm + 2 * AU * 4);  // [3*KK][MB*16]

  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int tile = bid % g.tiles;
  const int n = bid / g.tiles;
  const int ty = tile / g.tiles_w, tx = tile - ty * g.tiles_w;
  const int C = g.C, H = g.H, W = g.W;
  const int64_t HW = (int64_t)H * W;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int col16 = lane & 15, quad = lane >> 4;
  const int h = ty * kXtRows + wave;
  const int wb = tx * kXtCols + col16;  // column of block 0 (block 1 is +16)

  auto stage_a = [&](int bt, int buf) {
    const BufRes res = make_buf(pk + (int64_t)bt * AU * 4, (uint32_t)(AU * 16));
#pragma unroll
    for (int j = 0; j < (AU / 64 + kXtRows - 1) / kXtRows; ++j) {
      const int u = wave + kXtRows * j;
      if ((AU / 64) % kXtRows == 0 || u < AU / 64)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            res, (__attribute__((address_space(3))) void*)(abuf + buf * AU * 4 + 256 * u), 16,
            (uint32_t)(u * 64 + lane) * 16u, 0, 0, 0);
    }
  };

  stage_a(0, 0);
  for (int idx = tid; idx < 3 * KK * MB * 16; idx += kXtThreads) {
    const int m = idx % (MB * 16), bt = idx / (MB * 16);
    const int b = bt / KK, t = bt - b * KK;
    bs[idx] = m < C ? to_f(bias[(int64_t)(b * C + m) * KK + t]) : 0.f;
  }

  // identity branch of the concat
  const T* __restrict__ go = gout + (int64_t)n * 4 * C * HW;
  f32x4 acc[2][MB];
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    const int w = wb + 16 * blk;
    const bool ok = h < H && w < W;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int ch = mb * 16 + 4 * quad + e;
        acc[blk][mb][e] = (ok && ch < C) ? to_f(go[(int64_t)ch * HW + (int64_t)h * W + w]) : 0.f;
      }
  }
  const BufRes yres = make_buf(yt + (int64_t)n * HW * P * g.cp, (uint32_t)(HW * P * g.cp * 2));
  const BufRes gres = make_buf(go + (int64_t)C * HW, (uint32_t)(3 * C * HW * E));
  constexpr int CPc = NK * 32;                       // channels per pixel of the transposed y
  const uint32_t HWE = (uint32_t)HW * (uint32_t)E;   // bytes of one channel plane

  // Operands of one step (one 16-pixel block at one (branch, tap)): the B
  // fragments (8 consecutive channels of y at the source pixel) and the branch
  // gradient at the source pixel, channels mb*16 + 4*quad + e.  The next
  // step's set is loaded while the current one is consumed.
  struct Ops {
    V bf[NK][P];
    float gv[MB][4];
  };
  auto load_ops = [&](int bt, int blk, Ops& o) {
    const int b = bt / KK, t = bt - b * KK;
    const int ki = t / KS, kj = t - ki * KS;
    const int d = dil_of(b, g.d0, g.d1, g.d2);
    const int sh = h - (ki - r) * d;
    const int sw = wb + 16 * blk - (kj - r) * d;
    const bool ok = (unsigned)sh < (unsigned)H && (unsigned)sw < (unsigned)W;
    const uint32_t sp = (uint32_t)(sh * W + sw);
    // y: one offset per lane (kOob outside the image), the (kk, part) slice
    // as the instruction's immediate offset (read as zero past the end too)
    const uint32_t yoff = ok ? (sp * (uint32_t)(P * CPc) + 8 * quad) * 2u : kOob;
#pragma unroll
    for (int kk = 0; kk < NK; ++kk)
#pragma unroll
      for (int pp = 0; pp < P; ++pp)
        o.bf[kk][pp] = __builtin_bit_cast(
            V, __builtin_amdgcn_raw_buffer_load_b128(yres, yoff + (pp * CPc + kk * 32) * 2, 0, 0));
    const uint32_t goff = ((uint32_t)(b * C) * (uint32_t)HW + sp) * (uint32_t)E;
    if constexpr (CF) {
      // lane part of the channel in the offset, the uniform part (mb*16 + e)
      // planes in soffset: a masked lane's kOob stays past the end either way
      const uint32_t gq = ok ? goff + (uint32_t)(4 * quad) * HWE : kOob;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t so = (uint32_t)(mb * 16 + e) * HWE;
          if constexpr (E == 4)
            o.gv[mb][e] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(gres, gq, so, 0));
          else
            o.gv[mb][e] = to_f(__builtin_bit_cast(
                T, (unsigned short)__builtin_amdgcn_raw_buffer_load_b16(gres, gq, so, 0)));
        }
    } else {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int ch = mb * 16 + 4 * quad + e;
          o.gv[mb][e] = buf_load1<T>(gres, (ok && ch < C) ? goff + (uint32_t)ch * HWE : kOob);
        }
    }
  };
  // Generator at the source pixels of one step (A fragments of the tap are in
  // registers), rounded like the forward and weighted by the branch gradient.
  auto step = [&](const V (&afr)[MB][NK][P], const float* __restrict__ bsl, const Ops& o,
                  f32x4 (&ac)[MB]) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      f32x4 dacc = *reinterpret_cast<const f32x4*>(bsl + mb * 16 + 4 * quad);
#pragma unroll
      for (int kk = 0; kk < NK; ++kk) dacc = M::mac(afr[mb][kk], o.bf[kk], dacc);
#pragma unroll
      for (int e = 0; e < 4; ++e) ac[mb][e] = fmaf(quant<T>(dacc[e]), o.gv[mb][e], ac[mb][e]);
    }
  };

  Ops o0, o1;
  load_ops(0, 0, o0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

#pragma unroll 1
  for (int bt = 0; bt < 3 * KK; ++bt) {
    const int buf = bt & 1;
    if (bt + 1 < 3 * KK) stage_a(bt + 1, buf ^ 1);
    load_ops(bt, 1, o1);
    const uint32_t* __restrict__ ab = abuf + buf * AU * 4;
    V afr[MB][NK][P];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int kk = 0; kk < NK; ++kk)
#pragma unroll
        for (int pp = 0; pp < P; ++pp)
          afr[mb][kk][pp] = __builtin_bit_cast(
              V, *reinterpret_cast<const u32x4*>(ab + 4 * (((mb * NK + kk) * P + pp) * 64 + lane)));
    const float* __restrict__ bsl = bs + bt * (MB * 16);
    step(afr, bsl, o0, acc[0]);
    if (bt + 1 < 3 * KK) load_ops(bt + 1, 0, o0);
    step(afr, bsl, o1, acc[1]);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }

#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    const int w = wb + 16 * blk;
    if (h < H && w < W) {
      T* __restrict__ xo = gx + (int64_t)n * C * HW + (int64_t)h * W + w;
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
int xt_with_type(int dt, F&& f) {
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
int xt_with_mb(int mb, F&& f) {
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

int64_t xt_cp(int64_t c) { return (c + 31) / 32 * 32; }

// workspace: packed weight (fp32 size), then the transposed y (two parts)
int64_t xt_pack_bytes(int64_t c, int k) {
  const int64_t mb = (c + 15) / 16, nk = (mb + 1) / 2;
  return 3 * (int64_t)k * k * mb * nk * 2 * 64 * 16;
}
int64_t xt_yt_bytes(int64_t n, int64_t c, int64_t h, int64_t w) { return n * h * w * 2 * xt_cp(c) * 2; }

}  // namespace
}  // namespace ddpm

using namespace ddpm;

extern "C" int64_t ddpm_gen_bwd_x_workspace_bytes(int64_t n, int64_t c, int64_t h, int64_t w,
                                                  int kernel_size) {
  if (n <= 0 || c <= 0 || c > 64 || h <= 0 || w <= 0 || kernel_size < 1) return 0;
  return xt_pack_bytes(c, kernel_size) + xt_yt_bytes(n, c, h, w);
}

extern "C" int ddpm_gen_bwd_x(const void* y, const void* weight, const void* bias,
                              const void* grad_out, void* grad_x, void* workspace,
                              int64_t workspace_bytes, int64_t n, int64_t c, int64_t h, int64_t w,
                              int kernel_size, int d0, int d1, int d2, int dtype,
                              hipStream_t stream) {
  if (dtype < kF32 || dtype > kF16) return kBadArgument;
  GenGeom gg;
  int st = gen_make_geom(gg, n, c, h, w, kernel_size, d0, d1, d2);
  if (st != kOk) return st;
  if (n == 0 || c == 0 || h == 0 || w == 0) return kOk;
  if (!y || !weight || !bias || !grad_out || !grad_x) return kBadArgument;
  const int esz = dtype == kF32 ? 4 : 2;
  // 32-bit buffer offsets inside one image
  if (h * w * 2 * xt_cp(c) * 2 > 0x7fffffffLL || 3 * c * h * w * esz > 0x7fffffffLL)
    return kUnsupported;
  if (n * h > 0x7fffffffLL / 64) return kUnsupported;
  const int64_t need = ddpm_gen_bwd_x_workspace_bytes(n, c, h, w, kernel_size);
  if (!workspace || workspace_bytes < need) return kWorkspaceTooSmall;
  XGeom g;
  g.N = (int)n;
  g.C = (int)c;
  g.H = (int)h;
  g.W = (int)w;
  g.d0 = gg.d0;
  g.d1 = gg.d1;
  g.d2 = gg.d2;
  g.tiles_w = (int)((w + kXtCols - 1) / kXtCols);
  g.tiles = g.tiles_w * (int)((h + kXtRows - 1) / kXtRows);
  g.cp = (int)xt_cp(c);
  if ((int64_t)g.tiles * n > 0x7fffffffLL) return kUnsupported;
  uint32_t* pk = (uint32_t*)workspace;
  uint16_t* yt = (uint16_t*)((char*)workspace + xt_pack_bytes(c, kernel_size));
  const int mb = (int)((c + 15) / 16);
  return xt_with_type(dtype, [&](auto tag) {
    using T = decltype(tag);
    g.parts = Mma<T>::P;
    return xt_with_mb(mb, [&](auto mbc) {
      constexpr int MB = decltype(mbc)::value;
      constexpr int NK = (MB + 1) / 2;
      auto launch = [&](auto ks) {
        constexpr int KS = decltype(ks)::value;
        const int units = 3 * KS * KS * MB * NK * 64;
        hipLaunchKernelGGL((gen_pack_w_kernel<T, KS, MB>), dim3((units + 255) / 256), dim3(256), 0,
                           stream, (const T*)weight, pk, (int)c, NK);
        int e = (int)hipGetLastError();
        if (e != 0) return e;
        const int64_t segs = n * h * ((w + 63) / 64);
        hipLaunchKernelGGL((gen_ytrans_kernel<T>), dim3((unsigned)segs), dim3(256), 0, stream,
                           (const T*)y, yt, (int)c, (int)h, (int)w, g.cp);
        e = (int)hipGetLastError();
        if (e != 0) return e;
        constexpr int AU = MB * NK * Mma<T>::P * 64;
        const size_t lds = (size_t)2 * AU * 16 + (size_t)3 * KS * KS * MB * 16 * sizeof(float);
        const dim3 grid((unsigned)((int64_t)g.N * g.tiles));
        if (c == MB * 16)
          hipLaunchKernelGGL((gen_bwd_x_kernel<T, KS, MB, true>), grid, dim3(kXtThreads), lds,
                             stream, (const uint16_t*)yt, (const uint32_t*)pk, (const T*)bias,
                             (const T*)grad_out, (T*)grad_x, g);
        else
          hipLaunchKernelGGL((gen_bwd_x_kernel<T, KS, MB, false>), grid, dim3(kXtThreads), lds,
                             stream, (const uint16_t*)yt, (const uint32_t*)pk, (const T*)bias,
                             (const T*)grad_out, (T*)grad_x, g);
        return (int)hipGetLastError();
      };
      if (kernel_size == 1) return launch(std::integral_constant<int, 1>());
      if (kernel_size == 3) return launch(std::integral_constant<int, 3>());
      return (int)kUnsupported;
    });
  });
}
