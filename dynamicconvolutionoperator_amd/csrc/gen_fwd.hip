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
// reference does before consuming it (_triton_kernels.py:332-335).  The
// workgroup body (gen_tile.h) keeps the x halo tile in LDS and the generated
// taps in the MFMA result registers; the identity part of the concat is
// written from the registers that stage the halo tile.

#include "gen_tile.h"
#include <type_traits>

namespace ddpm {

// CB = 4: 256 registers per lane (one 8-wave workgroup per CU, whose 133 KB
// halo tile fills the LDS anyway); CB = 2: 128 registers, two workgroups per
// CU, unless the y operand needs more (gt_waves_per_eu).
template <typename T, int KS, int NK, int CB>
__global__ __launch_bounds__(kGtThreads) __attribute__((amdgpu_waves_per_eu(gt_waves_per_eu<T, NK, CB>()))) void gen_fwd_kernel(
    const T* __restrict__ x, const T* __restrict__ y, const T* __restrict__ wt,
    const T* __restrict__ bias, T* __restrict__ out, TileGeom g) {
  gen_tile_body<T, KS, NK, CB, false>(x, y, wt, bias, out, nullptr, g);
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

// Shared with the backward entry points.
int gen_make_geom(GenGeom& g, int64_t n, int64_t c, int64_t h, int64_t w, int k, int d0, int d1,
                  int d2) {
  if (n < 0 || c < 0 || h < 0 || w < 0) return kBadArgument;
  if (k < 1 || (k % 2) == 0 || d0 < 1 || d1 < 1 || d2 < 1) return kBadArgument;
  if (k > 3 || c > 128) return kUnsupported;
  if (h > (1 << 20) || w > (1 << 20) || h * w > ((int64_t)1 << 31)) return kUnsupported;
  if (k == 1) d0 = d1 = d2 = 1;  // a 1x1 tap has no neighbour to dilate
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
  return kOk;
}

}  // namespace ddpm

using namespace ddpm;

extern "C" int ddpm_gen_fwd(const void* x, const void* y, const void* weight, const void* bias,
                            void* out, int64_t n, int64_t c, int64_t h, int64_t w, int kernel_size,
                            int d0, int d1, int d2, int dtype, hipStream_t stream) {
  if (dtype < kF32 || dtype > kF16) return kBadArgument;
  GenGeom gg;
  int st = gen_make_geom(gg, n, c, h, w, kernel_size, d0, d1, d2);
  if (st != kOk) return st;
  if (n == 0 || c == 0 || h == 0 || w == 0) return kOk;
  if (!x || !y || !weight || !bias || !out) return kBadArgument;
  const int esz = dtype == kF32 ? 4 : 2;
  // 32-bit buffer offsets inside one image's [C][H][W] planes (and 16 planes
  // past a channel block's first one)
  if (c * h * w * esz > 0x7fffffffLL || 16 * h * w * esz > 0x7fffffffLL) return kUnsupported;
  TileGeom g;
  size_t lds = 0;
  const int parts = esz == 4 ? 2 : 1;
  const int nk = gt_nk((int)c);
  int cb = 4;
  st = tile_geom_for(g, gg, 4 * esz, parts, cb, lds);
  if (st != kOk) return st;
  return with_type(dtype, [&](auto tag) {
    using T = decltype(tag);
    auto launch = [&](auto kern) {
      const int ae = allow_dynamic_lds(reinterpret_cast<const void*>(kern), lds);
      if (ae != 0) return ae;
      hipLaunchKernelGGL(kern, dim3((unsigned)((int64_t)g.N * g.tiles * g.cblocks)),
                         dim3(kGtThreads), lds, stream, (const T*)x, (const T*)y,
                         (const T*)weight, (const T*)bias, (T*)out, g);
      return (int)hipGetLastError();
    };
    // 1 or 2 chunks of 32 input channels, or 4 (65..128 channels; chunks
    // past C read zeros)
    auto pick = [&](auto ks) {
      constexpr int KS = decltype(ks)::value;
      if (nk > 2) {
        return launch(gen_fwd_kernel<T, KS, 4, 2>);  // 32-column tiles
      }
      if (cb == 4)
        return nk == 1 ? launch(gen_fwd_kernel<T, KS, 1, 4>) : launch(gen_fwd_kernel<T, KS, 2, 4>);
      if (cb == 1)
        return nk == 1 ? launch(gen_fwd_kernel<T, KS, 1, 1>) : launch(gen_fwd_kernel<T, KS, 2, 1>);
      return nk == 1 ? launch(gen_fwd_kernel<T, KS, 1, 2>) : launch(gen_fwd_kernel<T, KS, 2, 2>);
    };
    if (kernel_size == 1) return pick(std::integral_constant<int, 1>());
    return pick(std::integral_constant<int, 3>());
  });
}
