// Gradient with respect to x of the fused op (recompute backward).
//
// Counterpart of _generator_dynamic_cat_bwd_x (_triton_kernels.py:430-531,
// launched at :944-961), which gathers per output pixel q:
//
//   gen[(b,c,t), p] = sum_i W[(b,c,t), i] * y[i, p] + bias[(b,c,t)]
//   dX[c, q] = gO_x[c, q] + sum_{b,t} q(gen[(b,c,t), q - off(b,t)]) * gO_b[c, q - off(b,t)]
//
// q() rounds a generated tap to bf16/f16 as the forward does
// (_triton_kernels.py:512-515).  Here the sum is evaluated in scatter form
// instead: the product q(gen[(b,c,t), p]) * gO_b[c, p] only needs y and gO_b
// at the unshifted pixel p, so every operand is read once per pixel (a gather
// would read y and gO_b once per tap).  Two kernels:
//   1. gen_bwd_x_tile_kernel (body in gen_tile.h, the forward's tiling):
//      per (image, 16-channel block, 16 x 16*CB tile) the generator runs on
//      MFMA with y in registers and weight slices in LDS, and each tap adds
//      its products at p + off into an fp32 LDS accumulator that covers the
//      tile and its halo of radius R = (K/2)*max(d); the accumulator is then
//      written out as this workgroup's partial (in-image pixels only);
//   2. gen_bwd_x_reduce_kernel: dX[c, q] = gO_x[c, q] + the partials of the
//      (at most 2 x 2) workgroups whose accumulator covers q, in a fixed
//      order, so the result is deterministic; 4 columns per thread, every
//      access 16 bytes wide (8 for 2-byte dX) when W % 4 == 0.

#include "gen_bwd_x.h"
#include <type_traits>

namespace ddpm {

template <typename T, int KS, int NK, int CB>
__global__ __launch_bounds__(kGtThreads) __attribute__((amdgpu_waves_per_eu(gt_waves_per_eu<T, NK, CB>()))) void gen_bwd_x_tile_kernel(
    const T* __restrict__ gout, const T* __restrict__ y, const T* __restrict__ wt,
    const T* __restrict__ bias, float* __restrict__ part, TileGeom g) {
  gen_tile_body<T, KS, NK, CB, true>(gout, y, wt, bias, nullptr, part, g);
}

// One thread per item (bx_reduce_item: VEC columns of one row of dX).
template <typename T, int VEC>
__global__ __launch_bounds__(256) void gen_bwd_x_reduce_kernel(const float* __restrict__ part,
                                                               const T* __restrict__ gout,
                                                               T* __restrict__ gx, TileGeom g) {
  bx_reduce_item<T, VEC>(part, gout, gx, g, (int64_t)blockIdx.x * 256 + threadIdx.x);
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

// Tiling of the scatter kernel (tile_geom_for) with 16-byte accumulator
// entries and fp32 weight slices whatever the dtype, so that the workspace
// size depends on the shape alone.
int bx_geom(TileGeom& g, const GenGeom& gg, int& cb, size_t& lds) {
  return tile_geom_for(g, gg, 16, 2, cb, lds);
}

int64_t bx_part_bytes(const TileGeom& g) {
  return (int64_t)g.N * g.tiles * g.cblocks * 16 * g.LH * g.LWp * 4;
}

}  // namespace
}  // namespace ddpm

using namespace ddpm;

extern "C" int64_t ddpm_gen_bwd_x_workspace_bytes(int64_t n, int64_t c, int64_t h, int64_t w,
                                                  int kernel_size, int d0, int d1, int d2) {
  GenGeom gg;
  if (gen_make_geom(gg, n, c, h, w, kernel_size, d0, d1, d2) != kOk) return 0;
  if (n == 0 || c == 0 || h == 0 || w == 0) return 0;
  TileGeom g;
  int cb;
  size_t lds;
  if (bx_geom(g, gg, cb, lds) != kOk) return 0;
  return bx_part_bytes(g);
}

int ddpm::bx_finish(const BxFinish& f, int dtype, hipStream_t stream) {
  return xt_with_type(dtype, [&](auto tag) {
    using T = decltype(tag);
    const dim3 rgrid((unsigned)((f.items + 255) / 256));
    if (f.vec == 4)
      hipLaunchKernelGGL((gen_bwd_x_reduce_kernel<T, 4>), rgrid, dim3(256), 0, stream, f.part,
                         (const T*)f.gout, (T*)f.gx, f.g);
    else
      hipLaunchKernelGGL((gen_bwd_x_reduce_kernel<T, 1>), rgrid, dim3(256), 0, stream, f.part,
                         (const T*)f.gout, (T*)f.gx, f.g);
    return (int)hipGetLastError();
  });
}

int ddpm::bx_run(const void* y, const void* weight, const void* bias, const void* grad_out,
                 void* grad_x, void* workspace, int64_t workspace_bytes, int64_t n, int64_t c,
                 int64_t h, int64_t w, int kernel_size, int d0, int d1, int d2, int dtype,
                 hipStream_t stream, BxFinish* defer) {
  if (dtype < kF32 || dtype > kF16) return kBadArgument;
  GenGeom gg;
  int st = gen_make_geom(gg, n, c, h, w, kernel_size, d0, d1, d2);
  if (st != kOk) return st;
  if (n == 0 || c == 0 || h == 0 || w == 0) return kOk;
  if (!y || !weight || !bias || !grad_out || !grad_x) return kBadArgument;
  const int esz = dtype == kF32 ? 4 : 2;
  // 32-bit buffer offsets inside one image's [C][H][W] planes (and 16 planes
  // past a channel block's first one)
  if (c * h * w * esz > 0x7fffffffLL || 16 * h * w * esz > 0x7fffffffLL) return kUnsupported;
  // reduce: one thread per group of `vec` columns of every row
  const int vec = w % 4 == 0 ? 4 : 1;
  const int64_t ritems = n * c * h * ((w + vec - 1) / vec);
  if ((ritems + 255) / 256 > 0x7fffffffLL || n * c * h > 0x7fffffffLL) return kUnsupported;
  TileGeom g;
  int cb;
  size_t lds;
  st = bx_geom(g, gg, cb, lds);
  if (st != kOk) return st;
  if (!workspace || workspace_bytes < bx_part_bytes(g)) return kWorkspaceTooSmall;
  float* part = (float*)workspace;
  const int nk = gt_nk((int)c);
  return xt_with_type(dtype, [&](auto tag) {
    using T = decltype(tag);
    auto launch = [&](auto kern) {
      const int ae = allow_dynamic_lds(reinterpret_cast<const void*>(kern), lds);
      if (ae != 0) return ae;
      hipLaunchKernelGGL(kern, dim3((unsigned)((int64_t)g.N * g.tiles * g.cblocks)),
                         dim3(kGtThreads), lds, stream, (const T*)grad_out, (const T*)y,
                         (const T*)weight, (const T*)bias, part, g);
      int e = (int)hipGetLastError();
      if (e != 0) return e;
      const BxFinish fin{part, grad_out, grad_x, g, ritems, vec};
      if (defer) {
        *defer = fin;
        return (int)kOk;
      }
      return bx_finish(fin, dtype, stream);
    };
    // 1 or 2 chunks of 32 input channels, or 4 (65..128 channels, always
    // 32-column tiles; chunks past C read zeros)
    auto pick = [&](auto ks) {
      constexpr int KS = decltype(ks)::value;
      if (nk > 2) return launch(gen_bwd_x_tile_kernel<T, KS, 4, 2>);
      if (cb == 4)
        return nk == 1 ? launch(gen_bwd_x_tile_kernel<T, KS, 1, 4>)
                       : launch(gen_bwd_x_tile_kernel<T, KS, 2, 4>);
      if (cb == 1)
        return nk == 1 ? launch(gen_bwd_x_tile_kernel<T, KS, 1, 1>)
                       : launch(gen_bwd_x_tile_kernel<T, KS, 2, 1>);
      return nk == 1 ? launch(gen_bwd_x_tile_kernel<T, KS, 1, 2>)
                     : launch(gen_bwd_x_tile_kernel<T, KS, 2, 2>);
    };
    if (kernel_size == 1) return pick(std::integral_constant<int, 1>());
    return pick(std::integral_constant<int, 3>());
  });
}

extern "C" int ddpm_gen_bwd_x(const void* y, const void* weight, const void* bias,
                              const void* grad_out, void* grad_x, void* workspace,
                              int64_t workspace_bytes, int64_t n, int64_t c, int64_t h, int64_t w,
                              int kernel_size, int d0, int d1, int d2, int dtype,
                              hipStream_t stream) {
  return bx_run(y, weight, bias, grad_out, grad_x, workspace, workspace_bytes, n, c, h, w,
                kernel_size, d0, d1, d2, dtype, stream, nullptr);
}
