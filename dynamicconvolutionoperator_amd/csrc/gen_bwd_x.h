// Halo reduction of the generator's input gradient (second step of
// ddpm_gen_bwd_x): the per-item body shared by its own kernel and by the
// helper workgroups that ddpm_gen_bwd_xw adds to the weight-gradient launch,
// plus the host-side description of a deferred reduction.
#pragma once

#include "gen_tile.h"

namespace ddpm {

// One item = VEC consecutive columns of one row of dX (VEC = 4 needs W % 4 ==
// 0: 16-byte aligned partial groups, as the tile kernel lays them out); items
// are flattened over all rows (n, c, h) so that every lane has work.  The halo of at most one vertical and one horizontal neighbour covers a
// pixel (R <= 8 is at most half a tile side), so the sum is gO_x + own +
// vertical + horizontal + diagonal partial, in that order.
template <typename T, int VEC>
__device__ __forceinline__ void bx_reduce_item(const float* __restrict__ part,
                                               const T* __restrict__ gout, T* __restrict__ gx,
                                               const TileGeom& g, int64_t item) {
  typedef float FV __attribute__((ext_vector_type(4)));
  typedef T TV __attribute__((ext_vector_type(4)));
  const int gpr = (g.W + VEC - 1) / VEC;  // column groups per row
  const int64_t rows = (int64_t)g.N * g.C * g.H;
  if (item >= rows * gpr) return;
  const int row = (int)(item / gpr);      // (n*C + c)*H + h
  const int gi = (int)(item - (int64_t)row * gpr);
  const int w = gi * VEC;
  const int nc = row / g.H, h = row - nc * g.H;
  const int n = nc / g.C, c = nc - n * g.C;
  const int cb = c >> 4, ch = c & 15;
  const int ty = h / kGtTH, lr = h - ty * kGtTH;
  const int tx = w / g.TW, lc = w - tx * g.TW;
  const int tiles_h = g.tiles / g.tiles_w;
  int dy = lr < g.R ? -1 : (lr >= kGtTH - g.R ? 1 : 0);
  if (ty + dy < 0 || ty + dy >= tiles_h) dy = 0;
  int dx = lc < g.R ? -1 : (lc + VEC - 1 >= g.TW - g.R ? 1 : 0);
  if (tx + dx < 0 || tx + dx >= g.tiles_w) dx = 0;
  const int64_t LHp = (int64_t)g.LH * g.LWp;
  auto at = [&](int ddy, int ddx) {
    const int64_t wg = ((int64_t)n * g.tiles + (ty + ddy) * g.tiles_w + tx + ddx) * g.cblocks + cb;
    return part + (wg * 16 + ch) * LHp + (lr + g.R - ddy * kGtTH) * g.LWp +
           (lc + g.R + g.pad - ddx * g.TW);
  };
  const int64_t HW = (int64_t)g.H * g.W;
  const int64_t pix = (int64_t)h * g.W + w;
  const T* __restrict__ go = gout + ((int64_t)n * 4 * g.C + c) * HW + pix;
  T* __restrict__ dst = gx + (int64_t)nc * HW + pix;
  if constexpr (VEC == 4) {
    const TV gv = *reinterpret_cast<const TV*>(go);
    FV s = {to_f(gv[0]), to_f(gv[1]), to_f(gv[2]), to_f(gv[3])};
    s += *reinterpret_cast<const FV*>(at(0, 0));
    if (dy != 0) s += *reinterpret_cast<const FV*>(at(dy, 0));
    if (dx != 0) s += *reinterpret_cast<const FV*>(at(0, dx));
    if (dy != 0 && dx != 0) s += *reinterpret_cast<const FV*>(at(dy, dx));
    const TV o = {from_f<T>(s[0]), from_f<T>(s[1]), from_f<T>(s[2]), from_f<T>(s[3])};
    *reinterpret_cast<TV*>(dst) = o;
  } else {
    float s = to_f(go[0]);
    s += *at(0, 0);
    if (dy != 0) s += *at(dy, 0);
    if (dx != 0) s += *at(0, dx);
    if (dy != 0 && dx != 0) s += *at(dy, dx);
    dst[0] = from_f<T>(s);
  }
}

// A halo reduction whose launch is left to a later kernel: the tile
// partials, gO (its x block is added), dX, the tiling and the item count.
struct BxFinish {
  const float* part;
  const void* gout;
  void* gx;
  TileGeom g;
  int64_t items;
  int vec;  // 4 (W % 4 == 0) or 1
};

// ddpm_gen_bwd_x's work: validates, launches the tile kernel and then either
// the reduction kernel (defer == nullptr) or nothing, describing the
// reduction in *defer instead.  Defined in gen_bwd_x.hip.
int bx_run(const void* y, const void* weight, const void* bias, const void* grad_out,
           void* grad_x, void* workspace, int64_t workspace_bytes, int64_t n, int64_t c,
           int64_t h, int64_t w, int kernel_size, int d0, int d1, int d2, int dtype,
           hipStream_t stream, BxFinish* defer);

// Launches the halo reduction `f` as its own kernel.  Defined in
// gen_bwd_x.hip.
int bx_finish(const BxFinish& f, int dtype, hipStream_t stream);

}  // namespace ddpm
