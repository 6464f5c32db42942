// Pieces of the fused generator's backward that ddpm_gen_bwd moves into
// other launches: the dY kernel's weight packing (run by helper workgroups of
// the weight-gradient launch, next to dX's halo reduction), and the host
// entry points of the dY path the combined call drives.
#pragma once

#include "gen_bwd_x.h"

namespace ddpm {

// Packed weight for the dY kernel's A fragments: 16-byte units
//   [ih][b][cc][t][ib][part][lane]   lane (i = (ih*MB + ib)*16 + (lane & 15),
//   q = lane >> 4) holding W[(b*C + c)*KK + t][i] for c = cc*32 + 4*e + q,
//   e = 0..7 (ih: the output-channel half of a workgroup; ib < MB).
template <typename T>
__host__ __device__ constexpr int yt_parts() {
  return sizeof(T) == 4 ? 2 : 1;
}

// One thread's share of the packing: 64-lane unit `idx` of
// ihalves * 3 * nc32 * KS*KS * MB * 64.
template <typename T, int KS, int MB>
__device__ __forceinline__ void yt_pack_item(const T* __restrict__ wt, uint32_t* __restrict__ pk,
                                             int C, int nc32, int idx) {
  constexpr int KK = KS * KS;
  constexpr int P = yt_parts<T>();
  const int lane = idx & 63;
  int rest = idx >> 6;
  const int ib = rest % MB;
  rest /= MB;
  const int t = rest % KK;
  rest /= KK;
  const int cc = rest % nc32;
  rest /= nc32;
  const int b = rest % 3;
  const int ih = rest / 3;
  const int i = (ih * MB + ib) * 16 + (lane & 15), q = lane >> 4;
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int c = cc * 32 + 4 * e + q;
    v[e] = (i < C && c < C) ? to_f(wt[((int64_t)(b * C + c) * KK + t) * C + i]) : 0.f;
  }
  typename Mma<T>::V o[P];
  Mma<T>::pack(v, o);
  u32x4* __restrict__ dst = reinterpret_cast<u32x4*>(pk);
  const int64_t unit = (((((int64_t)ih * 3 + b) * nc32 + cc) * KK + t) * MB + ib) * P * 64 + lane;
#pragma unroll
  for (int part = 0; part < P; ++part) dst[unit + part * 64] = __builtin_bit_cast(u32x4, o[part]);
}

// A dY weight packing to be run by another launch: weight, destination, C,
// 32-channel chunks and the number of 64-lane units (items).
struct YPack {
  const void* wt;
  uint32_t* pk;
  int C, nc32;
  int total;
};

// ddpm_gen_bwd_y's work by mode.  Defined in gen_bwd_y.hip.
enum YtMode {
  kYtFull = 0,   // validate, pack the weight into `workspace`, run the dY kernel
  kYtCheck = 1,  // validate only; describe the packing in *pack (total 0: empty shape)
  kYtMain = 2,   // run the dY kernel only: `workspace` already holds the packed weight
};
int yt_run(const void* x, const void* weight, const void* grad_out, void* grad_y, void* workspace,
           int64_t workspace_bytes, int64_t n, int64_t c, int64_t h, int64_t w, int kernel_size,
           int d0, int d1, int d2, int dtype, hipStream_t stream, int mode, YPack* pack);

// Launches the packing `p` as its own kernel.  Defined in gen_bwd_y.hip.
int yt_pack(const YPack& p, int kernel_size, int dtype, hipStream_t stream);

}  // namespace ddpm
