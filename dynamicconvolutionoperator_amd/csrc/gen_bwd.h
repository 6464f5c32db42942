// Pieces of the fused generator's backward that ddpm_gen_bwd moves into
// other launches: the dY kernel's weight packing (run by helper workgroups of
// the weight-gradient launch, next to dX's halo reduction), the weight
// gradient's split reduction (run by the dY kernel's workgroups), and the host
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

constexpr int kWgMaxSplits = 16;  // weight-gradient split partials at most (the reference's bound)

// The weight gradient's split partials -- fp32 [splits][3*KK*C][C] and
// [splits][3*KK*C] -- summed in split order into grad_weight / grad_bias in
// Conv2d parameter layout.  Item `item` of (3*KK*C*C / V) weight items (V
// consecutive input channels i of one (branch and tap, channel) row each)
// followed by 3*KK*C bias items; larger items do nothing.  Used by the
// reduction kernel and, in ddpm_gen_bwd, by the dY kernel's workgroups.
template <typename T, int V>
__device__ __forceinline__ void wg_reduce_item(const float* __restrict__ pw,
                                               const float* __restrict__ pb,
                                               T* __restrict__ dw_out, T* __restrict__ db_out,
                                               uint32_t C, uint32_t KK, int splits,
                                               uint32_t item) {
  const uint32_t per = 3u * KK * C * C, perb = 3u * KK * C;
  const uint32_t nv = per / V;
  if (item < nv) {
    const uint32_t idx = item * V;
    float v[V];
#pragma unroll
    for (int e = 0; e < V; ++e) v[e] = 0.f;
    auto add = [&](const f32x4& a) {
#pragma unroll
      for (int e = 0; e < V; ++e) v[e] += a[e];
    };
    auto get = [&](int s) {
      const float* __restrict__ src = pw + (size_t)s * per + idx;
      if constexpr (V == 4) return *reinterpret_cast<const f32x4*>(src);
      return (f32x4){src[0], 0.f, 0.f, 0.f};
    };
    if (splits == kWgMaxSplits) {
      // every load in flight before the first add
      f32x4 a[kWgMaxSplits];
#pragma unroll
      for (int s = 0; s < kWgMaxSplits; ++s) a[s] = get(s);
#pragma unroll
      for (int s = 0; s < kWgMaxSplits; ++s) add(a[s]);
    } else {
#pragma unroll 8
      for (int s = 0; s < splits; ++s) add(get(s));
    }
    // idx = (bt*C + c)*C + i  ->  row o = (b*C + c)*KK + t
    const uint32_t row = idx / C, i = idx - row * C;
    const uint32_t bt = row / C, c = row - bt * C;
    const uint32_t b = bt / KK, t = bt - b * KK;
    T* __restrict__ dst = dw_out + ((size_t)(b * C + c) * KK + t) * C + i;
    if constexpr (V == 4) {
      typedef T T4 __attribute__((ext_vector_type(4)));
      *reinterpret_cast<T4*>(dst) =
          (T4){from_f<T>(v[0]), from_f<T>(v[1]), from_f<T>(v[2]), from_f<T>(v[3])};
    } else {
      dst[0] = from_f<T>(v[0]);
    }
  } else if (item < nv + perb) {
    const uint32_t j = item - nv;
    float v = 0.f;
#pragma unroll 8
    for (int s = 0; s < splits; ++s) v += pb[(size_t)s * perb + j];
    const uint32_t bt = j / C, c = j - bt * C;
    const uint32_t b = bt / KK, t = bt - b * KK;
    db_out[(b * C + c) * KK + t] = from_f<T>(v);
  }
}

// A split reduction to be run by another launch: partials, outputs, C, K*K,
// splits, V = 4 (v4) or 1, and the item count (0: nothing to run).
struct WReduce {
  const float* pw;
  const float* pb;
  void* dw;
  void* db;
  uint32_t C, KK;
  int splits;
  int v4;
  int items;
};

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
// red (optional, kYtMain): a weight-gradient split reduction for the dY
// kernel's workgroups to run.
int yt_run(const void* x, const void* weight, const void* grad_out, void* grad_y, void* workspace,
           int64_t workspace_bytes, int64_t n, int64_t c, int64_t h, int64_t w, int kernel_size,
           int d0, int d1, int d2, int dtype, hipStream_t stream, int mode, YPack* pack,
           const WReduce* red = nullptr);

// Launches the packing `p` as its own kernel.  Defined in gen_bwd_y.hip.
int yt_pack(const YPack& p, int kernel_size, int dtype, hipStream_t stream);

}  // namespace ddpm
