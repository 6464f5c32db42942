// Pieces of the 3x3 fuse convolution shared by its input-gradient
// (conv3x3.hip) and weight-gradient (conv_wgrad.hip) launches: the geometry
// of the implicit-GEMM kernel, its weight packing per 64-lane unit, and the
// weight gradient's split reduction per item -- so that ddpm_fuse_conv_bwd
// can run the input gradient's packing inside the weight-gradient launch and
// the weight gradient's reduction inside the input-gradient launch.
#pragma once

#include "gen_common.h"

namespace ddpm {

struct ConvGeom {
  int N, K, M, H, W;  // K input planes, M output planes
  int rs, sw;         // segment rows and columns (rs * sw = kCvPix)
  int tiles_h, tiles_w;
  int nc32;           // ceil(K / 32)
  int mb;             // 16-plane blocks of m per workgroup
  int mgroups;        // ceil(M / (mb * 16))
  int mgl;            // m groups a workgroup runs one after another (divides mgroups)
  int ks;             // splits of the input planes (K): 1, or more for small images
  int cc_per;         // 32-plane chunks per K split
  int seg;            // staged elements per segment row (sw + 2 * kCvPad)
  int x4;             // input rows copied in 16-byte lanes (W % 8 == 0, aligned base)
};

template <typename T>
__host__ __device__ constexpr int cv_parts() {
  return sizeof(T) == 4 ? 2 : 1;
}

// Packed A: 16-byte units [mg][cc][ki][kj][ib][part][lane] (ib < g.mb), lane
// (m = (mg*mb + ib)*16 + (lane & 15), q = lane >> 4) holding
// A[m][cc*32 + 4e + q][ki][kj], e = 0..7 (`nat`: A[m][cc*32 + 8q + e][ki][kj],
// the slot order of the transposing B reads).  `rot` selects the
// input-gradient form (transposed, rotated).  One 64-lane unit `idx` of
// g.mgroups * g.nc32 * 9 * MB * 64 (32-bit: the host bounds it below 2^31).
template <typename T, int MB>
__device__ __forceinline__ void cv_pack_item(const T* __restrict__ wt, uint32_t* __restrict__ pk,
                                             const ConvGeom& g, int rot, int pairs, int nat,
                                             int idx) {
  constexpr int P = cv_parts<T>();
  const int lane = idx & 63;
  int rest = idx >> 6;
  const int ib = rest % MB;
  rest /= MB;
  const int tap = rest % 9;
  rest /= 9;
  const int cc = rest % g.nc32;
  const int mg = rest / g.nc32;
  const int ki = tap / 3, kj = tap - 3 * ki;
  const int m = (mg * MB + ib) * 16 + (lane & 15), q = lane >> 4;
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    // pair planes (kF32Pairs input): slot 8q + e holds channel 2(q + 4(e/2)) + e%2
    const int k = cc * 32 + (pairs ? 2 * q + 8 * (e >> 1) + (e & 1) : nat ? 8 * q + e : 4 * e + q);
    float a = 0.f;
    if (m < g.M && k < g.K) {
      // forward: weight[m][k][ki][kj]; input gradient: weight[k][m][2-ki][2-kj]
      const int64_t off = rot ? (((int64_t)k * g.M + m) * 3 + (2 - ki)) * 3 + (2 - kj)
                              : (((int64_t)m * g.K + k) * 3 + ki) * 3 + kj;
      a = to_f(wt[off]);
    }
    v[e] = a;
  }
  typename Mma<T>::V o[P];
  Mma<T>::pack(v, o);
  u32x4* __restrict__ dst = reinterpret_cast<u32x4*>(pk);
  const int64_t unit = (((((int64_t)mg * g.nc32 + cc) * 9 + tap) * MB + ib) * P) * 64 + lane;
#pragma unroll
  for (int part = 0; part < P; ++part) dst[unit + part * 64] = __builtin_bit_cast(u32x4, o[part]);
}


// A packing to be run by another launch's workgroups (total 0: none).
struct CvPack {
  const void* wt;
  uint32_t* pk;
  ConvGeom g;
  int rot, pairs, nat;
  int total;  // 64-lane units
};

template <typename T>
__device__ __forceinline__ void cv_pack_any(const CvPack& p, int idx) {
  const T* wt = static_cast<const T*>(p.wt);
  if (p.g.mb == 4)
    cv_pack_item<T, 4>(wt, p.pk, p.g, p.rot, p.pairs, p.nat, idx);
  else if (p.g.mb == 2)
    cv_pack_item<T, 2>(wt, p.pk, p.g, p.rot, p.pairs, p.nat, idx);
  else
    cv_pack_item<T, 1>(wt, p.pk, p.g, p.rot, p.pairs, p.nat, idx);
}

// Workgroup `wg` of `wgs`' share of a packing, `nthreads` threads.
template <typename T>
__device__ __forceinline__ void cv_pack_share(const CvPack& p, int wg, int wgs, int tid,
                                              int nthreads) {
  const int per = (p.total + wgs - 1) / wgs;
  for (int j = tid; j < per; j += nthreads) {
    const int idx = wg * per + j;
    if (idx < p.total) cv_pack_any<T>(p, idx);
  }
}

// The weight gradient's split partials -- fp32 [splits][nw] with nw =
// C * 4C * 9 in grad_weight's own [co][ci][t] order, then [splits][C] --
// summed in split order: item `item` of nw / V weight items (V consecutive
// elements) followed by C bias items; larger items do nothing.
constexpr int kCwMaxSplits = 16;
template <typename T, int V>
__device__ __forceinline__ void cw_reduce_item(const float* __restrict__ pw,
                                               const float* __restrict__ pb, T* __restrict__ dw,
                                               T* __restrict__ db, uint32_t nw, uint32_t C,
                                               int splits, uint32_t item) {
  const uint32_t nv = nw / V;
  if (item < nv) {
    const float* __restrict__ src = pw + (size_t)item * V;
    float v[V];
#pragma unroll
    for (int e = 0; e < V; ++e) v[e] = 0.f;
    auto get = [&](int s) {
      if constexpr (V == 4) return *reinterpret_cast<const f32x4*>(src + (size_t)s * nw);
      return (f32x4){src[(size_t)s * nw], 0.f, 0.f, 0.f};
    };
    auto add = [&](const f32x4& a) {
#pragma unroll
      for (int e = 0; e < V; ++e) v[e] += a[e];
    };
    if (splits == kCwMaxSplits) {
      // every load in flight before the first add
      f32x4 a[kCwMaxSplits];
#pragma unroll
      for (int s = 0; s < kCwMaxSplits; ++s) a[s] = get(s);
#pragma unroll
      for (int s = 0; s < kCwMaxSplits; ++s) add(a[s]);
    } else {
#pragma unroll 4
      for (int s = 0; s < splits; ++s) add(get(s));
    }
    T* __restrict__ dst = dw + (size_t)item * V;
    if constexpr (V == 4) {
      typedef T T4 __attribute__((ext_vector_type(4)));
      *reinterpret_cast<T4*>(dst) =
          (T4){from_f<T>(v[0]), from_f<T>(v[1]), from_f<T>(v[2]), from_f<T>(v[3])};
    } else {
      dst[0] = from_f<T>(v[0]);
    }
  } else if (item < nv + C) {
    const uint32_t co = item - nv;
    float v = 0.f;
    for (int s = 0; s < splits; ++s) v += pb[(size_t)s * C + co];
    db[co] = from_f<T>(v);
  }
}

// A split reduction to be run by another launch (items 0: none).
struct CwReduce {
  const float* pw;
  const float* pb;
  void* dw;
  void* db;
  uint32_t nw, C;
  int splits;
  int v4;     // V = 4 (else 1)
  int items;  // nw / V + C
};

// Workgroup `wg` of `wgs`' share of a reduction, `nthreads` threads.
template <typename T>
__device__ __forceinline__ void cw_reduce_share(const CwReduce& r, int wg, int wgs, int tid,
                                                int nthreads) {
  const int per = (r.items + wgs - 1) / wgs;
  for (int j = tid; j < per; j += nthreads) {
    const uint32_t item = (uint32_t)(wg * per + j);
    if (r.v4)
      cw_reduce_item<T, 4>(r.pw, r.pb, (T*)r.dw, (T*)r.db, r.nw, r.C, r.splits, item);
    else
      cw_reduce_item<T, 1>(r.pw, r.pb, (T*)r.dw, (T*)r.db, r.nw, r.C, r.splits, item);
  }
}

// The weight gradient's launch (defined in conv_wgrad.hip), arguments as
// ddpm_fuse_conv_bwd_weight's.  check_only: validate and return before
// launching.  pack (optional): a packing for its workgroups to run.  defer
// (optional): describe the split reduction there (items 0 with one split)
// instead of launching it.
int cw_run(const void* cat, const void* grad_out, void* grad_weight, void* grad_bias,
           void* workspace, int64_t workspace_bytes, int64_t n, int64_t c, int64_t h, int64_t w,
           int dtype, hipStream_t stream, bool check_only, const CvPack* pack, CwReduce* defer);

// The fuse convolution's forward weight packing as a descriptor for another
// launch (defined in conv3x3.hip): validates the forward's shape (n, 4c -> c,
// h, w; `dtype` the concat's code) and workspace (as for ddpm_fuse_conv_fwd),
// and describes packing `weight` into the start of `workspace` in the layout
// the forward over `cat` reads; total 0 for an empty shape.
int cv_fwd_pack(CvPack& p, const void* cat, const void* weight, void* workspace,
                int64_t workspace_bytes, int64_t n, int64_t c, int64_t h, int64_t w, int dtype);

}  // namespace ddpm
