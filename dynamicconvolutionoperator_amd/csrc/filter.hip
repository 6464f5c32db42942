// Materialized dynamic dilated depthwise filter: forward, dX and dK.
//
// Counterparts of the reference's _dynamic_cat_fwd / _dynamic_cat_bwd_x /
// _dynamic_cat_bwd_k (_triton_kernels.py:21-254), redesigned for CDNA4.  All
// three are HBM-bandwidth bound (they move 3*K*K + 4 or + 5 planes):
//   * one workgroup = one (n, c) plane x a tile of image rows (4 waves);
//   * the plane the dilated taps read (x for the forward and dK, the three
//     branch gradients for dX) is staged with its halo of R = (K/2)*max(d) in
//     LDS as fp32, zero outside the image, so all dilations read it there;
//   * forward / dK: a lane owns V consecutive pixels (16 bytes of kernel
//     plane: V = 4 for fp32, 8 for 2-byte types; 8 bytes, V = 4, for the
//     2-byte forward at K <= 5) and streams its 3*K*K kernel planes with
//     non-temporal vector loads issued before the x tile is staged (2-byte
//     forward: one branch's ahead); the LDS tile is stored phase-split (column j at phase j % V,
//     index j / V) so each of a lane's V shifted reads is bank-conflict free;
//   * dX is a gather (kernel planes read at the shifted source pixels): a lane
//     owns 16 bytes of consecutive pixels and loads the two aligned 16-byte
//     chunks around each tap's shifted window (realigned in registers by a
//     wave-uniform shift), the branch gradients staged one branch at a time
//     (double-buffered, each with its own dilation's halo), where those tiles
//     fit two workgroups per CU; otherwise one pixel in each of U column
//     blocks of 64, so every load of a kernel plane is 64 consecutive
//     elements;
//   * FP32 accumulation; outputs written once with non-temporal vector
//     stores (streamed, not read back by the kernel), no Unfold buffers.

#include "ddpm_common.h"

#include <type_traits>

namespace ddpm {

struct FilterGeom {
  int N, C, H, W, K;
  int d0, d1, d2;
  int R;         // halo radius (rows and columns)
  int CP;        // staged column pad: R rounded up to a multiple of V
  int lpr_log2;  // log2(lanes per image row); rows per wave = 64 >> lpr_log2
  int TH, TW;    // tile rows / columns
  int tiles_w, tiles;
  int LH;        // staged rows, TH + 2R
  int PS;        // floats per phase of a staged row
  int RS;        // floats per staged row (V * PS)
};

constexpr int kFilterThreads = 256;
constexpr int kFilterWaves = kFilterThreads / 64;

template <typename T, int V>
struct Vec {
  typedef T type __attribute__((ext_vector_type(V)));
};

// V consecutive elements at byte offset `off` of a buffer as fp32 (zero when
// the offset is past the end).
template <typename T, int V>
__device__ __forceinline__ void buf_loadv(BufRes r, uint32_t off, float (&v)[V]) {
  constexpr int B = V * (int)sizeof(T);
  if constexpr (B == 2 || B == 4) {
    v[0] = buf_load1<T>(r, off);
    if constexpr (V == 2) v[1] = buf_load1<T>(r, off + 2);
  } else if constexpr (B == 8) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 a = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
    const typename Vec<T, V>::type t = __builtin_bit_cast(typename Vec<T, V>::type, a);
#pragma unroll
    for (int e = 0; e < V; ++e) v[e] = to_f(t[e]);
  } else if constexpr (B == 16) {
    const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    const typename Vec<T, V>::type t = __builtin_bit_cast(typename Vec<T, V>::type, a);
#pragma unroll
    for (int e = 0; e < V; ++e) v[e] = to_f(t[e]);
  } else {
    static_assert(B == 32, "unsupported vector width");
    const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    const u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(r, off + 16u, 0, 0);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = __uint_as_float(a[e]);
      v[4 + e] = __uint_as_float(b[e]);
    }
  }
}

// Stage plane[h0 - R .. h0 + TH + R) x [w0 - CP .. w0 + TW + CP) into LDS as
// TS (fp32, or the plane's own 2-byte type: half the LDS; zero outside the
// image), phase-split by V.  Items are (row, V-wide
// column group); W % V == 0 so a group is inside or outside the image as a
// whole.  Each thread issues a batch of branch-free buffer loads before
// writing any of them, so the loads are in flight together.
template <typename T, int V, typename TS = float>
__device__ __forceinline__ void stage_plane(TS* __restrict__ s, const T* __restrict__ plane,
                                            const FilterGeom& g, int h0, int w0) {
  constexpr int NB = 8;
  const int groups = (g.TW + 2 * g.CP) / V;
  const int total = g.LH * groups;
  const BufRes res = make_buf(plane, (uint32_t)((int64_t)g.H * g.W * (int64_t)sizeof(T)));
  for (int base = 0; base < total; base += kFilterThreads * NB) {
    float v[NB][V];
    int dst[NB];
#pragma unroll
    for (int k = 0; k < NB; ++k) {
      const int item = base + (int)threadIdx.x + kFilterThreads * k;
      const int i = item / groups, m = item - i * groups;
      const int gh = h0 - g.R + i, gc = w0 - g.CP + m * V;
      const bool ok = item < total && (unsigned)gh < (unsigned)g.H && gc >= 0 && gc < g.W;
      buf_loadv<T, V>(res, ok ? (uint32_t)((int64_t)gh * g.W + gc) * (uint32_t)sizeof(T) : kOob, v[k]);
      dst[k] = item < total ? i * g.RS + m : -1;
    }
#pragma unroll
    for (int k = 0; k < NB; ++k) {
      if (dst[k] >= 0) {
#pragma unroll
        for (int e = 0; e < V; ++e) s[dst[k] + e * g.PS] = from_f<TS>(v[k][e]);
      }
    }
  }
}

// Staged value at tile row `lrow` (0 = first staged row) and staged column j
// = jc + t, for a lane whose first staged column jc is a multiple of V (the
// column pad CP and the lane's V * cl both are): `rb` = lrow * RS + jc / V is
// the lane's part, formed once per staged row, and `t` is
// wave-uniform (a tap's column shift plus the element index), so the phase
// and index arithmetic runs on the scalar unit and a read costs one vector
// add (per-element phase / index / multiply by PS had made the filter
// kernels VALU-bound).
template <int V, typename TS = float>
__device__ __forceinline__ float staged(const TS* __restrict__ s, const FilterGeom& g, int rb,
                                          int t) {
  if constexpr (V == 1) {
    return to_f(s[rb + t]);
  } else {
    constexpr int L = V == 8 ? 3 : (V == 4 ? 2 : 1);
    static_assert(V == 2 || V == 4 || V == 8, "phase split by a power of two");
    return to_f(s[rb + (t & (V - 1)) * g.PS + (t >> L)]);
  }
}

template <typename TX, typename TK, int KS, int V>
__global__ __launch_bounds__(kFilterThreads) void filter_fwd_kernel(const TX* __restrict__ x,
                                                                      const TK* __restrict__ kern,
                                                                      TK* __restrict__ out,
                                                                      FilterGeom g) {
  typedef typename Vec<TK, V>::type KV;
  extern __shared__ float xs[];
  // fp32: neighbouring row tiles of a plane (which share halo rows) on one
  // XCD -- measured 6% faster at 256x256 (so is the fp32 dX gather); the
  // 2-byte forward and the dK kernel measured faster in plain dispatch order
  const int bid = sizeof(TK) == 4 ? xcd_remap(blockIdx.x, gridDim.x) : (int)blockIdx.x;
  const int plane = bid / g.tiles;
  const int tile = bid - plane * g.tiles;
  const int n = plane / g.C, c = plane - n * g.C;
  const int ty = tile / g.tiles_w, tx = tile - ty * g.tiles_w;
  const int h0 = ty * g.TH, w0 = tx * g.TW;
  const int64_t HW = (int64_t)g.H * g.W;
  const int K = KS > 0 ? KS : g.K;
  const int KK = K * K, r = K / 2;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int lpr = 1 << g.lpr_log2;
  const int trow = wave * (64 >> g.lpr_log2) + (lane >> g.lpr_log2);
  const int cl = lane & (lpr - 1);
  const int gh = h0 + trow, gw = w0 + V * cl;
  const bool active = gh < g.H && gw < g.W && trow < g.TH;
  const int64_t p = (int64_t)gh * g.W + gw;
  const int64_t bstride = (int64_t)g.C * KK * HW;
  const TK* __restrict__ kp = kern + ((int64_t)n * 3 * g.C + c) * KK * HW + p;

  // K <= 3: kernel vectors are requested before the x tile is staged, so
  // the streamed loads overlap the staging -- fp32: all 3*K*K of them;
  // 2-byte kernels: branch 0's K*K, and each branch first requests the next
  // branch's (fewer registers, more waves per SIMD: measured 4% faster at
  // 256x256 bf16, 2% slower for fp32)
  constexpr bool PRE = KS > 0 && KS <= 3;
  constexpr bool ROLL = PRE && sizeof(TK) == 2;
  constexpr int NPRE = PRE ? (ROLL ? 1 : 3) * KS * KS : 1;
  constexpr int NNX = ROLL ? KS * KS : 1;
  KV kpre[NPRE], knx[NNX];
  if constexpr (PRE) {
    if (active) {
#pragma unroll
      for (int i = 0; i < NPRE; ++i) {
        const int b = i / (PRE ? KS * KS : 1), t = i - b * (PRE ? KS * KS : 1);
        kpre[i] = __builtin_nontemporal_load(reinterpret_cast<const KV*>(kp + b * bstride + t * HW));
      }
    }
  }
  stage_plane<TX, V>(xs, x + (int64_t)plane * HW, g, h0, w0);
  __syncthreads();
  if (!active) return;  // no barrier below

  TK* __restrict__ op = out + ((int64_t)n * 4 * g.C + c) * HW + p;
  const int64_t ostride = (int64_t)g.C * HW;
  const int jc = g.CP + V * cl;  // staged column of this lane's first pixel
  {
    float xv[V];
#pragma unroll
    for (int v = 0; v < V; ++v) xv[v] = staged<V>(xs, g, (trow + g.R) * g.RS + jc / V, v);
    VecIO<TK, V>::store_nt(op, xv);
  }
#pragma unroll
  for (int b = 0; b < 3; ++b) {
    const int d = dil_of(b, g.d0, g.d1, g.d2);
    if constexpr (ROLL) {
      if (b < 2) {
#pragma unroll
        for (int t = 0; t < KS * KS; ++t)
          knx[t] = __builtin_nontemporal_load(
              reinterpret_cast<const KV*>(kp + (b + 1) * bstride + t * HW));
      }
    }
    float acc[V];
#pragma unroll
    for (int v = 0; v < V; ++v) acc[v] = 0.f;
    for (int ki = 0; ki < K; ++ki) {
      const int rb = (trow + g.R + (ki - r) * d) * g.RS + jc / V;
      for (int kj = 0; kj < K; ++kj) {
        const int t = ki * K + kj;
        KV kv;
        if constexpr (ROLL)
          kv = kpre[t];
        else if constexpr (PRE)
          kv = kpre[b * KS * KS + t];
        else
          kv = __builtin_nontemporal_load(reinterpret_cast<const KV*>(kp + b * bstride + t * HW));
        const int t0 = (kj - r) * d;
#pragma unroll
        for (int v = 0; v < V; ++v) acc[v] = fmaf(to_f(kv[v]), staged<V>(xs, g, rb, t0 + v), acc[v]);
      }
    }
    VecIO<TK, V>::store_nt(op + (b + 1) * ostride, acc);
    if constexpr (ROLL) {
#pragma unroll
      for (int t = 0; t < KS * KS; ++t) kpre[t] = knx[t];
    }
  }
}

template <typename TX, typename TK, int KS, int V>
__global__ __launch_bounds__(kFilterThreads) void filter_bwd_k_kernel(const TX* __restrict__ x,
                                                                        const TK* __restrict__ gout,
                                                                        TK* __restrict__ gk,
                                                                        FilterGeom g) {
  extern __shared__ float xs[];
  const int bid = blockIdx.x;
  const int plane = bid / g.tiles;
  const int tile = bid - plane * g.tiles;
  const int n = plane / g.C, c = plane - n * g.C;
  const int ty = tile / g.tiles_w, tx = tile - ty * g.tiles_w;
  const int h0 = ty * g.TH, w0 = tx * g.TW;
  const int64_t HW = (int64_t)g.H * g.W;
  const int K = KS > 0 ? KS : g.K;
  const int KK = K * K, r = K / 2;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int lpr = 1 << g.lpr_log2;
  const int trow = wave * (64 >> g.lpr_log2) + (lane >> g.lpr_log2);
  const int cl = lane & (lpr - 1);
  const int gh = h0 + trow, gw = w0 + V * cl;
  const bool active = gh < g.H && gw < g.W && trow < g.TH;
  const int64_t p = (int64_t)gh * g.W + gw;

  // branch gradients at this lane's pixels, requested before staging x
  const TK* __restrict__ gp = gout + ((int64_t)n * 4 * g.C + c) * HW + p;
  const int64_t gstride = (int64_t)g.C * HW;
  float go[3][V];
  if (active) {
#pragma unroll
    for (int b = 0; b < 3; ++b) VecIO<TK, V>::load(gp + (b + 1) * gstride, go[b]);
  }
  stage_plane<TX, V>(xs, x + (int64_t)plane * HW, g, h0, w0);
  __syncthreads();
  if (!active) return;

  const int64_t bstride = (int64_t)g.C * KK * HW;
  TK* __restrict__ kp = gk + ((int64_t)n * 3 * g.C + c) * KK * HW + p;
  const int jc = g.CP + V * cl;
#pragma unroll
  for (int b = 0; b < 3; ++b) {
    const int d = dil_of(b, g.d0, g.d1, g.d2);
    for (int ki = 0; ki < K; ++ki) {
      const int rb = (trow + g.R + (ki - r) * d) * g.RS + jc / V;
      for (int kj = 0; kj < K; ++kj) {
        const int t0 = (kj - r) * d;
        float prod[V];
#pragma unroll
        for (int v = 0; v < V; ++v) prod[v] = go[b][v] * staged<V>(xs, g, rb, t0 + v);
        // non-temporal: the 3*K*K planes are written once and not read back
        // here (measured 17% faster than plain stores at 256x256)
        VecIO<TK, V>::store_nt(kp + b * bstride + (int64_t)(ki * K + kj) * HW, prod);
      }
    }
  }
}

// dX[c,q] = gO_x[c,q] + sum_b sum_tap k_b[c,tap,q-off] * gO_b[c,q-off]   (gather form)
// The three branch-gradient tiles (+ halo) are staged together in LDS (V = 1
// layout); the kernel planes are read at the shifted source pixels.  A lane
// owns pixel lane + 64*u of its row for u < U.
template <typename TX, typename TK, int KS, int U>
__global__ __launch_bounds__(kFilterThreads) void filter_bwd_x_kernel(const TK* __restrict__ gout,
                                                                        const TK* __restrict__ kern,
                                                                        TX* __restrict__ gx,
                                                                        FilterGeom g) {
  extern __shared__ float gs[];
  const int bid = blockIdx.x;
  const int plane = bid / g.tiles;
  const int tile = bid - plane * g.tiles;
  const int n = plane / g.C, c = plane - n * g.C;
  const int ty = tile / g.tiles_w, tx = tile - ty * g.tiles_w;
  const int h0 = ty * g.TH, w0 = tx * g.TW;
  const int64_t HW = (int64_t)g.H * g.W;
  const int K = KS > 0 ? KS : g.K;
  const int KK = K * K, r = K / 2;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  // U == 4 tiles are 64 lanes wide (one image row per wave): the row is
  // wave-uniform, so per-row buffer resources stay in scalar registers
  const int lpr = U == 4 ? 64 : 1 << g.lpr_log2;  // lanes per row; lane pixels are lpr apart
  const int trow = U == 4 ? wave : wave * (64 >> g.lpr_log2) + (lane >> g.lpr_log2);
  const int cl = lane & (lpr - 1);
  const int gh = h0 + trow;
  const bool row_active = gh < g.H && trow < g.TH;

  const int64_t bstride = (int64_t)g.C * KK * HW;
  const TK* __restrict__ kp = kern + ((int64_t)n * 3 * g.C + c) * KK * HW;
  const TK* __restrict__ gp = gout + ((int64_t)n * 4 * g.C + c) * HW;
  const int64_t gstride = (int64_t)g.C * HW;
  const int lplane = g.LH * g.RS;

  // kernel values at the gathered source pixels, requested before the
  // branch-gradient tiles are staged.  U == 4: one resource per source row
  // (columns past its end read zero, columns left of it are masked);
  // otherwise one per tap plane, with source pixels outside the image masked
  // by offset.  Both keep the resource wave-uniform.
  constexpr int NT = KS > 0 ? 3 * KS * KS : 1;
  float kvs[KS > 0 ? NT : 1][U];
  auto load_k = [&](int b, int ki, int kj, float (&kv)[U]) {
    const int d = dil_of(b, g.d0, g.d1, g.d2);
    const int dh = (ki - r) * d, dw = (kj - r) * d;
    const int sh = gh - dh;
    const bool sh_ok = row_active && (unsigned)sh < (unsigned)g.H;
    const TK* kt = kp + b * bstride + (int64_t)(ki * K + kj) * HW;
    if constexpr (U == 4) {
      const BufRes res = make_buf(sh_ok ? kt + (int64_t)sh * g.W : kt,
                                  sh_ok ? (uint32_t)(g.W * sizeof(TK)) : 0u);
      const int col0 = w0 + cl - dw;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int col = col0 + 64 * u;
        kv[u] = buf_load1<TK>(res, col >= 0 ? (uint32_t)col * (uint32_t)sizeof(TK) : kOob);
      }
    } else {
      const BufRes res = make_buf(kt, (uint32_t)(HW * (int64_t)sizeof(TK)));
      const int rowel = sh * g.W;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int col = w0 + cl + lpr * u - dw;
        const bool ok = sh_ok && (unsigned)col < (unsigned)g.W;
        kv[u] = buf_load1<TK>(res, ok ? (uint32_t)(rowel + col) * (uint32_t)sizeof(TK) : kOob);
      }
    }
  };
  if constexpr (KS > 0) {
#pragma unroll
    for (int b = 0; b < 3; ++b)
#pragma unroll
      for (int t = 0; t < KS * KS; ++t) load_k(b, t / KS, t % KS, kvs[b * KS * KS + t]);
  }
#pragma unroll
  for (int b = 0; b < 3; ++b) stage_plane<TK, 1>(gs + b * lplane, gp + (b + 1) * gstride, g, h0, w0);
  __syncthreads();
  if (!row_active) return;

  float acc[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int gw = w0 + cl + lpr * u;
    acc[u] = (gw < g.W) ? to_f(gp[(int64_t)gh * g.W + gw]) : 0.f;
  }
#pragma unroll
  for (int b = 0; b < 3; ++b) {
    const int d = dil_of(b, g.d0, g.d1, g.d2);
    const float* __restrict__ gb = gs + b * lplane;
    for (int ki = 0; ki < K; ++ki) {
      const int dh = (ki - r) * d;
      const int lrow = trow + g.R - dh;
      for (int kj = 0; kj < K; ++kj) {
        const int dw = (kj - r) * d;
        float kv[U];
        if constexpr (KS > 0) {
#pragma unroll
          for (int u = 0; u < U; ++u) kv[u] = kvs[(b * K + ki) * K + kj][u];
        } else {
          load_k(b, ki, kj, kv);
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
          acc[u] = fmaf(kv[u], gb[lrow * g.RS + g.CP + cl + lpr * u - dw], acc[u]);
      }
    }
  }
  TX* __restrict__ xo = gx + (int64_t)plane * HW + (int64_t)gh * g.W;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int gw = w0 + cl + lpr * u;
    if (gw < g.W) xo[gw] = from_f<TX>(acc[u]);
  }
}

// Elements s .. s+V-1 of the 2V consecutive kernel-plane elements held in
// two aligned 16-byte chunks (c0 first), as fp32.  s is wave-uniform (it
// depends only on the tap's column shift), so the dword selection is a
// uniform branch and the odd 2-byte shift one v_alignbyte per dword.
template <typename TK, int V>
__device__ __forceinline__ void realign(const u32x4& c0, const u32x4& c1, int s, float (&out)[V]) {
  const uint32_t D[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
  uint32_t e[5];
  const int k = sizeof(TK) == 4 ? s : s >> 1;  // first dword
  switch (k) {
    case 0:
#pragma unroll
      for (int j = 0; j < 5; ++j) e[j] = D[j];
      break;
    case 1:
#pragma unroll
      for (int j = 0; j < 5; ++j) e[j] = D[j + 1];
      break;
    case 2:
#pragma unroll
      for (int j = 0; j < 5; ++j) e[j] = D[j + 2];
      break;
    default:
#pragma unroll
      for (int j = 0; j < 5; ++j) e[j] = D[j + 3];
      break;
  }
  if constexpr (sizeof(TK) == 4) {
#pragma unroll
    for (int v = 0; v < 4; ++v) out[v] = __uint_as_float(e[v]);
  } else {
    const uint32_t sh = (uint32_t)(s & 1) * 2u;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t w = __builtin_amdgcn_alignbyte(e[j + 1], e[j], sh);
      typedef TK T2 __attribute__((ext_vector_type(2)));
      const T2 t = __builtin_bit_cast(T2, w);
      out[2 * j] = to_f(t[0]);
      out[2 * j + 1] = to_f(t[1]);
    }
  }
}

// One branch-gradient plane's part of the staged tile that the dilation d_b
// reads -- staged rows [R - Rb, R + TH + Rb) and columns [CP - CPb, CP + TW +
// CPb), Rb = (K/2) d_b and CPb = Rb rounded up to a multiple of V -- staged
// in two halves: issue() requests it into registers (16-byte loads, zero
// outside the image), commit() writes it to a tile buffer phase-split by V.
// A thread handles at most NB items (row, V-wide column group); the host
// checks that bound.
// CONTIG: rows stored contiguously (column j at row offset j, one 16-byte
// LDS write per group) instead of phase-split by V.
template <typename T, int V, typename TS, int NB, bool CONTIG = false>
struct BranchStage {
  static_assert(V * sizeof(T) == 16, "16-byte groups");
  u32x4 raw[NB];
  int dst[NB];

  __device__ __forceinline__ void issue(const T* __restrict__ plane, const FilterGeom& g, int h0,
                                        int w0, int rb) {
    const int cpb = (rb + V - 1) / V * V;
    const int r0 = g.R - rb, c0 = (g.CP - cpb) / V;
    const int groups = (g.TW + 2 * cpb) / V;
    const int total = (g.TH + 2 * rb) * groups;
    const BufRes res = make_buf(plane, (uint32_t)((int64_t)g.H * g.W * (int64_t)sizeof(T)));
#pragma unroll
    for (int k = 0; k < NB; ++k) {
      const int item = (int)threadIdx.x + kFilterThreads * k;
      const int i = item / groups, m = item - i * groups;
      const int srow = r0 + i, sgrp = c0 + m;
      const int gh = h0 - g.R + srow, gc = w0 - g.CP + sgrp * V;
      const bool ok = item < total && (unsigned)gh < (unsigned)g.H && gc >= 0 && gc < g.W;
      raw[k] = __builtin_amdgcn_raw_buffer_load_b128(
          res, ok ? (uint32_t)((int64_t)gh * g.W + gc) * (uint32_t)sizeof(T) : kOob, 0, 0);
      dst[k] = item < total ? srow * g.RS + (CONTIG ? sgrp * V : sgrp) : -1;
    }
  }

  __device__ __forceinline__ void commit(TS* __restrict__ s, const FilterGeom& g) const {
    typedef typename Vec<T, V>::type TV;
    if constexpr (CONTIG) {
      static_assert(std::is_same<T, TS>::value, "contiguous rows hold the plane's own type");
#pragma unroll
      for (int k = 0; k < NB; ++k)
        if (dst[k] >= 0) *reinterpret_cast<u32x4*>(s + dst[k]) = raw[k];
      return;
    }
#pragma unroll
    for (int k = 0; k < NB; ++k) {
      if (dst[k] >= 0) {
        const TV t = __builtin_bit_cast(TV, raw[k]);
#pragma unroll
        for (int e = 0; e < V; ++e) {
          if constexpr (std::is_same<T, TS>::value)
            s[dst[k] + e * g.PS] = t[e];  // staged in its own type: the bits as loaded
          else
            s[dst[k] + e * g.PS] = from_f<TS>(to_f(t[e]));
        }
      }
    }
  }
};

// Items per thread of BranchStage in filter_bwd_x_vec_kernel.
constexpr int kDxStageItems = 6;

// dX gather with V consecutive pixels per lane (16 bytes of kernel plane;
// W % V == 0): each tap's kernel values at the lane's shifted window come
// from the two aligned 16-byte chunks around it -- two loads per V pixels
// instead of V, every access aligned; the K taps of a kernel row are
// requested together, one row ahead of the FMAs.  The branch gradients are
// staged one branch at a time into two tile buffers (phase-split as in the
// forward), each with only the halo its own dilation reads: branch b+1's
// loads are in flight while branch b's taps run, and the tile takes a third
// of the LDS of staging all three at once, so more workgroups share a CU.
// CONTIG: the branch-gradient tiles hold contiguous rows and a lane reads
// its tap window as the two aligned 16-byte chunks around it, realigned like
// the kernel chunks (two LDS reads per V pixels instead of V).
template <typename TX, typename TK, int KS, int V, bool CONTIG = false>
__global__ __launch_bounds__(kFilterThreads) void filter_bwd_x_vec_kernel(const TK* __restrict__ gout,
                                                                            const TK* __restrict__ kern,
                                                                            TX* __restrict__ gx,
                                                                            FilterGeom g) {
  static_assert(KS >= 1 && V * sizeof(TK) == 16, "16-byte kernel chunks, fixed K");
  constexpr int KK = KS * KS, r = KS / 2;
  constexpr uint32_t E = sizeof(TK);
  // the gradient planes are staged in their own type: 2-byte planes take
  // half the LDS of fp32 ones
  typedef typename std::conditional<sizeof(TK) == 2, TK, float>::type TS;
  extern __shared__ __attribute__((aligned(16))) unsigned char gsm[];
  TS* __restrict__ gs = reinterpret_cast<TS*>(gsm);
  // fp32: neighbouring row tiles of a plane (which stage the same halo rows
  // of the branch gradients) on one XCD, as in the forward (256x256 K=3 95.7
  // -> 93.5 us, A/B; 2-byte planes unchanged or slower)
  const int bid = sizeof(TK) == 4 ? xcd_remap(blockIdx.x, gridDim.x) : (int)blockIdx.x;
  const int plane = bid / g.tiles;
  const int tile = bid - plane * g.tiles;
  const int n = plane / g.C, c = plane - n * g.C;
  const int ty = tile / g.tiles_w, tx = tile - ty * g.tiles_w;
  const int h0 = ty * g.TH, w0 = tx * g.TW;
  const int64_t HW = (int64_t)g.H * g.W;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int lpr = 1 << g.lpr_log2;
  const int trow = wave * (64 >> g.lpr_log2) + (lane >> g.lpr_log2);
  const int cl = lane & (lpr - 1);
  const int gh = h0 + trow, gw = w0 + V * cl;
  const bool active = gh < g.H && gw < g.W && trow < g.TH;
  const TK* __restrict__ gp = gout + ((int64_t)n * 4 * g.C + c) * HW;
  const int64_t gstride = (int64_t)g.C * HW;
  const int lplane = g.LH * g.RS;

  // the K*K tap planes of branch b for this (n, c): one resource per branch
  BufRes kres[3];
#pragma unroll
  for (int b = 0; b < 3; ++b)
    kres[b] = make_buf(kern + (((int64_t)n * 3 + b) * g.C + c) * KK * HW, (uint32_t)(KK * HW * E));
  // chunks of kernel row (b, ki): [tap kj][2]
  auto load_row = [&](int b, int ki, u32x4 (&ch)[KS][2]) {
    const int d = dil_of(b, g.d0, g.d1, g.d2);
    const BufRes kr = b == 0 ? kres[0] : (b == 1 ? kres[1] : kres[2]);
    const int sh = gh - (ki - r) * d;  // source row
    const bool rok = active && (unsigned)sh < (unsigned)g.H;
#pragma unroll
    for (int kj = 0; kj < KS; ++kj) {
      const int dw = (kj - r) * d;
      const int s = ((-dw) % V + V) % V;
      const int a0 = gw - dw - s;  // aligned start of the lane's window
      const uint32_t base = (uint32_t)((ki * KS + kj) * HW + (int64_t)sh * g.W);
      const bool ok0 = rok && a0 >= 0 && a0 < g.W;
      const bool ok1 = rok && a0 + V < g.W && a0 + V >= 0;
      ch[kj][0] = __builtin_amdgcn_raw_buffer_load_b128(kr, ok0 ? (base + (uint32_t)a0) * E : kOob, 0, 0);
      ch[kj][1] = s == 0 ? u32x4{0u, 0u, 0u, 0u}
                         : __builtin_amdgcn_raw_buffer_load_b128(
                               kr, ok1 ? (base + (uint32_t)(a0 + V)) * E : kOob, 0, 0);
    }
  };
  auto halo = [&](int b) { return r * dil_of(b, g.d0, g.d1, g.d2); };

  BranchStage<TK, V, TS, kDxStageItems, CONTIG> st;
  u32x4 nxt[KS][2];
  load_row(0, 0, nxt);
  st.issue(gp + gstride, g, h0, w0, halo(0));
  float acc[V];
  {
    // this lane's gO_x (zero for an inactive lane: it stores nothing)
    const BufRes xr = make_buf(gp, (uint32_t)(HW * (int64_t)E));
    buf_loadv<TK, V>(xr, active ? (uint32_t)((int64_t)gh * g.W + gw) * E : kOob, acc);
  }
  st.commit(gs, g);
  __syncthreads();
  const int jc = g.CP + V * cl;             // staged column of this lane's first pixel
  const int tr = active ? trow : 0;        // rows of inactive lanes stay inside the tile
  // a runtime loop: unrolled, the compiler would hoist every row's loads
#pragma unroll 1
  for (int it = 0; it < 3 * KS; ++it) {
    const int b = it / KS, ki = it - b * KS;
    if (ki == 0 && b < 2) st.issue(gp + (b + 2) * gstride, g, h0, w0, halo(b + 1));
    u32x4 cur[KS][2];
#pragma unroll
    for (int kj = 0; kj < KS; ++kj) {
      cur[kj][0] = nxt[kj][0];
      cur[kj][1] = nxt[kj][1];
    }
    if (it + 1 < 3 * KS) load_row((it + 1) / KS, (it + 1) % KS, nxt);
    const int d = dil_of(b, g.d0, g.d1, g.d2);
    const TS* __restrict__ gb = gs + (b & 1) * lplane;
    const int rb = (tr + g.R - (ki - r) * d) * g.RS + (CONTIG ? jc : jc / V);
#pragma unroll
    for (int kj = 0; kj < KS; ++kj) {
      const int dw = (kj - r) * d;
      const int s = ((-dw) % V + V) % V;
      float kv[V];
      realign<TK, V>(cur[kj][0], cur[kj][1], s, kv);
      if constexpr (CONTIG) {
        // the window [jc - dw, +V) of the lane's staged row: chunks at
        // jc - dw - s and V further (the second only for a shift within a chunk)
        const u32x4* __restrict__ gc = reinterpret_cast<const u32x4*>(gb + rb - dw - s);
        const u32x4 g0 = gc[0];
        const u32x4 g1 = s == 0 ? u32x4{0u, 0u, 0u, 0u} : gc[1];
        float gv[V];
        realign<TK, V>(g0, g1, s, gv);
#pragma unroll
        for (int v = 0; v < V; ++v) acc[v] = fmaf(kv[v], gv[v], acc[v]);
      } else {
#pragma unroll
        for (int v = 0; v < V; ++v) acc[v] = fmaf(kv[v], staged<V, TS>(gb, g, rb, v - dw), acc[v]);
      }
    }
    if (ki == KS - 1 && b < 2) {
      // every wave is past branch b-1, whose buffer branch b+1 takes
      st.commit(gs + ((b + 1) & 1) * lplane, g);
      __syncthreads();
    }
  }
  if (active) VecIO<TX, V>::store_nt(gx + (int64_t)plane * HW + (int64_t)gh * g.W + gw, acc);
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

constexpr size_t kFilterMaxLds = 160 * 1024;

// Tiling for a lane width of `lw` pixels (V consecutive, or U strided) and
// `planes` staged planes.
int make_geom(FilterGeom& g, int64_t n, int64_t c, int64_t h, int64_t w, int k, int d0, int d1,
              int d2, int vec, int lw, int planes, bool row_banks = false) {
  if (n < 0 || c < 0 || h < 0 || w < 0) return kBadArgument;
  if (k < 1 || (k % 2) == 0 || d0 < 1 || d1 < 1 || d2 < 1) return kBadArgument;
  if (c > (1 << 24) || h > (1 << 20) || w > (1 << 20) || h * w > ((int64_t)1 << 29)) return kUnsupported;
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
  if ((int64_t)(k / 2) * dmax > 4096) return kUnsupported;
  g.R = (k / 2) * dmax;
  g.CP = (g.R + vec - 1) / vec * vec;
  int lpr = pow2ceil((int)((w + lw - 1) / lw));
  if (lpr > 64) lpr = 64;
  g.lpr_log2 = ilog2(lpr);
  g.TW = lpr * lw;
  g.TH = kFilterWaves * (64 / lpr);  // each wave covers 64 / lpr image rows
  g.LH = g.TH + 2 * g.R;
  const int cols = g.TW + 2 * g.CP;
  g.PS = (cols + vec - 1) / vec;
  if (row_banks) {
    // the wave's image rows (lpr lanes each) start lpr banks apart, so one
    // phase read of all its rows is conflict-free; no padding when the rows
    // fill the wave or the pitch cannot reach lpr
    if (lpr < 64 && lpr % vec == 0)
      while ((vec * g.PS) % 64 != lpr) ++g.PS;
  } else if (vec > 1) {
    g.PS += ((64 / vec) - g.PS % 64 + 64) % 64;  // phases 64/V banks apart
  }
  g.RS = vec * g.PS;
  if ((size_t)planes * g.LH * g.RS * sizeof(float) > kFilterMaxLds) return kUnsupported;
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

template <typename Kern, typename... Args>
int launch_kernel(Kern kern, const FilterGeom& g, size_t lds, hipStream_t stream, Args... args) {
  const int ae = allow_dynamic_lds(reinterpret_cast<const void*>(kern), lds);
  if (ae != 0) return ae;
  hipLaunchKernelGGL(kern, dim3((unsigned)((int64_t)g.tiles * g.N * g.C)), dim3(kFilterThreads), lds,
                     stream, args...);
  return (int)hipGetLastError();
}

template <typename TX, typename TK, int KS>
int launch_ks(FilterOp op, const void* a, const void* b, void* o, const FilterGeom& g, int vec,
              hipStream_t stream) {
  const size_t lds1 = (size_t)g.LH * g.RS * sizeof(float);
  switch (op) {
    case FilterOp::kFwd:
      if (vec == 8)
        return launch_kernel(filter_fwd_kernel<TX, TK, KS, 8>, g, lds1, stream, (const TX*)a, (const TK*)b, (TK*)o, g);
      if (vec == 4)
        return launch_kernel(filter_fwd_kernel<TX, TK, KS, 4>, g, lds1, stream, (const TX*)a, (const TK*)b, (TK*)o, g);
      return launch_kernel(filter_fwd_kernel<TX, TK, KS, 1>, g, lds1, stream, (const TX*)a, (const TK*)b, (TK*)o, g);
    case FilterOp::kBwdK:
      if (vec == 8)
        return launch_kernel(filter_bwd_k_kernel<TX, TK, KS, 8>, g, lds1, stream, (const TX*)a, (const TK*)b, (TK*)o, g);
      if (vec == 4)
        return launch_kernel(filter_bwd_k_kernel<TX, TK, KS, 4>, g, lds1, stream, (const TX*)a, (const TK*)b, (TK*)o, g);
      return launch_kernel(filter_bwd_k_kernel<TX, TK, KS, 1>, g, lds1, stream, (const TX*)a, (const TK*)b, (TK*)o, g);
    case FilterOp::kBwdX:
      if constexpr (KS >= 1 && 16 % sizeof(TK) == 0) {
        constexpr int VK = 16 / (int)sizeof(TK);
        if (vec == VK)
          return launch_kernel(filter_bwd_x_vec_kernel<TX, TK, KS, VK, true>, g,
                               (size_t)2 * g.LH * g.RS * (sizeof(TK) == 2 ? 2 : 4), stream,
                               (const TK*)a, (const TK*)b, (TX*)o, g);
      }
      // 4 pixels per lane only for K <= 3 (larger K would not keep the
      // in-flight kernel values in registers)
      if constexpr (KS >= 1 && KS <= 3) {
        if (vec == 4)
          return launch_kernel(filter_bwd_x_kernel<TX, TK, KS, 4>, g, 3 * lds1, stream, (const TK*)a, (const TK*)b, (TX*)o, g);
      }
      return launch_kernel(filter_bwd_x_kernel<TX, TK, KS, 1>, g, 3 * lds1, stream, (const TK*)a, (const TK*)b, (TX*)o, g);
  }
  return kBadArgument;
}

template <typename TX, typename TK>
int launch_typed(FilterOp op, const void* a, const void* b, void* o, const FilterGeom& g, int vec,
                 hipStream_t stream) {
  switch (g.K) {
    case 1:
      return launch_ks<TX, TK, 1>(op, a, b, o, g, vec, stream);
    case 3:
      return launch_ks<TX, TK, 3>(op, a, b, o, g, vec, stream);
    case 5:
      return launch_ks<TX, TK, 5>(op, a, b, o, g, vec, stream);
    default:
      return launch_ks<TX, TK, 0>(op, a, b, o, g, vec, stream);
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
  int vec = 1, lw = 1;
  FilterGeom g;
  if (op == FilterOp::kBwdX) {
    // gather with 16 bytes of kernel plane per lane (aligned chunks around
    // each tap's window) where K has a kernel, rows hold whole chunks and a
    // branch's K*K tap planes fit one buffer resource
    const int v = k_dtype == kF32 ? 4 : 8;
    const bool kvec = (k == 1 || k == 3 || k == 5) && w % v == 0 && aligned(a, 16) &&
                      aligned(b, 16) && aligned(o, 16) &&
                      (int64_t)k * k * h * w * (int64_t)esize(k_dtype) <= 0x7fffffffLL;
    // ... and its two branch tiles (fp32, or 2-byte for 2-byte gradients)
    // leave room for two workgroups per CU (measured: at K = 5 with fp32
    // tiles of ~90 KB the vector gather was 30% slower than the
    // one-pixel-per-lane one), and a branch's staging takes at most
    // kDxStageItems 16-byte groups per thread
    if (kvec && make_geom(g, n, c, h, w, k, d0, d1, d2, v, v, 2, true) == kOk &&
        (size_t)2 * g.LH * g.RS * esize(k_dtype) <= kFilterMaxLds / 2 &&
        (int64_t)g.LH * ((g.TW + 2 * g.CP) / v) <= (int64_t)kDxStageItems * kFilterThreads) {
      return with_type(x_dtype, [&](auto tx) {
        using TX = decltype(tx);
        return with_type(k_dtype, [&](auto tk) {
          using TK = decltype(tk);
          return launch_typed<TX, TK>(op, a, b, o, g, v, stream);
        });
      });
    }
    // otherwise U = 4 pixels per lane, 64 lanes apart (K <= 3 keeps the
    // in-flight kernel values within the register budget); unvectorized
    vec = 1;
    lw = (w >= 256 && k <= 3) ? 4 : 1;
  } else {
    // 16 bytes of kernel plane per lane where rows and bases allow it; the
    // 2-byte forward at K <= 5 uses 8 (fewer registers for the kernel vectors
    // in flight, more waves per SIMD: measured 4% faster at 256x256 K=3, 19%
    // at 128x128 K=5)
    const int v = (k_dtype == kF32 || (op == FilterOp::kFwd && k <= 5)) ? 4 : 8;
    // `a` is x for both; its V-wide groups are read as one vector
    const bool ok = (w % v == 0) && aligned(b, 16) && aligned(o, 16) &&
                    aligned(a, (size_t)v * esize(x_dtype));
    if (ok) vec = lw = v;
  }
  int st = make_geom(g, n, c, h, w, k, d0, d1, d2, vec, lw, op == FilterOp::kBwdX ? 3 : 1);
  if (st != kOk) return st;
  return with_type(x_dtype, [&](auto tx) {
    using TX = decltype(tx);
    return with_type(k_dtype, [&](auto tk) {
      using TK = decltype(tk);
      return launch_typed<TX, TK>(op, a, b, o, g, op == FilterOp::kBwdX ? lw : vec, stream);
    });
  });
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
