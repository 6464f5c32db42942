// Generator weight / bias gradient of the fused op (recompute backward).
//
// Counterpart of _generator_dynamic_cat_bwd_weight_partial and
// _generator_dynamic_cat_bwd_weight_reduce (_triton_kernels.py:626-811,
// launched at :973-1053):
//
//   dK[(b,c,t), p] = gO_b[c, p] * x[c, p + off(b,t)]
//   dW[(b,c,t), i] = sum_p dK[(b,c,t), p] * y[i, p]
//   db[(b,c,t)]    = sum_p dK[(b,c,t), p]
//
// Work decomposition (CDNA4): one workgroup per (token split, branch b,
// 16-channel block of c).  Splits are ranges of image rows; at most 16 of
// them write fp32 partials that a second kernel sums in a fixed order
// (deterministic, no atomics).  A workgroup walks its rows in steps of one
// row segment of 128 columns.  Everything a step reads -- the K rows
// {h-d, h, h+d} of x (128 + 16 columns, 16 channels), the y row (all C
// channels) and the branch-gradient row (16 channels) -- is copied
// global -> LDS by buffer loads that write LDS directly (no registers; reads
// outside the image return zero), one step ahead into a second buffer.
// Wave (segment sg, tap half th) owns 32 tokens of the step and half of the
// K*K taps; it accumulates its taps x 16 c x C i with
// v_mfma_f32_16x16x32_{bf16,f16} (M = c, N = i, K = tokens; fp32 operands
// run as three bf16 products).  Two waves share each SIMD, so one wave's VALU
// work (forming and splitting dK) overlaps the other's MFMAs.

#include "gen_common.h"
#include <type_traits>

namespace ddpm {

constexpr int kWgSegs = 4;                   // 32-token segments per step
constexpr int kWgTW = 32 * kWgSegs;          // columns per step
constexpr int kWgPad = 8;                    // staged column halo (>= dilation), even
constexpr int kWgLW = kWgTW + 2 * kWgPad;    // staged x columns
constexpr int kWgMaxDil = kWgPad;
constexpr int kWgMaxSplits = 16;
constexpr int kWgTokensPerSplit = 1024;      // split target below the cap

struct WGradGeom {
  int N, C, H, W;
  int d0, d1, d2;
  int cblocks;         // ceil(C / 16)
  int col_blocks;      // ceil(W / kWgTW)
  int splits;
  int rows_per_split;  // image rows (n, h) per split
  int rows;            // N * H
  int direct;          // one split: write grad_weight / grad_bias directly
  int dma;             // rows start on dword boundaries: LDS-direct dword copies
  int x4;              // W % 8 == 0 and 16-byte aligned y / grad_out: 16-byte copies
};

// Tap halves per kernel size: the K = 3 taps are split over two waves.
template <int KS>
struct WgTaps {
  static constexpr int kHalves = KS == 1 ? 1 : 2;
  static constexpr int kPer = (KS * KS + kHalves - 1) / kHalves;
};

// One LDS staging buffer (dwords; elements of T packed):
//   x rows [KS*16][kXSD]   pitch 2 (mod 32) dwords; read element-wise
//   y rows [MB*16][kYC]    16-byte chunks, chunk k of row i stored at
//   g rows [16][kYC]       position k ^ (i & 15): the 16-byte B-fragment
//                          reads of 16 rows at one k hit distinct banks
template <typename T, int KS, int MB>
struct WgLds {
  static constexpr int kPerD = 4 / (int)sizeof(T);             // elements per dword
  static constexpr int kPerC = 4 * kPerD;                      // elements per 16-byte chunk
  static constexpr int kXD = kWgLW / kPerD;                    // dwords per staged x row
  static constexpr int kXI = (kXD + 63) / 64;                  // 64-dword copies per x row
  static constexpr int kXSD = kXD + ((2 - kXD % 32) + 32) % 32;
  static constexpr int kYC = kWgTW / kPerC;                    // chunks per y / g row (32 / 16)
  static constexpr int kYD = 4 * kYC;                          // dwords per y / g row
  static constexpr int kRPI = 64 / kYC;                        // y / g rows per 1 KB copy
  static constexpr int kXRows = KS * 16;
  static constexpr int kYRows = MB * 16;
  static constexpr int kYOff = kXRows * kXSD;
  static constexpr int kGOff = kYOff + kYRows * kYD;
  static constexpr int kBuf = kGOff + 16 * kYD;
  static_assert(kYC >= 16, "the chunk swizzle needs 16 chunks per row");
};

template <typename T>
__device__ __forceinline__ float lds_elem(const uint32_t* __restrict__ base, int idx) {
  if constexpr (sizeof(T) == 4) {
    return __uint_as_float(base[idx]);
  } else {
    return to_f(reinterpret_cast<const T*>(base)[idx]);
  }
}

// 8 consecutive elements of an LDS row as fp32: for fp32 the two 16-byte
// chunks at dwords p0 and p1, for 2-byte types the chunk at p0.
template <typename T>
__device__ __forceinline__ void lds_chunks8(const uint32_t* __restrict__ row, int p0, int p1,
                                            float (&v)[8]) {
  if constexpr (sizeof(T) == 4) {
    const u32x4 a = *reinterpret_cast<const u32x4*>(row + p0);
    const u32x4 b = *reinterpret_cast<const u32x4*>(row + p1);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = __uint_as_float(a[e]);
      v[4 + e] = __uint_as_float(b[e]);
    }
  } else {
    typedef T T8 __attribute__((ext_vector_type(8)));
    const T8 t = __builtin_bit_cast(T8, *reinterpret_cast<const u32x4*>(row + p0));
    (void)p1;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = to_f(t[e]);
  }
}

// Position of a step: image n, row h, first column w0 (column block cbk).
struct WgPos {
  int n, h, w0, cbk;
  __device__ __forceinline__ void advance(const WGradGeom& g) {
    w0 += kWgTW;
    if (++cbk == g.col_blocks) {
      cbk = 0;
      w0 = 0;
      if (++h == g.H) {
        h = 0;
        ++n;
      }
    }
  }
};

template <typename T, int KS, int MB>
__global__ __launch_bounds__(64 * kWgSegs * WgTaps<KS>::kHalves) void gen_bwd_w_partial_kernel(
    const T* __restrict__ x, const T* __restrict__ y, const T* __restrict__ gout,
    float* __restrict__ pw, float* __restrict__ pb, T* __restrict__ dw_out, T* __restrict__ db_out,
    WGradGeom g) {
  typedef Mma<T> M;
  typedef typename M::V V;
  typedef WgLds<T, KS, MB> L;
  constexpr int KK = KS * KS;
  constexpr int r = KS / 2;
  constexpr int NH = WgTaps<KS>::kHalves;
  constexpr int TPH = WgTaps<KS>::kPer;
  constexpr int NW = kWgSegs * NH;
  constexpr int NT = 64 * NW;
  constexpr int E = (int)sizeof(T);
  extern __shared__ __attribute__((aligned(16))) uint32_t wsm[];

  const int logical = xcd_remap(blockIdx.x, gridDim.x);
  const int per_split = 3 * g.cblocks;
  const int split = logical / per_split;
  const int rem = logical - split * per_split;
  const int b = rem / g.cblocks;
  const int cb = rem - b * g.cblocks;
  const int d = dil_of(b, g.d0, g.d1, g.d2);
  const int C = g.C, H = g.H, W = g.W;
  const int64_t HW = (int64_t)H * W;
  const int64_t CHW = (int64_t)C * HW;
  const uint32_t plane_bytes = (uint32_t)(CHW * E);
  const uint32_t row_bytes = (uint32_t)(W * E);
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int col16 = lane & 15, quad = lane >> 4;
  const int sg = wave % kWgSegs, th = wave / kWgSegs;

  const int row_beg = split * g.rows_per_split;
  int row_end = row_beg + g.rows_per_split;
  if (row_end > g.rows) row_end = g.rows;
  const int steps = row_end > row_beg ? (row_end - row_beg) * g.col_blocks : 0;
  const T* __restrict__ gbase = gout + (int64_t)(b + 1) * C * HW;

  // ---- operands of step `p` -> LDS buffer `buf`
  auto stage = [&](const WgPos& p, int buf) {
    uint32_t* __restrict__ dstb = wsm + buf * L::kBuf;
    if (g.dma) {
      // x rows: copies of 64 dwords (lane l moves dword l) from a resource
      // spanning one image row, so columns outside the image read zero
#pragma unroll
      for (int j = 0; j < (L::kXRows + NW - 1) / NW; ++j) {
        const int pr = wave + NW * j;
        if (L::kXRows % NW != 0 && pr >= L::kXRows) break;
        const int rr = pr >> 4, c = pr & 15;
        const int ch = cb * 16 + c, hh = p.h + (rr - r) * d;
        const bool ok = ch < C && (unsigned)hh < (unsigned)H;
        const BufRes res =
            make_buf(ok ? x + ((int64_t)p.n * C + ch) * HW + (int64_t)hh * W : x, ok ? row_bytes : 0u);
#pragma unroll
        for (int part = 0; part < L::kXI; ++part) {
          // the last copy ends at the row end (it may overlap the previous one)
          const int po = 64 * part < L::kXD - 64 ? 64 * part : L::kXD - 64;
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              res, (__attribute__((address_space(3))) void*)(dstb + pr * L::kXSD + po), 4,
              (uint32_t)(p.w0 - kWgPad + (po + lane) * L::kPerD) * (uint32_t)E, 0, 0, 0);
        }
      }
    }
    // y and branch-gradient rows in the swizzled chunk layout; channels
    // >= C read past the end of the resource (zero)
    const BufRes yres = make_buf(y + (int64_t)p.n * CHW, plane_bytes);
    const BufRes gres = make_buf(gbase + (int64_t)p.n * 4 * CHW, plane_bytes);
    const uint32_t rowel = (uint32_t)(p.h * W);
    if (g.x4) {
      // 1 KB copies: lane l moves chunk l, i.e. row i0 + l / kYC, position l % kYC
      const int ri = lane / L::kYC, pos = lane % L::kYC;
      constexpr int NY = L::kYRows / L::kRPI, NG = 16 / L::kRPI;
#pragma unroll
      for (int j = 0; j < (NY + NG + NW - 1) / NW; ++j) {
        const int ii = wave + NW * j;
        if ((NY + NG) % NW != 0 && ii >= NY + NG) break;
        const bool isy = ii < NY;
        const int row = (isy ? ii : ii - NY) * L::kRPI + ri;  // y row i or g row c
        const int w = p.w0 + (pos ^ (row & 15)) * L::kPerC;
        const int ch = isy ? row : cb * 16 + row;
        const uint32_t off = w < W ? ((uint32_t)ch * (uint32_t)HW + rowel + (uint32_t)w) * E : kOob;
        const int ldsd = (isy ? L::kYOff : L::kGOff) + (ii - (isy ? 0 : NY)) * 256;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(isy ? yres : gres,
                                                 (__attribute__((address_space(3))) void*)(dstb + ldsd),
                                                 16, off, 0, 0, 0);
      }
    } else if (g.dma) {
      // dword copies: lane l moves dword l of a 64-dword piece of one row
      constexpr int PPR = L::kYD / 64 > 0 ? L::kYD / 64 : 1;  // pieces per row
      constexpr int NY = L::kYRows * PPR, NG = 16 * PPR;
#pragma unroll
      for (int j = 0; j < (NY + NG + NW - 1) / NW; ++j) {
        const int ii = wave + NW * j;
        if ((NY + NG) % NW != 0 && ii >= NY + NG) break;
        const bool isy = ii < NY;
        const int k2 = isy ? ii : ii - NY;
        const int row = k2 / PPR, piece = k2 - row * PPR;
        const int dw = 64 * piece + lane;  // dword within the row
        const int kc = ((dw >> 2) ^ (row & 15)), wi = dw & 3;
        const int w = p.w0 + kc * L::kPerC + wi * L::kPerD;
        const int ch = isy ? row : cb * 16 + row;
        const uint32_t off = w < W ? ((uint32_t)ch * (uint32_t)HW + rowel + (uint32_t)w) * E : kOob;
        const int ldsd = (isy ? L::kYOff : L::kGOff) + row * L::kYD + 64 * piece;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(isy ? yres : gres,
                                                 (__attribute__((address_space(3))) void*)(dstb + ldsd),
                                                 4, off, 0, 0, 0);
      }
    }
    if (!g.dma) {
      // element-wise copy through registers (2-byte types with odd W)
      T* __restrict__ dst = reinterpret_cast<T*>(dstb);
      constexpr int PX = L::kXRows * kWgLW, PY = L::kYRows * kWgTW, PG = 16 * kWgTW;
      const BufRes xres = make_buf(x + (int64_t)p.n * CHW, plane_bytes);
      for (int idx = tid; idx < PX + PY + PG; idx += NT) {
        uint32_t off = kOob;
        int li;
        BufRes res;
        if (idx < PX) {
          const int pr = idx / kWgLW, j = idx - pr * kWgLW;
          const int rr = pr >> 4, c = pr & 15;
          const int ch = cb * 16 + c, hh = p.h + (rr - r) * d, gw = p.w0 - kWgPad + j;
          if (ch < C && (unsigned)hh < (unsigned)H && (unsigned)gw < (unsigned)W)
            off = (uint32_t)(((int64_t)ch * H + hh) * W + gw) * E;
          li = pr * L::kXSD * L::kPerD + j;
          res = xres;
        } else {
          const bool isy = idx < PX + PY;
          const int k2 = idx - PX - (isy ? 0 : PY);
          const int row = k2 / kWgTW, j = k2 - row * kWgTW, gw = p.w0 + j;
          const int ch = isy ? row : cb * 16 + row;
          if (ch < C && gw < W) off = ((uint32_t)ch * (uint32_t)HW + rowel + (uint32_t)gw) * E;
          const int kc = (j / L::kPerC) ^ (row & 15), wi = j % L::kPerC;
          li = ((isy ? L::kYOff : L::kGOff) + row * L::kYD) * L::kPerD + kc * L::kPerC + wi;
          res = isy ? yres : gres;
        }
        dst[li] = from_f<T>(buf_load1<T>(res, off));
      }
    }
  };

  f32x4 acc[TPH][MB];
#pragma unroll
  for (int tt = 0; tt < TPH; ++tt)
#pragma unroll
    for (int ib = 0; ib < MB; ++ib) acc[tt][ib] = f32x4{0.f, 0.f, 0.f, 0.f};
  float bacc[TPH];
#pragma unroll
  for (int tt = 0; tt < TPH; ++tt) bacc[tt] = 0.f;

  WgPos nxt;
  nxt.n = row_beg / H;
  nxt.h = row_beg - nxt.n * H;
  nxt.w0 = 0;
  nxt.cbk = 0;
  if (steps > 0) {
    stage(nxt, 0);
    nxt.advance(g);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  const int wl = 32 * sg + 8 * quad;  // this lane's first token within the step
  for (int s = 0; s < steps; ++s) {
    const int buf = s & 1;
    if (s + 1 < steps) {
      stage(nxt, buf ^ 1);
      nxt.advance(g);
    }
    const uint32_t* __restrict__ bb = wsm + buf * L::kBuf;
    // this lane's 8 tokens wl .. wl+7 sit in chunk(s) wl / kPerC (+1 for fp32)
    const int k0 = wl / L::kPerC;
    const int p0 = 4 * (k0 ^ col16), p1 = 4 * ((k0 + 1) ^ col16);
    V bfr[MB][M::P];
#pragma unroll
    for (int ib = 0; ib < MB; ++ib) {
      float yv[8];
      lds_chunks8<T>(bb + L::kYOff + (ib * 16 + col16) * L::kYD, p0, p1, yv);
      M::pack(yv, bfr[ib]);
    }
    float gv[8];
    lds_chunks8<T>(bb + L::kGOff + col16 * L::kYD, p0, p1, gv);
#pragma unroll
    for (int tt = 0; tt < TPH; ++tt) {
      const int t = th * TPH + tt;  // wave-uniform
      if (KK % NH != 0 && t >= KK) break;
      const int ki = t / KS, kj = t - ki * KS;
      const uint32_t* __restrict__ xr = bb + (ki * 16 + col16) * L::kXSD;
      const int xo = kWgPad + wl + (kj - r) * d;
      float dk[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) dk[e] = gv[e] * lds_elem<T>(xr, xo + e);
#pragma unroll
      for (int e = 0; e < 8; ++e) bacc[tt] += quant<T>(dk[e]);
      V afr[M::P];
      M::pack(dk, afr);
#pragma unroll
      for (int ib = 0; ib < MB; ++ib) acc[tt][ib] = M::mac(afr, bfr[ib], acc[tt][ib]);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }

  // ---- deterministic reduction over the segments (fixed order) through LDS
  constexpr int NO = MB * 16;
  constexpr int RS = NO + 1;
  float* __restrict__ red = reinterpret_cast<float*>(wsm);  // [KK][16 c][RS]
  float* __restrict__ rb = red + KK * 16 * RS;              // [KK][segs*4][16]
#pragma unroll
  for (int tt = 0; tt < TPH; ++tt) {
    const int t = th * TPH + tt;
    if (t < KK) rb[(t * kWgSegs * 4 + sg * 4 + quad) * 16 + col16] = bacc[tt];
  }
  for (int w = 0; w < kWgSegs; ++w) {
    if (sg == w) {
#pragma unroll
      for (int tt = 0; tt < TPH; ++tt) {
        const int t = th * TPH + tt;
        if (t >= KK) break;
#pragma unroll
        for (int ib = 0; ib < MB; ++ib)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float* dst = red + (t * 16 + 4 * quad + e) * RS + ib * 16 + col16;
            *dst = (w == 0 ? 0.f : *dst) + acc[tt][ib][e];
          }
      }
    }
    __syncthreads();
  }
  for (int idx = tid; idx < KK * 16 * NO; idx += NT) {
    const int t = idx / (16 * NO);
    const int rem2 = idx - t * 16 * NO;
    const int c = rem2 / NO, i = rem2 - c * NO;
    const int ch = cb * 16 + c;
    if (ch >= C || i >= C) continue;
    const float v = red[(t * 16 + c) * RS + i];
    if (g.direct)
      dw_out[((int64_t)(b * C + ch) * KK + t) * C + i] = from_f<T>(v);
    else
      pw[(((int64_t)split * 3 * KK + b * KK + t) * C + ch) * C + i] = v;
  }
  for (int idx = tid; idx < KK * 16; idx += NT) {
    const int t = idx >> 4, c = idx & 15;
    const int ch = cb * 16 + c;
    if (ch >= C) continue;
    float v = 0.f;
    for (int j = 0; j < kWgSegs * 4; ++j) v += rb[(t * kWgSegs * 4 + j) * 16 + c];
    if (g.direct)
      db_out[(int64_t)(b * C + ch) * KK + t] = from_f<T>(v);
    else
      pb[((int64_t)split * 3 * KK + b * KK + t) * C + ch] = v;
  }
}

// Fixed-order sum of the split partials, written in Conv2d parameter layout.
template <typename T>
__global__ __launch_bounds__(256) void gen_bwd_w_reduce_kernel(const float* __restrict__ pw,
                                                                 const float* __restrict__ pb,
                                                                 T* __restrict__ dw_out,
                                                                 T* __restrict__ db_out, int C,
                                                                 int KK, int splits) {
  const int64_t per = (int64_t)3 * KK * C * C;
  const int64_t perb = (int64_t)3 * KK * C;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx < per) {
    float v = 0.f;
    for (int s = 0; s < splits; ++s) v += pw[s * per + idx];
    // idx = (bt*C + c)*C + i  ->  row o = (b*C + c)*KK + t
    const int64_t i = idx % C;
    const int64_t c = (idx / C) % C;
    const int64_t bt = idx / ((int64_t)C * C);
    const int64_t b = bt / KK, t = bt % KK;
    dw_out[((b * C + c) * KK + t) * C + i] = from_f<T>(v);
  } else if (idx < per + perb) {
    const int64_t j = idx - per;
    float v = 0.f;
    for (int s = 0; s < splits; ++s) v += pb[s * perb + j];
    const int64_t c = j % C, bt = j / C;
    const int64_t b = bt / KK, t = bt % KK;
    db_out[(b * C + c) * KK + t] = from_f<T>(v);
  }
}

namespace {

template <typename F>
int wg_with_type(int dt, F&& f) {
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
int wg_with_mb(int mb, F&& f) {
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

// Splits: about kWgTokensPerSplit tokens each, at most 16 and at most one per
// image row; one split means grad_weight / grad_bias are written directly.
void wgrad_geom(WGradGeom& g, int64_t n, int64_t c, int64_t h, int64_t w, int d0, int d1, int d2) {
  g.N = (int)n;
  g.C = (int)c;
  g.H = (int)h;
  g.W = (int)w;
  g.d0 = d0;
  g.d1 = d1;
  g.d2 = d2;
  g.cblocks = (int)((c + 15) / 16);
  g.col_blocks = (int)((w + kWgTW - 1) / kWgTW);
  g.rows = (int)(n * h);
  const int64_t tokens = n * h * w;
  int64_t splits = (tokens + kWgTokensPerSplit - 1) / kWgTokensPerSplit;
  if (splits > kWgMaxSplits) splits = kWgMaxSplits;
  if (splits > g.rows) splits = g.rows;
  if (splits < 1) splits = 1;
  g.rows_per_split = (int)((g.rows + splits - 1) / splits);
  g.splits = (int)((g.rows + g.rows_per_split - 1) / g.rows_per_split);
  g.direct = g.splits == 1;
  g.dma = 0;
  g.x4 = 0;
}

}  // namespace
}  // namespace ddpm

using namespace ddpm;

extern "C" int64_t ddpm_gen_bwd_w_workspace_bytes(int64_t n, int64_t c, int64_t h, int64_t w,
                                                  int kernel_size) {
  if (n <= 0 || c <= 0 || h <= 0 || w <= 0 || kernel_size < 1) return 0;
  if (n * h > 0x7fffffffLL) return 0;
  WGradGeom g;
  wgrad_geom(g, n, c, h, w, 1, 1, 1);
  if (g.direct) return 0;
  const int64_t kk = (int64_t)kernel_size * kernel_size;
  return (int64_t)g.splits * 3 * kk * c * (c + 1) * (int64_t)sizeof(float);
}

extern "C" int ddpm_gen_bwd_w(const void* x, const void* y, const void* grad_out,
                              void* grad_weight, void* grad_bias, void* workspace,
                              int64_t workspace_bytes, int64_t n, int64_t c, int64_t h, int64_t w,
                              int kernel_size, int d0, int d1, int d2, int dtype,
                              hipStream_t stream) {
  if (dtype < kF32 || dtype > kF16) return kBadArgument;
  GenGeom gg;
  int st = gen_make_geom(gg, n, c, h, w, kernel_size, d0, d1, d2);
  if (st != kOk) return st;
  if (n == 0 || c == 0 || h == 0 || w == 0) return kOk;
  if (!x || !y || !grad_out || !grad_weight || !grad_bias) return kBadArgument;
  if (gg.d0 > kWgMaxDil || gg.d1 > kWgMaxDil || gg.d2 > kWgMaxDil) return kUnsupported;
  if (n * h > 0x7fffffffLL / 4) return kUnsupported;
  // 32-bit buffer offsets inside one image's [C][H][W] planes
  if (((c + 15) / 16) * 16 * h * w * (dtype == kF32 ? 4 : 2) > 0x7fffffffLL) return kUnsupported;
  WGradGeom g;
  wgrad_geom(g, n, c, h, w, gg.d0, gg.d1, gg.d2);
  const int64_t need = ddpm_gen_bwd_w_workspace_bytes(n, c, h, w, kernel_size);
  if (need > 0 && (!workspace || workspace_bytes < need)) return kWorkspaceTooSmall;
  const size_t esz = dtype == kF32 ? 4 : 2;
  // LDS-direct dword copies need every row to start on a dword boundary
  g.dma = (esz == 4) || ((w % 2 == 0) && ((uintptr_t)x % 4 == 0) && ((uintptr_t)y % 4 == 0) &&
                         ((uintptr_t)grad_out % 4 == 0));
  g.x4 = (w % 8 == 0) && ((uintptr_t)y % 16 == 0) && ((uintptr_t)grad_out % 16 == 0);
  const int mb = (int)((c + 15) / 16);
  const int kk = kernel_size * kernel_size;
  float* pw = (float*)workspace;
  float* pb = pw ? pw + (int64_t)g.splits * 3 * kk * c * c : nullptr;
  if (g.direct) pw = pb = nullptr;
  return wg_with_type(dtype, [&](auto tag) {
    using T = decltype(tag);
    auto launch = [&](auto ks, auto mbc) {
      constexpr int KS = decltype(ks)::value;
      constexpr int MB = decltype(mbc)::value;
      constexpr int KKc = KS * KS;
      typedef WgLds<T, KS, MB> L;
      const size_t stage = (size_t)2 * L::kBuf * 4;
      const size_t red = (size_t)(KKc * 16 * (MB * 16 + 1) + KKc * kWgSegs * 4 * 16) * sizeof(float);
      const size_t lds = stage > red ? stage : red;
      const dim3 grid((unsigned)(g.splits * 3 * g.cblocks));
      if (lds > 64 * 1024) {
        // up to 160 KB of LDS per workgroup on gfx950
        const hipError_t ae = hipFuncSetAttribute(
            reinterpret_cast<const void*>(&gen_bwd_w_partial_kernel<T, KS, MB>),
            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (ae != hipSuccess) return (int)ae;
      }
      hipLaunchKernelGGL((gen_bwd_w_partial_kernel<T, KS, MB>), grid,
                         dim3(64 * kWgSegs * WgTaps<KS>::kHalves), lds, stream, (const T*)x,
                         (const T*)y, (const T*)grad_out, pw, pb, (T*)grad_weight, (T*)grad_bias, g);
      int e = (int)hipGetLastError();
      if (e != 0 || g.direct) return e;
      const int64_t total = (int64_t)3 * KKc * c * c + (int64_t)3 * KKc * c;
      hipLaunchKernelGGL((gen_bwd_w_reduce_kernel<T>), dim3((unsigned)((total + 255) / 256)),
                         dim3(256), 0, stream, pw, pb, (T*)grad_weight, (T*)grad_bias, (int)c, KKc,
                         g.splits);
      return (int)hipGetLastError();
    };
    return wg_with_mb(mb, [&](auto mbc) {
      if (kernel_size == 1) return launch(std::integral_constant<int, 1>(), mbc);
      if (kernel_size == 3) return launch(std::integral_constant<int, 3>(), mbc);
      return (int)kUnsupported;
    });
  });
}
