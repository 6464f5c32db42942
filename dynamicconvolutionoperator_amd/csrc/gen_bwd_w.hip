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
// 16-channel block of c, and above 64 channels half of the input channels i).  Splits are equal ranges of steps -- one step is
// one row segment of 128 columns -- at most 16 of them (the reference's
// bound, :1001-1005) and at least 4 steps each (16 splits x 3 branches x 4
// channel blocks = 192 workgroups at C = 64, 256x256); they write fp32
// partials that a second kernel sums in a fixed order (deterministic, no
// atomics), and a single split writes grad_weight / grad_bias directly.  Everything a step reads -- the K rows
// {h-d, h, h+d} of x (128 + 16 columns, 16 channels), the y rows (all C
// channels) and the branch-gradient rows (16 channels) -- is copied
// global -> LDS by buffer loads that write LDS directly (no registers; reads
// outside the image return zero; 16-byte lanes where the rows allow), one
// step ahead into a second buffer.
// Wave (segment sg, tap group th) owns 32 tokens of the step and a third of
// the K*K taps.  It forms dK for its taps on the fly -- one multiply per element,
// plus the bf16 hi/lo split for fp32, is all its VALU work -- and
// accumulates taps x 16 c x C i with v_mfma_f32_16x16x32_{bf16,f16} (M = c,
// N = i, K = tokens; fp32 operands run as three bf16 products).  db is one
// more MFMA per tap and part against a column of ones.  For fp32, y is split
// into bf16 hi / lo rows while it is staged: each thread loads its 4-column
// pieces of the next step's y rows into registers at the start of a step and
// writes their split to LDS after the step's MFMAs (no pre-pass over y, no
// workspace planes), so every B fragment is a plain 16-byte LDS read.

#include "gen_bwd.h"
#include <type_traits>

namespace ddpm {

constexpr int kWgSegs = 4;                   // 32-token segments per step
constexpr int kWgTW = 32 * kWgSegs;          // columns per step
constexpr int kWgPad = 8;                    // staged column halo (>= dilation), even
constexpr int kWgMaxDil = kWgPad;
constexpr int kWgMinSteps = 4;               // steps per split at least

struct WGradGeom {
  int N, C, H, W;
  int d0, d1, d2;
  int cblocks;         // ceil(C / 16)
  int ihalves;         // 1, or 2 when C > 64: a workgroup covers 16*MB input channels i
  int tw;              // columns per step: kWgTW, or 2 * kWgTW (wg_step_cols)
  int col_blocks;      // ceil(W / tw)
  int splits;
  int steps;           // N * H * col_blocks
  int steps_per_split;
  int direct;          // one split: write grad_weight / grad_bias directly
  int xdma;            // x rows start on dword boundaries: LDS-direct dword copies
  int x16;             // x rows hold whole 16-byte chunks (W % (16/E) == 0, aligned): 16-byte copies
  int x4;              // y and gradient rows 16-byte aligned (W % 8 == 0): 16-byte copies
  int y4;              // fp32 y rows 16-byte aligned (W % 4 == 0): 16-byte register loads
  int dw_blocks;       // weight-gradient workgroups; any further ones are helpers (see below)
};

// Tap groups per kernel size: the K = 3 taps are split over three waves of 3
// (12 waves, three per SIMD: measured 4-11% faster than two groups of 5 and 4).
template <int KS>
struct WgTaps {
  static constexpr int kGroups = KS == 1 ? 1 : 3;
  static constexpr int kPer = (KS * KS + kGroups - 1) / kGroups;
};

// One LDS staging buffer (dwords):
//   x rows [KS*16][kXSD]      T elements; odd pitch, so the 64 lanes' reads of
//                             one element fall at most two to a bank
//   y rows [P][MB*16][kYD]    2-byte elements (the bf16 hi / lo planes of an
//                             fp32 y, or y itself): 16 chunks of 16 bytes,
//                             chunk k of row i stored at position k ^ (i & 15)
//   g rows [16][kGD]          T elements, chunks swizzled the same way
// The 16-byte fragment reads of 16 rows at one chunk index hit 16 distinct
// bank groups.
template <typename T, int KS, int MB, int SJ>
struct WgLds {
  static constexpr int P = Mma<T>::P;
  static constexpr int TW = kWgTW * SJ;                             // columns per step
  static constexpr int LW = TW + 2 * kWgPad;                        // staged x columns
  static constexpr int kPerD = 4 / (int)sizeof(T);                  // elements per dword
  static constexpr int kXD = LW / kPerD;                            // dwords per staged x row
  static constexpr int kXI = (kXD + 63) / 64;                       // 64-dword copies per x row
  static constexpr int kXSD = kXD + (sizeof(T) == 4 ? 1 : 3);
  static_assert(kXSD % 2 == 1, "odd x-row pitch");
  static_assert(kXD % 4 == 0, "16-byte x copies move whole rows");
  static constexpr int kYC = TW / 8;                                // chunks per y row (16 or 32)
  static constexpr int kYD = 4 * kYC;
  static constexpr int kGC = TW * (int)sizeof(T) / 16;              // chunks per g row
  static constexpr int kGD = 4 * kGC;
  static constexpr int kXRows = KS * 16;
  static constexpr int kYRows = P * MB * 16;
  static constexpr int kYOff = kXRows * kXSD;
  static constexpr int kGOff = kYOff + kYRows * kYD;
  static constexpr int kBuf = kGOff + 16 * kGD;
  static_assert(kYC >= 16 && kYC % 16 == 0 && kGC >= 16, "the chunk swizzle needs 16 chunks per row");
  static_assert(kXD / 4 <= 64, "one 16-byte x copy per lane and row");
};

template <typename T>
__device__ __forceinline__ float lds_elem(const uint32_t* __restrict__ base, int idx) {
  if constexpr (sizeof(T) == 4) {
    return __uint_as_float(base[idx]);
  } else {
    return to_f(reinterpret_cast<const T*>(base)[idx]);
  }
}

// Position of a step: image n, row h, first column w0 (column block cbk).
struct WgPos {
  int n, h, w0, cbk;
  __device__ __forceinline__ void advance(const WGradGeom& g) {
    w0 += g.tw;
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

// fp32 y -> bf16 hi / lo planes ys[n][part][c][hw] (hi = top 16 bits of the
// fp32 pattern, lo = the remainder rounded to nearest even).  Grid: x over
// one image's C*H*W elements, 8 per thread; y over images.  Each thread
// splits 8 consecutive elements: two 16-byte loads, two 16-byte stores when
// one image's planes hold a multiple of 8 elements, element-wise otherwise.
__global__ __launch_bounds__(256) void gen_ysplit_kernel(const float* __restrict__ y,
                                                         uint16_t* __restrict__ ys, uint32_t chw,
                                                         uint32_t nimg) {
  const uint32_t i0 = (blockIdx.x * 256u + threadIdx.x) * 8u;
  if (i0 >= chw) return;
  for (uint32_t n = blockIdx.y; n < nimg; n += gridDim.y) {
    const float* __restrict__ src = y + (int64_t)n * chw;
    uint16_t* __restrict__ h = ys + (int64_t)n * 2 * chw;
    if (chw % 8 == 0) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(src + i0);
      const f32x4 c = *reinterpret_cast<const f32x4*>(src + i0 + 4);
      uint32_t hi[4], lo[4];
      split_bf16x2(a[0], a[1], hi[0], lo[0]);
      split_bf16x2(a[2], a[3], hi[1], lo[1]);
      split_bf16x2(c[0], c[1], hi[2], lo[2]);
      split_bf16x2(c[2], c[3], hi[3], lo[3]);
      *reinterpret_cast<u32x4*>(h + i0) = (u32x4){hi[0], hi[1], hi[2], hi[3]};
      *reinterpret_cast<u32x4*>(h + chw + i0) = (u32x4){lo[0], lo[1], lo[2], lo[3]};
    } else {
      for (uint32_t i = i0; i < chw && i < i0 + 8; ++i) {
        uint32_t h2, l2;
        split_bf16x2(src[i], 0.f, h2, l2);
        h[i] = (uint16_t)h2;
        h[chw + i] = (uint16_t)l2;
      }
    }
  }
}

// Workgroups past g.dw_blocks (ddpm_gen_bwd_xw, ddpm_gen_bwd) are helpers:
// with at most 16 splits x 3 branches x the channel blocks, the weight
// gradient leaves CUs free (64 of 256 at C = 64), and the helpers run the dY
// kernel's weight packing (`yp`, none when yp.total is 0) and the input
// gradient's halo reduction (`fin`) there, alongside, instead of as kernels of
// their own.
// SJ: 128-column subsegments per step (2 for 2-byte types on wide images:
// twice the work per step and per barrier; each wave takes its 32-token
// segment in both).
template <typename T, int KS, int MB, int SJ, bool AL>
__global__ __launch_bounds__(64 * kWgSegs * WgTaps<KS>::kGroups) void gen_bwd_w_partial_kernel(
    const T* __restrict__ x, const T* __restrict__ y, const T* __restrict__ gout,
    float* __restrict__ pw, float* __restrict__ pb, T* __restrict__ dw_out, T* __restrict__ db_out,
    WGradGeom g, BxFinish fin, YPack yp) {
  typedef Mma<T> M;
  typedef typename M::V V;
  typedef typename M::E ME;
  typedef WgLds<T, KS, MB, SJ> L;
  constexpr int TW = L::TW, LW = L::LW;
  constexpr int KK = KS * KS;
  constexpr int r = KS / 2;
  constexpr int P = M::P;
  constexpr int NH = WgTaps<KS>::kGroups;
  constexpr int TPH = WgTaps<KS>::kPer;
  constexpr int NW = kWgSegs * NH;
  constexpr int NT = 64 * NW;
  constexpr int E = (int)sizeof(T);
  constexpr int PC = 16 / E;  // T elements per 16-byte chunk
  // fp32: y goes through registers and is split into its bf16 hi / lo rows on
  // the way to LDS; 2-byte types copy y global -> LDS directly
  constexpr bool kYReg = E == 4;
  // fp32: db sums the fp32 products on the VALU (frees the registers of the
  // bias MFMA's accumulators and column of ones); 2-byte types add the
  // bf16-rounded products with one more MFMA per tap against a column of ones
  constexpr bool kVBias = E == 4;
  extern __shared__ __attribute__((aligned(16))) uint32_t wsm[];

  if ((int)blockIdx.x >= g.dw_blocks) {
    // helper workgroup (uniform branch, before any barrier): items of the
    // halo reduction, grid-strided over the helpers
    const int64_t stride = (int64_t)(gridDim.x - g.dw_blocks) * NT;
    const int64_t first = (int64_t)(blockIdx.x - g.dw_blocks) * NT + threadIdx.x;
    const T* __restrict__ ywt = static_cast<const T*>(yp.wt);
    for (int64_t it = first; it < yp.total; it += stride)
      yt_pack_item<T, KS, MB>(ywt, yp.pk, yp.C, yp.nc32, (int)it);
    const T* __restrict__ fgo = static_cast<const T*>(fin.gout);
    T* __restrict__ fgx = static_cast<T*>(fin.gx);
    if (fin.vec == 4) {
      for (int64_t it = first; it < fin.items; it += stride) bx_reduce_item<T, 4>(fin.part, fgo, fgx, fin.g, it);
    } else {
      for (int64_t it = first; it < fin.items; it += stride) bx_reduce_item<T, 1>(fin.part, fgo, fgx, fin.g, it);
    }
    return;
  }
  const int logical = xcd_remap(blockIdx.x, g.dw_blocks);
  const int ih = logical % g.ihalves;
  const int lg = logical / g.ihalves;
  const int per_split = 3 * g.cblocks;
  const int split = lg / per_split;
  const int rem = lg - split * per_split;
  const int b = rem / g.cblocks;
  const int cb = rem - b * g.cblocks;
  const int i0 = ih * MB * 16;  // first input channel of this workgroup
  const int d = dil_of(b, g.d0, g.d1, g.d2);
  const int C = g.C, H = g.H, W = g.W;
  const int64_t HW = (int64_t)H * W;
  const int64_t CHW = (int64_t)C * HW;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int col16 = lane & 15, quad = lane >> 4;
  const int sg = wave % kWgSegs, th = wave / kWgSegs;

  const int step_beg = split * g.steps_per_split;
  int step_end = step_beg + g.steps_per_split;
  if (step_end > g.steps) step_end = g.steps;
  const int steps = step_end > step_beg ? step_end - step_beg : 0;
  const T* __restrict__ gbase = gout + (int64_t)(b + 1) * C * HW;

  // Step-invariant parts of this wave's copies, computed once:
  //   x rows: the lane's byte offset at column 0 of the staged row (may be
  //     negative: columns left of the image read zero);
  //   y / gradient rows (16-byte copies): the lane's byte offset within one
  //     image's planes at row 0, column 0 (kOob for channels >= C) and the
  //     column of its chunk.
  constexpr int YRPC = 64 / L::kYC;  // y rows per 1 KB copy
  constexpr int GRPC = 64 / L::kGC;  // gradient rows per 1 KB copy
  constexpr int NY = kYReg ? 0 : L::kYRows / YRPC, NG = 16 / GRPC;
  constexpr int NJ = (NY + NG + NW - 1) / NW;
  int xlo[L::kXI];
#pragma unroll
  for (int part = 0; part < L::kXI; ++part) {
    const int po = 64 * part < L::kXD - 64 ? 64 * part : L::kXD - 64;
    xlo[part] = (po + lane) * L::kPerD - kWgPad;  // column of the lane's dword relative to w0
  }
  uint32_t cpo[NJ];
  int cpc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int ii = wave + NW * j;
    cpo[j] = kOob;
    cpc[j] = 0;
    if (ii < NY) {
      const int row = ii * YRPC + lane / L::kYC, pos = lane % L::kYC;
      const int part = row / (MB * 16), i = row - part * (MB * 16);
      cpc[j] = (pos ^ (i & 15)) * 8;
      if (i0 + i < C)
        cpo[j] = ((uint32_t)(part * C + i0 + i) * (uint32_t)HW + (uint32_t)cpc[j]) * 2u;
    } else if (ii < NY + NG) {
      const int row = (ii - NY) * GRPC + lane / L::kGC, pos = lane % L::kGC;
      cpc[j] = (pos ^ (row & 15)) * PC;
      const int ch = cb * 16 + row;
      if (ch < C) cpo[j] = ((uint32_t)ch * (uint32_t)HW + (uint32_t)cpc[j]) * (uint32_t)E;
    }
  }

  // Buffer resources of one image's x, y and gradient planes, formed again
  // only when a step enters another image
  BufRes rx = make_buf(x, 0u), ry = make_buf(y, 0u), rg = make_buf(gbase, 0u);
  int rn = -1;
  auto image = [&](int n) {
    if (n != rn) {
      rn = n;
      rx = make_buf(x + (int64_t)n * CHW, (uint32_t)(CHW * E));
      ry = make_buf(y + (int64_t)n * CHW, (uint32_t)(CHW * E));
      rg = make_buf(gbase + (int64_t)n * 4 * CHW, (uint32_t)(CHW * E));
    }
  };

  // ---- operands of step `p` -> LDS buffer `buf`
  auto stage = [&](const WgPos& p, int buf) {
    uint32_t* __restrict__ dstb = wsm + buf * L::kBuf;
    const uint32_t rowel = (uint32_t)(p.h * W);
    if constexpr (AL) {
      // x rows, aligned layout: the offsets and resources of the step's KS
      // kernel rows are formed once (a row outside the image copies through
      // a resource with no records), each wave copies channel rows c = wave,
      // wave + NW, .. for every kernel row, under one lane mask
      const BufRes xnul = make_buf(x, 0u);
      uint32_t roff[KS];
      BufRes rres[KS];
#pragma unroll
      for (int rr = 0; rr < KS; ++rr) {
        const int hh = p.h + (rr - r) * d;
        const bool ok = (unsigned)hh < (unsigned)H;
        roff[rr] = ok ? (uint32_t)(hh * W) * E : 0u;
        rres[rr] = ok ? rx : xnul;
      }
      const uint32_t colb = (uint32_t)(p.w0 - kWgPad + 4 * L::kPerD * lane) * E;
      const bool left = p.w0 == 0 && lane < kWgPad / (4 * L::kPerD);  // the halo left of column 0
      const bool right = p.w0 + TW == W && 4 * L::kPerD * lane >= TW + kWgPad;
      const uint32_t colv = left || right ? kOob : colb;
      if (lane < L::kXD / 4) {
#pragma unroll
        for (int jc = 0; jc < (16 + NW - 1) / NW; ++jc) {
          const int c = wave + NW * jc;
          if (16 % NW != 0 && c >= 16) break;
          const int ch = cb * 16 + c;  // < C: the aligned layout has whole channel blocks
          const uint32_t cho = (uint32_t)ch * (uint32_t)HW * E;
#pragma unroll
          for (int rr = 0; rr < KS; ++rr) {
            const BufRes rs = rres[rr];
            // (the scalar offset goes through a named variable: written as an
            // expression in the call, the host pass drops the kernel's stub)
            const uint32_t so = cho + roff[rr];
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rs, (__attribute__((address_space(3))) void*)(dstb + (rr * 16 + c) * L::kXSD), 16,
                colv, so, 0, 0);
          }
        }
      }
    } else if (g.x16) {
      // x rows: one copy per row, lane l < kXD/4 moving the row's 16-byte
      // chunk l (three times fewer copy instructions, and their scalar set-up,
      // than dword copies: fp32 85.6 -> 82.1 us at 256x256); a row outside the
      // image or a channel >= C copies through a resource with no records
      const BufRes xres = make_buf(x + (int64_t)p.n * CHW, (uint32_t)(CHW * E));
      const BufRes xnul = make_buf(x, 0u);
      const int gw = p.w0 - kWgPad + 4 * L::kPerD * lane;
      const uint32_t colb =
          (lane < L::kXD / 4 && (unsigned)gw < (unsigned)W) ? (uint32_t)gw * E : kOob;
#pragma unroll
      for (int j = 0; j < (L::kXRows + NW - 1) / NW; ++j) {
        const int pr = wave + NW * j;
        if (L::kXRows % NW != 0 && pr >= L::kXRows) break;
        const int rr = pr >> 4, c = pr & 15;
        const int ch = cb * 16 + c, hh = p.h + (rr - r) * d;
        const bool ok = ch < C && (unsigned)hh < (unsigned)H;
        const uint32_t soff = ok ? ((uint32_t)ch * (uint32_t)HW + (uint32_t)(hh * W)) * E : 0u;
        const BufRes rs = ok ? xres : xnul;
        if (lane < L::kXD / 4)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              rs, (__attribute__((address_space(3))) void*)(dstb + pr * L::kXSD), 16, colb, soff,
              0, 0);
      }
    } else     if (g.xdma) {
      // x rows: copies of 64 dwords (lane l moves dword l) from one resource
      // per image.  The row's byte offset is the scalar offset of the copy
      // and the lane's column byte offset (kOob outside the image) is formed
      // once per step, so a copy costs no vector instructions; a row outside
      // the image (or a channel >= C) copies through a resource with no
      // records and reads zero.  (Per-lane offsets formed per copy cost ~4
      // vector instructions each: measured 2-5% slower.)
      const BufRes xres = make_buf(x + (int64_t)p.n * CHW, (uint32_t)(CHW * E));
      const BufRes xnul = make_buf(x, 0u);
      uint32_t colb[L::kXI];
#pragma unroll
      for (int part = 0; part < L::kXI; ++part) {
        const int gw = p.w0 + xlo[part];
        colb[part] = (unsigned)gw < (unsigned)W ? (uint32_t)gw * E : kOob;
      }
#pragma unroll
      for (int j = 0; j < (L::kXRows + NW - 1) / NW; ++j) {
        const int pr = wave + NW * j;
        if (L::kXRows % NW != 0 && pr >= L::kXRows) break;
        const int rr = pr >> 4, c = pr & 15;
        const int ch = cb * 16 + c, hh = p.h + (rr - r) * d;
        const bool ok = ch < C && (unsigned)hh < (unsigned)H;
        const uint32_t soff = ok ? ((uint32_t)ch * (uint32_t)HW + (uint32_t)(hh * W)) * E : 0u;
        const BufRes rs = ok ? xres : xnul;
#pragma unroll
        for (int part = 0; part < L::kXI; ++part) {
          // the last copy ends at the row end (it may overlap the previous one)
          const int po = 64 * part < L::kXD - 64 ? 64 * part : L::kXD - 64;
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              rs, (__attribute__((address_space(3))) void*)(dstb + pr * L::kXSD + po), 4, colb[part],
              soff, 0, 0);
        }
      }
    } else {
      // element-wise through registers (2-byte x with odd W or unaligned x)
      T* __restrict__ dst = reinterpret_cast<T*>(dstb);
      const BufRes xres = make_buf(x + (int64_t)p.n * CHW, (uint32_t)(CHW * E));
      for (int idx = tid; idx < L::kXRows * LW; idx += NT) {
        const int pr = idx / LW, j = idx - pr * LW;
        const int rr = pr >> 4, c = pr & 15;
        const int ch = cb * 16 + c, hh = p.h + (rr - r) * d, gw = p.w0 - kWgPad + j;
        const bool ok = ch < C && (unsigned)hh < (unsigned)H && (unsigned)gw < (unsigned)W;
        const uint32_t off = ok ? (uint32_t)(((int64_t)ch * H + hh) * W + gw) * E : kOob;
        dst[pr * L::kXSD * L::kPerD + j] = from_f<T>(buf_load1<T>(xres, off));
      }
    }
    // y rows (P parts x MB*16 channels) and branch-gradient rows (16
    // channels) in the swizzled chunk layout; channels >= C read zero
    const BufRes yres = AL ? ry : make_buf(y + (int64_t)p.n * CHW, (uint32_t)(CHW * E));
    const BufRes gres = AL ? rg : make_buf(gbase + (int64_t)p.n * 4 * CHW, (uint32_t)(CHW * E));
    if (AL || g.x4) {
      // 1 KB copies: lane l moves one 16-byte chunk; the step's byte offset
      // is the scalar offset, and lanes past the image's right edge are
      // masked only in a partial column block
      const uint32_t ystep = (rowel + (uint32_t)p.w0) * 2u, gstep = (rowel + (uint32_t)p.w0) * E;
      auto copies = [&](auto masked) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const int ii = wave + NW * j;
          if ((NY + NG) % NW != 0 && ii >= NY + NG) break;
          uint32_t vo = cpo[j];
          if constexpr (decltype(masked)::value) vo = p.w0 + cpc[j] < W ? vo : kOob;
          if (ii < NY) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                yres, (__attribute__((address_space(3))) void*)(dstb + L::kYOff + ii * 256), 16, vo,
                ystep, 0, 0);
          } else {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                gres, (__attribute__((address_space(3))) void*)(dstb + L::kGOff + (ii - NY) * 256), 16,
                vo, gstep, 0, 0);
          }
        }
      };
      if (AL || p.w0 + TW <= W)
        copies(std::false_type{});
      else
        copies(std::true_type{});
    } else {
      // element-wise through registers
      uint16_t* __restrict__ dy = reinterpret_cast<uint16_t*>(dstb + L::kYOff);
      T* __restrict__ dg = reinterpret_cast<T*>(dstb + L::kGOff);
      constexpr int PY = kYReg ? 0 : L::kYRows * TW, PG = 16 * TW;
      for (int idx = tid; idx < PY + PG; idx += NT) {
        if (idx < PY) {
          const int row = idx / TW, j = idx - row * TW;
          const int i = row;
          const int w = p.w0 + j;
          const uint32_t off =
              (i0 + i < C && w < W) ? ((uint32_t)(i0 + i) * (uint32_t)HW + rowel + (uint32_t)w) * 2u
                                    : kOob;
          const int kc = (j >> 3) ^ (i & 15);
          dy[row * L::kYD * 2 + kc * 8 + (j & 7)] =
              (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(yres, off, 0, 0);
        } else {
          const int k2 = idx - PY;
          const int row = k2 / TW, j = k2 - row * TW;
          const int ch = cb * 16 + row, w = p.w0 + j;
          const uint32_t off =
              (ch < C && w < W) ? ((uint32_t)ch * (uint32_t)HW + rowel + (uint32_t)w) * E : kOob;
          const int kc = (j / PC) ^ (row & 15);
          dg[row * L::kGD * L::kPerD + kc * PC + (j % PC)] = from_f<T>(buf_load1<T>(gres, off));
        }
      }
    }
  };

  // ---- fp32 y rows of step `p`: thread tid loads the 4-column pieces u = tid
  //      + NT*j (row u / 32, columns 4*(u % 32) .. +3) into registers
  //      (yload, issued before a step's MFMAs) and writes their bf16 hi / lo
  //      split to the y rows of LDS buffer `buf` (ystore, after them): the
  //      two 8-byte halves of the row's chunk (u % 32) / 2, swizzled as the
  //      LDS-direct copies place them.  Columns past the image and channels
  //      >= C read zero.
  constexpr int YU = kYReg ? MB * 16 * (TW / 4) : 1;  // 4-column pieces per step
  constexpr int YUT = (YU + NT - 1) / NT;
  f32x4 yreg[YUT];
  // aligned layout: the lane's byte offset of piece j within a step's rows
  uint32_t ylo[AL ? YUT : 1];
  if constexpr (AL && kYReg) {
#pragma unroll
    for (int j = 0; j < YUT; ++j) {
      const int u = tid + NT * j;
      ylo[j] = ((uint32_t)(i0 + (u >> 5)) * (uint32_t)HW + 4u * (uint32_t)(u & 31)) * 4u;
    }
  }
  auto yload = [&](const WgPos& p) {
    if constexpr (AL && kYReg) {
      const uint32_t ys = ((uint32_t)(p.h * W) + (uint32_t)p.w0) * 4u;
#pragma unroll
      for (int j = 0; j < YUT; ++j) {
        const int u = tid + NT * j;
        if (YU % NT != 0 && u >= YU) break;  // wave-uniform
        yreg[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(ry, ylo[j], ys, 0));
      }
    } else if constexpr (kYReg) {
      const BufRes yres = make_buf(y + (int64_t)p.n * CHW, (uint32_t)(CHW * E));
      const uint32_t rowel = (uint32_t)(p.h * W);
#pragma unroll
      for (int j = 0; j < YUT; ++j) {
        const int u = tid + NT * j;
        if (YU % NT != 0 && u >= YU) break;  // wave-uniform (NT and YU are multiples of 64)
        const int i = u >> 5, w = p.w0 + 4 * (u & 31);
        const bool okc = i0 + i < C;
        const uint32_t base = ((uint32_t)(i0 + i) * (uint32_t)HW + rowel + (uint32_t)w) * 4u;
        if (AL || g.y4) {
          yreg[j] = __builtin_bit_cast(
              f32x4,
              __builtin_amdgcn_raw_buffer_load_b128(yres, okc && (AL || w < W) ? base : kOob, 0, 0));
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            yreg[j][e] = buf_load1<float>(yres, okc && w + e < W ? base + 4u * e : kOob);
        }
      }
    }
  };
  auto ystore = [&](int buf) {
    if constexpr (kYReg) {
      uint32_t* __restrict__ yl = wsm + buf * L::kBuf + L::kYOff;
#pragma unroll
      for (int j = 0; j < YUT; ++j) {
        const int u = tid + NT * j;
        if (YU % NT != 0 && u >= YU) break;
        const int i = u >> 5, q = u & 31;
        const int dw = i * L::kYD + 4 * ((q >> 1) ^ (i & 15)) + 2 * (q & 1);
        uint32_t h0, l0, h1, l1;
        split_bf16x2(yreg[j][0], yreg[j][1], h0, l0);
        split_bf16x2(yreg[j][2], yreg[j][3], h1, l1);
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        *reinterpret_cast<u32x2*>(yl + dw) = (u32x2){h0, h1};
        *reinterpret_cast<u32x2*>(yl + MB * 16 * L::kYD + dw) = (u32x2){l0, l1};
      }
    }
  };

  // B fragment of the bias column: B[k][n] = (n == 0) for every k
  V ones;
  if constexpr (!kVBias) {
    const ME one = col16 == 0 ? (ME)1.0f : (ME)0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ones[e] = one;
  }
  f32x4 acc[TPH][MB], accb[TPH];
  float dbs[TPH];  // kVBias: sum of the lane's products per tap
#pragma unroll
  for (int tt = 0; tt < TPH; ++tt) {
    accb[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
    dbs[tt] = 0.f;
#pragma unroll
    for (int ib = 0; ib < MB; ++ib) acc[tt][ib] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  WgPos nxt;
  {
    const int row = step_beg / g.col_blocks;
    nxt.cbk = step_beg - row * g.col_blocks;
    nxt.w0 = nxt.cbk * TW;
    nxt.n = row / H;
    nxt.h = row - nxt.n * H;
  }
  if (steps > 0) {
    image(nxt.n);
    yload(nxt);
    stage(nxt, 0);
    nxt.advance(g);
    ystore(0);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  const int wl = 32 * sg + 8 * quad;  // this lane's first token within a 128-column subsegment
  // element index (from the buffer start) of the lane's first x value per tap
  int xel[TPH];
#pragma unroll
  for (int tt = 0; tt < TPH; ++tt) {
    const int t = th * TPH + tt;
    const int ki = t / KS, kj = t - ki * KS;
    xel[tt] = (ki * 16 + col16) * L::kXSD * L::kPerD + kWgPad + wl + (kj - r) * d;
  }
  for (int s = 0; s < steps; ++s) {
    const int buf = s & 1;
    const bool more = s + 1 < steps;
    if (more) {
      image(nxt.n);
      yload(nxt);
      stage(nxt, buf ^ 1);
      nxt.advance(g);
    }
    const uint32_t* __restrict__ bb = wsm + buf * L::kBuf;
#pragma unroll
    for (int j = 0; j < SJ; ++j) {
      // subsegment j: this lane's tokens wl + 128 j
      const int wlj = wl + kWgTW * j;
      const int kyj = (wlj >> 3) ^ col16;
      V bfr[MB][P];
#pragma unroll
      for (int ib = 0; ib < MB; ++ib)
#pragma unroll
        for (int pp = 0; pp < P; ++pp)
          bfr[ib][pp] = __builtin_bit_cast(
              V, *reinterpret_cast<const u32x4*>(bb + L::kYOff + ((pp * MB + ib) * 16 + col16) * L::kYD +
                                                 4 * kyj));
      // branch gradient of channel col16 at the lane's 8 tokens
      float gv[8];
      {
        const uint32_t* __restrict__ gr = bb + L::kGOff + col16 * L::kGD;
        if constexpr (E == 4) {
          const int kg = wlj >> 2;
          const u32x4 a0 = *reinterpret_cast<const u32x4*>(gr + 4 * (kg ^ col16));
          const u32x4 a1 = *reinterpret_cast<const u32x4*>(gr + 4 * ((kg + 1) ^ col16));
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            gv[e] = __uint_as_float(a0[e]);
            gv[4 + e] = __uint_as_float(a1[e]);
          }
        } else {
          typedef T T8 __attribute__((ext_vector_type(8)));
          const T8 t8 = __builtin_bit_cast(T8, *reinterpret_cast<const u32x4*>(gr + 4 * kyj));
#pragma unroll
          for (int e = 0; e < 8; ++e) gv[e] = to_f(t8[e]);
        }
      }
      // The A fragment of tap tt+1 (x reads, products, bf16 split) is formed
      // while tap tt's MFMAs run: the scheduling groups below put its LDS reads
      // first and then interleave each MFMA with 3 VALU instructions (measured
      // 3-5% faster than the compiler's clustering, which left the MFMA pipe
      // idle during each tap's VALU stretch)
      auto make_afr = [&](int tt, V (&af)[P]) {
        float dk[8];
        if constexpr (E == 2) {
          // the lane's 8 consecutive 2-byte x values by dword reads: 4 dwords
          // when the window starts on a dword, else 5 realigned by one element.
          // The parity is the tap shift's, (kj - r) * d: the row pitch, the pad
          // and the lane's token offset are even (wave-uniform branch)
          const int t = th * TPH + tt;
          const int kj = t - (t / KS) * KS;
          const int el = xel[tt] + kWgTW * j;
          const uint32_t* __restrict__ xp = bb + (el >> 1);
          uint32_t w[4];
          if (((kj - r) * d) & 1) {
            uint32_t d5[5];
#pragma unroll
            for (int k = 0; k < 5; ++k) d5[k] = xp[k];
#pragma unroll
            for (int k = 0; k < 4; ++k) w[k] = __builtin_amdgcn_alignbyte(d5[k + 1], d5[k], 2);
          } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) w[k] = xp[k];
          }
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            dk[2 * k] = gv[2 * k] * to_f(__builtin_bit_cast(T, (unsigned short)(w[k] & 0xffffu)));
            dk[2 * k + 1] = gv[2 * k + 1] * to_f(__builtin_bit_cast(T, (unsigned short)(w[k] >> 16)));
          }
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) dk[e] = gv[e] * lds_elem<T>(bb, xel[tt] + kWgTW * j + e);
        }
        M::pack(dk, af);
        if constexpr (kVBias)
          dbs[tt] += ((dk[0] + dk[1]) + (dk[2] + dk[3])) + ((dk[4] + dk[5]) + (dk[6] + dk[7]));
      };
      V afc[P];
      make_afr(0, afc);
#pragma unroll
      for (int tt = 0; tt < TPH; ++tt) {
        const int t = th * TPH + tt;  // wave-uniform
        if (KK % NH != 0 && t >= KK) break;
        V afn[P];
        if (tt + 1 < TPH) make_afr(tt + 1, afn);
#pragma unroll
        for (int ib = 0; ib < MB; ++ib) acc[tt][ib] = M::mac(afc, bfr[ib], acc[tt][ib]);
        if constexpr (!kVBias) {
#pragma unroll
          for (int pp = 0; pp < P; ++pp) accb[tt] = M::mac1(afc[pp], ones, accb[tt]);
        }
        if (tt + 1 < TPH) {
          __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // LDS reads
#pragma unroll
          for (int i = 0; i < MB * (P == 2 ? 3 : 1) + (kVBias ? 0 : P); ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // three VALU
          }
        }
#pragma unroll
        for (int pp = 0; pp < P; ++pp) afc[pp] = afn[pp];
      }
    }
    if (more) ystore(buf ^ 1);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }

  // ---- deterministic reduction over the segments (fixed order) through LDS:
  //      each segment's waves write their sums to the segment's own slice (one
  //      round, one barrier), and the store loop adds the slices in segment
  //      order -- the same sum, bit for bit, as accumulating segment by
  //      segment into one slice, which took four rounds of LDS
  //      read-modify-writes and barriers.  A thread stores 4 consecutive
  //      input channels (16 bytes of fp32 partials).
  constexpr int NO = MB * 16;
  constexpr int RS = NO + 1;
  constexpr int SL = KK * 16 * RS;                          // floats of one slice
  static_assert(kWgSegs == 4, "the slice sum below adds four segments");
  float* __restrict__ red = reinterpret_cast<float*>(wsm);  // [segs][KK][16 c][RS]
  float* __restrict__ rb = red + kWgSegs * SL;              // [KK][segs][16 c]
  if constexpr (kVBias) {
    // lanes col16 + 16*quad hold channel col16's sums over their 8 tokens:
    // added across the quads in a fixed order ((q0 + q1) + (q2 + q3))
#pragma unroll
    for (int tt = 0; tt < TPH; ++tt) {
      const int t = th * TPH + tt;
      if (t >= KK) break;
      float v = dbs[tt];
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      if (quad == 0) rb[(t * kWgSegs + sg) * 16 + col16] = v;
    }
  } else if (col16 == 0) {
#pragma unroll
    for (int tt = 0; tt < TPH; ++tt) {
      const int t = th * TPH + tt;
      if (t < KK)
#pragma unroll
        for (int e = 0; e < 4; ++e) rb[(t * kWgSegs + sg) * 16 + 4 * quad + e] = accb[tt][e];
    }
  }
#pragma unroll
  for (int tt = 0; tt < TPH; ++tt) {
    const int t = th * TPH + tt;
    if (t >= KK) break;
#pragma unroll
    for (int ib = 0; ib < MB; ++ib)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        red[sg * SL + (t * 16 + 4 * quad + e) * RS + ib * 16 + col16] = acc[tt][ib][e];
  }
  __syncthreads();
  // this workgroup's rows: partial row ((split*3 + b)*KK + t)*C + ch, or
  // grad_weight row (b*C + ch)*KK + t (32-bit offsets from these bases)
  float* __restrict__ pwb = pw + ((int64_t)split * 3 + b) * KK * C * C;
  T* __restrict__ dwb = dw_out + (int64_t)b * C * KK * C;
  const bool v4 = C % 4 == 0 && reinterpret_cast<uintptr_t>(pw) % 16 == 0;
  for (int idx = tid; idx < KK * 16 * NO / 4; idx += NT) {
    const int q = 4 * idx;
    const int t = q / (16 * NO);
    const int rem2 = q - t * 16 * NO;
    const int c = rem2 / NO, il = rem2 - c * NO;
    const int ch = cb * 16 + c, i = i0 + il;
    if (ch >= C || i >= C) continue;
    const float* __restrict__ sp = red + (t * 16 + c) * RS + il;
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = ((sp[e] + sp[SL + e]) + sp[2 * SL + e]) + sp[3 * SL + e];
    if (g.direct) {
      T* __restrict__ dst = dwb + (uint32_t)((ch * KK + t) * C + i);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (i + e < C) dst[e] = from_f<T>(v[e]);
    } else {
      float* __restrict__ dst = pwb + (uint32_t)((t * C + ch) * C + i);
      if (v4) {
        *reinterpret_cast<f32x4*>(dst) = (f32x4){v[0], v[1], v[2], v[3]};
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (i + e < C) dst[e] = v[e];
      }
    }
  }
  // the bias gradient: once, by the first input-channel half
  for (int idx = tid; idx < (ih == 0 ? KK * 16 : 0); idx += NT) {
    const int t = idx >> 4, c = idx & 15;
    const int ch = cb * 16 + c;
    if (ch >= C) continue;
    float v = 0.f;
    for (int j = 0; j < kWgSegs; ++j) v += rb[(t * kWgSegs + j) * 16 + c];
    if (g.direct)
      db_out[(int64_t)(b * C + ch) * KK + t] = from_f<T>(v);
    else
      pb[((int64_t)split * 3 * KK + b * KK + t) * C + ch] = v;
  }
}

// Fixed-order sum of the split partials (wg_reduce_item), one item per
// thread.  Indices are 32-bit (the host bounds 3*K*K*C*(C+1) below 2^31).
constexpr int kWgRedThreads = 256;
template <typename T, int V>
__global__ __launch_bounds__(kWgRedThreads) void gen_bwd_w_reduce_kernel(const float* __restrict__ pw,
                                                                 const float* __restrict__ pb,
                                                                 T* __restrict__ dw_out,
                                                                 T* __restrict__ db_out,
                                                                 uint32_t C, uint32_t KK,
                                                                 int splits) {
  const uint32_t item = blockIdx.x * (uint32_t)kWgRedThreads + threadIdx.x;
  wg_reduce_item<T, V>(pw, pb, dw_out, db_out, C, KK, splits, item);
}

int launch_ysplit(const float* y, uint16_t* ys, int64_t chw, int64_t total, hipStream_t stream) {
  if (total == 0) return 0;
  const int64_t n = total / chw;
  const dim3 grid((unsigned)((chw + 2047) / 2048), (unsigned)(n < 65535 ? n : 65535));
  hipLaunchKernelGGL(gen_ysplit_kernel, grid, dim3(256), 0, stream, y, ys, (uint32_t)chw,
                     (uint32_t)n);
  return (int)hipGetLastError();
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

// Splits: kWgMaxSplits, or fewer so that each has kWgMinSteps steps; one
// split means grad_weight / grad_bias are written directly.
// Columns per step: 256 for 2-byte types on images whose width is a multiple
// of 256 (twice the MFMA work per step and per barrier), else 128; a
// function of the dtype and the width only, so the workspace query agrees.
int wg_step_cols(int64_t w, int esz) { return (esz == 2 && w % (2 * kWgTW) == 0) ? 2 * kWgTW : kWgTW; }

void wgrad_geom(WGradGeom& g, int64_t n, int64_t c, int64_t h, int64_t w, int d0, int d1, int d2,
                int tw) {
  g.N = (int)n;
  g.C = (int)c;
  g.H = (int)h;
  g.W = (int)w;
  g.d0 = d0;
  g.d1 = d1;
  g.d2 = d2;
  g.cblocks = (int)((c + 15) / 16);
  g.ihalves = c > 64 ? 2 : 1;
  g.tw = tw;
  g.col_blocks = (int)((w + tw - 1) / tw);
  const int64_t steps = n * h * g.col_blocks;
  int64_t splits = kWgMaxSplits;
  if (splits > (steps + kWgMinSteps - 1) / kWgMinSteps) splits = (steps + kWgMinSteps - 1) / kWgMinSteps;
  if (splits < 1) splits = 1;
  g.steps = (int)steps;
  g.steps_per_split = (int)((steps + splits - 1) / splits);
  g.splits = (int)((steps + g.steps_per_split - 1) / g.steps_per_split);
  g.direct = g.splits == 1;
  g.xdma = 0;
  g.x16 = 0;
  g.x4 = 0;
  g.y4 = 0;
  g.dw_blocks = 0;
}

// Workspace: the fp32 split partials (none with one split).
int64_t wg_partial_bytes(const WGradGeom& g, int64_t c, int k) {
  if (g.direct) return 0;
  return (int64_t)g.splits * 3 * k * k * c * (c + 1) * (int64_t)sizeof(float);
}

}  // namespace
}  // namespace ddpm

using namespace ddpm;

extern "C" int64_t ddpm_gen_bwd_w_workspace_bytes(int64_t n, int64_t c, int64_t h, int64_t w,
                                                  int kernel_size, int dtype) {
  if (n <= 0 || c <= 0 || h <= 0 || w <= 0 || kernel_size < 1) return 0;
  if (dtype < kF32 || dtype > kF16) return 0;
  if (n * h * ((w + kWgTW - 1) / kWgTW) > 0x7fffffffLL) return 0;
  WGradGeom g;
  wgrad_geom(g, n, c, h, w, 1, 1, 1, wg_step_cols(w, dtype == kF32 ? 4 : 2));
  return wg_partial_bytes(g, c, kernel_size);
}

namespace {

// Helper workgroups for a deferred halo reduction: the CUs the weight-gradient
// grid leaves free, when that is at least a quarter of them (else the
// reduction runs as its own kernel after the partial kernel).
constexpr int kWgFillCUs = 256;
int wg_helpers(int dw_blocks) {
  const int free = kWgFillCUs - dw_blocks;
  return free >= kWgFillCUs / 4 ? free : 0;
}

// ddpm_gen_bwd_w's work.  check_only: validate and return before launching.
// fin (optional): a halo reduction of the input gradient to run alongside.
// yp (optional): the dY weight packing to run alongside.  defer (optional):
// describe the split reduction there (items 0 with one split) instead of
// launching it.
int bw_run(const void* x, const void* y, const void* grad_out, void* grad_weight,
           void* grad_bias, void* workspace, int64_t workspace_bytes, int64_t n, int64_t c,
           int64_t h, int64_t w, int kernel_size, int d0, int d1, int d2, int dtype,
           hipStream_t stream, bool check_only, const BxFinish* fin, const YPack* yp = nullptr,
           WReduce* defer = nullptr) {
  if (dtype < kF32 || dtype > kF16) return kBadArgument;
  GenGeom gg;
  int st = gen_make_geom(gg, n, c, h, w, kernel_size, d0, d1, d2);
  if (st != kOk) return st;
  if (n == 0 || c == 0 || h == 0 || w == 0) return kOk;
  if (!x || !y || !grad_out || !grad_weight || !grad_bias) return kBadArgument;
  if (gg.d0 > kWgMaxDil || gg.d1 > kWgMaxDil || gg.d2 > kWgMaxDil) return kUnsupported;
  if (n * h * ((w + kWgTW - 1) / kWgTW) > 0x7fffffffLL) return kUnsupported;
  const int esz = dtype == kF32 ? 4 : 2;
  // 32-bit buffer offsets inside one image's planes (channels padded to 16)
  if (((c + 15) / 16) * 16 * h * w * esz > 0x7fffffffLL) return kUnsupported;
  // 32-bit indices of the split reduction
  if ((int64_t)3 * kernel_size * kernel_size * c * (c + 1) > 0x7fffffffLL) return kUnsupported;
  WGradGeom g;
  wgrad_geom(g, n, c, h, w, gg.d0, gg.d1, gg.d2, wg_step_cols(w, esz));
  const int64_t need = wg_partial_bytes(g, c, kernel_size);
  if (need > 0 && (!workspace || workspace_bytes < need)) return kWorkspaceTooSmall;
  // LDS-direct dword copies of x rows need every row to start on a dword boundary
  g.xdma = (esz == 4) || ((w % 2 == 0) && ((uintptr_t)x % 4 == 0));
  g.x16 = (w % (16 / esz) == 0) && ((uintptr_t)x % 16 == 0);
  g.x4 = (w % 8 == 0) && ((uintptr_t)grad_out % 16 == 0) &&
         (esz == 4 || (uintptr_t)y % 16 == 0);
  g.y4 = (w % 4 == 0) && ((uintptr_t)y % 16 == 0);
  const int mb = c > 64 ? 4 : (int)((c + 15) / 16);  // 16-channel blocks of i per workgroup
  const int kk = kernel_size * kernel_size;
  if (kernel_size != 1 && kernel_size != 3) return kUnsupported;
  if (check_only) return kOk;
  g.dw_blocks = g.splits * 3 * g.cblocks * g.ihalves;
  const int helpers = (fin || yp) ? wg_helpers(g.dw_blocks) : 0;
  const BxFinish none{nullptr, nullptr, nullptr, TileGeom{}, 0, 1};
  const YPack nopack{nullptr, nullptr, 0, 0, 0};
  if (yp && helpers == 0) {
    const int e = yt_pack(*yp, kernel_size, dtype, stream);
    if (e != 0) return e;
  }
  float* pw = g.direct ? nullptr : (float*)workspace;
  float* pb = g.direct ? nullptr : pw + (int64_t)g.splits * 3 * kk * c * c;
  return wg_with_type(dtype, [&](auto tag) {
    using T = decltype(tag);
    auto launch = [&](auto ks, auto mbc, auto sjc, auto alc) {
      constexpr int KS = decltype(ks)::value;
      constexpr int MB = decltype(mbc)::value;
      constexpr int SJ = decltype(sjc)::value;
      constexpr bool AL = decltype(alc)::value;
      constexpr int KKc = KS * KS;
      typedef WgLds<T, KS, MB, SJ> L;
      const size_t stage = (size_t)2 * L::kBuf * 4;
      const size_t red = (size_t)(kWgSegs * KKc * 16 * (MB * 16 + 1) + KKc * kWgSegs * 16) * sizeof(float);
      const size_t lds = stage > red ? stage : red;
      const dim3 grid((unsigned)(g.dw_blocks + helpers));
      const int ae = allow_dynamic_lds(
          reinterpret_cast<const void*>(&gen_bwd_w_partial_kernel<T, KS, MB, SJ, AL>), lds);
      if (ae != 0) return ae;
      hipLaunchKernelGGL((gen_bwd_w_partial_kernel<T, KS, MB, SJ, AL>), grid,
                         dim3(64 * kWgSegs * WgTaps<KS>::kGroups), lds, stream, (const T*)x,
                         (const T*)y, (const T*)grad_out, pw, pb, (T*)grad_weight, (T*)grad_bias, g,
                         helpers > 0 && fin ? *fin : none, helpers > 0 && yp ? *yp : nopack);
      int e = (int)hipGetLastError();
      if (e == 0 && fin && helpers == 0) e = bx_finish(*fin, dtype, stream);
      if (e != 0 || g.direct) return e;
      const int64_t total_w = (int64_t)3 * KKc * c * c;
      // four input channels per thread when the rows allow 16-byte partial
      // loads and 4-element stores
      const bool v4 = c % 4 == 0 && reinterpret_cast<uintptr_t>(pw) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(grad_weight) % (4 * sizeof(T)) == 0;
      const int64_t items = (v4 ? total_w / 4 : total_w) + 3 * KKc * c;
      if (defer) {
        *defer = WReduce{pw, pb, grad_weight, grad_bias, (uint32_t)c, (uint32_t)KKc, g.splits,
                         v4 ? 1 : 0, (int)items};
        return 0;
      }
      if (v4)
        hipLaunchKernelGGL((gen_bwd_w_reduce_kernel<T, 4>),
                           dim3((unsigned)((items + kWgRedThreads - 1) / kWgRedThreads)),
                           dim3(kWgRedThreads), 0, stream, pw, pb, (T*)grad_weight, (T*)grad_bias,
                           (uint32_t)c, (uint32_t)KKc, g.splits);
      else
        hipLaunchKernelGGL((gen_bwd_w_reduce_kernel<T, 1>),
                           dim3((unsigned)((items + kWgRedThreads - 1) / kWgRedThreads)),
                           dim3(kWgRedThreads), 0, stream, pw, pb, (T*)grad_weight, (T*)grad_bias,
                           (uint32_t)c, (uint32_t)KKc, g.splits);
      return (int)hipGetLastError();
    };
    return wg_with_mb(mb, [&](auto mbc) {
      // aligned layout (16-byte x, y and gradient rows, whole steps, whole
      // 16-channel blocks): the copies take their fast forms without runtime
      // tests
      const bool al = g.x16 && g.x4 && (esz == 2 || g.y4) && w % g.tw == 0 && c % 16 == 0 &&
                      (c <= 64 || c == 128);
      auto by_k = [&](auto sjc) {
        auto by_al = [&](auto ks) {
          if (al) return launch(ks, mbc, sjc, std::true_type{});
          return launch(ks, mbc, sjc, std::false_type{});
        };
        if (kernel_size == 1) return by_al(std::integral_constant<int, 1>());
        return by_al(std::integral_constant<int, 3>());
      };
      if constexpr (sizeof(T) == 2) {
        if (g.tw == 2 * kWgTW) return by_k(std::integral_constant<int, 2>());
      }
      return by_k(std::integral_constant<int, 1>());
    });
  });
}

}  // namespace

extern "C" int ddpm_gen_bwd_w(const void* x, const void* y, const void* grad_out,
                              void* grad_weight, void* grad_bias, void* workspace,
                              int64_t workspace_bytes, int64_t n, int64_t c, int64_t h, int64_t w,
                              int kernel_size, int d0, int d1, int d2, int dtype,
                              hipStream_t stream) {
  return bw_run(x, y, grad_out, grad_weight, grad_bias, workspace, workspace_bytes, n, c, h, w,
                kernel_size, d0, d1, d2, dtype, stream, false, nullptr);
}

extern "C" int ddpm_gen_bwd_xw(const void* x, const void* y, const void* weight, const void* bias,
                               const void* grad_out, void* grad_x, void* grad_weight,
                               void* grad_bias, void* workspace_x, int64_t workspace_x_bytes,
                               void* workspace_w, int64_t workspace_w_bytes, int64_t n, int64_t c,
                               int64_t h, int64_t w, int kernel_size, int d0, int d1, int d2,
                               int dtype, hipStream_t stream) {
  // the weight-gradient part is validated first: nothing is launched when
  // either part would fail
  int st = bw_run(x, y, grad_out, grad_weight, grad_bias, workspace_w, workspace_w_bytes, n, c, h,
                  w, kernel_size, d0, d1, d2, dtype, stream, true, nullptr);
  if (st != kOk) return st;
  BxFinish fin{nullptr, nullptr, nullptr, TileGeom{}, 0, 1};
  st = bx_run(y, weight, bias, grad_out, grad_x, workspace_x, workspace_x_bytes, n, c, h, w,
              kernel_size, d0, d1, d2, dtype, stream, &fin);
  if (st != kOk || fin.part == nullptr) return st;  // fin stays empty for empty shapes
  return bw_run(x, y, grad_out, grad_weight, grad_bias, workspace_w, workspace_w_bytes, n, c, h, w,
                kernel_size, d0, d1, d2, dtype, stream, false, &fin);
}

extern "C" int ddpm_gen_bwd(const void* x, const void* y, const void* weight, const void* bias,
                            const void* grad_out, void* grad_x, void* grad_y, void* grad_weight,
                            void* grad_bias, void* workspace_x, int64_t workspace_x_bytes,
                            void* workspace_y, int64_t workspace_y_bytes, void* workspace_w,
                            int64_t workspace_w_bytes, int64_t n, int64_t c, int64_t h, int64_t w,
                            int kernel_size, int d0, int d1, int d2, int dtype,
                            hipStream_t stream) {
  // the weight- and y-gradient parts are validated first (the x part on its
  // launch): nothing is launched when any part would fail
  int st = bw_run(x, y, grad_out, grad_weight, grad_bias, workspace_w, workspace_w_bytes, n, c, h,
                  w, kernel_size, d0, d1, d2, dtype, stream, true, nullptr);
  if (st != kOk) return st;
  YPack yp{nullptr, nullptr, 0, 0, 0};
  st = yt_run(x, weight, grad_out, grad_y, workspace_y, workspace_y_bytes, n, c, h, w, kernel_size,
              d0, d1, d2, dtype, stream, kYtCheck, &yp);
  if (st != kOk || yp.total == 0) return st;  // total 0: empty shape
  BxFinish fin{nullptr, nullptr, nullptr, TileGeom{}, 0, 1};
  st = bx_run(y, weight, bias, grad_out, grad_x, workspace_x, workspace_x_bytes, n, c, h, w,
              kernel_size, d0, d1, d2, dtype, stream, &fin);
  if (st != kOk || fin.part == nullptr) return st;
  // dW; its helpers pack dY's weight and finish dX; the dY kernel's
  // workgroups then run dW's split reduction
  WReduce red{nullptr, nullptr, nullptr, nullptr, 0, 0, 0, 0, 0};
  st = bw_run(x, y, grad_out, grad_weight, grad_bias, workspace_w, workspace_w_bytes, n, c, h, w,
              kernel_size, d0, d1, d2, dtype, stream, false, &fin, &yp, &red);
  if (st != kOk) return st;
  return yt_run(x, weight, grad_out, grad_y, workspace_y, workspace_y_bytes, n, c, h, w,
                kernel_size, d0, d1, d2, dtype, stream, kYtMain, nullptr, &red);
}
