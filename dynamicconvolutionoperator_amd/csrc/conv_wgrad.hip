// Weight and bias gradients of the 3x3 fuse convolution on MFMA.
//
//   grad_weight[co][ci][ki][kj] = sum_{n,p} grad_out[n][co][p] * cat[n][ci][p + (ki-1, kj-1)]
//   grad_bias[co]               = sum_{n,p} grad_out[n][co][p]
//
// (zero padding), the backward-filter convolution the reference leaves to
// cuDNN (triton_impl.py:294, 392).  A GEMM with M = ci, N = co, K = pixels
// per tap, the same shape as the fused generator's weight gradient
// (gen_bwd_w.hip) with the shifted cat rows in place of dK and grad_out in
// place of y.  Work decomposition (CDNA4):
//   * one workgroup per (pixel split, 16-plane block of ci, and above 64
//     output planes half of the co planes): at most 16
//     splits of at least 4 steps -- a step is one image-row segment of 128
//     columns -- (16 splits x 16 blocks = 256 workgroups at C = 64, 256x256);
//     their fp32 partials are summed in split order by a second kernel
//     (deterministic, no atomics); a single split writes the gradients
//     directly;
//   * per step the 3 cat rows {h-1, h, h+1} of the 16 planes (128 + 16
//     columns) and the grad_out rows of the workgroup's (up to 64) output
//     planes are staged in LDS one step ahead, into a second buffer: cat and
//     2-byte grad_out rows by 16-byte buffer loads that write LDS directly
//     (zero outside the image); fp32 grad_out rows through registers, split
//     into bf16 hi / lo rows on the way (each thread loads its 4-column pieces
//     of the next step's rows before the step's MFMAs and writes their split
//     after them: no pre-pass over grad_out);
//   * 12 waves = 4 token segments x 3 kernel rows (three waves per SIMD); a
//     wave accumulates its row's 3 taps x 16 ci x C co on
//     v_mfma_f32_16x16x32_{bf16,f16} (fp32 operands as three bf16 products);
//   * grad_bias: workgroups of the first ceil(C/16) ci blocks each add up one
//     16-plane block of grad_out with one more MFMA per step and part (a
//     fragment of ones times grad_out).

#include "conv3x3.h"

#include <type_traits>

namespace ddpm {

constexpr int kCwSegs = 4;                  // 32-token segments per step
constexpr int kCwTW = 32 * kCwSegs;         // columns per step
constexpr int kCwPad = 8;                   // staged column halo (16 bytes of 2-byte values)
constexpr int kCwNW = 3 * kCwSegs;          // waves: segments x kernel rows
constexpr int kCwThreads = 64 * kCwNW;
constexpr int kCwMinSteps = 4;

struct CwGeom {
  int N, C, CI, H, W;   // C output planes (co), CI = 4C input planes (ci)
  int cblocks;          // ceil(CI / 16)
  int ohalves;          // 1, or 2 when C > 64: a workgroup covers 64 output planes co
  int tw;               // columns per step: kCwTW, or 2 * kCwTW (cw_step_cols)
  int col_blocks;       // ceil(W / tw)
  int splits, steps, steps_per_split;
  int direct;
  int x16;              // cat rows hold whole 16-byte chunks: one 16-byte copy per row
  int g16;              // 2-byte grad_out rows 16-byte aligned (W % 8 == 0): 16-byte copies
  int y4;               // fp32 grad_out rows 16-byte aligned (W % 4 == 0): 16-byte register loads
};

// One LDS staging buffer (dwords):
//   cat rows [3*16][kXSD]   T elements; odd pitch (the 64 lanes' reads of one
//                           element fall at most two to a bank)
//   gO rows  [P][MB*16][kYD] 2-byte elements (grad_out, or the bf16 hi / lo
//                           rows of an fp32 grad_out): 16 chunks of 16
//                           bytes, chunk k of row i at position k ^ (i & 15)
template <typename T, int MB, int SJ>
struct CwLds {
  static constexpr int P = Mma<T>::P;
  static constexpr int TW = kCwTW * SJ;  // columns per step
  static constexpr int LW = TW + 2 * kCwPad;
  static constexpr int kPerD = 4 / (int)sizeof(T);
  static constexpr int kXD = LW / kPerD;
  static constexpr int kXSD = kXD + (sizeof(T) == 4 ? 1 : 3);
  static constexpr int kYC = TW / 8;  // 16-byte chunks per gO row (16 or 32)
  static constexpr int kYD = 4 * kYC;
  static constexpr int kXRows = 3 * 16;
  static constexpr int kYRows = P * MB * 16;
  static constexpr int kYOff = kXRows * kXSD;
  static constexpr int kBuf = kYOff + kYRows * kYD;
  static_assert(kXSD % 2 == 1, "odd cat-row pitch");
  static_assert(kXD % 4 == 0, "16-byte copies move whole rows");
  static_assert(kYC % 16 == 0, "the chunk swizzle needs 16 chunks per row");
  static_assert(kXD / 4 <= 64, "one 16-byte cat copy per lane and row");
};

template <typename T>
__device__ __forceinline__ float cw_lds_elem(const uint32_t* __restrict__ base, int idx) {
  if constexpr (sizeof(T) == 4) {
    return __uint_as_float(base[idx]);
  } else {
    return to_f(reinterpret_cast<const T*>(base)[idx]);
  }
}

// Pair-plane index (kF32Pairs concat) of staged row c of 16-plane block cb:
// rows 0..7 the hi planes of the block's 8 channel pairs, rows 8..15 their lo
// planes (a 32-plane chunk holds 16 hi planes, then 16 lo planes).
__device__ __forceinline__ int cw_pair_plane(int cb, int c) {
  return (cb >> 1) * 32 + (c >> 3) * 16 + (cb & 1) * 8 + (c & 7);
}

struct CwPos {
  int n, h, w0, cbk;
  __device__ __forceinline__ void advance(const CwGeom& g) {
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

// PP (fp32): `cat` holds pair planes (kF32Pairs); staged row c < 8 of a
// 16-plane block holds the hi plane of its channels (2c, 2c+1), row 8 + c
// their lo plane.  SJ: 128-column subsegments per step (2 for 2-byte types on
// wide images: twice the work per step and per barrier; each wave takes its
// 32-token segment in both).
// AL: aligned layout (16-byte cat and grad_out rows, whole steps, whole
// 16-plane blocks of ci and co): copy offsets from per-lane parts formed once
// and scalar parts formed per step, without per-copy tests.
template <typename T, int MB, bool PP = false, int SJ = 1, bool AL = false>
__global__ __launch_bounds__(kCwThreads) void conv_wgrad_partial_kernel(
    const T* __restrict__ cat, const T* __restrict__ gout, float* __restrict__ pw,
    float* __restrict__ pb, T* __restrict__ dw_out, T* __restrict__ db_out, CwGeom g,
    CvPack pack) {
  typedef Mma<T> M;
  typedef typename M::V V;
  typedef typename M::E ME;
  typedef CwLds<T, MB, SJ> L;
  constexpr int TW = L::TW, LW = L::LW;
  static_assert(!PP || SJ == 1, "pair planes: 128-column steps");
  constexpr int P = M::P;
  constexpr int E = (int)sizeof(T);
  // fp32: grad_out goes through registers and is split into bf16 hi / lo rows
  // on the way to LDS; 2-byte types copy it global -> LDS directly
  constexpr bool kYReg = E == 4;
  extern __shared__ __attribute__((aligned(16))) uint32_t csm[];

  const int logical = xcd_remap(blockIdx.x, gridDim.x);
  const int oh = logical % g.ohalves;
  const int lsc = logical / g.ohalves;
  const int split = lsc / g.cblocks;
  const int cb = lsc - split * g.cblocks;
  const int co0 = oh * MB * 16;  // first output plane of this workgroup
  const int C = g.C, CI = g.CI, H = g.H, W = g.W;
  const int64_t HW = (int64_t)H * W;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int col16 = lane & 15, quad = lane >> 4;
  const int sg = wave % kCwSegs, ki = wave / kCwSegs;  // token segment, kernel row
  // bias: workgroup cb < ceil(C/16) of the half holding grad_out block cb sums
  // that block (kernel-row-0 waves)
  const bool bias_wg = cb < (C + 15) / 16 && cb / MB == oh;
  const bool do_bias = bias_wg && ki == 0;

  const int step_beg = split * g.steps_per_split;
  int step_end = step_beg + g.steps_per_split;
  if (step_end > g.steps) step_end = g.steps;
  const int steps = step_end > step_beg ? step_end - step_beg : 0;

  // gO copies (16-byte lanes): the lane's byte offset within one image's
  // planes at row 0, column 0 (kOob for planes >= C) and its chunk's column
  constexpr int YRPC = 64 / L::kYC;  // gO rows per 1 KB copy
  constexpr int NY = kYReg ? 0 : L::kYRows / YRPC;
  constexpr int NJ = NY > 0 ? (NY + kCwNW - 1) / kCwNW : 1;  // (no copies when NY = 0)
  uint32_t cpo[NJ];
  int cpc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int ii = wave + kCwNW * j;
    cpo[j] = kOob;
    cpc[j] = 0;
    if (ii < NY) {
      const int row = ii * YRPC + lane / L::kYC, pos = lane % L::kYC;
      const int part = row / (MB * 16), i = row - part * (MB * 16);
      cpc[j] = (pos ^ (i & 15)) * 8;
      if (co0 + i < C) cpo[j] = ((uint32_t)(part * C + co0 + i) * (uint32_t)HW + (uint32_t)cpc[j]) * 2u;
    }
  }

  // Buffer resources of one image's cat and grad_out planes, formed again only
  // when a step enters another image (aligned layout)
  BufRes rx = make_buf(cat, 0u), ry = make_buf(gout, 0u);
  int rn = -1;
  auto image = [&](int n) {
    if (AL && n != rn) {
      rn = n;
      rx = make_buf(cat + (int64_t)n * CI * HW, (uint32_t)(CI * HW * E));
      ry = make_buf(gout + (int64_t)n * C * HW, (uint32_t)(C * HW * E));
    }
  };

  // ---- operands of step `p` -> LDS buffer `buf`
  auto stage = [&](const CwPos& p, int buf) {
    uint32_t* __restrict__ dstb = csm + buf * L::kBuf;
    const BufRes xres = AL ? rx : make_buf(cat + (int64_t)p.n * CI * HW, (uint32_t)(CI * HW * E));
    if constexpr (AL) {
      // cat rows: offsets and resources of the step's 3 image rows formed
      // once (a row outside the image copies through a resource with no
      // records); each wave copies the planes c = wave, wave + 12, .. for all
      // three rows under one lane mask
      const BufRes xnul = make_buf(cat, 0u);
      uint32_t roff[3];
      BufRes rres[3];
#pragma unroll
      for (int rr = 0; rr < 3; ++rr) {
        const int hh = p.h + rr - 1;
        const bool ok = (unsigned)hh < (unsigned)H;
        roff[rr] = ok ? (uint32_t)(hh * W) * E : 0u;
        rres[rr] = ok ? xres : xnul;
      }
      const uint32_t colb = (uint32_t)(p.w0 - kCwPad + 4 * L::kPerD * lane) * E;
      const bool left = p.w0 == 0 && lane < kCwPad / (4 * L::kPerD);  // the halo left of column 0
      const bool right = p.w0 + TW == W && 4 * L::kPerD * lane >= TW + kCwPad;
      const uint32_t colv = left || right ? kOob : colb;
      if (lane < L::kXD / 4) {
#pragma unroll
        for (int jc = 0; jc < (16 + kCwNW - 1) / kCwNW; ++jc) {
          const int c = wave + kCwNW * jc;
          if (16 % kCwNW != 0 && c >= 16) break;
          const int ch = PP ? cw_pair_plane(cb, c) : cb * 16 + c;  // < CI: whole blocks
          const uint32_t cho = (uint32_t)ch * (uint32_t)HW * E;
#pragma unroll
          for (int rr = 0; rr < 3; ++rr) {
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
      // cat rows: one copy per row, lane l < kXD/4 moving the row's 16-byte chunk l
      const BufRes xnul = make_buf(cat, 0u);
      const int gw = p.w0 - kCwPad + 4 * L::kPerD * lane;
      const uint32_t colb =
          (lane < L::kXD / 4 && (unsigned)gw < (unsigned)W) ? (uint32_t)gw * E : kOob;
#pragma unroll
      for (int j = 0; j < (L::kXRows + kCwNW - 1) / kCwNW; ++j) {
        const int pr = wave + kCwNW * j;
        if (L::kXRows % kCwNW != 0 && pr >= L::kXRows) break;
        const int rr = pr >> 4, c = pr & 15;
        const int ch = PP ? cw_pair_plane(cb, c) : cb * 16 + c, hh = p.h + rr - 1;
        const bool ok = ch < CI && (unsigned)hh < (unsigned)H;
        const uint32_t soff = ok ? ((uint32_t)ch * (uint32_t)HW + (uint32_t)(hh * W)) * E : 0u;
        const BufRes rs = ok ? xres : xnul;
        if (lane < L::kXD / 4)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              rs, (__attribute__((address_space(3))) void*)(dstb + pr * L::kXSD), 16, colb, soff,
              0, 0);
      }
    } else {
      // element-wise through registers (W not a multiple of a 16-byte chunk)
      T* __restrict__ dst = reinterpret_cast<T*>(dstb);
      for (int idx = tid; idx < L::kXRows * LW; idx += kCwThreads) {
        const int pr = idx / LW, j = idx - pr * LW;
        const int rr = pr >> 4, c = pr & 15;
        const int ch = PP ? cw_pair_plane(cb, c) : cb * 16 + c;
        const int hh = p.h + rr - 1, gw = p.w0 - kCwPad + j;
        const bool ok = ch < CI && (unsigned)hh < (unsigned)H && (unsigned)gw < (unsigned)W;
        const uint32_t off = ok ? (uint32_t)(((int64_t)ch * H + hh) * W + gw) * E : kOob;
        dst[pr * L::kXSD * L::kPerD + j] = from_f<T>(buf_load1<T>(xres, off));
      }
    }
    // gO rows (P parts x MB*16 planes) in the swizzled chunk layout; planes >= C read zero
    const BufRes yres = AL ? ry : make_buf(gout + (int64_t)p.n * C * HW, (uint32_t)(C * HW * E));
    const uint32_t rowel = (uint32_t)(p.h * W);
    if (AL || g.g16) {
      const uint32_t ystep = (rowel + (uint32_t)p.w0) * 2u;
      const bool full = AL || p.w0 + TW <= W;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int ii = wave + kCwNW * j;
        if ((NY == 0 || NY % kCwNW != 0) && ii >= NY) break;
        uint32_t vo = cpo[j];
        if (!full) vo = p.w0 + cpc[j] < W ? vo : kOob;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            yres, (__attribute__((address_space(3))) void*)(dstb + L::kYOff + ii * 256), 16, vo,
            ystep, 0, 0);
      }
    } else {
      uint16_t* __restrict__ dy = reinterpret_cast<uint16_t*>(dstb + L::kYOff);
      constexpr int PY = kYReg ? 0 : L::kYRows * TW;
      for (int idx = tid; idx < PY; idx += kCwThreads) {
        const int row = idx / TW, j = idx - row * TW;
        const int i = row;
        const int w = p.w0 + j;
        const uint32_t off =
            (co0 + i < C && w < W) ? ((uint32_t)(co0 + i) * (uint32_t)HW + rowel + (uint32_t)w) * 2u
                                   : kOob;
        const int kc = (j >> 3) ^ (i & 15);
        dy[row * L::kYD * 2 + kc * 8 + (j & 7)] =
            (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(yres, off, 0, 0);
      }
    }
  };

  // ---- fp32 grad_out rows of step `p`: thread tid loads the 4-column pieces
  //      u = tid + NT*j (row u / 32, columns 4*(u % 32) .. +3) into registers
  //      (yload, before a step's MFMAs) and writes their bf16 hi / lo split to
  //      the gO rows of LDS buffer `buf` (ystore, after them), as the two
  //      8-byte halves of the row's chunk (u % 32) / 2 in the swizzled layout.
  //      Columns past the image and planes >= C read zero.
  constexpr int YU = kYReg ? MB * 16 * (TW / 4) : 1;
  constexpr int YUT = (YU + kCwThreads - 1) / kCwThreads;
  f32x4 yreg[YUT];
  // aligned layout: the lane's byte offset of piece j within a step's rows
  uint32_t ylo[AL ? YUT : 1];
  if constexpr (AL && kYReg) {
#pragma unroll
    for (int j = 0; j < YUT; ++j) {
      const int u = tid + kCwThreads * j;
      ylo[j] = ((uint32_t)(co0 + (u >> 5)) * (uint32_t)HW + 4u * (uint32_t)(u & 31)) * 4u;
    }
  }
  auto yload = [&](const CwPos& p) {
    if constexpr (AL && kYReg) {
      const uint32_t ys = ((uint32_t)(p.h * W) + (uint32_t)p.w0) * 4u;
#pragma unroll
      for (int j = 0; j < YUT; ++j) {
        const int u = tid + kCwThreads * j;
        if (YU % kCwThreads != 0 && u >= YU) break;  // wave-uniform
        yreg[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(ry, ylo[j], ys, 0));
      }
    } else if constexpr (kYReg) {
      const BufRes yres = make_buf(gout + (int64_t)p.n * C * HW, (uint32_t)(C * HW * E));
      const uint32_t rowel = (uint32_t)(p.h * W);
#pragma unroll
      for (int j = 0; j < YUT; ++j) {
        const int u = tid + kCwThreads * j;
        if (YU % kCwThreads != 0 && u >= YU) break;  // wave-uniform
        const int i = u >> 5, w = p.w0 + 4 * (u & 31);
        const bool okc = co0 + i < C;
        const uint32_t base = ((uint32_t)(co0 + i) * (uint32_t)HW + rowel + (uint32_t)w) * 4u;
        if (g.y4) {
          yreg[j] = __builtin_bit_cast(
              f32x4, __builtin_amdgcn_raw_buffer_load_b128(yres, okc && w < W ? base : kOob, 0, 0));
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
      uint32_t* __restrict__ yl = csm + buf * L::kBuf + L::kYOff;
#pragma unroll
      for (int j = 0; j < YUT; ++j) {
        const int u = tid + kCwThreads * j;
        if (YU % kCwThreads != 0 && u >= YU) break;
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

  // A fragment of ones for the bias sums
  V ones;
#pragma unroll
  for (int e = 0; e < 8; ++e) ones[e] = (ME)1.0f;
  f32x4 acc[3][MB], accb = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kj = 0; kj < 3; ++kj)
#pragma unroll
    for (int ib = 0; ib < MB; ++ib) acc[kj][ib] = f32x4{0.f, 0.f, 0.f, 0.f};

  CwPos nxt;
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
  // ddpm_fuse_conv_bwd: this workgroup's share of the input gradient's
  // weight packing, before the first step's copies are waited for
  if (pack.total > 0) cv_pack_share<T>(pack, (int)blockIdx.x, (int)gridDim.x, tid, kCwThreads);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  const int wl = 32 * sg + 8 * quad;  // this lane's first token within a 128-column subsegment
  // element index of the lane's first cat value per tap kj (row ki, plane col16)
  int xel[3];
#pragma unroll
  for (int kj = 0; kj < 3; ++kj) xel[kj] = (ki * 16 + col16) * L::kXSD * L::kPerD + kCwPad + wl + kj - 1;
  // PP: this lane's channel is half (col16 & 1) of the pair in rows col16/2 (hi)
  // and 8 + col16/2 (lo)
  const int ppel = (ki * 16 + (col16 >> 1)) * L::kXSD + kCwPad + wl - 1;
  const uint32_t ppsel = (col16 & 1) ? 0x07060302u : 0x05040100u;
  const int bib = cb - oh * MB;  // the staged gO block this workgroup sums for the bias
  for (int s = 0; s < steps; ++s) {
    const int buf = s & 1;
    const bool more = s + 1 < steps;
    if (more) {
      image(nxt.n);
      yload(nxt);
      stage(nxt, buf ^ 1);
      nxt.advance(g);
    }
    const uint32_t* __restrict__ bb = csm + buf * L::kBuf;
#pragma unroll
    for (int j = 0; j < SJ; ++j) {
      // subsegment j: this lane's tokens wl + 128 j
      const int kyj = ((wl + kCwTW * j) >> 3) ^ col16;
      V bfr[MB][P];
#pragma unroll
      for (int ib = 0; ib < MB; ++ib)
#pragma unroll
        for (int pp = 0; pp < P; ++pp)
          bfr[ib][pp] = __builtin_bit_cast(
              V, *reinterpret_cast<const u32x4*>(bb + L::kYOff + ((pp * MB + ib) * 16 + col16) * L::kYD +
                                                 4 * kyj));
      if (do_bias) {
        // grad_bias partials: ones x gO block bib (every row of D gets the sum)
#pragma unroll
        for (int ib = 0; ib < MB; ++ib)
          if (ib == bib)
#pragma unroll
            for (int pp = 0; pp < P; ++pp) accb = M::mac1(ones, bfr[ib][pp], accb);
      }
#pragma unroll
      for (int kj = 0; kj < 3; ++kj) {
        V afr[P];
        if constexpr (PP) {
          uint32_t dh[8], dl[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            dh[e] = bb[ppel + kCwTW * j + kj + e];
            dl[e] = bb[ppel + 8 * L::kXSD + kCwTW * j + kj + e];
          }
          u32x4 h4, l4;
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            h4[jj] = __builtin_amdgcn_perm(dh[2 * jj + 1], dh[2 * jj], ppsel);
            l4[jj] = __builtin_amdgcn_perm(dl[2 * jj + 1], dl[2 * jj], ppsel);
          }
          afr[0] = __builtin_bit_cast(V, h4);
          afr[1] = __builtin_bit_cast(V, l4);
        } else if constexpr (sizeof(T) == 4) {
          float xv[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) xv[e] = cw_lds_elem<T>(bb, xel[kj] + kCwTW * j + e);
          M::pack(xv, afr);
        } else {
          // the 8 two-byte values as staged, already the fragment's element
          // pairs: 4 dword reads where the window starts on a dword (kj = 1),
          // else 5 realigned by one element (the shift kj - 1 is odd; the row
          // pitch, the pad and the lane's token offset are even)
          const uint32_t* __restrict__ xp = bb + ((xel[kj] + kCwTW * j) >> 1);
          u32x4 wv;
          if (kj != 1) {
            uint32_t d5[5];
#pragma unroll
            for (int k = 0; k < 5; ++k) d5[k] = xp[k];
#pragma unroll
            for (int k = 0; k < 4; ++k) wv[k] = __builtin_amdgcn_alignbyte(d5[k + 1], d5[k], 2);
          } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) wv[k] = xp[k];
          }
          afr[0] = __builtin_bit_cast(V, wv);
        }
#pragma unroll
        for (int ib = 0; ib < MB; ++ib) acc[kj][ib] = M::mac(afr, bfr[ib], acc[kj][ib]);
      }
    }
    if (more) ystore(buf ^ 1);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }

  // ---- fixed-order reduction over the segments through LDS: each segment's
  //      waves write their sums to the segment's own slice; the store loop
  //      adds the slices in segment order
  constexpr int NO = MB * 16;
  constexpr int RS = NO + 1;
  constexpr int SL = 9 * 16 * RS;                           // floats of one slice
  float* __restrict__ red = reinterpret_cast<float*>(csm);  // [segs][9 taps][16 ci][RS]
  float* __restrict__ rb = red + kCwSegs * SL;              // [segs][16 co]
#pragma unroll
  for (int kj = 0; kj < 3; ++kj) {
    const int t = ki * 3 + kj;
#pragma unroll
    for (int ib = 0; ib < MB; ++ib)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        red[sg * SL + (t * 16 + 4 * quad + e) * RS + ib * 16 + col16] = acc[kj][ib][e];
  }
  if (do_bias && quad == 0) rb[sg * 16 + col16] = accb[0];  // row 0 of D: the column sums
  __syncthreads();
  // rows (tap t, ci = cb*16 + c), columns co; written in grad_weight's
  // [co][ci][t] order (runs of 16 ci x 9 taps per co): grad_weight directly,
  // or the split's partial [split][C][CI][9]
  float* __restrict__ pwb = pw + (int64_t)split * 9 * CI * C;
  for (int idx = tid; idx < NO * 16 * 9; idx += kCwThreads) {
    const int i = idx / (16 * 9), r = idx - i * (16 * 9);
    const int c = r / 9, t = r - c * 9;
    const int ci = cb * 16 + c;
    if (ci >= CI || co0 + i >= C) continue;
    const float* __restrict__ sp = red + (t * 16 + c) * RS + i;
    const float v = ((sp[0] + sp[SL]) + sp[2 * SL]) + sp[3 * SL];
    const int64_t o = ((int64_t)(co0 + i) * CI + ci) * 9 + t;
    if (g.direct)
      dw_out[o] = from_f<T>(v);
    else
      pwb[o] = v;
  }
  if (bias_wg && tid < 16) {
    const int co = cb * 16 + tid;
    if (co < C) {
      const float v = ((rb[tid] + rb[16 + tid]) + rb[32 + tid]) + rb[48 + tid];
      if (g.direct)
        db_out[co] = from_f<T>(v);
      else
        pb[(int64_t)split * C + co] = v;
    }
  }
}

// Fixed-order sum of the split partials (cw_reduce_item), one item per
// thread.
template <typename T, int V>
__global__ __launch_bounds__(256) void conv_wgrad_reduce_kernel(const float* __restrict__ pw,
                                                                const float* __restrict__ pb,
                                                                T* __restrict__ dw_out,
                                                                T* __restrict__ db_out, uint32_t nw,
                                                                uint32_t C, int splits) {
  const uint32_t item = blockIdx.x * 256u + threadIdx.x;
  cw_reduce_item<T, V>(pw, pb, dw_out, db_out, nw, C, splits, item);
}

// Zero fill (a kernel rather than a memset, so the call stays valid under
// stream capture): `count` elements of T.
template <typename T>
__global__ __launch_bounds__(256) void cw_zero_kernel(T* __restrict__ p, int64_t count) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < count) p[i] = from_f<T>(0.f);
}

namespace {

template <typename F>
int cw_with_type(int dt, F&& f) {
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
int cw_with_mb(int mb, F&& f) {
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

// Columns per step: 256 for 2-byte types on images whose width is a multiple
// of 256, else 128; a function of the dtype and the width only, so the
// workspace query agrees.
int cw_step_cols(int64_t w, int esz) { return (esz == 2 && w % (2 * kCwTW) == 0) ? 2 * kCwTW : kCwTW; }

void cw_geom(CwGeom& g, int64_t n, int64_t c, int64_t h, int64_t w, int tw) {
  g.N = (int)n;
  g.C = (int)c;
  g.CI = (int)(4 * c);
  g.H = (int)h;
  g.W = (int)w;
  g.cblocks = (int)((4 * c + 15) / 16);
  g.ohalves = c > 64 ? 2 : 1;
  g.tw = tw;
  g.col_blocks = (int)((w + tw - 1) / tw);
  const int64_t steps = n * h * g.col_blocks;
  int64_t splits = kCwMaxSplits;
  if (splits > (steps + kCwMinSteps - 1) / kCwMinSteps) splits = (steps + kCwMinSteps - 1) / kCwMinSteps;
  if (splits < 1) splits = 1;
  g.steps = (int)steps;
  g.steps_per_split = (int)((steps + splits - 1) / splits);
  g.splits = (int)((steps + g.steps_per_split - 1) / g.steps_per_split);
  g.direct = g.splits == 1;
  g.x16 = 0;
  g.g16 = 0;
  g.y4 = 0;
}

int64_t cw_partial_bytes(const CwGeom& g) {
  if (g.direct) return 0;
  return (int64_t)g.splits * ((int64_t)9 * g.CI * g.C + g.C) * (int64_t)sizeof(float);
}

}  // namespace
}  // namespace ddpm

using namespace ddpm;

extern "C" int64_t ddpm_fuse_conv_bwd_weight_workspace_bytes(int64_t n, int64_t c, int64_t h,
                                                             int64_t w, int dtype) {
  if (dtype == kF32Pairs) dtype = kF32;  // the same partials
  if (n <= 0 || c <= 0 || h <= 0 || w <= 0 || dtype < kF32 || dtype > kF16) return 0;
  if (n * h * ((w + kCwTW - 1) / kCwTW) > 0x7fffffffLL) return 0;
  CwGeom g;
  cw_geom(g, n, c, h, w, cw_step_cols(w, dtype == kF32 ? 4 : 2));
  return cw_partial_bytes(g);
}

int ddpm::cw_run(const void* cat, const void* grad_out, void* grad_weight, void* grad_bias,
                 void* workspace, int64_t workspace_bytes, int64_t n, int64_t c, int64_t h,
                 int64_t w, int dtype, hipStream_t stream, bool check_only, const CvPack* pack,
                 CwReduce* defer) {
  // kF32Pairs: `cat` in pair planes (whole 32-plane chunks: C % 8 == 0)
  const bool pp = dtype == kF32Pairs;
  if (pp) {
    if (c % 8 != 0) return kUnsupported;
    dtype = kF32;
  }
  if (dtype < kF32 || dtype > kF16) return kBadArgument;
  if (n < 0 || c < 0 || h < 0 || w < 0) return kBadArgument;
  if (c > 128) return kUnsupported;  // a workgroup stages the grad_out rows of 64 output planes
  if (c == 0) return kOk;
  if (!grad_weight || !grad_bias) return kBadArgument;
  const int esz = dtype == kF32 ? 4 : 2;
  if (n == 0 || h == 0 || w == 0) {
    if (check_only) return kOk;
    // an empty batch: zero gradients
    return cw_with_type(dtype, [&](auto tag) {
      using T = decltype(tag);
      const int64_t nw = c * 4 * c * 9;
      hipLaunchKernelGGL((cw_zero_kernel<T>), dim3((unsigned)((nw + 255) / 256)), dim3(256), 0,
                         stream, (T*)grad_weight, nw);
      hipLaunchKernelGGL((cw_zero_kernel<T>), dim3((unsigned)((c + 255) / 256)), dim3(256), 0,
                         stream, (T*)grad_bias, (int64_t)c);
      return (int)hipGetLastError();
    });
  }
  if (!cat || !grad_out) return kBadArgument;
  if (n * h * ((w + kCwTW - 1) / kCwTW) > 0x7fffffffLL) return kUnsupported;
  // 32-bit buffer offsets inside one image's planes
  if (4 * c * h * w * esz > 0x7fffffffLL) return kUnsupported;
  CwGeom g;
  cw_geom(g, n, c, h, w, pp ? kCwTW : cw_step_cols(w, esz));
  const int64_t need = cw_partial_bytes(g);
  if (need > 0 && (!workspace || workspace_bytes < need)) return kWorkspaceTooSmall;
  if (check_only) return kOk;
  g.x16 = (w % (16 / esz) == 0) && ((uintptr_t)cat % 16 == 0);
  g.g16 = (w % 8 == 0) && ((uintptr_t)grad_out % 16 == 0);
  g.y4 = (w % 4 == 0) && ((uintptr_t)grad_out % 16 == 0);
  float* pw = g.direct ? nullptr : (float*)workspace;
  float* pb = g.direct ? nullptr : pw + (int64_t)g.splits * 9 * 4 * c * c;
  const int mb = c > 64 ? 4 : (int)((c + 15) / 16);  // 16-plane blocks of co per workgroup
  const CvPack nopack{nullptr, nullptr, ConvGeom{}, 0, 0, 0, 0};
  return cw_with_type(dtype, [&](auto tag) {
    using T = decltype(tag);
    auto launch = [&](auto mbc, auto sjc) {
      constexpr int MB = decltype(mbc)::value;
      constexpr int SJ = decltype(sjc)::value;
      typedef CwLds<T, MB, SJ> L;
      const size_t stage = (size_t)2 * L::kBuf * 4;
      const size_t red = (size_t)(kCwSegs * 9 * 16 * (MB * 16 + 1) + kCwSegs * 16) * sizeof(float);
      const size_t lds = stage > red ? stage : red;
      // aligned layout: 16-byte rows, whole steps, whole 16-plane blocks of
      // ci (4C) and of co (one workgroup's MB blocks, or two halves of 64)
      const bool al = g.x16 && (esz == 4 ? g.y4 : g.g16) && w % g.tw == 0 && c % 4 == 0 &&
                      (c <= 64 ? c % 16 == 0 : c == 128);
      auto kern = pp ? (al ? conv_wgrad_partial_kernel<T, MB, sizeof(T) == 4 && SJ == 1, SJ, true>
                           : conv_wgrad_partial_kernel<T, MB, sizeof(T) == 4 && SJ == 1, SJ>)
                     : (al ? conv_wgrad_partial_kernel<T, MB, false, SJ, true>
                           : conv_wgrad_partial_kernel<T, MB, false, SJ>);
      const int ae = allow_dynamic_lds(reinterpret_cast<const void*>(kern), lds);
      if (ae != 0) return ae;
      hipLaunchKernelGGL(kern, dim3((unsigned)(g.splits * g.cblocks * g.ohalves)), dim3(kCwThreads), lds, stream,
                         (const T*)cat, (const T*)grad_out, pw, pb, (T*)grad_weight, (T*)grad_bias, g,
                         pack ? *pack : nopack);
      int e = (int)hipGetLastError();
      if (e != 0 || g.direct) return e;
      // four elements per item where the partials and grad_weight allow
      // 16-byte loads and 4-element stores (36 C^2 is a multiple of 4)
      const uint32_t nw = (uint32_t)(36 * c * c);
      const bool v4 = (uintptr_t)pw % 16 == 0 && (uintptr_t)grad_weight % (4 * sizeof(T)) == 0;
      const int items = (int)((v4 ? nw / 4 : nw) + c);
      if (defer) {
        *defer = CwReduce{pw, pb, grad_weight, grad_bias, nw, (uint32_t)c, g.splits, v4 ? 1 : 0,
                          items};
        return 0;
      }
      const dim3 rgrid((unsigned)((items + 255) / 256));
      if (v4)
        hipLaunchKernelGGL((conv_wgrad_reduce_kernel<T, 4>), rgrid, dim3(256), 0, stream,
                           (const float*)pw, (const float*)pb, (T*)grad_weight, (T*)grad_bias, nw,
                           (uint32_t)c, g.splits);
      else
        hipLaunchKernelGGL((conv_wgrad_reduce_kernel<T, 1>), rgrid, dim3(256), 0, stream,
                           (const float*)pw, (const float*)pb, (T*)grad_weight, (T*)grad_bias, nw,
                           (uint32_t)c, g.splits);
      return (int)hipGetLastError();
    };
    return cw_with_mb(mb, [&](auto mbc) {
      if constexpr (sizeof(T) == 2) {
        if (g.tw == 2 * kCwTW) return launch(mbc, std::integral_constant<int, 2>());
      }
      return launch(mbc, std::integral_constant<int, 1>());
    });
  });
}

extern "C" int ddpm_fuse_conv_bwd_weight(const void* cat, const void* grad_out, void* grad_weight,
                                         void* grad_bias, void* workspace, int64_t workspace_bytes,
                                         int64_t n, int64_t c, int64_t h, int64_t w, int dtype,
                                         hipStream_t stream) {
  return cw_run(cat, grad_out, grad_weight, grad_bias, workspace, workspace_bytes, n, c, h, w,
                dtype, stream, false, nullptr, nullptr);
}
