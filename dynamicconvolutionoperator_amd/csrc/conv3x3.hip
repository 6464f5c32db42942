// The 3x3 fuse convolution of the DDPM (Conv2d(4C -> C, 3, padding 1)) on
// MFMA, consuming the [x, d0, d1, d2] concat in its NCHW layout.
//
// The reference leaves this convolution to cuDNN (triton_impl.py:294, 392);
// this file is its MI355X implementation, an implicit GEMM over the input
// planes.  Forward and input gradient are one kernel shape:
//
//   out[m, p] = bias[m] + sum_{k, ki, kj} A[m][k][ki][kj] * in[k, p + (ki-1, kj-1)]
//
//   forward:        in = cat [N][4C][H][W], A = weight [C][4C][3][3], out [N][C][H][W]
//   input gradient: in = grad_out [N][C][H][W],
//                   A[ci][co][ki][kj] = weight[co][ci][2-ki][2-kj] (the transposed,
//                   rotated kernel), out = grad_cat [N][4C][H][W], no bias
//
// with zero padding outside the image.  Work decomposition (CDNA4):
//   * one workgroup per (segment of 256 pixels, group of 16*MB output planes
//     m); a segment is RS image rows x SW = 256/RS columns (SW = 256 for wide
//     images, down to 32, so narrow images do not leave lanes idle); 8 waves,
//     two per SIMD, each owning 32 pixels of one row (two MFMA column blocks)
//     x the group's planes; MB = 4, halved while the grid has fewer
//     workgroups than the chip has CUs (at 128x128 the forward's 64 output
//     planes go to 4 workgroups of 16);
//   * the K loop runs in stages (32-plane chunk of `in`, kernel row ki): a
//     stage needs the RS rows h + ki - 1 of 32 input planes, SW + 16 columns
//     each, and the group's A slice for the 3 taps of that kernel row; both
//     are copied global -> LDS by buffer loads that write LDS directly
//     (16-byte lanes; reads outside the image return zero), one stage ahead
//     into a second buffer;
//   * A is packed once per call by a small kernel into MFMA A-fragment order
//     (fp32: split into bf16 hi / lo), so a fragment is one 16-byte LDS read;
//   * MFMA slot k = 8*quad + e of a 32-plane chunk holds plane 4*e + quad (A
//     and B alike): a lane's 8 B-operand reads are 4 planes apart and, with a
//     row pitch of 16 (mod 64) dwords, bank-conflict free; the 2-byte
//     aligned-layout instantiations instead read their B operands by
//     transposing LDS reads in natural slot order (slot k = plane k) and form
//     the tap columns -1 / +1 by DPP lane shifts;
//   * where the grid would hold more than one workgroup per CU for a row
//     segment (the fp32 input gradient at 256x256: four m groups), a
//     workgroup runs several m groups in one staging pipeline;
//   * v_mfma_f32_16x16x32_{bf16,f16}; fp32 operands run as three bf16
//     products (hi*hi + hi*lo + lo*hi), accumulation in fp32.

#include "conv3x3.h"

#include <type_traits>

namespace ddpm {

constexpr int kCvWaves = 8;
constexpr int kCvThreads = 64 * kCvWaves;
constexpr int kCvPix = 32 * kCvWaves;      // output pixels per workgroup (RS rows x SW columns)
constexpr int kCvPad = 8;                  // staged column halo (one chunk of 2-byte values)
constexpr int kCvMaxMB = 4;                // 16-plane blocks of m per workgroup, at most
constexpr int kCvFillWGs = 256;            // workgroups to aim for (the CU count of an MI355X)

// The weight packing as its own kernel (cv_pack_item per thread).
template <typename T, int MB>
__global__ __launch_bounds__(256) void conv3x3_pack_kernel(const T* __restrict__ wt,
                                                           uint32_t* __restrict__ pk, ConvGeom g,
                                                           int rot, int pairs, int nat) {
  const int total = g.mgroups * g.nc32 * 9 * MB * 64;
  const int idx = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (idx < total) cv_pack_item<T, MB>(wt, pk, g, rot, pairs, nat, idx);
}

// One LDS staging buffer (dwords): input rows [CH * 32 planes][kXS] -- a
// plane holds its RS segment rows back to back, g.seg elements each -- then
// the A slices [CH chunks][3 taps][MB][P][64 lanes][4 dwords].  The plane pitch is a
// compile-time constant, so that the operand reads take their plane offsets
// as immediates: the staged plane of one-row segments (WIDE: 272 elements)
// or the largest over the segment shapes (8 rows x 48 columns), rounded to
// 16 (mod 64) dwords so that a lane's 8 plane reads hit distinct banks.
template <typename T, int MB, bool WIDE, int CH = 1>
struct CvLds {
  static constexpr int kE = (int)sizeof(T);
  static constexpr int kPerD = 4 / kE;
  static constexpr int kPC = 16 / kE;  // elements per 16-byte chunk
  static constexpr int kXD = (WIDE ? kCvPix + 2 * kCvPad : 8 * (32 + 2 * kCvPad)) / kPerD;
  static constexpr int kXS = kXD + ((16 - kXD % 64) + 64) % 64;
  static constexpr int kAOff = 32 * CH * kXS;
  static constexpr int kAUnits1 = 3 * MB * cv_parts<T>() * 64;  // 16-byte units of one chunk
  static constexpr int kAUnits = CH * kAUnits1;
  static constexpr int kBuf = kAOff + 4 * kAUnits;
  static_assert(kCvPix == 256, "segments hold at most kXD dwords per plane");
};

// The sums of m group mg: lane (col16, quad) holds out[m = (mg*MB + ib)*16 +
// 4*quad + e] at row h, columns w + 16*blk (blk = 0, 1); fp32 partials of K
// split `ksplit` where the input planes are split, else the result in T with
// the bias.
template <typename T, bool BIAS, int MB>
__device__ __forceinline__ void cv_store(const f32x4 (&acc)[2][MB], int mg, const ConvGeom& g,
                                         const T* __restrict__ bias, T* __restrict__ out,
                                         float* __restrict__ part, int ksplit, int n, int h, int w,
                                         int quad) {
  const int H = g.H, W = g.W;
  const int64_t HW = (int64_t)H * W;
  if (h >= H) return;
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    const int wb = w + 16 * blk;
    if (wb < W) {
      const int64_t o = ((int64_t)ksplit * g.N + n) * g.M * HW + (int64_t)h * W + wb;
#pragma unroll
      for (int ib = 0; ib < MB; ++ib)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int m = (mg * MB + ib) * 16 + 4 * quad + e;
          if (m < g.M) {
            float v = acc[blk][ib][e];
            if (g.ks > 1) {
              part[o + (int64_t)m * HW] = v;
            } else {
              if constexpr (BIAS) v += to_f(bias[m]);
              out[o + (int64_t)m * HW] = from_f<T>(v);
            }
          }
        }
    }
  }
}

// out: the result in T (ks = 1), or with K split (ks > 1) the fp32 partial
// sums part[ksplit][n][M][H*W] (no bias) that conv3x3_reduce_kernel adds up.
// CH: 32-plane chunks per stage (2 for 2-byte types when a K split's chunk
// count is even: twice the MFMA work per stage and per barrier).
// AL: aligned layout -- one-row segments of 256 columns on an image whose
// width is a multiple of 256, 16-byte input rows, whole 32-plane chunks: the
// copies take their offsets from per-lane parts formed once and scalar parts
// formed per stage, without per-copy tests.
// MGL: the workgroup runs g.mgl m groups one after another in one staging
// pipeline (g.mgl = 1 otherwise).
template <typename T, bool BIAS, int MB, bool WIDE, bool PAIR = false, int CH = 1, bool AL = false,
          bool MGL = false>
__global__ __launch_bounds__(kCvThreads) void conv3x3_kernel(const T* __restrict__ in,
                                                             const uint32_t* __restrict__ pk,
                                                             const T* __restrict__ bias,
                                                             T* __restrict__ out,
                                                             float* __restrict__ part, ConvGeom g,
                                                             CwReduce red) {
  typedef Mma<T> M;
  typedef typename M::V V;
  typedef CvLds<T, MB, WIDE, CH> L;
  static_assert(!PAIR || CH == 1, "pair planes: one chunk per stage");
  constexpr int P = M::P;
  constexpr int E = (int)sizeof(T);
  extern __shared__ __attribute__((aligned(16))) uint32_t csm[];

  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int mgl = MGL ? g.mgl : 1;
  const int mgw = g.mgroups / mgl;  // workgroups per (tile, K split)
  const int mg0 = (bid % mgw) * mgl;
  const int rest = bid / mgw;
  const int ksplit = rest % g.ks;
  const int tile = rest / g.ks;
  const int tiles_img = g.tiles_h * g.tiles_w;
  const int n = tile / tiles_img;
  const int trem = tile - n * tiles_img;
  const int ty = trem / g.tiles_w;
  const int h0 = ty * g.rs, w0 = (trem - ty * g.tiles_w) * g.sw;
  const int H = g.H, W = g.W;
  const int64_t HW = (int64_t)H * W;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int col16 = lane & 15, quad = lane >> 4;
  // stages (group of CH chunks from cc0, ki) of this workgroup's K split
  // (CH divides its chunk count)
  const int cc0 = ksplit * g.cc_per;
  const int cc1 = cc0 + g.cc_per < g.nc32 ? cc0 + g.cc_per : g.nc32;
  // stages of one m group; the workgroup runs its mgl m groups' stages in
  // one pipeline (m group mg0 + s / nst1), storing each group's sums after
  // its last stage (one workgroup per tile instead of mgl short ones: the
  // staging pipeline fills once)
  const int nst1 = cc1 > cc0 ? 3 * ((cc1 - cc0) / CH) : 0;
  const int nstage = nst1 * mgl;
  // this wave's 32 pixels: segment row wseg (wave-uniform), columns pcol0 ..
  const int wseg = (32 * wave) / g.sw;
  const int pcol0 = 32 * wave - wseg * g.sw;

  const BufRes xres = make_buf(in + (int64_t)n * g.K * HW, (uint32_t)(g.K * HW * (int64_t)E));
  // 16-byte copies of a staged plane: chunk ci = pc + lane of copy `part`
  // (the last copy ends at the plane's end and may overlap the previous one)
  // is column chunk cw of segment row sgr; both are stage-invariant
  const int cps = g.seg / L::kPC;  // chunks per segment row
  const int cpp = g.rs * cps;      // chunks per staged plane (at most 96)
  constexpr int kParts = 2;
  int cpos[kParts], crow[kParts], ccol[kParts];
#pragma unroll
  for (int part = 0; part < kParts; ++part) {
    const int pc = 64 * part < cpp - 64 ? 64 * part : (cpp > 64 ? cpp - 64 : 0);
    const int ci = pc + lane;
    crow[part] = ci / cps;
    ccol[part] = (ci - crow[part] * cps) * L::kPC - kCvPad;  // column relative to w0
    cpos[part] = 4 * pc;                                     // dword offset in the plane
  }
  const int nparts = (cpp + 63) / 64;
  // aligned layout: the lane's column byte offset per copy part (kOob for the
  // halo chunks left of column 0 and right of the last column)
  uint32_t alcol[kParts];
  if constexpr (AL) {
#pragma unroll
    for (int part = 0; part < kParts; ++part) {
      const int gw = w0 + ccol[part];
      alcol[part] = (unsigned)gw < (unsigned)W ? (uint32_t)gw * (uint32_t)E : kOob;
    }
  }
  const BufRes xnul = make_buf(in, 0u);
  // ---- stage s = (chunk group) * 3 + ki -> LDS buffer `buf`
  auto stage = [&](int s, int buf) {
    const int gs = MGL ? s / nst1 : 0;  // m group of stage s
    const int mg = mg0 + gs;
    const int s1 = s - gs * nst1;
    const int ki = s1 % 3;
    const int ccb = cc0 + (s1 / 3) * CH;  // first chunk of the group
    uint32_t* __restrict__ dstb = csm + buf * L::kBuf;
    if constexpr (AL) {
      // one image row per stage (a row outside the image copies through a
      // resource with no records); plane offset and row offset are scalar
      const int hh = h0 + ki - 1;
      const bool rok = (unsigned)hh < (unsigned)H;
      const BufRes rs = rok ? xres : xnul;
      const uint32_t roff = rok ? (uint32_t)(hh * W) * (uint32_t)E : 0u;
      // 16-byte chunks of a staged row: 68 (fp32, two overlapping copies) or
      // 34 (2-byte types, one copy of 34 lanes)
      constexpr int kCpp = (kCvPix + 2 * kCvPad) * E / 16;
      constexpr int kNp = (kCpp + 63) / 64;
      if (kCpp >= 64 || lane < kCpp) {
#pragma unroll
        for (int j = 0; j < 32 * CH / kCvWaves; ++j) {
          const int cr = wave + kCvWaves * j;
          const uint32_t so = (uint32_t)(ccb * 32 + cr) * (uint32_t)HW * (uint32_t)E + roff;
#pragma unroll
          for (int part = 0; part < kNp; ++part)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rs, (__attribute__((address_space(3))) void*)(dstb + cr * L::kXS + cpos[part]), 16,
                alcol[part], so, 0, 0);
        }
      }
    } else if (g.x4) {
      // one resource for the image; a chunk outside the image (column, row or
      // plane) reads zero through its offset (W % 8 == 0: chunks are whole)
#pragma unroll
      for (int j = 0; j < 32 * CH / kCvWaves; ++j) {
        const int cr = wave + kCvWaves * j;
        const int ch = ccb * 32 + cr;
#pragma unroll
        for (int part = 0; part < kParts; ++part) {
          if (part >= nparts) break;
          // one-row segments: the row is uniform over the wave
          const int hh = h0 + (WIDE ? 0 : crow[part]) + ki - 1;
          const int gw = w0 + ccol[part];
          const bool ok = ch < g.K && (unsigned)hh < (unsigned)H && (unsigned)gw < (unsigned)W;
          const uint32_t off =
              ok ? ((uint32_t)ch * (uint32_t)HW + (uint32_t)(hh * W + gw)) * (uint32_t)E : kOob;
          if (cpp >= 64 || lane < cpp)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                xres, (__attribute__((address_space(3))) void*)(dstb + cr * L::kXS + cpos[part]), 16,
                off, 0, 0, 0);
        }
      }
    } else {
      // element-wise copy through registers (W % 8 != 0 or unaligned input)
      T* __restrict__ dst = reinterpret_cast<T*>(dstb);
      const int plen = g.rs * g.seg;
      for (int idx = tid; idx < 32 * CH * plen; idx += kCvThreads) {
        const int cr = idx / plen, j = idx - cr * plen;
        const int sgr = j / g.seg, col = j - sgr * g.seg;
        const int ch = ccb * 32 + cr, hh = h0 + sgr + ki - 1, gw = w0 - kCvPad + col;
        const bool ok = ch < g.K && (unsigned)hh < (unsigned)H && (unsigned)gw < (unsigned)W;
        const uint32_t off = ok ? ((uint32_t)ch * (uint32_t)HW + (uint32_t)(hh * W + gw)) * E : kOob;
        dst[cr * L::kXS * L::kPerD + j] = from_f<T>(buf_load1<T>(xres, off));
      }
    }
    // A slices of the stage's 3 taps, one per chunk: each contiguous in the
    // packed weight
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const uint32_t* src = pk + ((((int64_t)mg * g.nc32 + ccb + c) * 9 + ki * 3) * MB * P * 64) * 4;
      const BufRes pres = make_buf(src, (uint32_t)(L::kAUnits1 * 16));
#pragma unroll
      for (int j = 0; j < (L::kAUnits1 / 64 + kCvWaves - 1) / kCvWaves; ++j) {
        const int u = wave + kCvWaves * j;
        if ((L::kAUnits1 / 64) % kCvWaves == 0 || u < L::kAUnits1 / 64)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              pres,
              (__attribute__((address_space(3))) void*)(dstb + L::kAOff + 4 * c * L::kAUnits1 + 256 * u),
              16, (uint32_t)(u * 64 + lane) * 16u, 0, 0, 0);
      }
    }
  };

  f32x4 acc[2][MB];
#pragma unroll
  for (int blk = 0; blk < 2; ++blk)
#pragma unroll
    for (int ib = 0; ib < MB; ++ib) acc[blk][ib] = f32x4{0.f, 0.f, 0.f, 0.f};

  // ---- store of m group mg: lane holds out[m = (mg*MB + ib)*16 + 4*quad +
  //      e][pixel col16 of block]
  auto store_mg = [&](int mg) {
    cv_store<T, BIAS, MB>(acc, mg, g, bias, out, part, ksplit, n, h0 + wseg, w0 + pcol0 + col16,
                          quad);
  };

  // staged element of this lane's block-0 pixel at tap column 0: segment row
  // wseg, column pad + pcol0 + col16
  const int el0 = wseg * g.seg + kCvPad + pcol0 + col16;
  // transposing B reads (2-byte aligned layout): lane 16q + 4a + b receives
  // element b of the 8-byte reads of lanes 16q + a + 4e, e = 0..3, so lane
  // 16q + a + 4e reads columns 4a .. 4a+3 of a 16-column block in plane
  // 32c + 8q + 4h + e, and each pixel lane gets its column's planes 8q + 4h
  // .. +3 (h = 0, 1: the fragment's halves).  Blocks -1 .. 2 around the
  // wave's 32 pixels: the tap columns -1 and +1 move the pixel blocks one
  // lane within each row of 16 lanes, the end lane taken from the
  // neighbouring block (its lane 15 or 0: the reads of those blocks keep to
  // that one column group, inside the staged row).
  constexpr bool TR = sizeof(T) == 2 && WIDE && AL && !PAIR;
  uint32_t trb[4];
  if constexpr (TR) {
    const int sa = lane & 3, se = (lane >> 2) & 3;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int a = b == 0 ? 3 : (b == 3 ? 0 : sa);
      trb[b] = (uint32_t)(((8 * quad + se) * L::kXS) * 4 + (el0 - col16 + 16 * (b - 1) + 4 * a) * E);
    }
  }
  if (nstage > 0) stage(0, 0);
  // ddpm_fuse_conv_bwd (input gradient): this workgroup's share of the
  // weight gradient's split reduction, its loads in flight together with the
  // first stage's copies
  if (red.items > 0) cw_reduce_share<T>(red, (int)blockIdx.x, (int)gridDim.x, tid, kCvThreads);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int s = 0; s < nstage; ++s) {
    const int buf = s & 1;
    if (s + 1 < nstage) stage(s + 1, buf ^ 1);
    const uint32_t* __restrict__ bb = csm + buf * L::kBuf;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      // this lane's input elements: plane 32c + 4e + quad, element el0 + 16 blk + dw
      const uint32_t* __restrict__ xq = bb + (32 * c + quad) * L::kXS;
      u32x4 braw[4];
      if constexpr (TR) {
        typedef short s16x4 __attribute__((ext_vector_type(4)));
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        const char* bc = reinterpret_cast<const char*>(bb) + 32 * c * L::kXS * 4;
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const s16x4 t = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) s16x4*)(bc + trb[b] + 4 * h * L::kXS * 4));
            const u32x2 d2 = __builtin_bit_cast(u32x2, t);
            braw[b][2 * h] = d2[0];
            braw[b][2 * h + 1] = d2[1];
          }
      }
#pragma unroll
      for (int kj = 0; kj < 3; ++kj) {
        const int dw = kj - 1;
        V afr[MB][P];
#pragma unroll
        for (int ib = 0; ib < MB; ++ib)
#pragma unroll
          for (int pp = 0; pp < P; ++pp)
            afr[ib][pp] = __builtin_bit_cast(
                V, *reinterpret_cast<const u32x4*>(
                       bb + L::kAOff + 4 * (c * L::kAUnits1 + (((kj * MB) + ib) * P + pp) * 64 + lane)));
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
          const int col = el0 + 16 * blk + dw;
          V bfr[P];
          if constexpr (TR) {
            // tap column kj - 1: the block's own reads (kj = 1), or shifted
            // one lane down (kj = 0: lane n takes lane n - 1, lane 0 the
            // previous block's lane 15) or up (kj = 2: lane n takes n + 1,
            // lane 15 the next block's lane 0) within each 16-lane row
            u32x4 wv;
#pragma unroll
            for (int d = 0; d < 4; ++d) {
              const uint32_t pv = braw[blk][d], ov = braw[blk + 1][d], nv = braw[blk + 2][d];
              wv[d] = kj == 1 ? ov : (kj == 0 ? lane_shift<-1>(pv, ov, nv) : lane_shift<1>(pv, ov, nv));
            }
            bfr[0] = __builtin_bit_cast(V, wv);
          } else if constexpr (PAIR) {
            // pair planes: dword jj of the hi / lo fragment is staged plane
            // quad + 4jj / 16 + quad + 4jj (the pair 8jj + 2quad, +1), already split
            u32x4 h4, l4;
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
              h4[jj] = xq[4 * jj * L::kXS + col];
              l4[jj] = xq[(16 + 4 * jj) * L::kXS + col];
            }
            bfr[0] = __builtin_bit_cast(V, h4);
            bfr[1] = __builtin_bit_cast(V, l4);
          } else if constexpr (sizeof(T) == 4) {
            float bv[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) bv[e] = __uint_as_float(xq[4 * e * L::kXS + col]);
            M::pack(bv, bfr);
          } else {
            // the 8 two-byte values as loaded, paired into dwords (no fp32 round trip)
            const uint16_t* __restrict__ xb = reinterpret_cast<const uint16_t*>(xq);
            u32x4 wv;
#pragma unroll
            for (int e2 = 0; e2 < 4; ++e2) {
              const uint32_t lo = xb[2 * (8 * e2) * L::kXS + col];
              const uint32_t hi = xb[2 * (8 * e2 + 4) * L::kXS + col];
              wv[e2] = lo | (hi << 16);
            }
            bfr[0] = __builtin_bit_cast(V, wv);
          }
#pragma unroll
          for (int ib = 0; ib < MB; ++ib) acc[blk][ib] = M::mac(afr[ib], bfr, acc[blk][ib]);
        }
      }
    }
    // (the stage's LDS-direct copies are vector memory operations: wait for
    // all of them, then the barrier)
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (MGL && (s + 1) % nst1 == 0) {
      // the m group's last stage: its sums out (the stores complete under the
      // next group's first stage), the accumulators cleared for that group
      store_mg(mg0 + s / nst1);
#pragma unroll
      for (int blk = 0; blk < 2; ++blk)
#pragma unroll
        for (int ib = 0; ib < MB; ++ib) acc[blk][ib] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }

  if (!MGL) {
    store_mg(mg0);
  } else if (nst1 == 0) {
    // no input planes in this K split: its partial sums are zero
    for (int mg = mg0; mg < mg0 + mgl; ++mg) store_mg(mg);
  }
}

// out[n][m][p] = bias[m] + sum over the K splits of part[s][n][m][p], in
// split order (deterministic); VEC consecutive pixels per thread.
template <typename T, bool BIAS, int VEC>
__global__ __launch_bounds__(256) void conv3x3_reduce_kernel(const float* __restrict__ part,
                                                             const T* __restrict__ bias,
                                                             T* __restrict__ out, int64_t total,
                                                             int64_t hw, int m, int ks) {
  const int64_t i0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * VEC;
  if (i0 >= total) return;
  float v[VEC];
  const float b = BIAS ? to_f(bias[(i0 / hw) % m]) : 0.f;  // VEC pixels share a plane (hw % VEC == 0)
#pragma unroll
  for (int e = 0; e < VEC; ++e) v[e] = b;
  for (int s = 0; s < ks; ++s) {
    if constexpr (VEC == 4) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(part + (int64_t)s * total + i0);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] += a[e];
    } else {
      v[0] += part[(int64_t)s * total + i0];
    }
  }
  VecIO<T, VEC>::store(out + i0, v);
}

namespace {

template <typename F>
int cv_with_type(int dt, F&& f) {
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

int cv_pow2ceil(int64_t v) {
  int p = 1;
  while (p < v && p < (1 << 30)) p <<= 1;
  return p;
}

// Segment shape and m-block count for a shape: SW = the image width rounded
// up to a power of two within [32, 256]; MB = 4, halved while the grid has
// fewer than kCvFillWGs workgroups.  `esz` sizes the LDS staging buffers.
void cv_geom(ConvGeom& g, int64_t n, int64_t k, int64_t m, int64_t h, int64_t w, int esz) {
  g.N = (int)n;
  g.K = (int)k;
  g.M = (int)m;
  g.H = (int)h;
  g.W = (int)w;
  int sw = cv_pow2ceil(w);
  sw = sw < 32 ? 32 : (sw > kCvPix ? kCvPix : sw);
  g.sw = sw;
  g.rs = kCvPix / sw;
  g.tiles_h = (int)((h + g.rs - 1) / g.rs);
  g.tiles_w = (int)((w + sw - 1) / sw);
  g.nc32 = (int)((k + 31) / 32);
  g.mb = kCvMaxMB;
  const int64_t tiles = n * g.tiles_h * g.tiles_w;
  // fewer workgroups than CUs with four-block m groups: first split the input
  // planes (K) over up to nc32 / 2 workgroups (fp32 partials summed by a
  // second kernel; each split keeps >= 2 chunks of 32 planes, so >= 6 stages),
  // then halve the m blocks
  g.ks = 1;
  const int64_t mg4 = (m + kCvMaxMB * 16 - 1) / (kCvMaxMB * 16);
  while (tiles * mg4 * g.ks < kCvFillWGs && 2 * g.ks * 2 <= g.nc32) g.ks *= 2;
  g.cc_per = (g.nc32 + g.ks - 1) / g.ks;
  g.ks = (g.nc32 + g.cc_per - 1) / g.cc_per;
  while (g.mb > 1 && tiles * ((m + g.mb * 16 - 1) / (g.mb * 16)) * g.ks < kCvFillWGs) g.mb /= 2;
  g.mgroups = (int)((m + g.mb * 16 - 1) / (g.mb * 16));
  // fp32: m groups per workgroup, the largest divisor of mgroups that leaves
  // at least kCvFillWGs workgroups (the input gradient at 256x256: 4 groups,
  // 256 workgroups of 4 x 6 stages instead of 1024 of 6: 76.0 -> 71.8 us).
  // 2-byte types keep one (their 1024 short workgroups run two to a CU: 35.8
  // -> 43.2 us with four groups each)
  g.mgl = 1;
  if (esz == 4)
    for (int d = g.mgroups; d > 1; --d)
      if (g.mgroups % d == 0 && tiles * (g.mgroups / d) * g.ks >= kCvFillWGs) {
        g.mgl = d;
        break;
      }
  g.seg = sw + 2 * kCvPad;
  g.x4 = 0;
}

int64_t cv_pack_bytes(const ConvGeom& g, int dtype) {
  return (int64_t)g.mgroups * g.nc32 * 9 * g.mb * (dtype == kF32 ? 2 : 1) * 64 * 16;
}

// Shape checks shared by both directions: K input planes, M output planes.
int cv_check(int64_t n, int64_t k, int64_t m, int64_t h, int64_t w, int dtype) {
  if (dtype < kF32 || dtype > kF16) return kBadArgument;
  if (n < 0 || k < 0 || m < 0 || h < 0 || w < 0) return kBadArgument;
  const int64_t esz = dtype == kF32 ? 4 : 2;
  // 32-bit buffer offsets inside one image's input and output planes
  if (k * h * w * esz > 0x7fffffffLL || m * h * w * esz > 0x7fffffffLL) return kUnsupported;
  if (h > (1 << 20) || w > (1 << 20)) return kUnsupported;
  // the grid at its largest (32-column segments of 8 rows, single m blocks)
  const int64_t groups = n * ((h + 7) / 8) * ((w + 31) / 32) * ((m + 15) / 16);
  if (groups > 0x7fffffffLL) return kUnsupported;
  // 32-bit indices of the weight packing: (m/16 + 4) blocks x 9 taps x 64 lanes per 32 planes
  if (((m + 15) / 16 + 4) * ((k + 31) / 32) * 9 * 64 > 0x7fffffffLL) return kUnsupported;
  return kOk;
}

int64_t cv_align(int64_t v) { return (v + 255) / 256 * 256; }

// Workspace of one direction: the packed weight, then (K split) the fp32
// partial sums [ks][n][m][h*w].
int64_t cv_workspace_bytes(const ConvGeom& g, int dtype) {
  const int64_t pk = cv_pack_bytes(g, dtype);
  if (g.ks <= 1) return pk;
  return cv_align(pk) + (int64_t)g.ks * g.N * g.M * g.H * g.W * (int64_t)sizeof(float);
}

// Launch plan of one direction: the geometry, the aligned layout (256-column
// segments on whole image rows, 16-byte rows, whole 32-plane chunks in every
// K split) and, with 2-byte types and four m blocks, the natural slot order of
// the transposing B reads; several m groups per workgroup only for the fp32
// input gradient's aligned layout (plain concat layout, no bias).
struct CvPlan {
  ConvGeom g;
  bool al, nat;
};
void cv_plan(CvPlan& p, const void* in, int64_t n, int64_t k, int64_t m, int64_t h, int64_t w,
             int dtype, bool pairs, bool bias) {
  const int esz = dtype == kF32 ? 4 : 2;
  ConvGeom& g = p.g;
  cv_geom(g, n, k, m, h, w, esz);
  g.x4 = (w % 8 == 0) && ((uintptr_t)in % 16 == 0);
  p.al = g.rs == 1 && g.sw == kCvPix && w % kCvPix == 0 && g.x4 && k % 32 == 0 &&
         g.nc32 % g.cc_per == 0;
  p.nat = esz == 2 && p.al && g.mb == 4;
  if (!(esz == 4 && p.al && g.mb == 4 && !pairs && !bias)) g.mgl = 1;
}

// red (optional): a weight-gradient split reduction for the kernel's
// workgroups to run.  pack false: `workspace` already holds the packed weight.
int cv_run(const void* in, const void* wt, const void* bias, void* out, void* workspace,
           int64_t workspace_bytes, int64_t n, int64_t k, int64_t m, int64_t h, int64_t w, int rot,
           int dtype, hipStream_t stream, bool pairs = false, const CwReduce* red = nullptr,
           bool pack = true) {
  CvPlan plan;
  cv_plan(plan, in, n, k, m, h, w, dtype, pairs, bias != nullptr);
  ConvGeom& g = plan.g;
  const int64_t need = cv_workspace_bytes(g, dtype);
  if (!workspace || workspace_bytes < need || (uintptr_t)workspace % 16 != 0)
    return kWorkspaceTooSmall;
  float* part = g.ks > 1 ? (float*)((char*)workspace + cv_align(cv_pack_bytes(g, dtype))) : nullptr;
  const CwReduce nored{nullptr, nullptr, nullptr, nullptr, 0, 0, 0, 0, 0};
  const CwReduce& rd = red ? *red : nored;
  return cv_with_type(dtype, [&](auto tag) {
    using T = decltype(tag);
    const bool al = plan.al, nat = plan.nat;
    const int64_t units = (int64_t)g.mgroups * g.nc32 * 9 * g.mb * 64;
    const dim3 pgrid((unsigned)((units + 255) / 256));
    if (pack) {
      if (g.mb == 4)
        hipLaunchKernelGGL((conv3x3_pack_kernel<T, 4>), pgrid, dim3(256), 0, stream, (const T*)wt,
                           (uint32_t*)workspace, g, rot, (int)pairs, (int)nat);
      else if (g.mb == 2)
        hipLaunchKernelGGL((conv3x3_pack_kernel<T, 2>), pgrid, dim3(256), 0, stream, (const T*)wt,
                           (uint32_t*)workspace, g, rot, (int)pairs, (int)nat);
      else
        hipLaunchKernelGGL((conv3x3_pack_kernel<T, 1>), pgrid, dim3(256), 0, stream, (const T*)wt,
                           (uint32_t*)workspace, g, rot, (int)pairs, (int)nat);
      const int e = (int)hipGetLastError();
      if (e != 0) return e;
    }
    const dim3 grid((unsigned)((int64_t)n * g.tiles_h * g.tiles_w * (g.mgroups / g.mgl) * g.ks));
    auto launch = [&](auto kern, size_t lds) {
      const int ae = allow_dynamic_lds(reinterpret_cast<const void*>(kern), lds);
      if (ae != 0) return ae;
      hipLaunchKernelGGL(kern, grid, dim3(kCvThreads), lds, stream, (const T*)in,
                         (const uint32_t*)workspace, (const T*)bias, (T*)out, part, g, rd);
      int e2 = (int)hipGetLastError();
      if (e2 != 0 || g.ks <= 1) return e2;
      // the K splits' partial sums (and the bias) in split order
      const int64_t total = n * m * h * w, hw = h * w;
      const bool v4 = hw % 4 == 0 && (uintptr_t)out % (4 * sizeof(T)) == 0;
      const int64_t items = v4 ? total / 4 : total;
      const dim3 rgrid((unsigned)((items + 255) / 256));
      auto reduce = [&](auto bconst, auto vconst) {
        constexpr bool RB = decltype(bconst)::value;
        constexpr int RV = decltype(vconst)::value;
        hipLaunchKernelGGL((conv3x3_reduce_kernel<T, RB, RV>), rgrid, dim3(256), 0, stream,
                           (const float*)part, (const T*)bias, (T*)out, total, hw, (int)m, g.ks);
        return (int)hipGetLastError();
      };
      if (bias)
        return v4 ? reduce(std::true_type(), std::integral_constant<int, 4>())
                  : reduce(std::true_type(), std::integral_constant<int, 1>());
      return v4 ? reduce(std::false_type(), std::integral_constant<int, 4>())
                : reduce(std::false_type(), std::integral_constant<int, 1>());
    };
    auto pick = [&](auto b, auto pr) {
      constexpr bool B = decltype(b)::value;
      constexpr bool PR = decltype(pr)::value && sizeof(T) == 4;
      // one-row segments (wide images) with the narrower staging pitch; 2-byte
      // types take two chunks per stage where every K split's chunk count is
      // even and the grid has one workgroup per CU at most (the 122 KB of LDS
      // leave no room for a second: with more workgroups, as the input
      // gradient's 1024 at 256x256, measured 37 -> 50 us; forward 41.1 ->
      // 40.2 us)
      if constexpr (sizeof(T) == 2) {
        if (g.mb == 4 && g.rs == 1 && g.cc_per % 2 == 0 && g.nc32 % g.cc_per == 0 &&
            (int64_t)grid.x <= kCvFillWGs) {
          if (al)
            return launch(conv3x3_kernel<T, B, 4, true, false, 2, true>,
                          (size_t)2 * CvLds<T, 4, true, 2>::kBuf * 4);
          return launch(conv3x3_kernel<T, B, 4, true, false, 2>,
                        (size_t)2 * CvLds<T, 4, true, 2>::kBuf * 4);
        }
      }
      if (g.mb == 4 && g.rs == 1) {
        if constexpr (sizeof(T) == 4 && !B && !PR) {
          if (g.mgl > 1)
            return launch(conv3x3_kernel<T, false, 4, true, false, 1, true, true>,
                          (size_t)2 * CvLds<T, 4, true>::kBuf * 4);
        }
        if (al)
          return launch(conv3x3_kernel<T, B, 4, true, PR, 1, true>,
                        (size_t)2 * CvLds<T, 4, true>::kBuf * 4);
        return launch(conv3x3_kernel<T, B, 4, true, PR>, (size_t)2 * CvLds<T, 4, true>::kBuf * 4);
      }
      if (g.mb == 4)
        return launch(conv3x3_kernel<T, B, 4, false, PR>, (size_t)2 * CvLds<T, 4, false>::kBuf * 4);
      if (g.mb == 2)
        return launch(conv3x3_kernel<T, B, 2, false, PR>, (size_t)2 * CvLds<T, 2, false>::kBuf * 4);
      return launch(conv3x3_kernel<T, B, 1, false, PR>, (size_t)2 * CvLds<T, 1, false>::kBuf * 4);
    };
    if (pairs) {
      if (bias) return pick(std::true_type(), std::true_type());
      return pick(std::false_type(), std::true_type());
    }
    if (bias) return pick(std::true_type(), std::false_type());
    return pick(std::false_type(), std::false_type());
  });
}

}  // namespace
}  // namespace ddpm

using namespace ddpm;

extern "C" int64_t ddpm_fuse_conv_workspace_bytes(int64_t n, int64_t c, int64_t h, int64_t w,
                                                  int dtype) {
  if (dtype == kF32Pairs) dtype = kF32;  // the same packed weight and partials
  if (n < 0 || c <= 0 || h < 0 || w < 0 || dtype < kF32 || dtype > kF16) return 0;
  if (n == 0 || h == 0 || w == 0) return 0;
  // the larger of the two directions' needs at this shape
  ConvGeom gf, gd;
  cv_geom(gf, n, 4 * c, c, h, w, dtype == kF32 ? 4 : 2);  // forward: K = 4C, M = C
  cv_geom(gd, n, c, 4 * c, h, w, dtype == kF32 ? 4 : 2);  // input gradient: K = C, M = 4C
  const int64_t a = cv_workspace_bytes(gf, dtype), b = cv_workspace_bytes(gd, dtype);
  return a > b ? a : b;
}

extern "C" int ddpm_fuse_conv_fwd(const void* cat, const void* weight, const void* bias, void* out,
                                  void* workspace, int64_t workspace_bytes, int64_t n, int64_t c,
                                  int64_t h, int64_t w, int dtype, hipStream_t stream) {
  // kF32Pairs: the concat in pair planes (whole 32-plane chunks: C % 8 == 0)
  const bool pairs = dtype == kF32Pairs;
  if (pairs) {
    if (c % 8 != 0) return kUnsupported;
    dtype = kF32;
  }
  int st = cv_check(n, 4 * c, c, h, w, dtype);
  if (st != kOk) return st;
  if (n == 0 || c == 0 || h == 0 || w == 0) return kOk;
  if (!cat || !weight || !out) return kBadArgument;
  return cv_run(cat, weight, bias, out, workspace, workspace_bytes, n, 4 * c, c, h, w, 0, dtype,
                stream, pairs);
}

int ddpm::cv_fwd_pack(CvPack& p, const void* cat, const void* weight, void* workspace,
                      int64_t workspace_bytes, int64_t n, int64_t c, int64_t h, int64_t w,
                      int dtype) {
  p = CvPack{nullptr, nullptr, ConvGeom{}, 0, 0, 0, 0};
  const bool pairs = dtype == kF32Pairs;
  if (pairs) {
    if (c % 8 != 0) return kUnsupported;
    dtype = kF32;
  }
  int st = cv_check(n, 4 * c, c, h, w, dtype);
  if (st != kOk) return st;
  if (n == 0 || c == 0 || h == 0 || w == 0) return kOk;
  if (!cat || !weight) return kBadArgument;
  CvPlan plan;
  cv_plan(plan, cat, n, 4 * c, c, h, w, dtype, pairs, false);
  if (!workspace || workspace_bytes < cv_workspace_bytes(plan.g, dtype) ||
      (uintptr_t)workspace % 16 != 0)
    return kWorkspaceTooSmall;
  p = CvPack{weight, (uint32_t*)workspace, plan.g, 0, pairs ? 1 : 0, plan.nat ? 1 : 0,
             plan.g.mgroups * plan.g.nc32 * 9 * plan.g.mb * 64};
  return kOk;
}

extern "C" int ddpm_fuse_conv_fwd_packed(const void* cat, const void* bias, void* out,
                                         void* workspace, int64_t workspace_bytes, int64_t n,
                                         int64_t c, int64_t h, int64_t w, int dtype,
                                         hipStream_t stream) {
  const bool pairs = dtype == kF32Pairs;
  if (pairs) {
    if (c % 8 != 0) return kUnsupported;
    dtype = kF32;
  }
  int st = cv_check(n, 4 * c, c, h, w, dtype);
  if (st != kOk) return st;
  if (n == 0 || c == 0 || h == 0 || w == 0) return kOk;
  if (!cat || !out) return kBadArgument;
  return cv_run(cat, nullptr, bias, out, workspace, workspace_bytes, n, 4 * c, c, h, w, 0, dtype,
                stream, pairs, nullptr, false);
}

extern "C" int ddpm_fuse_conv_bwd_data(const void* grad_out, const void* weight, void* grad_cat,
                                       void* workspace, int64_t workspace_bytes, int64_t n,
                                       int64_t c, int64_t h, int64_t w, int dtype,
                                       hipStream_t stream) {
  int st = cv_check(n, c, 4 * c, h, w, dtype);
  if (st != kOk) return st;
  if (n == 0 || c == 0 || h == 0 || w == 0) return kOk;
  if (!grad_out || !weight || !grad_cat) return kBadArgument;
  return cv_run(grad_out, weight, nullptr, grad_cat, workspace, workspace_bytes, n, c, 4 * c, h, w,
                1, dtype, stream);
}

extern "C" int ddpm_fuse_conv_bwd(const void* cat, const void* weight, const void* grad_out,
                                  void* grad_cat, void* grad_weight, void* grad_bias,
                                  void* workspace_data, int64_t workspace_data_bytes,
                                  void* workspace_weight, int64_t workspace_weight_bytes, int64_t n,
                                  int64_t c, int64_t h, int64_t w, int dtype, hipStream_t stream) {
  // `dtype` is the concat's code (kF32Pairs: pair planes, read by the weight
  // gradient only); grad_out, weight and grad_cat are plain
  const int ddt = dtype == kF32Pairs ? kF32 : dtype;
  int st = cv_check(n, c, 4 * c, h, w, ddt);
  if (st != kOk) return st;
  // the weight-gradient part is validated first: nothing is launched when
  // either part would fail
  st = cw_run(cat, grad_out, grad_weight, grad_bias, workspace_weight, workspace_weight_bytes, n, c,
              h, w, dtype, stream, true, nullptr, nullptr);
  if (st != kOk) return st;
  if (n == 0 || c == 0 || h == 0 || w == 0)  // zero weight gradients; grad_cat is empty
    return cw_run(cat, grad_out, grad_weight, grad_bias, workspace_weight, workspace_weight_bytes,
                  n, c, h, w, dtype, stream, false, nullptr, nullptr);
  if (!grad_out || !weight || !grad_cat) return kBadArgument;
  CvPlan plan;
  cv_plan(plan, grad_out, n, c, 4 * c, h, w, ddt, false, false);
  const int64_t need = cv_workspace_bytes(plan.g, ddt);
  if (!workspace_data || workspace_data_bytes < need || (uintptr_t)workspace_data % 16 != 0)
    return kWorkspaceTooSmall;
  // the weight-gradient launch packs the input gradient's weight; the input
  // gradient's launch sums the weight gradient's split partials
  const CvPack pack{weight, (uint32_t*)workspace_data, plan.g, 1, 0, plan.nat ? 1 : 0,
                    plan.g.mgroups * plan.g.nc32 * 9 * plan.g.mb * 64};
  CwReduce red{nullptr, nullptr, nullptr, nullptr, 0, 0, 0, 0, 0};
  st = cw_run(cat, grad_out, grad_weight, grad_bias, workspace_weight, workspace_weight_bytes, n, c,
              h, w, dtype, stream, false, &pack, &red);
  if (st != kOk) return st;
  return cv_run(grad_out, weight, nullptr, grad_cat, workspace_data, workspace_data_bytes, n, c,
                4 * c, h, w, 1, ddt, stream, false, &red, false);
}
