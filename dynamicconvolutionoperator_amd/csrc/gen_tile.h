// Generator tile: the workgroup body shared by the fused forward and by the
// fused backward with respect to x.
//
// One workgroup = (image n, 16-channel block, 16 x 16*CB pixel tile), 8
// waves; wave w owns tile rows 2w and 2w+1, i.e. 2*CB 16-pixel blocks (CB = 4:
// eight independent MFMA chains per wave and one weight read per 8 blocks;
// CB = 2 for halos too large for the 64-column tile).  The generator is an
// MFMA GEMM per (branch, tap): M = the 16 channels, N = 16 pixels, K = the
// input channels (v_mfma_f32_16x16x32_{bf16,f16}; fp32 runs as three bf16
// products).  Operands:
//   * y (B): each wave loads its pixel blocks once and keeps them in
//     registers for all 3*K*K products;
//   * W (A): the 16 x C slice of one (branch, tap) is converted once per
//     workgroup (fp32: split into bf16 hi/lo) into LDS in fragment order,
//     double-buffered one tap ahead, and read by all 8 waves.
// The LDS also holds a halo tile (16+2R) x (16*CB+2R) of the 16 channels as 4
// planes of 4-channel pixels, addressed per tap by a uniform shift:
//   * forward: x, zero outside the image; a lane's 4 output channels at the
//     shifted pixel are one ds_read_b128 (fp32) / ds_read_b64 (2-byte);
//     out_b[c, p] = sum_tap q(gen[(b,c,tap), p]) * x[c, p + off] stays in
//     registers until the branch's last tap;
//   * backward (BX): an fp32 accumulator, zero at the start; every tap adds
//     q(gen[(b,c,tap), p]) * gO_b[c, p] at p + off (one ds_read_b128 +
//     ds_write_b128 per lane and block).  A tap's shift is one-to-one, and
//     taps are separated by the workgroup barrier, so each accumulator entry
//     is updated by one lane at a time in the fixed tap order.  The tile, halo
//     included, is then written to a per-workgroup partial that a second
//     kernel sums over the (at most 2 x 2) workgroups covering each pixel.
// Every global access is a raw buffer access; lanes outside the image or the
// channel range use an offset past the resource's end (read as zero, write
// dropped) instead of a branch.
#pragma once

#include "conv3x3.h"

namespace ddpm {

constexpr int kGtWaves = 8;
constexpr int kGtThreads = 64 * kGtWaves;
constexpr int kGtTH = 2 * kGtWaves;  // tile rows, two per wave
constexpr int kGtMaxLds = 160 * 1024;

struct TileGeom {
  int N, C, H, W;
  int d0, d1, d2;
  int R;        // halo radius
  int cblocks;  // ceil(C/16)
  int tiles_w, tiles;
  int TW;       // tile columns (16 * CB)
  int LH, LW;   // halo tile rows / columns
  int npix;     // LH * LW
  int plane;    // bytes of one 4-channel plane of the halo tile (256-byte multiple)
  int pad;      // halo column j <-> position j + pad (R + pad = 0 mod 4) ...
  int LWp;      // ... of a row of LWp (multiple of 4) positions; see gen_tile_body
  int vec;      // W % 4 == 0: 4-column groups at positions 4k are whole inside or outside the image
};

// Waves per SIMD the tile kernels are compiled for: two (256 registers per
// lane) for the 64-column tile and for 65..128 input channels (NK = 4: the y
// operand alone takes 64 registers per 2-byte column block pair, 128 for
// fp32), else four.
template <typename T, int NK, int CB>
constexpr int gt_waves_per_eu() {
  return (CB == 4 || NK == 4) ? 2 : 4;
}

// Column blocks of 16 pixels per tile row the tile kernels try first: the y
// operand of the 64-column tile with more than 64 input channels (NK = 4)
// would not fit the registers, so those use 32 columns.
inline int gt_first_cb(int nk) { return nk > 2 ? 2 : 4; }

// Chunks of 32 input channels the tile kernels are instantiated for: 1, 2,
// or 4 for 65..128 channels (chunks past C hold zeros).
inline int gt_nk(int c) { return c <= 32 ? 1 : (c <= 64 ? 2 : 4); }

// Tiling and LDS bytes for a tile of 16 x 16*cb pixels whose LDS tile holds
// `entry` bytes per 4-channel pixel and whose weight slices have `parts`
// parts; kUnsupported when it does not fit the LDS.
inline int tile_geom(TileGeom& f, const GenGeom& g, int entry, int parts, int cb, size_t& lds) {
  f.N = g.N;
  f.C = g.C;
  f.H = g.H;
  f.W = g.W;
  f.d0 = g.d0;
  f.d1 = g.d1;
  f.d2 = g.d2;
  f.R = g.R;
  f.cblocks = g.cblocks;
  f.TW = 16 * cb;
  f.tiles_w = (g.W + f.TW - 1) / f.TW;
  f.tiles = f.tiles_w * ((g.H + kGtTH - 1) / kGtTH);
  f.LH = kGtTH + 2 * g.R;
  f.LW = f.TW + 2 * g.R;
  f.npix = f.LH * f.LW;
  f.pad = (4 - g.R % 4) % 4;
  f.LWp = (f.LW + f.pad + 3) / 4 * 4;
  f.vec = g.W % 4 == 0;
  // planes start on 256-byte boundaries: the four quads of a wave then read
  // their 4-channel entries with the fewest LDS bank conflicts (measured)
  f.plane = (f.npix * entry + 255) / 256 * 256;
  const int nk = gt_nk(g.C);
  lds = (size_t)4 * f.plane + (size_t)2 * nk * parts * 64 * 16 + (size_t)3 * g.K * g.K * 16 * 4;
  if (lds > (size_t)kGtMaxLds) return kUnsupported;
  if ((int64_t)f.tiles * g.cblocks * g.N > 0x7fffffffLL) return kUnsupported;
  return kOk;
}

// Workgroups the tile kernels aim to launch at least: the CU count of an
// MI355X (a fixed number, so that a workspace query made without a device
// agrees with the launch).
constexpr int kGtFillWGs = 256;

// Tiling of the tile kernels for a shape: 64-column tiles (32 for 65..128
// channels), 32 columns when the 64-column halo tile does not fit the LDS,
// then, for 1 or 2 input-channel chunks, narrower tiles (32, then 16
// columns) while the grid has fewer than kGtFillWGs workgroups -- at
// 128x128, C = 64 the 64-column tiles give 64 workgroups for 256 CUs
// (measured fp32 forward 43.5 -> 26.3 us with 16-column tiles).  Returns
// kOk with `cb` (16-column blocks per tile row), `f` and `lds` set.
inline int tile_geom_for(TileGeom& f, const GenGeom& g, int entry, int parts, int& cb, size_t& lds) {
  const int nk = gt_nk(g.C);
  cb = gt_first_cb(nk);
  int st = tile_geom(f, g, entry, parts, cb, lds);
  if (st == kUnsupported && cb == 4) {
    cb = 2;
    st = tile_geom(f, g, entry, parts, cb, lds);
  }
  if (st != kOk) return st;
  while (nk <= 2 && cb > 1 && (int64_t)f.N * f.tiles * f.cblocks < kGtFillWGs) {
    TileGeom f2;
    size_t lds2 = 0;
    if (tile_geom(f2, g, entry, parts, cb / 2, lds2) != kOk) break;
    f = f2;
    lds = lds2;
    cb /= 2;
  }
  return kOk;
}

// Raw element bits through a buffer resource (no conversion).
template <int E>
__device__ __forceinline__ uint32_t gf_load_raw(BufRes r, uint32_t off) {
  if constexpr (E == 4)
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
  else
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}
// The value of a raw element loaded by gf_load_raw<sizeof(T)>.
template <typename T>
__device__ __forceinline__ float gf_raw_to_f(uint32_t r) {
  if constexpr (sizeof(T) == 4)
    return __uint_as_float(r);
  else
    return to_f(__builtin_bit_cast(T, (unsigned short)r));
}
template <int E>
__device__ __forceinline__ void gf_store_raw(BufRes r, uint32_t off, uint32_t v) {
  if constexpr (E == 4)
    __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, 0);
  else
    __builtin_amdgcn_raw_buffer_store_b16((unsigned short)v, r, off, 0, 0);
}

// 4 consecutive elements at byte offset `off` (16-byte aligned for fp32,
// 8-byte for 2-byte types) as raw bits, one element per dword, and the
// matching store.
// Halo tile of x (zero outside the image) -> the 4 LDS planes of 4-channel
// entries (XB bytes each) for the workgroup's 16-channel block starting at
// channel c0 (nch of them), tile rows h0.., columns w0..; the tile's own
// pixels also go to the identity channels of the concat `out`.
// PP (fp32 only): the identity channels go to `out` as pair planes
// (kF32Pairs): channels (c, c+1) of a 32-plane chunk as one hi and one lo
// plane, 16 planes apart; C % 16 == 0.
template <typename T, int XB, int CB, bool PP = false>
__device__ __forceinline__ void gt_stage_x(const T* __restrict__ a, T* __restrict__ out,
                                           unsigned char* __restrict__ xs, const TileGeom& g,
                                           int n, int c0, int nch, int h0, int w0, int TW,
                                           int tid) {
  constexpr int E = (int)sizeof(T);
  typedef uint32_t XQ __attribute__((ext_vector_type(E)));  // one 4-channel x entry
  const int C = g.C, H = g.H, W = g.W, R = g.R, LW = g.LW;
  const int64_t HW = (int64_t)H * W;
  const uint32_t HWE = (uint32_t)HW * (uint32_t)E;
  // ---- halo tile of x (zero outside the image) -> LDS planes; the tile's
  //      own pixels also go to the identity channels of the output
  const BufRes xres = make_buf(a + ((int64_t)n * C + c0) * HW, (uint32_t)nch * HWE);
  const BufRes ores = PP ? make_buf(out + ((int64_t)n * 4 * C + (c0 & ~31)) * HW, 32u * HWE)
                        : make_buf(out + ((int64_t)n * 4 * C + c0) * HW, (uint32_t)nch * HWE);
  const uint32_t pp0 = (uint32_t)((c0 & 31) >> 1);  // PP: pair index of channels (c0, c0+1)
  if (g.vec) {
    // a task = (4-channel plane, halo row, 4 image columns a multiple of 4
    // apart from column 0): one 16-byte (8-byte) access per channel, the
    // 4 x 4 block transposed in registers into four 4-channel entries
    const int gpr = g.LWp / 4, cpos = R + g.pad;
    const int tasks = 4 * g.LH * gpr;
    // up to U tasks per thread with their loads in flight together: one
    // memory round trip for the whole halo tile up to R = 8 (at most 5, 3
    // and 2 tasks per thread for 64-, 32- and 16-column tiles); the elements
    // stay packed as loaded
    constexpr int U = CB == 4 ? 5 : CB == 2 ? 3 : 2;
    constexpr int ND = E == 4 ? 4 : 2;  // dwords of one channel's 4 columns
    typedef uint32_t VD __attribute__((ext_vector_type(ND)));
    for (int t0 = tid; t0 < tasks; t0 += U * kGtThreads) {
      VD v[U][4];  // [task][channel]
      uint32_t off[U];
      int ti[U], tk[U], tg[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int task = t0 + u * kGtThreads;
        const int k = task % gpr, rest = task / gpr;
        const int i = rest % g.LH, grp = task < tasks ? rest / g.LH : 0;
        const int gh = h0 - R + i, gc = w0 - cpos + 4 * k;
        const bool in = task < tasks && (unsigned)gh < (unsigned)H && (unsigned)gc < (unsigned)W;
        off[u] = in ? (uint32_t)(gh * W + gc) * (uint32_t)E : kOob;
        ti[u] = i;
        tk[u] = k;
        tg[u] = grp;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t o = off[u] + (uint32_t)(4 * grp + e) * HWE;
          if constexpr (E == 4)
            v[u][e] = __builtin_amdgcn_raw_buffer_load_b128(xres, o, 0, 0);
          else
            v[u][e] = __builtin_amdgcn_raw_buffer_load_b64(xres, o, 0, 0);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (t0 + u * kGtThreads >= tasks) break;
        const int i = ti[u], k = tk[u], grp = tg[u];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const int j = 4 * k + m - g.pad;
          if (j < 0 || j >= LW) continue;
          XQ q;
          if constexpr (E == 4) {
#pragma unroll
            for (int e = 0; e < 4; ++e) q[e] = v[u][e][m];
          } else {
            // channels (0, 1) and (2, 3) of column m: halves m & 1 of dword m >> 1
            const uint32_t sel = (m & 1) ? 0x07060302u : 0x05040100u;
            q[0] = __builtin_amdgcn_perm(v[u][1][m >> 1], v[u][0][m >> 1], sel);
            q[1] = __builtin_amdgcn_perm(v[u][3][m >> 1], v[u][2][m >> 1], sel);
          }
          *reinterpret_cast<XQ*>(xs + grp * g.plane + (i * LW + j) * XB) = q;
        }
        if (i >= R && i < R + kGtTH && 4 * k >= cpos && 4 * k < cpos + TW) {
          if constexpr (PP) {
            // channels (4grp + 2kp, +1): their 4 columns split into a hi and a lo vector
#pragma unroll
            for (int kp = 0; kp < 2; ++kp) {
              VD hv, lv;
#pragma unroll
              for (int m = 0; m < 4; ++m) {
                uint32_t hh, ll;
                split_bf16x2(__uint_as_float(v[u][2 * kp][m]), __uint_as_float(v[u][2 * kp + 1][m]),
                             hh, ll);
                hv[m] = hh;
                lv[m] = ll;
              }
              const uint32_t o = off[u] == kOob ? kOob : off[u] + (pp0 + 2 * grp + kp) * HWE;
              __builtin_amdgcn_raw_buffer_store_b128(hv, ores, o, 0, 0);
              __builtin_amdgcn_raw_buffer_store_b128(lv, ores, o == kOob ? kOob : o + 16u * HWE, 0, 0);
            }
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const uint32_t o = off[u] + (uint32_t)(4 * grp + e) * HWE;
              if constexpr (E == 4)
                __builtin_amdgcn_raw_buffer_store_b128(v[u][e], ores, o, 0, 0);
              else
                __builtin_amdgcn_raw_buffer_store_b64(v[u][e], ores, o, 0, 0);
            }
          }
        }
      }
    }
  } else {
    // element-wise: two pixels per thread and batch, 32 loads in flight
    // before any LDS write
    for (int p0 = tid; p0 < g.npix; p0 += 2 * kGtThreads) {
      uint32_t lo[2], so[2];
      int pix[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        pix[s] = p0 + s * kGtThreads;
        const int i = pix[s] / LW, j = pix[s] - i * LW;
        const int gh = h0 - R + i, gw = w0 - R + j;
        const bool in =
            pix[s] < g.npix && (unsigned)gh < (unsigned)H && (unsigned)gw < (unsigned)W;
        const bool inner = i >= R && i < R + kGtTH && j >= R && j < R + TW;
        lo[s] = in ? (uint32_t)(gh * W + gw) * (uint32_t)E : kOob;
        so[s] = (in && inner) ? lo[s] : kOob;
      }
      uint32_t v[2][16];
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int ch = 0; ch < 16; ++ch) v[s][ch] = gf_load_raw<E>(xres, lo[s] + ch * HWE);
      if constexpr (PP) {
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
          for (int kp = 0; kp < 8; ++kp) {
            uint32_t hh, ll;
            split_bf16x2(__uint_as_float(v[s][2 * kp]), __uint_as_float(v[s][2 * kp + 1]), hh, ll);
            const uint32_t o = so[s] == kOob ? kOob : so[s] + (pp0 + kp) * HWE;
            __builtin_amdgcn_raw_buffer_store_b32(hh, ores, o, 0, 0);
            __builtin_amdgcn_raw_buffer_store_b32(ll, ores, o == kOob ? kOob : o + 16u * HWE, 0, 0);
          }
      } else {
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
          for (int ch = 0; ch < 16; ++ch) gf_store_raw<E>(ores, so[s] + ch * HWE, v[s][ch]);
      }
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        if (pix[s] >= g.npix) continue;
#pragma unroll
        for (int grp = 0; grp < 4; ++grp) {
          XQ q;
          if constexpr (E == 4) {
#pragma unroll
            for (int e = 0; e < 4; ++e) q[e] = v[s][4 * grp + e];
          } else {
            q[0] = v[s][4 * grp] | (v[s][4 * grp + 1] << 16);
            q[1] = v[s][4 * grp + 2] | (v[s][4 * grp + 3] << 16);
          }
          *reinterpret_cast<XQ*>(xs + grp * g.plane + pix[s] * XB) = q;
        }
      }
    }
  }
}

// The y operand (B fragments, unshifted pixels) of this wave's NBW = 2*CB
// blocks of 16 pixels: 8 input channels per lane and 32-channel chunk.
template <typename T, int NK, int CB>
__device__ __forceinline__ void gt_load_y(const T* __restrict__ y,
                                          typename Mma<T>::V (&bfr)[2 * CB][NK][Mma<T>::P],
                                          const TileGeom& g, int n, int h0, int w0, int wave,
                                          int col16, int quad) {
  typedef Mma<T> M;
  constexpr int E = (int)sizeof(T);
  const int C = g.C, H = g.H, W = g.W;
  const int64_t HW = (int64_t)H * W;
  const uint32_t HWE = (uint32_t)HW * (uint32_t)E;
  const BufRes yres = make_buf(y + (int64_t)n * C * HW, (uint32_t)C * HWE);
#pragma unroll
  for (int blk = 0; blk < 2 * CB; ++blk) {
    const int gh = h0 + 2 * wave + blk / CB, gw = w0 + 16 * (blk % CB) + col16;
    const uint32_t po = (gh < H && gw < W) ? (uint32_t)(gh * W + gw) * (uint32_t)E : kOob;
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) {
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int i = 32 * kk + 8 * quad + e;
        v[e] = buf_load1<T>(yres, i < C ? po + (uint32_t)i * HWE : kOob);
      }
      M::pack(v, bfr[blk][kk]);
    }
  }
}

// a: x (forward) or grad_cat (BX); out: the concat (forward); part: the
// per-workgroup partials (BX), [N][tiles][cblocks][16][LH][LWp] fp32, halo
// column j at position j + pad and zero at the positions no column maps to:
// a tile column c (c % 4 == 0) then sits at a 16-byte aligned position in its
// own partial (c + R + pad) and in its left / right neighbour's (c + R + pad
// -/+ TW), and the 4-column groups that a neighbour's halo only partly covers
// read zeros for the rest.
template <typename T, int KS, int NK, int CB, bool BX, bool PP = false>
__device__ __forceinline__ void gen_tile_body(const T* __restrict__ a, const T* __restrict__ y,
                                              const T* __restrict__ wt, const T* __restrict__ bias,
                                              T* __restrict__ out, float* __restrict__ part,
                                              const TileGeom& g,
                                              CvPack fpk = CvPack{nullptr, nullptr, ConvGeom{}, 0,
                                                                  0, 0, 0}) {
  typedef Mma<T> M;
  typedef typename M::V V;
  constexpr int P = M::P;
  constexpr int KK = KS * KS;
  constexpr int NBT = 3 * KK;         // (branch, tap) steps
  constexpr int r = KS / 2;
  constexpr int E = (int)sizeof(T);
  constexpr int XB = BX ? 16 : 4 * E;  // bytes of one 4-channel entry of the LDS tile
  constexpr int AU = NK * P * 64;     // 16-byte units of one weight slice
  typedef uint32_t XQ __attribute__((ext_vector_type(E)));  // one 4-channel x entry
  constexpr int TW = 16 * CB;         // tile columns
  constexpr int NBW = 2 * CB;         // 16-pixel blocks per wave

  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  unsigned char* __restrict__ xs = smem;                                   // [4][plane]
  unsigned char* __restrict__ abuf = smem + 4 * g.plane;                   // [2][AU] x 16 B
  float* __restrict__ bs = reinterpret_cast<float*>(abuf + 2 * AU * 16);  // [NBT][16]

  // Block -> (n, tile, channel block), channel block fastest.
  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int cb = bid % g.cblocks;
  const int nt = bid / g.cblocks;
  const int tile = nt % g.tiles;
  const int n = nt / g.tiles;
  const int ty = tile / g.tiles_w, tx = tile - ty * g.tiles_w;
  const int h0 = ty * kGtTH, w0 = tx * TW;
  const int C = g.C, H = g.H, W = g.W, R = g.R, LW = g.LW;
  const int64_t HW = (int64_t)H * W;
  const uint32_t HWE = (uint32_t)HW * (uint32_t)E;  // bytes of one channel plane
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int col16 = lane & 15, quad = lane >> 4;
  const int c0 = cb * 16;
  const int nch = C - c0 < 16 ? C - c0 : 16;

  // ---- weight slices: thread -> (row m, input channels i, i+1) of every
  //      second 32-channel chunk; the slice of step bt is loaded during step
  //      bt-2 and written to LDS in step bt-1.  Wave (kk0, q) = (wave/4,
  //      wave%4), lane (m, e/2) = (lane%16, lane/16): the 64 lanes of a wave
  //      write 64 different LDS banks.
  constexpr int JW = (NK + 1) / 2;  // 32-channel chunks per thread
  const int wm = lane & 15, wsub = 8 * (wave & 3) + 2 * (lane >> 4), wk0 = wave >> 2;
  const BufRes wres = make_buf(wt, (uint32_t)(3 * C * KK * C * E));
  uint32_t wraw[JW][2];
  auto wload = [&](int bt) {
    const int b = bt / KK, t = bt - b * KK;
    const int c = c0 + wm;
    const uint32_t row = (uint32_t)(((b * C + c) * KK + t) * C);
#pragma unroll
    for (int j = 0; j < JW; ++j) {
      const int wi = (wk0 + 2 * j) * 32 + wsub;
      wraw[j][0] = gf_load_raw<E>(wres, (c < C && wi < C) ? (row + wi) * E : kOob);
      wraw[j][1] = gf_load_raw<E>(wres, (c < C && wi + 1 < C) ? (row + wi + 1) * E : kOob);
    }
  };
  auto wput = [&](int buf) {
#pragma unroll
    for (int j = 0; j < JW; ++j) {
      const int kk = wk0 + 2 * j;  // wave-uniform
      if (kk >= NK) break;
      // unit (kk, part, lane = m + 16*q) holds W[m][kk*32 + 8*q + e], e = 0..7
      uint32_t* __restrict__ dst = reinterpret_cast<uint32_t*>(abuf + buf * AU * 16) +
                                   (kk * P * 64 + wm + 16 * (wsub >> 3)) * 4 + ((wsub & 7) >> 1);
      if constexpr (E == 4) {
        uint32_t hi, lo;
        split_bf16x2(__uint_as_float(wraw[j][0]), __uint_as_float(wraw[j][1]), hi, lo);
        dst[0] = hi;
        dst[64 * 4] = lo;
      } else {
        dst[0] = wraw[j][0] | (wraw[j][1] << 16);
      }
    }
  };
  // ---- bias rows of this channel block, [bt][16] (raw buffer loads, kOob
  //      for the padding: no branch around them)
  constexpr int NBI = (NBT * 16 + kGtThreads - 1) / kGtThreads;
  uint32_t bv[NBI];
  auto bias_load = [&]() {
    const BufRes bres = make_buf(bias, (uint32_t)(3 * C * KK * E));
#pragma unroll
    for (int q = 0; q < NBI; ++q) {
      const int idx = tid + q * kGtThreads;
      const int m = idx & 15, bt = idx >> 4;
      const int b = bt / KK, t = bt - b * KK;
      bv[q] = gf_load_raw<E>(bres, (idx < NBT * 16 && m < nch)
                                       ? (uint32_t)((b * C + c0 + m) * KK + t) * (uint32_t)E
                                       : kOob);
    }
  };
  auto bias_put = [&]() {
#pragma unroll
    for (int q = 0; q < NBI; ++q)
      if (tid + q * kGtThreads < NBT * 16) bs[tid + q * kGtThreads] = gf_raw_to_f<T>(bv[q]);
  };
  V bfr[NBW][NK][P];  // y operand (unshifted pixels) of this wave's blocks
  if constexpr (BX) {
    bias_load();
    wload(0);
    // ---- accumulator tile = 0
    for (int i = tid; i < g.plane / 4; i += kGtThreads)
      reinterpret_cast<f32x4*>(xs)[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    bias_put();
    wput(0);
    if (NBT > 1) wload(1);
    gt_load_y<T, NK, CB>(y, bfr, g, n, h0, w0, wave, col16, quad);
  } else {
    // the x halo tile first (its loads are consumed there), then the bias
    // rows, the first weight slice and the y operand with their loads in
    // flight together
    gt_stage_x<T, XB, CB, PP>(a, out, xs, g, n, c0, nch, h0, w0, TW, tid);
    bias_load();
    wload(0);
    gt_load_y<T, NK, CB>(y, bfr, g, n, h0, w0, wave, col16, quad);
    bias_put();
    wput(0);
    if (NBT > 1) wload(1);
    // ddpm_gen_fwd_pack: this workgroup's share of the fuse convolution's
    // weight packing
    if (fpk.total > 0) cv_pack_share<T>(fpk, (int)blockIdx.x, (int)gridDim.x, tid, kGtThreads);
  }
  __syncthreads();

  // Addresses inside the loop are a lane part, kept in a few registers, plus
  // a part uniform over the wave; the asm barriers below keep the compiler
  // from hoisting their per-(block, channel) sums out of the loop, which
  // would hold one register each.
  //   LDS entry of this lane's pixel in block blk at zero shift:
  //     lbase + rbase(blk / CB) + 16 * (blk % CB) * XB, the last term the
  //     immediate offset of the LDS access
  const uint32_t lbase = (uint32_t)(quad * g.plane + col16 * XB);
  auto rbase = [&](int rr) { return (uint32_t)(((2 * wave + rr + R) * LW + R) * XB); };
  auto ebase = [&](int blk) { return rbase(blk / CB) + (uint32_t)(16 * (blk % CB) * XB); };
  //   global byte offset of channel 4*quad + e at this lane's pixel of block
  //   blk within a channel block's planes: lofs[blk % CB] + row and channel
  //   parts (kOob outside the image or the channel block)
  uint32_t lofs[CB];
#pragma unroll
  for (int cp = 0; cp < CB; ++cp) {
    const int gw = w0 + 16 * cp + col16;
    lofs[cp] = (gw < W && 4 * quad < nch) ? (uint32_t)gw * E + (uint32_t)(4 * quad) * HWE : kOob;
  }
  const int emax = nch - 4 * quad;  // channels 4*quad + e with e < emax exist
  auto goff = [&](const uint32_t (&lo)[CB], int blk, int e) {
    const int gh = h0 + 2 * wave + blk / CB;
    return (gh < H && e < emax) ? lo[blk % CB] + (uint32_t)(gh * W) * E + (uint32_t)e * HWE : kOob;
  };

  f32x4 acc[NBW];   // forward: branch output of this lane's 4 channels per block
  float go[NBW][4];  // BX: the branch gradient gO_b at this lane's pixel and 4 channels
#pragma unroll 1
  for (int bt = 0; bt < NBT; ++bt) {
    const int b = bt / KK, t = bt - b * KK;
    if (bt + 1 < NBT) {
      wput((bt + 1) & 1);
      if (bt + 2 < NBT) wload(bt + 2);
    }
    if constexpr (BX) {
      if (t == 0) {
        const BufRes gres = make_buf(a + ((int64_t)n * 4 * C + (int64_t)(b + 1) * C + c0) * HW,
                                     (uint32_t)nch * HWE);
        uint32_t lo[CB];
#pragma unroll
        for (int cp = 0; cp < CB; ++cp) {
          lo[cp] = lofs[cp];
          asm volatile("" : "+v"(lo[cp]));
        }
#pragma unroll
        for (int blk = 0; blk < NBW; ++blk)
#pragma unroll
          for (int e = 0; e < 4; ++e) go[blk][e] = buf_load1<T>(gres, goff(lo, blk, e));
      }
    }
    const int ki = t / KS, kj = t - ki * KS;
    const int d = dil_of(b, g.d0, g.d1, g.d2);
    const int shift = ((ki - r) * d * LW + (kj - r) * d) * XB;
    uint32_t lb = lbase;
    asm volatile("" : "+v"(lb));
    // forward: this lane's shifted entry in block rows 0 and 1 (the block's
    // column is the read's immediate offset); the read-modify-write of BX
    // measured 1-2% faster with one sum per block
    const unsigned char* __restrict__ px[2] = {xs + lb + (rbase(0) + shift),
                                               xs + lb + (rbase(1) + shift)};
    const unsigned char* __restrict__ ab = abuf + (bt & 1) * AU * 16;
    V afr[NK][P];
#pragma unroll
    for (int kk = 0; kk < NK; ++kk)
#pragma unroll
      for (int pp = 0; pp < P; ++pp)
        afr[kk][pp] = __builtin_bit_cast(
            V, *reinterpret_cast<const u32x4*>(ab + ((kk * P + pp) * 64 + lane) * 16));
    const f32x4 binit = *reinterpret_cast<const f32x4*>(bs + bt * 16 + 4 * quad);
    if constexpr (!BX) {
      if (t == 0) {
#pragma unroll
        for (int blk = 0; blk < NBW; ++blk) acc[blk] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
    // NBW independent accumulation chains
    f32x4 dacc[NBW];
#pragma unroll
    for (int blk = 0; blk < NBW; ++blk) dacc[blk] = binit;
#pragma unroll
    for (int kk = 0; kk < NK; ++kk)
#pragma unroll
      for (int blk = 0; blk < NBW; ++blk) dacc[blk] = M::mac(afr[kk], bfr[blk][kk], dacc[blk]);
    if constexpr (BX) {
#pragma unroll
      for (int blk = 0; blk < NBW; ++blk) {
        f32x4* __restrict__ pa = reinterpret_cast<f32x4*>(xs + lb + ebase(blk) + shift);
        f32x4 s = *pa;
        float q[4];
        quant4<T>(dacc[blk], q);
#pragma unroll
        for (int e = 0; e < 4; ++e) s[e] = fmaf(q[e], go[blk][e], s[e]);
        *pa = s;
      }
    } else {
#pragma unroll
      for (int blk = 0; blk < NBW; ++blk) {
        const XQ xq = *reinterpret_cast<const XQ*>(px[blk / CB] + 16 * (blk % CB) * XB);
        float xv[4];
        if constexpr (E == 4) {
#pragma unroll
          for (int e = 0; e < 4; ++e) xv[e] = __uint_as_float(xq[e]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            xv[e] = to_f(__builtin_bit_cast(T, (unsigned short)(xq[e >> 1] >> (16 * (e & 1)))));
        }
        float q[4];
        quant4<T>(dacc[blk], q);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[blk][e] = fmaf(q[e], xv[e], acc[blk][e]);
      }
      if (PP && t == KK - 1) {
        // ---- branch b as pair planes: channels (4quad + 2kp, +1) of output
        //      block b+1, split, to the hi / lo planes of their 32-plane chunk
        const int chb = (b + 1) * C + c0;
        const BufRes pres = make_buf(out + ((int64_t)n * 4 * C + (chb & ~31)) * HW, 32u * HWE);
        const uint32_t pbase = (uint32_t)(((chb & 31) >> 1) + 2 * quad);
        // the lane's column offsets, formed here (kept out of registers across
        // the loop, as lofs is for the plain stores)
        uint32_t pc[CB];
#pragma unroll
        for (int cp = 0; cp < CB; ++cp) {
          const int gw = w0 + 16 * cp + col16;
          pc[cp] = (gw < W && 4 * quad < nch) ? (uint32_t)gw * 4u : kOob;
          asm volatile("" : "+v"(pc[cp]));
        }
#pragma unroll
        for (int blk = 0; blk < NBW; ++blk) {
          const int gh = h0 + 2 * wave + blk / CB;
          const bool ok = gh < H && pc[blk % CB] != kOob;
#pragma unroll
          for (int kp = 0; kp < 2; ++kp) {
            uint32_t hh, ll;
            split_bf16x2(acc[blk][2 * kp], acc[blk][2 * kp + 1], hh, ll);
            const uint32_t o = ok ? pc[blk % CB] + (uint32_t)(gh * W) * 4u + (pbase + kp) * HWE : kOob;
            __builtin_amdgcn_raw_buffer_store_b32(hh, pres, o, 0, 0);
            __builtin_amdgcn_raw_buffer_store_b32(ll, pres, ok ? o + 16u * HWE : kOob, 0, 0);
          }
        }
      } else if (t == KK - 1) {
        // ---- branch b: channels c0 + 4*quad + e of output block b+1
        const BufRes bres = make_buf(out + ((int64_t)n * 4 * C + (int64_t)(b + 1) * C + c0) * HW,
                                     (uint32_t)nch * HWE);
        uint32_t lo[CB];
#pragma unroll
        for (int cp = 0; cp < CB; ++cp) {
          lo[cp] = lofs[cp];
          asm volatile("" : "+v"(lo[cp]));
        }
#pragma unroll
        for (int blk = 0; blk < NBW; ++blk)
#pragma unroll
          for (int e = 0; e < 4; ++e) buf_store1<T>(bres, goff(lo, blk, e), acc[blk][e]);
      }
    }
    lds_barrier();
  }

  if constexpr (BX) {
    // ---- the accumulator tile -> this workgroup's partial, rows inside the
    //      image only; a task = (4-channel plane, row, 4 positions): four LDS
    //      entries in, one 16-byte store per channel out.  The loop's last
    //      barrier ordered every update before these reads.
    const int64_t wg = ((int64_t)n * g.tiles + tile) * g.cblocks + cb;
    const int LHp = g.LH * g.LWp;
    const BufRes pres = make_buf(part + wg * 16 * LHp, (uint32_t)(nch * LHp * 4));
    const int gpr = g.LWp / 4;
    const int tasks = 4 * g.LH * gpr;
    for (int task = tid; task < tasks; task += kGtThreads) {
      const int k = task % gpr, rest = task / gpr;
      const int i = rest % g.LH, grp = rest / g.LH;
      const bool rowin = (unsigned)(h0 - R + i) < (unsigned)H;
      f32x4 v[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int j = 4 * k + m - g.pad;
        v[m] = (j >= 0 && j < LW)
                   ? *reinterpret_cast<const f32x4*>(xs + grp * g.plane + (i * LW + j) * 16)
                   : f32x4{0.f, 0.f, 0.f, 0.f};
      }
      const uint32_t off = rowin ? (uint32_t)(i * g.LWp + 4 * k) * 4u : kOob;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const f32x4 o = {v[0][e], v[1][e], v[2][e], v[3][e]};
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o), pres,
                                               off + (uint32_t)((4 * grp + e) * LHp * 4), 0, 0);
      }
    }
  }
}

}  // namespace ddpm
