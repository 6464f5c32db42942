// Generator 1x1 convolution of the materialized route:
//
//   kernels[n][o][p] = sum_i W[o][i] * y[n][i][p] + bias[o],   o < 3*C*K*K,
//
// written in the input dtype in the [N][3][C][K*K][H][W] layout the dynamic
// filter reads (the Conv2d output layout).  Counterpart of the reference's
// `self.generator(y)` on its materialized path (triton_impl.py:340-347), a
// cuDNN convolution there; MIOpen runs it here as a GEMM plus a separate
// bias pass over the whole output.
//
// The output is 3*K*K times the size of y, so the kernel is built around the
// store stream.  MFMA GEMM with M = 16 pixels, N = 16 output rows o and K =
// the input channels (v_mfma_f32_16x16x32_{bf16,f16}; fp32 runs as three
// bf16 products, hi*hi + hi*lo + lo*hi): a lane's result is 4 consecutive
// pixels of one output row, stored with the bias added and rounded once.
// fp32: one 16-byte write per block (a store instruction covers 16 rows x 64
// contiguous bytes).  2-byte types: the A rows of a pair of 16-pixel blocks
// interleave 4-pixel groups (row m of block 2j+s is pixel 32j + 8*(m/4) + 4s
// + m%4), so a lane holds 8 consecutive pixels of its row across the pair
// (16 bytes; 27% faster than two 8-byte writes), and each wave's 16 rows x
// 64 pixels then pass through a wave-private LDS tile so that a store covers
// 8 rows x 128 bytes instead of 16 rows x 64 (a write probe of this plane:
// 4.4 TB/s for the fragment shape, 6.6 TB/s for 4 rows x 256 bytes).  A wave keeps the y
// operand of its 64 pixels in registers for every output row of its chunk and
// streams the weight rows (16 bytes = 8 consecutive input channels per lane;
// all waves read the same rows, so they come from L1 / L2).

#include "gen_common.h"
#include <algorithm>
#include <type_traits>

namespace ddpm {

constexpr int kGkWaves = 4;
constexpr int kGkThreads = 64 * kGkWaves;
constexpr int kGkBlocks = 4;                          // 16-pixel blocks per wave
constexpr int kGkTP = 16 * kGkBlocks * kGkWaves;      // pixels per workgroup
constexpr int kGkMaxC = 128;                          // y operand held in registers
constexpr int kGkTargetGroups = 1024;                 // workgroups the row chunks aim for

struct GkGeom {
  int N, C, HW, O;
  int tiles;    // ceil(HW / kGkTP)
  int ochunks;  // output-row chunks per pixel tile
  int obpc;     // 16-row output blocks per chunk
  int vec;      // HW % 8 == 0 (fp32: % 4): a lane's 8 (4) pixels are stored whole
  int wvec;     // C % 8 == 0: 8 consecutive weights are one aligned vector
};

// 8 consecutive elements of a weight row starting at element `e0` (masked
// past `n` valid elements), converted to fp32.
template <typename T>
__device__ __forceinline__ void gk_load8(BufRes r, uint32_t e0, int n, bool vec, float (&v)[8]) {
  constexpr uint32_t E = sizeof(T);
  if (vec && n >= 8) {
    if constexpr (E == 4) {
      const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(r, e0 * 4u, 0, 0);
      const u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(r, e0 * 4u + 16u, 0, 0);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] = __uint_as_float(a[e]);
        v[4 + e] = __uint_as_float(b[e]);
      }
    } else {
      typedef T T8 __attribute__((ext_vector_type(8)));
      const T8 t = __builtin_bit_cast(T8, __builtin_amdgcn_raw_buffer_load_b128(r, e0 * 2u, 0, 0));
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = to_f(t[e]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = buf_load1<T>(r, e < n ? (e0 + e) * E : kOob);
  }
}

template <typename T, int NK>
__global__ __launch_bounds__(kGkThreads) void gen_kernels_kernel(const T* __restrict__ y,
                                                                 const T* __restrict__ wt,
                                                                 const T* __restrict__ bias,
                                                                 T* __restrict__ out, GkGeom g) {
  typedef Mma<T> M;
  typedef typename M::V V;
  constexpr int P = M::P;
  constexpr uint32_t E = sizeof(T);
  const int bid = blockIdx.x;
  const int oc = bid % g.ochunks;
  const int rest = bid / g.ochunks;
  const int tile = rest % g.tiles, n = rest / g.tiles;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int col16 = lane & 15, quad = lane >> 4;
  const int C = g.C, HW = g.HW, O = g.O;
  const int p0 = tile * kGkTP + wave * 16 * kGkBlocks;  // first pixel of this wave

  // ---- y operand: A row m of block blk = pixel p0 + 16*blk + m (fp32) or
  //      p0 + 32*(blk/2) + 8*(m/4) + 4*(blk%2) + m%4 (2-byte types, the pair
  //      interleave above), K = input channels
  constexpr bool kPair = E == 2;
  V afr[kGkBlocks][NK][P];
  {
    const BufRes yres = make_buf(y + (int64_t)n * C * HW, (uint32_t)C * (uint32_t)HW * E);
#pragma unroll
    for (int blk = 0; blk < kGkBlocks; ++blk) {
      const int px = kPair ? p0 + 32 * (blk >> 1) + 8 * (col16 >> 2) + 4 * (blk & 1) + (col16 & 3)
                           : p0 + 16 * blk + col16;
      const uint32_t po = px < HW ? (uint32_t)px * E : kOob;
#pragma unroll
      for (int kk = 0; kk < NK; ++kk) {
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int i = 32 * kk + 8 * quad + e;
          v[e] = buf_load1<T>(yres, i < C ? po + (uint32_t)i * (uint32_t)HW * E : kOob);
        }
        M::pack(v, afr[blk][kk]);
      }
    }
  }

  const int nob = (O + 15) / 16;
  const int ob0 = oc * g.obpc;
  const int ob1 = ob0 + g.obpc < nob ? ob0 + g.obpc : nob;
  const BufRes wres = make_buf(wt, (uint32_t)O * (uint32_t)C * E);
  const BufRes bres = make_buf(bias, (uint32_t)O * E);
  const BufRes ores = make_buf(out + (int64_t)n * O * HW, (uint32_t)O * (uint32_t)HW * E);
  const bool vec = g.vec != 0, wvec = g.wvec != 0;
  // 2-byte types: each wave turns its 16 rows x 64 pixels around in a private
  // LDS tile and stores 8 rows x 128 contiguous bytes per instruction instead
  // of 16 rows x 64 bytes (measured 6% faster; a wave's own LDS accesses are
  // ordered, so no barrier).  fp32 keeps the fragment-shaped stores: the same
  // transpose measured 40% slower at 128x128 K=5 (9% faster at 256x256 K=3).
  constexpr int TROW = 64 * (int)E + 16;  // padded tile row (bytes)
  constexpr int LPR = 64 * (int)E / 16;   // lanes per tile row
  constexpr int RPI = 64 / LPR;           // tile rows per store instruction
  __shared__ __attribute__((aligned(16))) char wtile[kPair ? kGkWaves : 1][kPair ? 16 * TROW : 16];
  char* __restrict__ wtp = wtile[kPair ? wave : 0];
  // one output block per iteration: the body is too large to unroll (asking
  // for two leaves the code unchanged)
#pragma unroll 1
  for (int ob = ob0; ob < ob1; ++ob) {
    const int o = ob * 16 + col16;  // this lane's output row (B column)
    const bool orow = o < O;
    // B fragments: W[o][32*kk + 8*quad + e]
    V bfr[NK][P];
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) {
      const int i0 = 32 * kk + 8 * quad;
      float v[8];
      gk_load8<T>(wres, (uint32_t)(o * C + i0), orow ? C - i0 : 0, wvec, v);
      M::pack(v, bfr[kk]);
    }
    const float bv = buf_load1<T>(bres, orow ? (uint32_t)o * E : kOob);
    const uint32_t rowoff = (uint32_t)o * (uint32_t)HW;
    if constexpr (!kPair) {
      // fp32: pixels px .. px+3 of row o per block
#pragma unroll
      for (int blk = 0; blk < kGkBlocks; ++blk) {
        f32x4 acc = {bv, bv, bv, bv};
#pragma unroll
        for (int kk = 0; kk < NK; ++kk) acc = M::mac(afr[blk][kk], bfr[kk], acc);
        const int px = p0 + 16 * blk + 4 * quad;
        if (vec) {
          const uint32_t off = (orow && px < HW) ? (rowoff + (uint32_t)px) * E : kOob;
          __builtin_amdgcn_raw_buffer_store_b128(
              (u32x4){__float_as_uint(acc[0]), __float_as_uint(acc[1]), __float_as_uint(acc[2]),
                      __float_as_uint(acc[3])},
              ores, off, 0, 0);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            buf_store1<T>(ores, (orow && px + r < HW) ? (rowoff + (uint32_t)(px + r)) * E : kOob,
                          acc[r]);
        }
      }
    } else {
      // 2-byte types: pixels px .. px+7 of row o per block pair, px = p0 + 32j + 8*quad
#pragma unroll
      for (int j = 0; j < kGkBlocks / 2; ++j) {
        f32x4 acc[2];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          acc[s] = f32x4{bv, bv, bv, bv};
#pragma unroll
          for (int kk = 0; kk < NK; ++kk) acc[s] = M::mac(afr[2 * j + s][kk], bfr[kk], acc[s]);
        }
        const int px = p0 + 32 * j + 8 * quad;
        if (vec) {
          typedef T T8 __attribute__((ext_vector_type(8)));
          const T8 t = {from_f<T>(acc[0][0]), from_f<T>(acc[0][1]), from_f<T>(acc[0][2]),
                        from_f<T>(acc[0][3]), from_f<T>(acc[1][0]), from_f<T>(acc[1][1]),
                        from_f<T>(acc[1][2]), from_f<T>(acc[1][3])};
          *reinterpret_cast<u32x4*>(wtp + col16 * TROW + (px - p0) * 2) = __builtin_bit_cast(u32x4, t);
        } else {
#pragma unroll
          for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int pr = px + 4 * s + r;
              buf_store1<T>(ores, (orow && pr < HW) ? (rowoff + (uint32_t)pr) * E : kOob, acc[s][r]);
            }
        }
      }
      if (vec) {
        // the compiler must not move the tile reads above the writes
        asm volatile("" ::: "memory");
#pragma unroll
        for (int r0 = 0; r0 < 16; r0 += RPI) {
          const int row = r0 + lane / LPR;
          const int cp = (lane % LPR) * (16 / (int)E);  // pixel within the wave's 64
          const u32x4 v = *reinterpret_cast<const u32x4*>(wtp + row * TROW + cp * (int)E);
          const int o2 = ob * 16 + row, px = p0 + cp;
          const uint32_t off = (o2 < O && px < HW) ? ((uint32_t)o2 * (uint32_t)HW + (uint32_t)px) * E : kOob;
          // whole 128-byte lines: a non-temporal store (6% faster at K=5 128x128 bf16)
          __builtin_amdgcn_raw_buffer_store_b128(v, ores, off, 0, kNtStore);
        }
        asm volatile("" ::: "memory");
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Backward of the generator convolution, weight and bias:
//
//   dW[o][i] = sum_{n,p} dK[n][o][p] * y[n][i][p],   db[o] = sum_{n,p} dK[n][o][p]
//
// (the Conv2d weight / bias gradients of `self.generator` on the reference's
// materialized path, triton_impl.py:340-347, computed there by cuDNN's
// backward-filter convolution).  dK is 3*K*K times the size of y and is read
// exactly once, so the kernel is built around that stream.  MFMA GEMM with
// M = 16 rows o, N = 16 channels i and K = 32 pixels: both operands are rows
// of the [o][p] / [i][p] planes, so a lane's fragment is 8 consecutive pixels
// of one row.  fp32 runs as three bf16 products against the bf16 hi / lo
// planes of y (split once per call); db is summed from the same dK values on
// the VALU (fp32 accumulation).
//
// gk_bwd_w_lds_kernel (16-byte aligned planes, H*W % 8 == 0): a workgroup
// owns 64 rows (16 per wave) and a range of pixel steps.  Per step the dK
// tile (64 rows x 256 bytes) and the y tile (all channels) are copied global
// -> LDS by 16-byte buffer loads that write LDS directly, four rows x 256
// contiguous bytes per copy (measured 6.8 TB/s for this pattern against 5.2
// for the 16 rows x 64 bytes a direct fragment load touches), one step ahead
// into a second buffer; chunk c of row r sits at position c ^ (r & mask) so
// that fragment reads of 16 rows hit distinct banks.  The four waves share
// the y tile and own disjoint rows: no cross-wave reduction.
// gk_bwd_w_kernel (any shape): fragments loaded element-wise straight into
// registers, 4 waves taking 32-pixel steps in turn, summed through LDS in
// wave order.
// Workgroups of one row tile write fp32 partials over disjoint pixel ranges
// that a second kernel sums in split order: deterministic, no atomics.
// ---------------------------------------------------------------------------

constexpr int kGwWaves = 4;
constexpr int kGwStep = 32;       // pixels per MFMA step
constexpr int kGwSlots = 512;     // workgroups the splits aim for (two per CU)

struct GwGeom {
  int N, C, HW, O;
  int sp;               // pixels per step
  int spi;              // steps per image, ceil(HW / sp)
  int steps;            // N * spi
  int rows;             // rows per workgroup
  int row_tiles;        // ceil(O / rows)
  int splits;
  int steps_per_split;
};

// LDS-staged tiling per dtype and channel blocks.
template <typename T, int CB>
struct GwLds {
  static constexpr int E = (int)sizeof(T);
  static constexpr int P = Mma<T>::P;
  static constexpr int SP = (CB <= 4 ? 64 : 32) * (4 / E);     // pixels per step (LDS <= 64 KB)
  static constexpr int KC = SP / 32;                          // MFMA k-chunks per step
  static constexpr int CPX = 16 / E;                          // pixels per 16-byte chunk of dK
  static constexpr int ACH = SP / CPX;                        // chunks per dK tile row
  static constexpr int YC = SP / 8;                           // chunks per y tile row (2-byte)
  static constexpr int YROWS = P * CB * 16;
  static constexpr int NA = ACH;                              // 1 KB copies of the 64-row dK tile
  static constexpr int NY = YROWS * YC / 64;                  // 1 KB copies of the y tile
  static constexpr int ABYTES = 64 * ACH * 16;
  static constexpr int BUF = ABYTES + YROWS * YC * 16;        // bytes per staging buffer
  static_assert(NA % kGwWaves == 0 && NY % kGwWaves == 0, "copies split evenly over the waves");
};

// 8 consecutive elements (pixels) of a plane row as raw MFMA operand dwords,
// element-wise with every pixel masked on its own (any H*W).  `off` is the
// element offset of the first pixel, `ok` whether the row exists, `nv` the
// number of valid pixels from the first.
template <typename T>
__device__ __forceinline__ void gw_load_row8(BufRes r, uint32_t off, bool ok, int nv,
                                             u32x4 (&d)[sizeof(T) == 4 ? 2 : 1]) {
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      d[e >> 2][e & 3] = __builtin_amdgcn_raw_buffer_load_b32(r, (ok && e < nv) ? (off + e) * 4u : kOob, 0, 0);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t lo = __builtin_amdgcn_raw_buffer_load_b16(r, (ok && 2 * e < nv) ? (off + 2 * e) * 2u : kOob, 0, 0);
      const uint32_t hi =
          __builtin_amdgcn_raw_buffer_load_b16(r, (ok && 2 * e + 1 < nv) ? (off + 2 * e + 1) * 2u : kOob, 0, 0);
      d[0][e] = (lo & 0xffffu) | (hi << 16);
    }
  }
}

// yb: y itself (2-byte types) or its bf16 hi / lo planes [N][2][C][HW] (fp32).
template <typename T, int RB, int CB>
__global__ __launch_bounds__(64 * kGwWaves) void gk_bwd_w_kernel(const T* __restrict__ gk,
                                                                const uint16_t* __restrict__ yb,
                                                                float* __restrict__ pw,
                                                                float* __restrict__ pb,
                                                                T* __restrict__ dw, T* __restrict__ db,
                                                                GwGeom g) {
  typedef Mma<T> M;
  typedef typename M::V V;
  constexpr int P = M::P;
  constexpr int AD = sizeof(T) == 4 ? 2 : 1;  // 16-byte dwords of a lane's 8 dK values
  constexpr uint32_t E = sizeof(T);
  constexpr int RS = CB * 16 + 1;
  constexpr int KC = 1;  // 32-pixel steps per iteration of a wave
  __shared__ float red[RB * 16 * RS];
  __shared__ float redb[RB * 16];

  const int rt = blockIdx.x % g.row_tiles;
  const int split = blockIdx.x / g.row_tiles;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int col16 = lane & 15, quad = lane >> 4;
  const int C = g.C, HW = g.HW, O = g.O;
  const int o0 = rt * 16 * RB;
  const int s_beg = split * g.steps_per_split;
  const int s_end = s_beg + g.steps_per_split < g.steps ? s_beg + g.steps_per_split : g.steps;

  f32x4 acc[RB][CB];
  float accb[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    accb[rb] = 0.f;
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) acc[rb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // this lane's rows o and channels i (element offsets of their rows)
  uint32_t arow[RB], brow[CB][P];
  bool aok[RB], bok[CB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int o = o0 + 16 * rb + col16;
    aok[rb] = o < O;
    arow[rb] = (uint32_t)o * (uint32_t)HW;
  }
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    const int i = 16 * cb + col16;
    bok[cb] = i < C;
#pragma unroll
    for (int pp = 0; pp < P; ++pp) brow[cb][pp] = (uint32_t)(pp * C + i) * (uint32_t)HW;
  }

  for (int u0 = s_beg + wave * KC; u0 < s_end; u0 += kGwWaves * KC) {
    u32x4 ac[KC][RB][AD], bc[KC][CB][P];
#pragma unroll
    for (int k = 0; k < KC; ++k) {
      const int u = u0 + k;
      const int n = u / g.spi;
      const int px = (u - n * g.spi) * kGwStep + 8 * quad;
      const int nv = u < s_end ? HW - px : 0;  // steps past the split read zero
      const BufRes ar = make_buf(gk + (int64_t)n * O * HW, (uint32_t)O * (uint32_t)HW * E);
      const BufRes br = make_buf(yb + (int64_t)n * P * C * HW, (uint32_t)(P * C) * (uint32_t)HW * 2u);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) gw_load_row8<T>(ar, arow[rb] + (uint32_t)px, aok[rb], nv, ac[k][rb]);
#pragma unroll
      for (int cb = 0; cb < CB; ++cb)
#pragma unroll
        for (int pp = 0; pp < P; ++pp) {
          u32x4 t[1];
          gw_load_row8<uint16_t>(br, brow[cb][pp] + (uint32_t)px, bok[cb], nv, t);
          bc[k][cb][pp] = t[0];
        }
    }
#pragma unroll
    for (int k = 0; k < KC; ++k) {
      V bf[CB][P];
#pragma unroll
      for (int cb = 0; cb < CB; ++cb)
#pragma unroll
        for (int pp = 0; pp < P; ++pp) bf[cb][pp] = __builtin_bit_cast(V, bc[k][cb][pp]);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        V af[P];
        float sum = 0.f;
        if constexpr (E == 4) {
          float v[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = __uint_as_float(ac[k][rb][e >> 2][e & 3]);
#pragma unroll
          for (int e = 0; e < 8; ++e) sum += v[e];
          M::pack(v, af);
        } else {
          typedef T T8 __attribute__((ext_vector_type(8)));
          const T8 t = __builtin_bit_cast(T8, ac[k][rb][0]);
#pragma unroll
          for (int e = 0; e < 8; ++e) sum += to_f(t[e]);
          af[0] = __builtin_bit_cast(V, ac[k][rb][0]);
        }
        accb[rb] += sum;
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) acc[rb][cb] = M::mac(af, bf[cb], acc[rb][cb]);
      }
    }
  }

  // db: the four lanes of a row (quads) hold partial sums of its pixels
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    accb[rb] += __shfl_xor(accb[rb], 16);
    accb[rb] += __shfl_xor(accb[rb], 32);
  }
  // fixed-order sum over the waves: D row 4*quad + r of block rb is row
  // o0 + 16*rb + 4*quad + r, column col16 of block cb is channel 16*cb + col16
  for (int w = 0; w < kGwWaves; ++w) {
    if (wave == w) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float* dst = red + (16 * rb + 4 * quad + r) * RS + 16 * cb + col16;
            *dst = (w == 0 ? 0.f : *dst) + acc[rb][cb][r];
          }
        if (quad == 0) {
          float* dst = redb + 16 * rb + col16;
          *dst = (w == 0 ? 0.f : *dst) + accb[rb];
        }
      }
    }
    __syncthreads();
  }
  const bool direct = g.splits == 1;
  for (int idx = tid; idx < RB * 16 * C; idx += 64 * kGwWaves) {
    const int row = idx / C, i = idx - row * C;
    const int o = o0 + row;
    if (o >= O) break;
    const float v = red[row * RS + i];
    if (direct)
      dw[(int64_t)o * C + i] = from_f<T>(v);
    else
      pw[((int64_t)split * O + o) * C + i] = v;
  }
  for (int row = tid; row < RB * 16; row += 64 * kGwWaves) {
    const int o = o0 + row;
    if (o >= O) break;
    if (direct)
      db[o] = from_f<T>(redb[row]);
    else
      pb[(int64_t)split * O + o] = redb[row];
  }
}

template <typename T, int CB>
__global__ __launch_bounds__(64 * kGwWaves) void gk_bwd_w_lds_kernel(const T* __restrict__ gk,
                                                                    const uint16_t* __restrict__ yb,
                                                                    float* __restrict__ pw,
                                                                    float* __restrict__ pb,
                                                                    T* __restrict__ dw,
                                                                    T* __restrict__ db, GwGeom g) {
  typedef GwLds<T, CB> L;
  typedef Mma<T> M;
  typedef typename M::V V;
  constexpr int P = M::P;
  constexpr uint32_t E = sizeof(T);
  constexpr int NAW = L::NA / kGwWaves, NYW = L::NY / kGwWaves;  // copies per wave
  extern __shared__ __attribute__((aligned(16))) uint32_t gsm[];

  const int rt = blockIdx.x % g.row_tiles;
  const int split = blockIdx.x / g.row_tiles;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int col16 = lane & 15, quad = lane >> 4;
  const int C = g.C, HW = g.HW, O = g.O;
  const int o0 = rt * 64;
  const int s_beg = split * g.steps_per_split;
  const int s_end = s_beg + g.steps_per_split < g.steps ? s_beg + g.steps_per_split : g.steps;

  // this lane's chunks of the copies: element offset in the image's planes
  // at pixel 0 and the chunk's first pixel (absent rows / channels: !ok)
  uint32_t aoff[NAW], yoff[NYW];
  int apx[NAW], ypx[NYW];
  bool aok[NAW], yok[NYW];
#pragma unroll
  for (int j = 0; j < NAW; ++j) {
    const int lc = (wave * NAW + j) * 64 + lane;
    const int row = lc / L::ACH, pos = lc % L::ACH;
    const int gc = pos ^ (row & (L::ACH - 1));
    apx[j] = gc * L::CPX;
    aok[j] = o0 + row < O;
    aoff[j] = (uint32_t)(o0 + row) * (uint32_t)HW + (uint32_t)apx[j];
  }
#pragma unroll
  for (int j = 0; j < NYW; ++j) {
    const int lc = (wave * NYW + j) * 64 + lane;
    const int r = lc / L::YC, pos = lc % L::YC;
    const int gc = pos ^ (r & (L::YC - 1));
    const int pp = r / (CB * 16), i = r - pp * (CB * 16);
    ypx[j] = gc * 8;
    yok[j] = i < C;
    yoff[j] = (uint32_t)(pp * C + i) * (uint32_t)HW + (uint32_t)ypx[j];
  }
  auto stage = [&](int u, int buf) {
    const int n = u / g.spi;
    const int px0 = (u - n * g.spi) * L::SP;
    const BufRes ar = make_buf(gk + (int64_t)n * O * HW, (uint32_t)O * (uint32_t)HW * E);
    const BufRes yr = make_buf(yb + (int64_t)n * P * C * HW, (uint32_t)(P * C) * (uint32_t)HW * 2u);
    char* dst = reinterpret_cast<char*>(gsm) + buf * L::BUF;
#pragma unroll
    for (int j = 0; j < NAW; ++j) {
      const uint32_t off = (aok[j] && px0 + apx[j] < HW) ? (aoff[j] + (uint32_t)px0) * E : kOob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          ar, (__attribute__((address_space(3))) void*)(dst + (wave * NAW + j) * 1024), 16, off, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < NYW; ++j) {
      const uint32_t off = (yok[j] && px0 + ypx[j] < HW) ? (yoff[j] + (uint32_t)px0) * 2u : kOob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          yr, (__attribute__((address_space(3))) void*)(dst + L::ABYTES + (wave * NYW + j) * 1024), 16,
          off, 0, 0, 0);
    }
  };

  f32x4 acc[CB];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) acc[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
  float accb = 0.f;
  const int arow = 16 * wave + col16;  // this lane's A row in the tile
  const int nst = s_end > s_beg ? s_end - s_beg : 0;
  if (nst > 0) stage(s_beg, 0);
  for (int it = 0; it < nst; ++it) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();  // buffer it & 1 is whole; buffer (it + 1) & 1 is no longer read
    if (it + 1 < nst) stage(s_beg + it + 1, (it + 1) & 1);
    const char* bb = reinterpret_cast<const char*>(gsm) + (it & 1) * L::BUF;
    const char* ab = bb + arow * (L::ACH * 16);
#pragma unroll
    for (int kc = 0; kc < L::KC; ++kc) {
      V af[P];
      float sum = 0.f;
      if constexpr (E == 4) {
        const int c0 = 8 * kc + 2 * quad;
        const u32x4 a0 = *reinterpret_cast<const u32x4*>(ab + 16 * (c0 ^ (arow & (L::ACH - 1))));
        const u32x4 a1 = *reinterpret_cast<const u32x4*>(ab + 16 * ((c0 + 1) ^ (arow & (L::ACH - 1))));
        float v[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = __uint_as_float(a0[e]);
          v[4 + e] = __uint_as_float(a1[e]);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) sum += v[e];
        M::pack(v, af);
      } else {
        const u32x4 a = *reinterpret_cast<const u32x4*>(ab + 16 * ((4 * kc + quad) ^ (arow & (L::ACH - 1))));
        typedef T T8 __attribute__((ext_vector_type(8)));
        const T8 t = __builtin_bit_cast(T8, a);
#pragma unroll
        for (int e = 0; e < 8; ++e) sum += to_f(t[e]);
        af[0] = __builtin_bit_cast(V, a);
      }
      accb += sum;
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        V bf[P];
#pragma unroll
        for (int pp = 0; pp < P; ++pp) {
          const int r = pp * CB * 16 + 16 * cb + col16;
          bf[pp] = __builtin_bit_cast(
              V, *reinterpret_cast<const u32x4*>(bb + L::ABYTES + r * (L::YC * 16) +
                                                  16 * ((4 * kc + quad) ^ (r & (L::YC - 1)))));
        }
        acc[cb] = M::mac(af, bf, acc[cb]);
      }
    }
  }

  // db: the four lanes of a row (quads) hold partial sums of its pixels
  accb += __shfl_xor(accb, 16);
  accb += __shfl_xor(accb, 32);
  // D row 4*quad + r of the wave's block is row o0 + 16*wave + 4*quad + r,
  // column col16 of block cb is channel 16*cb + col16
  const bool direct = g.splits == 1;
  const int ob = o0 + 16 * wave;
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    const int i = 16 * cb + col16;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int o = ob + 4 * quad + r;
      if (o < O && i < C) {
        if (direct)
          dw[(int64_t)o * C + i] = from_f<T>(acc[cb][r]);
        else
          pw[((int64_t)split * O + o) * C + i] = acc[cb][r];
      }
    }
  }
  if (quad == 0 && ob + col16 < O) {
    if (direct)
      db[ob + col16] = from_f<T>(accb);
    else
      pb[(int64_t)split * O + ob + col16] = accb;
  }
}

// Sum of the split partials in split order (also the zero gradients of an
// empty batch: splits = 0).
template <typename T>
__global__ __launch_bounds__(256) void gk_bwd_w_reduce_kernel(const float* __restrict__ pw,
                                                              const float* __restrict__ pb,
                                                              T* __restrict__ dw, T* __restrict__ db,
                                                              int64_t OC, int O, int splits) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx < OC) {
    float v = 0.f;
    for (int sp = 0; sp < splits; ++sp) v += pw[sp * OC + idx];
    dw[idx] = from_f<T>(v);
  } else if (idx < OC + O) {
    const int64_t j = idx - OC;
    float v = 0.f;
    for (int sp = 0; sp < splits; ++sp) v += pb[sp * O + j];
    db[j] = from_f<T>(v);
  }
}

// ---------------------------------------------------------------------------
// Backward of the generator convolution, input:
//
//   dY[n][i][p] = sum_o W[o][i] * dK[n][o][p]
//
// (the Conv2d input gradient of `self.generator` on the reference's
// materialized path, triton_impl.py:340-347).  MFMA with M = 16 channels i,
// N = 16 pixels, K = 32 rows o.  The A operand is W transposed, packed once
// per call in fragment order (fp32: bf16 hi / lo parts).  The reduction runs
// over the rows of dK, so a B fragment is 8 rows at one pixel: the dK tile
// (32*KCH rows x 128 pixels) is copied global -> LDS by 16-byte LDS-direct
// loads, 4 (2-byte) or 2 (fp32) rows x 256 / 512 contiguous bytes per copy,
// and read transposed, one 2- or 4-byte LDS read per element; chunk c of row
// r sits at position c ^ ((r >> 3) & 3) * (16 pixels / chunk width), so the
// 4 row groups of a fragment read hit disjoint banks.  A workgroup = 4 waves
// x 32 pixels, all channels; splits over o (fp32 partials summed in split
// order by a second kernel) when the pixel tiles alone cannot fill the GPU.
// ---------------------------------------------------------------------------

constexpr int kGyPX = 128;    // pixels per workgroup
constexpr int kGySlots = 512; // workgroups the splits aim for
constexpr int kGyMinStages = 4;

struct GyGeom {
  int N, C, HW, O;
  int tpi;               // pixel tiles per image
  int tiles;             // N * tpi
  int oc;                // 32-row chunks of o, ceil(O / 32)
  int stages;            // ceil(oc / KCH)
  int splits;
  int stages_per_split;
  int dma;               // dK rows start on 16-byte boundaries: LDS-direct chunk copies
};

template <typename T, int MB>
struct GyLds {
  static constexpr int E = (int)sizeof(T);
  static constexpr int P = Mma<T>::P;
  static constexpr int KCH = E == 2 ? 2 : 1;        // 32-row chunks per stage
  static constexpr int ROWS = 32 * KCH;
  static constexpr int CPX = 16 / E;                // pixels per 16-byte chunk
  static constexpr int CPR = kGyPX / CPX;           // chunks per tile row
  static constexpr int ROWB = kGyPX * E;            // bytes per tile row
  static constexpr int SWZ = 16 / CPX;              // chunks per 16 pixels
  static constexpr int DKB = ROWS * ROWB;           // dK tile bytes (16 KB)
  static constexpr int NDK = DKB / 1024;            // 1 KB copies of the dK tile
  static constexpr int NA = KCH * MB * P;           // 1 KB units of the W^T slice
  static constexpr int BUF = DKB + NA * 1024;
  static_assert(NDK % 4 == 0, "dK copies split evenly over the waves");
};

// W [O][C] -> packed A fragments: unit ((oc*MB + cb)*P + pp), lane m + 16q
// holds part pp of W[32oc + 8q + e][16cb + m], e < 8 (zero outside W)
template <typename T>
__global__ __launch_bounds__(256) void gk_pack_wt_kernel(const T* __restrict__ w,
                                                        uint32_t* __restrict__ pk, int O, int C,
                                                        int MB, int64_t total) {
  typedef Mma<T> M;
  constexpr int P = M::P;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;  // (oc, cb, lane)
  if (idx >= total) return;
  const int lane = (int)(idx & 63);
  const int64_t u = idx >> 6;
  const int cb = (int)(u % MB), oc = (int)(u / MB);
  const int m = lane & 15, q = lane >> 4;
  const int i = 16 * cb + m;
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int o = 32 * oc + 8 * q + e;
    v[e] = (o < O && i < C) ? to_f(w[(int64_t)o * C + i]) : 0.f;
  }
  typename M::V f[P];
  M::pack(v, f);
  u32x4* __restrict__ dst = reinterpret_cast<u32x4*>(pk);
#pragma unroll
  for (int pp = 0; pp < P; ++pp) dst[(u * P + pp) * 64 + lane] = __builtin_bit_cast(u32x4, f[pp]);
}

template <typename T, int MB>
__global__ __launch_bounds__(256) void gk_bwd_y_kernel(const T* __restrict__ gk,
                                                      const uint32_t* __restrict__ pk,
                                                      float* __restrict__ part, T* __restrict__ dy,
                                                      GyGeom g) {
  typedef GyLds<T, MB> L;
  typedef Mma<T> M;
  typedef typename M::V V;
  constexpr int P = M::P;
  constexpr uint32_t E = sizeof(T);
  constexpr int NDW = L::NDK / 4;                 // dK copies per wave
  constexpr int NAW = (L::NA + 3) / 4;            // W^T copies per wave (some idle)
  extern __shared__ __attribute__((aligned(16))) uint32_t ysm[];

  const int tile = blockIdx.x % g.tiles;
  const int split = blockIdx.x / g.tiles;
  const int n = tile / g.tpi;
  const int px0 = (tile - n * g.tpi) * kGyPX;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int col16 = lane & 15, quad = lane >> 4;
  const int C = g.C, HW = g.HW, O = g.O;
  const int st_beg = split * g.stages_per_split;
  const int st_end = st_beg + g.stages_per_split < g.stages ? st_beg + g.stages_per_split : g.stages;

  // this lane's chunk of each dK copy: tile row and first pixel
  int drow[NDW], dpx[NDW];
#pragma unroll
  for (int j = 0; j < NDW; ++j) {
    const int lc = (wave * NDW + j) * 64 + lane;
    const int row = lc / L::CPR, pos = lc % L::CPR;
    drow[j] = row;
    dpx[j] = (pos ^ (((row >> 3) & 3) * L::SWZ)) * L::CPX;
  }
  const BufRes dres = make_buf(gk + (int64_t)n * O * HW, (uint32_t)O * (uint32_t)HW * E);
  auto stage = [&](int st, int buf) {
    char* dst = reinterpret_cast<char*>(ysm) + buf * L::BUF;
    const int o0 = st * L::ROWS;
    if (g.dma) {
#pragma unroll
      for (int j = 0; j < NDW; ++j) {
        const int o = o0 + drow[j], px = px0 + dpx[j];
        const uint32_t off = (o < O && px < HW) ? ((uint32_t)o * (uint32_t)HW + (uint32_t)px) * E : kOob;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            dres, (__attribute__((address_space(3))) void*)(dst + (wave * NDW + j) * 1024), 16, off, 0,
            0, 0);
      }
    } else {
      // H*W with rows off 16-byte boundaries: the same chunks element by
      // element through registers (pixels past the row end read zero)
#pragma unroll
      for (int j = 0; j < NDW; ++j) {
        const int o = o0 + drow[j], px = px0 + dpx[j];
        constexpr int CPX = 16 / (int)E;
        uint32_t raw[CPX];
#pragma unroll
        for (int e = 0; e < CPX; ++e) {
          const uint32_t off = (o < O && px + e < HW)
                                   ? ((uint32_t)o * (uint32_t)HW + (uint32_t)(px + e)) * E
                                   : kOob;
          if constexpr (E == 4)
            raw[e] = __builtin_amdgcn_raw_buffer_load_b32(dres, off, 0, 0);
          else
            raw[e] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(dres, off, 0, 0);
        }
        u32x4 q;
        if constexpr (E == 4) {
#pragma unroll
          for (int e = 0; e < 4; ++e) q[e] = raw[e];
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) q[e] = raw[2 * e] | (raw[2 * e + 1] << 16);
        }
        *reinterpret_cast<u32x4*>(dst + (wave * NDW + j) * 1024 + lane * 16) = q;
      }
    }
    // the stage's W^T slice: KCH chunks x MB x P units, contiguous in pk
    const int units = (g.oc - st * L::KCH < L::KCH ? g.oc - st * L::KCH : L::KCH) * MB * P;
    const BufRes pres = make_buf(pk + (int64_t)st * L::NA * 256, (uint32_t)units * 1024u);
#pragma unroll
    for (int j = 0; j < NAW; ++j) {
      const int u = wave * NAW + j;
      if (u < L::NA)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            pres, (__attribute__((address_space(3))) void*)(dst + L::DKB + u * 1024), 16,
            (uint32_t)(u * 64 + lane) * 16u, 0, 0, 0);
    }
  };

  f32x4 acc[2][MB];
#pragma unroll
  for (int pb = 0; pb < 2; ++pb)
#pragma unroll
    for (int ib = 0; ib < MB; ++ib) acc[pb][ib] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int nst = st_end > st_beg ? st_end - st_beg : 0;
  if (nst > 0) stage(st_beg, 0);
  for (int it = 0; it < nst; ++it) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();  // buffer it & 1 is whole; buffer (it + 1) & 1 is no longer read
    if (it + 1 < nst) stage(st_beg + it + 1, (it + 1) & 1);
    const char* bb = reinterpret_cast<const char*>(ysm) + (it & 1) * L::BUF;
#pragma unroll
    for (int kc = 0; kc < L::KCH; ++kc) {
      V af[MB][P];
#pragma unroll
      for (int ib = 0; ib < MB; ++ib)
#pragma unroll
        for (int pp = 0; pp < P; ++pp)
          af[ib][pp] = __builtin_bit_cast(
              V, *reinterpret_cast<const u32x4*>(bb + L::DKB + (((kc * MB + ib) * P + pp) * 64 + lane) * 16));
#pragma unroll
      for (int pb = 0; pb < 2; ++pb) {
        const int pl = 32 * wave + 16 * pb + col16;  // pixel within the tile
        const int c = pl / L::CPX, within = (pl % L::CPX) * (int)E;
        V bf[P];
        if constexpr (E == 4) {
          float v[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int row = 32 * kc + 8 * quad + e;
            v[e] = *reinterpret_cast<const float*>(bb + row * L::ROWB +
                                                   16 * (c ^ (((row >> 3) & 3) * L::SWZ)) + within);
          }
          M::pack(v, bf);
        } else {
          // two transposing LDS reads (ds_read_b64_tr_b16): lane 16q + 4a + b
          // receives element b of the 8-byte reads of lanes 16q + a + 4e,
          // e = 0..3, so lane 16q + a + 4e reads pixels 4a .. 4a+3 of the
          // block in row 32kc + 8q + 4h + e, and the fragment's rows 8q + 4h
          // .. +3 arrive at every pixel lane (h = 0, 1: the two halves)
          typedef short s16x4 __attribute__((ext_vector_type(4)));
          const int sa = lane & 3, se = (lane >> 2) & 3;
          const int spl = 32 * wave + 16 * pb + 4 * sa;
          const int sc = spl / L::CPX, sw = (spl % L::CPX) * (int)E;
          u32x4 wd;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int row = 32 * kc + 8 * quad + 4 * h + se;
            const char* a = bb + row * L::ROWB + 16 * (sc ^ (((row >> 3) & 3) * L::SWZ)) + sw;
            const s16x4 t = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) s16x4*)(a));
            typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
            const u32x2 d2 = __builtin_bit_cast(u32x2, t);
            wd[2 * h] = d2[0];
            wd[2 * h + 1] = d2[1];
          }
          bf[0] = __builtin_bit_cast(V, wd);
        }
#pragma unroll
        for (int ib = 0; ib < MB; ++ib) acc[pb][ib] = M::mac(af[ib], bf, acc[pb][ib]);
      }
    }
  }

  // D row 4*quad + r of block ib is channel 16*ib + 4*quad + r, column col16
  // of block pb is pixel px0 + 32*wave + 16*pb + col16
  const bool direct = g.splits == 1;
#pragma unroll
  for (int pb = 0; pb < 2; ++pb) {
    const int px = px0 + 32 * wave + 16 * pb + col16;
    if (px >= HW) continue;
#pragma unroll
    for (int ib = 0; ib < MB; ++ib)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * ib + 4 * quad + r;
        if (i >= C) continue;
        const int64_t el = ((int64_t)n * C + i) * HW + px;
        if (direct)
          dy[el] = from_f<T>(acc[pb][ib][r]);
        else
          part[(int64_t)split * g.N * C * HW + el] = acc[pb][ib][r];
      }
  }
}

// dY = sum of the o-split partials in split order
template <typename T>
__global__ __launch_bounds__(256) void gk_bwd_y_reduce_kernel(const float* __restrict__ part,
                                                             T* __restrict__ dy, int64_t total,
                                                             int splits) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= total) return;
  float v = 0.f;
  for (int sp = 0; sp < splits; ++sp) v += part[sp * total + idx];
  dy[idx] = from_f<T>(v);
}

namespace {

template <typename F>
int gk_with_type(int dt, F&& f) {
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

}  // namespace

namespace {

// Row blocks per wave of the element-wise kernel by channel blocks
// (accumulators RB x CB <= 16 tiles)
int gw_cb(int64_t c) { return c <= 16 ? 1 : c <= 32 ? 2 : c <= 64 ? 4 : 8; }
int gw_rb(int cb) { return cb == 8 ? 2 : 4; }

// Splits of the pixel steps: as many as fill kGwSlots workgroups over the
// row tiles, with at least `min_steps` steps per workgroup.
void gw_geom(GwGeom& g, int64_t n, int64_t c, int64_t hw, int64_t o, int sp, int rows, int min_steps) {
  g.N = (int)n;
  g.C = (int)c;
  g.HW = (int)hw;
  g.O = (int)o;
  g.sp = sp;
  g.spi = (int)((hw + sp - 1) / sp);
  g.steps = (int)(n * g.spi);
  g.rows = rows;
  g.row_tiles = (int)((o + rows - 1) / rows);
  int64_t splits = kGwSlots / g.row_tiles;
  const int64_t most = ((int64_t)g.steps + min_steps - 1) / min_steps;
  if (splits > most) splits = most;
  if (splits < 1) splits = 1;
  g.steps_per_split = (int)((g.steps + splits - 1) / splits);
  g.splits = g.steps == 0 ? 0 : (g.steps + g.steps_per_split - 1) / g.steps_per_split;
}

// LDS-staged kernel: 64 rows per workgroup, at least 8 steps per workgroup
void gw_geom_lds(GwGeom& g, int64_t n, int64_t c, int64_t hw, int64_t o, int sp) {
  gw_geom(g, n, c, hw, o, sp, 64, 8);
}
// element-wise kernel: 32-pixel steps, at least 8 per wave
void gw_geom_elem(GwGeom& g, int64_t n, int64_t c, int64_t hw, int64_t o) {
  gw_geom(g, n, c, hw, o, kGwStep, 16 * gw_rb(gw_cb(c)), 8 * kGwWaves);
}

int64_t gw_align(int64_t v) { return (v + 255) / 256 * 256; }

int64_t gw_partial_bytes(const GwGeom& g) {
  if (g.splits <= 1) return 0;
  return (int64_t)g.splits * ((int64_t)g.O * g.C + g.O) * (int64_t)sizeof(float);
}


// Channel blocks of the dY kernel and its o splits: as many as fill
// kGySlots workgroups over the pixel tiles, at least kGyMinStages stages each.
int gy_mb(int64_t c) { return c <= 16 ? 1 : c <= 32 ? 2 : c <= 64 ? 4 : 8; }

void gy_geom(GyGeom& g, int64_t n, int64_t c, int64_t hw, int64_t o, int kch) {
  g.N = (int)n;
  g.C = (int)c;
  g.HW = (int)hw;
  g.O = (int)o;
  g.tpi = (int)((hw + kGyPX - 1) / kGyPX);
  g.tiles = (int)(n * g.tpi);
  g.oc = (int)((o + 31) / 32);
  g.stages = (g.oc + kch - 1) / kch;
  int64_t splits = g.tiles > 0 ? kGySlots / g.tiles : 1;
  const int64_t most = (g.stages + kGyMinStages - 1) / kGyMinStages;
  if (splits > most) splits = most;
  if (splits < 1) splits = 1;
  g.stages_per_split = (g.stages + (int)splits - 1) / (int)splits;
  g.splits = (g.stages + g.stages_per_split - 1) / g.stages_per_split;
}

int64_t gy_pack_bytes(const GyGeom& g, int parts) { return (int64_t)g.oc * gy_mb(g.C) * parts * 1024; }
int64_t gy_part_bytes(const GyGeom& g) {
  return g.splits > 1 ? (int64_t)g.splits * g.N * g.C * g.HW * (int64_t)sizeof(float) : 0;
}

}  // namespace
}  // namespace ddpm

using namespace ddpm;

// 1 when ddpm_gen_kernels and ddpm_gen_kernels_bwd_w take this shape and
// dtype: their 32-bit buffer offsets cover one image's planes (the 3CK^2
// generated planes, and for fp32 the two 2-byte planes of y) and their grids
// stay below 2^31 workgroups.  Host-only; the same bounds the entry points
// apply before launching.
extern "C" int ddpm_gen_kernels_supported(int64_t n, int64_t c, int64_t h, int64_t w,
                                          int kernel_size, int dtype) {
  if (dtype < kF32 || dtype > kF16) return 0;
  if (n < 0 || c < 1 || h < 0 || w < 0 || c > kGkMaxC) return 0;
  if (kernel_size < 1 || kernel_size % 2 == 0) return 0;
  const int64_t esz = dtype == kF32 ? 4 : 2;
  const int64_t hw = h * w, o = 3 * c * kernel_size * kernel_size;
  if (o * hw * esz > 0x7fffffffLL || c * hw * esz > 0x7fffffffLL || o * c * esz > 0x7fffffffLL)
    return 0;
  if (2 * c * hw * 2 > 0x7fffffffLL || o * c > 0x7fffffffLL) return 0;
  if (n * ((hw + kGwStep - 1) / kGwStep) > 0x7fffffffLL) return 0;
  if (n * ((hw + kGkTP - 1) / kGkTP) * ((o + 15) / 16) > 0x7fffffffLL) return 0;
  return 1;
}

extern "C" int ddpm_gen_kernels(const void* y, const void* weight, const void* bias, void* kernels,
                                int64_t n, int64_t c, int64_t h, int64_t w, int kernel_size,
                                int dtype, hipStream_t stream) {
  if (dtype < kF32 || dtype > kF16) return kBadArgument;
  if (n < 0 || c < 0 || h < 0 || w < 0) return kBadArgument;
  if (kernel_size < 1 || kernel_size % 2 == 0) return kBadArgument;
  if (c > kGkMaxC) return kUnsupported;
  if (n == 0 || c == 0 || h == 0 || w == 0) return kOk;
  if (!y || !weight || !bias || !kernels) return kBadArgument;
  const int64_t esz = dtype == kF32 ? 4 : 2;
  const int64_t hw = h * w, o = 3 * c * kernel_size * kernel_size;
  // 32-bit buffer offsets inside one image's input and output planes
  if (o * hw * esz > 0x7fffffffLL || c * hw * esz > 0x7fffffffLL || o * c * esz > 0x7fffffffLL)
    return kUnsupported;
  GkGeom g;
  g.N = (int)n;
  g.C = (int)c;
  g.HW = (int)hw;
  g.O = (int)o;
  g.tiles = (int)((hw + kGkTP - 1) / kGkTP);
  const int64_t nob = (o + 15) / 16;
  int64_t want = (kGkTargetGroups + n * g.tiles - 1) / (n * g.tiles);
  if (want > nob) want = nob;
  if (want < 1) want = 1;
  g.obpc = (int)((nob + want - 1) / want);
  g.ochunks = (int)((nob + g.obpc - 1) / g.obpc);
  g.vec = hw % (esz == 4 ? 4 : 8) == 0 && (uintptr_t)kernels % 16 == 0;
  g.wvec = c % 8 == 0 && (uintptr_t)weight % 16 == 0;
  const int64_t groups = n * g.tiles * g.ochunks;
  if (groups > 0x7fffffffLL) return kUnsupported;
  const int nk = (int)((c + 31) / 32);
  return gk_with_type(dtype, [&](auto tag) {
    using T = decltype(tag);
    auto launch = [&](auto kern) {
      hipLaunchKernelGGL(kern, dim3((unsigned)groups), dim3(kGkThreads), 0, stream, (const T*)y,
                         (const T*)weight, (const T*)bias, (T*)kernels, g);
      return (int)hipGetLastError();
    };
    switch (nk) {
      case 1:
        return launch(gen_kernels_kernel<T, 1>);
      case 2:
        return launch(gen_kernels_kernel<T, 2>);
      case 3:
        return launch(gen_kernels_kernel<T, 3>);
      default:
        return launch(gen_kernels_kernel<T, 4>);
    }
  });
}


extern "C" int64_t ddpm_gen_kernels_bwd_w_workspace_bytes(int64_t n, int64_t c, int64_t h, int64_t w,
                                                          int kernel_size) {
  if (n <= 0 || c <= 0 || h <= 0 || w <= 0 || kernel_size < 1 || kernel_size % 2 == 0) return 0;
  if (c > kGkMaxC || n * ((h * w + kGwStep - 1) / kGwStep) > 0x7fffffffLL) return 0;
  const int64_t hw = h * w, o = 3 * c * kernel_size * kernel_size;
  // the query takes no dtype or alignment: it covers the largest partials of
  // either kernel and fp32, whose y planes come on top
  GwGeom g;
  int64_t most = 0;
  const int sp1 = gw_cb(c) <= 4 ? 64 : 32;  // fp32 steps; 2-byte steps are twice as long
  for (int sp : {sp1, 2 * sp1}) {
    gw_geom_lds(g, n, c, hw, o, sp);
    most = std::max(most, gw_partial_bytes(g));
  }
  gw_geom_elem(g, n, c, hw, o);
  most = std::max(most, gw_partial_bytes(g));
  return gw_align(most) + n * 2 * c * hw * 2;
}

extern "C" int ddpm_gen_kernels_bwd_w(const void* y, const void* grad_kernels, void* grad_weight,
                                      void* grad_bias, void* workspace, int64_t workspace_bytes,
                                      int64_t n, int64_t c, int64_t h, int64_t w, int kernel_size,
                                      int dtype, hipStream_t stream) {
  if (dtype < kF32 || dtype > kF16) return kBadArgument;
  if (n < 0 || c < 0 || h < 0 || w < 0) return kBadArgument;
  if (kernel_size < 1 || kernel_size % 2 == 0) return kBadArgument;
  if (c > kGkMaxC) return kUnsupported;
  if (c == 0) return kOk;
  if (!grad_weight || !grad_bias) return kBadArgument;
  const int64_t esz = dtype == kF32 ? 4 : 2;
  const int64_t hw = h * w, o = 3 * c * kernel_size * kernel_size;
  if (n > 0 && hw > 0 && (!y || !grad_kernels)) return kBadArgument;
  // 32-bit buffer offsets inside one image's planes (fp32 y: two 2-byte planes)
  if (o * hw * esz > 0x7fffffffLL || 2 * c * hw * 2 > 0x7fffffffLL) return kUnsupported;
  if (n * ((hw + kGwStep - 1) / kGwStep) > 0x7fffffffLL || o * c > 0x7fffffffLL) return kUnsupported;
  const int cb = gw_cb(c);
  // LDS-staged kernel: 16-byte chunks of every plane row (the fp32 y planes
  // sit 256-byte aligned in the workspace)
  const bool lds = hw % 8 == 0 && (uintptr_t)grad_kernels % 16 == 0 &&
                   (dtype == kF32 ? (uintptr_t)workspace % 16 == 0 : (uintptr_t)y % 16 == 0);
  GwGeom g;
  if (lds)
    gw_geom_lds(g, n, c, hw, o, (cb <= 4 ? 64 : 32) * (int)(4 / esz));
  else
    gw_geom_elem(g, n, c, hw, o);
  const int64_t pbytes = gw_partial_bytes(g);
  const int64_t need = dtype == kF32 && g.steps > 0 ? gw_align(pbytes) + n * 2 * c * hw * 2 : pbytes;
  if (need > 0 && (!workspace || workspace_bytes < need)) return kWorkspaceTooSmall;
  float* pw = (float*)workspace;
  float* pb = pw ? pw + (int64_t)g.splits * o * c : nullptr;
  const uint16_t* yb = (const uint16_t*)y;
  if (dtype == kF32 && g.steps > 0) {
    uint16_t* ys = (uint16_t*)((char*)workspace + gw_align(pbytes));
    const int e = launch_ysplit((const float*)y, ys, c * hw, n * c * hw, stream);
    if (e != 0) return e;
    yb = ys;
  }
  return gk_with_type(dtype, [&](auto tag) {
    using T = decltype(tag);
    auto launch = [&](auto kern, size_t shm) {
      if (g.splits > 0) {
        const int ae = allow_dynamic_lds(reinterpret_cast<const void*>(kern), shm);
        if (ae != 0) return ae;
        hipLaunchKernelGGL(kern, dim3((unsigned)(g.row_tiles * g.splits)), dim3(64 * kGwWaves), shm,
                           stream, (const T*)grad_kernels, yb, pw, pb, (T*)grad_weight,
                           (T*)grad_bias, g);
        const int e = (int)hipGetLastError();
        if (e != 0 || g.splits == 1) return e;
      }
      const int64_t total = o * c + o;
      hipLaunchKernelGGL((gk_bwd_w_reduce_kernel<T>), dim3((unsigned)((total + 255) / 256)),
                         dim3(256), 0, stream, (const float*)pw, (const float*)pb, (T*)grad_weight,
                         (T*)grad_bias, o * c, (int)o, g.splits);
      return (int)hipGetLastError();
    };
    auto lds_launch = [&](auto cbc) {
      constexpr int CB = decltype(cbc)::value;
      return launch(gk_bwd_w_lds_kernel<T, CB>, (size_t)2 * GwLds<T, CB>::BUF);
    };
    if (lds) {
      switch (cb) {
        case 1:
          return lds_launch(std::integral_constant<int, 1>());
        case 2:
          return lds_launch(std::integral_constant<int, 2>());
        case 4:
          return lds_launch(std::integral_constant<int, 4>());
        default:
          return lds_launch(std::integral_constant<int, 8>());
      }
    }
    switch (cb) {
      case 1:
        return launch(gk_bwd_w_kernel<T, 4, 1>, 0);
      case 2:
        return launch(gk_bwd_w_kernel<T, 4, 2>, 0);
      case 4:
        return launch(gk_bwd_w_kernel<T, 4, 4>, 0);
      default:
        return launch(gk_bwd_w_kernel<T, 2, 8>, 0);
    }
  });
}


extern "C" int64_t ddpm_gen_kernels_bwd_y_workspace_bytes(int64_t n, int64_t c, int64_t h, int64_t w,
                                                          int kernel_size) {
  if (n <= 0 || c <= 0 || h <= 0 || w <= 0 || kernel_size < 1 || kernel_size % 2 == 0) return 0;
  if (c > kGkMaxC || n * ((h * w + kGyPX - 1) / kGyPX) > 0x7fffffffLL) return 0;
  const int64_t o = 3 * c * kernel_size * kernel_size;
  // the query takes no dtype: the largest of the 2-byte and fp32 layouts
  int64_t most = 0;
  for (int fp32 = 0; fp32 < 2; ++fp32) {
    GyGeom g;
    gy_geom(g, n, c, h * w, o, fp32 ? 1 : 2);
    most = std::max(most, gw_align(gy_pack_bytes(g, fp32 ? 2 : 1)) + gy_part_bytes(g));
  }
  return most;
}

extern "C" int ddpm_gen_kernels_bwd_y(const void* weight, const void* grad_kernels, void* grad_y,
                                      void* workspace, int64_t workspace_bytes, int64_t n, int64_t c,
                                      int64_t h, int64_t w, int kernel_size, int dtype,
                                      hipStream_t stream) {
  if (dtype < kF32 || dtype > kF16) return kBadArgument;
  if (n < 0 || c < 0 || h < 0 || w < 0) return kBadArgument;
  if (kernel_size < 1 || kernel_size % 2 == 0) return kBadArgument;
  if (c > kGkMaxC) return kUnsupported;
  if (n == 0 || c == 0 || h == 0 || w == 0) return kOk;
  if (!weight || !grad_kernels || !grad_y) return kBadArgument;
  const int64_t esz = dtype == kF32 ? 4 : 2;
  const int64_t hw = h * w, o = 3 * c * kernel_size * kernel_size;
  // 32-bit offsets inside one image's planes
  if (o * hw * esz > 0x7fffffffLL || n * ((hw + kGyPX - 1) / kGyPX) > 0x7fffffffLL) return kUnsupported;
  GyGeom g;
  gy_geom(g, n, c, hw, o, esz == 2 ? 2 : 1);
  // whole 16-byte chunks of every dK row: LDS-direct copies
  g.dma = (hw * esz) % 16 == 0 && (uintptr_t)grad_kernels % 16 == 0;
  const int parts = esz == 4 ? 2 : 1;
  const int64_t pkb = gy_pack_bytes(g, parts);
  if (!workspace || (uintptr_t)workspace % 16 != 0 ||
      workspace_bytes < gw_align(pkb) + gy_part_bytes(g))
    return kWorkspaceTooSmall;
  uint32_t* pk = (uint32_t*)workspace;
  float* part = (float*)((char*)workspace + gw_align(pkb));
  const int mb = gy_mb(c);
  return gk_with_type(dtype, [&](auto tag) {
    using T = decltype(tag);
    const int64_t ptotal = (int64_t)g.oc * mb * 64;
    hipLaunchKernelGGL((gk_pack_wt_kernel<T>), dim3((unsigned)((ptotal + 255) / 256)), dim3(256), 0,
                       stream, (const T*)weight, pk, (int)o, (int)c, mb, ptotal);
    int e = (int)hipGetLastError();
    if (e != 0) return e;
    auto launch = [&](auto mbc) {
      constexpr int MB = decltype(mbc)::value;
      const size_t shm = (size_t)2 * GyLds<T, MB>::BUF;
      auto kern = gk_bwd_y_kernel<T, MB>;
      const int ae = allow_dynamic_lds(reinterpret_cast<const void*>(kern), shm);
      if (ae != 0) return ae;
      hipLaunchKernelGGL(kern, dim3((unsigned)(g.tiles * g.splits)), dim3(256), shm, stream,
                         (const T*)grad_kernels, (const uint32_t*)pk, part, (T*)grad_y, g);
      int e2 = (int)hipGetLastError();
      if (e2 != 0 || g.splits == 1) return e2;
      const int64_t total = n * c * hw;
      hipLaunchKernelGGL((gk_bwd_y_reduce_kernel<T>), dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                         stream, (const float*)part, (T*)grad_y, total, g.splits);
      return (int)hipGetLastError();
    };
    switch (mb) {
      case 1:
        return launch(std::integral_constant<int, 1>());
      case 2:
        return launch(std::integral_constant<int, 2>());
      case 4:
        return launch(std::integral_constant<int, 4>());
      default:
        return launch(std::integral_constant<int, 8>());
    }
  });
}
