// Fused kernel generator + dynamic dilated filter + concat, forward.
//
// Counterpart of the reference's _generator_dynamic_cat_fwd
// (_triton_kernels.py:268-420, launched at :873-908), redesigned for CDNA4:
//
//   gen[(b,c,tap), p] = sum_i W[(b,c,tap), i] * y[i, p] + bias[(b,c,tap)]
//   out_b[c, p]       = sum_tap q(gen[(b,c,tap), p]) * x[c, p + off(b,tap)]
//   cat               = [x, out_0, out_1, out_2]
//
// q() rounds the generated tap to the input dtype (bf16/f16), as the
// reference does before consuming it (_triton_kernels.py:332-335).
//
// One workgroup = (image n, 16-channel block, 16 x 16*CB pixel tile), 8
// waves; wave w owns tile rows 2w and 2w+1, i.e. 2*CB 16-pixel blocks (CB = 4:
// eight independent MFMA chains per wave and one weight read per 8 blocks;
// CB = 2 for halos too large for the 64-column tile).  The
// generator is an MFMA GEMM per (branch, tap): M = the 16 channels, N = 16
// pixels, K = the input channels (v_mfma_f32_16x16x32_{bf16,f16}; fp32 runs
// as three bf16 products).  Operands:
//   * y (B): each wave loads its four pixel blocks once and keeps them in
//     registers for all 3*K*K products;
//   * W (A): the 16 x C slice of one (branch, tap) is converted once per
//     workgroup (fp32: split into bf16 hi/lo) into LDS in fragment order,
//     double-buffered one tap ahead, and read by all 8 waves;
//   * x: the halo tile (16+2R) x (32+2R) of the 16 channels sits in LDS as 4
//     planes of 4-channel pixels, so the shifted read of one lane's 4 output
//     channels is one ds_read_b128 (fp32) / ds_read_b64 (2-byte) whose
//     address moves by a uniform offset per tap.
// The generated taps never leave the MFMA result registers.  The identity
// part of the concat is written from the registers that stage the halo tile.
// Every global access is a raw buffer access; lanes outside the image or the
// channel range use an offset past the resource's end (read as zero, write
// dropped) instead of a branch.

#include "gen_common.h"
#include <type_traits>

namespace ddpm {

constexpr int kGfWaves = 8;
constexpr int kGfThreads = 64 * kGfWaves;
constexpr int kGfTH = 2 * kGfWaves;  // tile rows, two per wave
constexpr int kGfMaxLds = 160 * 1024;

struct FwdGeom {
  int N, C, H, W;
  int d0, d1, d2;
  int R;        // halo radius
  int cblocks;  // ceil(C/16)
  int tiles_w, tiles;
  int TW;       // tile columns (16 * CB)
  int LH, LW;   // halo tile rows / columns
  int npix;     // LH * LW
  int plane;    // bytes of one 4-channel plane of the halo tile (256-byte multiple)
};

// Raw element bits through a buffer resource (no conversion).
template <int E>
__device__ __forceinline__ uint32_t gf_load_raw(BufRes r, uint32_t off) {
  if constexpr (E == 4)
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
  else
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}
template <int E>
__device__ __forceinline__ void gf_store_raw(BufRes r, uint32_t off, uint32_t v) {
  if constexpr (E == 4)
    __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, 0);
  else
    __builtin_amdgcn_raw_buffer_store_b16((unsigned short)v, r, off, 0, 0);
}

// CB = 4: 256 registers per lane (one 8-wave workgroup per CU, whose 133 KB
// halo tile fills the LDS anyway); CB = 2: 128 registers, two workgroups per CU.
template <typename T, int KS, int NK, int CB>
__global__ __launch_bounds__(kGfThreads) __attribute__((amdgpu_waves_per_eu(CB == 4 ? 2 : 4))) void gen_fwd_kernel(
    const T* __restrict__ x, const T* __restrict__ y, const T* __restrict__ wt,
    const T* __restrict__ bias, T* __restrict__ out, FwdGeom g) {
  typedef Mma<T> M;
  typedef typename M::V V;
  constexpr int P = M::P;
  constexpr int KK = KS * KS;
  constexpr int NBT = 3 * KK;         // (branch, tap) steps
  constexpr int r = KS / 2;
  constexpr int E = (int)sizeof(T);
  constexpr int XB = 4 * E;           // bytes of one 4-channel pixel entry
  constexpr int AU = NK * P * 64;     // 16-byte units of one weight slice
  typedef uint32_t XQ __attribute__((ext_vector_type(E)));  // one 4-channel entry
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
  const int h0 = ty * kGfTH, w0 = tx * TW;
  const int C = g.C, H = g.H, W = g.W, R = g.R, LW = g.LW;
  const int64_t HW = (int64_t)H * W;
  const uint32_t HWE = (uint32_t)HW * (uint32_t)E;  // bytes of one channel plane
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int col16 = lane & 15, quad = lane >> 4;
  const int c0 = cb * 16;
  const int nch = C - c0 < 16 ? C - c0 : 16;

  // ---- weight slices: thread -> (row m, input channels i, i+1); the slice
  //      of step bt is loaded during step bt-2 and written to LDS in step bt-1.
  //      Wave (kk, q) = (wave/4, wave%4), lane (m, e/2) = (lane%16, lane/16):
  //      the 64 lanes of a wave write 64 different LDS banks.
  const int wm = lane & 15, wi = (wave >> 2) * 32 + 8 * (wave & 3) + 2 * (lane >> 4);
  const bool wlive = (wave >> 2) < NK;
  const BufRes wres = make_buf(wt, (uint32_t)(3 * C * KK * C * E));
  uint32_t wraw[2];
  auto wload = [&](int bt) {
    const int b = bt / KK, t = bt - b * KK;
    const int c = c0 + wm;
    const uint32_t row = (uint32_t)(((b * C + c) * KK + t) * C);
    wraw[0] = gf_load_raw<E>(wres, (c < C && wi < C) ? (row + wi) * E : kOob);
    wraw[1] = gf_load_raw<E>(wres, (c < C && wi + 1 < C) ? (row + wi + 1) * E : kOob);
  };
  auto wput = [&](int buf) {
    if (!wlive) return;
    // unit (kk, part, lane = m + 16*q) holds W[m][kk*32 + 8*q + e], e = 0..7
    uint32_t* __restrict__ dst = reinterpret_cast<uint32_t*>(abuf + buf * AU * 16) +
                                 ((wi >> 5) * P * 64 + wm + 16 * ((wi & 31) >> 3)) * 4 +
                                 ((wi & 7) >> 1);
    if constexpr (E == 4) {
      uint32_t hi, lo;
      split_bf16x2(__uint_as_float(wraw[0]), __uint_as_float(wraw[1]), hi, lo);
      dst[0] = hi;
      dst[64 * 4] = lo;
    } else {
      dst[0] = wraw[0] | (wraw[1] << 16);
    }
  };
  wload(0);

  // ---- halo tile of x (zero outside the image) -> LDS planes; interior
  //      pixels also go to the identity channels of the output.  Two pixels
  //      per thread and batch: 32 loads in flight before any LDS write.
  {
    const BufRes xres = make_buf(x + ((int64_t)n * C + c0) * HW, (uint32_t)nch * HWE);
    const BufRes ores = make_buf(out + ((int64_t)n * 4 * C + c0) * HW, (uint32_t)nch * HWE);
    for (int p0 = tid; p0 < g.npix; p0 += 2 * kGfThreads) {
      uint32_t lo[2], so[2];
      int pix[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        pix[s] = p0 + s * kGfThreads;
        const int i = pix[s] / LW, j = pix[s] - i * LW;
        const int gh = h0 - R + i, gw = w0 - R + j;
        const bool in =
            pix[s] < g.npix && (unsigned)gh < (unsigned)H && (unsigned)gw < (unsigned)W;
        const bool inner = i >= R && i < R + kGfTH && j >= R && j < R + TW;
        lo[s] = in ? (uint32_t)(gh * W + gw) * (uint32_t)E : kOob;
        so[s] = (in && inner) ? lo[s] : kOob;
      }
      uint32_t v[2][16];
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int ch = 0; ch < 16; ++ch) v[s][ch] = gf_load_raw<E>(xres, lo[s] + ch * HWE);
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int ch = 0; ch < 16; ++ch) gf_store_raw<E>(ores, so[s] + ch * HWE, v[s][ch]);
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

  // ---- bias rows of this channel block, [bt][16]
  for (int idx = tid; idx < NBT * 16; idx += kGfThreads) {
    const int m = idx & 15, bt = idx >> 4;
    const int b = bt / KK, t = bt - b * KK;
    bs[idx] = m < nch ? to_f(bias[(int64_t)(b * C + c0 + m) * KK + t]) : 0.f;
  }
  wput(0);
  if (NBT > 1) wload(1);

  // ---- y operand (unshifted pixels) of this wave's blocks; per block the
  //      LDS address of this lane's x entry at zero shift
  V bfr[NBW][NK][P];
  uint32_t pbase[NBW];
  auto pix_off = [&](int blk) {  // byte offset of this lane's pixel in a plane
    const int gh = h0 + 2 * wave + blk / CB, gw = w0 + 16 * (blk % CB) + col16;
    return (gh < H && gw < W) ? (uint32_t)(gh * W + gw) * (uint32_t)E : kOob;
  };
  {
    const BufRes yres = make_buf(y + (int64_t)n * C * HW, (uint32_t)C * HWE);
#pragma unroll
    for (int blk = 0; blk < NBW; ++blk) {
      const int lrow = 2 * wave + blk / CB, lcol = 16 * (blk % CB) + col16;
      const uint32_t po = pix_off(blk);
      pbase[blk] = (uint32_t)(quad * g.plane + ((lrow + R) * LW + lcol + R) * XB);
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
  __syncthreads();

  f32x4 acc[NBW];
#pragma unroll 1
  for (int bt = 0; bt < NBT; ++bt) {
    const int b = bt / KK, t = bt - b * KK;
    if (bt + 1 < NBT) {
      wput((bt + 1) & 1);
      if (bt + 2 < NBT) wload(bt + 2);
    }
    const int ki = t / KS, kj = t - ki * KS;
    const int d = dil_of(b, g.d0, g.d1, g.d2);
    const int shift = ((ki - r) * d * LW + (kj - r) * d) * XB;
    const unsigned char* __restrict__ ab = abuf + (bt & 1) * AU * 16;
    V afr[NK][P];
#pragma unroll
    for (int kk = 0; kk < NK; ++kk)
#pragma unroll
      for (int pp = 0; pp < P; ++pp)
        afr[kk][pp] = __builtin_bit_cast(
            V, *reinterpret_cast<const u32x4*>(ab + ((kk * P + pp) * 64 + lane) * 16));
    const f32x4 binit = *reinterpret_cast<const f32x4*>(bs + bt * 16 + 4 * quad);
    if (t == 0) {
#pragma unroll
      for (int blk = 0; blk < NBW; ++blk) acc[blk] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    // NBW independent accumulation chains
    f32x4 dacc[NBW];
#pragma unroll
    for (int blk = 0; blk < NBW; ++blk) dacc[blk] = binit;
#pragma unroll
    for (int kk = 0; kk < NK; ++kk)
#pragma unroll
      for (int blk = 0; blk < NBW; ++blk) dacc[blk] = M::mac(afr[kk], bfr[blk][kk], dacc[blk]);
#pragma unroll
    for (int blk = 0; blk < NBW; ++blk) {
      const XQ xq = *reinterpret_cast<const XQ*>(xs + pbase[blk] + shift);
      float xv[4];
      if constexpr (E == 4) {
#pragma unroll
        for (int e = 0; e < 4; ++e) xv[e] = __uint_as_float(xq[e]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          xv[e] = to_f(__builtin_bit_cast(T, (unsigned short)(xq[e >> 1] >> (16 * (e & 1)))));
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[blk][e] = fmaf(quant<T>(dacc[blk][e]), xv[e], acc[blk][e]);
    }
    if (t == KK - 1) {
      // ---- branch b: channels c0 + 4*quad + e of output block b+1
      const BufRes bres =
          make_buf(out + ((int64_t)n * 4 * C + (int64_t)(b + 1) * C + c0) * HW, (uint32_t)nch * HWE);
#pragma unroll
      for (int blk = 0; blk < NBW; ++blk) {
        const uint32_t po = pix_off(blk);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          buf_store1<T>(bres, po + (uint32_t)(4 * quad + e) * HWE, acc[blk][e]);
      }
    }
    __syncthreads();
  }
}

namespace {

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

// Forward tiling and LDS bytes for a tile of 16 x 16*cb pixels;
// kUnsupported when the halo tile does not fit.
int fwd_geom(FwdGeom& f, const GenGeom& g, int esz, int cb, size_t& lds) {
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
  f.tiles = f.tiles_w * ((g.H + kGfTH - 1) / kGfTH);
  f.LH = kGfTH + 2 * g.R;
  f.LW = f.TW + 2 * g.R;
  f.npix = f.LH * f.LW;
  // planes start on 256-byte boundaries: the four quads of a wave then read
  // their 4-channel entries with the fewest LDS bank conflicts (measured)
  f.plane = (f.npix * 4 * esz + 255) / 256 * 256;
  const int nk = (g.C + 31) / 32;
  const int parts = esz == 4 ? 2 : 1;
  lds = (size_t)4 * f.plane + (size_t)2 * nk * parts * 64 * 16 + (size_t)3 * g.K * g.K * 16 * 4;
  if (lds > (size_t)kGfMaxLds) return kUnsupported;
  if ((int64_t)f.tiles * g.cblocks * g.N > 0x7fffffffLL) return kUnsupported;
  return kOk;
}

}  // namespace

// Shared with the backward entry points.
int gen_make_geom(GenGeom& g, int64_t n, int64_t c, int64_t h, int64_t w, int k, int d0, int d1,
                  int d2) {
  if (n < 0 || c < 0 || h < 0 || w < 0) return kBadArgument;
  if (k < 1 || (k % 2) == 0 || d0 < 1 || d1 < 1 || d2 < 1) return kBadArgument;
  if (k > 3 || c > 64) return kUnsupported;
  if (h > (1 << 20) || w > (1 << 20) || h * w > ((int64_t)1 << 31)) return kUnsupported;
  if (k == 1) d0 = d1 = d2 = 1;  // a 1x1 tap has no neighbour to dilate
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
  g.R = (k / 2) * dmax;
  g.cblocks = (int)((c + 15) / 16);
  return kOk;
}

}  // namespace ddpm

using namespace ddpm;

extern "C" int ddpm_gen_fwd(const void* x, const void* y, const void* weight, const void* bias,
                            void* out, int64_t n, int64_t c, int64_t h, int64_t w, int kernel_size,
                            int d0, int d1, int d2, int dtype, hipStream_t stream) {
  if (dtype < kF32 || dtype > kF16) return kBadArgument;
  GenGeom gg;
  int st = gen_make_geom(gg, n, c, h, w, kernel_size, d0, d1, d2);
  if (st != kOk) return st;
  if (n == 0 || c == 0 || h == 0 || w == 0) return kOk;
  if (!x || !y || !weight || !bias || !out) return kBadArgument;
  const int esz = dtype == kF32 ? 4 : 2;
  // 32-bit buffer offsets inside one image's [C][H][W] planes
  if (c * h * w * esz > 0x7fffffffLL) return kUnsupported;
  // 64-column tiles when their halo tile fits the LDS, else 32 columns
  FwdGeom g;
  size_t lds = 0;
  int cb = 4;
  st = fwd_geom(g, gg, esz, cb, lds);
  if (st == kUnsupported) {
    cb = 2;
    st = fwd_geom(g, gg, esz, cb, lds);
  }
  if (st != kOk) return st;
  const int nk = (int)((c + 31) / 32);
  return with_type(dtype, [&](auto tag) {
    using T = decltype(tag);
    auto launch = [&](auto kern) {
      if (lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)lds);
        if (e != hipSuccess) return (int)e;
      }
      hipLaunchKernelGGL(kern, dim3((unsigned)((int64_t)g.N * g.tiles * g.cblocks)),
                         dim3(kGfThreads), lds, stream, (const T*)x, (const T*)y,
                         (const T*)weight, (const T*)bias, (T*)out, g);
      return (int)hipGetLastError();
    };
    auto pick = [&](auto ks) {
      constexpr int KS = decltype(ks)::value;
      if (cb == 4)
        return nk == 1 ? launch(gen_fwd_kernel<T, KS, 1, 4>) : launch(gen_fwd_kernel<T, KS, 2, 4>);
      return nk == 1 ? launch(gen_fwd_kernel<T, KS, 1, 2>) : launch(gen_fwd_kernel<T, KS, 2, 2>);
    };
    if (kernel_size == 1) return pick(std::integral_constant<int, 1>());
    return pick(std::integral_constant<int, 3>());
  });
}
