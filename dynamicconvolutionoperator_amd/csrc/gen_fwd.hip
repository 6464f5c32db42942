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
// reference does before consuming it (_triton_kernels.py:332-335).  The
// workgroup body (gen_tile.h) keeps the x halo tile in LDS and the generated
// taps in the MFMA result registers; the identity part of the concat is
// written from the registers that stage the halo tile.

#include "gen_tile.h"
#include <type_traits>

namespace ddpm {

// CB = 4: 256 registers per lane (one 8-wave workgroup per CU, whose 133 KB
// halo tile fills the LDS anyway); CB = 2: 128 registers, two workgroups per
// CU, unless the y operand needs more (gt_waves_per_eu).
// PP: the concat as pair planes (kF32Pairs, fp32 only).
template <typename T, int KS, int NK, int CB, bool PP = false>
__global__ __launch_bounds__(kGtThreads) __attribute__((amdgpu_waves_per_eu(gt_waves_per_eu<T, NK, CB>()))) void gen_fwd_kernel(
    const T* __restrict__ x, const T* __restrict__ y, const T* __restrict__ wt,
    const T* __restrict__ bias, T* __restrict__ out, TileGeom g, CvPack fpk) {
  gen_tile_body<T, KS, NK, CB, false, PP>(x, y, wt, bias, out, nullptr, g, fpk);
}

// Two fp32 values rounded to nearest-even in T (bf16 / f16), packed low/high.
template <typename T>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (sizeof(T) == 2 && __is_same(T, bf16)) {
    return pack_bf16x2(a, b);
  } else {
    typedef f16 f16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, f16x2));
  }
}

// a.lo * b.lo + a.hi * b.hi + c on packed T pairs (v_dot2_f32_bf16 / _f16).
template <typename T>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  if constexpr (__is_same(T, bf16)) {
    typedef bf16 v2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), c,
                                           false);
  } else {
    typedef f16 v2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), c, false);
  }
}

// Forward for 2-byte types at K = 3 with the taps paired in the MFMA rows.
// The generator rows of a step are 8 channels x 2 taps (row m: channel
// c0 + 8*mb + m/2, tap 2j + m%2; the fifth pair of a branch holds tap 8 and a
// zero row), so a lane's 4 results are (ca, t0), (ca, t1), (cb, t0), (cb, t1)
// for two channels ca, cb: one cvt_pk rounds a channel's two taps to T
// together and one v_dot2_f32 multiplies them by x at the two shifted pixels
// and accumulates -- 1.5 VALU instructions per (channel, tap, pixel) where the
// one-tap rows need 4 (round, widen, widen x, fma).  Every pair step's weight
// slice (15 x 2 row blocks x C input channels, 16-byte fragment units copied
// straight from the weight rows; C % 8 == 0) stays in LDS, so the loop has no
// barrier.  The x halo tile, the identity channels and the y operand are
// the tile kernels' (gen_tile.h).
template <typename T, int NK, int CB>
__global__ __launch_bounds__(kGtThreads) __attribute__((amdgpu_waves_per_eu(gt_waves_per_eu<T, NK, CB>()))) void gen_fwd_pair_kernel(
    const T* __restrict__ x, const T* __restrict__ y, const T* __restrict__ wt,
    const T* __restrict__ bias, T* __restrict__ out, TileGeom g, CvPack fpk) {
  static_assert(sizeof(T) == 2, "2-byte types");
  typedef Mma<T> M;
  typedef typename M::V V;
  constexpr int KK = 9;
  constexpr int NPB = 5;        // tap pairs per branch
  constexpr int NPS = 3 * NPB;  // pair steps
  constexpr int E = 2;
  constexpr int XB = 4 * E;     // bytes of one 4-channel x entry
  constexpr int SU = 2 * NK;    // fragment units (x 64 lanes x 16 B) of one pair step: [mb][kk]
  constexpr int TW = 16 * CB;
  constexpr int NBW = 2 * CB;

  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  unsigned char* __restrict__ xs = smem;                                         // [4][plane]
  unsigned char* __restrict__ abuf = smem + 4 * g.plane;                         // [NPS][SU][64] x 16 B
  float* __restrict__ bs = reinterpret_cast<float*>(abuf + NPS * SU * 64 * 16);  // [NPS][32]

  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int cb = bid % g.cblocks;
  const int nt = bid / g.cblocks;
  const int tile = nt % g.tiles;
  const int n = nt / g.tiles;
  const int ty = tile / g.tiles_w, tx = tile - ty * g.tiles_w;
  const int h0 = ty * kGtTH, w0 = tx * TW;
  const int C = g.C, H = g.H, W = g.W, R = g.R, LW = g.LW;
  const uint32_t HWE = (uint32_t)((int64_t)H * W) * (uint32_t)E;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int col16 = lane & 15, quad = lane >> 4;
  const int c0 = cb * 16;
  const int nch = C - c0 < 16 ? C - c0 : 16;

  // x halo tile first (its loads are consumed here); then the bias rows, the
  // weight slices and the y operand, all in flight together
  gt_stage_x<T, XB, CB>(x, out, xs, g, n, c0, nch, h0, w0, TW, tid);
  // ---- bias rows [ps][mb*16 + m], written to LDS at the end of the prologue
  static_assert(NPS * 32 <= kGtThreads, "one bias value per thread");
  uint32_t bv;
  {
    const int ps = tid >> 5, rr = tid & 31;
    const int mb = rr >> 4, m = rr & 15;
    const int b = ps / NPB, j = ps - b * NPB;
    const int c = c0 + 8 * mb + (m >> 1), t = 2 * j + (m & 1);
    const BufRes bres = make_buf(bias, (uint32_t)(3 * C * KK * E));
    bv = gf_load_raw<E>(bres, (tid < NPS * 32 && c < C && t < KK)
                                  ? (uint32_t)((b * C + c) * KK + t) * (uint32_t)E
                                  : kOob);
  }
  // ---- every pair step's weight slice -> LDS: unit (ps, mb, kk, lane) holds
  //      the 16 bytes W[(b, c0 + 8mb + m/2, 2j + m%2)][kk*32 + 8q .. +7],
  //      m = lane & 15, q = lane >> 4 (zero for tap 9 and channels >= C)
  {
    const BufRes wres = make_buf(wt, (uint32_t)(3 * C * KK * C * E));
    const int m = lane & 15;
    for (int u = wave; u < NPS * SU; u += kGtWaves) {
      const int ps = u / SU, rem = u - ps * SU;
      const int mb = rem / NK, kk = rem - mb * NK;
      const int b = ps / NPB, j = ps - b * NPB;
      const int c = c0 + 8 * mb + (m >> 1), t = 2 * j + (m & 1), i0 = kk * 32 + 8 * quad;
      const uint32_t off =
          (c < C && t < KK && i0 < C) ? (uint32_t)((((b * C + c) * KK + t) * C + i0) * E) : kOob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          wres, (__attribute__((address_space(3))) void*)(abuf + (size_t)u * 64 * 16), 16, off, 0, 0,
          0);
    }
  }
  V bfr[NBW][NK][1];
  gt_load_y<T, NK, CB>(y, bfr, g, n, h0, w0, wave, col16, quad);
  if (tid < NPS * 32) bs[tid] = gf_raw_to_f<T>(bv);
  // ddpm_gen_fwd_pack: this workgroup's share of the fuse convolution's
  // weight packing
  if (fpk.total > 0) cv_pack_share<T>(fpk, (int)blockIdx.x, (int)gridDim.x, tid, kGtThreads);
  __builtin_amdgcn_s_waitcnt(0);  // the LDS-direct weight copies
  __syncthreads();

  // x entry of this lane's two channels (8mb + 2q, +1) at its block-0 pixel:
  // plane 2mb + q/2, bytes 4*(q%2) .. +3 of the 4-channel entry
  uint32_t lb[2];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
    lb[mb] = (uint32_t)((2 * mb + (quad >> 1)) * g.plane + col16 * XB + 4 * (quad & 1));
  // byte offset of row rr (0, 1) of this wave's blocks at zero shift; block
  // blk sits at row blk / CB, 16 * (blk % CB) entries to the right
  auto rbase = [&](int rr) { return (uint32_t)(((2 * wave + rr + R) * LW + R) * XB); };
  // global byte offset of channel c0 + 8mb + 2q + e at this lane's pixel of
  // block blk (kOob outside the image or the channel block)
  auto goff = [&](int blk, int mb, int e) {
    const int gh = h0 + 2 * wave + blk / CB, gw = w0 + 16 * (blk % CB) + col16;
    const int cl = 8 * mb + 2 * quad + e;
    return (gh < H && gw < W && cl < nch) ? (uint32_t)cl * HWE + (uint32_t)(gh * W + gw) * E : kOob;
  };

  float acc[NBW][2][2];  // branch output of channels (ca, cb) of each row block, per pixel block
#pragma unroll 1
  for (int ps = 0; ps < NPS; ++ps) {
    const int b = ps / NPB, j = ps - b * NPB;
    const int d = dil_of(b, g.d0, g.d1, g.d2);
    const int t0 = 2 * j, t1 = t0 + 1;
    const int sh0 = ((t0 / 3 - 1) * d * LW + (t0 % 3 - 1) * d) * XB;
    const bool pair = t1 < KK;  // wave-uniform
    const int sh1 = pair ? ((t1 / 3 - 1) * d * LW + (t1 % 3 - 1) * d) * XB : sh0;
    // x pairs (channel a: t0, t1) and (channel b: t0, t1) from the two reads;
    // the lone tap 8 pairs with zero
    const uint32_t sela = pair ? 0x05040100u : 0x0c0c0100u;
    const uint32_t selb = pair ? 0x07060302u : 0x0c0c0302u;
    if (j == 0) {
#pragma unroll
      for (int blk = 0; blk < NBW; ++blk)
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) acc[blk][mb][0] = acc[blk][mb][1] = 0.f;
    }
    const unsigned char* __restrict__ ab = abuf + ps * SU * 64 * 16;
    // both row blocks' MFMAs first, then both epilogues: the second block's
    // MFMAs run while the first block's epilogue issues
    f32x4 dacc[2][NBW];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      V afr[NK];
#pragma unroll
      for (int kk = 0; kk < NK; ++kk)
        afr[kk] = __builtin_bit_cast(V, *reinterpret_cast<const u32x4*>(ab + ((mb * NK + kk) * 64 + lane) * 16));
      const f32x4 binit = *reinterpret_cast<const f32x4*>(bs + ps * 32 + mb * 16 + 4 * quad);
#pragma unroll
      for (int blk = 0; blk < NBW; ++blk) {
        dacc[mb][blk] = binit;
#pragma unroll
        for (int kk = 0; kk < NK; ++kk) dacc[mb][blk] = M::mac1(afr[kk], bfr[blk][kk][0], dacc[mb][blk]);
      }
    }
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      uint32_t l = lb[mb];
      asm volatile("" : "+v"(l));
      // one base per (row, shift); the block's column is the reads' immediate offset
      const unsigned char* __restrict__ p0[2] = {xs + l + (rbase(0) + sh0), xs + l + (rbase(1) + sh0)};
      const unsigned char* __restrict__ p1[2] = {xs + l + (rbase(0) + sh1), xs + l + (rbase(1) + sh1)};
#pragma unroll
      for (int blk = 0; blk < NBW; ++blk) {
        const int co = 16 * (blk % CB) * XB;
        const uint32_t x0 = *reinterpret_cast<const uint32_t*>(p0[blk / CB] + co);
        const uint32_t x1 = *reinterpret_cast<const uint32_t*>(p1[blk / CB] + co);
        const uint32_t qa = pack2<T>(dacc[mb][blk][0], dacc[mb][blk][1]);
        const uint32_t qb = pack2<T>(dacc[mb][blk][2], dacc[mb][blk][3]);
        acc[blk][mb][0] = dot2<T>(qa, __builtin_amdgcn_perm(x1, x0, sela), acc[blk][mb][0]);
        acc[blk][mb][1] = dot2<T>(qb, __builtin_amdgcn_perm(x1, x0, selb), acc[blk][mb][1]);
      }
    }
    if (j == NPB - 1) {
      // ---- branch b: channels c0 + 8mb + 2q + e of output block b+1
      const BufRes bres = make_buf(out + ((int64_t)n * 4 * C + (int64_t)(b + 1) * C + c0) * (H * (int64_t)W),
                                   (uint32_t)nch * HWE);
#pragma unroll
      for (int blk = 0; blk < NBW; ++blk)
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
          for (int e = 0; e < 2; ++e) buf_store1<T>(bres, goff(blk, mb, e), acc[blk][mb][e]);
    }
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

}  // namespace

// Shared with the backward entry points.
int gen_make_geom(GenGeom& g, int64_t n, int64_t c, int64_t h, int64_t w, int k, int d0, int d1,
                  int d2, int kmax) {
  if (n < 0 || c < 0 || h < 0 || w < 0) return kBadArgument;
  if (k < 1 || (k % 2) == 0 || d0 < 1 || d1 < 1 || d2 < 1) return kBadArgument;
  if (k > kmax || c > 128) return kUnsupported;
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

namespace {

// ddpm_gen_fwd's work; fpk (optional): a fuse-convolution weight packing for
// the kernel's workgroups to run.  check_only: validate and return before
// launching.
int gf_run(const void* x, const void* y, const void* weight, const void* bias, void* out,
           int64_t n, int64_t c, int64_t h, int64_t w, int kernel_size, int d0, int d1, int d2,
           int dtype, hipStream_t stream, const CvPack* fpk, bool check_only) {
  // kF32Pairs: fp32 inputs, the concat written as pair planes (C % 16 == 0)
  const bool pp = dtype == kF32Pairs;
  if (pp) {
    if (c % 16 != 0 || 32 * h * w * 4 > 0x7fffffffLL) return kUnsupported;
    dtype = kF32;
  }
  if (dtype < kF32 || dtype > kF16) return kBadArgument;
  GenGeom gg;
  int st = gen_make_geom(gg, n, c, h, w, kernel_size, d0, d1, d2, kGenFwdMaxK);
  if (st != kOk) return st;
  if (n == 0 || c == 0 || h == 0 || w == 0) return kOk;
  if (!x || !y || !weight || !bias || !out) return kBadArgument;
  if (check_only) return kOk;
  const int esz = dtype == kF32 ? 4 : 2;
  const CvPack pk = fpk ? *fpk : CvPack{nullptr, nullptr, ConvGeom{}, 0, 0, 0, 0};
  // 32-bit buffer offsets inside one image's [C][H][W] planes (and 16 planes
  // past a channel block's first one)
  if (c * h * w * esz > 0x7fffffffLL || 16 * h * w * esz > 0x7fffffffLL) return kUnsupported;
  TileGeom g;
  size_t lds = 0;
  const int parts = esz == 4 ? 2 : 1;
  const int nk = gt_nk((int)c);
  int cb = 4;
  st = tile_geom_for(g, gg, 4 * esz, parts, cb, lds);
  if (st != kOk) return st;
  // 2-byte types at K = 3 with up to 64 channels (C % 8 == 0, aligned
  // weight): taps paired in the MFMA rows, every weight slice resident in LDS
  const size_t lds_pair = (size_t)4 * g.plane + (size_t)15 * 2 * nk * 64 * 16 + (size_t)15 * 32 * 4;
  const bool pair = esz == 2 && kernel_size == 3 && nk <= 2 && c % 8 == 0 &&
                    (uintptr_t)weight % 16 == 0 && lds_pair <= (size_t)kGtMaxLds;
  if (pair) {
    return with_type(dtype, [&](auto tag) {
      using T = decltype(tag);
      if constexpr (sizeof(T) == 2) {
        auto launch = [&](auto kern) {
          const int ae = allow_dynamic_lds(reinterpret_cast<const void*>(kern), lds_pair);
          if (ae != 0) return ae;
          hipLaunchKernelGGL(kern, dim3((unsigned)((int64_t)g.N * g.tiles * g.cblocks)),
                             dim3(kGtThreads), lds_pair, stream, (const T*)x, (const T*)y,
                             (const T*)weight, (const T*)bias, (T*)out, g, pk);
          return (int)hipGetLastError();
        };
        if (cb == 4) return nk == 1 ? launch(gen_fwd_pair_kernel<T, 1, 4>) : launch(gen_fwd_pair_kernel<T, 2, 4>);
        if (cb == 2) return nk == 1 ? launch(gen_fwd_pair_kernel<T, 1, 2>) : launch(gen_fwd_pair_kernel<T, 2, 2>);
        return nk == 1 ? launch(gen_fwd_pair_kernel<T, 1, 1>) : launch(gen_fwd_pair_kernel<T, 2, 1>);
      } else {
        return (int)kBadArgument;
      }
    });
  }
  return with_type(dtype, [&](auto tag) {
    using T = decltype(tag);
    auto launch = [&](auto kern) {
      const int ae = allow_dynamic_lds(reinterpret_cast<const void*>(kern), lds);
      if (ae != 0) return ae;
      hipLaunchKernelGGL(kern, dim3((unsigned)((int64_t)g.N * g.tiles * g.cblocks)),
                         dim3(kGtThreads), lds, stream, (const T*)x, (const T*)y,
                         (const T*)weight, (const T*)bias, (T*)out, g, pk);
      return (int)hipGetLastError();
    };
    // 1 or 2 chunks of 32 input channels, or 4 (65..128 channels; chunks
    // past C read zeros)
    auto pick = [&](auto ks, auto ppc) {
      constexpr int KS = decltype(ks)::value;
      constexpr bool PP = decltype(ppc)::value && sizeof(T) == 4;
      if (nk > 2) {
        return launch(gen_fwd_kernel<T, KS, 4, 2, PP>);  // 32-column tiles
      }
      if (cb == 4)
        return nk == 1 ? launch(gen_fwd_kernel<T, KS, 1, 4, PP>) : launch(gen_fwd_kernel<T, KS, 2, 4, PP>);
      if (cb == 1)
        return nk == 1 ? launch(gen_fwd_kernel<T, KS, 1, 1, PP>) : launch(gen_fwd_kernel<T, KS, 2, 1, PP>);
      return nk == 1 ? launch(gen_fwd_kernel<T, KS, 1, 2, PP>) : launch(gen_fwd_kernel<T, KS, 2, 2, PP>);
    };
    auto by_k = [&](auto ppc) {
      if (kernel_size == 1) return pick(std::integral_constant<int, 1>(), ppc);
      if (kernel_size == 3) return pick(std::integral_constant<int, 3>(), ppc);
      return pick(std::integral_constant<int, 5>(), ppc);
    };
    return pp ? by_k(std::true_type()) : by_k(std::false_type());
  });
}

}  // namespace

extern "C" int ddpm_gen_fwd(const void* x, const void* y, const void* weight, const void* bias,
                            void* out, int64_t n, int64_t c, int64_t h, int64_t w, int kernel_size,
                            int d0, int d1, int d2, int dtype, hipStream_t stream) {
  return gf_run(x, y, weight, bias, out, n, c, h, w, kernel_size, d0, d1, d2, dtype, stream,
                nullptr, false);
}

extern "C" int ddpm_gen_fwd_pack(const void* x, const void* y, const void* weight,
                                 const void* bias, void* out, const void* fuse_weight,
                                 void* fuse_workspace, int64_t fuse_workspace_bytes, int64_t n,
                                 int64_t c, int64_t h, int64_t w, int kernel_size, int d0, int d1,
                                 int d2, int dtype, hipStream_t stream) {
  // both parts validated before anything is launched
  int st = gf_run(x, y, weight, bias, out, n, c, h, w, kernel_size, d0, d1, d2, dtype, stream,
                  nullptr, true);
  if (st != kOk) return st;
  CvPack pk;
  st = cv_fwd_pack(pk, out, fuse_weight, fuse_workspace, fuse_workspace_bytes, n, c, h, w, dtype);
  if (st != kOk) return st;
  return gf_run(x, y, weight, bias, out, n, c, h, w, kernel_size, d0, d1, d2, dtype, stream, &pk,
                false);
}
