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
// + m%4), so a lane holds 8 consecutive pixels of its row across the pair and
// writes them as one 16 bytes (measured 27% faster than two 8-byte writes).  A wave keeps the y
// operand of its 64 pixels in registers for every output row of its chunk and
// streams the weight rows (16 bytes = 8 consecutive input channels per lane;
// all waves read the same rows, so they come from L1 / L2).

#include "gen_common.h"
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
#pragma unroll 2
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
          const uint32_t off = (orow && px < HW) ? (rowoff + (uint32_t)px) * E : kOob;
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, t), ores, off, 0, 0);
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
    }
  }
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
}  // namespace ddpm

using namespace ddpm;

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
