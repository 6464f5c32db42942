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
//   * one workgroup per (image-row segment of 256 pixels, group of 64 output
//     planes m); 8 waves, two per SIMD, each owning 32 pixels (two MFMA
//     column blocks) x the group's 64 planes;
//   * the K loop runs in stages (32-plane chunk of `in`, kernel row ki): a
//     stage needs one row h + ki - 1 of 32 input planes, 256 + 16 columns,
//     and the group's A slice for the 3 taps of that row; both are copied
//     global -> LDS by buffer loads that write LDS directly (16-byte lanes;
//     reads outside the image return zero), one stage ahead into a second
//     buffer;
//   * A is packed once per call by a small kernel into MFMA A-fragment order
//     (fp32: split into bf16 hi / lo), so a fragment is one 16-byte LDS read;
//   * MFMA slot k = 8*quad + e of a 32-plane chunk holds plane 4*e + quad (A
//     and B alike): a lane's 8 B-operand reads are 4 planes apart and, with a
//     row pitch of 16 (mod 64) dwords, bank-conflict free;
//   * v_mfma_f32_16x16x32_{bf16,f16}; fp32 operands run as three bf16
//     products (hi*hi + hi*lo + lo*hi), accumulation in fp32.

#include "gen_common.h"

#include <type_traits>

namespace ddpm {

constexpr int kCvWaves = 8;
constexpr int kCvThreads = 64 * kCvWaves;
constexpr int kCvTW = 32 * kCvWaves;       // output columns per workgroup
constexpr int kCvPad = 8;                  // staged column halo (one chunk of 2-byte values)
constexpr int kCvLW = kCvTW + 2 * kCvPad;  // staged columns (272)
constexpr int kCvMB = 4;                   // 16-plane blocks of m per workgroup

struct ConvGeom {
  int N, K, M, H, W;  // K input planes, M output planes
  int col_tiles;      // ceil(W / kCvTW)
  int nc32;           // ceil(K / 32)
  int mgroups;        // ceil(M / (kCvMB * 16))
  int x4;             // input rows copied in 16-byte lanes (W % 8 == 0, aligned base)
};

template <typename T>
__host__ __device__ constexpr int cv_parts() {
  return sizeof(T) == 4 ? 2 : 1;
}

// Packed A: 16-byte units [mg][cc][ki][kj][ib][part][lane], lane (m = mg*64 +
// ib*16 + (lane & 15), q = lane >> 4) holding A[m][cc*32 + 4e + q][ki][kj],
// e = 0..7.  `rot` selects the input-gradient form (transposed, rotated).
template <typename T>
__global__ __launch_bounds__(256) void conv3x3_pack_kernel(const T* __restrict__ wt,
                                                           uint32_t* __restrict__ pk, ConvGeom g,
                                                           int rot) {
  constexpr int P = cv_parts<T>();
  const int64_t total = (int64_t)g.mgroups * g.nc32 * 9 * kCvMB * 64;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int lane = (int)(idx & 63);
  int64_t rest = idx >> 6;
  const int ib = (int)(rest % kCvMB);
  rest /= kCvMB;
  const int tap = (int)(rest % 9);
  rest /= 9;
  const int cc = (int)(rest % g.nc32);
  const int mg = (int)(rest / g.nc32);
  const int ki = tap / 3, kj = tap - 3 * ki;
  const int m = mg * kCvMB * 16 + ib * 16 + (lane & 15), q = lane >> 4;
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int k = cc * 32 + 4 * e + q;
    float a = 0.f;
    if (m < g.M && k < g.K) {
      // forward: weight[m][k][ki][kj]; input gradient: weight[k][m][2-ki][2-kj]
      const int64_t off = rot ? (((int64_t)k * g.M + m) * 3 + (2 - ki)) * 3 + (2 - kj)
                              : (((int64_t)m * g.K + k) * 3 + ki) * 3 + kj;
      a = to_f(wt[off]);
    }
    v[e] = a;
  }
  typename Mma<T>::V o[P];
  Mma<T>::pack(v, o);
  u32x4* __restrict__ dst = reinterpret_cast<u32x4*>(pk);
  const int64_t unit = (((((int64_t)mg * g.nc32 + cc) * 9 + tap) * kCvMB + ib) * P) * 64 + lane;
#pragma unroll
  for (int part = 0; part < P; ++part) dst[unit + part * 64] = __builtin_bit_cast(u32x4, o[part]);
}

// One LDS staging buffer (dwords): input rows [32 planes][kXS] then the A
// slice [3 taps][kCvMB][P][64 lanes][4 dwords].
template <typename T>
struct CvLds {
  static constexpr int kE = (int)sizeof(T);
  static constexpr int kPerD = 4 / kE;
  static constexpr int kXD = kCvLW / kPerD;  // dwords per staged row
  // pitch = 16 (mod 64) dwords: the 8 plane reads of a lane fall on distinct banks
  static constexpr int kXS = kXD + ((16 - kXD % 64) + 64) % 64;
  static constexpr int kXChunks = kXD / 4;  // 16-byte chunks per row
  static constexpr int kAOff = 32 * kXS;
  static constexpr int kAUnits = 3 * kCvMB * cv_parts<T>() * 64;  // 16-byte units
  static constexpr int kBuf = kAOff + 4 * kAUnits;
};

template <typename T, bool BIAS>
__global__ __launch_bounds__(kCvThreads) void conv3x3_kernel(const T* __restrict__ in,
                                                             const uint32_t* __restrict__ pk,
                                                             const T* __restrict__ bias,
                                                             T* __restrict__ out, ConvGeom g) {
  typedef Mma<T> M;
  typedef typename M::V V;
  typedef CvLds<T> L;
  constexpr int P = M::P;
  constexpr int E = (int)sizeof(T);
  extern __shared__ __attribute__((aligned(16))) uint32_t csm[];

  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int mg = bid % g.mgroups;
  const int tile = bid / g.mgroups;
  const int row = tile / g.col_tiles;  // image row n*H + h
  const int w0 = (tile - row * g.col_tiles) * kCvTW;
  const int n = row / g.H, h = row - n * g.H;
  const int H = g.H, W = g.W;
  const int64_t HW = (int64_t)H * W;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int col16 = lane & 15, quad = lane >> 4;
  const int nstage = 3 * g.nc32;  // (cc, ki)

  const BufRes xres = make_buf(in + (int64_t)n * g.K * HW, (uint32_t)(g.K * HW * (int64_t)E));
  // ---- stage s = cc * 3 + ki -> LDS buffer `buf`
  auto stage = [&](int s, int buf) {
    const int ki = s % 3;
    const int cc = s / 3;
    const int hh = h + ki - 1;
    uint32_t* __restrict__ dstb = csm + buf * L::kBuf;
    if (g.x4) {
      // one resource for the image; a chunk outside the image (column, row or
      // plane) reads zero through its offset (W % 8 == 0: chunks are whole)
#pragma unroll
      for (int j = 0; j < 32 / kCvWaves; ++j) {
        const int cr = wave + kCvWaves * j;
        const int ch = cc * 32 + cr;
        const bool ok = ch < g.K && (unsigned)hh < (unsigned)H;
        const uint32_t rowel = (uint32_t)ch * (uint32_t)HW + (uint32_t)(hh * W);
#pragma unroll
        for (int part = 0; part < (L::kXChunks + 63) / 64; ++part) {
          // the last copy ends at the row end (it may overlap the previous one)
          const int pc = 64 * part < L::kXChunks - 64 ? 64 * part
                                                      : (L::kXChunks > 64 ? L::kXChunks - 64 : 0);
          const int gw = w0 - kCvPad + (pc + lane) * 4 * L::kPerD;
          const uint32_t off =
              (ok && (unsigned)gw < (unsigned)W) ? (rowel + (uint32_t)gw) * (uint32_t)E : kOob;
          if (L::kXChunks >= 64 || lane < L::kXChunks)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                xres, (__attribute__((address_space(3))) void*)(dstb + cr * L::kXS + 4 * pc), 16,
                off, 0, 0, 0);
        }
      }
    } else {
      // element-wise copy through registers (W % 8 != 0 or unaligned input)
      T* __restrict__ dst = reinterpret_cast<T*>(dstb);
      for (int idx = tid; idx < 32 * kCvLW; idx += kCvThreads) {
        const int cr = idx / kCvLW, j = idx - cr * kCvLW;
        const int ch = cc * 32 + cr, gw = w0 - kCvPad + j;
        const bool ok = ch < g.K && (unsigned)hh < (unsigned)H && (unsigned)gw < (unsigned)W;
        const uint32_t off = ok ? ((uint32_t)ch * (uint32_t)HW + (uint32_t)(hh * W + gw)) * E : kOob;
        dst[cr * L::kXS * L::kPerD + j] = from_f<T>(buf_load1<T>(xres, off));
      }
    }
    // A slice of the stage's 3 taps: contiguous in the packed weight
    const uint32_t* src = pk + ((((int64_t)mg * g.nc32 + cc) * 9 + ki * 3) * kCvMB * P * 64) * 4;
    const BufRes pres = make_buf(src, (uint32_t)(L::kAUnits * 16));
#pragma unroll
    for (int j = 0; j < (L::kAUnits / 64 + kCvWaves - 1) / kCvWaves; ++j) {
      const int u = wave + kCvWaves * j;
      if ((L::kAUnits / 64) % kCvWaves == 0 || u < L::kAUnits / 64)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            pres, (__attribute__((address_space(3))) void*)(dstb + L::kAOff + 256 * u), 16,
            (uint32_t)(u * 64 + lane) * 16u, 0, 0, 0);
    }
  };

  f32x4 acc[2][kCvMB];
#pragma unroll
  for (int blk = 0; blk < 2; ++blk)
#pragma unroll
    for (int ib = 0; ib < kCvMB; ++ib) acc[blk][ib] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int px0 = 32 * wave + col16;  // pixel of block 0 within the tile; block 1 is +16
  stage(0, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int s = 0; s < nstage; ++s) {
    const int buf = s & 1;
    if (s + 1 < nstage) stage(s + 1, buf ^ 1);
    const uint32_t* __restrict__ bb = csm + buf * L::kBuf;
    // this lane's input elements: plane 4e + quad, column pad + px + dw
    const uint32_t* __restrict__ xq = bb + quad * L::kXS;
#pragma unroll
    for (int kj = 0; kj < 3; ++kj) {
      const int dw = kj - 1;
      V afr[kCvMB][P];
#pragma unroll
      for (int ib = 0; ib < kCvMB; ++ib)
#pragma unroll
        for (int pp = 0; pp < P; ++pp)
          afr[ib][pp] = __builtin_bit_cast(
              V, *reinterpret_cast<const u32x4*>(bb + L::kAOff +
                                                 4 * ((((kj * kCvMB) + ib) * P + pp) * 64 + lane)));
#pragma unroll
      for (int blk = 0; blk < 2; ++blk) {
        const int col = kCvPad + px0 + 16 * blk + dw;
        float bv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if constexpr (sizeof(T) == 4)
            bv[e] = __uint_as_float(xq[4 * e * L::kXS + col]);
          else
            bv[e] = to_f(reinterpret_cast<const T*>(xq + 4 * e * L::kXS)[col]);
        }
        V bfr[P];
        M::pack(bv, bfr);
#pragma unroll
        for (int ib = 0; ib < kCvMB; ++ib) acc[blk][ib] = M::mac(afr[ib], bfr, acc[blk][ib]);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }

  // ---- store: lane holds out[m = mg*64 + ib*16 + 4*quad + e][pixel col16 of block]
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    const int w = w0 + px0 + 16 * blk;
    if (w < W) {
      T* __restrict__ yo = out + (int64_t)n * g.M * HW + (int64_t)h * W + w;
#pragma unroll
      for (int ib = 0; ib < kCvMB; ++ib)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int m = mg * kCvMB * 16 + ib * 16 + 4 * quad + e;
          if (m < g.M) {
            float v = acc[blk][ib][e];
            if constexpr (BIAS) v += to_f(bias[m]);
            yo[(int64_t)m * HW] = from_f<T>(v);
          }
        }
    }
  }
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

void cv_geom(ConvGeom& g, int64_t n, int64_t k, int64_t m, int64_t h, int64_t w) {
  g.N = (int)n;
  g.K = (int)k;
  g.M = (int)m;
  g.H = (int)h;
  g.W = (int)w;
  g.col_tiles = (int)((w + kCvTW - 1) / kCvTW);
  g.nc32 = (int)((k + 31) / 32);
  g.mgroups = (int)((m + kCvMB * 16 - 1) / (kCvMB * 16));
  g.x4 = 0;
}

int64_t cv_pack_bytes(const ConvGeom& g, int dtype) {
  return (int64_t)g.mgroups * g.nc32 * 9 * kCvMB * (dtype == kF32 ? 2 : 1) * 64 * 16;
}

// Shape checks shared by both directions: K input planes, M output planes.
int cv_check(int64_t n, int64_t k, int64_t m, int64_t h, int64_t w, int dtype) {
  if (dtype < kF32 || dtype > kF16) return kBadArgument;
  if (n < 0 || k < 0 || m < 0 || h < 0 || w < 0) return kBadArgument;
  const int64_t esz = dtype == kF32 ? 4 : 2;
  // 32-bit buffer offsets inside one image's input and output planes
  if (k * h * w * esz > 0x7fffffffLL || m * h * w * esz > 0x7fffffffLL) return kUnsupported;
  if (h > (1 << 20) || w > (1 << 20)) return kUnsupported;
  const int64_t groups = n * h * ((w + kCvTW - 1) / kCvTW) * ((m + kCvMB * 16 - 1) / (kCvMB * 16));
  if (groups > 0x7fffffffLL) return kUnsupported;
  return kOk;
}

int cv_run(const void* in, const void* wt, const void* bias, void* out, void* workspace,
           int64_t workspace_bytes, int64_t n, int64_t k, int64_t m, int64_t h, int64_t w, int rot,
           int dtype, hipStream_t stream) {
  ConvGeom g;
  cv_geom(g, n, k, m, h, w);
  const int64_t need = cv_pack_bytes(g, dtype);
  if (!workspace || workspace_bytes < need || (uintptr_t)workspace % 16 != 0)
    return kWorkspaceTooSmall;
  const int esz = dtype == kF32 ? 4 : 2;
  g.x4 = (w % 8 == 0) && ((uintptr_t)in % 16 == 0);
  (void)esz;
  return cv_with_type(dtype, [&](auto tag) {
    using T = decltype(tag);
    typedef CvLds<T> L;
    const int64_t units = (int64_t)g.mgroups * g.nc32 * 9 * kCvMB * 64;
    hipLaunchKernelGGL((conv3x3_pack_kernel<T>), dim3((unsigned)((units + 255) / 256)), dim3(256), 0,
                       stream, (const T*)wt, (uint32_t*)workspace, g, rot);
    int e = (int)hipGetLastError();
    if (e != 0) return e;
    const size_t lds = (size_t)2 * L::kBuf * 4;
    const dim3 grid((unsigned)((int64_t)n * h * g.col_tiles * g.mgroups));
    auto launch = [&](auto kern) {
      const int ae = allow_dynamic_lds(reinterpret_cast<const void*>(kern), lds);
      if (ae != 0) return ae;
      hipLaunchKernelGGL(kern, grid, dim3(kCvThreads), lds, stream, (const T*)in,
                         (const uint32_t*)workspace, (const T*)bias, (T*)out, g);
      return (int)hipGetLastError();
    };
    if (bias) return launch(conv3x3_kernel<T, true>);
    return launch(conv3x3_kernel<T, false>);
  });
}

}  // namespace
}  // namespace ddpm

using namespace ddpm;

extern "C" int64_t ddpm_fuse_conv_workspace_bytes(int64_t c, int dtype) {
  if (c <= 0 || dtype < kF32 || dtype > kF16) return 0;
  ConvGeom gf, gd;
  cv_geom(gf, 1, 4 * c, c, 1, 1);  // forward: K = 4C input planes, M = C
  cv_geom(gd, 1, c, 4 * c, 1, 1);  // input gradient: K = C, M = 4C
  const int64_t a = cv_pack_bytes(gf, dtype), b = cv_pack_bytes(gd, dtype);
  return a > b ? a : b;
}

extern "C" int ddpm_fuse_conv_fwd(const void* cat, const void* weight, const void* bias, void* out,
                                  void* workspace, int64_t workspace_bytes, int64_t n, int64_t c,
                                  int64_t h, int64_t w, int dtype, hipStream_t stream) {
  int st = cv_check(n, 4 * c, c, h, w, dtype);
  if (st != kOk) return st;
  if (n == 0 || c == 0 || h == 0 || w == 0) return kOk;
  if (!cat || !weight || !out) return kBadArgument;
  return cv_run(cat, weight, bias, out, workspace, workspace_bytes, n, 4 * c, c, h, w, 0, dtype,
                stream);
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
