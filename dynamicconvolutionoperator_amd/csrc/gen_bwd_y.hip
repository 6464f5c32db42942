// Gradient with respect to y of the fused op (recompute backward).
//
// Counterpart of _generator_dynamic_cat_bwd_y (_triton_kernels.py:534-623,
// launched at :963-971):
//
//   dY[i, p] = sum_{b, t, c} W[(b,c,t), i] * dK[(b,c,t), p]
//   dK[(b,c,t), p] = gO_b[c, p] * x[c, p + off(b,t)]
//
// A GEMM with M = i, N = pixels and K = (b, t, c) whose B operand dK is
// formed on chip and never stored.  Work decomposition (CDNA4):
//   * one workgroup per image-row segment of 256 pixels (and, above 64
//     channels, per half of the output channels i); 8 waves, two per SIMD,
//     each owning 32 pixels (two MFMA column blocks) x all C i (x the
//     workgroup's 64 i);
//   * the K loop runs in stages (branch b, 32-channel chunk, tap row ki): a
//     stage needs one x row (h + dh) of 32 channels, 256 + 16 columns, and
//     the K-slice of the weight for its K taps; both are copied global -> LDS
//     by buffer loads that write LDS directly (16-byte lanes; out-of-image
//     reads return zero), one stage ahead into a second buffer;
//   * the weight is pre-split (bf16 hi/lo for fp32) and pre-transposed by a
//     small packing kernel into MFMA A-fragment order, so a fragment is one
//     16-byte LDS read per lane;
//   * MFMA slot k = 8*quad + e of a 32-channel chunk holds channel 4*e + quad
//     (A and B alike): a lane's 8 B-operand reads are 4 channels apart, and
//     with an x-row pitch of 16 (mod 64) dwords every read is bank-conflict
//     free;
//   * v_mfma_f32_16x16x32_{bf16,f16}; fp32 operands run as three bf16
//     products (hi*hi + hi*lo + lo*hi).

#include "gen_bwd.h"

#include <atomic>
#include <mutex>
#include <type_traits>

namespace ddpm {

constexpr int kYtWaves = 8;
constexpr int kYtThreads = 64 * kYtWaves;
constexpr int kYtTW = 32 * kYtWaves;        // output columns per workgroup
constexpr int kYtPad = 8;                   // staged column halo (>= dilation)
constexpr int kYtLW = kYtTW + 2 * kYtPad;   // staged x columns (272)
constexpr int kYtMaxDil = kYtPad;

struct YGeom {
  int N, C, H, W;
  int d0, d1, d2;
  int col_tiles;  // ceil(W / kYtTW)
  int nc32;       // ceil(C / 32)
  int ihalves;    // 1, or 2 when C > 64: workgroups per segment, 16*MB output channels each
  int x4;         // x rows can be copied in 16-byte lanes (W % 8 == 0, aligned base)
};

template <typename T, int KS, int MB>
__global__ __launch_bounds__(256) void gen_pack_wt_kernel(const T* __restrict__ wt,
                                                          uint32_t* __restrict__ pk, int C,
                                                          int nc32, int total) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx < total) yt_pack_item<T, KS, MB>(wt, pk, C, nc32, idx);
}

// One LDS staging buffer (dwords): x rows [CH * 32 channels][kXS] then the
// weight slices [CH chunks][KS taps][MB][P][64 lanes][4 dwords].
template <typename T, int KS, int MB, int CH>
struct YtLds {
  static constexpr int kE = (int)sizeof(T);
  static constexpr int kPerD = 4 / kE;
  static constexpr int kXD = kYtLW / kPerD;                      // dwords per staged row
  // pitch = 16 (mod 64) dwords for fp32 rows, 32 (mod 128) elements (16 mod 64
  // dwords) for 2-byte rows; a multiple of 4 dwords (16-byte copies)
  static constexpr int kXS = kXD + ((16 - kXD % 64) + 64) % 64;
  static constexpr int kXChunks = kXD / 4;                       // 16-byte chunks per row
  static constexpr int kXOff = 0;
  static constexpr int kAOff = 32 * CH * kXS;
  static constexpr int kAUnits1 = KS * MB * yt_parts<T>() * 64;  // 16-byte units of one chunk
  static constexpr int kAUnits = CH * kAUnits1;
  static constexpr int kBuf = kAOff + 4 * kAUnits;
};

// CH: 32-channel chunks per stage (2 for 2-byte types when the chunk count
// is even: twice the MFMA work per stage and per barrier, LDS 122 KB at
// C = 64).
// AL: aligned layout (16-byte x rows, whole 32-channel chunks): the x copies
// take the lane's column offset formed once per workgroup (kOob for the halo
// chunks outside the image) and a scalar row offset per stage, without
// per-copy tests.
template <typename T, int KS, int MB, int CH, bool AL = false>
__global__ __launch_bounds__(kYtThreads) void gen_bwd_y_kernel(const T* __restrict__ x,
                                                               const uint32_t* __restrict__ pk,
                                                               const T* __restrict__ gout,
                                                               T* __restrict__ gy, YGeom g,
                                                               WReduce red) {
  typedef Mma<T> M;
  typedef typename M::V V;
  typedef YtLds<T, KS, MB, CH> L;
  constexpr int KK = KS * KS;
  constexpr int r = KS / 2;
  constexpr int P = M::P;
  constexpr int E = (int)sizeof(T);
  extern __shared__ __attribute__((aligned(16))) uint32_t ysm[];

  const int logical = xcd_remap(blockIdx.x, gridDim.x);
  const int ih = logical % g.ihalves;  // output channels (ih*MB + ib)*16 + ...
  const int tile = logical / g.ihalves;
  const int row = tile / g.col_tiles;  // image row n*H + h
  const int w0 = (tile - row * g.col_tiles) * kYtTW;
  const int n = row / g.H, h = row - n * g.H;
  const int C = g.C, H = g.H, W = g.W;
  const int64_t HW = (int64_t)H * W;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int col16 = lane & 15, quad = lane >> 4;
  const int ncg = g.nc32 / CH;        // groups of CH chunks (CH divides nc32)
  const int nstage = 3 * ncg * KS;    // (b, chunk group, ki)

  // x planes of image n (per-row resources cost ~20 scalar instructions per
  // row and stage; measured bf16 44.9 -> 41.6 us)
  const BufRes xres = make_buf(x + (int64_t)n * C * HW, (uint32_t)(C * HW * (int64_t)E));
  const BufRes xnul = make_buf(x, 0u);
  constexpr int kXP = (L::kXChunks + 63) / 64;  // copies per staged row
  uint32_t alcol[kXP];
  if constexpr (AL) {
#pragma unroll
    for (int part = 0; part < kXP; ++part) {
      const int pc = 64 * part < L::kXChunks - 64 ? 64 * part : (L::kXChunks > 64 ? L::kXChunks - 64 : 0);
      const int gw = w0 - kYtPad + (pc + lane) * 4 * L::kPerD;
      alcol[part] = (unsigned)gw < (unsigned)W ? (uint32_t)gw * (uint32_t)E : kOob;
    }
  }
  // ---- stage s = ((b * ncg) + cg) * KS + ki -> LDS buffer `buf`
  auto stage = [&](int s, int buf) {
    const int ki = s % KS;
    const int bg = s / KS;
    const int cg = bg % ncg, b = bg / ncg;
    const int d = dil_of(b, g.d0, g.d1, g.d2);
    const int hh = h + (ki - r) * d;
    uint32_t* __restrict__ dstb = ysm + buf * L::kBuf;
    // x rows: 32 * CH channels of row hh, columns w0 - pad .. w0 + TW + pad
    if constexpr (AL) {
      // a row outside the image copies through a resource with no records
      const bool rok = (unsigned)hh < (unsigned)H;
      const BufRes rs = rok ? xres : xnul;
      const uint32_t roff = rok ? (uint32_t)(hh * W) * (uint32_t)E : 0u;
      if (L::kXChunks >= 64 || lane < L::kXChunks) {
#pragma unroll
        for (int j = 0; j < 32 * CH / kYtWaves; ++j) {
          const int cr = wave + kYtWaves * j;
          // (the offsets go through named variables: written as expressions
          // in the call, the host pass drops the kernel's stub)
          const uint32_t so = (uint32_t)(cg * CH * 32 + cr) * (uint32_t)HW * (uint32_t)E + roff;
#pragma unroll
          for (int part = 0; part < kXP; ++part) {
            const int pc = 64 * part < L::kXChunks - 64 ? 64 * part : (L::kXChunks > 64 ? L::kXChunks - 64 : 0);
            const uint32_t vo = alcol[part];
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rs, (__attribute__((address_space(3))) void*)(dstb + L::kXOff + cr * L::kXS + 4 * pc),
                16, vo, so, 0, 0);
          }
        }
      }
    } else if (g.x4) {
      // one resource for the image; a chunk outside the image (column, row or
      // channel) reads zero through its offset (W % 8 == 0: chunks are whole)
#pragma unroll
      for (int j = 0; j < 32 * CH / kYtWaves; ++j) {
        const int cr = wave + kYtWaves * j;
        const int ch = cg * CH * 32 + cr;
        const bool ok = ch < C && (unsigned)hh < (unsigned)H;
        const uint32_t rowel = (uint32_t)ch * (uint32_t)HW + (uint32_t)(hh * W);
#pragma unroll
        for (int part = 0; part < (L::kXChunks + 63) / 64; ++part) {
          // the last copy ends at the row end (it may overlap the previous one)
          const int pc = 64 * part < L::kXChunks - 64 ? 64 * part : (L::kXChunks > 64 ? L::kXChunks - 64 : 0);
          const int gw = w0 - kYtPad + (pc + lane) * 4 * L::kPerD;
          const uint32_t off = (ok && (unsigned)gw < (unsigned)W) ? (rowel + (uint32_t)gw) * (uint32_t)E : kOob;
          if (L::kXChunks >= 64 || lane < L::kXChunks)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                xres, (__attribute__((address_space(3))) void*)(dstb + L::kXOff + cr * L::kXS + 4 * pc),
                16, off, 0, 0, 0);
        }
      }
    } else {
      // element-wise copy through registers (W % 8 != 0 or unaligned x)
      T* __restrict__ dst = reinterpret_cast<T*>(dstb);
      for (int idx = tid; idx < 32 * CH * kYtLW; idx += kYtThreads) {
        const int cr = idx / kYtLW, j = idx - cr * kYtLW;
        const int ch = cg * CH * 32 + cr, gw = w0 - kYtPad + j;
        float v = 0.f;
        if (ch < C && (unsigned)hh < (unsigned)H && (unsigned)gw < (unsigned)W)
          v = to_f(x[((int64_t)n * C + ch) * HW + (int64_t)hh * W + gw]);
        dst[(L::kXOff + cr * L::kXS) * L::kPerD + j] = from_f<T>(v);
      }
    }
    // weight slices of the stage's K taps, one per chunk: each contiguous
    // in the packed weight
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int cc = cg * CH + c;
      const uint32_t* src =
          pk + (int64_t)(((ih * 3 * g.nc32 + b * g.nc32 + cc) * KK + ki * KS) * MB * P * 64) * 4;
      const BufRes pres = make_buf(src, (uint32_t)(L::kAUnits1 * 16));
#pragma unroll
      for (int j = 0; j < (L::kAUnits1 / 64 + kYtWaves - 1) / kYtWaves; ++j) {
        const int u = wave + kYtWaves * j;
        if ((L::kAUnits1 / 64) % kYtWaves == 0 || u < L::kAUnits1 / 64)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              pres,
              (__attribute__((address_space(3))) void*)(dstb + L::kAOff + 4 * c * L::kAUnits1 + 256 * u),
              16, (uint32_t)(u * 64 + lane) * 16u, 0, 0, 0);
      }
    }
  };

  // ---- branch-gradient values of this lane: channel cc*32 + 4e + quad of
  //      each chunk cc of the group at its two pixels (held for the KS
  //      stages of one (b, chunk group))
  const int px0 = 32 * wave + col16;  // pixel of block 0 within the tile; block 1 is +16
  // gv: the current (b, chunk group)'s values; gn: the next one's, loaded
  // during the last stage of the current one (its latency hidden behind that
  // stage's MFMAs, as the stage's copies are)
  float gv[CH][2][8], gn[CH][2][8];
  // aligned layout (whole 32-channel chunks): the lane's byte offset of
  // channel quad at its pixel of each block (kOob past the last column),
  // formed once; the channel's part goes in the loads' scalar offset
  uint32_t glo[2];
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    const int w = w0 + px0 + 16 * blk;
    glo[blk] = w < W ? ((uint32_t)quad * (uint32_t)HW + (uint32_t)(h * W + w)) * (uint32_t)E : kOob;
  }
  auto load_g = [&](int bg, float (&gd)[CH][2][8]) {
    const int cg = bg % ncg, b = bg / ncg;
    const BufRes gres = make_buf(gout + ((int64_t)n * 4 * C + (int64_t)(b + 1) * C) * HW,
                                 (uint32_t)(C * HW * (int64_t)E));
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
      for (int blk = 0; blk < 2; ++blk) {
        const int w = w0 + px0 + 16 * blk;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if constexpr (AL) {
            const uint32_t so = (uint32_t)((cg * CH + c) * 32 + 4 * e) * (uint32_t)HW * (uint32_t)E;
            gd[c][blk][e] = buf_load1<T>(gres, glo[blk], so);
          } else {
            const int ch = (cg * CH + c) * 32 + 4 * e + quad;
            const uint32_t off =
                (ch < C && w < W) ? (uint32_t)((int64_t)ch * HW + (int64_t)h * W + w) * E : kOob;
            gd[c][blk][e] = buf_load1<T>(gres, off);
          }
        }
      }
  };

  f32x4 acc[2][MB];
#pragma unroll
  for (int blk = 0; blk < 2; ++blk)
#pragma unroll
    for (int ib = 0; ib < MB; ++ib) acc[blk][ib] = f32x4{0.f, 0.f, 0.f, 0.f};

  stage(0, 0);
  load_g(0, gv);
  if (red.items > 0) {
    // ddpm_gen_bwd: this workgroup's share of the weight gradient's split
    // reduction (the partial kernel ran before this launch), its loads in
    // flight together with the first stage's copies
    const int per = (red.items + (int)gridDim.x - 1) / (int)gridDim.x;
    for (int j = tid; j < per; j += kYtThreads) {
      const uint32_t item = (uint32_t)((int)blockIdx.x * per + j);
      if (red.v4)
        wg_reduce_item<T, 4>(red.pw, red.pb, (T*)red.dw, (T*)red.db, red.C, red.KK, red.splits, item);
      else
        wg_reduce_item<T, 1>(red.pw, red.pb, (T*)red.dw, (T*)red.db, red.C, red.KK, red.splits, item);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int s = 0; s < nstage; ++s) {
    const int buf = s & 1;
    if (s + 1 < nstage) stage(s + 1, buf ^ 1);
    const int ki = s % KS;
    const int bg = s / KS;
    const int b = bg / ncg;
    const int d = dil_of(b, g.d0, g.d1, g.d2);
    // the next (b, chunk group)'s branch-gradient values, during this stage
    const bool gnext = ki == KS - 1 && s + 1 < nstage;
    if (gnext) load_g(bg + 1, gn);
    const uint32_t* __restrict__ bb = ysm + buf * L::kBuf;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      // this lane's x elements: channel 32c + 4e + quad, column pad + px + dw
      const uint32_t* __restrict__ xq = bb + L::kXOff + (32 * c + quad) * L::kXS;
#pragma unroll
      for (int kj = 0; kj < KS; ++kj) {
        const int dw = (kj - r) * d;
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
          const int col = kYtPad + px0 + 16 * blk + dw;
          float dk[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            float xv;
            if constexpr (sizeof(T) == 4)
              xv = __uint_as_float(xq[4 * e * L::kXS + col]);
            else
              xv = to_f(reinterpret_cast<const T*>(xq + 4 * e * L::kXS)[col]);
            dk[e] = gv[c][blk][e] * xv;
          }
          V bfr[P];
          M::pack(dk, bfr);
#pragma unroll
          for (int ib = 0; ib < MB; ++ib) acc[blk][ib] = M::mac(afr[ib], bfr, acc[blk][ib]);
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (gnext) {
#pragma unroll
      for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int blk = 0; blk < 2; ++blk)
#pragma unroll
          for (int e = 0; e < 8; ++e) gv[c][blk][e] = gn[c][blk][e];
    }
  }

  // ---- store: lane holds dY[i = ib*16 + 4*quad + e][pixel col16 of block]
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    const int w = w0 + px0 + 16 * blk;
    if (w < W) {
      T* __restrict__ yo = gy + (int64_t)n * C * HW + (int64_t)h * W + w;
#pragma unroll
      for (int ib = 0; ib < MB; ++ib)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = (ih * MB + ib) * 16 + 4 * quad + e;
          if (i < C) yo[(int64_t)i * HW] = from_f<T>(acc[blk][ib][e]);
        }
    }
  }
}

namespace {

template <typename F>
int yt_with_type(int dt, F&& f) {
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
int yt_with_mb(int mb, F&& f) {
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

// Output-channel halves per row segment and 16-channel blocks per half.
void yt_split(int64_t c, int& ihalves, int& mb) {
  ihalves = c > 64 ? 2 : 1;
  mb = c > 64 ? 4 : (int)((c + 15) / 16);
}

int64_t yt_pack_bytes(int64_t c, int k, int dtype) {
  int ih, mb;
  yt_split(c, ih, mb);
  const int64_t nc32 = (c + 31) / 32;
  return (int64_t)ih * 3 * nc32 * k * k * mb * (dtype == kF32 ? 2 : 1) * 64 * 16;
}

// Validates the arguments of both dY entry points; kOk, an error, or
// kOk with `empty` set when there is nothing to compute.
int yt_check(const void* x, const void* weight, const void* grad_out, void* grad_y, int64_t n,
             int64_t c, int64_t h, int64_t w, int kernel_size, int d0, int d1, int d2, int dtype,
             GenGeom& gg, bool& empty) {
  empty = false;
  if (dtype < kF32 || dtype > kF16) return kBadArgument;
  int st = gen_make_geom(gg, n, c, h, w, kernel_size, d0, d1, d2);
  if (st != kOk) return st;
  if (n == 0 || c == 0 || h == 0 || w == 0) {
    empty = true;
    return kOk;
  }
  if (!x || !weight || !grad_out || !grad_y) return kBadArgument;
  if (gg.d0 > kYtMaxDil || gg.d1 > kYtMaxDil || gg.d2 > kYtMaxDil) return kUnsupported;
  // 32-bit buffer offsets inside one image's [C][H][W] planes
  if (c * h * w * (dtype == kF32 ? 4 : 2) > 0x7fffffffLL) return kUnsupported;
  if (2 * n * h * ((w + kYtTW - 1) / kYtTW) > 0x7fffffffLL) return kUnsupported;
  return kOk;
}

// Packs the weight into `packed` and launches the dY kernel (arguments
// already validated by yt_check; `packed` holds yt_pack_bytes bytes).
int yt_launch(const void* x, const void* weight, const void* grad_out, void* grad_y, void* packed,
              int64_t n, int64_t c, int64_t h, int64_t w, int kernel_size, const GenGeom& gg,
              int dtype, hipStream_t stream, bool pack = true, const WReduce* red = nullptr);

}  // namespace

// Scratch of the no-allocation entry point: the packed weight, at most
// kYtScratchBytes (enough for every channel count and kernel size the fused
// kernels accept).  Each device holds its own copy for the life of the
// process; host code reaches it only through the address that
// hipGetSymbolAddress returns for the current device.
constexpr int64_t kYtScratchBytes = (int64_t)2 << 20;
static __device__ __align__(256) unsigned char scratch[kYtScratchBytes];

namespace {

constexpr int kYtMaxDevices = 64;
std::atomic<void*> g_scratch[kYtMaxDevices];
std::mutex g_scratch_mu;

// This device's address of `scratch`, looked up once per device.
int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kYtMaxDevices) return kUnsupported;
  void* p = g_scratch[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return (int)e;
      if (p == nullptr) return (int)hipErrorInvalidSymbol;
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return kOk;
}

}  // namespace
}  // namespace ddpm

using namespace ddpm;

extern "C" int64_t ddpm_gen_bwd_y_workspace_bytes(int64_t c, int kernel_size) {
  if (c <= 0 || c > 128 || kernel_size < 1) return 0;
  return yt_pack_bytes(c, kernel_size, kF32);
}

int ddpm::yt_run(const void* x, const void* weight, const void* grad_out, void* grad_y,
                 void* workspace, int64_t workspace_bytes, int64_t n, int64_t c, int64_t h,
                 int64_t w, int kernel_size, int d0, int d1, int d2, int dtype, hipStream_t stream,
                 int mode, YPack* pack, const WReduce* red) {
  GenGeom gg;
  bool empty;
  const int st =
      yt_check(x, weight, grad_out, grad_y, n, c, h, w, kernel_size, d0, d1, d2, dtype, gg, empty);
  if (pack) *pack = YPack{weight, (uint32_t*)workspace, (int)c, (int)((c + 31) / 32), 0};
  if (st != kOk || empty) return st;
  const int64_t need = yt_pack_bytes(c, kernel_size, dtype);
  if (!workspace || workspace_bytes < need) return kWorkspaceTooSmall;
  if (kernel_size != 1 && kernel_size != 3) return kUnsupported;
  if (mode == kYtCheck) {
    if (pack) {
      int ih, mb;
      yt_split(c, ih, mb);
      pack->total = ih * 3 * pack->nc32 * kernel_size * kernel_size * mb * 64;
    }
    return kOk;
  }
  return yt_launch(x, weight, grad_out, grad_y, workspace, n, c, h, w, kernel_size, gg, dtype,
                   stream, mode != kYtMain, red);
}

int ddpm::yt_pack(const YPack& p, int kernel_size, int dtype, hipStream_t stream) {
  int ih, mb;
  yt_split(p.C, ih, mb);
  return yt_with_type(dtype, [&](auto tag) {
    using T = decltype(tag);
    return yt_with_mb(mb, [&](auto mbc) {
      constexpr int MB = decltype(mbc)::value;
      const dim3 grid((unsigned)((p.total + 255) / 256));
      if (kernel_size == 1)
        hipLaunchKernelGGL((gen_pack_wt_kernel<T, 1, MB>), grid, dim3(256), 0, stream,
                           (const T*)p.wt, p.pk, p.C, p.nc32, p.total);
      else
        hipLaunchKernelGGL((gen_pack_wt_kernel<T, 3, MB>), grid, dim3(256), 0, stream,
                           (const T*)p.wt, p.pk, p.C, p.nc32, p.total);
      return (int)hipGetLastError();
    });
  });
}

extern "C" int ddpm_gen_bwd_y(const void* x, const void* weight, const void* grad_out,
                              void* grad_y, void* workspace, int64_t workspace_bytes, int64_t n,
                              int64_t c, int64_t h, int64_t w, int kernel_size, int d0, int d1,
                              int d2, int dtype, hipStream_t stream) {
  return yt_run(x, weight, grad_out, grad_y, workspace, workspace_bytes, n, c, h, w, kernel_size,
                d0, d1, d2, dtype, stream, kYtFull, nullptr);
}

extern "C" int ddpm_gen_bwd_y_noalloc(const void* x, const void* weight, const void* grad_out,
                                      void* grad_y, int64_t n, int64_t c, int64_t h, int64_t w,
                                      int kernel_size, int d0, int d1, int d2, int dtype,
                                      hipStream_t stream) {
  GenGeom gg;
  bool empty;
  int st =
      yt_check(x, weight, grad_out, grad_y, n, c, h, w, kernel_size, d0, d1, d2, dtype, gg, empty);
  if (st != kOk || empty) return st;
  if (yt_pack_bytes(c, kernel_size, dtype) > kYtScratchBytes) return kScratchTooSmall;
  void* packed = nullptr;
  st = scratch_address(&packed);
  if (st != kOk) return st;
  return yt_launch(x, weight, grad_out, grad_y, packed, n, c, h, w, kernel_size, gg, dtype, stream);
}

extern "C" int64_t ddpm_gen_bwd_y_noalloc_scratch_bytes(void) { return kYtScratchBytes; }

namespace ddpm {
namespace {

int yt_launch(const void* x, const void* weight, const void* grad_out, void* grad_y, void* packed,
              int64_t n, int64_t c, int64_t h, int64_t w, int kernel_size, const GenGeom& gg,
              int dtype, hipStream_t stream, bool pack, const WReduce* red) {
  void* workspace = packed;
  YGeom g;
  g.N = (int)n;
  g.C = (int)c;
  g.H = (int)h;
  g.W = (int)w;
  g.d0 = gg.d0;
  g.d1 = gg.d1;
  g.d2 = gg.d2;
  g.col_tiles = (int)((w + kYtTW - 1) / kYtTW);
  g.nc32 = (int)((c + 31) / 32);
  g.x4 = (w % 8 == 0) && ((uintptr_t)x % 16 == 0);
  int mb;
  yt_split(c, g.ihalves, mb);
  const int64_t tiles = n * h * g.col_tiles * g.ihalves;  // below 2^31 (yt_check)
  return yt_with_type(dtype, [&](auto tag) {
    using T = decltype(tag);
    return yt_with_mb(mb, [&](auto mbc) {
      constexpr int MB = decltype(mbc)::value;
      auto launch = [&](auto ks, auto chc) {
        constexpr int KS = decltype(ks)::value;
        constexpr int CH = decltype(chc)::value;
        typedef YtLds<T, KS, MB, CH> L;
        if (pack) {
          const int units = g.ihalves * 3 * g.nc32 * KS * KS * MB * 64;
          hipLaunchKernelGGL((gen_pack_wt_kernel<T, KS, MB>), dim3((units + 255) / 256), dim3(256),
                             0, stream, (const T*)weight, (uint32_t*)workspace, (int)c, g.nc32,
                             units);
          int e = (int)hipGetLastError();
          if (e != 0) return e;
        }
        const size_t lds = (size_t)2 * L::kBuf * 4;
        // aligned layout: 16-byte x rows and whole 32-channel chunks
        auto kern = g.x4 && c % 32 == 0 ? gen_bwd_y_kernel<T, KS, MB, CH, true>
                                        : gen_bwd_y_kernel<T, KS, MB, CH>;
        const int ae = allow_dynamic_lds(reinterpret_cast<const void*>(kern), lds);
        if (ae != 0) return ae;
        const WReduce nored{nullptr, nullptr, nullptr, nullptr, 0, 0, 0, 0, 0};
        hipLaunchKernelGGL(kern, dim3((unsigned)tiles), dim3(kYtThreads), lds, stream, (const T*)x,
                           (const uint32_t*)workspace, (const T*)grad_out, (T*)grad_y, g,
                           red ? *red : nored);
        return (int)hipGetLastError();
      };
      auto by_ch = [&](auto ks) {
        // 2-byte types with an even chunk count: two chunks per stage
        if constexpr (sizeof(T) == 2) {
          if (g.nc32 % 2 == 0) return launch(ks, std::integral_constant<int, 2>());
        }
        return launch(ks, std::integral_constant<int, 1>());
      };
      if (kernel_size == 1) return by_ch(std::integral_constant<int, 1>());
      if (kernel_size == 3) return by_ch(std::integral_constant<int, 3>());
      return (int)kUnsupported;
    });
  });
}

}  // namespace
}  // namespace ddpm
