// Shared device helpers for the DDPM HIP kernels (gfx950 / CDNA4).
//
// Conventions used by every kernel in this library:
//   x, y, dX, dY          [N][C][H][W]
//   kernels, dK           [N][3][C][K*K][H][W]     row o = (b*C + c)*K*K + tap
//   weight                [3*C*K*K][C] (Conv2d 1x1 layout, trailing 1x1 dropped)
//   cat / grad_cat        [N][4*C][H][W] = [x, d0, d1, d2]
//   tap = ki*K + kj; neighbour of (h,w) at dilation d is (h+(ki-r)d, w+(kj-r)d),
//   r = K/2, zero outside the image.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ddpm {

typedef __bf16 bf16;
typedef _Float16 f16;
typedef bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

enum DType : int { kF32 = 0, kBF16 = 1, kF16 = 2, kF32Pairs = 3 };
// kF32Pairs: fp32 data whose 4C-plane concat is stored as bf16 (hi, lo) pair
// planes -- per 32-plane chunk, plane j < 16 holds the hi halves of channels
// (2j, 2j+1) (low / high 16 bits) and plane 16 + j their lo halves (hi = the
// top 16 bits of the fp32 pattern, lo = the remainder rounded to nearest
// even): the same bytes as the fp32 concat, already split the way the fp32
// MFMA path splits its operands.

// Error codes returned next to hipError_t values (chosen above hipError_t's range).
enum Status : int {
  kOk = 0,
  kBadArgument = 10001,
  kUnsupported = 10002,
  kWorkspaceTooSmall = 10003,
  kScratchTooSmall = 10004,  // shape exceeds a no-allocation entry point's fixed scratch
};

template <typename T>
__device__ __forceinline__ float to_f(T v) {
  return (float)v;
}
template <typename T>
__device__ __forceinline__ T from_f(float v) {
  return (T)v;  // round-to-nearest-even for bf16 and f16 (v_cvt_pk_bf16_f32 / v_cvt_f16_f32)
}
// Rounds a generated tap to the storage precision, as the 1x1 generator's
// output tensor would hold it (fp32: unchanged).
template <typename T>
__device__ __forceinline__ float quant(float v) {
  return (float)(T)v;
}
template <>
__device__ __forceinline__ float quant<float>(float v) {
  return v;
}

// quant() of four values: for bf16 two v_cvt_pk_bf16_f32 and four widening
// shifts / masks (6 instructions where four separate roundings take 8).
template <typename T>
__device__ __forceinline__ void quant4(const f32x4& v, float (&q)[4]);

// Two fp32 values rounded to nearest-even bf16, packed low/high
// (one v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  const bf16x2 r = __builtin_convertvector((f32x2){a, b}, bf16x2);
  return __builtin_bit_cast(uint32_t, r);
}

template <typename T>
__device__ __forceinline__ void quant4(const f32x4& v, float (&q)[4]) {
  if constexpr (__is_same(T, bf16)) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t p = pack_bf16x2(v[2 * h], v[2 * h + 1]);
      q[2 * h] = __uint_as_float(p << 16);
      q[2 * h + 1] = __uint_as_float(p & 0xffff0000u);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) q[e] = quant<T>(v[e]);
  }
}

// Splits two fp32 values into bf16 pairs hi + lo with a ~= hi_a + lo_a:
// hi keeps the top 16 bits of the fp32 pattern (so a - hi is exact in fp32)
// and lo is that remainder rounded to nearest-even bf16; |a - hi - lo| <=
// 2^-17 |a|.  Six VALU instructions per pair (2 and, perm, 2 sub, cvt_pk).
__device__ __forceinline__ void split_bf16x2(float a, float b, uint32_t& hi, uint32_t& lo) {
  const uint32_t ua = __float_as_uint(a), ub = __float_as_uint(b);
  hi = __builtin_amdgcn_perm(ub, ua, 0x07060302u);  // [hi16(a) | hi16(b) << 16]
  const float la = a - __uint_as_float(ua & 0xffff0000u);
  const float lb = b - __uint_as_float(ub & 0xffff0000u);
  lo = pack_bf16x2(la, lb);
}

// ---------------------------------------------------------------------------
// MFMA 16x16x32 (gfx950), lane layout (verified on the device):
//   A (16x32): lane l holds A[l&15][8*(l>>4) + e], e=0..7
//   B (32x16): lane l holds B[8*(l>>4) + e][l&15]
//   D (16x16): lane l holds D[4*(l>>4) + r][l&15],  r=0..3
// fp32 operands run as three bf16 products (hi*hi + hi*lo + lo*hi), each
// split exact to ~2^-17 relative; bf16 / f16 operands run one product.
// ---------------------------------------------------------------------------
template <typename T>
struct Mma;

template <>
struct Mma<float> {
  static constexpr int P = 2;
  typedef bf16 E;
  typedef bf16x8 V;
  static __device__ __forceinline__ void pack(const float (&v)[8], V (&o)[2]) {
    uint32_t hi[4], lo[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) split_bf16x2(v[2 * e], v[2 * e + 1], hi[e], lo[e]);
    o[0] = __builtin_bit_cast(V, (u32x4){hi[0], hi[1], hi[2], hi[3]});
    o[1] = __builtin_bit_cast(V, (u32x4){lo[0], lo[1], lo[2], lo[3]});
  }
  // one product of single parts (for operands exact in bf16)
  static __device__ __forceinline__ f32x4 mac1(V a, V b, f32x4 acc) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mac(const V (&a)[2], const V (&b)[2], f32x4 acc) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[1], b[0], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b[1], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b[0], acc, 0, 0, 0);
    return acc;
  }
};

template <>
struct Mma<bf16> {
  static constexpr int P = 1;
  typedef bf16 E;
  typedef bf16x8 V;
  static __device__ __forceinline__ void pack(const float (&v)[8], V (&o)[1]) {
    u32x4 p;
#pragma unroll
    for (int e = 0; e < 4; ++e) p[e] = pack_bf16x2(v[2 * e], v[2 * e + 1]);
    o[0] = __builtin_bit_cast(V, p);
  }
  static __device__ __forceinline__ f32x4 mac1(V a, V b, f32x4 acc) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mac(const V (&a)[1], const V (&b)[1], f32x4 acc) {
    return mac1(a[0], b[0], acc);
  }
};

template <>
struct Mma<f16> {
  static constexpr int P = 1;
  typedef f16 E;
  typedef f16x8 V;
  static __device__ __forceinline__ void pack(const float (&v)[8], V (&o)[1]) {
#pragma unroll
    for (int e = 0; e < 8; ++e) o[0][e] = (f16)v[e];
  }
  static __device__ __forceinline__ f32x4 mac1(V a, V b, f32x4 acc) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mac(const V (&a)[1], const V (&b)[1], f32x4 acc) {
    return mac1(a[0], b[0], acc);
  }
};

// ---------------------------------------------------------------------------
// Column shift of a B fragment held as 16-column blocks (B lane l holds
// column l & 15 of its block): the fragment of the block `own` moved by S
// columns (|S| <= 15), each lane taking lane n + S of its 16-lane row (DPP
// row_shl / row_shr) and the lanes past the row's end the neighbouring
// block's (`next` for S > 0, `prev` for S < 0) by a row rotation (row_ror),
// whose result stays in place where the shift has no source lane
// (bound_ctrl off).  One dword of the fragment per call.
// ---------------------------------------------------------------------------
template <int S>
__device__ __forceinline__ uint32_t lane_shift(uint32_t prev, uint32_t own, uint32_t next) {
  static_assert(S >= -15 && S <= 15, "one 16-lane row at most");
  if constexpr (S == 0) {
    (void)prev;
    (void)next;
    return own;
  } else if constexpr (S > 0) {
    (void)prev;
    const int end = __builtin_amdgcn_update_dpp(0, (int)next, 0x120 + (16 - S), 0xf, 0xf, false);
    return (uint32_t)__builtin_amdgcn_update_dpp(end, (int)own, 0x100 + S, 0xf, 0xf, false);
  } else {
    (void)next;
    const int end = __builtin_amdgcn_update_dpp(0, (int)prev, 0x120 - S, 0xf, 0xf, false);
    return (uint32_t)__builtin_amdgcn_update_dpp(end, (int)own, 0x110 - S, 0xf, 0xf, false);
  }
}

// ---------------------------------------------------------------------------
// Vector loads/stores of VEC consecutive elements as fp32 (VEC in {1,2,4,8}).
// Callers guarantee alignment of VEC*sizeof(T) bytes when VEC > 1.
// ---------------------------------------------------------------------------
template <typename T, int VEC>
struct VecIO {
  static __device__ __forceinline__ void load(const T* p, float (&v)[VEC]) {
    if constexpr (VEC == 1) {
      v[0] = to_f(p[0]);
    } else {
      typedef T TV __attribute__((ext_vector_type(VEC)));
      const TV t = *reinterpret_cast<const TV*>(p);
#pragma unroll
      for (int e = 0; e < VEC; ++e) v[e] = to_f(t[e]);
    }
  }
  // Non-temporal variant for data read exactly once (streamed kernel planes):
  // keeps them from displacing reused lines in L2 / MALL.
  static __device__ __forceinline__ void load_nt(const T* p, float (&v)[VEC]) {
    if constexpr (VEC == 1) {
      v[0] = to_f(__builtin_nontemporal_load(p));
    } else {
      typedef T TV __attribute__((ext_vector_type(VEC)));
      const TV t = __builtin_nontemporal_load(reinterpret_cast<const TV*>(p));
#pragma unroll
      for (int e = 0; e < VEC; ++e) v[e] = to_f(t[e]);
    }
  }
  static __device__ __forceinline__ void store_nt(T* p, const float (&v)[VEC]) {
    if constexpr (VEC == 1) {
      __builtin_nontemporal_store(from_f<T>(v[0]), p);
    } else {
      typedef T TV __attribute__((ext_vector_type(VEC)));
      TV t;
#pragma unroll
      for (int e = 0; e < VEC; ++e) t[e] = from_f<T>(v[e]);
      __builtin_nontemporal_store(t, reinterpret_cast<TV*>(p));
    }
  }
  static __device__ __forceinline__ void store(T* p, const float (&v)[VEC]) {
    if constexpr (VEC == 1) {
      p[0] = from_f<T>(v[0]);
    } else {
      typedef T TV __attribute__((ext_vector_type(VEC)));
      TV t;
#pragma unroll
      for (int e = 0; e < VEC; ++e) t[e] = from_f<T>(v[e]);
      *reinterpret_cast<TV*>(p) = t;
    }
  }
};

// ---------------------------------------------------------------------------
// Buffer loads (gfx9 raw buffers): a load whose byte offset is at or beyond
// the resource's num_records returns zero, so out-of-image pixels, padded
// channels and halo columns are read branch-free by pointing their offset
// past the end (kOob) or by giving a whole row num_records = 0.
// ---------------------------------------------------------------------------
typedef __amdgpu_buffer_rsrc_t BufRes;
constexpr uint32_t kOob = 0x80000000u;

// Cache-policy operand of the raw buffer store builtins selecting a
// non-temporal (streaming) store on gfx950: for output planes that a kernel
// writes once, in whole 128-byte lines, and does not read back (stores of
// partial lines -- the 64- and 32-byte pixel runs of the fused forward's
// fragment-shaped stores -- measured 25-37% more HBM write bytes with it).
constexpr int kNtStore = 2;

__device__ __forceinline__ BufRes make_buf(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// `soff`: a wave-uniform part of the offset, added in the load's scalar
// offset (no vector instruction); with off = kOob the sum stays past the end.
template <typename T>
__device__ __forceinline__ float buf_load1(BufRes r, uint32_t off, uint32_t soff = 0) {
  if constexpr (sizeof(T) == 4) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, soff, 0));
  } else {
    const unsigned short s = __builtin_amdgcn_raw_buffer_load_b16(r, off, soff, 0);
    return to_f(__builtin_bit_cast(T, s));
  }
}

// Buffer stores follow the same rule: a store at or beyond num_records is
// dropped, so masked lanes write nothing without a branch.
template <typename T, int AUX = 0>
__device__ __forceinline__ void buf_store1(BufRes r, uint32_t off, float v) {
  if constexpr (sizeof(T) == 4) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, off, 0, AUX);
  } else {
    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, from_f<T>(v)), r, off,
                                          0, AUX);
  }
}

// 8 consecutive elements at byte offset `off` (16-byte aligned for 2-byte
// types, 16-byte aligned pairs for fp32), converted to fp32.
template <typename T>
__device__ __forceinline__ void buf_load8(BufRes r, uint32_t off, float (&v)[8]) {
  if constexpr (sizeof(T) == 4) {
    const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    const u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(r, off + 16u, 0, 0);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = __uint_as_float(a[e]);
      v[4 + e] = __uint_as_float(b[e]);
    }
  } else {
    typedef T T8 __attribute__((ext_vector_type(8)));
    const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    const T8 t = __builtin_bit_cast(T8, a);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = to_f(t[e]);
  }
}

// Workgroup barrier for loops whose waves exchange data through LDS only:
// waits for this wave's LDS (and scalar) operations, then s_barrier.
// __syncthreads() also waits for every outstanding global load and store
// (vmcnt(0)), which would stall each step on stores and on loads that are
// only consumed later; the compiler still waits for a global load before the
// first use of its register.  The empty asm statements keep the compiler
// from moving memory accesses across the barrier.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);  // vmcnt(63) expcnt(7) lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Workgroups are dispatched round-robin over the 8 XCDs (each with its own L2).
// Remap the hardware block id so that each XCD receives one contiguous range of
// logical block ids: neighbouring spatial tiles (which share halo rows) then
// run on the same XCD and hit the same L2.
__device__ __forceinline__ int xcd_remap(int bid, int total) {
  const int xcd = bid & 7;
  const int idx = bid >> 3;
  const int per = total >> 3;
  const int rem = total & 7;
  return xcd * per + (xcd < rem ? xcd : rem) + idx;
}

__device__ __forceinline__ int dil_of(int b, int d0, int d1, int d2) {
  return b == 0 ? d0 : (b == 1 ? d1 : d2);
}

// Host: lets kernel `fn` launch with `bytes` of dynamic LDS (up to the 160 KB
// of a gfx950 CU) on the current device.  hipFuncSetAttribute runs only the
// first time a (kernel, device) pair needs more than the limit already set,
// not on every launch.  Returns 0 or the hipError_t of the attribute call.
int allow_dynamic_lds(const void* fn, size_t bytes);

}  // namespace ddpm
