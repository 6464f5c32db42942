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

enum DType : int { kF32 = 0, kBF16 = 1, kF16 = 2 };

// Error codes returned next to hipError_t values (chosen above hipError_t's range).
enum Status : int {
  kOk = 0,
  kBadArgument = 10001,
  kUnsupported = 10002,
  kWorkspaceTooSmall = 10003,
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
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const bf16 h = (bf16)v[e];
      o[0][e] = h;
      o[1][e] = (bf16)(v[e] - (float)h);
    }
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
#pragma unroll
    for (int e = 0; e < 8; ++e) o[0][e] = (bf16)v[e];
  }
  static __device__ __forceinline__ f32x4 mac(const V (&a)[1], const V (&b)[1], f32x4 acc) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b[0], acc, 0, 0, 0);
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
  static __device__ __forceinline__ f32x4 mac(const V (&a)[1], const V (&b)[1], f32x4 acc) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a[0], b[0], acc, 0, 0, 0);
  }
};

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

}  // namespace ddpm
