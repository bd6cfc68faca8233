// Shared device helpers for the compact_amd HIP kernels (gfx950 / CDNA4).
//
// Numeric conventions every kernel here relies on (they decide bit-exactness
// of the quantised cache against the reference's PyTorch codec,
// src/flashffn.py:1055-1110):
//   * float division is IEEE correctly rounded (hipcc's default
//     -fhip-fp32-correctly-rounded-divide-sqrt; the build passes it explicitly);
//   * fp32 denormals are kept (-fno-gpu-flush-denormals-to-zero);
//   * no FMA contraction in the codec/GLU file (-ffp-contract=off);
//   * rint is v_rndne_f32 (round half to even), fp16 conversion is
//     v_cvt_f16_f32 in the default round-to-nearest-even mode;
//   * bf16 rounding is v_cvt_pk_bf16_f32 (round to nearest even, like
//     c10::BFloat16 for every non-NaN value).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cpt {

// dtype codes of the C ABI (include/compact_amd.h)
enum DType : int { kF32 = 0, kF16 = 1, kBF16 = 2 };

// status codes of the C ABI
enum Status : int {
  kOk = 0,
  kErrBits = 1,          // bits not in {4, 8}
  kErrRagged = 2,        // D % group_size != 0
  kErrGroupPow2 = 3,     // group_size not a positive power of two
  kErrShape = 4,         // negative or inconsistent sizes / null pointer
  kErrDType = 5,         // unsupported dtype code
  kErrLaunch = 6,        // hipLaunchKernel / hipGetLastError failure
  kErrAlign = 7,         // pointer alignment the kernel requires is not met
  kErrTooLarge = 8,      // size beyond what the kernel indexes
};

__device__ __forceinline__ float bf16_to_f32(uint32_t b16) {
  return __uint_as_float(b16 << 16);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// bf16 round-to-nearest-even of two floats, packed (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  bf16x2_t v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) { return pack_bf16x2(f, 0.0f) & 0xFFFFu; }

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// Load / store one element of a storage dtype as float32.
template <int DT> struct Elem;
template <> struct Elem<kF32> {
  using T = float;
  static __device__ __forceinline__ float ld(const T* p) { return *p; }
  static __device__ __forceinline__ void st(T* p, float v) { *p = v; }
};
template <> struct Elem<kF16> {
  using T = uint16_t;
  static __device__ __forceinline__ float ld(const T* p) { return f16_bits_to_f32(*p); }
  static __device__ __forceinline__ void st(T* p, float v) { *p = f32_to_f16_bits(v); }
};
template <> struct Elem<kBF16> {
  using T = uint16_t;
  static __device__ __forceinline__ float ld(const T* p) { return bf16_to_f32(*p); }
  static __device__ __forceinline__ void st(T* p, float v) { *p = (uint16_t)f32_to_bf16_bits(v); }
};

// Eight consecutive elements of a storage dtype <-> float[8], using 128-bit
// accesses (two for float32).  Callers guarantee 16-byte alignment.
template <int DT> struct Vec8;
template <> struct Vec8<kF32> {
  static __device__ __forceinline__ void ld(const void* base, int64_t i8, float v[8]) {
    const float4* p = reinterpret_cast<const float4*>(base) + 2 * i8;
    float4 a = p[0], b = p[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
  static __device__ __forceinline__ void st(void* base, int64_t i8, const float v[8]) {
    float4* p = reinterpret_cast<float4*>(base) + 2 * i8;
    p[0] = make_float4(v[0], v[1], v[2], v[3]);
    p[1] = make_float4(v[4], v[5], v[6], v[7]);
  }
};
template <int DT> struct Vec8Half {  // 16-bit formats
  static __device__ __forceinline__ void ld(const void* base, int64_t i8, float v[8]) {
    uint4 w = reinterpret_cast<const uint4*>(base)[i8];
    uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (DT == kBF16) {
        v[2 * j] = __uint_as_float(ws[j] << 16);
        v[2 * j + 1] = __uint_as_float(ws[j] & 0xFFFF0000u);
      } else {
        v[2 * j] = f16_bits_to_f32((uint16_t)(ws[j] & 0xFFFFu));
        v[2 * j + 1] = f16_bits_to_f32((uint16_t)(ws[j] >> 16));
      }
    }
  }
  static __device__ __forceinline__ void st(void* base, int64_t i8, const float v[8]) {
    uint32_t ws[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (DT == kBF16) {
        ws[j] = pack_bf16x2(v[2 * j], v[2 * j + 1]);
      } else {
        ws[j] = (uint32_t)f32_to_f16_bits(v[2 * j]) | ((uint32_t)f32_to_f16_bits(v[2 * j + 1]) << 16);
      }
    }
    reinterpret_cast<uint4*>(base)[i8] = make_uint4(ws[0], ws[1], ws[2], ws[3]);
  }
};
template <> struct Vec8<kF16> : Vec8Half<kF16> {};
template <> struct Vec8<kBF16> : Vec8Half<kBF16> {};

__host__ __device__ __forceinline__ bool is_pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }

// Unsigned 32-bit division by a run-time invariant divisor with one multiply-high
// (Granlund & Montgomery, "Division by Invariant Integers using Multiplication",
// PLDI 1994, section 4): l = ceil(log2 d), m = floor(2^32 (2^l - d) / d) + 1,
// n / d = (t + ((n - t) >> 1)) >> (l - 1) with t = mulhi(m, n); exact for all
// 32-bit n and d >= 1.
struct FastDivU32 {
  uint32_t d = 1, m = 1;
  int l = 0;
  __host__ static FastDivU32 make(uint32_t divisor) {
    FastDivU32 f;
    f.d = divisor;
    int l = 0;
    while ((1ull << l) < divisor) ++l;
    f.l = l;
    f.m = (uint32_t)((((1ull << 32) * ((1ull << l) - divisor)) / divisor) + 1);
    return f;
  }
  __device__ __forceinline__ uint32_t div(uint32_t n) const {
    if (d == 1) return n;
    const uint32_t t = __umulhi(m, n);
    return (t + ((n - t) >> 1)) >> (l - 1);
  }
};

__host__ __forceinline__ bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

}  // namespace cpt
