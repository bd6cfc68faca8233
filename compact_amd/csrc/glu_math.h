// Elementwise math shared by the standalone codec/GLU kernels (codec.hip) and
// the fused GEMM epilogues (gemm.hip).  Both include this one definition, so a
// fused kernel and its unfused composition agree bit for bit.
//
// References (SDMuhsin/CompAct): GLU forward src/flashffn.py:71-76, backward
// :109-123, codec :1071-1088 (quantise) and :1099-1110 (dequantise), the
// bf16 round trip of the dequantised cache :1251-1253.
#pragma once

#include <type_traits>

#include "common.h"

namespace cpt {

// sigmoid(x) = 1 / (1 + e^-x) on the transcendental unit: v_exp_f32 (2^x) and
// v_rcp_f32, each about 1 ulp.  Large |x| saturate to exactly 0 or 1.
__device__ __forceinline__ float sigmoid_f32(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.4426950408889634f));
}

// float -> bf16 -> float
__device__ __forceinline__ float round_bf16(float x) {
  return __uint_as_float(pack_bf16x2(x, 0.0f) << 16);
}

// GLU forward of one element: (g * sigmoid(g)) * u
__device__ __forceinline__ float silu_mul1(float g, float u) { return (g * sigmoid_f32(g)) * u; }

// GLU backward of one element (op order of the reference's _swiglu_bwd_kernel).
__device__ __forceinline__ void swiglu_bwd1(float dh, float g, float u, float& dg, float& du,
                                            float& hact) {
  const float sig = sigmoid_f32(g);
  hact = g * sig;
  const float grad_h_act = dh * u;
  du = dh * hact;
  const float dsilu = sig * (1.0f + g * (1.0f - sig));
  dg = grad_h_act * dsilu;
}

// Max over each aligned group of LPG lanes (LPG a power of two <= 64), every
// lane of a group receiving it.  Up to 16 lanes it is a DPP butterfly inside
// the 16-lane row, VALU only: swap neighbours, swap pairs (quad_perm
// [1,0,3,2], [2,3,0,1]), then mirror within 8 and within 16 lanes
// (row_half_mirror, row_mirror), each step pairing every lane with one from
// the other half of its growing group.  Wider groups add ds_bpermute
// exchanges (__shfl_xor) across rows.
template <int LPG>
__device__ __forceinline__ uint32_t group_max_u32(uint32_t v) {
  static_assert(LPG >= 1 && LPG <= 64 && (LPG & (LPG - 1)) == 0, "group of 1..64 lanes");
  auto dpp_max = [](uint32_t x, auto ctrl) {
    return max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, decltype(ctrl)::value, 0xF,
                                                        0xF, false));
  };
  if constexpr (LPG >= 2) v = dpp_max(v, std::integral_constant<int, 0xB1>{});   // quad_perm [1,0,3,2]
  if constexpr (LPG >= 4) v = dpp_max(v, std::integral_constant<int, 0x4E>{});   // quad_perm [2,3,0,1]
  if constexpr (LPG >= 8) v = dpp_max(v, std::integral_constant<int, 0x141>{});  // row_half_mirror
  if constexpr (LPG >= 16) v = dpp_max(v, std::integral_constant<int, 0x140>{}); // row_mirror
#pragma unroll
  for (int off = 16; off < LPG; off <<= 1) v = max(v, (uint32_t)__shfl_xor((int)v, off));
  return v;
}

template <int BITS> struct QMax;
template <> struct QMax<4> { static constexpr float v = 7.0f; };
template <> struct QMax<8> { static constexpr float v = 127.0f; };

// scale = fp16(fp32(absmax / qmax))  (absmax given as the bits of |x|).
// Fast path: y = absmax * fp32(1/qmax) and the correctly rounded quotient are
// each within 1 fp32 ulp of the exact one, so within 2 ulp of each other.
// They round to the same fp16 unless an fp16 rounding midpoint lies between
// them: in fp16's normal range, where the 13 fp32 mantissa bits below fp16's
// read 0x1000 at a midpoint, y more than 4 ulp from that pattern decides.
// Elsewhere (fp16 subnormal or overflow range, NaN) and near a midpoint
// (about one group in a thousand) the division decides.
template <int BITS>
__device__ __forceinline__ uint16_t scale_bits(uint32_t absmax_bits) {
  const float a = __uint_as_float(absmax_bits);
  float y = a * (1.0f / QMax<BITS>::v);
  const uint32_t b = __float_as_uint(y);
  const uint32_t ex = b >> 23;                      // y >= 0: the biased exponent
  const int low = (int)(b & 0x1FFFu) - 0x1000;
  if (!(ex >= 113u && ex <= 142u && (low > 4 || low < -4))) y = a / QMax<BITS>::v;
  return f32_to_f16_bits(y);
}

// safe = scale > 0 ? scale : 1
__device__ __forceinline__ float safe_scale(uint16_t sh) {
  const float s = f16_bits_to_f32(sh);
  return s > 0.0f ? s : 1.0f;
}

// code = clamp(rint(fp32(v / safe)), -qmax, qmax), the reference's definition.
// Fast path: q = v * rcp(safe).  Every quotient here has |v / safe| < 256
// (at most qmax * 1.5, reached with fp16-subnormal scales), where
// |q - v/safe| <= 2^-14 and |fp32(v/safe) - v/safe| <= 2^-17.  So whenever q
// is farther than 2^-12 from a half-integer, rint(q) == rint(fp32(v/safe)).
// Otherwise (rare) the correctly rounded division decides.  safe = inf gives
// rcp = 0 and code 0, as v / inf does.
template <int BITS>
__device__ __forceinline__ int quant_code(float v, float safe, float rsafe) {
  const float q = v * rsafe;
  float r = __builtin_rintf(q);
  if (__builtin_fabsf(q - r) > 0.5f - 0.000244140625f) r = __builtin_rintf(v / safe);
  r = fminf(fmaxf(r, -QMax<BITS>::v), QMax<BITS>::v);
  return (int)r;
}

// quant_code as a clamped integral float (the form the byte packers take).
template <int BITS>
__device__ __forceinline__ float quant_rint(float v, float safe, float rsafe) {
  const float q = v * rsafe;
  float r = __builtin_rintf(q);
  if (__builtin_fabsf(q - r) > 0.5f - 0.000244140625f) r = __builtin_rintf(v / safe);
  return fminf(fmaxf(r, -QMax<BITS>::v), QMax<BITS>::v);
}

// Codes of bf16 values with no division and no fallback: the same codes as
// quant_rint, from v * rcp(safe) rounded twice.
//   (1) y = fma(v, rs, 3072): the exact product, rounded once onto the
//       2^-12 grid (fp32 values in [2048, 4096) are the multiples of 2^-12;
//       |v * rs| < 256 keeps y inside).
//   (2) z = y + (1.5 * 2^23 - 3072 + off) = 1.5 * 2^23 + off + rint(y - 3072),
//       exactly: fp32 values in [2^23, 2^24) are the integers, and the sum is
//       rounded to nearest even.
// Why rint(y - 3072) = rint(fp32(v / safe)).  Write v = m_v 2^a (integer
// m_v < 256, v bf16) and safe = m_s 2^b (integer 1 <= m_s < 2048, safe fp16
// or 1).  For a half-integer h >= 1/2, v / safe - h = (2 m_v 2^(a-b) -
// (2k+1) m_s) / (2 m_s).  If a - b >= -1 the numerator is an integer, so
// v / safe is h or at least 1 / 4094 from it.  If a - b <= -2 it is a
// multiple of 2^(a-b+1), and v / safe > 1/2 - 2^-12 forces 2^(a-b) >
// m_s / 511, so the distance is 0 or above 1/511.  Quotients here satisfy
// |v / safe| < 256 (at most 1.5 qmax, with fp16-subnormal scales), and rs =
// v_rcp_f32(safe) is within 1 ulp of 1 / safe, so |v * rs - v / safe| <=
// 2^-15.  A tie (v / safe = h) then lies within 2^-15 < 2^-13 of the grid
// point h and (1) returns h exactly, whose rint in (2) is round-half-even,
// as rint of the exact fp32 quotient h.  Any other quotient lies at least
// 1/4094 - 2^-15 > 2^-13 from every h, so (1) keeps it on its side of each
// h, as does fp32's own rounding of the quotient (at most 2^-17): both
// rints agree.  An exhaustive check over every bf16 v and fp16 scale, with
// rs up to 2 ulp off, is in tests/quant_snap_check.c.  Not valid for fp16 or
// fp32 inputs (more significant bits close the gap).
//
// z stays an fp32, clamped to the code range; its low byte is then the
// stored byte: int8 off = 0, the two's complement of the code (1.5 * 2^23
// has 22 zero low bits); int4 off = 8, code + 8.
template <int BITS>
__device__ __forceinline__ void quant_snap8(const float v[8], float rs, float z[8]) {
  constexpr float kGrid = 3072.0f;
  constexpr float kInt = 12582912.0f;                   // 1.5 * 2^23
  constexpr float kOff = BITS == 4 ? 8.0f : 0.0f;
  constexpr float kLo = kInt + kOff - QMax<BITS>::v, kHi = kInt + kOff + QMax<BITS>::v;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float y = __builtin_fmaf(v[e], rs, kGrid);
    z[e] = fminf(fmaxf(y + (kInt - kGrid + kOff), kLo), kHi);
  }
}

// Byte 0 of each of four words, in order, as one word.
__device__ __forceinline__ uint32_t low_bytes4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  // v_perm_b32 (S0, S1, sel): selectors 0-3 pick bytes of S1, 4-7 of S0,
  // 0x0C gives a zero byte
  const uint32_t ab = __builtin_amdgcn_perm(b, a, 0x0C0C0400u);
  const uint32_t cd = __builtin_amdgcn_perm(d, c, 0x0C0C0400u);
  return __builtin_amdgcn_perm(cd, ab, 0x05040100u);
}

// quant_snap8's eight values packed as stored (same bytes as pack_codes8_*).
__device__ __forceinline__ uint2 pack_snap8_int8(const float z[8]) {
  uint32_t b[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) b[e] = __float_as_uint(z[e]);
  return make_uint2(low_bytes4(b[0], b[1], b[2], b[3]), low_bytes4(b[4], b[5], b[6], b[7]));
}

__device__ __forceinline__ uint32_t pack_snap8_int4(const float z[8]) {
  // byte 0 of (odd << 4) | even: the even column's code + 8 in the low
  // nibble, the odd one's in the high nibble
  uint32_t p[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = (__float_as_uint(z[2 * i + 1]) << 4) | __float_as_uint(z[2 * i]);
  return low_bytes4(p[0], p[1], p[2], p[3]);
}

// Eight codes (quant_rint's integral floats) packed as stored
// (src/flashffn.py:1081-1085).  int4: byte b holds column 2b in its low
// nibble and 2b + 1 in its high one, each as code + 8; the byte's value
// r[2b] + 16 r[2b+1] + 136 is a small integer, exact in fp32, and
// v_cvt_pk_u8_f32 writes it into byte b.  int8: code + 128 as an unsigned
// byte, then XOR 0x80 turns it into the two's complement byte of the code.
__device__ __forceinline__ uint32_t pack_codes8_int4(const float r[8]) {
  uint32_t w = 0;
#pragma unroll
  for (int b = 0; b < 4; ++b)
    w = __builtin_amdgcn_cvt_pk_u8_f32(__builtin_fmaf(r[2 * b + 1], 16.0f, r[2 * b]) + 136.0f,
                                       b, w);
  return w;
}

__device__ __forceinline__ uint2 pack_codes8_int8(const float r[8]) {
  uint32_t w0 = 0, w1 = 0;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    w0 = __builtin_amdgcn_cvt_pk_u8_f32(r[b] + 128.0f, b, w0);
    w1 = __builtin_amdgcn_cvt_pk_u8_f32(r[4 + b] + 128.0f, b, w1);
  }
  return make_uint2(w0 ^ 0x80808080u, w1 ^ 0x80808080u);
}

}  // namespace cpt
