// Memory-bound kernels of the FlashFFN v3 hot path for gfx950:
//   * per-group absmax codec (quantise / dequantise)           ref src/flashffn.py:1055-1110
//   * K1: SiLU(g)*u + codec of both g and u in one pass         ref src/flashffn.py:1149-1225
//   * K2: dequantise + SwiGLU backward (+ h_mid^)              ref src/flashffn.py:1228-1300
//   * plain GLU forward / backward / in-place backward         ref src/flashffn.py:50-198
//
// Layout: every tensor is row-major and contiguous.  Because D is a multiple
// of the group size, a group never straddles a row, so the kernels treat an
// [N, D] tensor as a flat array and a group as group_size consecutive
// elements; scales are the flat [N * D / group_size] array.
//
// Fast path: one thread owns 8 consecutive elements (one 128-bit load of a
// bf16 tensor), a group of 8..512 elements is owned by group_size/8
// consecutive lanes of one wavefront, and the group absmax is reduced with
// lane shuffles.  The absmax is taken as an unsigned max over the bit
// patterns with the sign cleared: for non-negative floats that order is the
// float order, so the reduction is exact and order independent.
// Generic path (any dtype / alignment / group size): one thread per group.

#include "common.h"
#include "compact_amd.h"
#include "glu_math.h"

namespace cpt {

constexpr int kBlock = 256;

// Codes of 8 consecutive elements as floats.
template <int BITS>
__device__ __forceinline__ void load_codes8(const uint8_t* q, int64_t c, float code[8]) {
  if (BITS == 8) {
    uint2 w = reinterpret_cast<const uint2*>(q)[c];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      code[j] = (float)(int8_t)((w.x >> (8 * j)) & 0xFFu);
      code[4 + j] = (float)(int8_t)((w.y >> (8 * j)) & 0xFFu);
    }
  } else {
    uint32_t w = reinterpret_cast<const uint32_t*>(q)[c];
#pragma unroll
    for (int j = 0; j < 8; ++j) code[j] = (float)((w >> (4 * j)) & 0xFu) - 8.0f;
  }
}

// Group absmax over LPG consecutive lanes (LPG a power of two <= 64).
template <int LPG>
__device__ __forceinline__ uint32_t group_absmax8(const float v[8]) {
  uint32_t am = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) am = max(am, __float_as_uint(v[j]) & 0x7FFFFFFFu);
  return group_max_u32<LPG>(am);
}

// Quantisation of the 8 elements a thread owns (lane 0 of each group writes
// the scale) in two steps, so that a kernel can form every output before it
// stores any: on gfx950 a wait for a load also waits for the stores issued
// before it (one counter for both), so loads consumed after a store stall on
// that store.  Codes packed as stored: int8 -> 8 bytes, int4 -> 4 bytes of
// (code+8) nibbles, even column low (src/flashffn.py:1081-1085).
struct QuantChunk {
  uint16_t sh;      // fp16 scale bits of the group
  uint32_t w0, w1;  // packed codes (int4: w0; int8: w0, w1)
};

// BF16_IN: the values are bf16, so the division-free quant_snap8 applies.
template <int BITS, int LPG, bool BF16_IN>
__device__ __forceinline__ QuantChunk quant_form(const float v[8]) {
  QuantChunk r;
  r.sh = scale_bits<BITS>(group_absmax8<LPG>(v));
  const float safe = safe_scale(r.sh), rs = __builtin_amdgcn_rcpf(safe);
  if constexpr (BF16_IN) {
    float z[8];
    quant_snap8<BITS>(v, rs, z);
    if (BITS == 8) {
      const uint2 w = pack_snap8_int8(z);
      r.w0 = w.x;
      r.w1 = w.y;
    } else {
      r.w0 = pack_snap8_int4(z);
      r.w1 = 0;
    }
    return r;
  }
  float code[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) code[e] = quant_rint<BITS>(v[e], safe, rs);
  if (BITS == 8) {
    const uint2 w = pack_codes8_int8(code);
    r.w0 = w.x;
    r.w1 = w.y;
  } else {
    r.w0 = pack_codes8_int4(code);
    r.w1 = 0;
  }
  return r;
}

template <int BITS, int LPG>
__device__ __forceinline__ void quant_store(const QuantChunk& r, int64_t c, uint8_t* q,
                                            uint16_t* s) {
  if ((c & (LPG - 1)) == 0) s[c / LPG] = r.sh;
  if (BITS == 8) reinterpret_cast<uint2*>(q)[c] = make_uint2(r.w0, r.w1);
  else reinterpret_cast<uint32_t*>(q)[c] = r.w0;
}

// Outlier channels (zero-and-store): columns with slot[col] >= 0 are copied
// out as bf16 into out[row * k + slot] and zeroed before the codec sees them
// (HyC-LoRA's outlier extraction, hyclora/operators/compress_function.py:111-143,
// on the v3 per-group codec).
struct Outliers {
  const int16_t* slot;   // [D], -1 for ordinary columns
  uint16_t* out;         // [N, k] bf16
  int64_t k;
  FastDivU32 rows;       // divides a chunk index by the chunks per row (D / 8)
};

// (row, first column) of 8-element chunk c of a row-major [N, D] tensor;
// chunk indices fit 32 bits (checked on the host)
__device__ __forceinline__ void chunk_rc(int64_t c, int64_t d, const Outliers& o, int64_t& row,
                                         int64_t& col) {
  const uint32_t r = o.rows.div((uint32_t)c);
  row = r;
  col = ((int64_t)((uint32_t)c - r * o.rows.d)) * 8;
}

// The outlier columns of one 8-column chunk: slot values (8 x int16, -1 for
// ordinary columns) and the 8-bit mask of those with slot >= 0, from the sign
// bits, branch-free.
struct ChunkSlots {
  uint32_t w[4];
  uint32_t mask;
  __device__ __forceinline__ int slot(int j) const {
    return (int16_t)((w[j >> 1] >> (16 * (j & 1))) & 0xFFFFu);
  }
};

__device__ __forceinline__ ChunkSlots load_slots8(const Outliers& o, int64_t col, bool valid) {
  ChunkSlots cs;
  uint4 v = make_uint4(0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu);
  if (valid) v = *reinterpret_cast<const uint4*>(o.slot + col);
  cs.w[0] = v.x; cs.w[1] = v.y; cs.w[2] = v.z; cs.w[3] = v.w;
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m |= ((~cs.w[i] >> 15) & 1u) << (2 * i);
    m |= ((~cs.w[i] >> 31) & 1u) << (2 * i + 1);
  }
  cs.mask = m;
  return cs;
}

// The stored bf16 values of the chunk's outlier columns (0 elsewhere),
// fetched ahead of the dequantisation they replace.
__device__ __forceinline__ void fetch_outliers8(float ov[8], int64_t row, const ChunkSlots& cs,
                                                const Outliers& o) {
#pragma unroll
  for (int j = 0; j < 8; ++j) ov[j] = 0.0f;
  if (cs.mask) {
    const uint16_t* src = o.out + row * o.k;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if ((cs.mask >> j) & 1u) ov[j] = bf16_to_f32(src[cs.slot(j)]);
  }
}

// Overwrite dequantised values of outlier columns with the stored bf16 values
// (compress_function.py:147-174).
__device__ __forceinline__ void restore_outliers8(float v[8], const float ov[8],
                                                  const ChunkSlots& cs) {
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = ((cs.mask >> j) & 1u) ? ov[j] : v[j];
}

// ---------------------------------------------------------------------------
// standalone quantise, fast path (input dtype DT, group size 8*LPG)
// ---------------------------------------------------------------------------
constexpr int kQuantCPT = 2;   // chunks per thread: both loads in flight before either codes

template <int DT, int BITS, int LPG, bool OUTL>
__global__ __launch_bounds__(kBlock) void quantize_fast_kernel(
    const void* __restrict__ t, uint8_t* __restrict__ q, uint16_t* __restrict__ s,
    int64_t nchunk, int64_t d, Outliers o) {
  const int64_t base = (int64_t)blockIdx.x * kBlock * kQuantCPT + threadIdx.x;
  float v[kQuantCPT][8];
  ChunkSlots cs[kQuantCPT];
  int64_t row[kQuantCPT];
#pragma unroll
  for (int i = 0; i < kQuantCPT; ++i) {
    const int64_t c = base + i * kBlock;
    // lanes past the end work on the last chunk and store nothing
    const int64_t cl = c < nchunk ? c : nchunk - 1;
    if (OUTL) {
      int64_t col = 0;
      chunk_rc(cl, d, o, row[i], col);
      cs[i] = load_slots8(o, col, true);
    }
    Vec8<DT>::ld(t, cl, v[i]);
  }
  // every output formed before the first store (a wait for a load also waits
  // for the stores issued before it)
  QuantChunk r[kQuantCPT];
#pragma unroll
  for (int i = 0; i < kQuantCPT; ++i) {
    float z[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) z[e] = (OUTL && ((cs[i].mask >> e) & 1u)) ? 0.0f : v[i][e];
    r[i] = quant_form<BITS, LPG, DT == kBF16>(z);
  }
#pragma unroll
  for (int i = 0; i < kQuantCPT; ++i) {
    const int64_t c = base + i * kBlock;
    if (c >= nchunk) continue;
    if (OUTL && cs[i].mask) {
      uint16_t* dst = o.out + row[i] * o.k;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if ((cs[i].mask >> e) & 1u) dst[cs[i].slot(e)] = (uint16_t)f32_to_bf16_bits(v[i][e]);
    }
    quant_store<BITS, LPG>(r[i], c, q, s);
  }
}

// ---------------------------------------------------------------------------
// K1: h_mid = SiLU(g)*u (bf16) + codec of g and u, fast path
// ---------------------------------------------------------------------------
template <int BITS, int LPG>
__global__ __launch_bounds__(kBlock) void silu_mul_quant_kernel(
    const uint16_t* __restrict__ g, const uint16_t* __restrict__ u, uint16_t* __restrict__ hm,
    uint8_t* __restrict__ qg, uint16_t* __restrict__ sg, uint8_t* __restrict__ qu,
    uint16_t* __restrict__ su, int64_t nchunk) {
  const int64_t c = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const bool valid = c < nchunk;
  // lanes past the end load the last chunk and store nothing (they form
  // whole groups: nchunk is a multiple of the lanes per group)
  const int64_t cl = valid ? c : nchunk - 1;
  float gv[8], uv[8], h[8];
  Vec8<kBF16>::ld(g, cl, gv);
  Vec8<kBF16>::ld(u, cl, uv);
#pragma unroll
  for (int j = 0; j < 8; ++j) h[j] = silu_mul1(gv[j], uv[j]);  // src/flashffn.py:1212-1215
  const QuantChunk rg = quant_form<BITS, LPG, true>(gv);
  const QuantChunk ru = quant_form<BITS, LPG, true>(uv);
  if (!valid) return;
  Vec8<kBF16>::st(hm, c, h);
  quant_store<BITS, LPG>(rg, c, qg, sg);
  quant_store<BITS, LPG>(ru, c, qu, su);
}

// ---------------------------------------------------------------------------
// generic path: one thread per span of `span` elements (a whole number of
// groups, even so int4 bytes are never shared between threads)
// ---------------------------------------------------------------------------
template <int DT, int BITS, bool GLU>
__global__ __launch_bounds__(kBlock) void quant_generic_kernel(
    const void* __restrict__ tg, const void* __restrict__ tu, void* __restrict__ hm,
    uint8_t* __restrict__ qg, uint16_t* __restrict__ sg, uint8_t* __restrict__ qu,
    uint16_t* __restrict__ su, int64_t nspan, int64_t span, int64_t gs) {
  using E = Elem<DT>;
  const int64_t sp = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (sp >= nspan) return;
  const typename E::T* pg = reinterpret_cast<const typename E::T*>(tg);
  const typename E::T* pu = reinterpret_cast<const typename E::T*>(tu);
  const int64_t e0 = sp * span;
  if (GLU) {
    typename E::T* ph = reinterpret_cast<typename E::T*>(hm);
    for (int64_t e = e0; e < e0 + span; ++e) {
      E::st(ph + e, silu_mul1(E::ld(pg + e), E::ld(pu + e)));
    }
  }
  for (int pass = 0; pass < (GLU ? 2 : 1); ++pass) {
    const typename E::T* p = pass == 0 ? pg : pu;
    uint8_t* q = pass == 0 ? qg : qu;
    uint16_t* s = pass == 0 ? sg : su;
    for (int64_t g0 = e0; g0 < e0 + span; g0 += gs) {
      uint32_t am = 0;
      for (int64_t e = g0; e < g0 + gs; ++e) am = max(am, __float_as_uint(E::ld(p + e)) & 0x7FFFFFFFu);
      const uint16_t sh = scale_bits<BITS>(am);
      s[g0 / gs] = sh;
      const float safe = safe_scale(sh);
      const float rs = __builtin_amdgcn_rcpf(safe);
      for (int64_t e = g0; e < g0 + gs; ++e) {
        const int code = quant_code<BITS>(E::ld(p + e), safe, rs);
        if (BITS == 8) {
          q[e] = (uint8_t)(code & 0xFF);
        } else if ((e & 1) == 0) {
          q[e >> 1] = (uint8_t)((q[e >> 1] & 0xF0u) | (uint32_t)(code + 8));
        } else {
          q[e >> 1] = (uint8_t)((q[e >> 1] & 0x0Fu) | ((uint32_t)(code + 8) << 4));
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// dequantise: out = dtype(fp32(code) * fp32(scale))   (src/flashffn.py:1099-1110)
// ---------------------------------------------------------------------------
template <int BITS, int OUT_DT, bool OUTL>
__global__ __launch_bounds__(kBlock) void dequantize_fast_kernel(
    const uint8_t* __restrict__ q, const uint16_t* __restrict__ s, void* __restrict__ out,
    int64_t nchunk, int gs_shift, int64_t d, Outliers o) {
  const int64_t c = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (c >= nchunk) return;
  float code[8], v[8], ov[8];
  load_codes8<BITS>(q, c, code);
  const float sc = f16_bits_to_f32(s[(c * 8) >> gs_shift]);
  ChunkSlots cs;
  if (OUTL) {
    int64_t row, col;
    chunk_rc(c, d, o, row, col);
    cs = load_slots8(o, col, true);
    fetch_outliers8(ov, row, cs, o);
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = code[j] * sc;
  if (OUTL) {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = round_bf16(v[j]);
    restore_outliers8(v, ov, cs);
  }
  Vec8<OUT_DT>::st(out, c, v);
}

template <int BITS, int OUT_DT>
__global__ __launch_bounds__(kBlock) void dequantize_generic_kernel(
    const uint8_t* __restrict__ q, const uint16_t* __restrict__ s, void* __restrict__ out,
    int64_t n_el, int64_t gs) {
  using E = Elem<OUT_DT>;
  const int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (e >= n_el) return;
  float code;
  if (BITS == 8) {
    code = (float)(int8_t)q[e];
  } else {
    const uint32_t b = q[e >> 1];
    code = (float)((e & 1) ? (b >> 4) : (b & 0xFu)) - 8.0f;
  }
  E::st(reinterpret_cast<typename E::T*>(out) + e, code * f16_bits_to_f32(s[e / gs]));
}

// ---------------------------------------------------------------------------
// K2: dequantise through bf16, SwiGLU backward, optional h_mid^.
// grad_h_gate may be written over grad_h_mid (the caller's private buffer):
// each thread reads its 8 elements of gmid before it stores the same 8 of
// dg, so gmid, dg, du and hm carry no __restrict__.
// ---------------------------------------------------------------------------
template <int BITS, bool WANT_HM>
__global__ __launch_bounds__(kBlock) void dequant_swiglu_bwd_kernel(
    const uint16_t* gmid, const uint8_t* __restrict__ qg, const uint16_t* __restrict__ sg,
    const uint8_t* __restrict__ qu, const uint16_t* __restrict__ su, uint16_t* dg, uint16_t* du,
    uint16_t* hm, int64_t nchunk, int gs_shift) {
  const int64_t c = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (c >= nchunk) return;
  float cg[8], cu[8], dh[8], og[8], ou[8], oh[8], hg[8], hu[8];
  load_codes8<BITS>(qg, c, cg);
  load_codes8<BITS>(qu, c, cu);
  Vec8<kBF16>::ld(gmid, c, dh);
  const int64_t si = (c * 8) >> gs_shift;
  const float scg = f16_bits_to_f32(sg[si]);
  const float scu = f16_bits_to_f32(su[si]);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    // bf16 round trip of the dequantised cache (src/flashffn.py:1251-1253)
    hg[j] = round_bf16(cg[j] * scg);
    hu[j] = round_bf16(cu[j] * scu);
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    float hact;
    swiglu_bwd1(dh[j], hg[j], hu[j], og[j], ou[j], hact);
    oh[j] = hact * hu[j];  // src/flashffn.py:1298-1300
  }
  Vec8<kBF16>::st(dg, c, og);
  Vec8<kBF16>::st(du, c, ou);
  if (WANT_HM) Vec8<kBF16>::st(hm, c, oh);
}

// generic K2 (group sizes below 8, misaligned pointers): one thread per element
template <int BITS, bool WANT_HM>
__global__ __launch_bounds__(kBlock) void dequant_swiglu_bwd_generic_kernel(
    const uint16_t* gmid, const uint8_t* __restrict__ qg, const uint16_t* __restrict__ sg,
    const uint8_t* __restrict__ qu, const uint16_t* __restrict__ su, uint16_t* dg, uint16_t* du,
    uint16_t* hm, int64_t n_el, int64_t gs) {
  const int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (e >= n_el) return;
  float code_g, code_u;
  if (BITS == 8) {
    code_g = (float)(int8_t)qg[e];
    code_u = (float)(int8_t)qu[e];
  } else {
    const uint32_t bg = qg[e >> 1], bu = qu[e >> 1];
    code_g = (float)((e & 1) ? (bg >> 4) : (bg & 0xFu)) - 8.0f;
    code_u = (float)((e & 1) ? (bu >> 4) : (bu & 0xFu)) - 8.0f;
  }
  const float hg = round_bf16(code_g * f16_bits_to_f32(sg[e / gs]));
  const float hu = round_bf16(code_u * f16_bits_to_f32(su[e / gs]));
  float og, ou, hact;
  swiglu_bwd1(bf16_to_f32(gmid[e]), hg, hu, og, ou, hact);
  dg[e] = (uint16_t)f32_to_bf16_bits(og);
  du[e] = (uint16_t)f32_to_bf16_bits(ou);
  if (WANT_HM) hm[e] = (uint16_t)f32_to_bf16_bits(hact * hu);
}

// ---------------------------------------------------------------------------
// K1 and K2 with outlier channels on packed bf16 pairs.  Thread c owns chunk
// c (8 consecutive columns of one row) as in the plain kernels.  A slot word
// holds the int16 slots of two adjacent columns, the payload word their two
// bf16 values, so the outlier work runs on words: an arithmetic shift of each
// 16-bit slot by 15 gives the pair's keep mask (0xFFFF for an ordinary column,
// slot -1; 0 for an outlier column), which zeroes (K1) or replaces (K2) the
// outlier halves with one AND or bit-select per word.  Only lanes whose chunk
// holds an outlier column (a 4-word AND of the slot words differs from all
// ones) store or load outlier values.  At C3 (8192 x 11008, int4 g64, 110
// outlier columns) these measured 135 / 169 us against 139-141 / 173 us for
// the same work on floats with 8-bit column masks (K1 / K2).
// ---------------------------------------------------------------------------
typedef short short2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t keep_mask2(uint32_t slot_word) {
  const short2_t v = __builtin_bit_cast(short2_t, slot_word) >> (short2_t){15, 15};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ uint4 load_slot_words(const Outliers& o, uint32_t j, bool ok) {
  uint4 w = make_uint4(0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu);
  if (ok) w = *reinterpret_cast<const uint4*>(o.slot + (int64_t)j * 8);
  return w;
}

__device__ __forceinline__ bool any_outlier(const uint4& w) {
  return (w.x & w.y & w.z & w.w) != 0xFFFFFFFFu;
}

// Copy the outlier columns of one chunk (raw bf16 words `p`) to out[row][slot]:
// one store per outlier column, a loop over the set bits of the chunk's mask
// (a chunk holds one outlier column or none nearly always, so the wavefront
// issues one or two stores where an unrolled test of all 8 columns issued 8)
__device__ __forceinline__ void store_outlier_words(const uint4& w, const uint4& p, uint32_t row,
                                                    const Outliers& o) {
  uint16_t* dst = o.out + (int64_t)row * o.k;
  uint32_t m = 0;   // bit j: column j's slot is >= 0
  m |= ((~w.x >> 15) & 1u) | ((~w.x >> 30) & 2u);
  m |= (((~w.y >> 15) & 1u) | ((~w.y >> 30) & 2u)) << 2;
  m |= (((~w.z >> 15) & 1u) | ((~w.z >> 30) & 2u)) << 4;
  m |= (((~w.w >> 15) & 1u) | ((~w.w >> 30) & 2u)) << 6;
  while (m) {
    const int j = __builtin_ctz(m);
    m &= m - 1;
    const int q = j >> 1, sh = (j & 1) * 16;
    const uint32_t sw = q == 0 ? w.x : q == 1 ? w.y : q == 2 ? w.z : w.w;
    const uint32_t pw = q == 0 ? p.x : q == 1 ? p.y : q == 2 ? p.z : p.w;
    dst[(int16_t)((sw >> sh) & 0xFFFFu)] = (uint16_t)((pw >> sh) & 0xFFFFu);
  }
}

// The stored bf16 values of one chunk's outlier columns as packed pairs; the
// ordinary halves hold the row's slot-0 value, which the caller's keep mask
// discards.  The 8 loads go out unconditionally, one after the other, so the
// lane waits for them once: loads under per-column branches were each
// followed by their own wait.
__device__ __forceinline__ uint4 load_outlier_words(const uint4& w, uint32_t row,
                                                    const Outliers& o) {
  const uint16_t* src = o.out + (int64_t)row * o.k;
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
  uint32_t v[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int lo = (int16_t)(ws[i] & 0xFFFFu), hi = (int32_t)ws[i] >> 16;
    v[2 * i] = src[max(lo, 0)];
    v[2 * i + 1] = src[max(hi, 0)];
  }
  return make_uint4(v[0] | (v[1] << 16), v[2] | (v[3] << 16), v[4] | (v[5] << 16),
                    v[6] | (v[7] << 16));
}

__device__ __forceinline__ void unpack_bf16x8(const uint4& p, float v[8]) {
  const uint32_t ps[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(ps[i] << 16);
    v[2 * i + 1] = __uint_as_float(ps[i] & 0xFFFF0000u);
  }
}

__device__ __forceinline__ uint4 and_words(const uint4& p, const uint4& slots) {
  return make_uint4(p.x & keep_mask2(slots.x), p.y & keep_mask2(slots.y),
                    p.z & keep_mask2(slots.z), p.w & keep_mask2(slots.w));
}

template <int BITS, int LPG>
__global__ __launch_bounds__(kBlock) void silu_mul_quant_outlier_kernel(
    const uint16_t* __restrict__ g, const uint16_t* __restrict__ u, uint16_t* __restrict__ hm,
    uint8_t* __restrict__ qg, uint16_t* __restrict__ sg, uint8_t* __restrict__ qu,
    uint16_t* __restrict__ su, int64_t nchunk, Outliers og, Outliers ou) {
  const int64_t c = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const bool valid = c < nchunk;
  // lanes past the end work on the last chunk and store nothing (whole groups)
  const int64_t cl = valid ? c : nchunk - 1;
  const uint32_t row = og.rows.div((uint32_t)cl);
  const uint32_t j = (uint32_t)cl - row * og.rows.d;
  const uint4 wg = load_slot_words(og, j, true);
  const uint4 wu = load_slot_words(ou, j, true);
  const uint4 pg = reinterpret_cast<const uint4*>(g)[cl];
  const uint4 pu = reinterpret_cast<const uint4*>(u)[cl];
  float gv[8], uv[8], h[8];
  unpack_bf16x8(pg, gv);
  unpack_bf16x8(pu, uv);
#pragma unroll
  for (int e = 0; e < 8; ++e) h[e] = silu_mul1(gv[e], uv[e]);  // src/flashffn.py:1212-1215
  // zero-and-store (compress_function.py:111-143): the codec sees 0 in the
  // outlier columns
  unpack_bf16x8(and_words(pg, wg), gv);
  unpack_bf16x8(and_words(pu, wu), uv);
  const QuantChunk rg = quant_form<BITS, LPG, true>(gv);
  const QuantChunk ru = quant_form<BITS, LPG, true>(uv);
  if (!valid) return;
  Vec8<kBF16>::st(hm, c, h);
  if (any_outlier(wg)) store_outlier_words(wg, pg, row, og);
  if (any_outlier(wu)) store_outlier_words(wu, pu, row, ou);
  quant_store<BITS, LPG>(rg, c, qg, sg);
  quant_store<BITS, LPG>(ru, c, qu, su);
}

// Outlier values for the K2 kernel below, from HBM (any k) or, STAGED, from
// the block's LDS copy of the outlier rows it touches.
__device__ __forceinline__ uint4 lds_outlier_words(const uint4& w, const uint16_t* so) {
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
  uint32_t v[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int lo = (int16_t)(ws[i] & 0xFFFFu), hi = (int32_t)ws[i] >> 16;
    v[2 * i] = so[max(lo, 0)];
    v[2 * i + 1] = so[max(hi, 0)];
  }
  return make_uint4(v[0] | (v[1] << 16), v[2] | (v[3] << 16), v[4] | (v[5] << 16),
                    v[6] | (v[7] << 16));
}

// Outlier counts the staged K2 takes: the two rows a block can touch, k values
// each, one value per thread and tensor.
constexpr int kStagedOutliersMax = kBlock / 2;

// STAGED (k <= kStagedOutliersMax, D / 8 >= kBlock so a block's chunks lie in
// at most two rows r0, r0 + 1): the block copies those rows' outlier values,
// 2k contiguous elements of each [N, k] block, into LDS with loads that do not
// wait on the slot map, so a lane's outlier values are an LDS read away once
// its slot words arrive.  Otherwise they are loaded from HBM after them.
template <int BITS, bool WANT_HM, bool STAGED>
__global__ __launch_bounds__(kBlock) void dequant_swiglu_bwd_outlier_kernel(
    const uint16_t* gmid, const uint8_t* __restrict__ qg, const uint16_t* __restrict__ sg,
    const uint8_t* __restrict__ qu, const uint16_t* __restrict__ su, uint16_t* dg, uint16_t* du,
    uint16_t* hm, int64_t nchunk, int gs_shift, Outliers og, Outliers ou) {
  __shared__ uint16_t so[STAGED ? 4 * kStagedOutliersMax : 1];   // [tensor][2 rows][k]
  const int64_t c = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const bool valid = c < nchunk;
  // lanes past the end work on the last chunk and store nothing
  const int64_t cl = valid ? c : nchunk - 1;
  const uint32_t row = og.rows.div((uint32_t)cl);
  const uint32_t j = (uint32_t)cl - row * og.rows.d;
  const int k = (int)og.k;
  uint32_t r0 = 0, sv_g = 0, sv_u = 0;
  bool st_lane = false;
  if constexpr (STAGED) {
    // the rows of the block's first and last chunks (one row for most blocks)
    const int64_t c_last = min((int64_t)blockIdx.x * kBlock + kBlock - 1, nchunk - 1);
    r0 = og.rows.div(blockIdx.x * (uint32_t)kBlock);
    const int64_t avail = (int64_t)(og.rows.div((uint32_t)c_last) - r0 + 1) * k;
    st_lane = (int)threadIdx.x < 2 * k;
    const bool st_ok = st_lane && (int64_t)threadIdx.x < avail;
    const int64_t off = st_ok ? (int64_t)r0 * k + threadIdx.x : 0;
    sv_g = og.out[off];
    sv_u = ou.out[off];
    if (!st_ok) sv_g = sv_u = 0;
    // issued before the payload loads, so their LDS writes wait on them alone
    asm volatile("" ::: "memory");
  }
  const uint4 wg = load_slot_words(og, j, true);
  const uint4 wu = load_slot_words(ou, j, true);
  float cg[8], cu[8], dh[8];
  load_codes8<BITS>(qg, cl, cg);
  load_codes8<BITS>(qu, cl, cu);
  Vec8<kBF16>::ld(gmid, cl, dh);
  const int64_t si = (cl * 8) >> gs_shift;
  const float scg = f16_bits_to_f32(sg[si]);
  const float scu = f16_bits_to_f32(su[si]);
  uint4 og4 = make_uint4(0, 0, 0, 0), ou4 = og4;
  if constexpr (STAGED) {
    if (st_lane) {
      so[threadIdx.x] = (uint16_t)sv_g;
      so[2 * k + threadIdx.x] = (uint16_t)sv_u;
    }
    // the stage's writes complete, then a plain barrier (one asm statement,
    // so no LDS read moves above it): __syncthreads() would also wait for the
    // payload loads still in flight
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (any_outlier(wg) || any_outlier(wu)) {
      const uint32_t dr = row - r0;
      og4 = lds_outlier_words(wg, so + dr * k);
      ou4 = lds_outlier_words(wu, so + (2 + dr) * k);
    }
  } else {
    if (any_outlier(wg) || any_outlier(wu)) {
      og4 = load_outlier_words(wg, row, og);
      ou4 = load_outlier_words(wu, row, ou);
    }
  }
  const uint32_t wgs[4] = {wg.x, wg.y, wg.z, wg.w}, wus[4] = {wu.x, wu.y, wu.z, wu.w};
  const uint32_t ogs[4] = {og4.x, og4.y, og4.z, og4.w}, ous[4] = {ou4.x, ou4.y, ou4.z, ou4.w};
  uint32_t hgw[4], huw[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    // bf16 round trip of the dequantised cache (src/flashffn.py:1251-1253), then
    // the stored value of an outlier column (compress_function.py:147-174)
    const uint32_t kg = keep_mask2(wgs[i]), ku = keep_mask2(wus[i]);
    hgw[i] = (pack_bf16x2(cg[2 * i] * scg, cg[2 * i + 1] * scg) & kg) | (ogs[i] & ~kg);
    huw[i] = (pack_bf16x2(cu[2 * i] * scu, cu[2 * i + 1] * scu) & ku) | (ous[i] & ~ku);
  }
  float hg[8], hu[8], ogr[8], our[8], oh[8];
  unpack_bf16x8(make_uint4(hgw[0], hgw[1], hgw[2], hgw[3]), hg);
  unpack_bf16x8(make_uint4(huw[0], huw[1], huw[2], huw[3]), hu);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float hact;
    swiglu_bwd1(dh[e], hg[e], hu[e], ogr[e], our[e], hact);
    oh[e] = hact * hu[e];  // src/flashffn.py:1298-1300
  }
  if (!valid) return;
  Vec8<kBF16>::st(dg, c, ogr);
  Vec8<kBF16>::st(du, c, our);
  if (WANT_HM) Vec8<kBF16>::st(hm, c, oh);
}

// ---------------------------------------------------------------------------
// plain GLU kernels (any float dtype).  Thread c owns elements [8c, 8c+8);
// the last thread takes the ragged tail element by element.  VEC=false is
// the path for pointers that are not 16-byte aligned.
// ---------------------------------------------------------------------------
template <int DT, bool VEC>
__global__ __launch_bounds__(kBlock) void silu_mul_kernel(
    const void* __restrict__ g, const void* __restrict__ u, void* __restrict__ out, int64_t n) {
  using E = Elem<DT>;
  const int64_t c = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const int64_t e0 = c * 8;
  if (e0 >= n) return;
  if (VEC && e0 + 8 <= n) {
    float gv[8], uv[8], h[8];
    Vec8<DT>::ld(g, c, gv);
    Vec8<DT>::ld(u, c, uv);
#pragma unroll
    for (int j = 0; j < 8; ++j) h[j] = silu_mul1(gv[j], uv[j]);
    Vec8<DT>::st(out, c, h);
    return;
  }
  const typename E::T* pg = reinterpret_cast<const typename E::T*>(g);
  const typename E::T* pu = reinterpret_cast<const typename E::T*>(u);
  typename E::T* po = reinterpret_cast<typename E::T*>(out);
  for (int64_t e = e0; e < n && e < e0 + 8; ++e) {
    const float gv = E::ld(pg + e);
    E::st(po + e, silu_mul1(gv, E::ld(pu + e)));
  }
}

// Outputs may alias inputs (src/flashffn.py:129-198): every element is read
// before anything is written, and no two threads share an element, so no
// pointer here is __restrict__.
template <int DT, bool VEC, bool WANT_HM>
__global__ __launch_bounds__(kBlock) void swiglu_bwd_kernel(
    const void* dh, const void* g, const void* u, void* dg, void* du, void* hm, int64_t n) {
  using E = Elem<DT>;
  const int64_t c = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const int64_t e0 = c * 8;
  if (e0 >= n) return;
  if (VEC && e0 + 8 <= n) {
    float a[8], gv[8], uv[8], og[8], ou[8], oh[8];
    Vec8<DT>::ld(dh, c, a);
    Vec8<DT>::ld(g, c, gv);
    Vec8<DT>::ld(u, c, uv);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float hact;
      swiglu_bwd1(a[j], gv[j], uv[j], og[j], ou[j], hact);
      oh[j] = hact * uv[j];
    }
    if (WANT_HM) Vec8<DT>::st(hm, c, oh);
    Vec8<DT>::st(dg, c, og);
    Vec8<DT>::st(du, c, ou);
    return;
  }
  const typename E::T* pdh = reinterpret_cast<const typename E::T*>(dh);
  const typename E::T* pg = reinterpret_cast<const typename E::T*>(g);
  const typename E::T* pu = reinterpret_cast<const typename E::T*>(u);
  for (int64_t e = e0; e < n && e < e0 + 8; ++e) {
    const float a = E::ld(pdh + e), gv = E::ld(pg + e), uv = E::ld(pu + e);
    float og, ou, hact;
    swiglu_bwd1(a, gv, uv, og, ou, hact);
    if (WANT_HM) E::st(reinterpret_cast<typename E::T*>(hm) + e, hact * uv);
    E::st(reinterpret_cast<typename E::T*>(dg) + e, og);
    E::st(reinterpret_cast<typename E::T*>(du) + e, ou);
  }
}

// ---------------------------------------------------------------------------
// host-side dispatch helpers
// ---------------------------------------------------------------------------
inline unsigned grid_for(int64_t items) { return (unsigned)((items + kBlock - 1) / kBlock); }

inline int launch_status() {
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

inline int log2_exact(int64_t v) {
  int s = 0;
  while ((int64_t(1) << s) < v) ++s;
  return s;
}

// Argument contract of the codec (src/flashffn.py:1070-1072, 1303-1311).
inline int check_codec(int64_t n, int64_t d, int bits, int64_t gs, bool need_pow2) {
  if (bits != 4 && bits != 8) return kErrBits;
  if (n < 0 || d < 0 || gs <= 0) return kErrShape;
  if (d % gs != 0) return kErrRagged;
  if (need_pow2 && !is_pow2(gs)) return kErrGroupPow2;
  if (bits == 4 && (d & 1)) return kErrShape;
  return kOk;
}

template <int BITS, int LPG, bool OUTL>
void launch_quant_fast(int dt, const void* t, uint8_t* q, uint16_t* s, int64_t nchunk, int64_t d,
                       Outliers o, hipStream_t st) {
  const unsigned grid = grid_for((nchunk + kQuantCPT - 1) / kQuantCPT);
  if (dt == kBF16)
    quantize_fast_kernel<kBF16, BITS, LPG, OUTL><<<grid, kBlock, 0, st>>>(t, q, s, nchunk, d, o);
  else if (dt == kF16)
    quantize_fast_kernel<kF16, BITS, LPG, OUTL><<<grid, kBlock, 0, st>>>(t, q, s, nchunk, d, o);
  else
    quantize_fast_kernel<kF32, BITS, LPG, OUTL><<<grid, kBlock, 0, st>>>(t, q, s, nchunk, d, o);
}

template <int BITS, bool OUTL>
void launch_quant_fast_lpg(int dt, int lpg, const void* t, uint8_t* q, uint16_t* s,
                           int64_t nchunk, int64_t d, Outliers o, hipStream_t st) {
  switch (lpg) {
    case 1: launch_quant_fast<BITS, 1, OUTL>(dt, t, q, s, nchunk, d, o, st); break;
    case 2: launch_quant_fast<BITS, 2, OUTL>(dt, t, q, s, nchunk, d, o, st); break;
    case 4: launch_quant_fast<BITS, 4, OUTL>(dt, t, q, s, nchunk, d, o, st); break;
    case 8: launch_quant_fast<BITS, 8, OUTL>(dt, t, q, s, nchunk, d, o, st); break;
    case 16: launch_quant_fast<BITS, 16, OUTL>(dt, t, q, s, nchunk, d, o, st); break;
    case 32: launch_quant_fast<BITS, 32, OUTL>(dt, t, q, s, nchunk, d, o, st); break;
    default: launch_quant_fast<BITS, 64, OUTL>(dt, t, q, s, nchunk, d, o, st); break;
  }
}

template <int BITS>
void launch_quant_generic(int dt, bool glu, const void* g, const void* u, void* hm, uint8_t* qg,
                          uint16_t* sg, uint8_t* qu, uint16_t* su, int64_t n_el, int64_t gs,
                          hipStream_t st) {
  // int4 packs two columns per byte: a span must hold an even number of elements
  const int64_t span = (BITS == 4 && (gs & 1)) ? 2 * gs : gs;
  const int64_t nspan = n_el / span;
  const unsigned grid = grid_for(nspan);
  if (glu) {
    quant_generic_kernel<kBF16, BITS, true>
        <<<grid, kBlock, 0, st>>>(g, u, hm, qg, sg, qu, su, nspan, span, gs);
  } else if (dt == kBF16) {
    quant_generic_kernel<kBF16, BITS, false>
        <<<grid, kBlock, 0, st>>>(g, g, nullptr, qg, sg, qg, sg, nspan, span, gs);
  } else if (dt == kF16) {
    quant_generic_kernel<kF16, BITS, false>
        <<<grid, kBlock, 0, st>>>(g, g, nullptr, qg, sg, qg, sg, nspan, span, gs);
  } else {
    quant_generic_kernel<kF32, BITS, false>
        <<<grid, kBlock, 0, st>>>(g, g, nullptr, qg, sg, qg, sg, nspan, span, gs);
  }
}

// K1, plain or with outlier channels (OUTL: og, ou used)
template <int BITS, int LPG, bool OUTL>
void launch_k1(const uint16_t* g, const uint16_t* u, uint16_t* hm, uint8_t* qg, uint16_t* sg,
               uint8_t* qu, uint16_t* su, int64_t nchunk, const Outliers& og, const Outliers& ou,
               hipStream_t st) {
  if (OUTL)
    silu_mul_quant_outlier_kernel<BITS, LPG>
        <<<grid_for(nchunk), kBlock, 0, st>>>(g, u, hm, qg, sg, qu, su, nchunk, og, ou);
  else
    silu_mul_quant_kernel<BITS, LPG>
        <<<grid_for(nchunk), kBlock, 0, st>>>(g, u, hm, qg, sg, qu, su, nchunk);
}

template <int BITS, bool OUTL>
void launch_k1_lpg(int lpg, const uint16_t* g, const uint16_t* u, uint16_t* hm, uint8_t* qg,
                   uint16_t* sg, uint8_t* qu, uint16_t* su, int64_t nchunk, const Outliers& og,
                   const Outliers& ou, hipStream_t st) {
  switch (lpg) {
    case 1: launch_k1<BITS, 1, OUTL>(g, u, hm, qg, sg, qu, su, nchunk, og, ou, st); break;
    case 2: launch_k1<BITS, 2, OUTL>(g, u, hm, qg, sg, qu, su, nchunk, og, ou, st); break;
    case 4: launch_k1<BITS, 4, OUTL>(g, u, hm, qg, sg, qu, su, nchunk, og, ou, st); break;
    case 8: launch_k1<BITS, 8, OUTL>(g, u, hm, qg, sg, qu, su, nchunk, og, ou, st); break;
    case 16: launch_k1<BITS, 16, OUTL>(g, u, hm, qg, sg, qu, su, nchunk, og, ou, st); break;
    case 32: launch_k1<BITS, 32, OUTL>(g, u, hm, qg, sg, qu, su, nchunk, og, ou, st); break;
    default: launch_k1<BITS, 64, OUTL>(g, u, hm, qg, sg, qu, su, nchunk, og, ou, st); break;
  }
}

template <int DT>
void launch_glu(int op, bool vec, const void* a, const void* g, const void* u, void* o1,
                void* o2, void* o3, int64_t n, hipStream_t st) {
  const unsigned grid = grid_for((n + 7) / 8);
  if (op == 0) {
    if (vec) silu_mul_kernel<DT, true><<<grid, kBlock, 0, st>>>(g, u, o1, n);
    else silu_mul_kernel<DT, false><<<grid, kBlock, 0, st>>>(g, u, o1, n);
  } else if (o3 == nullptr) {
    if (vec) swiglu_bwd_kernel<DT, true, false><<<grid, kBlock, 0, st>>>(a, g, u, o1, o2, o3, n);
    else swiglu_bwd_kernel<DT, false, false><<<grid, kBlock, 0, st>>>(a, g, u, o1, o2, o3, n);
  } else {
    if (vec) swiglu_bwd_kernel<DT, true, true><<<grid, kBlock, 0, st>>>(a, g, u, o1, o2, o3, n);
    else swiglu_bwd_kernel<DT, false, true><<<grid, kBlock, 0, st>>>(a, g, u, o1, o2, o3, n);
  }
}

inline int glu_dispatch(int op, int dt, const void* a, const void* g, const void* u, void* o1,
                        void* o2, void* o3, int64_t n, hipStream_t st) {
  if (n < 0) return kErrShape;
  if (n == 0) return kOk;
  if (!g || !u || !o1 || (op != 0 && (!a || !o2))) return kErrShape;
  bool vec = aligned16(g) && aligned16(u) && aligned16(o1);
  if (op != 0) vec = vec && aligned16(a) && aligned16(o2) && (o3 == nullptr || aligned16(o3));
  switch (dt) {
    case kF32: launch_glu<kF32>(op, vec, a, g, u, o1, o2, o3, n, st); break;
    case kF16: launch_glu<kF16>(op, vec, a, g, u, o1, o2, o3, n, st); break;
    case kBF16: launch_glu<kBF16>(op, vec, a, g, u, o1, o2, o3, n, st); break;
    default: return kErrDType;
  }
  return launch_status();
}

// ---------------------------------------------------------------------------
// outlier channel selection: the k columns with the largest L2 norm over the
// rows given (the caller passes the first sample's rows, as HyC-LoRA's
// get_statistics_channel_base ranks x_[0], compress_function.py:80-88),
// ties to the lower column index, slots in ascending column order.
// Deterministic: fp64 sums in a fixed order.
// ---------------------------------------------------------------------------
constexpr int kColRows = 64;    // rows per partial sum

// partial[chunk][col] = sum over rows [chunk*kColRows, +kColRows) of t^2 (fp64)
// Outlier selection runs on one tensor or on two of one shape (gate and up)
// in the same launches: blockIdx.z picks the tensor's pointers.
struct SelectOne {
  const void* t;          // [n(+), d] activations (the first n rows rank)
  double* partial;        // [chunks, d] fp64 partial sums
  double* sumsq;          // [d]
  int16_t* slot;          // [d]
  int32_t* idx;           // [k]
};
struct SelectSet {
  SelectOne s[2];
};

template <int DT>
__global__ __launch_bounds__(64) void colsumsq_partial_kernel(SelectSet S, int64_t n, int64_t d) {
  // one wavefront per 512-column strip and kColRows rows; 8 columns per lane
  // (one 128-bit load of bf16/fp16), fp64 accumulation in row order
  using E = Elem<DT>;
  const void* __restrict__ t = S.s[blockIdx.z].t;
  double* __restrict__ partial = S.s[blockIdx.z].partial;
  const int64_t col = ((int64_t)blockIdx.x * 64 + threadIdx.x) * 8;
  const int64_t r0 = (int64_t)blockIdx.y * kColRows;
  if (col >= d) return;
  const int64_t r1 = r0 + kColRows < n ? r0 + kColRows : n;
  double acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.0;
  auto load = [&](int64_t r, float (&v)[8]) {
    if constexpr (DT == kF32) {
      const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(t) + r * d + col);
      const float4 a = p[0], b = p[1];
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
      Vec8<DT>::ld(reinterpret_cast<const typename E::T*>(t) + r * d + col, 0, v);
    }
  };
  // 8 rows' loads in flight before their (row-ordered) accumulation
  constexpr int kU = 8;
  int64_t r = r0;
  for (; r + kU <= r1; r += kU) {
    float v[kU][8];
#pragma unroll
    for (int u = 0; u < kU; ++u) load(r + u, v[u]);
#pragma unroll
    for (int u = 0; u < kU; ++u)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += (double)v[u][e] * (double)v[u][e];
  }
  for (; r < r1; ++r) {
    float v[8];
    load(r, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] += (double)v[e] * (double)v[e];
  }
  double* out = partial + blockIdx.y * d + col;
#pragma unroll
  for (int e = 0; e < 8; ++e) out[e] = acc[e];
}

__global__ __launch_bounds__(kBlock) void colsumsq_reduce_kernel(SelectSet S, int64_t d,
                                                                  int chunks) {
  // 64 columns per block; wave w sums chunks w, w + 4, ...; the four wave
  // sums are added in wave order (fixed order, deterministic)
  __shared__ double part[kBlock / 64][64];
  const double* __restrict__ partial = S.s[blockIdx.z].partial;
  double* __restrict__ sumsq = S.s[blockIdx.z].sumsq;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t col = (int64_t)blockIdx.x * 64 + lane;
  double acc = 0.0;
  if (col < d)
    for (int c = wave; c < chunks; c += kBlock / 64) acc += partial[(int64_t)c * d + col];
  part[wave][lane] = acc;
  __syncthreads();
  if (wave == 0 && col < d) sumsq[col] = ((part[0][lane] + part[1][lane]) + part[2][lane]) + part[3][lane];
}

// One block picks the k columns with the largest sum of squares (ties to the
// lower column): slot[c] = the column's position among the picked ones in
// ascending column order, or -1; idx[pos] = c.  The k-th largest is found by
// radix select over the fp64 bit patterns (sums of squares are >= 0, so
// their unsigned bit order is their numeric order), 8 bits per pass, each
// pass a 256-bin LDS histogram; wave 0 picks the digit.  A final pass in
// column order keeps the values above the threshold and the lowest-column
// ties (ballot prefix counts).
constexpr int kPickThreads = 1024;
constexpr int64_t kPickStagedMax = 16384;  // 128 KiB of fp64 sums staged in LDS
constexpr int kPickWaves = kPickThreads / 64;

template <bool STAGED>
__global__ __launch_bounds__(kPickThreads) void outlier_pick_kernel(SelectSet S, int64_t d,
                                                                    int64_t k) {
  // STAGED: the d sums are copied to LDS once and every pass reads them there
  extern __shared__ __align__(16) unsigned char pick_smem[];
  const double* __restrict__ vg = S.s[blockIdx.z].sumsq;
  int16_t* __restrict__ slot = S.s[blockIdx.z].slot;
  int32_t* __restrict__ idx = S.s[blockIdx.z].idx;
  const double* v = vg;
  if constexpr (STAGED) {
    double* sv = reinterpret_cast<double*>(pick_smem);
    for (int64_t i = threadIdx.x; i < d; i += kPickThreads) sv[i] = vg[i];
    __syncthreads();
    v = sv;
  }
  __shared__ int hist[256];
  __shared__ unsigned long long sh_prefix;
  __shared__ int sh_rem, sh_done;
  __shared__ int sh_cnt[kPickWaves][2];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  unsigned long long prefix = 0, mask = 0;
  int remaining = (int)k;
  if (k > 0) {
    for (int pass = 7; pass >= 0; --pass) {
      const int shift = pass * 8;
      if (tid < 256) hist[tid] = 0;
      __syncthreads();
      for (int64_t i0 = 0; i0 < d; i0 += kPickThreads) {
        // the top byte (sign, high exponent bits) is shared by nearly all
        // sums: there, one LDS atomic per distinct digit in the wavefront
        // instead of 64 atomics on one bin.  From the next byte on (low
        // exponent and mantissa bits) the digits spread over tens of bins,
        // where a loop over distinct digits costs more than plain atomics.
        const int64_t i = i0 + tid;
        int digit = -1;
        if (i < d) {
          const unsigned long long key = (unsigned long long)__double_as_longlong(v[i]);
          if ((key & mask) == prefix) digit = (int)((key >> shift) & 0xFF);
        }
        if (pass < 7) {
          if (digit >= 0) atomicAdd(&hist[digit], 1);
          continue;
        }
        uint64_t pending = __ballot(digit >= 0);
        while (pending) {
          const int leader = __ffsll((unsigned long long)pending) - 1;
          const int dl = __shfl(digit, leader);
          const uint64_t same = __ballot(digit == dl);
          if (lane == leader) atomicAdd(&hist[dl], (int)__popcll(same));
          pending &= ~same;
        }
      }
      __syncthreads();
      if (wave == 0) {
        // lane l owns digits 255-4l .. 252-4l (descending)
        int c[4], local = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          c[q] = hist[255 - 4 * lane - q];
          local += c[q];
        }
        int cum = local;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          const int u = __shfl_up(cum, off);
          if (lane >= off) cum += u;
        }
        int before = cum - local;   // counts of all larger digits
        if (before < remaining && cum >= remaining) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            if (before + c[q] >= remaining) {
              sh_prefix = prefix | ((unsigned long long)(255 - 4 * lane - q) << shift);
              sh_rem = remaining - before;
              // the digit's whole bucket is needed: every key in it is
              // picked, so the lower bytes need not be resolved
              sh_done = before + c[q] == remaining;
              break;
            }
            before += c[q];
          }
        }
      }
      __syncthreads();
      prefix = sh_prefix;
      remaining = sh_rem;
      const int done = sh_done;
      mask |= 0xFFull << shift;
      __syncthreads();
      if (done) break;
    }
  }
  // thr: the k-th largest key, or (early exit) the bucket's prefix with the
  // unresolved low bytes zero.  Keys above thr are picked, and the first
  // need_eq keys equal to it in column order; after an early exit every key
  // of the bucket is > thr or == thr and need_eq covers them all, so the
  // pick is the same k columns.
  const unsigned long long thr = prefix;
  const int need_eq = remaining;
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  int run_eq = 0, run_sel = 0;
  for (int64_t c0 = 0; c0 < d; c0 += kPickThreads) {
    const int64_t c = c0 + tid;
    bool gt = false, eq = false;
    if (c < d && k > 0) {
      const unsigned long long key = (unsigned long long)__double_as_longlong(v[c]);
      gt = key > thr;
      eq = key == thr;
    }
    const uint64_t m_eq = __ballot(eq);
    if (lane == 0) sh_cnt[wave][0] = __popcll(m_eq);
    __syncthreads();
    int eq_before = run_eq + __popcll(m_eq & below), eq_tot = 0;
#pragma unroll
    for (int w = 0; w < kPickWaves; ++w) {
      eq_before += w < wave ? sh_cnt[w][0] : 0;
      eq_tot += sh_cnt[w][0];
    }
    const bool sel = gt || (eq && eq_before < need_eq);
    const uint64_t m_sel = __ballot(sel);
    if (lane == 0) sh_cnt[wave][1] = __popcll(m_sel);
    __syncthreads();
    int pos = run_sel + __popcll(m_sel & below), sel_tot = 0;
#pragma unroll
    for (int w = 0; w < kPickWaves; ++w) {
      pos += w < wave ? sh_cnt[w][1] : 0;
      sel_tot += sh_cnt[w][1];
    }
    if (c < d) {
      if (sel && pos < k) {
        slot[c] = (int16_t)pos;
        idx[pos] = (int32_t)c;
      } else {
        slot[c] = -1;
      }
    }
    run_eq += eq_tot;
    run_sel += sel_tot;
    __syncthreads();
  }
}

inline bool outlier_args_ok(const void* slot, const void* out, int64_t k, int64_t d) {
  return slot && aligned16(slot) && (d % 8) == 0 && k >= 0 && k < 32768 && (k == 0 || out);
}

}  // namespace cpt

using namespace cpt;

extern "C" {

int cpt_v3_quantize_group_absmax(const void* t, int dtype, int64_t n, int64_t d, int bits,
                                 int64_t group_size, void* payload, void* scales,
                                 void* stream) {
  int rc = check_codec(n, d, bits, group_size, false);
  if (rc) return rc;
  if (dtype != kF32 && dtype != kF16 && dtype != kBF16) return kErrDType;
  const int64_t n_el = n * d;
  if (n_el == 0) return kOk;
  if (!t || !payload || !scales) return kErrShape;
  hipStream_t st = (hipStream_t)stream;
  uint8_t* q = (uint8_t*)payload;
  uint16_t* s = (uint16_t*)scales;
  const bool fast = is_pow2(group_size) && group_size >= 8 && group_size <= 512 &&
                    aligned16(t) && ((uintptr_t)payload & 7u) == 0;
  if (fast) {
    const int lpg = (int)(group_size / 8);
    if (bits == 4) launch_quant_fast_lpg<4, false>(dtype, lpg, t, q, s, n_el / 8, d, Outliers{}, st);
    else launch_quant_fast_lpg<8, false>(dtype, lpg, t, q, s, n_el / 8, d, Outliers{}, st);
  } else {
    if (bits == 4) launch_quant_generic<4>(dtype, false, t, t, nullptr, q, s, q, s, n_el, group_size, st);
    else launch_quant_generic<8>(dtype, false, t, t, nullptr, q, s, q, s, n_el, group_size, st);
  }
  return launch_status();
}

int cpt_v3_dequantize_group_absmax(const void* payload, const void* scales, int64_t n, int64_t d,
                                   int bits, int64_t group_size, void* out, int out_dtype,
                                   void* stream) {
  int rc = check_codec(n, d, bits, group_size, false);
  if (rc) return rc;
  if (out_dtype != kF32 && out_dtype != kF16 && out_dtype != kBF16) return kErrDType;
  const int64_t n_el = n * d;
  if (n_el == 0) return kOk;
  if (!payload || !scales || !out) return kErrShape;
  hipStream_t st = (hipStream_t)stream;
  const uint8_t* q = (const uint8_t*)payload;
  const uint16_t* s = (const uint16_t*)scales;
  const bool fast = is_pow2(group_size) && group_size >= 8 && aligned16(out) &&
                    ((uintptr_t)payload & 7u) == 0;
  if (fast) {
    const int64_t nchunk = n_el / 8;
    const int sh = log2_exact(group_size);
    const unsigned grid = grid_for(nchunk);
#define CPT_DQ(B, O) dequantize_fast_kernel<B, O, false><<<grid, kBlock, 0, st>>>(q, s, out, nchunk, sh, d, Outliers{})
    if (bits == 4) {
      if (out_dtype == kBF16) CPT_DQ(4, kBF16); else if (out_dtype == kF16) CPT_DQ(4, kF16); else CPT_DQ(4, kF32);
    } else {
      if (out_dtype == kBF16) CPT_DQ(8, kBF16); else if (out_dtype == kF16) CPT_DQ(8, kF16); else CPT_DQ(8, kF32);
    }
#undef CPT_DQ
  } else {
    const unsigned grid = grid_for(n_el);
#define CPT_DQG(B, O) dequantize_generic_kernel<B, O><<<grid, kBlock, 0, st>>>(q, s, out, n_el, group_size)
    if (bits == 4) {
      if (out_dtype == kBF16) CPT_DQG(4, kBF16); else if (out_dtype == kF16) CPT_DQG(4, kF16); else CPT_DQG(4, kF32);
    } else {
      if (out_dtype == kBF16) CPT_DQG(8, kBF16); else if (out_dtype == kF16) CPT_DQG(8, kF16); else CPT_DQG(8, kF32);
    }
#undef CPT_DQG
  }
  return launch_status();
}

int cpt_silu_mul(const void* h_gate, const void* h_up, void* out, int64_t n_elements, int dtype,
                 void* stream) {
  return glu_dispatch(0, dtype, nullptr, h_gate, h_up, out, nullptr, nullptr, n_elements,
                      (hipStream_t)stream);
}

int cpt_swiglu_backward(const void* grad_h_mid, const void* h_gate, const void* h_up,
                        void* grad_h_gate, void* grad_h_up, int64_t n_elements, int dtype,
                        void* stream) {
  return glu_dispatch(1, dtype, grad_h_mid, h_gate, h_up, grad_h_gate, grad_h_up, nullptr,
                      n_elements, (hipStream_t)stream);
}

int cpt_swiglu_backward_glu(const void* grad_h_mid, const void* h_gate, const void* h_up,
                            void* grad_h_gate, void* grad_h_up, void* h_mid, int64_t n_elements,
                            int dtype, void* stream) {
  return glu_dispatch(1, dtype, grad_h_mid, h_gate, h_up, grad_h_gate, grad_h_up, h_mid,
                      n_elements, (hipStream_t)stream);
}

int cpt_silu_mul_quant(const void* h_gate, const void* h_up, int64_t n, int64_t d, int bits,
                       int64_t group_size, void* h_mid, void* q_gate, void* s_gate, void* q_up,
                       void* s_up, void* stream) {
  int rc = check_codec(n, d, bits, group_size, true);
  if (rc) return rc;
  const int64_t n_el = n * d;
  if (n_el == 0) return kOk;
  if (!h_gate || !h_up || !h_mid || !q_gate || !s_gate || !q_up || !s_up) return kErrShape;
  hipStream_t st = (hipStream_t)stream;
  const uint16_t* g = (const uint16_t*)h_gate;
  const uint16_t* u = (const uint16_t*)h_up;
  uint16_t* hm = (uint16_t*)h_mid;
  uint8_t* qg = (uint8_t*)q_gate;
  uint8_t* qu = (uint8_t*)q_up;
  uint16_t* sg = (uint16_t*)s_gate;
  uint16_t* su = (uint16_t*)s_up;
  const bool fast = group_size >= 8 && group_size <= 512 && aligned16(g) && aligned16(u) &&
                    aligned16(hm) && ((uintptr_t)qg & 7u) == 0 && ((uintptr_t)qu & 7u) == 0;
  if (fast) {
    const int lpg = (int)(group_size / 8);
    if (bits == 4) launch_k1_lpg<4, false>(lpg, g, u, hm, qg, sg, qu, su, n_el / 8, Outliers{}, Outliers{}, st);
    else launch_k1_lpg<8, false>(lpg, g, u, hm, qg, sg, qu, su, n_el / 8, Outliers{}, Outliers{}, st);
  } else {
    if (bits == 4) launch_quant_generic<4>(kBF16, true, g, u, hm, qg, sg, qu, su, n_el, group_size, st);
    else launch_quant_generic<8>(kBF16, true, g, u, hm, qg, sg, qu, su, n_el, group_size, st);
  }
  return launch_status();
}

int cpt_dequant_swiglu_backward(const void* grad_h_mid, const void* q_gate, const void* s_gate,
                                const void* q_up, const void* s_up, int64_t n, int64_t d,
                                int bits, int64_t group_size, void* grad_h_gate,
                                void* grad_h_up, void* h_mid_hat, void* stream) {
  int rc = check_codec(n, d, bits, group_size, true);
  if (rc) return rc;
  const int64_t n_el = n * d;
  if (n_el == 0) return kOk;
  if (!grad_h_mid || !q_gate || !s_gate || !q_up || !s_up || !grad_h_gate || !grad_h_up)
    return kErrShape;
  hipStream_t st = (hipStream_t)stream;
  const uint16_t* gm = (const uint16_t*)grad_h_mid;
  const uint8_t* qg = (const uint8_t*)q_gate;
  const uint8_t* qu = (const uint8_t*)q_up;
  const uint16_t* sg = (const uint16_t*)s_gate;
  const uint16_t* su = (const uint16_t*)s_up;
  uint16_t* og = (uint16_t*)grad_h_gate;
  uint16_t* ou = (uint16_t*)grad_h_up;
  uint16_t* oh = (uint16_t*)h_mid_hat;
  const bool fast = group_size >= 8 && aligned16(gm) && aligned16(og) && aligned16(ou) &&
                    (oh == nullptr || aligned16(oh)) && ((uintptr_t)qg & 7u) == 0 &&
                    ((uintptr_t)qu & 7u) == 0;
  if (fast) {
    const int64_t nchunk = n_el / 8;
    const unsigned grid = grid_for(nchunk);
    const int sh = log2_exact(group_size);
#define CPT_K2(B, W) dequant_swiglu_bwd_kernel<B, W><<<grid, kBlock, 0, st>>>(gm, qg, sg, qu, su, og, ou, oh, nchunk, sh)
    if (bits == 4) { if (oh) CPT_K2(4, true); else CPT_K2(4, false); }
    else { if (oh) CPT_K2(8, true); else CPT_K2(8, false); }
#undef CPT_K2
  } else {
    const unsigned grid = grid_for(n_el);
#define CPT_K2G(B, W) dequant_swiglu_bwd_generic_kernel<B, W><<<grid, kBlock, 0, st>>>(gm, qg, sg, qu, su, og, ou, oh, n_el, group_size)
    if (bits == 4) { if (oh) CPT_K2G(4, true); else CPT_K2G(4, false); }
    else { if (oh) CPT_K2G(8, true); else CPT_K2G(8, false); }
#undef CPT_K2G
  }
  return launch_status();
}

namespace {
// ntensor (1 or 2) selections of one shape, in three launches
int outlier_select_set(const SelectSet& S, int ntensor, int dtype, int64_t n, int64_t d,
                       int64_t k, hipStream_t st) {
  const int chunks = (int)((n + kColRows - 1) / kColRows);
  const unsigned z = (unsigned)ntensor;
  if (chunks > 0) {
    dim3 grid((unsigned)((d + 511) / 512), (unsigned)chunks, z);
    if (dtype == kBF16) colsumsq_partial_kernel<kBF16><<<grid, 64, 0, st>>>(S, n, d);
    else if (dtype == kF16) colsumsq_partial_kernel<kF16><<<grid, 64, 0, st>>>(S, n, d);
    else colsumsq_partial_kernel<kF32><<<grid, 64, 0, st>>>(S, n, d);
  }
  colsumsq_reduce_kernel<<<dim3((unsigned)((d + 63) / 64), 1, z), kBlock, 0, st>>>(S, d, chunks);
  static bool staged_attr = false;
  if (!staged_attr) {
    staged_attr = hipFuncSetAttribute((const void*)outlier_pick_kernel<true>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                      (int)(kPickStagedMax * sizeof(double))) == hipSuccess;
  }
  if (staged_attr && d <= kPickStagedMax)
    outlier_pick_kernel<true><<<dim3(1, 1, z), kPickThreads, (size_t)d * sizeof(double), st>>>(
        S, d, k);
  else
    outlier_pick_kernel<false><<<dim3(1, 1, z), kPickThreads, 0, st>>>(S, d, k);
  return launch_status();
}

int select_args_ok(const void* t, int64_t n, int64_t d, int64_t k, const void* partial,
                   const void* sumsq, const void* slot, const void* idx) {
  if (!slot || !sumsq || (n > 0 && (!t || !partial)) || (k > 0 && !idx)) return kErrShape;
  if (n > 0 && ((d % 8) || !aligned16(t))) return kErrAlign;   // 8-column vector loads
  return kOk;
}
}  // namespace

int cpt_outlier_select(const void* t, int dtype, int64_t n, int64_t d, int64_t k,
                       void* partial, void* sumsq, void* slot, void* idx, void* stream) {
  if (n < 0 || d < 0 || k < 0 || k > d || k >= 32768) return kErrShape;
  if (dtype != kF32 && dtype != kF16 && dtype != kBF16) return kErrDType;
  if (d == 0) return kOk;
  const int rc = select_args_ok(t, n, d, k, partial, sumsq, slot, idx);
  if (rc) return rc;
  SelectSet S{};
  S.s[0] = {t, (double*)partial, (double*)sumsq, (int16_t*)slot, (int32_t*)idx};
  S.s[1] = S.s[0];
  return outlier_select_set(S, 1, dtype, n, d, k, (hipStream_t)stream);
}

int cpt_outlier_select_pair(const void* t0, const void* t1, int dtype, int64_t n, int64_t d,
                            int64_t k, void* partial, void* sumsq, void* slot0, void* idx0,
                            void* slot1, void* idx1, void* stream) {
  if (n < 0 || d < 0 || k < 0 || k > d || k >= 32768) return kErrShape;
  if (dtype != kF32 && dtype != kF16 && dtype != kBF16) return kErrDType;
  if (d == 0) return kOk;
  const int64_t chunks = (n + kColRows - 1) / kColRows;
  double* p1 = partial ? (double*)partial + chunks * d : nullptr;
  double* q1 = sumsq ? (double*)sumsq + d : nullptr;
  int rc = select_args_ok(t0, n, d, k, partial, sumsq, slot0, idx0);
  if (!rc) rc = select_args_ok(t1, n, d, k, p1, q1, slot1, idx1);
  if (rc) return rc;
  SelectSet S{};
  S.s[0] = {t0, (double*)partial, (double*)sumsq, (int16_t*)slot0, (int32_t*)idx0};
  S.s[1] = {t1, p1, q1, (int16_t*)slot1, (int32_t*)idx1};
  return outlier_select_set(S, 2, dtype, n, d, k, (hipStream_t)stream);
}

int cpt_v3_quantize_outlier(const void* t, int dtype, int64_t n, int64_t d, int bits,
                            int64_t group_size, const void* slot, int64_t k, void* outliers,
                            void* payload, void* scales, void* stream) {
  int rc = check_codec(n, d, bits, group_size, true);
  if (rc) return rc;
  if (dtype != kF32 && dtype != kF16 && dtype != kBF16) return kErrDType;
  if (n * d == 0) return kOk;
  if (!t || !payload || !scales) return kErrShape;
  if (group_size < 8 || group_size > 512 || !aligned16(t) || ((uintptr_t)payload & 7) ||
      !outlier_args_ok(slot, outliers, k, d))
    return kErrAlign;
  if (n * d / 8 > 0xFFFFFFFFll) return kErrTooLarge;   // 32-bit chunk indices
  Outliers o{(const int16_t*)slot, (uint16_t*)outliers, k, FastDivU32::make((uint32_t)(d / 8))};
  hipStream_t st = (hipStream_t)stream;
  const int lpg = (int)(group_size / 8);
  if (bits == 4) launch_quant_fast_lpg<4, true>(dtype, lpg, t, (uint8_t*)payload, (uint16_t*)scales, n * d / 8, d, o, st);
  else launch_quant_fast_lpg<8, true>(dtype, lpg, t, (uint8_t*)payload, (uint16_t*)scales, n * d / 8, d, o, st);
  return launch_status();
}

int cpt_v3_dequantize_outlier(const void* payload, const void* scales, const void* slot, int64_t k,
                              const void* outliers, int64_t n, int64_t d, int bits,
                              int64_t group_size, void* out, void* stream) {
  int rc = check_codec(n, d, bits, group_size, true);
  if (rc) return rc;
  if (n * d == 0) return kOk;
  if (!payload || !scales || !out) return kErrShape;
  if (group_size < 8 || !aligned16(out) || ((uintptr_t)payload & 7) ||
      !outlier_args_ok(slot, outliers, k, d))
    return kErrAlign;
  if (n * d / 8 > 0xFFFFFFFFll) return kErrTooLarge;   // 32-bit chunk indices
  Outliers o{(const int16_t*)slot, (uint16_t*)outliers, k, FastDivU32::make((uint32_t)(d / 8))};
  hipStream_t st = (hipStream_t)stream;
  const int64_t nchunk = n * d / 8;
  const int sh = log2_exact(group_size);
  if (bits == 4)
    dequantize_fast_kernel<4, kBF16, true><<<grid_for(nchunk), kBlock, 0, st>>>((const uint8_t*)payload, (const uint16_t*)scales, out, nchunk, sh, d, o);
  else
    dequantize_fast_kernel<8, kBF16, true><<<grid_for(nchunk), kBlock, 0, st>>>((const uint8_t*)payload, (const uint16_t*)scales, out, nchunk, sh, d, o);
  return launch_status();
}

int cpt_silu_mul_quant_outlier(const void* h_gate, const void* h_up, int64_t n, int64_t d,
                               int bits, int64_t group_size, const void* slot_gate,
                               const void* slot_up, int64_t k, void* h_mid, void* q_gate,
                               void* s_gate, void* o_gate, void* q_up, void* s_up, void* o_up,
                               void* stream) {
  int rc = check_codec(n, d, bits, group_size, true);
  if (rc) return rc;
  if (n * d == 0) return kOk;
  if (!h_gate || !h_up || !h_mid || !q_gate || !s_gate || !q_up || !s_up) return kErrShape;
  if (group_size < 8 || group_size > 512 || !aligned16(h_gate) || !aligned16(h_up) ||
      !aligned16(h_mid) || ((uintptr_t)q_gate & 7) || ((uintptr_t)q_up & 7) ||
      !outlier_args_ok(slot_gate, o_gate, k, d) || !outlier_args_ok(slot_up, o_up, k, d))
    return kErrAlign;
  if (n * d / 8 > 0xFFFFFFFFll) return kErrTooLarge;   // 32-bit chunk indices
  Outliers og{(const int16_t*)slot_gate, (uint16_t*)o_gate, k, FastDivU32::make((uint32_t)(d / 8))};
  Outliers ou{(const int16_t*)slot_up, (uint16_t*)o_up, k, FastDivU32::make((uint32_t)(d / 8))};
  hipStream_t st = (hipStream_t)stream;
  const int lpg = (int)(group_size / 8);
  if (bits == 4)
    launch_k1_lpg<4, true>(lpg, (const uint16_t*)h_gate, (const uint16_t*)h_up, (uint16_t*)h_mid,
                           (uint8_t*)q_gate, (uint16_t*)s_gate, (uint8_t*)q_up, (uint16_t*)s_up,
                           n * d / 8, og, ou, st);
  else
    launch_k1_lpg<8, true>(lpg, (const uint16_t*)h_gate, (const uint16_t*)h_up, (uint16_t*)h_mid,
                           (uint8_t*)q_gate, (uint16_t*)s_gate, (uint8_t*)q_up, (uint16_t*)s_up,
                           n * d / 8, og, ou, st);
  return launch_status();
}

int cpt_dequant_swiglu_backward_outlier(const void* grad_h_mid, const void* q_gate,
                                        const void* s_gate, const void* slot_gate,
                                        const void* o_gate, const void* q_up, const void* s_up,
                                        const void* slot_up, const void* o_up, int64_t k,
                                        int64_t n, int64_t d, int bits, int64_t group_size,
                                        void* grad_h_gate, void* grad_h_up, void* h_mid_hat,
                                        void* stream) {
  int rc = check_codec(n, d, bits, group_size, true);
  if (rc) return rc;
  if (n * d == 0) return kOk;
  if (!grad_h_mid || !q_gate || !s_gate || !q_up || !s_up || !grad_h_gate || !grad_h_up)
    return kErrShape;
  if (group_size < 8 || !aligned16(grad_h_mid) || !aligned16(grad_h_gate) ||
      !aligned16(grad_h_up) || (h_mid_hat && !aligned16(h_mid_hat)) ||
      ((uintptr_t)q_gate & 7) || ((uintptr_t)q_up & 7) ||
      !outlier_args_ok(slot_gate, o_gate, k, d) || !outlier_args_ok(slot_up, o_up, k, d))
    return kErrAlign;
  if (n * d / 8 > 0xFFFFFFFFll) return kErrTooLarge;   // 32-bit chunk indices
  Outliers og{(const int16_t*)slot_gate, (uint16_t*)o_gate, k, FastDivU32::make((uint32_t)(d / 8))};
  Outliers ou{(const int16_t*)slot_up, (uint16_t*)o_up, k, FastDivU32::make((uint32_t)(d / 8))};
  hipStream_t st = (hipStream_t)stream;
  const int64_t nchunk = n * d / 8;
  const unsigned grid = grid_for(nchunk);
  const int sh = log2_exact(group_size);
  const uint16_t* gm = (const uint16_t*)grad_h_mid;
  const uint8_t* qg = (const uint8_t*)q_gate;
  const uint8_t* qu = (const uint8_t*)q_up;
  const uint16_t* sg = (const uint16_t*)s_gate;
  const uint16_t* su = (const uint16_t*)s_up;
  uint16_t* dg = (uint16_t*)grad_h_gate;
  uint16_t* du = (uint16_t*)grad_h_up;
  uint16_t* hm = (uint16_t*)h_mid_hat;
  const bool staged = k >= 1 && k <= kStagedOutliersMax && d / 8 >= kBlock;
#define CPT_K2O(B, W, S) dequant_swiglu_bwd_outlier_kernel<B, W, S><<<grid, kBlock, 0, st>>>(gm, qg, sg, qu, su, dg, du, hm, nchunk, sh, og, ou)
  if (staged) {
    if (bits == 4) { if (hm) CPT_K2O(4, true, true); else CPT_K2O(4, false, true); }
    else { if (hm) CPT_K2O(8, true, true); else CPT_K2O(8, false, true); }
  } else {
    if (bits == 4) { if (hm) CPT_K2O(4, true, false); else CPT_K2O(4, false, false); }
    else { if (hm) CPT_K2O(8, true, false); else CPT_K2O(8, false, false); }
  }
#undef CPT_K2O
  return launch_status();
}

const char* cpt_status_string(int status) {
  switch (status) {
    case kOk: return "ok";
    case kErrBits: return "unsupported bits (expected 4 or 8)";
    case kErrRagged: return "D not divisible by group_size";
    case kErrGroupPow2: return "group_size must be a power of two";
    case kErrShape: return "bad shape or null pointer";
    case kErrDType: return "unsupported dtype";
    case kErrLaunch: return "kernel launch failed";
    case kErrAlign: return "pointer alignment not met";
    case kErrTooLarge: return "size beyond the supported maximum";
    default: return "unknown status";
  }
}

int cpt_abi_version(void) { return 1; }

}  // extern "C"
