// bf16 GEMM on v_mfma_f32_16x16x32_bf16 with direct-to-LDS operand loads:
//   C[M, N] = A[M, K] . B[K, N] (+ A2 . B2 over a second K range), fp32
//   accumulate, each operand K-major (rows of K) or MN-major (rows of M or N;
//   fragments through transposing LDS reads).
// Two epilogues:
//   EPI_STORE  C = bf16(acc): the plain products of cpt_gemm_bf16 in every
//              operand layout (N a multiple of 8, K of 64);
//   EPI_GLU    F1 (x . [W_gate; W_up]^T, the GLU and the cache codec of
//              glu_finish; d_ff a multiple of 8, K of 64).
// M and N are free: the last tile row and column are masked at the store, and
// operand loads past the edge read zeros through the buffer range check (rows
// of a K-major operand past its end, 8-column chunks of an MN-major one past
// its edge).
// Adapter terms (LT = 1, 2) are added in either epilogue, of rank up to 16
// (HI = false) or 17..32 (HI = true: a kernel of its own, one tile per
// block).  Every other product runs on the 32x32x16 engine in gemm_kernel.h.
// The instantiations live in gemm16*.hip.
//
// Why a second main loop.  At the 1400 W board limit the MFMA work per joule
// sets the rate: 16x16x32 spends 0.63 pJ per FLOP against 0.71 for 32x32x16
// (register-only probe), and loading the operands straight into LDS
// (buffer_load ... lds) drops the engine's 16 ds_write_b128 per thread and
// k-tile and the 64 VGPRs that hold a tile in flight.
//
// Block: 256 threads (4 waves, one per SIMD), a 256 x 256 output tile, k
// steps of 64; wave w owns C rows 128 (w / 2) .. +127 and columns
// 128 (w % 2) .. +127 as 8 x 8 MFMA blocks of 16 x 16.
//
// LDS: 2 stages x 2 operands x [256 rows][64 k] bf16, unpadded, 128 KiB.
// Row r keeps its 8 chunks of 8 k-values at chunk position c ^ (r & 6): a
// 16x16x32 fragment read (lane l: row l % 16, chunk l / 16 or l / 16 + 4)
// then touches every bank once per 16 lanes (conflict-free under gfx950's
// 128-bit read grouping).  A direct-to-LDS load writes 64 lanes x 16 bytes
// contiguously, so the swizzle is applied on the global side: lane l of a
// load fetches row 8 q + l / 8, chunk (l % 8) ^ (row & 6) into LDS row
// 8 q + l / 8, chunk position l % 8.
//
// Schedule of one k-tile kt (stage s = kt & 1) over its 128 MFMA slots t:
//   t < 64   sub-step 0 (k 0..31) on fragment set F0, in triangular (i, j)
//            order so the first MFMAs need only the first fragments read;
//   t >= 64  sub-step 1 (k 32..63) on F1;
//   t = 2q   (q < 16) F1 reads of tile kt from stage s;
//   t = 33   barrier A (after lgkmcnt(0)): every wave has read stage s;
//   t = 34 + 6p (p < 16)  load p of tile kt + 2 into stage s;
//   t = 95   barrier B (after this wave's loads of tile kt + 1 have landed:
//            vmcnt = the loads of tile kt + 2 issued since);
//   t = 96 + 2q  F0 reads of tile kt + 1 from stage s ^ 1.
// Spreading the 16 loads over 90 slots matters: issued in one burst after a
// single barrier the loop ran at 0.57 TF/GHz, spread this way at 0.82-0.85
// (the engine 0.81-0.86).  At the board's power cap the loop spends 8-12% less
// energy per FLOP than the engine and runs the C2 products 8-14% faster.  Both
// barriers are plain s_barrier: __syncthreads()'s release fence makes the
// compiler wait for every load in flight, the direct-to-LDS ones included,
// which drains the pipeline.

#pragma once

#include "gemm_kernel.h"

namespace cpt {
namespace gemm {
namespace nt16 {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;

constexpr int kBK = 64;
constexpr int kThreads = 256;
constexpr int kStage = 256 * kBK;                 // elements of one operand in one stage
constexpr int kMainLds = 4 * kStage * 2;          // 2 stages x 2 operands: 128 KiB
constexpr int kLdOut = 264;                       // staged output rows (elements)
constexpr int kOutLds = 256 * kLdOut * 2;         // 132 KiB
constexpr int kMax2 = kMainLds > kOutLds ? kMainLds : kOutLds;
constexpr int kLds = kMax2 > kGluLdsBytes ? kMax2 : kGluLdsBytes;
static_assert(kLds <= 160 * 1024, "LDS per block");

constexpr int kBarA = 34;                         // first slot after barrier A
constexpr int kLdEvery = 6;                       // slots between loads of one tile
constexpr int kBarB = 96;                         // first slot after barrier B
constexpr int kLoadsBeforeB = (kBarB - 1 - kBarA) / kLdEvery + 1;
static_assert(kBarA - 1 > 2 * 15, "barrier A follows the last F1 read");
static_assert(kBarA + kLdEvery * 15 < 128, "every load of a tile inside the tile");
static_assert(kBarB + 2 * 15 < 128, "F0 reads inside the tile");
static_assert(kLoadsBeforeB <= 16, "vmcnt of barrier B");

// sub-step 0 order: (i, j) over 8 x 8 blocks, block n = max(i, j) ascending
struct Order {
  uint8_t i[64], j[64];
  constexpr Order() : i(), j() {
    int t = 0;
    for (int n = 0; n < 8; ++n) {
      for (int q = 0; q < n; ++q) { i[t] = n; j[t] = q; ++t; }
      for (int q = 0; q < n; ++q) { i[t] = q; j[t] = n; ++t; }
      i[t] = n; j[t] = n; ++t;
    }
  }
};

__device__ __forceinline__ int lds_off(int row, int chunk) {
  return row * kBK + ((chunk ^ (row & 6)) << 3);
}

// The accumulator is tied in place ("+a"): with the builtin, LLVM rotates the
// 64 four-register blocks through copies.
__device__ __forceinline__ void mfma(f32x4& c, const bf16x8& a, const bf16x8& b) {
  asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}

// Buffer descriptor as four SGPRs (the inline-asm form of make_rsrc).
typedef int i32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i32x4 rsrc_sgpr(const void* p, int64_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  const uint32_t n = bytes > 0x7FFFFFFF ? 0x7FFFFFFFu : bytes < 0 ? 0u : (uint32_t)bytes;
  return i32x4{(int)(uint32_t)a, (int)((uint32_t)(a >> 32) & 0xFFFFu), (int)n, kRsrcWord3};
}

// 16 bytes per lane from the buffer at voff + soff into LDS at dst + 16 * lane
// bytes.  Inline asm, not the builtin: the compiler counts a builtin load as a
// pending LDS write and then puts vmcnt(0) (every load in flight, the next
// tiles' included) before the transposing LDS reads.  Every wait these loads
// need is explicit in the schedule (barrier B's vmcnt, the epilogue's vmcnt(0)).
// voff is the loop-invariant per-lane offset, soff the uniform k-tile delta.
__device__ __forceinline__ void load_lds(const i32x4& r, uint16_t* dst, uint32_t voff,
                                         uint32_t soff) {
  const uint32_t m0v = (uint32_t)(uintptr_t)(lds_void_t*)dst;
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :: "s"(m0v), "v"(voff), "s"(r), "s"(soff) : "memory", "m0");
}

// MN-major tile: [64 k][256 mn] rows of 512 bytes; the 16-byte chunk c of
// row k sits at position c ^ mn_swz(k).  A 32-lane pass of the transposing
// fragment read covers rows k0 + 0..3 and k0 + 8..11 (lanes 0-15, 16-31) at
// two chunks each; the XOR gives those 8 rows 8 different chunk pairs, so the
// pass touches each of the 64 banks once.
__device__ __forceinline__ int mn_swz(int k) { return 2 * ((k & 3) | ((k & 8) >> 1)); }

// ---------------------------------------------------------------------------
// Adapter (LoRA) terms in the epilogue: out = bf16(bf16(acc) + bf16(alpha *
// bf16(P_t Q_t^T))) per term, PEFT's order.  The rank-sized product of each
// 16 x 16 block is one v_mfma_f32_16x16x16_bf16 over k 0..15 (and, for a rank
// above 16, a second over k 16..31 accumulated onto it): lane l supplies k
// 4 (l / 16) .. + 3 of row l % 16 of a block (Q for the n side, P for the m
// side); k past the rank, rows past an operand's end and an absent term's null
// P read zero through the buffer range check.  An absent term also has
// alpha = -0.0, and x + bf16(-0.0 * 0) == x for every x: no branch.
// ---------------------------------------------------------------------------
typedef short s16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ s16x4 lora4_km(__amdgpu_buffer_rsrc_t rs, int64_t ld, int64_t row, int r,
                                          int lane, int kb = 0) {
  const int k0 = kb + (lane >> 4) * 4;
  const uint32_t off = k0 < r ? (uint32_t)((row * ld + k0) * 2) : kOOB;
  return __builtin_bit_cast(s16x4, __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, 0));
}

// Q stored [r][ld] (n contiguous): 4 k of column n, one 2-byte load each
__device__ __forceinline__ s16x4 lora4_mn(__amdgpu_buffer_rsrc_t rs, int64_t ld, int64_t n, int r,
                                          int lane, int kb = 0) {
  const int k0 = kb + (lane >> 4) * 4;
  s16x4 v;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t off = k0 + e < r ? (uint32_t)(((int64_t)(k0 + e) * ld + n) * 2) : kOOB;
    v[e] = (short)__builtin_amdgcn_raw_buffer_load_b16(rs, off, 0, 0);
  }
  return v;
}

// One wave's adapter fragments: p[t][j] the m-side rows of P_t (block j),
// q[t][i] the n-side rows of Q_t (block i; DUAL: term t's blocks only, gate
// i < 4 and up i >= 4), over k 0..15.  HI (ranks 17..32, kernels of their
// own, so the rank-16 kernels keep their code and registers): ph / qh the
// same over k 16..31, which a second MFMA accumulates.
template <bool HI>
struct Lora16 {
  s16x4 p[2][8];
  s16x4 q[2][8];
};
template <>
struct Lora16<true> {
  s16x4 p[2][8];
  s16x4 q[2][8];
  s16x4 ph[2][8];
  s16x4 qh[2][8];
};

template <bool DUAL, int LT, bool HI>
__device__ __forceinline__ void lora16_load(const KArgs& A, int64_t m0, int64_t n0, int wm, int wn,
                                            int lane, Lora16<HI>& F) {
  const int r = A.lrank;
#pragma unroll
  for (int t = 0; t < LT; ++t) {
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(A.lp[t], A.lp[t] ? A.M * A.lldp * 2 : 0);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      F.p[t][j] = lora4_km(rp, A.lldp, m0 + wm * 128 + 16 * j + (lane & 15), r, lane);
    if constexpr (HI) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        F.ph[t][j] = lora4_km(rp, A.lldp, m0 + wm * 128 + 16 * j + (lane & 15), r, lane, 16);
    }
    if constexpr (DUAL) {
      const __amdgpu_buffer_rsrc_t rq = make_rsrc(A.lq[t], A.lq[t] ? A.D * r * 2 : 0);
#pragma unroll
      for (int ii = 0; ii < 4; ++ii)
        F.q[t][4 * t + ii] = lora4_km(rq, r, (n0 >> 1) + wn * 64 + 16 * ii + (lane & 15), r, lane);
      if constexpr (HI) {
#pragma unroll
        for (int ii = 0; ii < 4; ++ii)
          F.qh[t][4 * t + ii] =
              lora4_km(rq, r, (n0 >> 1) + wn * 64 + 16 * ii + (lane & 15), r, lane, 16);
      }
    } else {
      const int64_t qbytes = A.lq_km ? A.N * r * 2 : (int64_t)r * A.lldq * 2;
      const __amdgpu_buffer_rsrc_t rq = make_rsrc(A.lq[t], qbytes);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int64_t n = n0 + wn * 128 + 16 * i + (lane & 15);
        F.q[t][i] = A.lq_km ? lora4_km(rq, r, n, r, lane) : lora4_mn(rq, A.lldq, n, r, lane);
        if constexpr (HI)
          F.qh[t][i] = A.lq_km ? lora4_km(rq, r, n, r, lane, 16)
                               : lora4_mn(rq, A.lldq, n, r, lane, 16);
      }
    }
  }
}

// accumulator block (i, j) with the kernel's LT adapter terms applied
template <bool DUAL, int LT, bool HI>
__device__ __forceinline__ f32x4 acc16(const KArgs& A, const f32x4& a, const Lora16<HI>& F, int i,
                                       int j) {
  f32x4 v = a;
#pragma unroll
  for (int t = 0; t < LT; ++t) {
    if (DUAL && (i >> 2) != t) continue;
    f32x4 l = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(F.q[t][i], F.p[t][j],
                                                       f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
    if constexpr (HI)   // k 16..31 onto the fp32 sum of k 0..15
      l = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(F.qh[t][i], F.ph[t][j], l, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 4; ++r)
      v[r] = round_bf16(round_bf16(v[r]) + round_bf16(A.lalpha[t] * round_bf16(l[r])));
  }
  return v;
}

// ---------------------------------------------------------------------------
// Stream-K (plain-store products).  A product whose tile count T is not a
// multiple of the CU count S leaves its last wave of tiles part-empty.  The
// host then runs T' = T - (T mod S) - S tiles data-parallel (one block each)
// and shares the k-iterations of the other (T mod S) + S tiles evenly over S
// more blocks: the block of rank s owns global iterations [s I / S,
// (s + 1) I / S) of those tiles (I = their tile count x k-tiles per tile),
// one to two tiles' worth, so a tile spans at most two ranks.  Ranks are
// dealt so that the blocks of one XCD hold consecutive ranks.  A block walks
// its tiles from the last to the first.
//   - A tile it covers whole it finishes alone.
//   - A tile whose k-range continues past its range (its last tile, taken
//     first) it leaves as a partial: fp32 accumulators to slot s of the
//     workspace, then a ready flag.
//   - A tile whose k-range began in rank s - 1 (its first tile, taken last)
//     it finishes: it waits for that rank's flag, adds its partial, clears
//     the flag and runs the epilogue.  The result is deterministic for a
//     given shape and CU count.
// The S stream-K blocks fit on the chip at once (one block per CU) and the
// data-parallel blocks ahead of them never wait, so every wait ends; it is
// bounded anyway (kSkSpin polls), and a wait that runs out counts an error in
// the word after the flags and goes on.
// ---------------------------------------------------------------------------
constexpr int kRoleWhole = 0, kRolePartial = 1, kRoleFinish = 2;
// 0 as a value the compiler cannot hoist: a flag address built from it does
// not pin a zero VGPR across the main loop (which spilled it)
__device__ __forceinline__ int fresh_zero() {
  int z = 0;
  asm volatile("" : "+v"(z));
  return z;
}
constexpr int kSc1 = 16;                          // buffer cache policy: agent-coherent (sc1)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int64_t kSkSlot = 256 * 256;            // floats per partial (one tile)
constexpr int kSkSpin = 1 << 22;

template <bool AK, bool BK, int EPI, int CACHE, int GS, int LT, bool SK, bool HI>
__device__ __forceinline__ void nt16_tile(const KArgs& A, uint16_t* lds, int tm, int tn, int kb,
                                          int ke, int role, int sk_s) {
  static_assert(LT == 0 || AK, "adapter terms ride with a K-major A (P's rows are tokens)");
  static_assert(EPI == EPI_STORE || EPI == EPI_GLU || EPI == EPI_DGLU || EPI == EPI_GLUO,
                "epilogues of the 16x16x32 loop");
  static_assert(EPI != EPI_DGLU || (AK && !BK), "B1: gy (K-major) . W_d (MN-major)");
  constexpr bool DUAL = EPI == EPI_GLU || EPI == EPI_GLUO;
  static_assert(!DUAL || (AK && BK), "F1's operands are K-major");
  // per-lane values are derived afresh for each tile of a stream-K block:
  // hoisted out of its tile loop they would stay live across the main loop
  const int tid = epi_tid();
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave & 1, wm = wave >> 1;
  const int64_t m0 = (int64_t)tm * 256, n0 = (int64_t)tn * 256;
  // k-tiles [kb, ke) of the tile; [0, nk0) come from pair 0, the rest from
  // pair 1 (K-concatenated)
  const int nk0 = (int)(A.K[0] / kBK);
  const int64_t lda = A.a[0].ld, ldb = A.b[0].ld;   // pair 1 shares them (host check)

  // Buffers: a K-major operand at the tile's first row (257 rows < 2 GiB), an
  // MN-major one at the tile's first column (K + 256 rows < 2 GiB; host checks).
  // DUAL: the tile's 256 B rows are gate rows d0 .. d0 + 63, up rows d0 .. +63,
  // gate rows d0 + 64 .. +127, up rows d0 + 64 .. +127 (d0 = n0 / 2), so each
  // wave's 128 columns hold 64 gate and the same 64 up columns.
  const int64_t nb0 = DUAL ? n0 / 2 : n0;
  const int64_t nrows = DUAL ? A.D : A.N;
  auto rsrc_a = [&](int pr) {
    return AK ? rsrc_sgpr(A.a[pr].p + m0 * lda, (A.M - m0) * lda * 2)
              : rsrc_sgpr(A.a[pr].p + m0, (A.K[pr] * lda - m0) * 2);
  };
  auto rsrc_b = [&](int pr, const uint16_t* p) {
    return BK ? rsrc_sgpr(p + nb0 * ldb, (nrows - nb0) * ldb * 2)
              : rsrc_sgpr(p + n0, (A.K[pr] * ldb - n0) * 2);
  };
  const bool two = A.npairs == 2;
  const i32x4 ra0 = rsrc_a(0), rb0 = rsrc_b(0, A.b[0].p);
  const i32x4 ra1 = two ? rsrc_a(1) : ra0;
  const i32x4 rb1 = two ? rsrc_b(1, A.b[1].p) : rb0;
  const i32x4 rbu = DUAL ? rsrc_b(0, A.b_up) : rb0;
  // Load i of an operand fills LDS block q = 4 i + wave (1 KiB):
  //   K-major: rows 8 q .. 8 q + 7; lane l row 8 q + l / 8 (row & 6 = (l / 8) & 6),
  //            16-byte k chunk (l % 8) ^ (row & 6) (DUAL B: source row per block as above);
  //   MN-major: k-rows 2 q, 2 q + 1; lane l k-row 2 q + l / 32, mn chunk
  //            (l % 32) ^ mn_swz(k-row).
  // Out of range is always decided by this VGPR offset, never by the
  // soffset delta below (the raw-buffer range check covers the VGPR offset):
  // K-major rows past the operand's end lie past num_records; MN-major
  // 8-column chunks past the edge (M, N multiples of 8 there) get kOOB.
  uint32_t oa[8], ob[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int q = 4 * i + wave;
    const int r = 8 * q + (lane >> 3);
    const int ck = (lane & 7) ^ ((lane >> 3) & 6);
    const int kr = 2 * q + (lane >> 5);
    const int cm = (lane & 31) ^ mn_swz(kr);
    const int rw = DUAL ? 64 * (i >> 2) + 8 * (4 * (i & 1) + wave) + (lane >> 3) : r;
    oa[i] = AK ? (uint32_t)(((int64_t)r * lda + ck * 8) * 2)
               : m0 + cm * 8 < A.M ? (uint32_t)(((int64_t)kr * lda + cm * 8) * 2) : kOOB;
    ob[i] = BK ? (uint32_t)(((int64_t)rw * ldb + ck * 8) * 2)
               : n0 + cm * 8 < A.N ? (uint32_t)(((int64_t)kr * ldb + cm * 8) * 2) : kOOB;
  }
  // per k-tile: the pair's buffers and each operand's byte delta (k0 * 2 for a
  // K-major operand, k0 * ld * 2 for an MN-major one), passed as soffset.  The
  // two tiles the loop loads past the last one re-read the last tile (valid
  // memory; their stage is never read): soffset is outside the range check,
  // so an out-of-range delta there would be a real access.
  struct TileLd {
    i32x4 a, b;
    uint32_t da, db;
  };
  // bytes per k-tile, 32-bit (an MN-major operand's K + 256 rows are < 2 GiB):
  // a 64-bit product here is VALU work, and the buffers selected with it then
  // land in VGPRs (a readfirstlane loop around every load)
  const uint32_t stepa = AK ? (uint32_t)(kBK * 2) : (uint32_t)(kBK * lda * 2);
  const uint32_t stepb = BK ? (uint32_t)(kBK * 2) : (uint32_t)(kBK * ldb * 2);
  auto tile = [&](int kt) -> TileLd {
    const int kc = kt < ke ? kt : ke - 1;
    const bool p1 = kc >= nk0;
    const uint32_t lk = (uint32_t)(kc - (p1 ? nk0 : 0));
    return TileLd{p1 ? ra1 : ra0, p1 ? rb1 : rb0, lk * stepa, lk * stepb};
  };
  // load p (0..15) of a tile into stage st: even p -> A block p / 2, odd -> B
  auto issue = [&](int p, int st, const TileLd& T) {
    const int i = p >> 1;
    uint16_t* dst = lds + (st * 2 + (p & 1)) * kStage + (4 * i + wave) * 512;
    if (p & 1) load_lds(DUAL && ((i >> 1) & 1) ? rbu : T.b, dst, ob[i], T.db);
    else load_lds(T.a, dst, oa[i], T.da);
  };

  f32x4 acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // Fragment q of a sub-step s (k 32 s .. 32 s + 31): even q -> B (n block q / 2),
  // odd q -> A (m block q / 2).  Lane l holds 8 consecutive k (8 (l / 16) ..)
  // of row l % 16 of the block:
  //   K-major: one 16-byte read;
  //   MN-major: two transposing reads (4 k each).  In a 16-lane group lane l'
  //     reads k-row 8 (l / 16) + (l' % 16) / 4 (+ 4), columns 4 (l' % 4) .. + 3 of
  //     the block; the chunk position is 16 w + 2 (block ^ f') + (l % 4) / 2 with
  //     f' = mn_swz(k-row) / 2, the same for both reads and both sub-steps.
  const int nofs0 = lds_off(wn * 128 + (lane & 15), lane >> 4);
  const int mofs0 = lds_off(wm * 128 + (lane & 15), lane >> 4);
  const int nofs1 = lds_off(wn * 128 + (lane & 15), (lane >> 4) + 4);
  const int mofs1 = lds_off(wm * 128 + (lane & 15), (lane >> 4) + 4);
  const int mn_lane = (8 * (lane >> 4) + ((lane & 15) >> 2)) * 256 + ((lane & 3) >> 1) * 8 + (lane & 1) * 4;
  const int mn_fx = 8 * mn_swz(8 * (lane >> 4) + ((lane & 15) >> 2));   // 16 f'
  bf16x8 f0[16], f1[16];
  auto rd = [&](int st, int s, int q) -> bf16x8 {
    const uint16_t* base = lds + st * 2 * kStage;
    const bool bside = (q & 1) == 0;
    if ((bside && BK) || (!bside && AK)) {
      const int o = bside ? kStage + (s ? nofs1 : nofs0) : (s ? mofs1 : mofs0);
      return *reinterpret_cast<const bf16x8*>(base + o + (q >> 1) * 16 * kBK);
    }
    const uint16_t* p = base + (bside ? kStage + 128 * wn : 128 * wm) + mn_lane + s * 32 * 256 +
                        ((16 * (q >> 1)) ^ mn_fx);
    const i16x4 lo = lds_read_tr(p);
    const i16x4 hi = lds_read_tr(p + 4 * 256);
    return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  };

  // prologue: k-tile kb -> stage 0, kb + 1 -> stage 1; kb landed; F0 of kb
  {
    const TileLd T0 = tile(kb), T1 = tile(kb + 1);
#pragma unroll
    for (int p = 0; p < 16; ++p) issue(p, 0, T0);
#pragma unroll
    for (int p = 0; p < 16; ++p) issue(p, 1, T1);
  }
  asm volatile("s_waitcnt vmcnt(16)\n\ts_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  // read order pinned so the loop header's merged waits stay counts, not lgkmcnt(0)
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    f0[q] = rd(0, 0, q);
    __builtin_amdgcn_sched_barrier(0);
  }

  constexpr Order ord;
  for (int kt = kb; kt < ke; ++kt) {
    const int stage = (kt - kb) & 1;
    const TileLd T2 = tile(kt + 2);
    static_for<0, 128>([&](auto tc) {
      constexpr int t = decltype(tc)::value;
      if constexpr (t < 64) {
        constexpr int i = ord.i[t], j = ord.j[t];
        mfma(acc[i][j], f0[2 * i], f0[2 * j + 1]);
      } else {
        constexpr int i = (t - 64) >> 3, j = (t - 64) & 7;
        mfma(acc[i][j], f1[2 * i], f1[2 * j + 1]);
      }
      if constexpr (t % 2 == 0 && t / 2 < 16) f1[t / 2] = rd(stage, 1, t / 2);
      if constexpr (t == kBarA - 1) asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      if constexpr (t >= kBarA && (t - kBarA) % kLdEvery == 0 && (t - kBarA) / kLdEvery < 16)
        issue((t - kBarA) / kLdEvery, stage, T2);
      if constexpr (t == kBarB - 1)
        asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(kLoadsBeforeB) : "memory");
      if constexpr (t >= kBarB && (t - kBarB) % 2 == 0 && (t - kBarB) / 2 < 16)
        f0[(t - kBarB) / 2] = rd(stage ^ 1, 0, (t - kBarB) / 2);
      __builtin_amdgcn_sched_barrier(0);
    });
  }
  // the loads past the last tile (re-reads of tile ke - 1) are still landing
  // in LDS: wait for them (every wave) before the output is staged there
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");

  if constexpr (SK) {
    if (role == kRolePartial) {
      // this block's share of a tile that a higher block finishes
      // agent-coherent (sc1) stores write through to memory, so no cache
      // writeback is needed before the flag; waiting for them is enough
      const int ptid = epi_tid();
      const __amdgpu_buffer_rsrc_t rw = make_rsrc(A.sk_ws + (int64_t)sk_s * kSkSlot, kSkSlot * 4);
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          f32x4 v = acc[i][j];
          asm volatile("" : "+v"(v));
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rw,
                                                 ((i * 8 + j) * 256 + ptid) * 16, 0, kSc1);
        }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (ptid == 0) __hip_atomic_store(A.sk_flags + sk_s + fresh_zero(), 1, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
    if (role == kRoleFinish) {
      // wait for the partial of block sk_s - 1, the tile's only other
      // contributor (each stream-K block owns more than one tile's
      // k-iterations); the epilogue adds it to the accumulators
      if (epi_tid() == 0) {
        int* const flag = A.sk_flags + (sk_s - 1) + fresh_zero();
        int spin = 0;
        while (__hip_atomic_load(flag, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT) == 0 &&
               ++spin < kSkSpin)
          __builtin_amdgcn_s_sleep(2);
        if (spin >= kSkSpin)
          __hip_atomic_fetch_add(A.sk_flags + A.sk_blocks + fresh_zero(), 1, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(flag, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __syncthreads();
    }
  }
  // the partial this tile's epilogue adds (stream-K finisher), read with
  // agent-coherent (sc1) loads: no cache invalidation needed
  const bool part = SK && role == kRoleFinish;
  const __amdgpu_buffer_rsrc_t rpart =
      make_rsrc(part ? A.sk_ws + (int64_t)(sk_s - 1) * kSkSlot : nullptr, part ? kSkSlot * 4 : 0);

  // lane holds tile column (n side) 128 wn + 16 i + 4 (lane / 16) + 0..3 of
  // tile row (m side) 128 wm + 16 j + lane % 16 in acc[i][j].  The epilogue
  // takes its thread index afresh (epi_tid), so no prologue value has to stay
  // live across the main loop.
  const int etid = epi_tid();
  const int elane = etid & 63;
  Lora16<HI> F;
  if constexpr (LT > 0) lora16_load<DUAL, LT, HI>(A, m0, n0, wm, wn, elane, F);
  if constexpr (EPI == EPI_STORE || EPI == EPI_DGLU) {
    // bf16(acc) is staged as a row-major tile (rows kLdOut apart: 32 lanes of
    // one 8-byte write cover the 64 banks once), then 32 threads store each
    // 512-byte row, or (B1) dglu_finish runs the dequantise + SwiGLU backward
    // on it row by row.
    static_assert(kLdOut == kDgluLd, "B1's staged tile layout");
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      // a stream-K finisher adds the other block's partial, 8 blocks at a time
      f32x4 pv[8];
      if (part) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
          pv[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                 rpart, ((i * 8 + j) * 256 + etid) * 16, 0, kSc1));
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int ml = wm * 128 + 16 * j + (elane & 15);
        const int nl = wn * 128 + 16 * i + 4 * (elane >> 4);
        f32x4 base = acc[i][j];
        // one block's accumulators at a time: read all at once, the 256
        // accumulator copies spilled the values that live across the loop
        asm volatile("" : "+v"(base));
        if (part) base += pv[j];
        const f32x4 v = LT > 0 ? acc16<false, LT, HI>(A, base, F, i, j) : base;
        *reinterpret_cast<uint2*>(lds + ml * kLdOut + nl) =
            make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
      }
    }
    __syncthreads();
    if constexpr (EPI == EPI_DGLU) {
      dglu_finish<CACHE, GS>(A, m0, n0, lds);
      return;
    }
    // ragged M and N: rows past M and 8-column pieces past N (N % 8 == 0) stay
    // unwritten; the operand loads read zeros or discarded values there
    const int cl = (etid & 31) * 8;
    const bool nok = n0 + cl < A.N;
#pragma unroll 4
    for (int p = 0; p < 32; ++p) {
      const int r = p * 8 + (etid >> 5);
      const uint4 w = *reinterpret_cast<const uint4*>(lds + r * kLdOut + cl);
      if (nok && m0 + r < A.M) *reinterpret_cast<uint4*>(A.C + (m0 + r) * A.ldc + n0 + cl) = w;
    }
  } else {
    // F1: blocks i < 4 are gate columns d = 64 wn + 16 i + ..., i >= 4 the
    // same up columns; staged as glu_finish's two tiles (rows kGluLd apart:
    // 32 lanes of one 8-byte write cover the 64 banks once)
    uint16_t* sg = lds;
    uint16_t* su = lds + 256 * kGluLd;
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int ml = wm * 128 + 16 * j + (elane & 15);
        const int dl = wn * 64 + 16 * (i & 3) + 4 * (elane >> 4);
        f32x4 v = LT > 0 ? acc16<true, LT, HI>(A, acc[i][j], F, i, j) : acc[i][j];
        asm volatile("" : "+v"(v));
        *reinterpret_cast<uint2*>((i < 4 ? sg : su) + ml * kGluLd + dl) =
            make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
      }
    __syncthreads();
    glu_finish<CACHE, GS, EPI == EPI_GLUO>(A, m0, n0, lds);
  }
}

// SK: the stream-K schedule (plain store with a K-major A only); without it
// one whole tile per block.  Two kernels, so the one-tile-per-block kernel
// keeps its own register allocation.  HI: adapter ranks 17..32 (a third
// kernel, one tile per block).
template <bool AK, bool BK, int EPI, int CACHE, int GS, int LT, bool SK, bool HI = false>
__global__ __launch_bounds__(kThreads, 1) void nt16_kernel(const KArgs A) {
  static_assert(!SK || (EPI == EPI_STORE && AK), "stream-K: plain store, K-major A");
  static_assert(!HI || (LT > 0 && !SK), "ranks above 16: adapter kernels, one tile per block");
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  const int nk = (int)(A.K[0] / kBK) + (A.npairs == 2 ? (int)(A.K[1] / kBK) : 0);
  const int b = blockIdx.x;
  if constexpr (!SK) {
    int tm, tn;
    tile_coords_of(b, gridDim.x, A.tiles_m, A.tiles_n, tm, tn);
    nt16_tile<AK, BK, EPI, CACHE, GS, LT, SK, HI>(A, lds, tm, tn, 0, nk, kRoleWhole, 0);
    return;
  }
  // A data-parallel block (b < sk_dp) has one item, its whole tile.  Stream-K
  // block s has the global iterations [lo, hi) of the logical tiles sk_dp ..
  // T - 1: sk_q each, one more for s < sk_r (32-bit: the host keeps their
  // count below 2^31), taken from its last tile to its first.
  const bool dp = b < A.sk_dp;
  // rank of the stream-K block: the blocks an XCD runs (every 8th) take
  // consecutive ranks, so an XCD's blocks share operand panels in its L2
  const int sb = b - A.sk_dp;
  const int s = (A.sk_blocks & 7) == 0 ? (sb & 7) * (A.sk_blocks >> 3) + (sb >> 3) : sb;
  const int lo = dp ? 0 : s * A.sk_q + min(s, A.sk_r);
  const int hi = dp ? nk : lo + A.sk_q + (s < A.sk_r ? 1 : 0);
  const int t_top = (hi - 1) / nk, t_bot = lo / nk;
  for (int t = t_top; t >= t_bot; --t) {
    const int ts = t * nk;
    const int kb = max(lo, ts) - ts;
    const int ke = min(hi, ts + nk) - ts;
    const int role = (kb == 0 && ke == nk) ? kRoleWhole
                     : ke < nk             ? kRolePartial
                                           : kRoleFinish;
    int tm, tn;
    if (dp) tile_coords_of(b, A.sk_dp, A.tiles_m, A.tiles_n, tm, tn);
    else logical_coords(A.sk_dp + t, A.tiles_m, A.tiles_n, tm, tn);
    if (t != t_top) __syncthreads();   // the last item's epilogue read LDS
    nt16_tile<AK, BK, EPI, CACHE, GS, LT, SK, false>(A, lds, tm, tn, kb, ke, role, s);
  }
}

}  // namespace nt16

template <bool AK, bool BK, int EPI, int CACHE, int GS, int LT>
int launch_nt16(const KArgs& A, hipStream_t st) {
  // stream-K only where it measured faster: plain stores with a K-major A
  // (gy W_d, x W^T); with an MN-major A (the weight gradients) the shared
  // tail ran 10-25% slower than one tile per block
  constexpr bool kSkOk = EPI == EPI_STORE && AK;
  auto kern = nt16::nt16_kernel<AK, BK, EPI, CACHE, GS, LT, false>;
  auto kern_sk = nt16::nt16_kernel<AK, BK, EPI, CACHE, GS, LT, kSkOk>;
  // adapter ranks 17..32 (LT == 0: the same kernel as kern)
  auto kern_hi = nt16::nt16_kernel<AK, BK, EPI, CACHE, GS, LT, false, (LT > 0)>;
  static bool attr_set = false;   // per instantiation
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                            nt16::kLds) != hipSuccess ||
        hipFuncSetAttribute((const void*)kern_sk, hipFuncAttributeMaxDynamicSharedMemorySize,
                            nt16::kLds) != hipSuccess ||
        hipFuncSetAttribute((const void*)kern_hi, hipFuncAttributeMaxDynamicSharedMemorySize,
                            nt16::kLds) != hipSuccess)
      return kErrLaunch;
    attr_set = true;
  }
  const bool hi = LT > 0 && A.lrank > 16;
  const int64_t tiles = (int64_t)A.tiles_m * A.tiles_n;
  if (tiles <= 0) return kOk;
  if (tiles > 0x7FFFFFFF) return kErrTooLarge;
  KArgs B = A;
  B.sk_dp = (int)tiles;
  B.sk_blocks = 0;
  if constexpr (kSkOk) {
    const int nk = (int)(A.K[0] / nt16::kBK) + (A.npairs == 2 ? (int)(A.K[1] / nt16::kBK) : 0);
    StreamK sk;
    // the stream-K kernels carry adapter ranks up to 16
    if (!hi && stream_k_plan(tiles, nk, sk)) {
      B.sk_dp = (int)(tiles - sk.tiles);
      B.sk_blocks = sk.blocks;
      const int64_t iters = sk.tiles * nk;   // < 2^31 (stream_k_plan)
      B.sk_q = (int)(iters / sk.blocks);
      B.sk_r = (int)(iters % sk.blocks);
      B.sk_ws = sk.ws;
      B.sk_flags = sk.flags;
    }
  }
  const int64_t grid = (int64_t)B.sk_dp + B.sk_blocks;
  hipLaunchKernelGGL(hi ? kern_hi : B.sk_blocks ? kern_sk : kern, dim3((unsigned)grid),
                     dim3(nt16::kThreads), nt16::kLds, st, B);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

}  // namespace gemm
}  // namespace cpt
