// MFMA bf16 GEMM engine for gfx950 with the FlashFFN epilogues fused in.
//
// C[M, N] = sum over pairs p of  A_p[M, K_p] . B_p[K_p, N]   (fp32 accumulation)
//
// Operands are bf16.  Each operand is either K-major (K contiguous: A stored
// [M][lda], B stored [N][ldb] -- the nn.Linear weight layout) or MN-major
// (A stored [K][lda], B stored [K][ldb]).  Tiles go to LDS in their memory
// layout: a K-major fragment is one 128-bit LDS read, an MN-major fragment two
// LDS transpose reads (ds_read_b64_tr_b16), so no operand is transposed in
// registers.
//
// Block tile 256 (m) x 256 (n) x 64 (k), 256 threads = 4 wavefronts in a
// 2 x 2 arrangement, each owning 128 x 128 outputs as 4 x 4 tiles of
// v_mfma_f32_32x32x16_bf16.  The MFMA "A" slot is fed from the n-side operand
// and the "B" slot from the m-side operand, so a lane ends up holding, for one
// output row m, runs of 4 consecutive output columns n: the layout the fused
// epilogues want (a quantisation group is a run of columns of one row).
//   acc[i][j][r] -> n = nw + 32 i + 8 (r / 4) + 4 (lane / 32) + r % 4
//                   m = mw + 32 j + lane % 32
// LDS: two stages x two operands x 256 x 64 bf16 in padded rows (146 KiB; see
// lds_off and lds_mn), conflict-free on gfx950's 64 banks for the fragment
// reads and for the stores of either operand layout.
// Grid: one block per output tile, block ids remapped so each XCD works on a
// contiguous range of tiles, grouped GROUP_ROWS (4) tile-rows deep for L2 reuse.
//
// This header holds the device code and the launch template; gemm.hip holds
// the host API and gemm_inst_*.hip the kernel instantiations.

#pragma once

#include <type_traits>

#include "common.h"
#include "compact_amd.h"
#include "glu_math.h"

namespace cpt {
namespace gemm {

// Compile-time loop: f(std::integral_constant<int, I>) for I in [B, E), so
// accumulator indices in the epilogues are constants and stay in registers.
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BM = 256, BN = 256, BK = 64, NTHR = 256;
constexpr int TILE_ELEMS = 256 * 72 + 32 * 8;  // one operand stage in LDS (padded rows)
constexpr int LDS_BYTES = 4 * TILE_ELEMS * 2;   // 2 stages x 2 operands (146 KiB)
#ifndef CPT_GROUP_ROWS
#define CPT_GROUP_ROWS 4
#endif
constexpr int GROUP_ROWS = CPT_GROUP_ROWS;     // tile-rows per L2 group

// K-major tiles: row r (m or n) at r * 64 + (r / 2) * 8 elements, 8-element
// (16-byte) k chunks.  LDS is 64 banks of 4 bytes on gfx950 and a 128-bit
// access takes 4 cycles of 16 lanes, so each 16-lane set must cover 64
// distinct banks.  Measured with SQ_LDS_BANK_CONFLICT on one wave's patterns:
// a read serves lanes {0-7, 24-31}, {8-15, 16-23}, {32-39, 56-63} and
// {40-47, 48-55} together; a write serves 16 consecutive lanes.  The
// 32x32x16 fragment read (lanes 0-31 take rows 0-31 at one chunk) then puts
// rows 0-7 and 24-31 together, 1-way in this layout; the stores (2 rows x 8
// chunks per 16 lanes) are 1-way too.  The address stays affine in the
// chunk, so fragment addresses are immediate offsets.
__device__ __forceinline__ int lds_off(int row, int chunk) {
  return row * 64 + ((row >> 1) << 3) + (chunk << 3);
}

// MN-major tiles are kept as they lie in memory: 64 k-rows of 256 mn, rows
// LDM = 288 elements apart (576 bytes, 64 mod 256).  Stores are plain 16-byte
// row segments (16 lanes = 256 contiguous bytes).  Fragments (8 consecutive k
// of one mn per lane) come out of the gfx950 transpose read ds_read_b64_tr_b16:
// within each 16-lane group, lane s addresses the 4 elements at k-row s / 4,
// mn 4 (s % 4) of a 4 x 16 block and lane j receives column j of it, element e
// from row e.  One read yields 4 k of the fragment, two reads make the 8.  A
// 32-lane pass reads 4 rows x 64 bytes, which the 64-byte row skew spreads over
// all 64 banks.
constexpr int LDM = 288;
__device__ __forceinline__ int lds_mn(int k, int mn) { return k * LDM + mn; }
static_assert(64 * LDM <= TILE_ELEMS, "MN-major stage must fit the stage size");

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

__device__ __forceinline__ i16x4 lds_read_tr(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
}

// ---------------------------------------------------------------------------
// registers -> LDS (the tile's global loads are in Loader / mainloop_pp)
// ---------------------------------------------------------------------------

// K-major tile: the thread holds 8 16-byte chunks q = tid + 256 it, chunk
// q % 8 (8 k) of row q / 8; 8 consecutive threads cover one 128-byte row slice.
__device__ __forceinline__ void sstore_kmajor(uint16_t* lds, int tid, const uint4 (&reg)[8]) {
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    const int q = tid + NTHR * it;
    *reinterpret_cast<uint4*>(lds + lds_off(q >> 3, q & 7)) = reg[it];
  }
}

// MN-major tile: the thread holds an 8 (k) x 8 (mn) block, k = 8 (tid / 32)
// + r, mn = 8 (tid % 32) + 0..7; its row r goes into its 16-byte mn segment,
// untransposed.
__device__ __forceinline__ void sstore_mn_row(uint16_t* lds, int tid, int r, const uint4& v) {
  *reinterpret_cast<uint4*>(lds + lds_mn((tid >> 5) * 8 + r, (tid & 31) * 8)) = v;
}
__device__ __forceinline__ void sstore_mnmajor(uint16_t* lds, int tid, const uint4 (&reg)[8]) {
#pragma unroll
  for (int r = 0; r < 8; ++r) sstore_mn_row(lds, tid, r, reg[r]);
}

// ---------------------------------------------------------------------------
// arguments
// ---------------------------------------------------------------------------
struct Operand {
  const uint16_t* p;
  int64_t ld;
};

// C = sum_p A_p . B_p ; A_p logical [M, K_p] (m-side), B_p logical [K_p, N] (n-side)
struct KArgs {
  Operand a[2], b[2];
  int64_t K[2];
  int npairs;
  const uint16_t* b_up;    // dual gate/up GEMM: up weight (layout of b[0])
  int64_t M, N;            // output extent; dual: N = 2 * D (virtual columns)
  int tiles_m, tiles_n;
  int ksplit;              // >1: split-K, block b works on k-tiles [s*kts, (s+1)*kts)
  int kt_per_split;
  // plain output
  uint16_t* C;
  int64_t ldc;
  float alpha;             // EPI_ADD scale
  float* ws;               // EPI_F32: fp32 partials [ksplit][M][N]
  // FlashFFN epilogues
  int64_t D;               // d_ff (inter)
  uint16_t* h_mid;         // F1 out (may be null)
  uint16_t* h_gate;        // F1 out (bf16 cache) / B1 in (bf16 cache)
  uint16_t* h_up;
  uint8_t* q_gate;         // F1 out / B1 in (codes)
  uint16_t* s_gate;
  uint8_t* q_up;
  uint16_t* s_up;
  uint16_t* grad_gate;     // B1 out
  uint16_t* grad_up;
  uint16_t* h_mid_hat;     // B1 out (may be null)
  // B1 outlier channels (C3): columns with slot[d] >= 0 take the stored bf16
  // value o[m * k_out + slot] after the dequantisation (slot_g null: none)
  const int16_t* slot_g;
  const int16_t* slot_u;
  uint16_t* o_g;           // (F1 with outliers writes them, B1 reads them)
  uint16_t* o_u;
  int64_t k_out;
  int64_t lgs;             // group size of the int cache a BQ operand is the GLU of
  // low-rank adapter terms applied as the epilogue reads the accumulators
  // (acc_block); lrank == 0: none
  const uint16_t* lp[2];   // P_t [M, lrank], rows lldp apart (tokens x rank)
  const uint16_t* lq[2];   // Q_t: [N, lrank] rows lrank apart (lq_km) or [lrank, N] rows lldq apart
  float lalpha[2];
  int64_t lldp, lldq;
  int lrank;
  int lq_km;
  // stream-K schedule of the 16x16x32 loop (gemm16_kernel.h): blocks
  // [0, sk_dp) take one whole tile each (logical tiles 0 .. sk_dp - 1), blocks
  // sk_dp .. sk_dp + sk_blocks - 1 share the k-iterations of the other tiles
  // evenly; fp32 partials of shared tiles go to sk_ws, one slot of 256 x 256
  // floats per block, with a ready flag per block in sk_flags (zero between
  // launches).  sk_blocks == 0: every block takes one whole tile.
  int sk_dp;
  int sk_blocks;
  int sk_q, sk_r;          // iterations per stream-K block: sk_q, +1 for the first sk_r
  float* sk_ws;
  int* sk_flags;
};

// EPI_GLUO: F1 with the outlier channels in its codec (16x16x32 loop only)
enum Epi { EPI_STORE = 0, EPI_GLU = 1, EPI_DGLU = 2, EPI_ADD = 3, EPI_F32 = 4, EPI_GLUO = 5 };
enum Cache { CACHE_NONE = 0, CACHE_BF16 = 1, CACHE_INT4 = 4, CACHE_INT8 = 8 };

// ---------------------------------------------------------------------------
// tile scheduling
// ---------------------------------------------------------------------------
// logical tile -> (tile row, tile column): GROUP_ROWS tile-rows at a time,
// column by column, so consecutive logical tiles share operand panels
__device__ __forceinline__ void logical_coords(int logical, int tiles_m, int tiles_n, int& tm,
                                               int& tn) {
  const int per_group = GROUP_ROWS * tiles_n;
  const int g = logical / per_group;
  const int first = g * GROUP_ROWS;
  const int rows = min(GROUP_ROWS, tiles_m - first);
  const int in = logical - g * per_group;
  tm = first + in % rows;
  tn = in / rows;
}

// block b of nb -> its tile.  Blocks are dispatched round-robin over the 8
// XCDs: each XCD gets a contiguous range of logical tiles so co-resident
// tiles share L2 panels.
__device__ __forceinline__ void tile_coords_of(int b, int nb, int tiles_m, int tiles_n, int& tm,
                                               int& tn) {
  const int xcd = b & 7, idx = b >> 3;
  const int base = nb >> 3, extra = nb & 7;
  logical_coords(xcd * base + min(xcd, extra) + idx, tiles_m, tiles_n, tm, tn);
}

__device__ __forceinline__ void tile_coords(int tiles_m, int tiles_n, int& tm, int& tn) {
  const int nb = gridDim.x;
  const int b = blockIdx.x;
  const int xcd = b & 7, idx = b >> 3;
  const int base = nb >> 3, extra = nb & 7;
  const int logical = xcd * base + min(xcd, extra) + idx;
  const int per_group = GROUP_ROWS * tiles_n;
  const int g = logical / per_group;
  const int first = g * GROUP_ROWS;
  const int rows = min(GROUP_ROWS, tiles_m - first);
  const int in = logical - g * per_group;
  tm = first + in % rows;
  tn = in / rows;
}

// ---------------------------------------------------------------------------
// main loop
// ---------------------------------------------------------------------------
struct Acc {
  f32x16 v[4][4];
};

// ---------------------------------------------------------------------------
// Branch-free tile loads with buffer instructions.  Every operand gets a
// buffer resource whose num_records ends at the operand's last valid byte in
// the strided direction (rows for K-major, k for MN-major), so rows past the
// edge read as zero in hardware; the remaining edge (k for K-major, mn for
// MN-major) is handled by pushing the offset past num_records (kOOB).
// Offsets are 32-bit, so every resource starts where the block's reads start:
// a K-major operand at the tile's first row (its 256 rows are all the block
// reads), an MN-major operand at the block's first k row (the start of its
// split-K range).  A K-major operand of any size works; an MN-major one as
// long as one block's k range spans < 2 GiB (the host checks both and splits
// K when needed).  num_records still ends at the operand's last row.
// ---------------------------------------------------------------------------
constexpr uint32_t kOOB = 0x80000000u;
constexpr int kRsrcWord3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, int64_t bytes) {
  const uint32_t n = bytes > 0x7FFFFFFF ? 0x7FFFFFFFu : bytes < 0 ? 0u : (uint32_t)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)n, kRsrcWord3);
}

__device__ __forceinline__ uint4 bload(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  return *reinterpret_cast<uint4*>(&v);
}

template <bool AK, bool BKM, bool DUAL, int BQ = 0>
struct Loader {
  __amdgpu_buffer_rsrc_t ra[2], rb[2], rup;
  uint32_t oa[8], ob[8];   // per-thread byte offsets at the resource start (kOOB if out)
  int64_t K[2];
  int64_t kbase[2];        // k row an MN-major resource starts at (per pair)
  int nk0;
  int64_t lda, ldb;
  // BQ (B = the GLU of an int-BQ cache, MN-major [K][D]): the code and scale
  // tensors of gate and up, and per-row byte offsets into them (kOOB if out)
  __amdgpu_buffer_rsrc_t rqg, rqu, rsg, rsu;
  uint32_t os[8];
  int64_t qrow, srow;      // bytes per k row of the codes / of the scales

  // kt0: the block's first k-tile (split-K), within pair 0
  __device__ __forceinline__ void init(const KArgs& A, int64_t m0, int64_t n0, int tid, int kt0) {
    lda = A.a[0].ld;
    ldb = A.b[0].ld;
    K[0] = A.K[0];
    K[1] = A.npairs > 1 ? A.K[1] : 0;
    nk0 = (int)((A.K[0] + BK - 1) / BK);
    kbase[0] = kt0 < nk0 ? (int64_t)kt0 * BK : 0;
    kbase[1] = 0;
    constexpr bool BK_ = BKM || DUAL;
    const int64_t nb0 = DUAL ? (n0 >> 1) : n0;   // dual: the tile's first weight row
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      if (p == 1 && A.npairs < 2) { ra[1] = ra[0]; rb[1] = rb[0]; continue; }
      const char* pa = reinterpret_cast<const char*>(A.a[p].p);
      const char* pb = reinterpret_cast<const char*>(A.b[p].p);
      // K-major: rows [m0, M) from the tile's first row; MN-major: k rows
      // [kbase, K) from the block's first k row
      ra[p] = AK ? make_rsrc(pa + m0 * lda * 2, (A.M - m0) * lda * 2)
                 : make_rsrc(pa + kbase[p] * lda * 2, (K[p] - kbase[p]) * lda * 2);
      rb[p] = BK_ ? make_rsrc(pb + nb0 * ldb * 2, ((DUAL ? A.D : A.N) - nb0) * ldb * 2)
                  : make_rsrc(pb + kbase[p] * ldb * 2, (K[p] - kbase[p]) * ldb * 2);
    }
    rup = DUAL ? make_rsrc(reinterpret_cast<const char*>(A.b_up) + nb0 * ldb * 2,
                           (A.D - nb0) * ldb * 2)
               : rb[0];
    if (AK) {
#pragma unroll
      for (int it = 0; it < 8; ++it) {
        const int64_t row = (tid >> 3) + 32 * it;
        oa[it] = (uint32_t)((row * lda + (tid & 7) * 8) * 2);
      }
    } else {
      const int64_t mn = m0 + (tid & 31) * 8;
#pragma unroll
      for (int r = 0; r < 8; ++r)
        oa[r] = mn < A.M ? (uint32_t)((((tid >> 5) * 8 + r) * lda + mn) * 2) : kOOB;
    }
    if constexpr (BQ != 0) {
      // codes [K][D] (int8) or [K][D/2] (int4 nibbles), scales fp16 [K][G];
      // rows [kbase, K) from the block's first k row, as for MN-major bf16
      qrow = BQ == 8 ? A.D : A.D / 2;
      srow = (A.D / A.lgs) * 2;
      const int64_t kb = kbase[0];
      rqg = make_rsrc(A.q_gate + kb * qrow, (K[0] - kb) * qrow);
      rqu = make_rsrc(A.q_up + kb * qrow, (K[0] - kb) * qrow);
      rsg = make_rsrc(reinterpret_cast<const char*>(A.s_gate) + kb * srow, (K[0] - kb) * srow);
      rsu = make_rsrc(reinterpret_cast<const char*>(A.s_up) + kb * srow, (K[0] - kb) * srow);
      const int64_t mn = n0 + (tid & 31) * 8;
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const int64_t kr = (tid >> 5) * 8 + r;
        ob[r] = mn < A.N ? (uint32_t)(kr * qrow + (BQ == 8 ? mn : mn / 2)) : kOOB;
        os[r] = mn < A.N ? (uint32_t)(kr * srow + (mn / A.lgs) * 2) : kOOB;
      }
    } else if (DUAL) {
#pragma unroll
      for (int it = 0; it < 8; ++it) {
        const int blk = it >> 1;
        const int64_t d = ((blk >> 1) << 6) + (tid >> 3) + 32 * (it & 1);
        ob[it] = (uint32_t)((d * ldb + (tid & 7) * 8) * 2);
      }
    } else if (BKM) {
#pragma unroll
      for (int it = 0; it < 8; ++it) {
        const int64_t row = (tid >> 3) + 32 * it;
        ob[it] = (uint32_t)((row * ldb + (tid & 7) * 8) * 2);
      }
    } else {
      const int64_t mn = n0 + (tid & 31) * 8;
#pragma unroll
      for (int r = 0; r < 8; ++r)
        ob[r] = mn < A.N ? (uint32_t)((((tid >> 5) * 8 + r) * ldb + mn) * 2) : kOOB;
    }
  }
};

struct Frags {
  bf16x8 n[4];   // n-side fragments (MFMA A slot)
  bf16x8 m[4];   // m-side fragments (MFMA B slot)
};

// One k row of 8 columns of a B operand given as the GLU of an int cache:
// the gate and up codes (int8: 8 bytes each; int4: 4 bytes of nibbles) and
// their fp16 scales.
struct RawQ {
  uint32_t g0, g1, u0, u1;
  uint32_t sg, su;
};

// h^ = bf16(SiLU(hg^) * hu^) of the 8 columns, hg^ / hu^ dequantised through
// bf16: K2's h_mid^ (src/flashffn.py:1251-1253,1298-1300), bit for bit.
template <int BITS>
__device__ __forceinline__ uint4 deq_glu8(const RawQ& q) {
  const float sg = f16_bits_to_f32((uint16_t)q.sg), su = f16_bits_to_f32((uint16_t)q.su);
  float h[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float cg, cu;
    if constexpr (BITS == 8) {
      cg = (float)(int8_t)(((e < 4 ? q.g0 : q.g1) >> (8 * (e & 3))) & 0xFFu);
      cu = (float)(int8_t)(((e < 4 ? q.u0 : q.u1) >> (8 * (e & 3))) & 0xFFu);
    } else {
      cg = (float)((q.g0 >> (4 * e)) & 0xFu) - 8.0f;
      cu = (float)((q.u0 >> (4 * e)) & 0xFu) - 8.0f;
    }
    h[e] = silu_mul1(round_bf16(cg * sg), round_bf16(cu * su));
  }
  return make_uint4(pack_bf16x2(h[0], h[1]), pack_bf16x2(h[2], h[3]), pack_bf16x2(h[4], h[5]),
                    pack_bf16x2(h[6], h[7]));
}

// MFMA fragment of an MN-major tile: 8 consecutive k (sub-step s, lane half)
// of mn row rowbase + lane % 32, as two transpose reads of 4 k each.
__device__ __forceinline__ bf16x8 frag_mn(const uint16_t* t, int rowbase, int s, int lane) {
  // lds_mn(k, mn) is affine in s and rowbase: one lane base, the rest immediates
  const int lane_ofs = lds_mn(8 * (lane >> 5) + ((lane & 15) >> 2),
                              16 * ((lane >> 4) & 1) + 4 * (lane & 3));
  const uint16_t* p = t + lane_ofs + s * 16 * LDM + rowbase;
  const i16x4 lo = lds_read_tr(p);
  const i16x4 hi = lds_read_tr(p + 4 * LDM);
  return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

template <bool AKM, bool BKM>
__device__ __forceinline__ void read_frags(const uint16_t* stage_base, int wn, int wm, int lane,
                                           int s, Frags& f) {
  const uint16_t* sa = stage_base;
  const uint16_t* sb = stage_base + TILE_ELEMS;
  // K-major fragment (row R0 + 32 i, chunk 2 s + lane / 32) sits at
  // lds_off(R0, lane / 32) + 2176 i + 16 s: one lane base, the rest immediates
  constexpr int kRowBlk = 32 * 64 + 16 * 8;   // lds_off step of 32 rows
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (BKM)
      f.n[i] = *reinterpret_cast<const bf16x8*>(
          sb + lds_off(wn * 128 + (lane & 31), lane >> 5) + i * kRowBlk + s * 16);
    else
      f.n[i] = frag_mn(sb, wn * 128 + i * 32, s, lane);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (AKM)
      f.m[j] = *reinterpret_cast<const bf16x8*>(
          sa + lds_off(wm * 128 + (lane & 31), lane >> 5) + j * kRowBlk + s * 16);
    else
      f.m[j] = frag_mn(sa, wm * 128 + j * 32, s, lane);
  }
}

template <int I0, int I1>
__device__ __forceinline__ void mfma_range(const Frags& f, Acc& acc) {
#pragma unroll
  for (int t = I0; t < I1; ++t) {
    const int i = t >> 2, j = t & 3;
    acc.v[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.n[i], f.m[j], acc.v[i][j], 0, 0, 0);
  }
}

// scheduling-group masks (LLVM AMDGPU sched_group_barrier)
constexpr int SG_MFMA = 0x008, SG_VMEM_R = 0x020, SG_DS_R = 0x100, SG_DS_W = 0x200;

template <int N, int MASK, int PER = 1>
__device__ __forceinline__ void sched_interleave() {
  // N times: one MFMA, then PER instructions of MASK
#pragma unroll
  for (int t = 0; t < N; ++t) {
    __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
    __builtin_amdgcn_sched_group_barrier(MASK, PER, 0);
  }
}

// Continuous-pipeline main loop: during k-tile kt the registers hold tile kt+1,
// which is written to the other LDS stage group by group across the four
// sub-steps, each group reloaded with tile kt+2 right after its write.  Loads
// and LDS writes are spread evenly (no burst), and each load has a whole
// k-tile to land.  Each operand goes 2 registers per group.
template <bool AK, bool BKM, bool DUAL, int BQ = 0>
__device__ __forceinline__ void mainloop_pp(const KArgs& A, int64_t m0, int64_t n0, uint16_t* lds,
                                            Acc& acc, int kt0 = 0, int kt_end = -1) {
  static_assert(BQ == 0 || (!BKM && !DUAL), "the int-cache B operand is MN-major");
  constexpr bool BK_ = BKM || DUAL;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wn = wave & 1, wm = wave >> 1;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc.v[i][j][r] = 0.0f;
  Loader<AK, BKM, DUAL, BQ> L;
  L.init(A, m0, n0, tid, kt0);
  int nk_all = L.nk0;
  if (A.npairs > 1) nk_all += (int)((A.K[1] + BK - 1) / BK);
  if (kt_end < 0 || kt_end > nk_all) kt_end = nk_all;
  // k-tiles [kt0, kt_end); the prefetch past kt_end stays inside the operands
  // or reads zero past K
  const int nk = kt_end - kt0;
  if (nk <= 0) return;   // empty range: the accumulators stay zero
  using BReg = std::conditional_t<BQ != 0, RawQ, uint4>;
  uint4 va[8];
  BReg vb[8];
  // Per-tile load state, computed once per k-tile: the pair's buffer and a
  // per-lane byte delta added to every fixed per-thread offset.  An offset at
  // or past kOOB reads zero (records < 2^31 and offsets + delta < 2^32), so
  // MN-major lanes outside the tile keep reading zero with no select, and a
  // K-major lane whose chunk lies past K gets delta kOOB (one select per
  // operand per tile, not per load).
  struct TileLd {
    __amdgpu_buffer_rsrc_t ra, rb;
    uint32_t da, db, ds;
  };
  auto tile = [&](int kt) -> TileLd {
    TileLd T;
    const int p = kt >= L.nk0 ? 1 : 0;
    const int64_t k0 = (int64_t)(kt - p * L.nk0) * BK;
    const int64_t Kp = p ? L.K[1] : L.K[0];
    T.ra = p ? L.ra[1] : L.ra[0];
    T.rb = p ? L.rb[1] : L.rb[0];
    const bool kok = k0 + (tid & 7) * 8 < Kp;
    // MN-major: rows from the resource's first k row (rows past Kp read zero)
    const int64_t kr = k0 - (p ? L.kbase[1] : L.kbase[0]);
    T.da = AK ? (kok ? (uint32_t)(k0 * 2) : kOOB) : (uint32_t)(kr * L.lda * 2);
    T.db = BK_ ? (kok ? (uint32_t)(k0 * 2) : kOOB) : (uint32_t)(kr * L.ldb * 2);
    if constexpr (BQ != 0) {
      T.db = (uint32_t)(kr * L.qrow);
      T.ds = (uint32_t)(kr * L.srow);
    } else {
      T.ds = 0;
    }
    return T;
  };
  auto ldA = [&](const TileLd& T, int it) -> uint4 { return bload(T.ra, L.oa[it] + T.da); };
  auto ldB = [&](const TileLd& T, int it) -> BReg {
    if constexpr (BQ != 0) {
      RawQ q;
      if constexpr (BQ == 8) {
        const auto g = __builtin_amdgcn_raw_buffer_load_b64(L.rqg, L.ob[it] + T.db, 0, 0);
        const auto u = __builtin_amdgcn_raw_buffer_load_b64(L.rqu, L.ob[it] + T.db, 0, 0);
        q.g0 = g[0]; q.g1 = g[1]; q.u0 = u[0]; q.u1 = u[1];
      } else {
        q.g0 = __builtin_amdgcn_raw_buffer_load_b32(L.rqg, L.ob[it] + T.db, 0, 0);
        q.u0 = __builtin_amdgcn_raw_buffer_load_b32(L.rqu, L.ob[it] + T.db, 0, 0);
        q.g1 = q.u1 = 0;
      }
      q.sg = __builtin_amdgcn_raw_buffer_load_b16(L.rsg, L.os[it] + T.ds, 0, 0);
      q.su = __builtin_amdgcn_raw_buffer_load_b16(L.rsu, L.os[it] + T.ds, 0, 0);
      return q;
    } else {
      const __amdgpu_buffer_rsrc_t r = (DUAL && ((it >> 1) & 1)) ? L.rup : T.rb;
      return bload(r, L.ob[it] + T.db);
    }
  };
  // B registers -> LDS row (the int-cache operand is turned into h^ here)
  auto stB_row = [&](uint16_t* sb, int it) {
    if constexpr (BQ != 0) sstore_mn_row(sb, tid, it, deq_glu8<BQ>(vb[it]));
    else sstore_mn_row(sb, tid, it, vb[it]);
  };
  const int wofs = lds_off(tid >> 3, tid & 7);
  // group g of tile kt: store the held registers into `stage`, reload them with tile T
  auto group = [&](int g, int stage, const TileLd& T) {
    uint16_t* sa = lds + stage * 2 * TILE_ELEMS;
    uint16_t* sb = sa + TILE_ELEMS;
    // K-major chunk q = tid + 256 it sits at lds_off(tid / 8, tid % 8) + 2176 it
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int it = 2 * g + h;
      if (AK) *reinterpret_cast<uint4*>(sa + wofs + it * 2176) = va[it];
      else sstore_mn_row(sa, tid, it, va[it]);
      va[it] = ldA(T, it);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int it = 2 * g + h;
      if constexpr (BK_) *reinterpret_cast<uint4*>(sb + wofs + it * 2176) = vb[it];
      else stB_row(sb, it);
      vb[it] = ldB(T, it);
    }
  };
  // prologue: tile 0 into stage 0, tile 1 into registers
  {
    const TileLd T0 = tile(kt0);
#pragma unroll
    for (int it = 0; it < 8; ++it) { va[it] = ldA(T0, it); vb[it] = ldB(T0, it); }
  }
  {
    uint16_t* sa = lds;
    uint16_t* sb = sa + TILE_ELEMS;
    if (AK) sstore_kmajor(sa, tid, va); else sstore_mnmajor(sa, tid, va);
    if constexpr (BK_) {
      sstore_kmajor(sb, tid, vb);
    } else {
#pragma unroll
      for (int r = 0; r < 8; ++r) stB_row(sb, r);
    }
  }
  {
    // Tile 1's loads go out in the order the loop's groups reissue them (per
    // group: A 2g, 2g+1, then B 2g, 2g+1), pinned by scheduling barriers.  The
    // loop header joins this path and the back edge, and the compiler's wait
    // before each LDS write must cover both: with the same order on both,
    // the first write of a k-tile waits for its own (oldest) load only, not
    // for most of the 16 in flight.
    const TileLd T1 = tile(kt0 + 1);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        va[2 * g + h] = ldA(T1, 2 * g + h);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        vb[2 * g + h] = ldB(T1, 2 * g + h);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  __syncthreads();
  Frags f0, f1;
  read_frags<AK, BK_>(lds, wn, wm, lane, 0, f0);
  constexpr int MASK = SG_DS_R | SG_DS_W | SG_VMEM_R;
  // memory instructions per MFMA: an MN-major operand's fragments take two
  // transpose reads each
  constexpr int PER = (AK && BK_) ? 1 : 2;
  for (int kt = 0; kt + 1 < nk; ++kt) {
    const int stage = kt & 1;
    const uint16_t* base = lds + stage * 2 * TILE_ELEMS;
    const TileLd T2 = tile(kt0 + kt + 2);
    read_frags<AK, BK_>(base, wn, wm, lane, 1, f1);
    mfma_range<0, 16>(f0, acc);
    group(0, stage ^ 1, T2);
    sched_interleave<16, MASK, PER>();
    read_frags<AK, BK_>(base, wn, wm, lane, 2, f0);
    mfma_range<0, 16>(f1, acc);
    group(1, stage ^ 1, T2);
    sched_interleave<16, MASK, PER>();
    read_frags<AK, BK_>(base, wn, wm, lane, 3, f1);
    mfma_range<0, 16>(f0, acc);
    group(2, stage ^ 1, T2);
    sched_interleave<16, MASK, PER>();
    mfma_range<0, 8>(f1, acc);
    group(3, stage ^ 1, T2);
    sched_interleave<8, MASK, 1>();
    __syncthreads();
    read_frags<AK, BK_>(lds + (stage ^ 1) * 2 * TILE_ELEMS, wn, wm, lane, 0, f0);
    mfma_range<8, 16>(f1, acc);
    sched_interleave<8, SG_DS_R, PER>();
  }
  {
    const uint16_t* base = lds + ((nk - 1) & 1) * 2 * TILE_ELEMS;
    read_frags<AK, BK_>(base, wn, wm, lane, 1, f1);
    mfma_range<0, 16>(f0, acc);
    read_frags<AK, BK_>(base, wn, wm, lane, 2, f0);
    mfma_range<0, 16>(f1, acc);
    read_frags<AK, BK_>(base, wn, wm, lane, 3, f1);
    mfma_range<0, 16>(f0, acc);
    mfma_range<0, 16>(f1, acc);
  }
  __syncthreads();
}

__device__ __forceinline__ uint32_t absbits(float x) { return __float_as_uint(x) & 0x7FFFFFFFu; }

// ---------------------------------------------------------------------------
// Low-rank adapter terms in PEFT's op order (h + s * B(A(x)),
// src/flashffn.py:1414,1420,1439,1529,1558-1566), applied to each accumulator
// block as the epilogue reads it out (acc_block):
//   acc = bf16(bf16(acc) + bf16(alpha_t * bf16(P_t . Q_t)))   term 0, then 1
// The rank is at most 16, so each 32 x 32 block of a term is one
// v_mfma_f32_32x32x16_bf16 with k past the rank read as zero; the fragments
// come straight from global memory (P and Q are a few hundred KB and stay in
// L2).  The epilogues round acc to bf16 again, which leaves these values as
// they are.  In the dual gate/up GEMM term 0 belongs to the gate columns and
// term 1 to the up columns.  The accumulators themselves are never rewritten:
// they live in AGPRs, and a pass that modified them through VALU would force
// copies of all 256.
// ---------------------------------------------------------------------------
// Fragments come through buffer loads whose records end at the operand's last
// byte, so rows past the edge (and an absent term's null P, zero records) read
// as zero without a branch; k past the rank is pushed out of range.
__device__ __forceinline__ bf16x8 lora_frag_km(__amdgpu_buffer_rsrc_t rs, int64_t ld, int64_t row,
                                               int r, int lane) {
  const int k0 = (lane >> 5) * 8;
  const uint32_t off = k0 < r ? (uint32_t)((row * ld + k0) * 2) : kOOB;
  return __builtin_bit_cast(bf16x8, bload(rs, off));
}

// Q stored [r][ld] (n contiguous): 8 k of column n, one 2-byte load each
__device__ __forceinline__ bf16x8 lora_frag_mn(__amdgpu_buffer_rsrc_t rs, int64_t ld, int64_t n,
                                               int r, int lane) {
  const int k0 = (lane >> 5) * 8;
  uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t off = k0 + e < r ? (uint32_t)(((int64_t)(k0 + e) * ld + n) * 2) : kOOB;
    w[e >> 1] |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, off, 0, 0) << ((e & 1) * 16);
  }
  return __builtin_bit_cast(bf16x8, make_uint4(w[0], w[1], w[2], w[3]));
}

// threadIdx.x for an epilogue, as a value the compiler cannot match with the
// prologue's: index arithmetic shared with the prologue would otherwise stay
// live across the main loop, which holds every VGPR, and spill to scratch.
__device__ __forceinline__ int epi_tid() {
  int t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

// The adapter fragments of one wave, loaded once per tile ahead of the
// epilogue: p[t][j] the m-side rows of P_t (block j), q[t][i] the n-side rows
// of Q_t (block i; in the dual GEMM only the blocks of term t's columns).
struct LoraFr {
  bf16x8 p[2][4];
  bf16x8 q[2][4];
};

template <bool DUAL, int LT>
__device__ __forceinline__ void lora_load(const KArgs& A, int64_t m0, int64_t n0, LoraFr& F) {
  const int tid = epi_tid();
  const int lane = tid & 63, wave = tid >> 6;
  const int wn = wave & 1, wm = wave >> 1;
  const int r = A.lrank;
#pragma unroll
  for (int t = 0; t < LT; ++t) {
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(A.lp[t], A.lp[t] ? A.M * A.lldp * 2 : 0);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      F.p[t][j] = lora_frag_km(rp, A.lldp, m0 + wm * 128 + j * 32 + (lane & 31), r, lane);
    if constexpr (DUAL) {
      // virtual columns: blocks 0, 1 are gate d0 + 64 wn + 32 i, blocks 2, 3 the same d of up
      const __amdgpu_buffer_rsrc_t rq = make_rsrc(A.lq[t], A.lq[t] ? A.D * r * 2 : 0);
#pragma unroll
      for (int ii = 0; ii < 2; ++ii)
        F.q[t][2 * t + ii] = lora_frag_km(rq, r, (n0 >> 1) + wn * 64 + ii * 32 + (lane & 31), r, lane);
    } else {
      const int64_t qbytes = A.lq_km ? A.N * r * 2 : (int64_t)r * A.lldq * 2;
      const __amdgpu_buffer_rsrc_t rq = make_rsrc(A.lq[t], qbytes);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t n = n0 + wn * 128 + i * 32 + (lane & 31);
        F.q[t][i] = A.lq_km ? lora_frag_km(rq, r, n, r, lane) : lora_frag_mn(rq, A.lldq, n, r, lane);
      }
    }
  }
}

__device__ __forceinline__ f32x16 lora_term(const f32x16& a, const bf16x8& qf, const bf16x8& pf,
                                            float alpha) {
  const f32x16 zero = {};
  const f32x16 l = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qf, pf, zero, 0, 0, 0);
  f32x16 o;
#pragma unroll
  for (int r = 0; r < 16; ++r)
    o[r] = round_bf16(round_bf16(a[r]) + round_bf16(alpha * round_bf16(l[r])));
  return o;
}

// Accumulator block (i, j) as the epilogue should see it: with the kernel's
// LT adapter terms applied.  An absent term has a null P (zero fragments) and
// alpha = -0.0, so its bf16(alpha * 0) is -0.0 and x + (-0.0) == x for every x,
// signed zeros included: no branch is needed.
template <bool DUAL, int LT>
__device__ __forceinline__ f32x16 acc_block(const KArgs& A, const Acc& acc, const LoraFr& F,
                                            int i, int j) {
  f32x16 v = acc.v[i][j];
#pragma unroll
  for (int t = 0; t < LT; ++t) {
    if (DUAL && (i >> 1) != t) continue;
    v = lora_term(v, F.q[t][i], F.p[t][j], A.lalpha[t]);
  }
  return v;
}

// ---------------------------------------------------------------------------
// epilogue: plain bf16 store.  bf16(acc) (adapter terms added) is staged
// through LDS as a row-major tile, rows 264 elements apart; 32 consecutive
// threads then store one 512-byte row, so every store instruction writes
// whole 128-byte lines.  Stored straight from the accumulator layout, each
// instruction wrote 16 bytes into each of 32 rows.  The staged stores took a
// K = 64 product (1376 tiles, almost all epilogue) from 87 to 78 us and a C2
// step from 5.625 to 5.604 ms, bit-identical.
// ---------------------------------------------------------------------------
template <int LT>
__device__ __forceinline__ void epi_store(const KArgs& A, const Acc& acc, int64_t m0, int64_t n0,
                                          uint16_t* lds) {
  constexpr int LD = 264;
  static_assert(BM * LD * 2 <= LDS_BYTES, "the staged tile must fit the main loop's LDS");
  const int tid = epi_tid();
  const int lane = tid & 63, wave = tid >> 6;
  const int wn = wave & 1, wm = wave >> 1;
  LoraFr F;
  if constexpr (LT > 0) lora_load<false, LT>(A, m0, n0, F);
  static_for<0, 4>([&](auto j) {
    const int ml = wm * 128 + j * 32 + (lane & 31);
    static_for<0, 4>([&](auto i) {
      const f32x16 a = acc_block<false, LT>(A, acc, F, i, j);
      static_for<0, 4>([&](auto g) {
        const int nl = wn * 128 + i * 32 + g * 8 + (lane >> 5) * 4;
        *reinterpret_cast<uint2*>(lds + ml * LD + nl) =
            make_uint2(pack_bf16x2(a[g * 4 + 0], a[g * 4 + 1]), pack_bf16x2(a[g * 4 + 2], a[g * 4 + 3]));
      });
    });
  });
  __syncthreads();
  const int cl = (tid & 31) * 8;
  const int64_t n = n0 + cl;
  const bool vec = ((A.ldc & 7) == 0) && ((reinterpret_cast<uintptr_t>(A.C) & 15) == 0);
#pragma unroll 4
  for (int p = 0; p < 32; ++p) {
    const int r = p * 8 + (tid >> 5);
    const int64_t m = m0 + r;
    if (m >= A.M || n >= A.N) continue;
    const uint4 w = *reinterpret_cast<const uint4*>(lds + r * LD + cl);
    uint16_t* cp = A.C + m * A.ldc + n;
    if (vec && n + 7 < A.N) {
      *reinterpret_cast<uint4*>(cp) = w;
    } else {
      const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
      for (int e = 0; e < 8 && n + e < A.N; ++e)
        cp[e] = (uint16_t)(e & 1 ? ww[e >> 1] >> 16 : ww[e >> 1] & 0xFFFFu);
    }
  }
}

// ---------------------------------------------------------------------------
// epilogue ADD: C = bf16(C + bf16(alpha * bf16(acc)))   (PEFT's h + s * B(A(x))
// in bf16: the product, the scaling and the sum are each rounded)
// ---------------------------------------------------------------------------
__device__ __forceinline__ void epi_add(const KArgs& A, const Acc& acc, int64_t m0, int64_t n0,
                                        uint16_t* lds) {
  // bf16(acc) is staged through LDS as a row-major tile; 32 consecutive
  // threads then own one row (8 columns each), so C is read and written back
  // in contiguous row segments
  constexpr int LD = 264;
  const int tid = epi_tid();
  const int lane = tid & 63, wave = tid >> 6;
  const int wn = wave & 1, wm = wave >> 1;
  static_for<0, 4>([&](auto j) {
    const int ml = wm * 128 + j * 32 + (lane & 31);
    static_for<0, 4>([&](auto i) {
      const f32x16& a = acc.v[i][j];
      static_for<0, 4>([&](auto g) {
        const int nl = wn * 128 + i * 32 + g * 8 + (lane >> 5) * 4;
        *reinterpret_cast<uint2*>(lds + ml * LD + nl) =
            make_uint2(pack_bf16x2(a[g * 4 + 0], a[g * 4 + 1]), pack_bf16x2(a[g * 4 + 2], a[g * 4 + 3]));
      });
    });
  });
  __syncthreads();
  const int cl = (tid & 31) * 8;
  const int64_t n = n0 + cl;
  const bool vec = ((A.ldc & 7) == 0) && ((reinterpret_cast<uintptr_t>(A.C) & 15) == 0);
#pragma unroll 4
  for (int p = 0; p < 32; ++p) {
    const int r = p * 8 + (tid >> 5);
    const int64_t m = m0 + r;
    if (m >= A.M || n >= A.N) continue;
    const uint4 w = *reinterpret_cast<const uint4*>(lds + r * LD + cl);
    const uint32_t aw[4] = {w.x, w.y, w.z, w.w};
    float t[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
      t[e] = round_bf16(A.alpha * __uint_as_float(e & 1 ? aw[e >> 1] & 0xFFFF0000u : aw[e >> 1] << 16));
    uint16_t* cp = A.C + m * A.ldc + n;
    if (vec && n + 7 < A.N) {
      const uint4 c = *reinterpret_cast<const uint4*>(cp);
      const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        o[e] = __uint_as_float(e & 1 ? cw[e >> 1] & 0xFFFF0000u : cw[e >> 1] << 16) + t[e];
      *reinterpret_cast<uint4*>(cp) = make_uint4(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]),
                                                 pack_bf16x2(o[4], o[5]), pack_bf16x2(o[6], o[7]));
    } else {
      for (int e = 0; e < 8; ++e) {
        if (n + e >= A.N) break;
        cp[e] = (uint16_t)f32_to_bf16_bits(bf16_to_f32(cp[e]) + t[e]);
      }
    }
  }
}

// epilogue F32: fp32 partial of this split into ws[split][M][N]
__device__ __forceinline__ void epi_f32(const KArgs& A, const Acc& acc, int64_t m0, int64_t n0,
                                        int split) {
  const int tid = epi_tid();
  const int lane = tid & 63, wave = tid >> 6;
  const int wn = wave & 1, wm = wave >> 1;
  float* base = A.ws + (int64_t)split * A.M * A.N;
  static_for<0, 4>([&](auto j) {
    const int64_t m = m0 + wm * 128 + j * 32 + (lane & 31);
    static_for<0, 4>([&](auto i) {
      static_for<0, 4>([&](auto g) {
        const int64_t n = n0 + wn * 128 + i * 32 + g * 8 + (lane >> 5) * 4;
        if (m >= A.M) return;
        if (n + 3 < A.N && (A.N & 3) == 0) {
          *reinterpret_cast<float4*>(base + m * A.N + n) =
              make_float4(acc.v[i][j][g * 4 + 0], acc.v[i][j][g * 4 + 1], acc.v[i][j][g * 4 + 2],
                          acc.v[i][j][g * 4 + 3]);
        } else {
          for (int e = 0; e < 4; ++e)
            if (n + e < A.N) base[m * A.N + n + e] = acc.v[i][j][g * 4 + e];
        }
      });
    });
  });
}


// ---------------------------------------------------------------------------
// epilogue F1: h_gate/h_up rounded to bf16 -> h_mid = SiLU(g)*u, and the
// per-group absmax codec of g and u (or their bf16 copies).
// Wave (wn, wm) holds gate in acc[0..1][j] and up in acc[2..3][j] for
// d = d0 + 64 wn + 32 i + 8 q + 4 (lane/32) + e, m = m0 + 128 wm + 32 j + lane%32.
// ---------------------------------------------------------------------------
// F1 epilogue, second half (shared by both main loops): h_gate and h_up of the
// tile sit in LDS as two row-major 256 x 128 bf16 tiles, rows kGluLd apart
// (gate at lds, up at lds + 256 kGluLd), written by the caller's staging and a
// block barrier.  16 consecutive threads own one row (8 columns each): h_mid,
// the bf16 cache or the codes go out as contiguous row segments, and a
// quantisation group is GS / 8 consecutive lanes (shuffle-xor max).
constexpr int kGluLd = 136;               // LDS row stride in bf16 (272 bytes)
constexpr int kGluLdsBytes = 2 * 256 * kGluLd * 2;

// OUTL (int caches): the outlier channels of config C3 (A.slot_g / slot_u,
// A.o_g / o_u, A.k_out): a column with slot >= 0 is copied out as bf16 to
// o[m * k_out + slot] and zeroed before the group absmax, after h_mid took
// its value (the standalone K1 with outliers, HyC-LoRA's zero-and-store).
template <int CACHE, int GS, bool OUTL = false>
__device__ __forceinline__ void glu_finish(const KArgs& A, int64_t m0, int64_t n0,
                                           const uint16_t* lds) {
  static_assert(GS >= 8 && GS <= 128 && 128 % GS == 0, "group must divide the 128-column tile");
  constexpr int BITS = CACHE == CACHE_INT4 ? 4 : 8;
  constexpr bool QUANT = CACHE == CACHE_INT4 || CACHE == CACHE_INT8;
  static_assert(!OUTL || QUANT, "outlier channels ride with an int cache");
  constexpr int LD = kGluLd;
  const int tid = epi_tid();
  const uint16_t* sg = lds;
  const uint16_t* su = lds + 256 * LD;
  const int64_t D = A.D;
  const int64_t G = D / GS;
  const int cl = (tid & 15) * 8;
  const int64_t d = (n0 >> 1) + cl;        // D % 8 == 0: 8 columns all in or all out
  const bool dok = d < D;
  // this thread's 8 columns are the same in every row: their slots once
  int slg[8], slu[8];
  uint32_t mkg = 0, mku = 0;
  if constexpr (OUTL) {
    uint4 wg = make_uint4(0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu), wu = wg;
    if (dok) {
      wg = *reinterpret_cast<const uint4*>(A.slot_g + d);
      wu = *reinterpret_cast<const uint4*>(A.slot_u + d);
    }
    const uint32_t ag[4] = {wg.x, wg.y, wg.z, wg.w}, au[4] = {wu.x, wu.y, wu.z, wu.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      slg[e] = (int16_t)((ag[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
      slu[e] = (int16_t)((au[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
      mkg |= (slg[e] >= 0 ? 1u : 0u) << e;
      mku |= (slu[e] >= 0 ? 1u : 0u) << e;
    }
  }
#pragma unroll 2
  for (int p = 0; p < 16; ++p) {
    const int r = p * 16 + (tid >> 4);
    const int64_t m = m0 + r;
    const bool ok = dok && m < A.M;
    const uint4 wg = *reinterpret_cast<const uint4*>(sg + r * LD + cl);
    const uint4 wu = *reinterpret_cast<const uint4*>(su + r * LD + cl);
    const uint32_t gw[4] = {wg.x, wg.y, wg.z, wg.w};
    const uint32_t uw[4] = {wu.x, wu.y, wu.z, wu.w};
    float g[8], u[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      g[e] = __uint_as_float(e & 1 ? gw[e >> 1] & 0xFFFF0000u : gw[e >> 1] << 16);
      u[e] = __uint_as_float(e & 1 ? uw[e >> 1] & 0xFFFF0000u : uw[e >> 1] << 16);
    }
    const int64_t off = m * D + d;
    if (A.h_mid && ok) {
      float h[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) h[e] = silu_mul1(g[e], u[e]);
      *reinterpret_cast<uint4*>(A.h_mid + off) =
          make_uint4(pack_bf16x2(h[0], h[1]), pack_bf16x2(h[2], h[3]),
                     pack_bf16x2(h[4], h[5]), pack_bf16x2(h[6], h[7]));
    }
    if constexpr (CACHE == CACHE_BF16) {
      if (ok) {
        *reinterpret_cast<uint4*>(A.h_gate + off) = wg;
        *reinterpret_cast<uint4*>(A.h_up + off) = wu;
      }
    }
    if constexpr (OUTL) {
      if (ok && (mkg | mku)) {
        uint16_t* og = A.o_g + m * A.k_out;
        uint16_t* ou = A.o_u + m * A.k_out;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if ((mkg >> e) & 1u) og[slg[e]] = (uint16_t)f32_to_bf16_bits(g[e]);
          if ((mku >> e) & 1u) ou[slu[e]] = (uint16_t)f32_to_bf16_bits(u[e]);
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        g[e] = ((mkg >> e) & 1u) ? 0.0f : g[e];
        u[e] = ((mku >> e) & 1u) ? 0.0f : u[e];
      }
    }
    if constexpr (QUANT) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const float* v = t ? u : g;
        uint32_t am = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) am = max(am, absbits(v[e]));
        am = group_max_u32<GS / 8>(am);
        const uint16_t sh = scale_bits<BITS>(am);
        const float safe = safe_scale(sh);
        const float rs = __builtin_amdgcn_rcpf(safe);
        if (!ok) continue;
        if ((tid & (GS / 8 - 1)) == 0) (t ? A.s_up : A.s_gate)[m * G + d / GS] = sh;
        uint8_t* qp = t ? A.q_up : A.q_gate;
        float z[8];
        quant_snap8<BITS>(v, rs, z);    // v is bf16 (the staged tile)
        if constexpr (BITS == 8)
          *reinterpret_cast<uint2*>(qp + off) = pack_snap8_int8(z);
        else
          *reinterpret_cast<uint32_t*>(qp + m * (D >> 1) + (d >> 1)) = pack_snap8_int4(z);
      }
    }
  }
}

template <int CACHE, int GS, int LT>
__device__ __forceinline__ void epi_glu(const KArgs& A, const Acc& acc, int64_t m0, int64_t n0,
                                        uint16_t* lds) {
  // F1: h_gate = bf16(acc gate half), h_up = bf16(acc up half) are staged
  // through LDS (glu_finish's layout), then glu_finish writes the outputs.
  static_assert(BM * kGluLd * 2 * 2 <= LDS_BYTES, "the staged tiles must fit the main loop's LDS");
  constexpr int LD = kGluLd;
  const int tid = epi_tid();
  const int lane = tid & 63, wave = tid >> 6;
  const int wn = wave & 1, wm = wave >> 1;
  const int half = lane >> 5;
  uint16_t* sg = lds;
  uint16_t* su = lds + 256 * LD;
  LoraFr F;
  if constexpr (LT > 0) lora_load<true, LT>(A, m0, n0, F);
  // acc[i][j] (i = 0, 1 gate; i = 2, 3 up) -> d = 64 wn + 32 (i & 1) + 8 q + 4 half + e
  static_for<0, 4>([&](auto j) {
    const int ml = wm * 128 + j * 32 + (lane & 31);
    static_for<0, 2>([&](auto i) {
      const f32x16 ag = acc_block<true, LT>(A, acc, F, i, j);
      const f32x16 au = acc_block<true, LT>(A, acc, F, i + 2, j);
      static_for<0, 4>([&](auto q) {
        const int dl = wn * 64 + i * 32 + q * 8 + half * 4;
        *reinterpret_cast<uint2*>(sg + ml * LD + dl) =
            make_uint2(pack_bf16x2(ag[q * 4 + 0], ag[q * 4 + 1]), pack_bf16x2(ag[q * 4 + 2], ag[q * 4 + 3]));
        *reinterpret_cast<uint2*>(su + ml * LD + dl) =
            make_uint2(pack_bf16x2(au[q * 4 + 0], au[q * 4 + 1]), pack_bf16x2(au[q * 4 + 2], au[q * 4 + 3]));
      });
    });
  });
  __syncthreads();
  glu_finish<CACHE, GS>(A, m0, n0, lds);
}

// ---------------------------------------------------------------------------
// epilogue B1: grad_h_mid = bf16(acc); dequantise the cache through bf16 (or
// read the bf16 cache); SwiGLU backward -> grad_h_gate, grad_h_up, h_mid^.
// n-side = d: d = n0 + 128 wn + 32 i + 8 q + 4 (lane/32) + e.
// ---------------------------------------------------------------------------
constexpr int kDgluLd = 264;   // B1's staged tile: LDS row stride in bf16 (528 bytes)
template <int CACHE, int GS>
__device__ __forceinline__ void dglu_finish(const KArgs& A, int64_t m0, int64_t n0,
                                            const uint16_t* lds);

template <int CACHE, int GS, int LT>
__device__ __forceinline__ void epi_dglu(const KArgs& A, const Acc& acc, int64_t m0, int64_t n0,
                                         uint16_t* lds) {
  // B1: grad_h_mid = bf16(acc) is staged through LDS as a row-major
  // 256 x 256 bf16 tile, then dglu_finish processes it row by row (the MFMA
  // layout would scatter the cache loads and stores over 32 rows per
  // instruction).
  constexpr int LD = kDgluLd;
  const int tid = epi_tid();
  const int lane = tid & 63, wave = tid >> 6;
  const int wn = wave & 1, wm = wave >> 1;
  LoraFr F;
  if constexpr (LT > 0) lora_load<false, LT>(A, m0, n0, F);
  static_for<0, 4>([&](auto j) {
    const int ml = wm * 128 + j * 32 + (lane & 31);
    static_for<0, 4>([&](auto i) {
      const f32x16 a = acc_block<false, LT>(A, acc, F, i, j);
      static_for<0, 4>([&](auto g) {
        const int nl = wn * 128 + i * 32 + g * 8 + (lane >> 5) * 4;
        *reinterpret_cast<uint2*>(lds + ml * LD + nl) =
            make_uint2(pack_bf16x2(a[g * 4 + 0], a[g * 4 + 1]), pack_bf16x2(a[g * 4 + 2], a[g * 4 + 3]));
      });
    });
  });
  __syncthreads();
  dglu_finish<CACHE, GS>(A, m0, n0, lds);
}

// B1's second half, shared by both main loops: grad_h_mid (a row-major
// 256 x 256 bf16 tile in LDS, rows kDgluLd apart) -> dequantised cache ->
// SwiGLU backward -> grad_h_gate, grad_h_up (and h_mid^).  Each row is
// processed by 32 consecutive threads owning 8 columns each, so every cache
// load and output store is a contiguous, coalesced row segment.
template <int CACHE, int GS>
__device__ __forceinline__ void dglu_finish(const KArgs& A, int64_t m0, int64_t n0,
                                            const uint16_t* lds) {
  constexpr int BITS = CACHE == CACHE_INT4 ? 4 : 8;
  constexpr int LD = kDgluLd;
  const int tid = epi_tid();
  const int64_t D = A.D;
  const int64_t G = D / GS;
  const int cl = (tid & 31) * 8;
  const int64_t d = n0 + cl;           // D % 8 == 0: the 8 columns are all in or all out
  const bool dok = d < D;
  // outlier channels among this thread's 8 columns (the same for every row)
  int sg8[8], su8[8];
  bool any_out = false;
#pragma unroll
  for (int e = 0; e < 8; ++e) sg8[e] = su8[e] = -1;
  if (CACHE != CACHE_BF16 && A.slot_g && dok) {
    const uint4 wg = *reinterpret_cast<const uint4*>(A.slot_g + d);
    const uint4 wu = *reinterpret_cast<const uint4*>(A.slot_u + d);
    const uint32_t ag[4] = {wg.x, wg.y, wg.z, wg.w}, au[4] = {wu.x, wu.y, wu.z, wu.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      sg8[e] = (int16_t)((ag[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
      su8[e] = (int16_t)((au[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
      any_out |= sg8[e] >= 0 || su8[e] >= 0;
    }
  }
  // Rows go UNROLL at a time, software-pipelined: the cache loads of the next
  // rows are issued before this batch's stores.  A wait for a load also waits
  // for the stores issued before it (one counter for both), so loads issued
  // after a batch's stores would stall on them.
  constexpr int UNROLL = 4;
  uint4 dh[UNROLL];
  uint4 cg[UNROLL], cu[UNROLL];    // codes (low bytes used) or bf16 cache
  float sgv[UNROLL], suv[UNROLL];
  bool ok[UNROLL];
  int64_t mrow[UNROLL];
  auto load_rows = [&](int p0) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int r = (p0 + u) * 8 + (tid >> 5);
      const int64_t m = m0 + r;
      mrow[u] = m;
      ok[u] = dok && m < A.M;
      dh[u] = *reinterpret_cast<const uint4*>(lds + r * LD + cl);
      cg[u] = cu[u] = make_uint4(0, 0, 0, 0);
      sgv[u] = suv[u] = 0.0f;
      if (ok[u]) {
        if constexpr (CACHE == CACHE_BF16) {
          cg[u] = *reinterpret_cast<const uint4*>(A.h_gate + m * D + d);
          cu[u] = *reinterpret_cast<const uint4*>(A.h_up + m * D + d);
        } else {
          sgv[u] = f16_bits_to_f32(A.s_gate[m * G + d / GS]);
          suv[u] = f16_bits_to_f32(A.s_up[m * G + d / GS]);
          if constexpr (BITS == 8) {
            const uint2 wg = *reinterpret_cast<const uint2*>(A.q_gate + m * D + d);
            const uint2 wu = *reinterpret_cast<const uint2*>(A.q_up + m * D + d);
            cg[u] = make_uint4(wg.x, wg.y, 0, 0);
            cu[u] = make_uint4(wu.x, wu.y, 0, 0);
          } else {
            cg[u].x = *reinterpret_cast<const uint32_t*>(A.q_gate + m * (D >> 1) + (d >> 1));
            cu[u].x = *reinterpret_cast<const uint32_t*>(A.q_up + m * (D >> 1) + (d >> 1));
          }
        }
      }
    }
  };
  load_rows(0);
#pragma unroll 1
  for (int p0 = 0; p0 < 32; p0 += UNROLL) {
    uint4 og4[UNROLL], ou4[UNROLL], oh4[UNROLL];
    bool ok_now[UNROLL];
    int64_t off_now[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      ok_now[u] = ok[u];
      off_now[u] = mrow[u] * D + d;
      if (!ok[u]) continue;
      float hg[8], hu[8], dhf[8];
      const uint32_t dw[4] = {dh[u].x, dh[u].y, dh[u].z, dh[u].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) dhf[e] = __uint_as_float(e & 1 ? dw[e >> 1] & 0xFFFF0000u : dw[e >> 1] << 16);
      if constexpr (CACHE == CACHE_BF16) {
        const uint32_t wg[4] = {cg[u].x, cg[u].y, cg[u].z, cg[u].w};
        const uint32_t wu[4] = {cu[u].x, cu[u].y, cu[u].z, cu[u].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          hg[e] = __uint_as_float(e & 1 ? wg[e >> 1] & 0xFFFF0000u : wg[e >> 1] << 16);
          hu[e] = __uint_as_float(e & 1 ? wu[e >> 1] & 0xFFFF0000u : wu[e >> 1] << 16);
        }
      } else if constexpr (BITS == 8) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t wg = e < 4 ? cg[u].x : cg[u].y, wu = e < 4 ? cu[u].x : cu[u].y;
          hg[e] = round_bf16((float)(int8_t)((wg >> (8 * (e & 3))) & 0xFFu) * sgv[u]);
          hu[e] = round_bf16((float)(int8_t)((wu >> (8 * (e & 3))) & 0xFFu) * suv[u]);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          hg[e] = round_bf16(((float)((cg[u].x >> (4 * e)) & 0xFu) - 8.0f) * sgv[u]);
          hu[e] = round_bf16(((float)((cu[u].x >> (4 * e)) & 0xFu) - 8.0f) * suv[u]);
        }
      }
      if (CACHE != CACHE_BF16 && any_out) {
        // outlier columns: the stored bf16 value replaces the dequantised one
        // (HyC-LoRA's zero-and-overwrite, restored after the bf16 round trip)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if (sg8[e] >= 0) hg[e] = bf16_to_f32(A.o_g[mrow[u] * A.k_out + sg8[e]]);
          if (su8[e] >= 0) hu[e] = bf16_to_f32(A.o_u[mrow[u] * A.k_out + su8[e]]);
        }
      }
      float og[8], ou[8], oh[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float hact;
        swiglu_bwd1(dhf[e], hg[e], hu[e], og[e], ou[e], hact);
        oh[e] = hact * hu[e];
      }
      og4[u] = make_uint4(pack_bf16x2(og[0], og[1]), pack_bf16x2(og[2], og[3]),
                          pack_bf16x2(og[4], og[5]), pack_bf16x2(og[6], og[7]));
      ou4[u] = make_uint4(pack_bf16x2(ou[0], ou[1]), pack_bf16x2(ou[2], ou[3]),
                          pack_bf16x2(ou[4], ou[5]), pack_bf16x2(ou[6], ou[7]));
      oh4[u] = make_uint4(pack_bf16x2(oh[0], oh[1]), pack_bf16x2(oh[2], oh[3]),
                          pack_bf16x2(oh[4], oh[5]), pack_bf16x2(oh[6], oh[7]));
    }
    if (p0 + UNROLL < 32) load_rows(p0 + UNROLL);
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      if (!ok_now[u]) continue;
      *reinterpret_cast<uint4*>(A.grad_gate + off_now[u]) = og4[u];
      *reinterpret_cast<uint4*>(A.grad_up + off_now[u]) = ou4[u];
      if (A.h_mid_hat) *reinterpret_cast<uint4*>(A.h_mid_hat + off_now[u]) = oh4[u];
    }
  }
}

// ---------------------------------------------------------------------------
// kernel
// ---------------------------------------------------------------------------
template <bool AK, bool BKM, int EPI, int CACHE, int GS, int LT = 0>
__global__ __launch_bounds__(NTHR, 1) void gemm_kernel(KArgs A) {
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  int tm, tn, split = 0;
  if (A.ksplit > 1) {
    const int tiles = A.tiles_m * A.tiles_n;
    const int t = blockIdx.x % tiles;
    split = blockIdx.x / tiles;
    tm = t % A.tiles_m;
    tn = t / A.tiles_m;
  } else {
    tile_coords(A.tiles_m, A.tiles_n, tm, tn);
  }
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  Acc acc;
  if constexpr (EPI == EPI_F32) {
    mainloop_pp<AK, BKM, false>(A, m0, n0, lds, acc, split * A.kt_per_split,
                                (split + 1) * A.kt_per_split);
    epi_f32(A, acc, m0, n0, split);
    return;
  } else {
    // a plain-store kernel instantiated with an int cache multiplies by the
    // GLU of that cache (B = h^, the wgrad of the down projection)
    constexpr int BQ = (EPI == EPI_STORE && CACHE == CACHE_INT8) ? 8
                       : (EPI == EPI_STORE && CACHE == CACHE_INT4) ? 4 : 0;
    mainloop_pp<AK, BKM, EPI == EPI_GLU, BQ>(A, m0, n0, lds, acc);
  }
  if constexpr (EPI == EPI_STORE) epi_store<LT>(A, acc, m0, n0, lds);
  else if constexpr (EPI == EPI_ADD) epi_add(A, acc, m0, n0, lds);
  else if constexpr (EPI == EPI_GLU) epi_glu<CACHE, GS, LT>(A, acc, m0, n0, lds);
  else if constexpr (EPI == EPI_DGLU) epi_dglu<CACHE, GS, LT>(A, acc, m0, n0, lds);
}

// ---------------------------------------------------------------------------
// launch: one block per output tile (times the split-K factor)
// ---------------------------------------------------------------------------
template <bool AK, bool BKM, int EPI, int CACHE, int GS, int LT = 0>
int launch(KArgs& A, hipStream_t st) {
  auto kern = gemm_kernel<AK, BKM, EPI, CACHE, GS, LT>;
  static bool attr_set = false;   // per instantiation
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                            LDS_BYTES) != hipSuccess)
      return kErrLaunch;
    attr_set = true;
  }
  const int64_t tiles = (int64_t)A.tiles_m * A.tiles_n * (A.ksplit > 1 ? A.ksplit : 1);
  if (tiles <= 0) return kOk;
  if (tiles > 0x7FFFFFFF) return kErrTooLarge;
  hipLaunchKernelGGL(kern, dim3((unsigned)tiles), dim3(NTHR), LDS_BYTES, st, A);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

// Products on the 16x16x32 direct-to-LDS main loop (gemm16_kernel.h), K of
// each pair a multiple of 64, adapter terms (LT) with a K-major A: EPI_STORE
// in every operand layout with N a multiple of 8 and C rows 16-byte aligned
// (nt16_fits); EPI_GLU (F1, both operands K-major, one pair).  M, N and d_ff
// need not fill whole tiles.
bool nt16_fits(int64_t M, int64_t N, int64_t K, const void* c, int64_t ldc);

// Stream-K plan of a plain-store product on the 16x16x32 loop (gemm16.hip):
// true when the current device has a stream-K workspace attached and `tiles`
// tiles of `nk` k-tiles leave a part-empty last wave.  Then the last `tiles`
// of the plan's logical tiles go to `blocks` stream-K blocks.
struct StreamK {
  int64_t tiles;
  int blocks;
  float* ws;
  int* flags;
};
bool stream_k_plan(int64_t tiles, int nk, StreamK& sk);
int64_t stream_k_bytes(int cus);
template <bool AK, bool BK, int EPI, int CACHE, int GS, int LT>
int launch_nt16(const KArgs& A, hipStream_t st);

// ---------------------------------------------------------------------------
// Instantiations of launch<AK, BKM, EPI, CACHE, GS, LT>.  Each group is
// compiled in its own translation unit (gemm_inst_*.hip) so the kernels
// build in parallel; gemm.hip declares them all extern.
// ---------------------------------------------------------------------------
#define CPT_GEMM_INST_STORE(X)                                               \
  X(true, true, EPI_STORE, 0, 0, 0) X(true, false, EPI_STORE, 0, 0, 0)       \
  X(false, false, EPI_STORE, 0, 0, 0) X(false, true, EPI_STORE, 0, 0, 0)     \
  X(true, true, EPI_STORE, 0, 0, 1) X(true, false, EPI_STORE, 0, 0, 1)       \
  X(true, true, EPI_STORE, 0, 0, 2) X(true, false, EPI_STORE, 0, 0, 2)
#define CPT_GEMM_INST_AUX(X)                                                 \
  X(true, true, EPI_ADD, 0, 0, 0) X(true, false, EPI_ADD, 0, 0, 0)           \
  X(false, false, EPI_ADD, 0, 0, 0) X(false, true, EPI_ADD, 0, 0, 0)         \
  X(true, true, EPI_F32, 0, 0, 0) X(true, false, EPI_F32, 0, 0, 0)           \
  X(false, false, EPI_F32, 0, 0, 0) X(false, true, EPI_F32, 0, 0, 0)
#define CPT_GEMM_INST_GLU_A(X)                                               \
  X(true, true, EPI_GLU, CACHE_NONE, 64, 0) X(true, true, EPI_GLU, CACHE_NONE, 64, 2) \
  X(true, true, EPI_GLU, CACHE_BF16, 64, 0) X(true, true, EPI_GLU, CACHE_BF16, 64, 2) \
  X(true, true, EPI_GLU, CACHE_INT4, 32, 0) X(true, true, EPI_GLU, CACHE_INT4, 32, 2) \
  X(true, true, EPI_GLU, CACHE_INT4, 64, 0) X(true, true, EPI_GLU, CACHE_INT4, 64, 2) \
  X(true, true, EPI_GLU, CACHE_INT4, 128, 0) X(true, true, EPI_GLU, CACHE_INT4, 128, 2)
#define CPT_GEMM_INST_GLU_B(X)                                               \
  X(true, true, EPI_GLU, CACHE_INT8, 32, 0) X(true, true, EPI_GLU, CACHE_INT8, 32, 2) \
  X(true, true, EPI_GLU, CACHE_INT8, 64, 0) X(true, true, EPI_GLU, CACHE_INT8, 64, 2) \
  X(true, true, EPI_GLU, CACHE_INT8, 128, 0) X(true, true, EPI_GLU, CACHE_INT8, 128, 2)
#define CPT_GEMM_INST_DGLU_A(X)                                              \
  X(true, false, EPI_DGLU, CACHE_BF16, 64, 0) X(true, false, EPI_DGLU, CACHE_BF16, 64, 1) \
  X(true, false, EPI_DGLU, CACHE_INT4, 32, 0) X(true, false, EPI_DGLU, CACHE_INT4, 32, 1) \
  X(true, false, EPI_DGLU, CACHE_INT4, 64, 0) X(true, false, EPI_DGLU, CACHE_INT4, 64, 1) \
  X(true, false, EPI_DGLU, CACHE_INT4, 128, 0) X(true, false, EPI_DGLU, CACHE_INT4, 128, 1)
#define CPT_GEMM_INST_DGLU_B(X)                                              \
  X(true, false, EPI_DGLU, CACHE_INT8, 32, 0) X(true, false, EPI_DGLU, CACHE_INT8, 32, 1) \
  X(true, false, EPI_DGLU, CACHE_INT8, 64, 0) X(true, false, EPI_DGLU, CACHE_INT8, 64, 1) \
  X(true, false, EPI_DGLU, CACHE_INT8, 128, 0) X(true, false, EPI_DGLU, CACHE_INT8, 128, 1)
#define CPT_GEMM_INST_WGLU(X)                                                \
  X(false, false, EPI_STORE, CACHE_INT8, 32, 0) X(false, false, EPI_STORE, CACHE_INT8, 64, 0) \
  X(false, false, EPI_STORE, CACHE_INT8, 128, 0) X(false, false, EPI_STORE, CACHE_INT4, 32, 0) \
  X(false, false, EPI_STORE, CACHE_INT4, 64, 0) X(false, false, EPI_STORE, CACHE_INT4, 128, 0)
#define CPT_GEMM_INST_ALL(X)                                                 \
  CPT_GEMM_INST_STORE(X) CPT_GEMM_INST_AUX(X) CPT_GEMM_INST_GLU_A(X)         \
  CPT_GEMM_INST_GLU_B(X) CPT_GEMM_INST_DGLU_A(X) CPT_GEMM_INST_DGLU_B(X)     \
  CPT_GEMM_INST_WGLU(X)
#define CPT_NT16_INST_STORE(X)                                               \
  X(true, true, EPI_STORE, 0, 0, 0) X(true, false, EPI_STORE, 0, 0, 0)       \
  X(false, false, EPI_STORE, 0, 0, 0) X(false, true, EPI_STORE, 0, 0, 0)     \
  X(true, true, EPI_STORE, 0, 0, 1) X(true, false, EPI_STORE, 0, 0, 1)       \
  X(true, true, EPI_STORE, 0, 0, 2) X(true, false, EPI_STORE, 0, 0, 2)
#define CPT_NT16_INST_GLU_A(X)                                               \
  X(true, true, EPI_GLU, CACHE_NONE, 64, 0) X(true, true, EPI_GLU, CACHE_NONE, 64, 2) \
  X(true, true, EPI_GLU, CACHE_BF16, 64, 0) X(true, true, EPI_GLU, CACHE_BF16, 64, 2)
#define CPT_NT16_INST_GLU_B(X)                                               \
  X(true, true, EPI_GLU, CACHE_INT8, 32, 0) X(true, true, EPI_GLU, CACHE_INT8, 32, 2) \
  X(true, true, EPI_GLU, CACHE_INT8, 64, 0) X(true, true, EPI_GLU, CACHE_INT8, 64, 2) \
  X(true, true, EPI_GLU, CACHE_INT8, 128, 0) X(true, true, EPI_GLU, CACHE_INT8, 128, 2)
#define CPT_NT16_INST_GLU_C(X)                                               \
  X(true, true, EPI_GLU, CACHE_INT4, 32, 0) X(true, true, EPI_GLU, CACHE_INT4, 32, 2) \
  X(true, true, EPI_GLU, CACHE_INT4, 64, 0) X(true, true, EPI_GLU, CACHE_INT4, 64, 2) \
  X(true, true, EPI_GLU, CACHE_INT4, 128, 0) X(true, true, EPI_GLU, CACHE_INT4, 128, 2)
#define CPT_NT16_INST_DGLU_A(X)                                              \
  X(true, false, EPI_DGLU, CACHE_BF16, 64, 0) X(true, false, EPI_DGLU, CACHE_BF16, 64, 1) \
  X(true, false, EPI_DGLU, CACHE_INT4, 32, 0) X(true, false, EPI_DGLU, CACHE_INT4, 32, 1) \
  X(true, false, EPI_DGLU, CACHE_INT4, 64, 0) X(true, false, EPI_DGLU, CACHE_INT4, 64, 1) \
  X(true, false, EPI_DGLU, CACHE_INT4, 128, 0) X(true, false, EPI_DGLU, CACHE_INT4, 128, 1)
#define CPT_NT16_INST_DGLU_B(X)                                              \
  X(true, false, EPI_DGLU, CACHE_INT8, 32, 0) X(true, false, EPI_DGLU, CACHE_INT8, 32, 1) \
  X(true, false, EPI_DGLU, CACHE_INT8, 64, 0) X(true, false, EPI_DGLU, CACHE_INT8, 64, 1) \
  X(true, false, EPI_DGLU, CACHE_INT8, 128, 0) X(true, false, EPI_DGLU, CACHE_INT8, 128, 1)
#define CPT_NT16_INST_GLUO(X)                                                \
  X(true, true, EPI_GLUO, CACHE_INT4, 32, 0) X(true, true, EPI_GLUO, CACHE_INT4, 32, 2) \
  X(true, true, EPI_GLUO, CACHE_INT4, 64, 0) X(true, true, EPI_GLUO, CACHE_INT4, 64, 2) \
  X(true, true, EPI_GLUO, CACHE_INT4, 128, 0) X(true, true, EPI_GLUO, CACHE_INT4, 128, 2) \
  X(true, true, EPI_GLUO, CACHE_INT8, 32, 0) X(true, true, EPI_GLUO, CACHE_INT8, 32, 2) \
  X(true, true, EPI_GLUO, CACHE_INT8, 64, 0) X(true, true, EPI_GLUO, CACHE_INT8, 64, 2) \
  X(true, true, EPI_GLUO, CACHE_INT8, 128, 0) X(true, true, EPI_GLUO, CACHE_INT8, 128, 2)
#define CPT_NT16_INST_ALL(X)                                                 \
  CPT_NT16_INST_STORE(X) CPT_NT16_INST_GLU_A(X) CPT_NT16_INST_GLU_B(X) CPT_NT16_INST_GLU_C(X) \
  CPT_NT16_INST_DGLU_A(X) CPT_NT16_INST_DGLU_B(X) CPT_NT16_INST_GLUO(X)
#define CPT_NT16_DEFINE(AK, BK, EPI, CACHE, GS, LT) \
  template int launch_nt16<AK, BK, EPI, CACHE, GS, LT>(const KArgs&, hipStream_t);
#define CPT_NT16_DECLARE(AK, BK, EPI, CACHE, GS, LT) \
  extern template int launch_nt16<AK, BK, EPI, CACHE, GS, LT>(const KArgs&, hipStream_t);
#define CPT_GEMM_DEFINE(AK, BKM, EPI, CACHE, GS, LT) \
  template int launch<AK, BKM, EPI, CACHE, GS, LT>(KArgs&, hipStream_t);
#define CPT_GEMM_DECLARE(AK, BKM, EPI, CACHE, GS, LT) \
  extern template int launch<AK, BKM, EPI, CACHE, GS, LT>(KArgs&, hipStream_t);

}  // namespace gemm
}  // namespace cpt
