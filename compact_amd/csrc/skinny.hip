// Skinny products of the low-rank adapters: C[M, R] = alpha * A[M, K] . Q^T
// with Q [R, K] and R <= 32 (the rank).  These are the thin GEMMs of the LoRA
// terms that the reference issues through F.linear / @ (src/flashffn.py:1414,
// 1420,1439 forward: x A^T and h_mid A_d^T; :1521,1556-1557 backward: grad_y
// B_d, grad_h_gate B_g, grad_h_up B_u).
//
// They read a tall token-major operand once (x, h_mid, grad_y, grad_h_*: up
// to 180 MB) and produce a [tokens, rank] result, so they are HBM-bound: a
// 256 x 256 MFMA tile would waste 15/16 of its work and, with only M/256
// tiles, leave most CUs idle.  Here each wavefront owns 32 rows and one K
// range, loads A in whole 128-byte row lines, and passes them through its own
// piece of LDS into the A slot of v_mfma_f32_16x16x32_bf16 (8 consecutive k
// of one row per lane), with Q's fragments (a few hundred KB, L2 resident,
// loaded straight into the operand layout) in the B slot.  The last k of a
// range that do not fill a 64-wide step load straight into the A slot.  K is split across blocks so the grid has enough
// waves in flight to cover HBM latency; the fp32 partials [splits][M][R] are
// then summed in split order (deterministic) and rounded to bf16 once.
//
// 16x16x32 bf16 MFMA operand layout: lane l holds A[l % 16][8 (l / 16) + e]
// and B[8 (l / 16) + e][l % 16], e = 0..7; the result lane l holds
// D[4 (l / 16) + i][l % 16], i = 0..3.

#include <mutex>
#include <type_traits>

#include "common.h"
#include "compact_amd.h"

namespace cpt {
namespace skinny {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kOOB = 0x80000000u;   // offsets >= 2^31 read zero (records < 2^31)
constexpr int kRsrcWord3 = 0x00020000;
constexpr int kRowBlocks = 2;                  // 16-row blocks per wavefront (share Q's fragments)
constexpr int kRowsPerBlock = 4 * 16 * kRowBlocks;   // 4 wavefronts per block
constexpr int kUnroll = 4;                     // k-64 steps in flight per wavefront

// A wavefront's 32 rows x 64 k of A pass through its own 4 KiB of LDS: loaded
// as whole 128-byte row lines (lane l: row l / 8 + 8 i, k chunk l % 8, 8 rows
// per instruction) and read back in the MFMA operand layout (lane l: row
// l % 16 of a row block, k chunk l / 16 of a k-32 half).  Rows are 64
// elements with the 16-byte chunk index XORed with (row & 6): on gfx950 a
// 128-bit read serves lanes {0-7, 24-31}, {8-15, 16-23}, ... together, and
// both access patterns are then free of bank conflicts.  Loading whole lines
// instead of 64-byte row pieces straight into the operand layout took the
// C3 projections from ~235 to ~210 us per step.
__device__ __forceinline__ int stage_off(int row, int chunk) {
  return row * 64 + ((chunk ^ (row & 6)) << 3);
}

// records clamped to [0, 2^31 - 1]: resources start where a block's reads
// start, so offsets stay 32-bit for operands of any size
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, int64_t bytes) {
  const int n = bytes > 0x7FFFFFFF ? 0x7FFFFFFF : bytes < 0 ? 0 : (int)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, n, kRsrcWord3);
}

// Orders one wavefront's LDS accesses across lanes: the hardware runs them in
// issue order, and these fences stop the compiler from moving a lane's access
// across another lane's (their addresses differ, so it sees no dependence).
__device__ __forceinline__ void wave_lds_order() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ bf16x8 bload(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  return __builtin_bit_cast(bf16x8, v);
}

// NB column blocks of 16 (R <= 16 NB); each wavefront owns kRowBlocks blocks
// of 16 rows, so one Q fragment serves kRowBlocks MFMAs.  Grid:
// (ceil(M / kRowsPerBlock), splits); split s covers k in
// [s * kchunk, min(K, (s + 1) * kchunk)), kchunk % 32 == 0.
// ws != null: fp32 partials ws[(s * M + m) * R + r]; else C = bf16(alpha * acc).
template <int NB>
__global__ __launch_bounds__(256) void skinny_proj_kernel(
    const uint16_t* __restrict__ a, int64_t lda, const uint16_t* __restrict__ q, int64_t ldq,
    int64_t M, int R, int64_t K, int64_t kchunk, float* __restrict__ ws, uint16_t* __restrict__ c,
    int64_t ldc, float alpha) {
  constexpr int RB = kRowBlocks;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t m0 = ((int64_t)blockIdx.x * 4 + wave) * 16 * RB;
  if (m0 >= M) return;   // whole wavefront
  const int s = blockIdx.y;
  const int64_t k_begin = (int64_t)s * kchunk;
  const int64_t k_end = min(K, k_begin + kchunk);
  // A from the wavefront's first row: rows past M and rows of Q past R read
  // zero through the records
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(a + m0 * lda, (M - m0) * lda * 2);
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(q, (int64_t)R * ldq * 2);
  const int kq = 8 * (lane >> 4);
  uint32_t oa[RB];
#pragma unroll
  for (int b = 0; b < RB; ++b) oa[b] = (uint32_t)((((int64_t)16 * b + (lane & 15)) * lda + kq) * 2);
  uint32_t oq[NB];
#pragma unroll
  for (int t = 0; t < NB; ++t) oq[t] = (uint32_t)(((int64_t)(t * 16 + (lane & 15)) * ldq + kq) * 2);
  f32x4 acc[RB][NB];
#pragma unroll
  for (int b = 0; b < RB; ++b)
#pragma unroll
    for (int t = 0; t < NB; ++t) acc[b][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  __shared__ __attribute__((aligned(16))) uint16_t stage[4][2][32 * 64];
  uint16_t* const mine = &stage[wave][0][0];
  uint32_t ol[4];   // line loads: row l / 8 + 8 i, chunk l % 8
  int wofs[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    ol[i] = (uint32_t)((((int64_t)(lane >> 3) + 8 * i) * lda + (lane & 7) * 8) * 2);
    wofs[i] = stage_off((lane >> 3) + 8 * i, lane & 7);
  }
  int rofs[RB][2];  // operand reads: row 16 b + l % 16, chunk 4 h + l / 16
#pragma unroll
  for (int b = 0; b < RB; ++b)
#pragma unroll
    for (int h = 0; h < 2; ++h) rofs[b][h] = stage_off(16 * b + (lane & 15), 4 * h + (lane >> 4));
  int64_t k = k_begin;
  // U k-64 steps per pass: all loads first, then each step through LDS.  The
  // k order of the MFMAs is the same as one k-32 step at a time.
  auto pass = [&](auto uc) {
    constexpr int U = decltype(uc)::value;
    for (; k + 64 * U <= k_end; k += 64 * U) {
      bf16x8 lv[U][4], qv[U][2][NB];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint32_t dk = (uint32_t)((k + 64 * u) * 2);
#pragma unroll
        for (int i = 0; i < 4; ++i) lv[u][i] = bload(ra, ol[i] + dk);
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int t = 0; t < NB; ++t) qv[u][h][t] = bload(rq, oq[t] + dk + 64 * h);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        uint16_t* buf = mine + (u & 1) * 32 * 64;
#pragma unroll
        for (int i = 0; i < 4; ++i) *reinterpret_cast<bf16x8*>(buf + wofs[i]) = lv[u][i];
        wave_lds_order();   // other lanes' stores before this lane's reads
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int b = 0; b < RB; ++b) {
            const bf16x8 av = *reinterpret_cast<const bf16x8*>(buf + rofs[b][h]);
#pragma unroll
            for (int t = 0; t < NB; ++t)
              acc[b][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, qv[u][h][t], acc[b][t], 0, 0, 0);
          }
        wave_lds_order();   // these reads before the buffer's next stores
      }
    }
  };
  pass(std::integral_constant<int, kUnroll>{});
  pass(std::integral_constant<int, 1>{});
  for (; k < k_end; k += 32) {
    // K % 8 == 0 and kchunk % 32 == 0: a lane's 8-wide chunk is wholly in or out
    const bool ok = k + kq < k_end;
    const uint32_t dk = (uint32_t)(k * 2);
    bf16x8 qv[NB];
#pragma unroll
    for (int t = 0; t < NB; ++t) qv[t] = bload(rq, ok ? oq[t] + dk : kOOB);
#pragma unroll
    for (int b = 0; b < RB; ++b) {
      const bf16x8 av = bload(ra, ok ? oa[b] + dk : kOOB);
#pragma unroll
      for (int t = 0; t < NB; ++t)
        acc[b][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, qv[t], acc[b][t], 0, 0, 0);
    }
  }
#pragma unroll
  for (int b = 0; b < RB; ++b)
#pragma unroll
    for (int t = 0; t < NB; ++t) {
      const int col = t * 16 + (lane & 15);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t row = m0 + 16 * b + 4 * (lane >> 4) + i;
        if (row >= M || col >= R) continue;
        if (ws)
          ws[((int64_t)s * M + row) * R + col] = acc[b][t][i];
        else
          c[row * ldc + col] = (uint16_t)f32_to_bf16_bits(alpha * acc[b][t][i]);
      }
    }
}

// sum_s p[s * stride], s = 0 .. splits - 1, added in split order; the loads
// of 8 splits are issued together (the additions stay in order, so the sum is
// that of the one-at-a-time loop)
__device__ __forceinline__ float sum_splits(const float* __restrict__ p, int64_t stride,
                                            int splits) {
  float sum = 0.0f;
  int s = 0;
  for (; s + 8 <= splits; s += 8) {
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = p[(int64_t)(s + j) * stride];
#pragma unroll
    for (int j = 0; j < 8; ++j) sum += v[j];
  }
  for (; s < splits; ++s) sum += p[(int64_t)s * stride];
  return sum;
}

// C[m, r] = bf16(alpha * sum_s ws[s][m][r]), splits summed in order
__global__ __launch_bounds__(256) void skinny_reduce_kernel(const float* __restrict__ ws,
                                                            uint16_t* __restrict__ c, int64_t M,
                                                            int R, int64_t ldc, int splits,
                                                            float alpha) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= M * R) return;
  const float sum = sum_splits(ws + e, M * R, splits);
  const int64_t m = e / R, r = e - m * R;
  c[m * ldc + r] = (uint16_t)f32_to_bf16_bits(alpha * sum);
}

// ---------------------------------------------------------------------------
// Token reductions of the adapter gradients: Z[N, R] = alpha * X^T . P with
// X [T, N] and P [T, R] token-major (rows t), R <= 32: grad_B = s * grad_y^T
// (x A^T) and grad_A^T = s * x^T (grad B) (src/flashffn.py:1538-1545,
// 1575-1582).  The reduction runs over the tokens, which are X's strided
// dimension, so a block stages a [64 tokens x 64 columns] piece of X (and the
// matching [64 x R] piece of P) in LDS with coalesced 128-byte row loads and
// the MFMA fragments (8 consecutive tokens of one column) come out of
// ds_read_b64_tr_b16.  Each wavefront owns 16 of the 64 columns; blocks split
// the tokens, and the fp32 partials [splits][N][R] are summed in split order.
// ---------------------------------------------------------------------------
constexpr int kRedCols = 64;    // X columns per block (16 per wavefront)
constexpr int kRedTok = 64;     // tokens per step
constexpr int kRedLdX = 72;     // LDS row stride of the X piece (elements)
constexpr int kRedLdP = 40;     // LDS row stride of the P piece (elements)

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

__device__ __forceinline__ i16x4 lds_read_tr(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
}

// fragment of 8 consecutive tokens (k) of column `col` from a [tokens][ld]
// LDS piece: ds_read_b64_tr_b16 gives, within each 16-lane group, lane j the
// 4 tokens of column j of a 4 x 16 block whose rows the lanes address
// (lane s: token row s / 4, columns 4 (s % 4)); two reads make the 8
template <int LD>
__device__ __forceinline__ bf16x8 red_frag(const uint16_t* piece, int k0, int col0, int lane) {
  const int k = k0 + 8 * (lane >> 4) + ((lane & 15) >> 2);
  const int c = col0 + 4 * (lane & 3);
  const i16x4 lo = lds_read_tr(piece + k * LD + c);
  const i16x4 hi = lds_read_tr(piece + (k + 4) * LD + c);
  return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// Grid: (ceil(N / 64), splits); split s covers tokens [s * tchunk,
// min(T, (s + 1) * tchunk)), tchunk % 64 == 0.  N % 8 == 0, R % 8 == 0.
template <int NB>
__global__ __launch_bounds__(256) void skinny_red_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const uint16_t* __restrict__ p, int64_t ldp,
    int64_t T, int64_t N, int R, int64_t tchunk, float* __restrict__ ws) {
  __shared__ __attribute__((aligned(16))) uint16_t xs[2][kRedTok * kRedLdX];
  __shared__ __attribute__((aligned(16))) uint16_t ps[2][kRedTok * kRedLdP];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t n0 = (int64_t)blockIdx.x * kRedCols;
  const int s = blockIdx.y;
  const int64_t t_begin = (int64_t)s * tchunk;
  const int64_t t_end = min(T, t_begin + tchunk);
  // both from the split's first token (offsets relative to t_begin); tokens
  // past T read zero through the records; columns past N / R are masked per
  // 8-wide chunk (N % 8 == 0, R % 8 == 0)
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + t_begin * ldx, (T - t_begin) * ldx * 2);
  const __amdgpu_buffer_rsrc_t rp = make_rsrc(p + t_begin * ldp, (T - t_begin) * ldp * 2);
  // X piece: thread loads rows tid / 8 and tid / 8 + 32, columns 8 (tid % 8)
  const int xr = tid >> 3, xc = (tid & 7) * 8;
  const bool xok = n0 + xc < N;
  // P piece: 64 tokens x R (<= 32) columns, 8 columns per thread
  const int pcpr = (R + 7) / 8;                 // 8-wide chunks per token row
  const int pr = tid / 4, pc = (tid % 4) * 8;   // 4 chunks per row slot (R <= 32)
  const bool pok = pc < R;
  f32x4 acc[NB];
#pragma unroll
  for (int t = 0; t < NB; ++t) acc[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  (void)pcpr;
  uint4 vx0, vx1, vp;
  auto load = [&](int64_t t0) {
    const bool in = t0 < t_end;
    const int64_t tr = t0 - t_begin;
    const uint32_t ox0 = (uint32_t)(((tr + xr) * ldx + n0 + xc) * 2);
    const uint32_t ox1 = (uint32_t)(((tr + xr + 32) * ldx + n0 + xc) * 2);
    const uint32_t op = (uint32_t)(((tr + pr) * ldp + pc) * 2);
    auto v0 = __builtin_amdgcn_raw_buffer_load_b128(rx, (in && xok && t0 + xr < t_end) ? ox0 : kOOB, 0, 0);
    auto v1 = __builtin_amdgcn_raw_buffer_load_b128(rx, (in && xok && t0 + xr + 32 < t_end) ? ox1 : kOOB, 0, 0);
    auto v2 = __builtin_amdgcn_raw_buffer_load_b128(rp, (in && pok && t0 + pr < t_end) ? op : kOOB, 0, 0);
    vx0 = __builtin_bit_cast(uint4, v0);
    vx1 = __builtin_bit_cast(uint4, v1);
    vp = __builtin_bit_cast(uint4, v2);
  };
  auto store = [&](int buf) {
    *reinterpret_cast<uint4*>(&xs[buf][xr * kRedLdX + xc]) = vx0;
    *reinterpret_cast<uint4*>(&xs[buf][(xr + 32) * kRedLdX + xc]) = vx1;
    *reinterpret_cast<uint4*>(&ps[buf][pr * kRedLdP + pc]) = vp;
  };
  int buf = 0;
  load(t_begin);
  store(0);
  __syncthreads();
  for (int64_t t0 = t_begin; t0 < t_end; t0 += kRedTok) {
    load(t0 + kRedTok);   // next piece in flight while this one is used
#pragma unroll
    for (int kk = 0; kk < kRedTok; kk += 32) {
      const bf16x8 a = red_frag<kRedLdX>(xs[buf], kk, wave * 16, lane);
#pragma unroll
      for (int t = 0; t < NB; ++t) {
        const bf16x8 b = red_frag<kRedLdP>(ps[buf], kk, t * 16, lane);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[t], 0, 0, 0);
      }
    }
    buf ^= 1;
    store(buf);           // the other buffer was last read before the previous barrier
    __syncthreads();
  }
  float* w = ws + (int64_t)s * N * R;
#pragma unroll
  for (int t = 0; t < NB; ++t) {
    const int col = t * 16 + (lane & 15);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t n = n0 + wave * 16 + 4 * (lane >> 4) + i;
      if (n < N && col < R) w[n * R + col] = acc[t][i];
    }
  }
}

// out = bf16(alpha * sum_s ws[s][n][r]) at out[n * ldo + r] or, transposed,
// out[r * ldo + n]; splits summed in order
__global__ __launch_bounds__(256) void skinny_red_reduce_kernel(const float* __restrict__ ws,
                                                                uint16_t* __restrict__ out,
                                                                int64_t N, int R, int64_t ldo,
                                                                int trans, int splits,
                                                                float alpha) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= N * R) return;
  // consecutive threads read consecutive partials (r fastest); a transposed
  // output then takes scattered 2-byte stores (N R of them, against splits N R
  // partial reads)
  const int64_t n = e / R;
  const int64_t r = e % R;
  const float sum = sum_splits(ws + e, N * R, splits);
  out[trans ? r * ldo + n : n * ldo + r] = (uint16_t)f32_to_bf16_bits(alpha * sum);
}

// Both split sums of a skinny_dual pass in one launch: elements [0, T R) sum
// the projection's column-block partials into C, the rest the reduction's
// token-split partials into Z (each as the two kernels above)
__global__ __launch_bounds__(256) void skinny_dual_reduce_kernel(
    const float* __restrict__ ws_c, uint16_t* __restrict__ c, int64_t T, int64_t ldc,
    int csplits, float alpha_c, const float* __restrict__ ws_z, uint16_t* __restrict__ z,
    int64_t N, int64_t ldz, int z_trans, int splits, float alpha_z, int R) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e < T * R) {
    const float sum = sum_splits(ws_c + e, T * R, csplits);
    const int64_t m = e / R, r = e - m * R;
    c[m * ldc + r] = (uint16_t)f32_to_bf16_bits(alpha_c * sum);
    return;
  }
  const int64_t ez = e - T * R;
  if (ez >= N * R) return;
  const int64_t n = ez / R, r = ez % R;
  const float sum = sum_splits(ws_z + ez, N * R, splits);
  z[z_trans ? r * ldz + n : n * ldz + r] = (uint16_t)f32_to_bf16_bits(alpha_z * sum);
}

// ---------------------------------------------------------------------------
// Both adapter products of one token-major operand in one pass over it:
//   C[T, R] = X[T, N] . Q^T  (Q [R, N]: the projection, X B)
//   Z[N, R] = X^T . P        (P [T, R]: the token reduction, X^T (x A^T))
// The backward of a LoRA projection needs both of one tensor: grad_h_gate B_g
// and s grad_h_gate^T (x A_g^T) (src/flashffn.py:1556-1557,1575-1582), likewise
// grad_h_up, and grad_y B_d with s grad_y^T (h_mid A_d^T) (:1521,1538-1545).
// Apart they read the [T, N] operand (up to 180 MB) twice.
//
// Block (column block cb, token split ts): 512 columns and the split's
// tokens, 64 at a time.  Each piece [64 tokens x 512 columns] goes through LDS
// once (rows kDualLd apart) and feeds
//   - the projection: wavefront w takes the piece's tokens 16 w .. 16 w + 15
//     over all 512 columns (Q's fragments for them loaded once: the block's
//     columns are fixed), a [16, R] partial written as the column block's
//     partial of those C rows (ws_c[cb][t][r]);
//   - the reduction: wavefront w takes columns 128 w .. 128 w + 127 (8 blocks
//     of 16) over the piece's 64 tokens, accumulated over every piece of the
//     split (fragments through ds_read_b64_tr_b16, as skinny_red_kernel) and
//     written once as the split's partial of Z (ws_z[ts][n][r]).
// The next piece loads into registers while this one is used.  The partials
// are then summed in split order (deterministic) by the two reduce kernels.
// ---------------------------------------------------------------------------
constexpr int kDualCols = 512;   // X columns per block
constexpr int kDualTok = 64;     // tokens per piece (16 per wavefront for the projection)
constexpr int kDualLd = 520;     // LDS row stride of the X piece (elements)
constexpr int kDualLdP = 40;     // LDS row stride of the P piece (elements)
constexpr int kDualQLd = 32;     // LDS row stride of the staged B slice (elements, R <= 32)

template <int NB>
__global__ __launch_bounds__(256) void skinny_dual_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const uint16_t* __restrict__ q, int64_t ldq,
    const uint16_t* __restrict__ p, int64_t ldp, int64_t T, int64_t N, int R, int64_t tchunk,
    float* __restrict__ ws_c, float* __restrict__ ws_z, int qmode) {
  __shared__ __attribute__((aligned(16))) uint16_t xs[kDualTok * kDualLd];
  __shared__ __attribute__((aligned(16))) uint16_t ps[kDualTok * kDualLdP];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int cb = blockIdx.x, ts = blockIdx.y;
  const int64_t n0 = (int64_t)cb * kDualCols;
  const int64_t t_begin = (int64_t)ts * tchunk;
  const int64_t t_end = min(T, t_begin + tchunk);
  // X and P from the split's first token (32-bit offsets: the host checks the
  // split plus one piece stays below 2 GiB); tokens past t_end and columns
  // past N read zero (offsets past the records)
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + t_begin * ldx, (T - t_begin) * ldx * 2);
  const __amdgpu_buffer_rsrc_t rp = make_rsrc(p + t_begin * ldp, (T - t_begin) * ldp * 2);
  // Q as [R][ldq] (rank rows, qmode 0) or [N][ldq] (the B factor itself:
  // qmode 1 with 16-byte rows, staged through LDS; qmode 2 otherwise, 8
  // two-byte loads per fragment), read once per block
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(q, (qmode ? N : (int64_t)R) * ldq * 2);
  // X piece loads: 16 per thread, row 4 i + tid / 64, 16-byte chunk tid % 64
  const int xr = tid >> 6, xc = (tid & 63) * 8;
  const bool xok = n0 + xc < N;
  // P piece: row tid / 4, chunk tid % 4 (R <= 32)
  const int pr = tid >> 2, pc = (tid & 3) * 8;
  const bool pok = pc < R;
  // Q fragments of the block's 512 columns: k-step st (32 columns), term t
  bf16x8 qf[16][NB];
  if (qmode == 1) {
    // B [N][ldq] as stored, ldq % 8 == 0: the block's 512 rows x R ranks go
    // through LDS (xs, before the first piece) in 16-byte loads, rows
    // kDualQLd apart, and each fragment (8 consecutive rows of one rank) comes
    // back with two transposing reads
#pragma unroll
    for (int i = 0; i < kDualCols * 4 / 256; ++i) {
      const int e = i * 256 + tid, rb = e >> 2, ch = e & 3;
      const bool ok = ch * 8 < R && n0 + rb < N;
      const uint4 v = __builtin_bit_cast(
          uint4, __builtin_amdgcn_raw_buffer_load_b128(
                     rq, ok ? (uint32_t)(((n0 + rb) * ldq + ch * 8) * 2) : kOOB, 0, 0));
      *reinterpret_cast<uint4*>(&xs[rb * kDualQLd + ch * 8]) = v;
    }
    __syncthreads();
#pragma unroll
    for (int st = 0; st < 16; ++st)
#pragma unroll
      for (int t = 0; t < NB; ++t) qf[st][t] = red_frag<kDualQLd>(xs, st * 32, t * 16, lane);
    // the main loop's first barrier orders these reads before xs is rewritten
  } else {
#pragma unroll
    for (int st = 0; st < 16; ++st)
#pragma unroll
      for (int t = 0; t < NB; ++t) {
        const int64_t col = n0 + st * 32 + 8 * (lane >> 4);
        const int r = t * 16 + (lane & 15);
        if (qmode == 0) {
          qf[st][t] = bload(rq, col < N && r < R ? (uint32_t)(((int64_t)r * ldq + col) * 2) : kOOB);
        } else {
          // B as stored with a row stride that is not a multiple of 8
          uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const uint32_t off =
                col + e < N && r < R ? (uint32_t)(((col + e) * ldq + r) * 2) : kOOB;
            w[e >> 1] |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rq, off, 0, 0)
                         << ((e & 1) * 16);
          }
          qf[st][t] = __builtin_bit_cast(bf16x8, make_uint4(w[0], w[1], w[2], w[3]));
        }
      }
  }
  f32x4 az[8][NB];
#pragma unroll
  for (int c = 0; c < 8; ++c)
#pragma unroll
    for (int t = 0; t < NB; ++t) az[c][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  uint4 vx[16], vp;
  auto load = [&](int64_t t0) {
    const int64_t tr = t0 - t_begin;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = 4 * i + xr;
      const bool ok = xok && t0 + row < t_end;
      vx[i] = __builtin_bit_cast(
          uint4, __builtin_amdgcn_raw_buffer_load_b128(
                     rx, ok ? (uint32_t)(((tr + row) * ldx + n0 + xc) * 2) : kOOB, 0, 0));
    }
    const bool okp = pok && t0 + pr < t_end;
    vp = __builtin_bit_cast(
        uint4, __builtin_amdgcn_raw_buffer_load_b128(
                   rp, okp ? (uint32_t)(((tr + pr) * ldp + pc) * 2) : kOOB, 0, 0));
  };
  load(t_begin);
  for (int64_t t0 = t_begin; t0 < t_end; t0 += kDualTok) {
    __syncthreads();   // the previous piece's reads are done
#pragma unroll
    for (int i = 0; i < 16; ++i)
      *reinterpret_cast<uint4*>(&xs[(4 * i + xr) * kDualLd + xc]) = vx[i];
    *reinterpret_cast<uint4*>(&ps[pr * kDualLdP + pc]) = vp;
    __syncthreads();
    load(t0 + kDualTok);   // in flight during this piece
    // projection: tokens 16 w .. + 15 of the piece over the 512 columns
    f32x4 ac[NB];
#pragma unroll
    for (int t = 0; t < NB; ++t) ac[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int st = 0; st < 16; ++st) {
      const bf16x8 a = *reinterpret_cast<const bf16x8*>(
          &xs[(16 * wave + (lane & 15)) * kDualLd + st * 32 + 8 * (lane >> 4)]);
#pragma unroll
      for (int t = 0; t < NB; ++t)
        ac[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[st][t], ac[t], 0, 0, 0);
    }
    // reduction: 8 column blocks of 16 over the piece's 64 tokens
#pragma unroll
    for (int kk = 0; kk < kDualTok; kk += 32)
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const bf16x8 a = red_frag<kDualLd>(xs, kk, wave * 128 + c * 16, lane);
#pragma unroll
        for (int t = 0; t < NB; ++t) {
          const bf16x8 bq = red_frag<kDualLdP>(ps, kk, t * 16, lane);
          az[c][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bq, az[c][t], 0, 0, 0);
        }
      }
    // lane holds C rows 16 w + 4 (lane / 16) + i, rank t * 16 + lane % 16
#pragma unroll
    for (int t = 0; t < NB; ++t) {
      const int col = t * 16 + (lane & 15);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t tk = t0 + 16 * wave + 4 * (lane >> 4) + i;
        if (tk < t_end && col < R) ws_c[((int64_t)cb * T + tk) * R + col] = ac[t][i];
      }
    }
  }
  float* wz = ws_z + (int64_t)ts * N * R;
#pragma unroll
  for (int c = 0; c < 8; ++c)
#pragma unroll
    for (int t = 0; t < NB; ++t) {
      const int col = t * 16 + (lane & 15);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t n = n0 + wave * 128 + c * 16 + 4 * (lane >> 4) + i;
        if (n < N && col < R) wz[n * R + col] = az[c][t][i];
      }
    }
}

inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---------------------------------------------------------------------------
// Scratch for cpt_gemm_bf16_skinny_t_noalloc: the split partials live in this
// fixed device array instead of a caller workspace, for callers that cannot
// allocate (HIP graph capture, serving loops).  Each GPU holds its own copy,
// at its own address, for the life of the process; host code reaches it only
// through the address hipGetSymbolAddress returns for the current device
// (the array's name is a host-side stand-in, not a device address).  Every
// call on a GPU shares that GPU's array: calls that overlap on one GPU race.
// The kernels write every partial they later sum, so nothing needs clearing.
// ---------------------------------------------------------------------------
constexpr int64_t kScratchBytes = (int64_t)16 << 20;   // CPT_NOALLOC_SCRATCH_BYTES
static __device__ __align__(256) float scratch[kScratchBytes / 4];

constexpr int kMaxDevices = 64;

// The current device's address of `scratch`, looked up once per device.
inline int scratch_ptr(void** out) {
  static std::mutex mu;
  static void* ptrs[kMaxDevices] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return kErrLaunch;
  if (dev < 0 || dev >= kMaxDevices) return kErrShape;
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return kErrLaunch;
    ptrs[dev] = ptr;
  }
  *out = ptrs[dev];
  return kOk;
}

int skinny_t_impl(const void* x, int64_t ldx, const void* p, int64_t ldp, void* out,
                  int64_t ldo, int out_trans, int64_t T, int64_t N, int64_t R, float alpha,
                  int splits, void* workspace, int64_t workspace_bytes, void* stream);

}  // namespace skinny
}  // namespace cpt

using namespace cpt;
using namespace cpt::skinny;

extern "C" {

int cpt_gemm_bf16_skinny(const void* a, int64_t lda, const void* q, int64_t ldq, void* c,
                         int64_t ldc, int64_t M, int64_t R, int64_t K, float alpha, int splits,
                         void* workspace, void* stream) {
  if (M < 0 || R < 0 || K < 0 || splits < 1) return kErrShape;
  if (R > 32) return kErrShape;
  if (M == 0 || R == 0) return kOk;
  if (!a || !q || !c || !al16(a) || !al16(q) || (lda & 7) || (ldq & 7) || (K & 7) || lda < K ||
      ldq < K || ldc < R)
    return kErrAlign;
  // 32-bit buffer offsets from each wavefront's first row: 16 * kRowBlocks
  // rows of A, 32 of Q
  if ((16 * kRowBlocks + 1) * lda * 2 >= ((int64_t)1 << 31) || 32 * ldq * 2 >= ((int64_t)1 << 31))
    return kErrTooLarge;
  const int64_t kchunk = ((K + splits - 1) / splits + 31) / 32 * 32;
  splits = (int)(kchunk > 0 ? (K + kchunk - 1) / kchunk : 1);
  if (splits < 1) splits = 1;
  if (splits > 1 && (!workspace || ((uintptr_t)workspace & 3))) return kErrAlign;
  const int64_t blocks = (M + kRowsPerBlock - 1) / kRowsPerBlock;
  if (blocks > 0x7FFFFFFF || splits > 65535) return kErrTooLarge;
  hipStream_t st = (hipStream_t)stream;
  float* ws = splits > 1 ? (float*)workspace : nullptr;
  const dim3 grid((unsigned)blocks, (unsigned)splits);
  if (R <= 16)
    hipLaunchKernelGGL(skinny_proj_kernel<1>, grid, dim3(256), 0, st, (const uint16_t*)a, lda,
                       (const uint16_t*)q, ldq, M, (int)R, K, kchunk, ws, (uint16_t*)c, ldc, alpha);
  else
    hipLaunchKernelGGL(skinny_proj_kernel<2>, grid, dim3(256), 0, st, (const uint16_t*)a, lda,
                       (const uint16_t*)q, ldq, M, (int)R, K, kchunk, ws, (uint16_t*)c, ldc, alpha);
  if (hipGetLastError() != hipSuccess) return kErrLaunch;
  if (splits > 1) {
    const int64_t total = M * R;
    hipLaunchKernelGGL(skinny_reduce_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       st, (const float*)ws, (uint16_t*)c, M, (int)R, ldc, splits, alpha);
    if (hipGetLastError() != hipSuccess) return kErrLaunch;
  }
  return kOk;
}

}  // extern "C"

extern "C" {

int cpt_gemm_bf16_skinny_t(const void* x, int64_t ldx, const void* p, int64_t ldp, void* out,
                           int64_t ldo, int out_trans, int64_t T, int64_t N, int64_t R,
                           float alpha, int splits, void* workspace, void* stream) {
  return skinny_t_impl(x, ldx, p, ldp, out, ldo, out_trans, T, N, R, alpha, splits, workspace, -1,
                       stream);
}

int cpt_gemm_bf16_skinny_t_noalloc(const void* x, int64_t ldx, const void* p, int64_t ldp,
                                   void* out, int64_t ldo, int out_trans, int64_t T, int64_t N,
                                   int64_t R, float alpha, int splits, void* stream) {
  if (T < 0 || N < 0 || R < 0 || splits < 1 || R > 32) return kErrShape;
  if (N == 0 || R == 0) return kOk;
  void* ws = nullptr;
  if (const int rc = scratch_ptr(&ws)) return rc;
  return skinny_t_impl(x, ldx, p, ldp, out, ldo, out_trans, T, N, R, alpha, splits, ws,
                       kScratchBytes, stream);
}

}  // extern "C"

namespace cpt {
namespace skinny {

// workspace_bytes < 0: the caller's workspace holds splits * N * R floats
// (cpt_gemm_bf16_skinny_t's contract); otherwise the split partials must fit
// in workspace_bytes.
int skinny_t_impl(const void* x, int64_t ldx, const void* p, int64_t ldp, void* out,
                  int64_t ldo, int out_trans, int64_t T, int64_t N, int64_t R, float alpha,
                  int splits, void* workspace, int64_t workspace_bytes, void* stream) {
  if (T < 0 || N < 0 || R < 0 || splits < 1) return kErrShape;
  if (R > 32) return kErrShape;
  if (N == 0 || R == 0) return kOk;
  if (!x || !p || !out || !workspace || !al16(x) || !al16(p) || (ldx & 7) || (ldp & 7) ||
      (N & 7) || (R & 7) || ldx < N || ldp < R || ldo < (out_trans ? N : R) ||
      ((uintptr_t)workspace & 3))
    return kErrAlign;
  const int64_t tchunk = ((T + splits - 1) / splits + kRedTok - 1) / kRedTok * kRedTok;
  splits = (int)(tchunk > 0 ? (T + tchunk - 1) / tchunk : 1);
  if (splits < 1) splits = 1;
  // 32-bit buffer offsets from each split's first token: its tokens plus the
  // prefetched piece past its end
  if ((tchunk + 2 * kRedTok) * ldx * 2 >= ((int64_t)1 << 31) ||
      (tchunk + 2 * kRedTok) * ldp * 2 >= ((int64_t)1 << 31))
    return kErrTooLarge;
  const int64_t blocks = (N + kRedCols - 1) / kRedCols;
  if (blocks > 0x7FFFFFFF || splits > 65535) return kErrTooLarge;
  if (workspace_bytes >= 0 && (int64_t)splits * N * R * 4 > workspace_bytes) return kErrTooLarge;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)blocks, (unsigned)splits);
  if (R <= 16)
    hipLaunchKernelGGL(skinny_red_kernel<1>, grid, dim3(256), 0, st, (const uint16_t*)x, ldx,
                       (const uint16_t*)p, ldp, T, N, (int)R, tchunk, (float*)workspace);
  else
    hipLaunchKernelGGL(skinny_red_kernel<2>, grid, dim3(256), 0, st, (const uint16_t*)x, ldx,
                       (const uint16_t*)p, ldp, T, N, (int)R, tchunk, (float*)workspace);
  if (hipGetLastError() != hipSuccess) return kErrLaunch;
  const int64_t total = N * R;
  hipLaunchKernelGGL(skinny_red_reduce_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256),
                     0, st, (const float*)workspace, (uint16_t*)out, N, (int)R, ldo,
                     out_trans ? 1 : 0, splits, alpha);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

}  // namespace skinny
}  // namespace cpt

extern "C" {

int64_t cpt_gemm_bf16_skinny_dual_workspace_bytes(int64_t T, int64_t N, int64_t R, int splits) {
  if (T < 0 || N < 0 || R < 0 || splits < 1) return -1;
  const int64_t csplits = (N + kDualCols - 1) / kDualCols;
  return (csplits * T * R + (int64_t)splits * N * R) * 4;
}

int cpt_gemm_bf16_skinny_dual(const void* x, int64_t ldx, const void* q, int64_t ldq, int q_nr,
                              const void* p, int64_t ldp, void* c, int64_t ldc, float alpha_c,
                              void* z, int64_t ldz, int z_trans, float alpha_z, int64_t T,
                              int64_t N, int64_t R, int splits, void* workspace, void* stream) {
  if (T < 0 || N < 0 || R < 0 || splits < 1 || R > 32) return kErrShape;
  if (N == 0 || R == 0) return kOk;
  if (!x || !q || !p || !c || !z || !workspace || !al16(x) || !al16(q) || !al16(p) ||
      (ldx & 7) || (ldp & 7) || (N & 7) || (R & 7) || ldx < N || ldq < (q_nr ? R : N) ||
      (!q_nr && (ldq & 7)) || ldp < R || ldc < R || ldz < (z_trans ? N : R) ||
      ((uintptr_t)workspace & 3))
    return kErrAlign;
  if ((q_nr ? N : 32) * ldq * 2 >= ((int64_t)1 << 31)) return kErrTooLarge;
  const int64_t tchunk =
      ((T + splits - 1) / splits + kDualTok - 1) / kDualTok * kDualTok;
  splits = (int)(tchunk > 0 ? (T + tchunk - 1) / tchunk : 1);
  if (splits < 1) splits = 1;
  // 32-bit buffer offsets from each split's first token: its tokens plus the
  // prefetched piece past its end
  if ((tchunk + 2 * kDualTok) * ldx * 2 >= ((int64_t)1 << 31) ||
      (tchunk + 2 * kDualTok) * ldp * 2 >= ((int64_t)1 << 31))
    return kErrTooLarge;
  const int64_t csplits = (N + kDualCols - 1) / kDualCols;
  if (csplits > 0x7FFFFFFF || splits > 65535) return kErrTooLarge;
  float* ws_c = (float*)workspace;
  float* ws_z = ws_c + csplits * T * R;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)csplits, (unsigned)splits);
  // Q's form in the kernel: 0 rank rows, 1 B as stored with 16-byte rows
  // (staged through LDS), 2 B as stored otherwise
  const int qmode = !q_nr ? 0 : ((ldq & 7) == 0 && al16(q) ? 1 : 2);
  if (T > 0) {
    if (R <= 16)
      hipLaunchKernelGGL(skinny_dual_kernel<1>, grid, dim3(256), 0, st, (const uint16_t*)x, ldx,
                         (const uint16_t*)q, ldq, (const uint16_t*)p, ldp, T, N, (int)R, tchunk,
                         ws_c, ws_z, qmode);
    else
      hipLaunchKernelGGL(skinny_dual_kernel<2>, grid, dim3(256), 0, st, (const uint16_t*)x, ldx,
                         (const uint16_t*)q, ldq, (const uint16_t*)p, ldp, T, N, (int)R, tchunk,
                         ws_c, ws_z, qmode);
    if (hipGetLastError() != hipSuccess) return kErrLaunch;
  } else {
    // no tokens: C has no rows and Z is the empty sum (zero partials summed)
    splits = 0;
  }
  // both split sums in one launch
  const int64_t total = T * R + N * R;
  hipLaunchKernelGGL(skinny_dual_reduce_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256),
                     0, st, (const float*)ws_c, (uint16_t*)c, T, ldc, (int)csplits, alpha_c,
                     (const float*)ws_z, (uint16_t*)z, N, ldz, z_trans ? 1 : 0, splits, alpha_z,
                     (int)R);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

}  // extern "C"
