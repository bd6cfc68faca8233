// Host API of the MFMA bf16 GEMM engine (kernels in gemm_kernel.h): argument
// checks, operand layouts, adapter terms and the dispatch to the kernel
// instantiations, plus the small split-K reduce and thin LoRA-add kernels.

#include "gemm_kernel.h"

namespace cpt {
namespace gemm {

CPT_GEMM_INST_ALL(CPT_GEMM_DECLARE)
CPT_NT16_INST_ALL(CPT_NT16_DECLARE)

// out[m, n] = bf16(alpha * sum_s ws[s][m][n])  (split-K reduction, fixed order)
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ ws,
                                                            uint16_t* __restrict__ out, int64_t M,
                                                            int64_t N, int64_t ldc, int splits,
                                                            float alpha) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= M * N) return;
  // splits added in order; the loads of 8 splits are issued together
  float sum = 0.0f;
  int s = 0;
  for (; s + 8 <= splits; s += 8) {
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = ws[(int64_t)(s + j) * M * N + e];
#pragma unroll
    for (int j = 0; j < 8; ++j) sum += v[j];
  }
  for (; s < splits; ++s) sum += ws[(int64_t)s * M * N + e];
  const int64_t m = e / N, n = e - m * N;
  out[m * ldc + n] = (uint16_t)f32_to_bf16_bits(alpha * sum);
}

// ---------------------------------------------------------------------------
// thin LoRA add: C = bf16(C + bf16(alpha * bf16(A . B))) for K <= 16 (the
// rank).  The product is K multiply-adds per output, so the op is the
// read-modify-write of C: one thread owns 8 columns of a 256-column strip,
// keeps B's 8 x K values in registers and walks 32 rows, reading and writing
// C in 16-byte row segments.  Products of bf16 values are exact in fp32, so
// the fp32 sum matches an MFMA's up to summation order.
// ---------------------------------------------------------------------------
constexpr int kThinK = 16;
constexpr int kThinRows = 256;

template <bool AVEC, int BVEC>
__global__ __launch_bounds__(256) void thin_add_kernel(const uint16_t* __restrict__ a, int64_t sam,
                                                       int64_t sak, const uint16_t* __restrict__ b,
                                                       int64_t sbk, int64_t sbn, uint16_t* c,
                                                       int64_t ldc, int64_t M, int64_t N, int K,
                                                       float alpha, bool cvec) {
  constexpr int RU = 4;   // rows in flight per thread
  const int tid = threadIdx.x;
  const int64_t n = (int64_t)blockIdx.x * 256 + (tid & 31) * 8;
  if (n >= N) return;
  float bw[8][kThinK];
  if constexpr (BVEC == 2) {   // MN-major B: one 16-byte load of the 8 columns per k
#pragma unroll
    for (int k = 0; k < kThinK; ++k) {
      const uint4 w4 = (k < K && n + 7 < N) ? *reinterpret_cast<const uint4*>(b + k * sbk + n)
                                           : make_uint4(0, 0, 0, 0);
      const uint32_t w[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
      for (int e = 0; e < 8; ++e)
        bw[e][k] = __uint_as_float(e & 1 ? w[e >> 1] & 0xFFFF0000u : w[e >> 1] << 16);
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    if constexpr (BVEC == 2) {
      // loaded above
    } else if constexpr (BVEC == 1) {   // K-major B with K == 16: two 16-byte loads per column
      const bool ok = n + e < N;
      const uint4* bp = reinterpret_cast<const uint4*>(b + (n + e) * sbn);
      const uint4 w0 = ok ? bp[0] : make_uint4(0, 0, 0, 0), w1 = ok ? bp[1] : make_uint4(0, 0, 0, 0);
      const uint32_t w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
      for (int k = 0; k < kThinK; ++k)
        bw[e][k] = __uint_as_float(k & 1 ? w[k >> 1] & 0xFFFF0000u : w[k >> 1] << 16);
    } else {
#pragma unroll
      for (int k = 0; k < kThinK; ++k)
        bw[e][k] = (k < K && n + e < N) ? bf16_to_f32(b[k * sbk + (n + e) * sbn]) : 0.0f;
    }
  }
  const int64_t m0 = (int64_t)blockIdx.y * kThinRows;
  const int64_t m1 = m0 + kThinRows < M ? m0 + kThinRows : M;
  for (int64_t mb = m0 + (tid >> 5); mb < m1; mb += 8 * RU) {
    uint4 aw[RU][2], cw[RU];
    bool ok[RU];
#pragma unroll
    for (int q = 0; q < RU; ++q) {
      const int64_t m = mb + 8 * q;
      ok[q] = m < m1;
      aw[q][0] = aw[q][1] = cw[q] = make_uint4(0, 0, 0, 0);
      if (!ok[q]) continue;
      if constexpr (AVEC) {
        const uint4* ap = reinterpret_cast<const uint4*>(a + m * sam);
        aw[q][0] = ap[0];
        aw[q][1] = ap[1];
      }
      if (cvec && n + 7 < N) cw[q] = *reinterpret_cast<const uint4*>(c + m * ldc + n);
    }
#pragma unroll
    for (int q = 0; q < RU; ++q) {
      if (!ok[q]) continue;
      const int64_t m = mb + 8 * q;
      float av[kThinK];
      if constexpr (AVEC) {
        const uint32_t w[8] = {aw[q][0].x, aw[q][0].y, aw[q][0].z, aw[q][0].w,
                               aw[q][1].x, aw[q][1].y, aw[q][1].z, aw[q][1].w};
#pragma unroll
        for (int k = 0; k < kThinK; ++k)
          av[k] = __uint_as_float(k & 1 ? w[k >> 1] & 0xFFFF0000u : w[k >> 1] << 16);
      } else {
#pragma unroll
        for (int k = 0; k < kThinK; ++k) av[k] = k < K ? bf16_to_f32(a[m * sam + k * sak]) : 0.0f;
      }
      float t[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < kThinK; ++k) acc += av[k] * bw[e][k];
        t[e] = round_bf16(alpha * round_bf16(acc));
      }
      uint16_t* cp = c + m * ldc + n;
      if (cvec && n + 7 < N) {
        const uint32_t w[4] = {cw[q].x, cw[q].y, cw[q].z, cw[q].w};
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
          o[e] = __uint_as_float(e & 1 ? w[e >> 1] & 0xFFFF0000u : w[e >> 1] << 16) + t[e];
        *reinterpret_cast<uint4*>(cp) = make_uint4(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]),
                                                   pack_bf16x2(o[4], o[5]), pack_bf16x2(o[6], o[7]));
      } else {
        for (int e = 0; e < 8; ++e) {
          if (n + e >= N) break;
          cp[e] = (uint16_t)f32_to_bf16_bits(bf16_to_f32(cp[e]) + t[e]);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }


// layout checks for one operand: 16-byte aligned rows and vectors
inline bool operand_ok(const void* p, int64_t ld, bool kmajor, int64_t mn, int64_t K) {
  if (!p || !al16(p) || (ld & 7)) return false;
  if (kmajor) return (K & 7) == 0 && ld >= K;
  return (mn & 7) == 0 && ld >= mn;
}

// 32-bit buffer offsets from where each block's reads start (Loader): a
// K-major operand spans one 256-row panel of any operand size; an MN-major
// one the block's k range, here all of K plus the prefetch overhang (split-K
// launches check their ranges with operand_fits_k).
inline bool operand_fits(int64_t ld, bool kmajor, int64_t mn, int64_t K) {
  (void)mn;
  const int64_t rows = kmajor ? 256 + 1 : K + 256;
  return rows * ld * 2 < ((int64_t)1 << 31);
}

inline bool operand_fits_k(int64_t ld, bool kmajor, int64_t k_range) {
  return operand_fits(ld, kmajor, 0, k_range);
}

template <int EPI, int CACHE, int LT>
int dispatch_gs(int64_t gs, KArgs& A, hipStream_t st) {
  // fused epilogues exist for the operand layouts of the FFN: F1 (k, k), B1 (k, mn)
  constexpr bool BKM = EPI == EPI_GLU;
  switch (gs) {
    case 32: return launch<true, BKM, EPI, CACHE, 32, LT>(A, st);
    case 64: return launch<true, BKM, EPI, CACHE, 64, LT>(A, st);
    case 128: return launch<true, BKM, EPI, CACHE, 128, LT>(A, st);
    default: return kErrGroupPow2;
  }
}

// Adapter terms of one call (see acc_block).  P_t [M, rank] with rows ldp
// apart; Q_t [n_q, rank] contiguous (q_kmajor) or [rank, n_q] with rows ldq
// apart.  rank 0: no terms.
struct LoraTerms {
  int rank = 0;
  int q_kmajor = 1;
  int64_t ldp = 0, ldq = 0;
  const void* p[2] = {nullptr, nullptr};
  const void* q[2] = {nullptr, nullptr};
  float alpha[2] = {0.0f, 0.0f};
};

// n_q: the extent of Q's n side (N, or inter for the fused FFN kernels);
// m_p: P's rows.  An absent term keeps a null P and alpha = -0.0 (a no-op,
// see acc_block).  Returns the number of terms the kernel must carry.
inline int set_lora(KArgs& A, const LoraTerms& L, int64_t m_p, int64_t n_q, int& terms) {
  terms = 0;
  A.lalpha[0] = A.lalpha[1] = -0.0f;
  if (L.rank == 0) return kOk;
  if (L.rank != 8 && L.rank != 16 && L.rank != 24 && L.rank != 32) return kErrShape;
  if (L.ldp < L.rank || (L.ldp & 7)) return kErrAlign;
  if (!L.q_kmajor && L.ldq < n_q) return kErrShape;
  if (!L.p[0] && !L.p[1]) return kErrShape;
  // 32-bit buffer offsets, with one tile of overhang past the last row
  if ((m_p + 256) * L.ldp * 2 >= ((int64_t)1 << 31)) return kErrTooLarge;
  if ((L.q_kmajor ? (n_q + 256) * L.rank : L.rank * L.ldq) * 2 >= ((int64_t)1 << 31))
    return kErrTooLarge;
  for (int t = 0; t < 2; ++t) {
    if (!L.p[t]) continue;
    if (!L.q[t]) return kErrShape;
    if (!al16(L.p[t]) || (L.q_kmajor && !al16(L.q[t]))) return kErrAlign;
    A.lp[t] = (const uint16_t*)L.p[t];
    A.lq[t] = (const uint16_t*)L.q[t];
    A.lalpha[t] = L.alpha[t];
    terms = t + 1;
  }
  A.lrank = L.rank;
  A.lq_km = L.q_kmajor;
  A.lldp = L.ldp;
  A.lldq = L.ldq;
  return kOk;
}

int gemm_bf16_impl(const void* a, int64_t lda, int a_kmajor, const void* b, int64_t ldb,
                   int b_kmajor, const void* a2, int64_t lda2, const void* b2, int64_t ldb2,
                   int64_t K2, void* c, int64_t ldc, int64_t M, int64_t N, int64_t K,
                   const LoraTerms& L, void* stream) {
  if (M < 0 || N < 0 || K < 0 || K2 < 0) return kErrShape;
  if (M == 0 || N == 0) return kOk;
  if (!c || !al16(c) || (ldc & 3) || ldc < N) return kErrAlign;
  if (K > 0 && (!operand_ok(a, lda, a_kmajor, M, K) || !operand_ok(b, ldb, b_kmajor, N, K)))
    return kErrAlign;
  if (!operand_fits(lda, a_kmajor, M, K) || !operand_fits(ldb, b_kmajor, N, K))
    return kErrTooLarge;
  const bool two = a2 != nullptr;
  if (two && (!operand_ok(a2, lda2, a_kmajor, M, K2) || !operand_ok(b2, ldb2, b_kmajor, N, K2)))
    return kErrAlign;
  // the second pair shares the first pair's per-thread offsets
  if (two && (lda2 != lda || ldb2 != ldb)) return kErrShape;
  if (two && (!operand_fits(lda, a_kmajor, M, K2) || !operand_fits(ldb, b_kmajor, N, K2)))
    return kErrTooLarge;
  KArgs A{};
  A.a[0] = {(const uint16_t*)a, lda};
  A.b[0] = {(const uint16_t*)b, ldb};
  A.K[0] = K;
  A.npairs = 1;
  if (two) {
    A.a[1] = {(const uint16_t*)a2, lda2};
    A.b[1] = {(const uint16_t*)b2, ldb2};
    A.K[1] = K2;
    A.npairs = 2;
  }
  A.M = M; A.N = N;
  A.tiles_m = (int)((M + BM - 1) / BM);
  A.tiles_n = (int)((N + BN - 1) / BN);
  A.C = (uint16_t*)c;
  A.ldc = ldc;
  int terms = 0;
  if (const int rc = set_lora(A, L, M, N, terms)) return rc;
  hipStream_t st = (hipStream_t)stream;
  // K of each pair a multiple of 64, N of 8: the 16x16x32 loop (another fp32
  // summation order than the engine's; cpt_gemm_bf16_ex mode 0 keeps the
  // engine's)
  const bool nt16 =
      nt16_fits(M, N, K, c, ldc) && (!two || (K2 > 0 && K2 % 64 == 0 && K2 <= 0x7FFFFFFF));
  if (terms) {
    // adapter terms are carried by the layouts that need them: K-major A
    if (!a_kmajor) return kErrShape;
    if (nt16 && terms == 1)
      return b_kmajor ? launch_nt16<true, true, EPI_STORE, 0, 0, 1>(A, st)
                      : launch_nt16<true, false, EPI_STORE, 0, 0, 1>(A, st);
    if (nt16)
      return b_kmajor ? launch_nt16<true, true, EPI_STORE, 0, 0, 2>(A, st)
                      : launch_nt16<true, false, EPI_STORE, 0, 0, 2>(A, st);
    // the engine carries adapter ranks up to 16
    if (L.rank > 16) return kErrShape;
    if (terms == 1)
      return b_kmajor ? launch<true, true, EPI_STORE, 0, 0, 1>(A, st)
                      : launch<true, false, EPI_STORE, 0, 0, 1>(A, st);
    return b_kmajor ? launch<true, true, EPI_STORE, 0, 0, 2>(A, st)
                    : launch<true, false, EPI_STORE, 0, 0, 2>(A, st);
  }
  if (nt16) {
    if (a_kmajor && b_kmajor) return launch_nt16<true, true, EPI_STORE, 0, 0, 0>(A, st);
    if (a_kmajor && !b_kmajor) return launch_nt16<true, false, EPI_STORE, 0, 0, 0>(A, st);
    if (!a_kmajor && !b_kmajor) return launch_nt16<false, false, EPI_STORE, 0, 0, 0>(A, st);
    return launch_nt16<false, true, EPI_STORE, 0, 0, 0>(A, st);
  }
  if (a_kmajor && b_kmajor) return launch<true, true, EPI_STORE, 0, 0>(A, st);
  if (a_kmajor && !b_kmajor) return launch<true, false, EPI_STORE, 0, 0>(A, st);
  if (!a_kmajor && !b_kmajor) return launch<false, false, EPI_STORE, 0, 0>(A, st);
  return launch<false, true, EPI_STORE, 0, 0>(A, st);
}

// F1 on the 16x16x32 loop: d_model a multiple of 64 (d_ff is one of 8 and
// the token count free, as for the engine)
inline bool ffn_nt16_fits(int64_t n_tok, int64_t inter, int64_t hidden) {
  constexpr int64_t kIntMax = 0x7FFFFFFF;
  return n_tok > 0 && inter > 0 && hidden > 0 && n_tok <= kIntMax && inter <= kIntMax &&
         hidden <= kIntMax && inter % 8 == 0 && hidden % 64 == 0 &&
         ((n_tok + 255) / 256) * ((inter + 127) / 128) <= kIntMax;
}

// B1 on the 16x16x32 loop: d_model (the k of gy . W_d) a multiple of 64;
// d_ff is one of 8 and the token count free, as for the engine
inline bool dgrad_nt16_fits(int64_t n_tok, int64_t inter, int64_t hidden) {
  constexpr int64_t kIntMax = 0x7FFFFFFF;
  return n_tok > 0 && inter > 0 && hidden > 0 && n_tok <= kIntMax && inter <= kIntMax &&
         hidden <= kIntMax && inter % 8 == 0 && hidden % 64 == 0 &&
         ((n_tok + 255) / 256) * ((inter + 255) / 256) <= kIntMax;
}

// outlier channels of the F1 and B1 epilogues (k == 0: none)
struct OutlierArgs {
  const void* slot_gate = nullptr;
  const void* o_gate = nullptr;
  const void* slot_up = nullptr;
  const void* o_up = nullptr;
  int64_t k = 0;
};

int ffn_gate_up_impl(const void* x, const void* w_gate, const void* w_up, int64_t n_tok,
                     int64_t hidden, int64_t inter, int cache, int64_t group_size, void* h_mid,
                     void* h_gate, void* h_up, void* q_gate, void* s_gate, void* q_up,
                     void* s_up, const LoraTerms& L, const OutlierArgs& O, void* stream) {
  if (n_tok < 0 || hidden < 0 || inter < 0) return kErrShape;
  if (cache != CACHE_NONE && cache != CACHE_BF16 && cache != CACHE_INT4 && cache != CACHE_INT8)
    return kErrBits;
  const bool quant = cache == CACHE_INT4 || cache == CACHE_INT8;
  if (quant) {
    if (group_size <= 0 || inter % group_size) return kErrRagged;
    if (!is_pow2(group_size)) return kErrGroupPow2;
    if (group_size != 32 && group_size != 64 && group_size != 128) return kErrGroupPow2;
    if (!q_gate || !s_gate || !q_up || !s_up) return kErrShape;
  }
  if (cache == CACHE_BF16 && (!h_gate || !h_up || !al16(h_gate) || !al16(h_up))) return kErrShape;
  if (!quant && cache != CACHE_BF16 && !h_mid) return kErrShape;
  if (n_tok == 0 || inter == 0) return kOk;
  if ((inter & 7) || !operand_ok(x, hidden, true, n_tok, hidden) ||
      !operand_ok(w_gate, hidden, true, inter, hidden) ||
      !operand_ok(w_up, hidden, true, inter, hidden) || (h_mid && !al16(h_mid)))
    return kErrAlign;
  // the epilogue stores 8 codes per access: 8 bytes (int8) or 4 bytes (int4)
  const uintptr_t qmask = cache == CACHE_INT8 ? 7u : 3u;
  if (quant && (((uintptr_t)q_gate & qmask) || ((uintptr_t)q_up & qmask))) return kErrAlign;
  if (!operand_fits(hidden, true, n_tok, hidden) || !operand_fits(hidden, true, inter, hidden))
    return kErrTooLarge;
  KArgs A{};
  A.a[0] = {(const uint16_t*)x, hidden};
  A.b[0] = {(const uint16_t*)w_gate, hidden};
  A.K[0] = hidden;
  A.npairs = 1;
  A.b_up = (const uint16_t*)w_up;
  A.M = n_tok;
  A.N = 2 * inter;
  A.D = inter;
  A.tiles_m = (int)((n_tok + BM - 1) / BM);
  A.tiles_n = (int)((inter + 127) / 128);
  A.h_mid = (uint16_t*)h_mid;
  A.h_gate = (uint16_t*)h_gate;
  A.h_up = (uint16_t*)h_up;
  A.q_gate = (uint8_t*)q_gate;
  A.s_gate = (uint16_t*)s_gate;
  A.q_up = (uint8_t*)q_up;
  A.s_up = (uint16_t*)s_up;
  int terms = 0;
  if (const int rc = set_lora(A, L, n_tok, inter, terms)) return rc;
  hipStream_t st = (hipStream_t)stream;
  if (O.k > 0) {
    // the outlier channels ride in the codec epilogue of the 16x16x32 loop
    if (!quant || !ffn_nt16_fits(n_tok, inter, hidden)) return kErrShape;
    if (!O.slot_gate || !O.slot_up || !O.o_gate || !O.o_up || !al16(O.slot_gate) ||
        !al16(O.slot_up) || O.k >= 32768 || O.k > inter)
      return kErrAlign;
    if (n_tok * O.k >= ((int64_t)1 << 31)) return kErrTooLarge;
    A.slot_g = (const int16_t*)O.slot_gate;
    A.slot_u = (const int16_t*)O.slot_up;
    A.o_g = (uint16_t*)O.o_gate;
    A.o_u = (uint16_t*)O.o_up;
    A.k_out = O.k;
#define CPT_F1O_NT16(CACHE, GS) \
  (terms ? launch_nt16<true, true, EPI_GLUO, CACHE, GS, 2>(A, st) \
         : launch_nt16<true, true, EPI_GLUO, CACHE, GS, 0>(A, st))
    if (cache == CACHE_INT4)
      return group_size == 32   ? CPT_F1O_NT16(CACHE_INT4, 32)
             : group_size == 64 ? CPT_F1O_NT16(CACHE_INT4, 64)
                                : CPT_F1O_NT16(CACHE_INT4, 128);
    return group_size == 32   ? CPT_F1O_NT16(CACHE_INT8, 32)
           : group_size == 64 ? CPT_F1O_NT16(CACHE_INT8, 64)
                              : CPT_F1O_NT16(CACHE_INT8, 128);
#undef CPT_F1O_NT16
  }
  // d_model a multiple of 64: the 16x16x32 loop (its summation order is that
  // of cpt_gemm_bf16's products with K a multiple of 64, not of
  // cpt_gemm_bf16_ex mode 0); the dual kernel carries both adapter terms
  if (ffn_nt16_fits(n_tok, inter, hidden)) {
#define CPT_F1_NT16(CACHE, GS) \
  (terms ? launch_nt16<true, true, EPI_GLU, CACHE, GS, 2>(A, st) \
         : launch_nt16<true, true, EPI_GLU, CACHE, GS, 0>(A, st))
    switch (cache) {
      case CACHE_NONE: return CPT_F1_NT16(CACHE_NONE, 64);
      case CACHE_BF16: return CPT_F1_NT16(CACHE_BF16, 64);
      case CACHE_INT4:
        return group_size == 32   ? CPT_F1_NT16(CACHE_INT4, 32)
               : group_size == 64 ? CPT_F1_NT16(CACHE_INT4, 64)
                                  : CPT_F1_NT16(CACHE_INT4, 128);
      default:
        return group_size == 32   ? CPT_F1_NT16(CACHE_INT8, 32)
               : group_size == 64 ? CPT_F1_NT16(CACHE_INT8, 64)
                                  : CPT_F1_NT16(CACHE_INT8, 128);
    }
#undef CPT_F1_NT16
  }
  // the engine carries adapter ranks up to 16
  if (L.rank > 16) return kErrShape;
  // the dual kernel carries both terms (gate, up); an absent one is a no-op
  switch (cache) {
    case CACHE_NONE:
      return terms ? launch<true, true, EPI_GLU, CACHE_NONE, 64, 2>(A, st)
                   : launch<true, true, EPI_GLU, CACHE_NONE, 64>(A, st);
    case CACHE_BF16:
      return terms ? launch<true, true, EPI_GLU, CACHE_BF16, 64, 2>(A, st)
                   : launch<true, true, EPI_GLU, CACHE_BF16, 64>(A, st);
    case CACHE_INT4:
      return terms ? dispatch_gs<EPI_GLU, CACHE_INT4, 2>(group_size, A, st)
                   : dispatch_gs<EPI_GLU, CACHE_INT4, 0>(group_size, A, st);
    default:
      return terms ? dispatch_gs<EPI_GLU, CACHE_INT8, 2>(group_size, A, st)
                   : dispatch_gs<EPI_GLU, CACHE_INT8, 0>(group_size, A, st);
  }
}

int ffn_down_dgrad_impl(const void* grad_y, const void* w_down, int64_t n_tok, int64_t hidden,
                        int64_t inter, int cache, int64_t group_size, const void* c_gate,
                        const void* s_gate, const void* c_up, const void* s_up,
                        void* grad_h_gate, void* grad_h_up, void* h_mid_hat,
                        const OutlierArgs& O,
                        const LoraTerms& L, void* stream) {
  if (n_tok < 0 || hidden < 0 || inter < 0) return kErrShape;
  if (cache != CACHE_BF16 && cache != CACHE_INT4 && cache != CACHE_INT8) return kErrBits;
  const bool quant = cache != CACHE_BF16;
  if (quant) {
    if (group_size <= 0 || inter % group_size) return kErrRagged;
    if (!is_pow2(group_size)) return kErrGroupPow2;
    if (group_size != 32 && group_size != 64 && group_size != 128) return kErrGroupPow2;
    if (!s_gate || !s_up) return kErrShape;
  }
  if (!c_gate || !c_up || !grad_h_gate || !grad_h_up) return kErrShape;
  if (n_tok == 0 || inter == 0) return kOk;
  if ((inter & 7) || !operand_ok(grad_y, hidden, true, n_tok, hidden) ||
      !operand_ok(w_down, inter, false, inter, hidden) || !al16(grad_h_gate) ||
      !al16(grad_h_up) || (h_mid_hat && !al16(h_mid_hat)))
    return kErrAlign;
  // the epilogue reads 8 columns per access: 16 B of bf16 cache, 8 B of int8
  // codes or 4 B of int4 codes
  const uintptr_t cmask = cache == CACHE_BF16 ? 15u : (cache == CACHE_INT8 ? 7u : 3u);
  if (((uintptr_t)c_gate & cmask) || ((uintptr_t)c_up & cmask)) return kErrAlign;
  if (!operand_fits(hidden, true, n_tok, hidden) || !operand_fits(inter, false, inter, hidden))
    return kErrTooLarge;
  KArgs A{};
  A.a[0] = {(const uint16_t*)grad_y, hidden};
  A.b[0] = {(const uint16_t*)w_down, inter};   // W_d [H, D]: n-side d, k = h, MN-major
  A.K[0] = hidden;
  A.npairs = 1;
  A.M = n_tok;
  A.N = inter;
  A.D = inter;
  A.tiles_m = (int)((n_tok + BM - 1) / BM);
  A.tiles_n = (int)((inter + BN - 1) / BN);
  if (quant) {
    A.q_gate = (uint8_t*)c_gate;
    A.q_up = (uint8_t*)c_up;
    A.s_gate = (uint16_t*)s_gate;
    A.s_up = (uint16_t*)s_up;
  } else {
    A.h_gate = (uint16_t*)c_gate;
    A.h_up = (uint16_t*)c_up;
  }
  A.grad_gate = (uint16_t*)grad_h_gate;
  A.grad_up = (uint16_t*)grad_h_up;
  A.h_mid_hat = (uint16_t*)h_mid_hat;
  if (O.k > 0) {
    if (!quant) return kErrShape;
    if (!O.slot_gate || !O.slot_up || !O.o_gate || !O.o_up || !al16(O.slot_gate) ||
        !al16(O.slot_up) || O.k >= 32768)
      return kErrAlign;
    if (n_tok * O.k >= ((int64_t)1 << 31)) return kErrTooLarge;
    A.slot_g = (const int16_t*)O.slot_gate;
    A.slot_u = (const int16_t*)O.slot_up;
    A.o_g = (uint16_t*)O.o_gate;
    A.o_u = (uint16_t*)O.o_up;
    A.k_out = O.k;
  }
  int terms = 0;
  if (const int rc = set_lora(A, L, n_tok, inter, terms)) return rc;
  if (terms > 1) return kErrShape;
  hipStream_t st = (hipStream_t)stream;
  if (dgrad_nt16_fits(n_tok, inter, hidden)) {
    // the 16x16x32 loop: d_model a multiple of 64 (its summation order is
    // that of cpt_gemm_bf16's product gy . W_d on the same loop)
#define CPT_B1_NT16(CACHE, GS) \
  (terms ? launch_nt16<true, false, EPI_DGLU, CACHE, GS, 1>(A, st) \
         : launch_nt16<true, false, EPI_DGLU, CACHE, GS, 0>(A, st))
    switch (cache) {
      case CACHE_BF16: return CPT_B1_NT16(CACHE_BF16, 64);
      case CACHE_INT4:
        return group_size == 32   ? CPT_B1_NT16(CACHE_INT4, 32)
               : group_size == 64 ? CPT_B1_NT16(CACHE_INT4, 64)
                                  : CPT_B1_NT16(CACHE_INT4, 128);
      default:
        return group_size == 32   ? CPT_B1_NT16(CACHE_INT8, 32)
               : group_size == 64 ? CPT_B1_NT16(CACHE_INT8, 64)
                                  : CPT_B1_NT16(CACHE_INT8, 128);
    }
#undef CPT_B1_NT16
  }
  if (L.rank > 16) return kErrShape;   // the engine carries adapter ranks up to 16
  switch (cache) {
    case CACHE_BF16:
      return terms ? launch<true, false, EPI_DGLU, CACHE_BF16, 64, 1>(A, st)
                   : launch<true, false, EPI_DGLU, CACHE_BF16, 64>(A, st);
    case CACHE_INT4:
      return terms ? dispatch_gs<EPI_DGLU, CACHE_INT4, 1>(group_size, A, st)
                   : dispatch_gs<EPI_DGLU, CACHE_INT4, 0>(group_size, A, st);
    default:
      return terms ? dispatch_gs<EPI_DGLU, CACHE_INT8, 1>(group_size, A, st)
                   : dispatch_gs<EPI_DGLU, CACHE_INT8, 0>(group_size, A, st);
  }
}

// C[hidden, inter] = grad_y^T . h^ with h^ = bf16(SiLU(hg^) * hu^) formed from
// the int cache in the B operand's staging (the weight gradient of the down
// projection without K2's h_mid^ in HBM).
int wgrad_glu_impl(const void* grad_y, int64_t ldg, int cache, int64_t gs, const void* q_gate,
                   const void* s_gate, const void* q_up, const void* s_up, void* c, int64_t ldc,
                   int64_t hidden, int64_t inter, int64_t n_tok, void* stream) {
  if (hidden < 0 || inter < 0 || n_tok < 0) return kErrShape;
  if (cache != CACHE_INT4 && cache != CACHE_INT8) return kErrBits;
  if (gs <= 0 || inter % gs) return kErrRagged;
  if (!is_pow2(gs)) return kErrGroupPow2;
  if (gs != 32 && gs != 64 && gs != 128) return kErrGroupPow2;
  if (hidden == 0 || inter == 0) return kOk;
  if (!q_gate || !s_gate || !q_up || !s_up || !c) return kErrShape;
  const uintptr_t qmask = cache == CACHE_INT8 ? 7u : 3u;
  if ((inter & 7) || ((uintptr_t)q_gate & qmask) || ((uintptr_t)q_up & qmask) ||
      ((uintptr_t)s_gate & 1u) || ((uintptr_t)s_up & 1u) || !al16(c) || (ldc & 3) ||
      ldc < inter || (n_tok > 0 && !operand_ok(grad_y, ldg, false, hidden, n_tok)))
    return kErrAlign;
  // 32-bit offsets: grad_y's k rows and the cache's rows (plus a tile of prefetch)
  const int64_t qrow = cache == CACHE_INT8 ? inter : inter / 2;
  if (!operand_fits(ldg, false, hidden, n_tok) || (n_tok + 256) * qrow >= ((int64_t)1 << 31) ||
      (n_tok + 256) * (inter / gs) * 2 >= ((int64_t)1 << 31))
    return kErrTooLarge;
  KArgs A{};
  A.a[0] = {(const uint16_t*)grad_y, ldg};
  A.b[0] = {nullptr, inter};
  A.K[0] = n_tok;
  A.npairs = 1;
  A.M = hidden;
  A.N = inter;
  A.D = inter;
  A.lgs = gs;
  A.tiles_m = (int)((hidden + BM - 1) / BM);
  A.tiles_n = (int)((inter + BN - 1) / BN);
  A.C = (uint16_t*)c;
  A.ldc = ldc;
  A.q_gate = (uint8_t*)q_gate;
  A.q_up = (uint8_t*)q_up;
  A.s_gate = (uint16_t*)s_gate;
  A.s_up = (uint16_t*)s_up;
  hipStream_t st = (hipStream_t)stream;
  if (cache == CACHE_INT8) {
    switch (gs) {
      case 32: return launch<false, false, EPI_STORE, CACHE_INT8, 32>(A, st);
      case 64: return launch<false, false, EPI_STORE, CACHE_INT8, 64>(A, st);
      default: return launch<false, false, EPI_STORE, CACHE_INT8, 128>(A, st);
    }
  }
  switch (gs) {
    case 32: return launch<false, false, EPI_STORE, CACHE_INT4, 32>(A, st);
    case 64: return launch<false, false, EPI_STORE, CACHE_INT4, 64>(A, st);
    default: return launch<false, false, EPI_STORE, CACHE_INT4, 128>(A, st);
  }
}

}  // namespace gemm
}  // namespace cpt

using namespace cpt;
using namespace cpt::gemm;

extern "C" {

int cpt_gemm_bf16(const void* a, int64_t lda, int a_kmajor, const void* b, int64_t ldb,
                  int b_kmajor, const void* a2, int64_t lda2, const void* b2, int64_t ldb2,
                  int64_t K2, void* c, int64_t ldc, int64_t M, int64_t N, int64_t K,
                  void* stream) {
  return gemm_bf16_impl(a, lda, a_kmajor, b, ldb, b_kmajor, a2, lda2, b2, ldb2, K2, c, ldc, M, N,
                        K, LoraTerms{}, stream);
}

int cpt_gemm_bf16_lora(const void* a, int64_t lda, int a_kmajor, const void* b, int64_t ldb,
                       int b_kmajor, const void* a2, int64_t lda2, const void* b2, int64_t ldb2,
                       int64_t K2, void* c, int64_t ldc, int64_t M, int64_t N, int64_t K,
                       int64_t rank, int64_t ldp, int q_kmajor, int64_t ldq, const void* p0,
                       const void* q0, float alpha0, const void* p1, const void* q1,
                       float alpha1, void* stream) {
  if (rank <= 0) return kErrShape;
  LoraTerms L;
  L.rank = (int)rank; L.ldp = ldp; L.q_kmajor = q_kmajor ? 1 : 0; L.ldq = ldq;
  L.p[0] = p0; L.q[0] = q0; L.alpha[0] = alpha0;
  L.p[1] = p1; L.q[1] = q1; L.alpha[1] = alpha1;
  return gemm_bf16_impl(a, lda, a_kmajor, b, ldb, b_kmajor, a2, lda2, b2, ldb2, K2, c, ldc, M, N,
                        K, L, stream);
}


int cpt_gemm_bf16_ex(const void* a, int64_t lda, int a_kmajor, const void* b, int64_t ldb,
                     int b_kmajor, void* c, int64_t ldc, int64_t M, int64_t N, int64_t K,
                     float alpha, int mode, int splits, void* workspace, void* stream) {
  if (M < 0 || N < 0 || K < 0) return kErrShape;
  if (mode < 0 || mode > 2) return kErrShape;
  if (M == 0 || N == 0) return kOk;
  if (!c || (mode != 1 && (!al16(c) || (ldc & 3))) || ldc < N) return kErrAlign;
  if (K > 0 && (!operand_ok(a, lda, a_kmajor, M, K) || !operand_ok(b, ldb, b_kmajor, N, K)))
    return kErrAlign;
  // split-K blocks read one k range each: mode 2 checks the range below
  if (mode != 2 && (!operand_fits(lda, a_kmajor, M, K) || !operand_fits(ldb, b_kmajor, N, K)))
    return kErrTooLarge;
  KArgs A{};
  A.a[0] = {(const uint16_t*)a, lda};
  A.b[0] = {(const uint16_t*)b, ldb};
  A.K[0] = K;
  A.npairs = 1;
  A.M = M; A.N = N;
  A.tiles_m = (int)((M + BM - 1) / BM);
  A.tiles_n = (int)((N + BN - 1) / BN);
  A.C = (uint16_t*)c;
  A.ldc = ldc;
  A.alpha = alpha;
  hipStream_t st = (hipStream_t)stream;
  if (mode == 0) {
    if (a_kmajor && b_kmajor) return launch<true, true, EPI_STORE, 0, 0>(A, st);
    if (a_kmajor && !b_kmajor) return launch<true, false, EPI_STORE, 0, 0>(A, st);
    if (!a_kmajor && !b_kmajor) return launch<false, false, EPI_STORE, 0, 0>(A, st);
    return launch<false, true, EPI_STORE, 0, 0>(A, st);
  }
  if (mode == 1 && K > 0 && K <= kThinK) {
    const int64_t sam = a_kmajor ? lda : 1, sak = a_kmajor ? 1 : lda;
    const int64_t sbk = b_kmajor ? 1 : ldb, sbn = b_kmajor ? ldb : 1;
    const bool avec = a_kmajor && K == kThinK && (lda & 7) == 0 && al16(a);
    // 1: K-major B, K == 16, rows 16-byte aligned; 2: MN-major B whose 8-column
    // runs are 16-byte aligned and complete (N % 8 == 0)
    const int bvec = (b_kmajor && K == kThinK && (ldb & 7) == 0 && al16(b)) ? 1
                     : (!b_kmajor && (ldb & 7) == 0 && (N & 7) == 0 && al16(b)) ? 2 : 0;
    const bool cvec = (ldc & 7) == 0 && al16(c);
    const dim3 grid((unsigned)((N + 255) / 256), (unsigned)((M + kThinRows - 1) / kThinRows));
    if (grid.y > 65535) return kErrTooLarge;
#define CPT_THIN(AV, BV)                                                                         \
  hipLaunchKernelGGL((thin_add_kernel<AV, BV>), grid, dim3(256), 0, st, (const uint16_t*)a, sam, \
                     sak, (const uint16_t*)b, sbk, sbn, (uint16_t*)c, ldc, M, N, (int)K, alpha,  \
                     cvec)
    if (avec) {
      if (bvec == 1) CPT_THIN(true, 1); else if (bvec == 2) CPT_THIN(true, 2); else CPT_THIN(true, 0);
    } else {
      if (bvec == 1) CPT_THIN(false, 1); else if (bvec == 2) CPT_THIN(false, 2); else CPT_THIN(false, 0);
    }
#undef CPT_THIN
    return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
  }
  if (mode == 1) {
    if (a_kmajor && b_kmajor) return launch<true, true, EPI_ADD, 0, 0>(A, st);
    if (a_kmajor && !b_kmajor) return launch<true, false, EPI_ADD, 0, 0>(A, st);
    if (!a_kmajor && !b_kmajor) return launch<false, false, EPI_ADD, 0, 0>(A, st);
    return launch<false, true, EPI_ADD, 0, 0>(A, st);
  }
  // split-K: fp32 partials in the caller's workspace, then a fixed-order reduce
  const int nk = (int)((K + BK - 1) / BK);
  if (splits < 1) return kErrShape;
  if (splits > nk) splits = nk > 0 ? nk : 1;
  if (!workspace || ((uintptr_t)workspace & 15)) return kErrAlign;
  A.ws = (float*)workspace;
  A.ksplit = splits;
  A.kt_per_split = (nk + splits - 1) / splits;
  const int64_t k_range = (int64_t)A.kt_per_split * BK;
  if (!operand_fits_k(lda, a_kmajor, k_range) || !operand_fits_k(ldb, b_kmajor, k_range))
    return kErrTooLarge;
  int rc;
  if (a_kmajor && b_kmajor) rc = launch<true, true, EPI_F32, 0, 0>(A, st);
  else if (a_kmajor && !b_kmajor) rc = launch<true, false, EPI_F32, 0, 0>(A, st);
  else if (!a_kmajor && !b_kmajor) rc = launch<false, false, EPI_F32, 0, 0>(A, st);
  else rc = launch<false, true, EPI_F32, 0, 0>(A, st);
  if (rc) return rc;
  const int64_t total = M * N;
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     st, (const float*)workspace, (uint16_t*)c, M, N, ldc, splits, alpha);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}



int cpt_ffn_gate_up(const void* x, const void* w_gate, const void* w_up, int64_t n_tok,
                    int64_t hidden, int64_t inter, int cache, int64_t group_size, void* h_mid,
                    void* h_gate, void* h_up, void* q_gate, void* s_gate, void* q_up,
                    void* s_up, void* stream) {
  return ffn_gate_up_impl(x, w_gate, w_up, n_tok, hidden, inter, cache, group_size, h_mid, h_gate,
                          h_up, q_gate, s_gate, q_up, s_up, LoraTerms{}, OutlierArgs{}, stream);
}

int cpt_ffn_gate_up_lora(const void* x, const void* w_gate, const void* w_up, int64_t n_tok,
                         int64_t hidden, int64_t inter, int cache, int64_t group_size,
                         void* h_mid, void* h_gate, void* h_up, void* q_gate, void* s_gate,
                         void* q_up, void* s_up, int64_t rank, int64_t ldp, const void* p_gate,
                         const void* b_gate, float alpha_gate, const void* p_up,
                         const void* b_up, float alpha_up, void* stream) {
  if (rank <= 0) return kErrShape;
  LoraTerms L;
  L.rank = (int)rank; L.ldp = ldp; L.q_kmajor = 1;
  L.p[0] = p_gate; L.q[0] = b_gate; L.alpha[0] = alpha_gate;
  L.p[1] = p_up; L.q[1] = b_up; L.alpha[1] = alpha_up;
  return ffn_gate_up_impl(x, w_gate, w_up, n_tok, hidden, inter, cache, group_size, h_mid, h_gate,
                          h_up, q_gate, s_gate, q_up, s_up, L, OutlierArgs{}, stream);
}

int cpt_ffn_gate_up_outlier(const void* x, const void* w_gate, const void* w_up, int64_t n_tok,
                            int64_t hidden, int64_t inter, int cache, int64_t group_size,
                            void* h_mid, void* q_gate, void* s_gate, void* q_up, void* s_up,
                            const void* slot_gate, void* o_gate, const void* slot_up, void* o_up,
                            int64_t k, int64_t rank, int64_t ldp, const void* p_gate,
                            const void* b_gate, float alpha_gate, const void* p_up,
                            const void* b_up, float alpha_up, void* stream) {
  if (k <= 0 || rank < 0) return kErrShape;
  LoraTerms L;
  if (rank > 0) {
    L.rank = (int)rank; L.ldp = ldp; L.q_kmajor = 1;
    L.p[0] = p_gate; L.q[0] = b_gate; L.alpha[0] = alpha_gate;
    L.p[1] = p_up; L.q[1] = b_up; L.alpha[1] = alpha_up;
  }
  OutlierArgs O;
  O.slot_gate = slot_gate; O.o_gate = o_gate; O.slot_up = slot_up; O.o_up = o_up; O.k = k;
  return ffn_gate_up_impl(x, w_gate, w_up, n_tok, hidden, inter, cache, group_size, h_mid,
                          nullptr, nullptr, q_gate, s_gate, q_up, s_up, L, O, stream);
}

int cpt_ffn_down_dgrad(const void* grad_y, const void* w_down, int64_t n_tok, int64_t hidden,
                       int64_t inter, int cache, int64_t group_size, const void* c_gate,
                       const void* s_gate, const void* c_up, const void* s_up, void* grad_h_gate,
                       void* grad_h_up, void* h_mid_hat, void* stream) {
  return ffn_down_dgrad_impl(grad_y, w_down, n_tok, hidden, inter, cache, group_size, c_gate,
                             s_gate, c_up, s_up, grad_h_gate, grad_h_up, h_mid_hat, OutlierArgs{},
                             LoraTerms{}, stream);
}

int cpt_ffn_down_dgrad_lora(const void* grad_y, const void* w_down, int64_t n_tok,
                            int64_t hidden, int64_t inter, int cache, int64_t group_size,
                            const void* c_gate, const void* s_gate, const void* c_up,
                            const void* s_up, void* grad_h_gate, void* grad_h_up,
                            void* h_mid_hat, int64_t rank, int64_t ldp, const void* p,
                            const void* a_down, float alpha, void* stream) {
  if (rank <= 0) return kErrShape;
  LoraTerms L;
  L.rank = (int)rank; L.ldp = ldp; L.q_kmajor = 0; L.ldq = inter;
  L.p[0] = p; L.q[0] = a_down; L.alpha[0] = alpha;
  return ffn_down_dgrad_impl(grad_y, w_down, n_tok, hidden, inter, cache, group_size, c_gate,
                             s_gate, c_up, s_up, grad_h_gate, grad_h_up, h_mid_hat, OutlierArgs{},
                             L, stream);
}

int cpt_ffn_down_dgrad_outlier(const void* grad_y, const void* w_down, int64_t n_tok,
                               int64_t hidden, int64_t inter, int cache, int64_t group_size,
                               const void* c_gate, const void* s_gate, const void* slot_gate,
                               const void* o_gate, const void* c_up, const void* s_up,
                               const void* slot_up, const void* o_up, int64_t k,
                               void* grad_h_gate, void* grad_h_up, void* h_mid_hat,
                               int64_t rank, int64_t ldp, const void* p, const void* a_down,
                               float alpha, void* stream) {
  if (k < 0 || rank < 0) return kErrShape;
  OutlierArgs O;
  O.slot_gate = slot_gate; O.o_gate = o_gate; O.slot_up = slot_up; O.o_up = o_up; O.k = k;
  LoraTerms L;
  if (rank > 0) {
    L.rank = (int)rank; L.ldp = ldp; L.q_kmajor = 0; L.ldq = inter;
    L.p[0] = p; L.q[0] = a_down; L.alpha[0] = alpha;
  }
  return ffn_down_dgrad_impl(grad_y, w_down, n_tok, hidden, inter, cache, group_size, c_gate,
                             s_gate, c_up, s_up, grad_h_gate, grad_h_up, h_mid_hat, O, L, stream);
}

int cpt_gemm_wgrad_glu(const void* grad_y, int64_t ldg, int cache, int64_t group_size,
                       const void* q_gate, const void* s_gate, const void* q_up,
                       const void* s_up, void* c, int64_t ldc, int64_t hidden, int64_t inter,
                       int64_t n_tok, void* stream) {
  return wgrad_glu_impl(grad_y, ldg, cache, group_size, q_gate, s_gate, q_up, s_up, c, ldc,
                        hidden, inter, n_tok, stream);
}

}  // extern "C"
