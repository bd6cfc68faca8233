// General-layout GEMM for every product the bf16 MFMA engine (gemm_kernel.h)
// does not take: float32 and float16 operands (config C1 runs in float32),
// bf16 views whose rows are not 16-byte aligned, and ranks or extents that
// are not multiples of 8 (rank-1 adapter factors, ragged widths).
//
//   C[M, N]  =  epi( A[M, K] . B[K, N] )      fp32 accumulation
//   A(m, k) = a[m * sam + k * sak]   B(k, n) = b[k * sbk + n * sbn]
//   C(m, n) = c[m * scm + n * scn]
//
// Elements of any storage dtype are widened to fp32 on their way into LDS and
// multiplied on v_mfma_f32_32x32x2_f32, so bf16 and fp16 products are exact
// and every accumulation is fp32, as in the library GEMMs the reference
// calls (src/flashffn.py:1410-1439,1503-1587 through F.linear / @).  The
// epilogues restate the reference's eager op order with each step rounded to
// the output dtype (rd):
//   STORE  c = rd(acc)                          x @ w
//   ADD    c = rd(c + rd(alpha * rd(acc)))      h + s * F.linear(xa, b)
//   SCALE  c = rd(alpha * rd(acc))              s * (a @ b)
//
// Block tile 128 x 128 x 16, 256 threads = 4 wavefronts in 2 x 2, each owning
// 64 x 64 outputs as 2 x 2 tiles of 32 x 32.  Each operand tile is read with
// the thread mapping that makes its unit-stride dimension the fast one, so the
// global reads are coalesced for row-major and transposed views alike; a
// general strided view still works, element by element.  Tiles are staged
// k-major in LDS (row = k, 128 m or n per row, padded to 132 floats), so a
// fragment read (32 consecutive m or n at one k) is conflict-free.  Two LDS
// stages; the next tile's global loads are in flight while the current one
// is multiplied.

#include "common.h"
#include "compact_amd.h"

namespace cpt {
namespace gemm_any {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BK = 16, NTHR = 256;
constexpr int LDT = 132;                 // LDS row (one k) of a 128-wide tile, padded
constexpr int STAGE = 2 * BK * LDT;      // A tile + B tile, floats

enum Epi { EPI_STORE = 0, EPI_ADD = 1, EPI_SCALE = 2 };

struct Args {
  const void* a;
  const void* b;
  void* c;
  int64_t sam, sak, sbk, sbn, scm, scn;
  int64_t M, N, K;
  float alpha;
  int a_kfast;   // A's unit-stride dimension is k (else m)
  int b_kfast;   // B's unit-stride dimension is k (else n)
};

// One operand tile (rows = the 128-wide m or n side, k = 16) into registers.
// kfast: 16 consecutive threads take 16 consecutive k of one row (k is the
// unit stride); else 128 consecutive threads take 128 consecutive rows at one k.
template <int DT>
__device__ __forceinline__ void load_tile(const void* base, int64_t s_row, int64_t s_k,
                                          int64_t row0, int64_t rows, int64_t k0, int64_t K,
                                          bool kfast, int tid, float (&v)[8]) {
  using E = Elem<DT>;
  const typename E::T* p = reinterpret_cast<const typename E::T*>(base);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = kfast ? (tid >> 4) + 16 * i : (tid & 127);
    const int k = kfast ? (tid & 15) : (tid >> 7) + 2 * i;
    const int64_t gr = row0 + r, gk = k0 + k;
    v[i] = (gr < rows && gk < K) ? E::ld(p + gr * s_row + gk * s_k) : 0.0f;
  }
}

__device__ __forceinline__ void store_tile(float* t, bool kfast, int tid, const float (&v)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = kfast ? (tid >> 4) + 16 * i : (tid & 127);
    const int k = kfast ? (tid & 15) : (tid >> 7) + 2 * i;
    t[k * LDT + r] = v[i];
  }
}

template <int DT>
__device__ __forceinline__ float rd(float v) {
  if constexpr (DT == kBF16) return bf16_to_f32(f32_to_bf16_bits(v));
  if constexpr (DT == kF16) return f16_bits_to_f32(f32_to_f16_bits(v));
  return v;
}

template <int DT, int EPI>
__global__ __launch_bounds__(NTHR) void gemm_any_kernel(Args A) {
  __shared__ float lds[2 * STAGE];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  const bool akf = A.a_kfast != 0, bkf = A.b_kfast != 0;

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int nk = (int)((A.K + BK - 1) / BK);
  float va[8], vb[8];
  if (nk > 0) {
    load_tile<DT>(A.a, A.sam, A.sak, m0, A.M, 0, A.K, akf, tid, va);
    load_tile<DT>(A.b, A.sbn, A.sbk, n0, A.N, 0, A.K, bkf, tid, vb);
    store_tile(lds, akf, tid, va);
    store_tile(lds + BK * LDT, bkf, tid, vb);
  }
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const float* sa = lds + (kt & 1) * STAGE;
    const float* sb = sa + BK * LDT;
    const bool more = kt + 1 < nk;
    if (more) {
      const int64_t k0 = (int64_t)(kt + 1) * BK;
      load_tile<DT>(A.a, A.sam, A.sak, m0, A.M, k0, A.K, akf, tid, va);
      load_tile<DT>(A.b, A.sbn, A.sbk, n0, A.N, k0, A.K, bkf, tid, vb);
    }
#pragma unroll
    for (int kk = 0; kk < BK; kk += 2) {
      // lane supplies element (row lane % 32, k lane / 32) of each fragment
      const int k = kk + (lane >> 5);
      float fa[2], fb[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) fa[i] = sa[k * LDT + wm * 64 + i * 32 + (lane & 31)];
#pragma unroll
      for (int j = 0; j < 2; ++j) fb[j] = sb[k * LDT + wn * 64 + j * 32 + (lane & 31)];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    if (more) {
      float* da = lds + ((kt + 1) & 1) * STAGE;
      store_tile(da, akf, tid, va);
      store_tile(da + BK * LDT, bkf, tid, vb);
    }
    __syncthreads();
  }

  // acc[i][j][r]: m = m0 + 64 wm + 32 i + 8 (r / 4) + 4 (lane / 32) + r % 4,
  //               n = n0 + 64 wn + 32 j + lane % 32
  using E = Elem<DT>;
  typename E::T* c = reinterpret_cast<typename E::T*>(A.c);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t n = n0 + wn * 64 + j * 32 + (lane & 31);
      if (n >= A.N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m >= A.M) continue;
        typename E::T* cp = c + m * A.scm + n * A.scn;
        const float p = rd<DT>(acc[i][j][r]);
        if constexpr (EPI == EPI_STORE) {
          E::st(cp, p);
        } else if constexpr (EPI == EPI_SCALE) {
          E::st(cp, A.alpha * p);
        } else {
          E::st(cp, E::ld(cp) + rd<DT>(A.alpha * p));
        }
      }
    }
}

template <int DT, int EPI>
int launch(const Args& A, hipStream_t st) {
  const int64_t gx = (A.N + BN - 1) / BN, gy = (A.M + BM - 1) / BM;
  if (gx > 0x7FFFFFFF || gy > 65535) return kErrTooLarge;
  hipLaunchKernelGGL((gemm_any_kernel<DT, EPI>), dim3((unsigned)gx, (unsigned)gy), dim3(NTHR), 0,
                     st, A);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

template <int DT>
int dispatch_epi(int mode, const Args& A, hipStream_t st) {
  switch (mode) {
    case EPI_STORE: return launch<DT, EPI_STORE>(A, st);
    case EPI_ADD: return launch<DT, EPI_ADD>(A, st);
    default: return launch<DT, EPI_SCALE>(A, st);
  }
}

}  // namespace gemm_any
}  // namespace cpt

using namespace cpt;

extern "C" int cpt_gemm_any(int dtype, const void* a, int64_t sam, int64_t sak, const void* b,
                            int64_t sbk, int64_t sbn, void* c, int64_t scm, int64_t scn,
                            int64_t M, int64_t N, int64_t K, float alpha, int mode,
                            void* stream) {
  using namespace cpt::gemm_any;
  if (M < 0 || N < 0 || K < 0) return kErrShape;
  if (mode < EPI_STORE || mode > EPI_SCALE) return kErrShape;
  if (dtype != kF32 && dtype != kF16 && dtype != kBF16) return kErrDType;
  if (M == 0 || N == 0) return kOk;
  if (!c || (K > 0 && (!a || !b))) return kErrShape;
  const int64_t esz = dtype == kF32 ? 4 : 2;
  const uintptr_t emask = (uintptr_t)esz - 1;
  if (((uintptr_t)a & emask) || ((uintptr_t)b & emask) || ((uintptr_t)c & emask))
    return kErrAlign;
  Args A{};
  A.a = a; A.b = b; A.c = c;
  A.sam = sam; A.sak = sak; A.sbk = sbk; A.sbn = sbn; A.scm = scm; A.scn = scn;
  A.M = M; A.N = N; A.K = K;
  A.alpha = alpha;
  // read along the unit-stride dimension (k when both are, or neither is, unit)
  A.a_kfast = (sak == 1 || sam != 1) ? 1 : 0;
  A.b_kfast = (sbk == 1 || sbn != 1) ? 1 : 0;
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case kF32: return dispatch_epi<kF32>(mode, A, st);
    case kF16: return dispatch_epi<kF16>(mode, A, st);
    default: return dispatch_epi<kBF16>(mode, A, st);
  }
}
