// Memory-bound kernels of the adapter path (DoRA / VeRA / AdaLoRA / DyLoRA on
// the FlashFFN v3 cache), reference src/flashffn.py:1697-2230.  VeRA, AdaLoRA
// and DyLoRA enter the Function as composed or sliced thin factors, so only
// DoRA's magnitude needs kernels of its own:
//
//   dora_scale     out[i, j] = rd(x[i, j] * rd(m[j] / nu[j]))   the post-bypass
//                  column scale c = m / nu (:1967-1975) and its chain rule
//                  g * c (:2054, :2128-2130).  out may alias x.
//   col_dot_div    out[j] = rd((sum_i rd(a[i, j] * b[i, j])) / den[j]), the sum
//                  in fp32 over fixed row chunks, then the chunks in order:
//                  the magnitude gradients (:2086-2089, :2112-2125).
//   dora_col_norm  nu[j] = ||W_j + s (B A)_j||_2 through the Gram identity
//                  nu^2 = ||W_j||^2 + 2s sum_k B_jk (W A^T)_jk
//                         + s^2 sum_l (B G)_jl B_jl,   G = A A^T,
//                  all in fp32, never forming B A (:1824-1840).
// rd() rounds to the tensors' storage dtype (round to nearest even), which is
// how the reference's eager bf16 ops round each result.

#include "common.h"
#include "compact_amd.h"

namespace cpt {
namespace adapters {

constexpr int kBlock = 256;
constexpr int kDotThreads = 64;    // col_dot: one wavefront per column strip
constexpr int kDotRows = 128;      // rows per col_dot partial
constexpr int kRowsPerWave = 4;    // dora_rows: rows of W one wavefront owns
constexpr int kRankTile = 8;       // dora_rows: columns of W A^T per block

template <int DT> using St = typename Elem<DT>::T;

template <int DT>
__device__ __forceinline__ float rd(float v) {
  St<DT> t;
  Elem<DT>::st(&t, v);
  return Elem<DT>::ld(&t);
}

// ---------------------------------------------------------------------------
// dora_scale
// ---------------------------------------------------------------------------

template <int DT>
__global__ __launch_bounds__(kBlock) void dora_scale_vec_kernel(const void* x, const St<DT>* m,
                                                                const St<DT>* nu, void* out,
                                                                int64_t n8, int64_t d) {
  const int64_t e8 = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (e8 >= n8) return;
  const int64_t j0 = (e8 * 8) % d;   // d % 8 == 0: the 8 elements share a row
  float v[8];
  Vec8<DT>::ld(x, e8, v);
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const float c = rd<DT>(Elem<DT>::ld(m + j0 + t) / Elem<DT>::ld(nu + j0 + t));
    v[t] = v[t] * c;
  }
  Vec8<DT>::st(out, e8, v);
}

template <int DT>
__global__ __launch_bounds__(kBlock) void dora_scale_kernel(const St<DT>* x, const St<DT>* m,
                                                            const St<DT>* nu, St<DT>* out,
                                                            int64_t total, int64_t d) {
  const int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (e >= total) return;
  const int64_t j = e % d;
  const float c = rd<DT>(Elem<DT>::ld(m + j) / Elem<DT>::ld(nu + j));
  Elem<DT>::st(out + e, Elem<DT>::ld(x + e) * c);
}

// ---------------------------------------------------------------------------
// col_dot_div
// ---------------------------------------------------------------------------

// VEC consecutive columns per lane; grid (column strips, row chunks)
template <int DT, int VEC>
__global__ __launch_bounds__(kDotThreads) void col_dot_partial_kernel(
    const St<DT>* __restrict__ a, const St<DT>* __restrict__ b, float* __restrict__ partial,
    int64_t n, int64_t d) {
  const int64_t col = ((int64_t)blockIdx.x * kDotThreads + threadIdx.x) * VEC;
  if (col >= d) return;
  const int64_t r0 = (int64_t)blockIdx.y * kDotRows;
  const int64_t r1 = r0 + kDotRows < n ? r0 + kDotRows : n;
  float acc[VEC];
#pragma unroll
  for (int t = 0; t < VEC; ++t) acc[t] = 0.0f;
  for (int64_t r = r0; r < r1; ++r) {
    float va[VEC], vb[VEC];
    if constexpr (VEC == 8) {
      Vec8<DT>::ld(a, (r * d + col) / 8, va);
      Vec8<DT>::ld(b, (r * d + col) / 8, vb);
    } else {
      va[0] = Elem<DT>::ld(a + r * d + col);
      vb[0] = Elem<DT>::ld(b + r * d + col);
    }
#pragma unroll
    for (int t = 0; t < VEC; ++t) acc[t] += rd<DT>(va[t] * vb[t]);
  }
  float* p = partial + (int64_t)blockIdx.y * d + col;
#pragma unroll
  for (int t = 0; t < VEC; ++t) p[t] = acc[t];
}

template <int DT>
__global__ __launch_bounds__(kBlock) void col_dot_finish_kernel(const float* __restrict__ partial,
                                                                const St<DT>* __restrict__ den,
                                                                St<DT>* __restrict__ out,
                                                                int64_t d, int64_t chunks) {
  const int64_t col = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (col >= d) return;
  float acc = 0.0f;
  for (int64_t c = 0; c < chunks; ++c) acc += partial[c * d + col];
  Elem<DT>::st(out + col, acc / Elem<DT>::ld(den + col));
}

// ---------------------------------------------------------------------------
// dora_col_norm
// ---------------------------------------------------------------------------

// Per row j of W [rows, cols]: w2[j] = sum_i W_ji^2 (blockIdx.y == 0 only) and
// wa[j, k] = sum_i W_ji A_ki for the kRankTile ranks k of blockIdx.y.  Each
// wavefront owns kRowsPerWave rows, so one load of A serves all of them.
template <int DT, int VEC>
__global__ __launch_bounds__(kBlock) void dora_rows_kernel(const St<DT>* __restrict__ w,
                                                           const St<DT>* __restrict__ a,
                                                           int64_t rows, int64_t cols, int r,
                                                           float* __restrict__ w2,
                                                           float* __restrict__ wa) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t row0 = ((int64_t)blockIdx.x * (kBlock / 64) + wave) * kRowsPerWave;
  if (row0 >= rows) return;
  const int k0 = blockIdx.y * kRankTile;
  const bool do_sq = blockIdx.y == 0;
  float acc[kRowsPerWave][kRankTile];
  float sq[kRowsPerWave];
#pragma unroll
  for (int q = 0; q < kRowsPerWave; ++q) {
    sq[q] = 0.0f;
#pragma unroll
    for (int k = 0; k < kRankTile; ++k) acc[q][k] = 0.0f;
  }
  for (int64_t i = (int64_t)lane * VEC; i < cols; i += 64 * VEC) {
    float wv[kRowsPerWave][VEC];
#pragma unroll
    for (int q = 0; q < kRowsPerWave; ++q) {
      const int64_t row = row0 + q;
      if (row < rows) {
        if constexpr (VEC == 8) {
          Vec8<DT>::ld(w, (row * cols + i) / 8, wv[q]);
        } else {
          wv[q][0] = Elem<DT>::ld(w + row * cols + i);
        }
      } else {
#pragma unroll
        for (int t = 0; t < VEC; ++t) wv[q][t] = 0.0f;
      }
      if (do_sq) {
#pragma unroll
        for (int t = 0; t < VEC; ++t) sq[q] += wv[q][t] * wv[q][t];
      }
    }
#pragma unroll
    for (int k = 0; k < kRankTile; ++k) {
      if (k0 + k >= r) break;
      float av[VEC];
      if constexpr (VEC == 8) {
        Vec8<DT>::ld(a, ((int64_t)(k0 + k) * cols + i) / 8, av);
      } else {
        av[0] = Elem<DT>::ld(a + (int64_t)(k0 + k) * cols + i);
      }
#pragma unroll
      for (int q = 0; q < kRowsPerWave; ++q) {
#pragma unroll
        for (int t = 0; t < VEC; ++t) acc[q][k] += wv[q][t] * av[t];
      }
    }
  }
#pragma unroll
  for (int q = 0; q < kRowsPerWave; ++q) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sq[q] += __shfl_xor(sq[q], off);
#pragma unroll
    for (int k = 0; k < kRankTile; ++k) {
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) acc[q][k] += __shfl_xor(acc[q][k], off);
    }
  }
  if (lane != 0) return;
#pragma unroll
  for (int q = 0; q < kRowsPerWave; ++q) {
    const int64_t row = row0 + q;
    if (row >= rows) break;
    if (do_sq) w2[row] = sq[q];
#pragma unroll
    for (int k = 0; k < kRankTile; ++k) {
      if (k0 + k < r) wa[row * r + k0 + k] = acc[q][k];
    }
  }
}

// G[k, l] = sum_i A_ki A_li, one block per (k, l)
template <int DT>
__global__ __launch_bounds__(kBlock) void gram_kernel(const St<DT>* __restrict__ a, int64_t cols,
                                                      int r, float* __restrict__ g) {
  const int k = blockIdx.x / r;
  const int l = blockIdx.x % r;
  float acc = 0.0f;
  for (int64_t i = threadIdx.x; i < cols; i += kBlock)
    acc += Elem<DT>::ld(a + (int64_t)k * cols + i) * Elem<DT>::ld(a + (int64_t)l * cols + i);
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
  __shared__ float part[kBlock / 64];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) g[blockIdx.x] = (part[0] + part[1]) + (part[2] + part[3]);
}

// nu[j] = sqrt(max((w2 + 2s * sum_k B_jk wa_jk) + s^2 * sum_l (B G)_jl B_jl, 0))
template <int DT, int OUT_DT>
__global__ __launch_bounds__(kBlock) void dora_finish_kernel(const float* __restrict__ w2,
                                                             const float* __restrict__ wa,
                                                             const St<DT>* __restrict__ b,
                                                             const float* __restrict__ g,
                                                             float two_s, float s_sq,
                                                             int64_t rows, int r,
                                                             St<OUT_DT>* __restrict__ nu) {
  const int64_t j = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (j >= rows) return;
  const St<DT>* bj = b + j * r;
  float cross = 0.0f;
  for (int k = 0; k < r; ++k) cross += Elem<DT>::ld(bj + k) * wa[j * r + k];
  float quad = 0.0f;
  for (int l = 0; l < r; ++l) {
    float t = 0.0f;
    for (int k = 0; k < r; ++k) t += Elem<DT>::ld(bj + k) * g[k * r + l];
    quad += t * Elem<DT>::ld(bj + l);
  }
  const float v = (w2[j] + two_s * cross) + s_sq * quad;
  Elem<OUT_DT>::st(nu + j, sqrtf(v > 0.0f ? v : 0.0f));
}

inline unsigned blocks(int64_t items, int per) { return (unsigned)((items + per - 1) / per); }
inline int launched() { return hipGetLastError() == hipSuccess ? kOk : kErrLaunch; }
inline bool dtype_ok(int dt) { return dt == kF32 || dt == kF16 || dt == kBF16; }

template <int DT>
bool vec8_ok(const void* p, int64_t d) {
  return d % 8 == 0 && aligned16(p);
}

inline int64_t dot_chunks(int64_t n) { return (n + kDotRows - 1) / kDotRows; }

template <int DT>
int dora_scale_t(const void* x, const void* m, const void* nu, int64_t n, int64_t d, void* out,
                 hipStream_t st) {
  const int64_t total = n * d;
  if (vec8_ok<DT>(x, d) && aligned16(out)) {
    dora_scale_vec_kernel<DT><<<blocks(total / 8, kBlock), kBlock, 0, st>>>(
        x, (const St<DT>*)m, (const St<DT>*)nu, out, total / 8, d);
  } else {
    dora_scale_kernel<DT><<<blocks(total, kBlock), kBlock, 0, st>>>(
        (const St<DT>*)x, (const St<DT>*)m, (const St<DT>*)nu, (St<DT>*)out, total, d);
  }
  return launched();
}

template <int DT>
int col_dot_t(const void* a, const void* b, const void* den, int64_t n, int64_t d,
              void* workspace, void* out, hipStream_t st) {
  const int64_t chunks = dot_chunks(n);
  float* partial = (float*)workspace;
  if (chunks > 0) {
    if (vec8_ok<DT>(a, d) && aligned16(b)) {
      col_dot_partial_kernel<DT, 8><<<dim3(blocks(d / 8, kDotThreads), (unsigned)chunks),
                                      kDotThreads, 0, st>>>((const St<DT>*)a, (const St<DT>*)b,
                                                            partial, n, d);
    } else {
      col_dot_partial_kernel<DT, 1><<<dim3(blocks(d, kDotThreads), (unsigned)chunks),
                                      kDotThreads, 0, st>>>((const St<DT>*)a, (const St<DT>*)b,
                                                            partial, n, d);
    }
  }
  col_dot_finish_kernel<DT><<<blocks(d, kBlock), kBlock, 0, st>>>(partial, (const St<DT>*)den,
                                                                  (St<DT>*)out, d, chunks);
  return launched();
}

template <int DT, int OUT_DT>
void dora_finish_t(const float* w2, const float* wa, const void* b, const float* g, double s,
                   int64_t rows, int r, void* nu, hipStream_t st) {
  dora_finish_kernel<DT, OUT_DT><<<blocks(rows, kBlock), kBlock, 0, st>>>(
      w2, wa, (const St<DT>*)b, g, (float)(2.0 * s), (float)(s * s), rows, r, (St<OUT_DT>*)nu);
}

template <int DT>
int dora_col_norm_t(const void* w, const void* a, const void* b, int64_t rows, int64_t cols,
                    int r, double s, void* workspace, void* nu, int nu_dtype, hipStream_t st) {
  float* w2 = (float*)workspace;
  float* wa = w2 + rows;
  float* g = wa + rows * r;
  const unsigned row_blocks = blocks(rows, (kBlock / 64) * kRowsPerWave);
  const unsigned rank_tiles = r > 0 ? (unsigned)((r + kRankTile - 1) / kRankTile) : 1u;
  if (vec8_ok<DT>(w, cols) && aligned16(a)) {
    dora_rows_kernel<DT, 8><<<dim3(row_blocks, rank_tiles), kBlock, 0, st>>>(
        (const St<DT>*)w, (const St<DT>*)a, rows, cols, r, w2, wa);
  } else {
    dora_rows_kernel<DT, 1><<<dim3(row_blocks, rank_tiles), kBlock, 0, st>>>(
        (const St<DT>*)w, (const St<DT>*)a, rows, cols, r, w2, wa);
  }
  if (r > 0) gram_kernel<DT><<<(unsigned)(r * r), kBlock, 0, st>>>((const St<DT>*)a, cols, r, g);
  switch (nu_dtype) {
    case kF32: dora_finish_t<DT, kF32>(w2, wa, b, g, s, rows, r, nu, st); break;
    case kF16: dora_finish_t<DT, kF16>(w2, wa, b, g, s, rows, r, nu, st); break;
    default: dora_finish_t<DT, kBF16>(w2, wa, b, g, s, rows, r, nu, st); break;
  }
  return launched();
}

}  // namespace adapters
}  // namespace cpt

using namespace cpt;
using namespace cpt::adapters;

extern "C" {

int cpt_dora_scale(const void* x, const void* m, const void* nu, int64_t n, int64_t d, int dtype,
                   void* out, void* stream) {
  if (!dtype_ok(dtype)) return kErrDType;
  if (n < 0 || d < 0) return kErrShape;
  if (n == 0 || d == 0) return kOk;
  if (!x || !m || !nu || !out) return kErrShape;
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case kF32: return dora_scale_t<kF32>(x, m, nu, n, d, out, st);
    case kF16: return dora_scale_t<kF16>(x, m, nu, n, d, out, st);
    default: return dora_scale_t<kBF16>(x, m, nu, n, d, out, st);
  }
}

int64_t cpt_col_dot_workspace_bytes(int64_t n, int64_t d) {
  if (n < 0 || d < 0) return -1;
  const int64_t chunks = dot_chunks(n);
  return (chunks > 0 ? chunks : 1) * d * (int64_t)sizeof(float);
}

int cpt_col_dot_div(const void* a, const void* b, const void* den, int64_t n, int64_t d,
                    int dtype, void* workspace, void* out, void* stream) {
  if (!dtype_ok(dtype)) return kErrDType;
  if (n < 0 || d < 0) return kErrShape;
  if (d == 0) return kOk;
  if (!den || !out || (n > 0 && (!a || !b || !workspace))) return kErrShape;
  if (dot_chunks(n) > 65535) return kErrTooLarge;
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case kF32: return col_dot_t<kF32>(a, b, den, n, d, workspace, out, st);
    case kF16: return col_dot_t<kF16>(a, b, den, n, d, workspace, out, st);
    default: return col_dot_t<kBF16>(a, b, den, n, d, workspace, out, st);
  }
}

int64_t cpt_dora_col_norm_workspace_bytes(int64_t rows, int64_t r) {
  if (rows < 0 || r < 0) return -1;
  return (rows + rows * r + r * r) * (int64_t)sizeof(float);
}

int cpt_dora_col_norm(const void* w, const void* a, const void* b, int64_t rows, int64_t cols,
                      int64_t r, double s, int dtype, void* workspace, void* nu, int nu_dtype,
                      void* stream) {
  if (!dtype_ok(dtype) || !dtype_ok(nu_dtype)) return kErrDType;
  if (rows < 0 || cols < 0 || r < 0) return kErrShape;
  if (rows == 0) return kOk;
  if (!w || !nu || !workspace || (r > 0 && (!a || !b))) return kErrShape;
  if (r > 4096 || rows > ((int64_t)1 << 40)) return kErrTooLarge;
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case kF32: return dora_col_norm_t<kF32>(w, a, b, rows, cols, (int)r, s, workspace, nu, nu_dtype, st);
    case kF16: return dora_col_norm_t<kF16>(w, a, b, rows, cols, (int)r, s, workspace, nu, nu_dtype, st);
    default: return dora_col_norm_t<kBF16>(w, a, b, rows, cols, (int)r, s, workspace, nu, nu_dtype, st);
  }
}

}  // extern "C"
