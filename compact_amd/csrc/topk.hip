// Top-K activation compression of the FlashFFN v1/v2 API (reference
// src/flashffn.py:300-470): per row of h_mid [n, d], the k entries of largest
// magnitude and their column indices (int16), and the inverse scatter back to
// a dense [n, d] row with zeros elsewhere.
//
//   topk_abs      one workgroup per row.  The k-th largest |x| is found by a
//                 radix select over the magnitude bits (8 bits per pass: two
//                 passes for 16-bit dtypes, four for fp32), each pass a
//                 256-bin LDS histogram of the row restricted to the prefix
//                 chosen so far.  A final pass in column order keeps every
//                 entry above that threshold and, of the entries equal to it,
//                 the ones with the lowest columns; the output is in
//                 ascending column order.  The reference calls torch.topk
//                 with sorted=False, whose order and tie choice are
//                 unspecified; this kernel fixes both.
//   topk_scatter  one workgroup per row: the row is assembled in LDS (zeros,
//                 then the k values at their columns) and written coalesced.
// Magnitude keys are the IEEE bits with the sign cleared, so their unsigned
// order is the order of |x| (NaN above inf, as torch.topk orders it).

#include "common.h"
#include "compact_amd.h"

namespace cpt {
namespace topk {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / 64;

template <int DT> struct Key;
template <> struct Key<kF32> {
  static constexpr int kPasses = 4;
  static __device__ __forceinline__ uint32_t of(const float* p, int64_t i) {
    return __float_as_uint(p[i]) & 0x7FFFFFFFu;
  }
};
template <> struct Key<kBF16> {
  static constexpr int kPasses = 2;
  static __device__ __forceinline__ uint32_t of(const uint16_t* p, int64_t i) {
    return p[i] & 0x7FFFu;
  }
};
template <> struct Key<kF16> : Key<kBF16> {};

template <int DT> using St = typename Elem<DT>::T;

// Inclusive scan of one value per thread across the workgroup.  `tmp` holds
// kWaves ints of LDS.  Ends with a barrier, so `tmp` may be reused.
__device__ __forceinline__ int block_inclusive_scan(int v, int* tmp) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int u = __shfl_up(v, off);
    if (lane >= off) v += u;
  }
  if (lane == 63) tmp[wave] = v;
  __syncthreads();
  int base = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) base += w < wave ? tmp[w] : 0;
  __syncthreads();
  return v + base;
}

template <int DT>
__global__ __launch_bounds__(kBlock) void topk_abs_kernel(const St<DT>* __restrict__ t,
                                                          int64_t d, int64_t k,
                                                          St<DT>* __restrict__ values,
                                                          int16_t* __restrict__ indices) {
  __shared__ int hist[256];
  __shared__ int tmp[kWaves];
  __shared__ uint32_t sh_prefix;
  __shared__ int sh_remaining;
  __shared__ int sh_wave[kWaves][2];

  const int64_t row = blockIdx.x;
  const St<DT>* x = t + row * d;
  const int tid = threadIdx.x;

  uint32_t prefix = 0, mask = 0;
  int remaining = (int)k;
  for (int pass = Key<DT>::kPasses - 1; pass >= 0; --pass) {
    const int shift = pass * 8;
    hist[tid] = 0;
    __syncthreads();
    for (int64_t i = tid; i < d; i += kBlock) {
      const uint32_t key = Key<DT>::of(x, i);
      if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 0xFF], 1);
    }
    __syncthreads();
    // thread t takes digit 255 - t: cumulative counts from the largest digit
    const int c = hist[255 - tid];
    const int cum = block_inclusive_scan(c, tmp);
    if (cum >= remaining && cum - c < remaining) {
      sh_prefix = prefix | ((uint32_t)(255 - tid) << shift);
      sh_remaining = remaining - (cum - c);
    }
    __syncthreads();
    prefix = sh_prefix;
    remaining = sh_remaining;
    mask |= 0xFFu << shift;
    __syncthreads();
  }
  // prefix is the k-th largest key; take every key above it and the first
  // `remaining` keys equal to it, in column order
  const uint32_t thr = prefix;
  const int need_eq = remaining;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int run_eq = 0, run_sel = 0;
  for (int64_t c0 = 0; c0 < d; c0 += kBlock) {
    const int64_t i = c0 + tid;
    uint32_t key = 0;
    bool gt = false, eq = false;
    if (i < d) {
      key = Key<DT>::of(x, i);
      gt = key > thr;
      eq = key == thr;
    }
    const uint64_t m_eq = __ballot(eq);
    if (lane == 0) sh_wave[wave][0] = __popcll(m_eq);
    __syncthreads();
    int eq_before = run_eq + __popcll(m_eq & below);
    int eq_total = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      eq_before += w < wave ? sh_wave[w][0] : 0;
      eq_total += sh_wave[w][0];
    }
    const bool sel = gt || (eq && eq_before < need_eq);
    const uint64_t m_sel = __ballot(sel);
    if (lane == 0) sh_wave[wave][1] = __popcll(m_sel);
    __syncthreads();
    int pos = run_sel + __popcll(m_sel & below);
    int sel_total = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      pos += w < wave ? sh_wave[w][1] : 0;
      sel_total += sh_wave[w][1];
    }
    if (sel && pos < k) {
      values[row * k + pos] = x[i];
      indices[row * k + pos] = (int16_t)i;
    }
    run_eq += eq_total;
    run_sel += sel_total;
    __syncthreads();
  }
}

template <int DT>
__global__ __launch_bounds__(kBlock) void topk_scatter_kernel(const St<DT>* __restrict__ values,
                                                              const int16_t* __restrict__ indices,
                                                              int64_t d, int64_t k,
                                                              St<DT>* __restrict__ out) {
  extern __shared__ __align__(16) unsigned char smem[];
  St<DT>* rowbuf = reinterpret_cast<St<DT>*>(smem);
  const int64_t row = blockIdx.x;
  for (int64_t i = threadIdx.x; i < d; i += kBlock) rowbuf[i] = (St<DT>)0;
  __syncthreads();
  for (int64_t j = threadIdx.x; j < k; j += kBlock) {
    const int c = indices[row * k + j];
    if (c >= 0 && c < d) rowbuf[c] = values[row * k + j];
  }
  __syncthreads();
  for (int64_t i = threadIdx.x; i < d; i += kBlock) out[row * d + i] = rowbuf[i];
}

inline int launched() { return hipGetLastError() == hipSuccess ? kOk : kErrLaunch; }

int elem_bytes(int dt) { return dt == kF32 ? 4 : 2; }

}  // namespace topk
}  // namespace cpt

using namespace cpt;
using namespace cpt::topk;

extern "C" {

int cpt_topk_abs(const void* t, int dtype, int64_t n, int64_t d, int64_t k, void* values,
                 void* indices, void* stream) {
  if (dtype != kF32 && dtype != kF16 && dtype != kBF16) return kErrDType;
  if (n < 0 || d < 0 || k < 0 || k > d) return kErrShape;
  if (d > 32767 || n > 0x7FFFFFFF) return kErrTooLarge;   // int16 column indices
  if (n == 0 || k == 0) return kOk;
  if (!t || !values || !indices) return kErrShape;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)n);
  switch (dtype) {
    case kF32:
      topk_abs_kernel<kF32><<<grid, kBlock, 0, st>>>((const float*)t, d, k, (float*)values,
                                                     (int16_t*)indices);
      break;
    case kF16:
      topk_abs_kernel<kF16><<<grid, kBlock, 0, st>>>((const uint16_t*)t, d, k,
                                                     (uint16_t*)values, (int16_t*)indices);
      break;
    default:
      topk_abs_kernel<kBF16><<<grid, kBlock, 0, st>>>((const uint16_t*)t, d, k,
                                                      (uint16_t*)values, (int16_t*)indices);
      break;
  }
  return launched();
}

int cpt_topk_scatter(const void* values, const void* indices, int dtype, int64_t n, int64_t d,
                     int64_t k, void* out, void* stream) {
  if (dtype != kF32 && dtype != kF16 && dtype != kBF16) return kErrDType;
  if (n < 0 || d < 0 || k < 0) return kErrShape;
  if (d > 32767 || n > 0x7FFFFFFF || d * elem_bytes(dtype) > 65536) return kErrTooLarge;
  if (n == 0 || d == 0) return kOk;
  if (!out || (k > 0 && (!values || !indices))) return kErrShape;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)n);
  const size_t lds = (size_t)d * elem_bytes(dtype);
  switch (dtype) {
    case kF32:
      topk_scatter_kernel<kF32><<<grid, kBlock, lds, st>>>((const float*)values,
                                                           (const int16_t*)indices, d, k,
                                                           (float*)out);
      break;
    case kF16:
      topk_scatter_kernel<kF16><<<grid, kBlock, lds, st>>>((const uint16_t*)values,
                                                           (const int16_t*)indices, d, k,
                                                           (uint16_t*)out);
      break;
    default:
      topk_scatter_kernel<kBF16><<<grid, kBlock, lds, st>>>((const uint16_t*)values,
                                                            (const int16_t*)indices, d, k,
                                                            (uint16_t*)out);
      break;
  }
  return launched();
}

}  // extern "C"
