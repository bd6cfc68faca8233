// Measurement probes.
//
// cpt_probe_mfma_rate: the sustained bf16 MFMA rate of the part, for the
// achievable-peak figure the GEMM roofline is read against.
//
// Every wavefront issues `iters` rounds of 16 independent MFMAs of one shape
// (16 accumulator blocks, so no MFMA waits on another's result) on register
// operands: no memory traffic and no LDS in the loop.  Shape 0 is
// v_mfma_f32_32x32x16_bf16 (2 * 32 * 32 * 16 = 32768 FLOPs), shape 1
// v_mfma_f32_16x16x32_bf16 (16384 FLOPs).  One block of 4 wavefronts per CU
// (one per SIMD), `blocks` blocks.  The accumulators are summed into
// out[4 * block + wave] so the work is not removed.
// FLOPs per launch = blocks * 4 * iters * 16 * (FLOPs per MFMA).

#include "common.h"
#include "compact_amd.h"

namespace cpt {
namespace probe {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Accumulator block of one MFMA shape and the instruction that updates it.
// The tied "+a" operand keeps each block in its own AGPRs (the builtin form
// lets the register allocator move blocks between rounds, which adds
// accvgpr copies to the loop).
template <int SHAPE>
struct Mfma;
template <>
struct Mfma<0> {  // v_mfma_f32_32x32x16_bf16: 32768 FLOPs
  typedef f32x16 acc_t;
  static constexpr int N = 16;
  __device__ static void issue(acc_t& c, const bf16x8& a, const bf16x8& b) {
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
  }
};
template <>
struct Mfma<1> {  // v_mfma_f32_16x16x32_bf16: 16384 FLOPs
  typedef f32x4 acc_t;
  static constexpr int N = 4;
  __device__ static void issue(acc_t& c, const bf16x8& a, const bf16x8& b) {
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
  }
};

template <int SHAPE>
__global__ __launch_bounds__(256, 1) void mfma_rate_kernel(int iters, float seed, float* out) {
  typedef Mfma<SHAPE> M;
  const int lane = threadIdx.x & 63;
  // two operand sets of hashed values in [-1, 1), used alternately so the
  // operand buses toggle on every issue as they do in a GEMM on random data
  bf16x8 a[2], b[2];
#pragma unroll
  for (int k = 0; k < 2; ++k)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      uint32_t h = (uint32_t)(((k * 64 + lane) * 8 + e) * 2) * 2654435761u ^ __float_as_uint(seed);
      h ^= h >> 15;
      h *= 2246822519u;
      h ^= h >> 13;
      a[k][e] = (__bf16)((float)(h & 0xffff) * (1.0f / 32768.0f) - 1.0f);
      b[k][e] = (__bf16)((float)(h >> 16) * (1.0f / 32768.0f) - 1.0f);
    }
  typename M::acc_t acc[16];
#pragma unroll
  for (int t = 0; t < 16; ++t)
#pragma unroll
    for (int r = 0; r < M::N; ++r) acc[t][r] = 0.0f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int t = 0; t < 16; ++t) M::issue(acc[t], a[t & 1], b[t & 1]);
  }
  float s = 0.0f;
#pragma unroll
  for (int t = 0; t < 16; ++t)
#pragma unroll
    for (int r = 0; r < M::N; ++r) s += acc[t][r];
  // one partial per wavefront, written through a vector store
  if (lane == 0) out[blockIdx.x * 4 + (threadIdx.x >> 6)] = s;
}

}  // namespace probe
}  // namespace cpt

extern "C" int cpt_probe_mfma_rate(int shape, int blocks, int iters, float seed, void* out,
                                   void* stream) {
  if (blocks <= 0 || iters <= 0 || !out) return cpt::kErrShape;
  if (shape == 0)
    hipLaunchKernelGGL(cpt::probe::mfma_rate_kernel<0>, dim3((unsigned)blocks), dim3(256), 0,
                       (hipStream_t)stream, iters, seed, (float*)out);
  else if (shape == 1)
    hipLaunchKernelGGL(cpt::probe::mfma_rate_kernel<1>, dim3((unsigned)blocks), dim3(256), 0,
                       (hipStream_t)stream, iters, seed, (float*)out);
  else
    return cpt::kErrShape;
  return hipGetLastError() == hipSuccess ? cpt::kOk : cpt::kErrLaunch;
}
