// bf16 transpose for GEMM operands: dst [cols][ld_dst] = src [rows][ld_src]^T.
//
// The weight gradients dg^T x and du^T x read x along its rows, the reduction
// (token) dimension, which makes x an MN-major B operand of the 16x16x32 loop:
// its fragments come from two transposing LDS reads each.  With x^T written
// once, both products read B K-major (one 128-bit LDS read per fragment); the
// k order of their MFMAs is unchanged, so the results are bit-identical.
//
// Each thread transposes an 8 x 8 block in registers: 8 16-byte loads (one per
// source row), 32 byte permutes, 8 16-byte stores (one per destination row).
// The 8 threads of a block row cover 128 contiguous bytes of each source row
// and of each destination row, so loads and stores are 128-byte segments; no
// LDS, no barrier.  A wavefront covers a 64 x 64 tile.  HBM-bound: rows *
// cols * 4 bytes per launch.

#include "common.h"
#include "compact_amd.h"

namespace cpt {
namespace {

constexpr int kTile = 64;   // rows and columns per wavefront

__global__ __launch_bounds__(256) void transpose_bf16_kernel(
    const uint16_t* __restrict__ src, int64_t ld_src, uint16_t* __restrict__ dst,
    int64_t ld_dst, int64_t rows, int64_t cols) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // block: 4 wavefronts side by side along the columns
  const int64_t r0 = (int64_t)blockIdx.y * kTile + (lane >> 3) * 8;
  const int64_t c0 = ((int64_t)blockIdx.x * 4 + wave) * kTile + (lane & 7) * 8;
  // rows and columns are multiples of 8 (checked on the host): an 8 x 8 block
  // is wholly in or out
  if (r0 >= rows || c0 >= cols) return;
  uint32_t w[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint4 v = *reinterpret_cast<const uint4*>(src + (r0 + i) * ld_src + c0);
    w[i][0] = v.x; w[i][1] = v.y; w[i][2] = v.z; w[i][3] = v.w;
  }
  // destination row c0 + c holds column c of the 8 source rows: word k pairs
  // rows 2k (low half) and 2k + 1 (high half) of that column
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t a = w[2 * k][c >> 1], b = w[2 * k + 1][c >> 1];
      // v_perm_b32 (S0 = b, S1 = a): selectors 0-3 pick bytes of a, 4-7 of b;
      // result byte i is selector byte i
      o[k] = (c & 1) ? __builtin_amdgcn_perm(b, a, 0x07060302u)    // a.hi | b.hi << 16
                     : __builtin_amdgcn_perm(b, a, 0x05040100u);   // a.lo | b.lo << 16
    }
    *reinterpret_cast<uint4*>(dst + (c0 + c) * ld_dst + r0) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

}  // namespace
}  // namespace cpt

extern "C" int cpt_transpose_bf16(const void* src, int64_t ld_src, int64_t rows, int64_t cols,
                                  void* dst, int64_t ld_dst, void* stream) {
  using namespace cpt;
  if (rows < 0 || cols < 0) return kErrShape;
  if (rows == 0 || cols == 0) return kOk;
  if (!src || !dst || ld_src < cols || ld_dst < rows) return kErrShape;
  if ((rows & 7) || (cols & 7) || (ld_src & 7) || (ld_dst & 7) || !aligned16(src) ||
      !aligned16(dst))
    return kErrAlign;
  const int64_t gx = (cols + 4 * kTile - 1) / (4 * kTile), gy = (rows + kTile - 1) / kTile;
  if (gx > 0x7FFFFFFF || gy > 65535) return kErrTooLarge;
  hipLaunchKernelGGL(transpose_bf16_kernel, dim3((unsigned)gx, (unsigned)gy), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)src, ld_src, (uint16_t*)dst, ld_dst,
                     rows, cols);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}
