// Instantiations of the 16x16x32 NT loop (gemm16_kernel.h): the plain store,
// and the shape test the host dispatch uses for it.

#include "gemm16_kernel.h"

namespace cpt {
namespace gemm {

bool nt16_fits(int64_t M, int64_t N, int64_t K, const void* c, int64_t ldc) {
  constexpr int64_t kIntMax = 0x7FFFFFFF;
  return M > 0 && N > 0 && K > 0 && M <= kIntMax && N <= kIntMax && K <= kIntMax &&
         N % 8 == 0 && K % nt16::kBK == 0 && (ldc & 7) == 0 &&
         (reinterpret_cast<uintptr_t>(c) & 15) == 0 &&
         ((M + 255) / 256) * ((N + 255) / 256) <= kIntMax;
}

// Stream-K workspace attached per device (cpt_gemm_stream_k_workspace): the
// caller's memory, never allocated here.
namespace {
constexpr int kMaxDevices = 64;
struct SkSlot {
  void* ptr = nullptr;
  int64_t bytes = 0;
  int cus = 0;
};
SkSlot g_sk[kMaxDevices];

int device_cus(int dev) {
  if (g_sk[dev].cus == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return 0;
    g_sk[dev].cus = n;
  }
  return g_sk[dev].cus;
}
}  // namespace

int64_t stream_k_bytes(int cus) {
  // cus partial slots of one tile's fp32 accumulators, then cus flags and
  // one error count
  return (int64_t)cus * nt16::kSkSlot * 4 + ((int64_t)cus + 1) * 4;
}

bool stream_k_plan(int64_t tiles, int nk, StreamK& sk) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return false;
  const SkSlot& w = g_sk[dev];
  if (!w.ptr) return false;
  const int S = device_cus(dev);
  // worth it only past one wave, with a part-empty last wave and enough
  // k-tiles per tile to amortise the partials
  if (S <= 0 || tiles <= S || tiles % S == 0 || nk < 4) return false;
  // 32-bit iteration counts in the kernel
  if ((tiles % S + S) * (int64_t)nk >= ((int64_t)1 << 31)) return false;
  if (w.bytes < stream_k_bytes(S)) return false;
  sk.tiles = tiles % S + S;
  sk.blocks = S;
  sk.ws = static_cast<float*>(w.ptr);
  sk.flags = reinterpret_cast<int*>(static_cast<char*>(w.ptr) + (int64_t)S * nt16::kSkSlot * 4);
  return true;
}

CPT_NT16_INST_STORE(CPT_NT16_DEFINE)

}  // namespace gemm
}  // namespace cpt

extern "C" int64_t cpt_gemm_stream_k_bytes(void) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= cpt::gemm::kMaxDevices) return -1;
  const int cus = cpt::gemm::device_cus(dev);
  return cus > 0 ? cpt::gemm::stream_k_bytes(cus) : -1;
}

extern "C" int cpt_gemm_stream_k_workspace(void* workspace, int64_t bytes) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= cpt::gemm::kMaxDevices)
    return cpt::kErrLaunch;
  if (workspace && (bytes < cpt_gemm_stream_k_bytes() ||
                    (reinterpret_cast<uintptr_t>(workspace) & 255) != 0))
    return cpt::kErrShape;
  cpt::gemm::g_sk[dev].ptr = workspace;
  cpt::gemm::g_sk[dev].bytes = workspace ? bytes : 0;
  return cpt::kOk;
}
