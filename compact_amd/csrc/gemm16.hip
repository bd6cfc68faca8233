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

CPT_NT16_INST_STORE(CPT_NT16_DEFINE)

}  // namespace gemm
}  // namespace cpt
