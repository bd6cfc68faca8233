// Instantiations of the 16x16x32 NT loop (gemm16_kernel.h): F1 with the
// outlier channels in its codec epilogue, group CPT_NT16_INST_GLUO (compiled
// on their own so the groups build in parallel).

#include "gemm16_kernel.h"

namespace cpt {
namespace gemm {

CPT_NT16_INST_GLUO(CPT_NT16_DEFINE)

}  // namespace gemm
}  // namespace cpt
