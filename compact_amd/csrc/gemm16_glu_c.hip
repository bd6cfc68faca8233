// Instantiations of the 16x16x32 NT loop (gemm16_kernel.h): the F1 epilogues,
// group CPT_NT16_INST_GLU_C (compiled on their own so the groups build in parallel).

#include "gemm16_kernel.h"

namespace cpt {
namespace gemm {

CPT_NT16_INST_GLU_C(CPT_NT16_DEFINE)

}  // namespace gemm
}  // namespace cpt
