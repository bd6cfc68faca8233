// Instantiations of the 16x16x32 NT loop (gemm16_kernel.h): B1, the down
// projection's dgrad with the dequantise + SwiGLU backward epilogue, group
// CPT_NT16_INST_DGLU_B (compiled on their own so the groups build in parallel).

#include "gemm16_kernel.h"

namespace cpt {
namespace gemm {

CPT_NT16_INST_DGLU_B(CPT_NT16_DEFINE)

}  // namespace gemm
}  // namespace cpt
