// Kernel instantiations of the GEMM engine: the CPT_GEMM_INST_WGLU group
// (see gemm_kernel.h), compiled on their own so the groups build in parallel.

#include "gemm_kernel.h"

namespace cpt {
namespace gemm {

CPT_GEMM_INST_WGLU(CPT_GEMM_DEFINE)

}  // namespace gemm
}  // namespace cpt
