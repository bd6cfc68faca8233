// Kernel instantiations of the GEMM engine: the CPT_GEMM_INST_STORE group
// (see gemm_kernel.h), compiled on their own so the groups build in parallel.

#include "gemm_kernel.h"

namespace cpt {
namespace gemm {

CPT_GEMM_INST_STORE(CPT_GEMM_DEFINE)

}  // namespace gemm
}  // namespace cpt
