// Launcher instantiations: MBS_BDIRECT_SHAPES_E of gemm_kernels.h (one translation unit
// per group so the kernel families build in parallel).
#include "gemm_kernels.h"

namespace mbs {
MBS_BDIRECT_SHAPES_E(MBS_BDIRECT_INST)
}  // namespace mbs
