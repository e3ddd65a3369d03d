// Launcher instantiations: MBS_SKINNY_SHAPES of gemm_kernels.h (one translation unit
// per group so the kernel families build in parallel).
#include "gemm_kernels.h"

namespace mbs {
MBS_SKINNY_SHAPES(MBS_SKINNY_INST)
}  // namespace mbs
