// Launcher instantiations: MBS_SKINNY_SHAPES of gemm_kernels.h (one translation unit
// per group so the kernel families build in parallel).
#include "gemm_kernels.h"

namespace mbs {
MBS_SKINNY_SHAPES(MBS_SKINNY_INST)
MBS_SKINNY_BF16A_SHAPES(MBS_SKINNY_BF16A_INST)
}  // namespace mbs
