// Launcher instantiations: MBS_TILED_SHAPES of gemm_kernels.h (one translation unit
// per group so the kernel families build in parallel).
#include "gemm_kernels.h"

namespace mbs {
MBS_TILED_SHAPES(MBS_TILED_INST)
}  // namespace mbs
