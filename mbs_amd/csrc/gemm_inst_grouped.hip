// Launcher instantiations: MBS_GROUPED_SHAPES of gemm_kernels.h (one translation
// unit per group so the kernel families build in parallel).
#include "gemm_kernels.h"

namespace mbs {
MBS_GROUPED_SHAPES(MBS_GROUPED_INST)
}  // namespace mbs
