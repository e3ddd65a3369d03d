// Launcher instantiations: MBS_GROUPED_SHAPES_M of gemm_kernels.h (the grouped
// 32x32x64-MFMA tiles, in their own translation unit so they build in parallel).
#include "gemm_kernels.h"

namespace mbs {
MBS_GROUPED_SHAPES_M(MBS_GROUPED_INST)
}  // namespace mbs
