// Contraction kernels of tile configuration TileS (bf_gemm_kernel.h).

#include "bf_gemm_kernel.h"

namespace bf {
BF_DEFINE_LAUNCH_TILE(TileS)
}  // namespace bf
