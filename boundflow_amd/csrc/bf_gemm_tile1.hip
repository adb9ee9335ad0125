// Contraction kernels of tile configuration TileB (bf_gemm_kernel.h).

#include "bf_gemm_kernel.h"

namespace bf {
BF_DEFINE_LAUNCH_TILE(TileB)
}  // namespace bf
