// Contraction kernels of tile configuration TileQ (bf_gemm_kernel.h).

#include "bf_gemm_kernel.h"

namespace bf {
BF_DEFINE_LAUNCH_TILE(TileQ)
}  // namespace bf
