// Tile GEMM kernels with 128 x 128 blocks (waves 2 x 4): bf16 and fp8, every store mode.
#include "hkx_launch.hpp"

namespace hkx {
HKX_TILE_LAUNCHER(128, 128, 2)
}  // namespace hkx
