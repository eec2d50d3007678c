// Tile GEMM kernels with 64 x 256 blocks (waves 1 x 8): bf16 and fp8, every store mode.
#include "hkx_launch.hpp"

namespace hkx {
HKX_TILE_LAUNCHER(64, 256, 1)
}  // namespace hkx
