// Tile GEMM kernels with 256 x 256 blocks (waves 2 x 4): bf16 and fp8, every store mode.
#include "hkx_launch.hpp"

namespace hkx {
HKX_TILE_LAUNCHER(256, 256, 2)
}  // namespace hkx
