// Tile GEMM kernels with 256 x 128 blocks (waves 4 x 2): bf16 and fp8, every store mode.
#include "hkx_launch.hpp"

namespace hkx {
HKX_TILE_LAUNCHER(256, 128, 4)
}  // namespace hkx
