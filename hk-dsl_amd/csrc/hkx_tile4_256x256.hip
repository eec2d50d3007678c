// 4-wave tile GEMM kernels with 256 x 256 blocks: bf16 and fp8, every store mode.
#include "hkx_launch.hpp"

namespace hkx {
HKX_TILE4_LAUNCHER(256, 256)
}  // namespace hkx
