// 4-wave tile GEMM kernels with 128 x 128 blocks: bf16 and fp8, every store mode.
#include "hkx_launch.hpp"

namespace hkx {
HKX_TILE4_LAUNCHER(128, 128)
}  // namespace hkx
