// Host-side launchers of the kernel templates, one explicit instantiation set per
// translation unit (hkx_tile_*.hip, hkx_decode.hip, hkx_reduce.hip) so the build
// compiles them in parallel.
#pragma once

#include <hip/hip_runtime.h>

#include "hkx_decode.hpp"
#include "hkx_reduce.hpp"
#include "hkx_tile.hpp"
#include "hkx_tile4.hpp"

namespace hkx {

template <int BM, int BN, int WM>
hipError_t launch_tile(const TileArgs& a, bool fp8, int mode, dim3 grid, hipStream_t s);

template <int BM, int BN>
hipError_t launch_tile4(const TileArgs& a, bool fp8, int mode, dim3 grid,
                        hipStream_t s);

// A 16- or 8-bit C with the fused form's activation fixed at compile time (the epilogue is
// then straight-line code); any other store takes it at run time.
#define HKX_TILE4_STAGED(BM, BN, FP8, MODE)                                                 \
  switch (a.ep.form == HKX_EP_FUSED ? a.ep.act : HKX_ACT_NONE) {                            \
    case HKX_ACT_GELU_TANH: hipLaunchKernelGGL((tile4_kernel<BM, BN, FP8, MODE, HKX_ACT_GELU_TANH>), grid, block, 0, s, a); break; \
    case HKX_ACT_SILU: hipLaunchKernelGGL((tile4_kernel<BM, BN, FP8, MODE, HKX_ACT_SILU>), grid, block, 0, s, a); break;           \
    case HKX_ACT_RELU: hipLaunchKernelGGL((tile4_kernel<BM, BN, FP8, MODE, HKX_ACT_RELU>), grid, block, 0, s, a); break;           \
    default: hipLaunchKernelGGL((tile4_kernel<BM, BN, FP8, MODE, HKX_ACT_NONE>), grid, block, 0, s, a); break;                    \
  }

hipError_t launch_pp(const TileArgs& a, bool fp8, int mode, bool mf16, dim3 grid, hipStream_t s);

// The persistent ring kernel (hkx_ring.hpp): grid.x workgroups, each every grid.x-th tile.
// Returns hipErrorInvalidValue for a call it does not take (ring_takes is false).
bool ring_takes(const TileArgs& a, bool fp8, int mode);
hipError_t launch_ring(const TileArgs& a, bool fp8, int mode, dim3 grid, hipStream_t s);
hipError_t launch_ring_bf16(const TileArgs& a, int mode, int epf, int act, dim3 grid, hipStream_t s);
hipError_t launch_ring_fp8(const TileArgs& a, int mode, int epf, int act, dim3 grid, hipStream_t s);
// The quadrant ring kernel (hkx_quad.hpp): a 16-bit bf16 C, no split; bf16 operands with no
// epilogue, a bias and an activation, a residual tile, or the paired silu * up form; fp8
// operands with no epilogue or the dequant forms (row and column fp32 scales, a bf16 bias).
// Vectors of unit stride, 16-byte aligned. Or, unpaired, a K split's fp32 shares (mode
// kStoreF32, blockIdx.y the split). quad_takes says which calls.
bool quad_takes(const TileArgs& a, bool fp8, int mode);
// The quadrant kernel on 128 x 256 tiles (bf16, one phase a K-tile): the calls it takes, and
// its launch (grid: one workgroup a CU at most).
bool quad128_takes(const TileArgs& a, bool fp8, int mode);
hipError_t launch_quad128(const TileArgs& a, int mode, dim3 grid, hipStream_t s);
hipError_t launch_quad(const TileArgs& a, bool fp8, int mode, dim3 grid, hipStream_t s);
// Its MX form (fp8 operands, E8M0 block scales in a.sa / a.sb, bf16 C, one pass).
hipError_t launch_quad_mx(const TileArgs& a, dim3 grid, hipStream_t s);
// The MX form (fp8 operands, E8M0 block scales in a.sa / a.sb), no epilogue: bf16 C, or
// fp32 shares of a K split (f32_shares, a.c the workspace, grid.y the splits).
hipError_t launch_ring_mx(const TileArgs& a, bool f32_shares, dim3 grid, hipStream_t s);
// MX quantization of bf16 rows (hkx_mx_quant).
hipError_t launch_mx_quant(const void* x, int64_t ldx, void* q, int64_t ldq, uint8_t* sc,
                           int64_t lds, int m, int k, hipStream_t s);

hipError_t launch_decode(const DecodeArgs& a, int waves, int fn, int mf, int mode, dim3 grid,
                         hipStream_t s);

// The streaming decode kernel (stream_kernel): M <= 16, K a multiple of 1024 up to 32768,
// no split, unpaired.
bool stream_takes(const DecodeArgs& a, int splits, bool pair);
hipError_t launch_stream(const DecodeArgs& a, dim3 grid, hipStream_t s);
// the whole-row decode kernel (K = 4096, M <= 4, N <= 32768), for calls stream_takes accepts
bool rows_takes(const DecodeArgs& a);
hipError_t launch_rows(const DecodeArgs& a, dim3 grid, hipStream_t s);
// the per-wave whole-row decode kernel (K = 1024 with M <= 3, K = 2048 with M <= 2), for calls
// stream_takes accepts; grid: the workgroups it will be launched with
bool roww_takes(const DecodeArgs& a, int grid);
hipError_t launch_roww(const DecodeArgs& a, dim3 grid, hipStream_t s);

hipError_t launch_reduce(const ReduceArgs& a, const HkxEpilogue& ep, bool program, dim3 grid,
                         hipStream_t s);

#define HKX_TILE_LAUNCHER(BM, BN, WM)                                                        \
  template <>                                                                                \
  hipError_t launch_tile<BM, BN, WM>(const TileArgs& a, bool fp8, int mode, dim3 grid,       \
                                     hipStream_t s) {                                        \
    const dim3 block(512);                                                                   \
    if (fp8) {                                                                               \
      switch (mode) {                                                                        \
        case kStore16: hipLaunchKernelGGL((tile_kernel<BM, BN, WM, true, kStore16>), grid, block, 0, s, a); break;   \
        case kStore8: hipLaunchKernelGGL((tile_kernel<BM, BN, WM, true, kStore8>), grid, block, 0, s, a); break;     \
        case kStoreF32: hipLaunchKernelGGL((tile_kernel<BM, BN, WM, true, kStoreF32>), grid, block, 0, s, a); break; \
        default: return hipErrorInvalidValue;                                                \
      }                                                                                      \
    } else {                                                                                 \
      switch (mode) {                                                                        \
        case kStore16: hipLaunchKernelGGL((tile_kernel<BM, BN, WM, false, kStore16>), grid, block, 0, s, a); break;   \
        case kStore8: hipLaunchKernelGGL((tile_kernel<BM, BN, WM, false, kStore8>), grid, block, 0, s, a); break;     \
        case kStoreF32: hipLaunchKernelGGL((tile_kernel<BM, BN, WM, false, kStoreF32>), grid, block, 0, s, a); break; \
        case kPair16: hipLaunchKernelGGL((tile_kernel<BM, BN, WM, false, kPair16>), grid, block, 0, s, a); break;     \
        case kPairWs: hipLaunchKernelGGL((tile_kernel<BM, BN, WM, false, kPairWs>), grid, block, 0, s, a); break;     \
        default: return hipErrorInvalidValue;                                                \
      }                                                                                      \
    }                                                                                        \
    return hipGetLastError();                                                                \
  }

#define HKX_TILE4_LAUNCHER(BM, BN)                                                           \
  template <>                                                                                \
  hipError_t launch_tile4<BM, BN>(const TileArgs& a, bool fp8, int mode, dim3 grid,        \
                                  hipStream_t s) {                                           \
    const dim3 block(256);                                                                   \
    if (fp8) {                                                                               \
      switch (mode) {                                                                        \
        case kStore16: HKX_TILE4_STAGED(BM, BN, true, kStore16) break;                                \
        case kStore8: HKX_TILE4_STAGED(BM, BN, true, kStore8) break;                         \
        case kStoreF32: hipLaunchKernelGGL((tile4_kernel<BM, BN, true, kStoreF32>), grid, block, 0, s, a); break; \
        default: return hipErrorInvalidValue;                                                \
      }                                                                                      \
    } else {                                                                                 \
      switch (mode) {                                                                        \
        case kStore16: HKX_TILE4_STAGED(BM, BN, false, kStore16) break;                               \
        case kStore8: HKX_TILE4_STAGED(BM, BN, false, kStore8) break;                        \
        case kStoreF32: hipLaunchKernelGGL((tile4_kernel<BM, BN, false, kStoreF32>), grid, block, 0, s, a); break; \
        case kPair16: hipLaunchKernelGGL((tile4_kernel<BM, BN, false, kPair16>), grid, block, 0, s, a); break;     \
        case kPairWs: hipLaunchKernelGGL((tile4_kernel<BM, BN, false, kPairWs>), grid, block, 0, s, a); break;     \
        default: return hipErrorInvalidValue;                                                \
      }                                                                                      \
    }                                                                                        \
    return hipGetLastError();                                                                \
  }

}  // namespace hkx
