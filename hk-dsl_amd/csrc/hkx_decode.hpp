// The decode GEMM: C (M <= 32, N) = epilogue(X . W^T) with W streamed from HBM once.
//
// Replaces python/hk/ops/decode_gemm.py:37-180 (and the weight-streaming dp32x48nt
// blocks the reference's table routes M <= 32 to, python/hk/ops/gemm_cdna_dp.py). At
// these M the arithmetic is free and the whole cost is reading W, so:
//
// * no LDS staging: each lane loads W straight into its MFMA operand registers, 16
//   bytes at a time, four loads covering 256 contiguous bytes of 16 rows per wave;
// * a workgroup owns 16 * FN rows of W and NW waves split K between them in 128-element
//   groups (wave w takes groups w, w + NW, ...), U groups in flight per wave;
// * X (M x K, a few KB to 256 KB) is read through the caches as the other MFMA operand;
//   its rows past M read 0 through the buffer bound;
// * v_mfma_f32_16x16x32_bf16 with W's fragment first, so a lane ends with C[m][n..n+3];
// * the NW partial sums meet in LDS and one wave per fragment applies the epilogue
//   and stores -- or, split over K across workgroups (blockIdx.y), stores fp32 shares
//   that the reduction kernel sums in order and finishes.
#pragma once

#include "hkx_device.hpp"

namespace hkx {

struct DecodeArgs {
  const void* a;  // X (M, K)
  const void* b;  // W (N, K) -- (2N, K) paired
  void* c;        // C, or the fp32 shares
  uint32_t a_bytes, b_bytes;
  uint32_t lda_b, ldb_b;
  int64_t ldc;
  int64_t split_stride;
  int32_t M, N;
  int32_t g_total;  // 128-element K groups in all
  int32_t g_split;  // per split
  int32_t pair_off;
  int32_t c_dt;
  Fused ep;
};

constexpr int kDecOut = 0;     // C with the fused epilogue
constexpr int kDecWs = 1;      // fp32 shares, (M, N) per split
constexpr int kDecPair = 2;    // silu(gate) * up into C
constexpr int kDecPairWs = 3;  // gate and up fp32 shares, (M, 2N) per split

template <int NW, int FN, int MF, int U, int MODE>
__global__ void __launch_bounds__(NW * 64) decode_kernel(const DecodeArgs p) {
  constexpr bool PAIR = (MODE == kDecPair || MODE == kDecPairWs);
  constexpr int NF = MF * FN;
  static_assert(!PAIR || FN % 2 == 0, "gate/up fragment pairs");
  __shared__ f32x4 red[NW][NF][64];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rf = lane & 15, kq = lane >> 4;
  const int outw = PAIR ? 8 * FN : 16 * FN;  // C columns of this workgroup
  const int n0 = blockIdx.x * outw;

  const int split = blockIdx.y;
  const int g0 = split * p.g_split;
  const int ng = min(p.g_split, p.g_total - g0);

  const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.b, p.b_bytes);
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.a, p.a_bytes);
  uint32_t vw[FN], vx[MF];
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    int row;
    if constexpr (PAIR)
      row = n0 + (j >> 1) * 16 + rf + ((j & 1) ? p.pair_off : 0);
    else
      row = n0 + j * 16 + rf;
    vw[j] = (uint32_t)row * p.ldb_b + kq * 16;
  }
#pragma unroll
  for (int i = 0; i < MF; ++i) vx[i] = (uint32_t)(i * 16 + rf) * p.lda_b + kq * 16;

  f32x4 acc[MF][FN];
#pragma unroll
  for (int i = 0; i < MF; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int base = wave; base < ng; base += NW * U) {
    i32x4 w[U][FN][4], x[U][MF][4];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int g = base + u * NW;
      if (g < ng) {
        const uint32_t so = (uint32_t)(g0 + g) * 256u;
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int s = 0; s < 4; ++s) w[u][j][s] = buf_load16(rw, vw[j] + s * 64, so);
#pragma unroll
        for (int i = 0; i < MF; ++i)
#pragma unroll
          for (int s = 0; s < 4; ++s) x[u][i][s] = buf_load16(rx, vx[i] + s * 64, so);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (base + u * NW < ng) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
          for (int i = 0; i < MF; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                  __builtin_bit_cast(bf16x8, w[u][j][s]), __builtin_bit_cast(bf16x8, x[u][i][s]),
                  acc[i][j], 0, 0, 0);
      }
    }
  }

#pragma unroll
  for (int i = 0; i < MF; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) red[wave][i * FN + j][lane] = acc[i][j];
  __syncthreads();

  if constexpr (!PAIR) {
    for (int f = wave; f < NF; f += NW) {
      f32x4 s = red[0][f][lane];
#pragma unroll
      for (int w2 = 1; w2 < NW; ++w2) s += red[w2][f][lane];
      const int i = f / FN, j = f - i * FN;
      const int m = i * 16 + rf, n = n0 + j * 16 + 4 * kq;
      if (m < p.M && n < p.N) {
        if constexpr (MODE == kDecWs) {
          *(f32x4*)((float*)p.c + (int64_t)split * p.split_stride + (int64_t)m * p.ldc + n) = s;
        } else {
          store4(p.c, p.c_dt, (int64_t)m * p.ldc + n, fused_apply(p.ep, s, m, n, true));
        }
      }
    }
  } else {
    constexpr int NP = MF * FN / 2;
    for (int f = wave; f < NP; f += NW) {
      const int i = f / (FN / 2), jp = f - i * (FN / 2);
      const int fg = i * FN + 2 * jp;
      f32x4 g = red[0][fg][lane], u = red[0][fg + 1][lane];
#pragma unroll
      for (int w2 = 1; w2 < NW; ++w2) {
        g += red[w2][fg][lane];
        u += red[w2][fg + 1][lane];
      }
      const int m = i * 16 + rf, n = n0 + jp * 16 + 4 * kq;
      if (m < p.M && n < p.N) {
        if constexpr (MODE == kDecPairWs) {
          float* out = (float*)p.c + (int64_t)split * p.split_stride + (int64_t)m * p.ldc;
          *(f32x4*)(out + n) = g;
          *(f32x4*)(out + p.N + n) = u;
        } else {
          store4(p.c, p.c_dt, (int64_t)m * p.ldc + n, silu_mul4(g, u));
        }
      }
    }
  }
}

}  // namespace hkx
