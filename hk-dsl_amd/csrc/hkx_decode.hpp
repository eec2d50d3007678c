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

// s_waitcnt vmcnt(n) (gfx9 encoding: bits 3:0 and 15:14; expcnt and lgkmcnt left alone)
constexpr int wait_vm_dec(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

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


// The streaming decode GEMM: one workgroup a CU walks the 16-row blocks of W (every
// gridDim.x-th), for M <= 16 (one 16-token fragment), unpaired, no split, K a multiple of
// 1024 up to 1024 CPB.
//
// * W goes HBM -> LDS by buffer loads (`buffer_load_dwordx4 ... lds`), each instruction 1 KB
//   of one row, contiguous -- the access a pure streaming read reaches HBM's ceiling with --
//   in chunks of 16 rows x 1024 K (32 KB) through a ring of four: chunk q + 3 is in flight
//   while chunk q is multiplied. A row's 128 16-byte pieces are stored XOR-swizzled by the
//   row (piece c at c ^ (r % 16)), applied on the global side, so the MFMA fragment reads
//   (16 rows, one piece each) are conflict-free.
// * X is the same for every block: wave w owns the 128-element group w of every chunk, and
//   loads its share of X (CPB groups of 16 rows) into registers once.
// * v_mfma_f32_16x16x32_bf16 with W's fragment first; the 8 waves' partial sums of a block
//   meet in LDS (double-buffered by block parity), and wave 0 sums, applies the epilogue and
//   stores after the next chunk's barrier, under the other waves' MFMAs.
template <int CPB>
__global__ void __launch_bounds__(512) stream_kernel(const DecodeArgs p) {
  constexpr int NW = 8;
  constexpr int CH = 16 * 2048;  // a chunk: 16 rows x 2 KB
  constexpr int NR = 4;          // ring slots
  constexpr int RED = NR * CH;   // then the partial sums: [block parity][wave][lane], 16 B each
  __shared__ __attribute__((aligned(16))) uint8_t ring[RED + 2 * NW * 64 * 16];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rf = lane & 15, kq = lane >> 4;
  const int nb = (p.N + 15) / 16;
  const int G = gridDim.x;
  if ((int)blockIdx.x >= nb) return;
  const int my_blocks = (nb - (int)blockIdx.x + G - 1) / G;
  const int nq = my_blocks * CPB;  // chunks of this workgroup

  const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.b, p.b_bytes);
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.a, p.a_bytes);
  auto ds_read16 = [&](uint32_t off) { return *(const i32x4*)(ring + off); };
  auto ds_write16 = [&](uint32_t off, i32x4 v) { *(i32x4*)(ring + off) = v; };
  // Barriers are bare s_barrier with the waits written out: __syncthreads() would also wait
  // for every fill in flight (its fence orders the LDS-DMA writes too).

  // fills: wave w moves rows 2 w and 2 w + 1 of a chunk, 1 KB (half a row) an instruction;
  // lane l's 16 bytes land at piece 64 h + l of row r, which holds global piece
  // (64 h + l) ^ (r % 16) of the row's 2 KB. The per-lane part of the address is
  // loop-invariant; the block and the chunk go in the scalar offset.
  uint32_t fv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 2 * wave + (i >> 1), h = i & 1;
    fv[i] = (uint32_t)r * p.ldb_b + (uint32_t)(((64 * h + lane) ^ r) << 4);
  }
  auto fill = [&](int q) {
    q = min(q, nq - 1);  // past the end: fetch the last chunk again (nothing reads it)
    const int bi = (int)blockIdx.x + (q / CPB) * G, kc = q % CPB;
    const uint32_t so = __builtin_amdgcn_readfirstlane((uint32_t)bi * 16u * p.ldb_b + (uint32_t)kc * 2048u);
    uint8_t* slot = ring + (q & (NR - 1)) * CH;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 2 * wave + (i >> 1), h = i & 1;
      buf_load16_lds(rw, slot + r * 2048 + h * 1024, fv[i], so);
    }
  };
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  // the MFMAs of this wave's group of chunk q (its slot landed and visible)
  auto mma = [&](int q, const i32x4 (&xc)[4]) {
    const uint32_t slot = (uint32_t)(q & (NR - 1)) * CH;
    i32x4 w[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int piece = 16 * wave + kq + 4 * s;  // global piece of the row in this chunk
      w[s] = ds_read16(slot + rf * 2048 + ((piece ^ rf) << 4));
    }
#pragma unroll
    for (int s = 0; s < 4; ++s)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, w[s]),
                                                    __builtin_bit_cast(bf16x8, xc[s]), acc, 0, 0, 0);
  };
  // block j of this workgroup: its partial sums are at parity j & 1
  auto finish = [&](int j) {
    const int bi = (int)blockIdx.x + j * G;
    i32x4 part[NW];
#pragma unroll
    for (int w2 = 0; w2 < NW; ++w2) part[w2] = ds_read16(RED + (((j & 1) * NW + w2) * 64 + lane) * 16);
    f32x4 sum = __builtin_bit_cast(f32x4, part[0]);
#pragma unroll
    for (int w2 = 1; w2 < NW; ++w2) sum += __builtin_bit_cast(f32x4, part[w2]);
    const int m = rf, n = bi * 16 + 4 * kq;
    if (m < p.M && n < p.N) store4(p.c, p.c_dt, (int64_t)m * p.ldc + n, fused_apply(p.ep, sum, m, n, true));
  };

  // X first: lane l holds row l % 16, 16 bytes at 16 (l / 16) + 64 s of K group
  // 8 c + wave (chunk c's group of this wave), for k-steps s; then chunks 0-2 in flight.
  // Waiting for all but the 12 newest loads leaves the chunks in flight and X landed.
  i32x4 x[CPB][4];
#pragma unroll
  for (int c = 0; c < CPB; ++c)
#pragma unroll
    for (int s = 0; s < 4; ++s)
      x[c][s] = buf_load16(rx, (uint32_t)rf * p.lda_b + kq * 16 + s * 64, (uint32_t)(8 * c + wave) * 256u);
  fill(0);
  fill(1);
  fill(2);
  __builtin_amdgcn_s_waitcnt(wait_vm_dec(12));
  for (int j = 0; j < my_blocks; ++j) {
#pragma unroll
    for (int c = 0; c < CPB; ++c) {
      const int q = j * CPB + c;
      // chunk q landed (all but this wave's 8 newest loads: chunks q + 1, q + 2) and every
      // wave is done with chunk q - 1, whose slot the fill of q + 3 takes
      __builtin_amdgcn_s_waitcnt(wait_vm_dec(8) & ~(15 << 8));  // and lgkmcnt(0)
      __builtin_amdgcn_s_barrier();
      fill(q + 3);
      if (c == 0 && j > 0 && wave == 0) finish(j - 1);
      mma(q, x[c]);
    }
    ds_write16(RED + (((j & 1) * NW + wave) * 64 + lane) * 16, __builtin_bit_cast(i32x4, acc));
    acc = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the last partial sums written
  __builtin_amdgcn_s_barrier();
  if (wave == 0) finish(my_blocks - 1);
  __builtin_amdgcn_s_waitcnt(wait_vm_dec(0));  // no fill lands in LDS after the exit
}

}  // namespace hkx
