// The ping-pong MFMA GEMM for gfx950: 8 waves, two a SIMD, that take turns at the matrix
// cores. A 256 x 256 tile of C; each wave owns a 64 x 128 block of it (2 x 4 fragments
// of 32 x 32, 128 fp32 accumulators a lane).
//
// Why: with one wave a SIMD every wait of that wave -- for an LDS read, for a fill, at a
// barrier -- idles the SIMD's matrix core. Here the waves of a SIMD are in two groups
// (waves 0-3 and 4-7; a SIMD holds wave w and w + 4) that run the same program one phase
// apart: while one group issues a phase's MFMAs (at raised priority), the other reads the
// next phase's fragments from LDS and issues fills, and one barrier of all 8 waves ends
// every phase. The matrix core only waits for the barrier's turnaround.
//
// * K advances in 64-byte half-stages (32 bf16 or 64 fp8 of every row). One phase of a
//   wave is one half-stage: 2 x 4 fragments x 2 k-steps of v_mfma_f32_32x32x16_bf16, or
//   2 x 4 x 1 of v_mfma_scale_f32_32x32x64_f8f6f4 -- 512 cycles of matrix core either way.
// * LDS: a ring of four half-stage buffers, each 256 A rows and 256 B rows of 64 bytes
//   (32 KB). Buffer u % 4 is refilled with half-stage u + 4 once both groups have read
//   half-stage u, so a fill has five phases to land.
// * Fills: direct global -> LDS buffer loads (`buffer_load_dwordx4 ... lds`), 16 bytes a
//   lane; each wave fills 4 x 16 rows of every half-stage. Rows are stored with their
//   four 16-byte chunks XOR-swizzled by bits 3 and 4 of the row (chunk c at
//   c ^ (r4 | 2 r3)), which makes the fragment reads -- 32 rows with one chunk each, or 16
//   rows with four -- run at the LDS's full ds_read_b128 rate (measured over all 1024
//   swizzles that XOR row-bit parities into the chunk: this one reads at 480 GB/s a CU,
//   as fast as any; no swizzle reads at a third of that, a swizzle by bits 1-3 at 60%).
//   The swizzle is applied on the global side: lane l fetches the logical chunk that
//   belongs at its LDS slot.
// * MFMA operands are swapped (B's fragment first) so a lane ends with runs of four
//   consecutive columns of one row of C, which the epilogue and the store want.
//
// The tile order, the epilogue (applied in registers, converted once, staged through LDS,
// stored as 16-byte pieces of rows) and the store modes are those of hkx_tile4.hpp.
#pragma once

#include "hkx_tile.hpp"

namespace hkx {


template <bool FP8, int MODE, int ACT = -1, bool MF16 = false>
__global__ void __launch_bounds__(512, 1) pp_kernel(const TileArgs p) {
  constexpr int BM = 256, BN = 256;
  constexpr int FR = MF16 ? 16 : 32;              // fragment edge
  constexpr int FM = 64 / FR, FN = 128 / FR;      // fragments of a wave: 64 x 128
  constexpr int HS = 32 * 1024;  // one half-stage buffer: 512 rows x 64 bytes
  constexpr int NBUF = 4;
  constexpr bool PAIR = (MODE == kPair16 || MODE == kPairWs);
  constexpr int OB = (MODE == kStore8) ? 1 : 2;
  constexpr int OUTW = PAIR ? BN / 2 : BN;
  constexpr bool STAGED = (MODE == kStore16 || MODE == kStore8 || MODE == kPair16);
  constexpr int RS = OUTW * OB + 16;
  constexpr int STAGING = STAGED ? BM * RS : 0;
  constexpr int ROWOP = (NBUF * HS > STAGING) ? NBUF * HS : STAGING;
  constexpr int SMEM = ROWOP + 2 * BN * 4;
  static_assert(SMEM <= 160 * 1024, "LDS");
  static_assert(!MF16 || (!FP8 && !PAIR), "16 x 16 fragments: bf16, unpaired");
  using Frag = typename std::conditional<FP8, i32x8, bf16x8>::type;

  __shared__ __attribute__((aligned(16))) uint8_t smem[SMEM];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2;  // the ping-pong group
  const int wm = (wave >> 1) & 1, wn = wave & 1;
  const int row0 = grp * 128 + wm * 64;  // the wave's block of the tile
  const int col0 = wn * 128;

  // Tiles: one a workgroup, or -- a grid smaller than the tile count -- every gridDim.x-th
  // in turn (the stores of one tile drain while the next one's first fills are issued).
  const int total = p.tiles_m * p.tiles_n;
  for (int vt = blockIdx.x; vt < total; vt += gridDim.x) {
    // ---- which tile: XCD-chunked renumbering, then a grouped raster
    int L = vt;
    if ((total & 7) == 0) L = (L & 7) * (total >> 3) + (L >> 3);
    const int per = p.wgm * p.tiles_n;
    const int gi = L / per;
    const int first = gi * p.wgm;
    const int gm = min(p.tiles_m - first, p.wgm);
    const int in = L - gi * per;
    const int tm = first + in % gm, tn = in / gm;
    const int m0 = tm * BM;
    const int n0 = tn * OUTW;

    const int split = blockIdx.y;
    const int u0 = 2 * split * p.kt_split;                       // first half-stage
    const int nu = 2 * min(p.kt_split, p.kt_total - split * p.kt_split);  // half-stages

    // ---- fills: wave w's instruction i covers buffer rows 16 (w + 8 i) + [0, 16); lane l
    // writes bytes 16 l of that 1 KB: row + (l >> 2), physical chunk l & 3
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a, p.a_bytes);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.b, p.b_bytes);
    uint32_t voff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * (wave + 8 * i) + (lane >> 2);
      const uint32_t ch = (uint32_t)(((lane & 3) ^ swz4(r)) << 4);
      if (i < 2) {
        voff[i] = (uint32_t)(m0 + r) * p.lda_b + ch;
      } else {
        const int v = r - BM;
        int brow;
        if constexpr (PAIR) {
          const int fv = v >> 5;
          brow = n0 + (fv >> 1) * 32 + (v & 31) + ((fv & 1) ? p.pair_off : 0);
        } else {
          brow = n0 + v;
        }
        voff[i] = (uint32_t)brow * p.ldb_b + ch;
      }
    }
    // half-stage u (clamped to the last one: fills past the end are kept, so the wait
    // counts stay uniform, and never read)
    auto fill = [&](int u) {
      const int uc = min(u, nu - 1);
      const uint32_t so = __builtin_amdgcn_readfirstlane((uint32_t)(u0 + uc) * 64u);
      uint8_t* base = smem + (u & (NBUF - 1)) * HS + wave * 1024;
#pragma unroll
      for (int i = 0; i < 4; ++i) buf_load16_lds(i < 2 ? ra : rb, base + i * 8192, voff[i], so);
    };

    // ---- fragment reads: lane l reads row l & 31 of a fragment; bf16 k-step q takes
    // logical chunk 2 q + (l >> 5), fp8 chunks 2 (l >> 5) and + 1
    // (16 x 16 fragments: lane l reads row l & 15, chunk l >> 4 -- one k-step of 32)
    // The swizzle takes bits 3-4 of the row: a 32-row fragment's lane supplies them, a
    // 16-row fragment's bit 4 is the fragment's parity (rdo[1] serves the odd ones).
    const int rf = lane & (FR - 1), h = lane / FR;
    uint32_t rdo[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int lc = MF16 ? h : (FP8 ? (2 * h + q) : (2 * q + h));
      const int sw = swz4(MF16 ? rf + 16 * q : rf);
      rdo[q] = rf * 64 + ((lc ^ sw) << 4);
    }
    constexpr int FB = FR * 64;  // bytes of a fragment's rows
    const int a_off = row0 * 64, b_off = (BM + col0) * 64;

    Frag af[2][FM], bfr[2][FN];  // 32 x 32 bf16: [k-step]; fp8 and 16 x 16: [0] only
    auto read_frags = [&](int u) {
      const uint8_t* s = smem + (u & (NBUF - 1)) * HS;
      if constexpr (FP8) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const i32x4 lo = *(const i32x4*)(s + b_off + j * 2048 + rdo[0]);
          const i32x4 hi = *(const i32x4*)(s + b_off + j * 2048 + rdo[1]);
          bfr[0][j] = i32x8{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        }
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          const i32x4 lo = *(const i32x4*)(s + a_off + i * 2048 + rdo[0]);
          const i32x4 hi = *(const i32x4*)(s + a_off + i * 2048 + rdo[1]);
          af[0][i] = i32x8{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        }
      } else {
#pragma unroll
        for (int q = 0; q < (MF16 ? 1 : 2); ++q) {
#pragma unroll
          for (int j = 0; j < FN; ++j)
            bfr[q][j] = *(const bf16x8*)(s + b_off + j * FB + rdo[MF16 ? (j & 1) : q]);
#pragma unroll
          for (int i = 0; i < FM; ++i)
            af[q][i] = *(const bf16x8*)(s + a_off + i * FB + rdo[MF16 ? (i & 1) : q]);
        }
      }
    };

    using Acc = typename std::conditional<MF16, f32x4, f32x16>::type;
    Acc acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = Acc{};

    auto mma = [&]() {
      if constexpr (FP8) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bfr[0][j], af[0][i],
                                                                       acc[i][j], 0, 0, 0, 0, 0, 0);
      } else if constexpr (MF16) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bfr[0][j], af[0][i], acc[i][j], 0, 0, 0);
      } else {
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
          for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[q][j], af[q][i], acc[i][j],
                                                                  0, 0, 0);
      }
    };

    // ---- the epilogue's operands, loaded now so their latency hides under the K loop
    const Fused& e = p.ep;
    const bool fused = !PAIR && e.form == HKX_EP_FUSED;
    float* rowop = (float*)(smem + ROWOP);  // [0, BN): row scale, [BN, 2 BN): row add
    if (tid < BN) {
      const int n = n0 + tid;
      const bool ok = fused && n < p.N;
      rowop[tid] = (ok && e.rs.p) ? ld1(e.rs.p, e.rs.dt, e.rs.ld ? n : 0) : 1.0f;
      rowop[BN + tid] = (ok && e.ra.p) ? ld1(e.ra.p, e.ra.dt, e.ra.ld ? n : 0) : 0.0f;
    }
    float csv[FM];
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int m = m0 + row0 + FR * i + rf;
      csv[i] = (fused && e.cs.p && m < p.M) ? ld_col(e.cs, m) * e.cmul : e.cmul;
    }

    // ---- the K loop. Phase boundaries are barriers of all 8 waves; group 1 starts one
    // barrier late and group 0 ends with one extra, so they alternate:
    //   phase 2u + grp: read half-stage u into registers, fill half-stage u + 3
    //   phase 2u + grp + 1: the MFMAs of half-stage u
    // Before every barrier a wave waits for its reads (the LDS operations) and for its
    // fills but the last 8 (the two newest half-stages): the fill of half-stage v was issued
    // in phase 2 (v - 3) + grp and must have landed at the barrier before phase 2 v, where
    // group 0 reads it.
    fill(0);
    fill(1);
    fill(2);
    __builtin_amdgcn_s_waitcnt(0x3f78);  // vmcnt(8): this wave's half-stage 0 landed
    __builtin_amdgcn_s_barrier();
    if (grp == 1) __builtin_amdgcn_s_barrier();
    for (int u = 0; u < nu; ++u) {
      // memory phase
      read_frags(u);
      fill(u + 3);
      __builtin_amdgcn_s_waitcnt(0x3078);  // lgkmcnt(0) vmcnt(8)
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      // matrix phase
      __builtin_amdgcn_s_setprio(1);
      mma();
      __builtin_amdgcn_s_setprio(0);
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(0x3f78);  // vmcnt(8)
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
    }
    if (grp == 0) __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_s_waitcnt(0x3f70);  // the last (unused) fills land before LDS is reused

    // ---- the store. Lane l holds, for fragment (i, j) and run g, C[m][n .. n + 3] with
    // m = row0 + FR i + (l % FR), n = col0 + FR j + 8 g + 4 (l / FR) -- four runs g of a
    // 32 x 32 fragment, one of a 16 x 16.
    constexpr int NG = MF16 ? 1 : 4;
    const int mw = row0 + rf;
    const int nw = col0 + 4 * h;
    auto run = [&](int i, int j, int g) -> f32x4 {
      if constexpr (MF16) return acc[i][j];
      else return f32x4{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
    };
    if constexpr (MODE == kStoreF32 || MODE == kPairWs) {
      float* out = (float*)p.c + (int64_t)split * p.split_stride;
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int m = m0 + mw + FR * i;
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int g = 0; g < NG; ++g) {
            __builtin_amdgcn_sched_barrier(0);
            f32x4 v = run(i, j, g);
            if constexpr (MODE == kStoreF32) {
              const int n = n0 + nw + FR * j + 8 * g;
              if (m < p.M && n < p.N) {
                if (fused) {
                  const int nl = nw + FR * j + 8 * g;
                  v = v * (*(const f32x4*)(rowop + nl) * csv[i]) + *(const f32x4*)(rowop + BN + nl);
                  if (e.ta.p) v += ld_tile(e.ta, m, n);
                  v = act4(e.act, v + e.cadd);
                }
                *(f32x4*)(out + (int64_t)m * p.ldc + n) = v;
              }
            } else {
              const int fv = wn * FN + j;
              const int oc = n0 + (fv >> 1) * 32 + 8 * g + 4 * h;
              if (m < p.M && oc < p.N)
                *(f32x4*)(out + (int64_t)m * p.ldc + oc + ((fv & 1) ? p.N : 0)) = v;
            }
          }
      }
    } else {
      __syncthreads();  // the ring is reused as the staging tile
      auto group = [&](int i, int j, int g, bool tile_op) {
        const int ml = mw + FR * i;
        f32x4 v = run(i, j, g);
        int cl;
        if constexpr (MODE == kPair16) {
          const f32x4 u = run(i, j + 1, g);
          v = silu_mul4(v, u);
          cl = ((wn * FN + j) >> 1) * 32 + 8 * g + 4 * h;
        } else {
          cl = nw + FR * j + 8 * g;
          v = v * (*(const f32x4*)(rowop + cl) * csv[i]) + *(const f32x4*)(rowop + BN + cl);
          if (tile_op) {
            const int m = min(m0 + ml, p.M - 1), n = min(n0 + cl, p.N - 4);
            v += ld_tile(e.ta, m, n);
          }
          v = act4c<ACT>(e.act, v + e.cadd);
        }
        const u32x2 w = pack4<OB>(p.c_dt, v);
        if constexpr (OB == 2)
          *(u32x2*)(smem + ml * RS + cl * 2) = w;
        else
          *(uint32_t*)(smem + ml * RS + cl) = w.x;
      };
      const bool tile_op = fused && e.ta.p;
#pragma unroll
      for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          if (PAIR && (j & 1)) continue;
          __builtin_amdgcn_sched_barrier(0);
          if (tile_op) {
#pragma unroll
            for (int g = 0; g < NG; ++g) group(i, j, g, true);
          } else {
#pragma unroll
            for (int g = 0; g < NG; ++g) group(i, j, g, false);
          }
        }
      }
      __syncthreads();
      constexpr int CPR = OUTW * OB / 16;
      constexpr int EPC = 16 / OB;
#pragma unroll 4
      for (int q = tid; q < BM * CPR; q += 512) {
        const int row = q / CPR, ch = q - row * CPR;
        const int gmr = m0 + row, gn = n0 + ch * EPC;
        if (gmr < p.M && gn < p.N) {
          const uint8_t* src = smem + row * RS + ch * 16;
          uint8_t* dst = (uint8_t*)p.c + ((int64_t)gmr * p.ldc + gn) * OB;
          if (p.c_aligned && gn + EPC <= p.N) {
            *(i32x4*)dst = *(const i32x4*)src;
          } else {
            const int cnt = min(EPC, p.N - gn) * OB;
            for (int x = 0; x < cnt; ++x) dst[x] = src[x];
          }
        }
      }
    }
    __syncthreads();  // LDS is reused by the next tile
  }
}

}  // namespace hkx
