// The large-tile MFMA GEMM for gfx950: 4 waves (2 x 2), each a (BM/2) x (BN/2) sub-tile
// of 32 x 32 fragments -- 128 x 128 at the 256 x 256 tile, 256 fp32 accumulators a lane,
// held in the AGPR half of the 512-entry register file (one wave per SIMD).
//
// Why this shape: the LDS traffic of the K loop is sum over waves of (TM + TN) x 128
// bytes per 128-byte K stage, so one wave per SIMD with the biggest wave tile halves it
// against 8 waves of 128 x 64 (128 KB against 196 KB per stage, beside 64 KB of fills).
//
// * Fills: direct global -> LDS buffer loads (`buffer_load_dwordx4 ... lds`): the data
//   never touches a VGPR. Wave w's i-th load fills bytes [1024 w + 4096 i, +1024) of the
//   stage; lane l's 16 bytes land at +16 l, so the XOR swizzle is chosen on the global
//   side (lane l fetches logical chunk (l & 7) ^ swz(row & 15) of its row).
// * NST LDS stages, as many as fit up to four: four at BN = 128 (4 x 24 or 32 KB), three
//   at 128 x 256 and 64 x 256 (3 x 48 or 40 KB), two at 256 x 256.
//   The fills of tile kt + NST go into the stage iteration kt read, begun right after its
//   one barrier and spread under the next iteration's k-steps; with three stages they have
//   one iteration more to land (a wave a SIMD has nothing else to hide their latency with).
// * Fragment reads are software-pipelined one k-step ahead (two register sets), and the
//   reads of the next stage's first k-step are issued under the last k-step's MFMAs.
// * MFMA: v_mfma_f32_32x32x16_bf16 / v_mfma_f32_32x32x64_f8f6f4 (fp8 e4m3), B's fragment
//   first, so a lane ends with runs of four consecutive columns of one row of C.
//
// Everything else -- operands, ragged edges through the buffer bounds, the XCD-aware
// block order, the stores and the epilogue -- is as in the 8-wave kernel (hkx_tile.hpp).
#pragma once

#include "hkx_tile.hpp"

namespace hkx {

typedef float f32x16 __attribute__((ext_vector_type(16)));

// s_waitcnt vmcnt(n) lgkmcnt(0) (gfx9 encoding: vmcnt bits 3:0 and 15:14)
constexpr int tile4_vmcnt_lgkm0(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4); }

template <int BM, int BN, bool FP8, int MODE, int ACT = -1>
__global__ void __launch_bounds__(256, 1) tile4_kernel(const TileArgs p) {
  constexpr int TM = BM / 2, TN = BN / 2;
  constexpr int FM = TM / 32, FN = TN / 32;
  constexpr int ROWS = BM + BN;
  constexpr int NCH = ROWS / 32;  // 16-byte chunks a thread fills per stage
  constexpr int NA = BM / 32;     // of which from A
  constexpr int STAGE = ROWS * 128;
  constexpr int KS = FP8 ? 2 : 4;  // MFMA k-steps per stage
  constexpr bool PAIR = (MODE == kPair16 || MODE == kPairWs);
  constexpr int OB = (MODE == kStore8) ? 1 : 2;
  constexpr int OUTW = PAIR ? BN / 2 : BN;  // C columns a tile covers
  constexpr bool STAGED = (MODE == kStore16 || MODE == kStore8 || MODE == kPair16);
  constexpr int RS = OUTW * OB + 16;  // staging row stride, bytes
  constexpr int STAGING = STAGED ? BM * RS : 0;
  // LDS stages: as many as fit beside the row operands, up to four
  constexpr int NST = 4 * STAGE + 2 * BN * 4 <= 160 * 1024   ? 4
                      : 3 * STAGE + 2 * BN * 4 <= 160 * 1024 ? 3
                                                             : 2;
  constexpr int ROWOP = (NST * STAGE > STAGING) ? NST * STAGE : STAGING;  // + the row operands
  constexpr int SMEM = ROWOP + 2 * BN * 4;
  static_assert(FM >= 1 && FN >= 1 && BM % 64 == 0 && (BN == 256 || BN == 128), "tiling");
  static_assert(!PAIR || FN % 2 == 0, "the paired form needs gate/up fragment pairs");
  static_assert(SMEM <= 160 * 1024, "LDS");
  using Frag = typename std::conditional<FP8, i32x8, bf16x8>::type;

  // (+16 bytes: the split finish's flag. A second __shared__ object would make the compiler
  // wait for every LDS-DMA fill before each LDS read: it could no longer tell the fills'
  // destination from the flag, and the main loop ran 2x slower)
  __shared__ __attribute__((aligned(16))) uint8_t smem[SMEM + 16];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  // ---- which tile
  const int total = p.tiles_m * p.tiles_n;
  int L = blockIdx.x;
  if ((total & 7) == 0) L = (L & 7) * (total >> 3) + (L >> 3);
  const int per = p.wgm * p.tiles_n;
  const int grp = L / per;
  const int first = grp * p.wgm;
  const int gm = min(p.tiles_m - first, p.wgm);
  const int in = L - grp * per;
  const int tm = first + in % gm, tn = in / gm;
  const int m0 = tm * BM;
  const int n0 = tn * OUTW;

  const int split = blockIdx.y;
  const int kt0 = split * p.kt_split;
  const int nkt = min(p.kt_split, p.kt_total - kt0);

  // ---- fills: chunk i of thread t is stage row (t >> 3) + 32 i, physical chunk t & 7
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a, p.a_bytes);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.b, p.b_bytes);
  const int lrow = tid >> 3;
  const uint32_t lch16 = (uint32_t)(((tid & 7) ^ swz(lrow & 15)) << 4);
  uint32_t voff[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int r = lrow + 32 * i;
    if (i < NA) {
      voff[i] = (uint32_t)(m0 + r) * p.lda_b + lch16;
    } else {
      const int v = r - BM;
      int brow;
      if constexpr (PAIR) {
        const int fv = v >> 5;
        brow = n0 + (fv >> 1) * 32 + (v & 31) + ((fv & 1) ? p.pair_off : 0);
      } else {
        brow = n0 + v;
      }
      voff[i] = (uint32_t)brow * p.ldb_b + lch16;
    }
  }
  // Fills chunks [lo, hi) of a stage: a stage's fills are spread over three k-steps.
  auto fill_part = [&](int kt, int s, int lo, int hi) {
    const uint32_t so = __builtin_amdgcn_readfirstlane((uint32_t)(kt0 + kt) * 128u);
    uint8_t* base = smem + s * STAGE + wave * 1024;
#pragma unroll
    for (int i = 0; i < NCH; ++i)
      if (i >= lo && i < hi) buf_load16_lds(i < NA ? ra : rb, base + i * 4096, voff[i], so);
  };

  // ---- fragment reads: lane l reads row l & 31 of a fragment, k-half l >> 5
  const int rf = lane & 31, h = lane >> 5;
  const int sw = swz(rf & 15);
  uint32_t rdo[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    // bf16: k-step q reads logical chunk 2q + h. fp8: k-step q / 2 reads chunks
    // 4 (q / 2) + 2h and + 1, as halves q & 1.
    const int lc = FP8 ? (4 * (q >> 1) + 2 * h + (q & 1)) : (2 * q + h);
    rdo[q] = rf * 128 + ((lc ^ sw) << 4);
  }
  const int a_base = wm * TM * 128;
  const int b_base = (BM + wn * TN) * 128;

  auto read_frags = [&](int s, int ks, Frag (&af)[FM], Frag (&bf)[FN]) {
    const uint8_t* sa = smem + s * STAGE + a_base;
    const uint8_t* sb = smem + s * STAGE + b_base;
    if constexpr (FP8) {
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        i32x4 lo = *(const i32x4*)(sb + j * 4096 + rdo[2 * ks]);
        i32x4 hi = *(const i32x4*)(sb + j * 4096 + rdo[2 * ks + 1]);
        bf[j] = i32x8{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
      }
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        i32x4 lo = *(const i32x4*)(sa + i * 4096 + rdo[2 * ks]);
        i32x4 hi = *(const i32x4*)(sa + i * 4096 + rdo[2 * ks + 1]);
        af[i] = i32x8{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
      }
    } else {
#pragma unroll
      for (int j = 0; j < FN; ++j) bf[j] = *(const bf16x8*)(sb + j * 4096 + rdo[ks]);
#pragma unroll
      for (int i = 0; i < FM; ++i) af[i] = *(const bf16x8*)(sa + i * 4096 + rdo[ks]);
    }
  };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x16{};

  auto mma = [&](const Frag (&af)[FM], const Frag (&bf)[FN]) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        if constexpr (FP8)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bf[j], af[i], acc[i][j], 0,
                                                                     0, 0, 0, 0, 0);
        else
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bf[j], af[i], acc[i][j], 0, 0, 0);
      }
  };

  Frag a0[FM], b0[FN], a1[FM], b1[FN];

  // ---- the epilogue's operands, loaded now, so their latency hides under the K loop:
  // the row operands (one value per column of the tile) into LDS, fp32, thread t
  // column n0 + t; the column scale for each of this lane's rows into a register.
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
    const int m = m0 + wm * TM + 32 * i + (lane & 31);
    csv[i] = (fused && e.cs.p && m < p.M) ? ld_col(e.cs, m) * e.cmul : e.cmul;
  }

  // ---- prologue: stages 0 .. NST - 2 in flight and the first fills of stage NST - 1 (as
  // the barrier before iteration 0 would have issued them), stage 0 landed, its first
  // fragments read. Every wait below is "all but this wave's newest n fill instructions"
  // (buffer loads complete in order) followed by a bare s_barrier: __syncthreads()'s fence
  // would wait for every fill in flight, the next stages' included.
  constexpr int F0 = NCH * 3 / 8;  // fills of a stage issued at the barrier that frees it
  // at iteration kt's barrier the newest fills are those of tiles kt + 2 .. kt + NST - 1
  // (whole: the last one's began at the barrier before); in the prologue, those of stages
  // 1 .. NST - 2 and the first F0 of stage NST - 1
  constexpr int WAIT_LOOP = (NST - 2) * NCH;
  constexpr int WAIT_PRO = (NST - 2) * NCH + F0;
  auto sync_fills = [&](bool prologue) {
    __builtin_amdgcn_sched_barrier(0);
    if (prologue) __builtin_amdgcn_s_waitcnt(tile4_vmcnt_lgkm0(WAIT_PRO));
    else __builtin_amdgcn_s_waitcnt(tile4_vmcnt_lgkm0(WAIT_LOOP));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
  };
#pragma unroll
  for (int st = 0; st < NST - 1; ++st) fill_part(min(st, nkt - 1), st, 0, NCH);
  fill_part(min(NST - 1, nkt - 1), NST - 1, 0, F0);
  sync_fills(true);
  read_frags(0, 0, a0, b0);

  // One iteration is one 128-byte K stage: KS k-steps of FM x FN MFMAs, fragment reads one
  // k-step ahead. The body is one basic block (fills and reads past the last stage are
  // kept, pointed at the last stage again, and never used), so the MFMAs, the reads and
  // the fills are interleaved by sched_group_barrier: the next tile's fills -- into the
  // stage freed at this iteration's barrier -- start under the last k-step (3/8 of them)
  // and go on under the next iteration's first two k-steps. A burst of fills blocks the
  // wave's in-order issue (every wave of the CU issues its 16 at once and they queue at
  // the address unit), so spread out they cost a third less; spread over three k-steps
  // they still land before the barrier that waits for them.
  constexpr int NRD = FP8 ? 2 * (FM + FN) : (FM + FN);  // ds_read_b128 per k-step
  for (int kt = 0; kt < nkt; ++kt) {
    const int s = kt % NST;
    const int tk = min(kt + NST - 1, nkt - 1);  // the tile whose fills go on under this one
    const int sf = (kt + NST - 1) % NST;        // and its stage
#pragma unroll
    for (int ks = 0; ks < KS - 1; ++ks) {
      if (ks & 1) {
        read_frags(s, ks + 1, a0, b0);
        mma(a1, b1);
      } else {
        read_frags(s, ks + 1, a1, b1);
        mma(a0, b0);
      }
      {
        // the rest of tile kt + 1's fills, begun under iteration kt - 1's last k-step
        constexpr int F1 = NCH * 11 / 16;
        if (KS == 2) {
          fill_part(tk, sf, F0, NCH);
        } else {
          if (ks == 0) fill_part(tk, sf, F0, F1);
          if (ks == 1) fill_part(tk, sf, F1, NCH);
        }
#pragma unroll
        for (int q = 0; q < NRD; ++q) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 1 LDS read
          __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // 1 fill
        }
        __builtin_amdgcn_sched_group_barrier(0x008, FM * FN - NRD, 0);
        __builtin_amdgcn_sched_group_barrier(0x020, NCH, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // every wave is done reading stage s once this barrier passes (its last reads were
    // waited for), and the next stage -- tile kt + 1 -- has landed: each wave waits for its
    // own fills of it: all but its newest (NST - 2) NCH
    sync_fills(false);
    fill_part(min(kt + NST, nkt - 1), s, 0, F0);
    // KS is even: step KS-1 multiplies set 1 while the next stage's step 0 reads set 0
    read_frags((kt + 1) % NST, 0, a0, b0);
    mma(a1, b1);
#pragma unroll
    for (int q = 0; q < NRD; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, FM * FN - NRD, 0);
    __builtin_amdgcn_sched_group_barrier(0x020, NCH, 0);
    __builtin_amdgcn_sched_barrier(0);
  }
  __builtin_amdgcn_s_waitcnt(0x3f70);  // the last (unused) fills land before LDS is reused

  // ---- the store. Lane l holds, for fragment (i, j) and run g, C[m][n .. n + 3] with
  // m = wm TM + 32 i + (l & 31), n = wn TN + 32 j + 8 g + 4 (l >> 5). The fused epilogue
  // runs on them in registers; a 16- or 8-bit C is converted once and staged in LDS, then
  // stored as 16-byte pieces of whole rows (row-contiguous stores cost half of the
  // scattered 8-byte ones); an fp32 C or the fp32 shares go straight from the registers.
  const int mw = wm * TM + (lane & 31);
  const int nw = wn * TN + 4 * h;
  if constexpr (MODE == kStoreF32 || MODE == kPairWs) {
    float* out = (float*)p.c + (int64_t)split * p.split_stride;
    // (a share finished in the kernel goes out through its buffer, coherent device-wide)
    const __amdgpu_buffer_rsrc_t rshare = make_rsrc(out, (uint32_t)p.M * (uint32_t)p.ldc * 4u);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int m = m0 + mw + 32 * i;
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          __builtin_amdgcn_sched_barrier(0);
          f32x4 v = f32x4{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                          acc[i][j][4 * g + 3]};
          if constexpr (MODE == kStoreF32) {
            const int n = n0 + nw + 32 * j + 8 * g;
            if (m < p.M && n < p.N) {
              if (fused) {
                const int nl = nw + 32 * j + 8 * g;
                v = v * (*(const f32x4*)(rowop + nl) * csv[i]) + *(const f32x4*)(rowop + BN + nl);
                if (e.ta.p) v += ld_tile(e.ta, m, n);
                v = act4(e.act, v + e.cadd);
              }
              if (p.cnt) share_store4(rshare, ((uint32_t)m * (uint32_t)p.ldc + (uint32_t)n) * 4u, v);
              else *(f32x4*)(out + (int64_t)m * p.ldc + n) = v;
            }
          } else {
            const int fv = wn * FN + j;
            const int oc = n0 + (fv >> 1) * 32 + 8 * g + 4 * h;
            if (m < p.M && oc < p.N)
              *(f32x4*)(out + (int64_t)m * p.ldc + oc + ((fv & 1) ? p.N : 0)) = v;
          }
        }
    }
    if constexpr (MODE == kStoreF32) {
      if (p.cnt) finish_split<BM, OUTW, 256>(p, blockIdx.x, m0, n0, (int*)(smem + SMEM));
    }
  } else {
    __syncthreads();  // the stages are reused as the staging tile
    // Straight-line code, no branch between the element groups, so the scheduler can
    // overlap one group's dependent chain (AGPR read, math, convert, LDS write) with the
    // next's -- with one wave a SIMD nothing else would hide its latency. Absent row and
    // column operands hold 1 and 0 (the identity); rows past M and columns past N are
    // computed from clamped, in-bounds loads and never stored.
    auto group = [&](int i, int j, int g, bool tile_op) {
      const int ml = mw + 32 * i;
      f32x4 v = f32x4{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                      acc[i][j][4 * g + 3]};
      int cl;
      if constexpr (MODE == kPair16) {
        const f32x4 u = f32x4{acc[i][j + 1][4 * g], acc[i][j + 1][4 * g + 1],
                              acc[i][j + 1][4 * g + 2], acc[i][j + 1][4 * g + 3]};
        v = silu_mul4(v, u);
        cl = ((wn * FN + j) >> 1) * 32 + 8 * g + 4 * h;
      } else {
        cl = nw + 32 * j + 8 * g;
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
        __builtin_amdgcn_sched_barrier(0);  // a fragment (16 elements) at a time
        if (tile_op) {
#pragma unroll
          for (int g = 0; g < 4; ++g) group(i, j, g, true);
        } else {
#pragma unroll
          for (int g = 0; g < 4; ++g) group(i, j, g, false);
        }
      }
    }
    __syncthreads();
    constexpr int CPR = OUTW * OB / 16;  // 16-byte chunks a row
    constexpr int EPC = 16 / OB;         // elements a chunk
#pragma unroll 4
    for (int q = tid; q < BM * CPR; q += 256) {
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
}

}  // namespace hkx
