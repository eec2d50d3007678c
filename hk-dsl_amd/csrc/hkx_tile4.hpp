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
// * Two LDS stages; the fill of stage kt + 2 is issued right after the one barrier of
//   iteration kt and has a whole iteration to land.
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

template <int BM, int BN, bool FP8, int MODE, int SCHED = 1>
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
  constexpr int SMEM = 2 * STAGE;
  static_assert(FM >= 1 && FN >= 1 && BM % 64 == 0 && BN == 256, "tiling");
  static_assert(!PAIR || FN % 2 == 0, "the paired form needs gate/up fragment pairs");
  static_assert(SMEM <= 160 * 1024, "LDS");
  using Frag = typename std::conditional<FP8, i32x8, bf16x8>::type;

  __shared__ __attribute__((aligned(16))) uint8_t smem[SMEM];

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
  auto fill = [&](int kt, int s) {
    const uint32_t so = (uint32_t)(kt0 + kt) * 128u;
    uint8_t* base = smem + s * STAGE + wave * 1024;
#pragma unroll
    for (int i = 0; i < NCH; ++i)
      buf_load16_lds(i < NA ? ra : rb, base + i * 4096, voff[i], so);
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

  // ---- prologue: stages 0 and 1 in flight, stage 0 landed, its first fragments read
  fill(0, 0);
  if (nkt > 1) fill(1, 1);
  __builtin_amdgcn_s_waitcnt(0x3f70);  // vmcnt(0): stages 0 and 1 landed
  __syncthreads();
  read_frags(0, 0, a0, b0);

  // One iteration is one 128-byte K stage: KS k-steps of FM x FN MFMAs. The body is one
  // basic block (the fills and reads past the last stage are kept, pointed at the last
  // stage again, and never used), so the MFMAs, the fragment reads and the fills can be
  // interleaved explicitly: SCHED 1 puts one LDS read after each of the first MFMAs of a
  // step, and in the last step the fills too, so the MFMA pipe is never left waiting on
  // an issue slot. SCHED 0 leaves the order to the compiler.
  constexpr int NRD = FP8 ? 2 * (FM + FN) : (FM + FN);  // ds_read_b128 per k-step
  for (int kt = 0; kt < nkt; ++kt) {
    const int s = kt & 1;
#pragma unroll
    for (int ks = 0; ks < KS - 1; ++ks) {
      if (ks & 1) {
        read_frags(s, ks + 1, a0, b0);
        mma(a1, b1);
      } else {
        read_frags(s, ks + 1, a1, b1);
        mma(a0, b0);
      }
      if constexpr (SCHED == 1) {
#pragma unroll
        for (int q = 0; q < NRD; ++q) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 1 LDS read
        }
        __builtin_amdgcn_sched_group_barrier(0x008, FM * FN - NRD, 0);
      }
      if constexpr (SCHED != 0) __builtin_amdgcn_sched_barrier(0);
    }
    // every wave is done reading stage s once this barrier passes (its last reads were
    // waited for), and stage s ^ 1 -- the next tile, filled since iteration kt - 1 --
    // has landed: each wave waits for its own fills first (the barrier's fence waits
    // only for LDS operations, not for these buffer loads)
    __builtin_amdgcn_s_waitcnt(0x3f70);  // vmcnt(0)
    __syncthreads();
    fill(min(kt + 2, nkt - 1), s);
    // KS is even: step KS-1 multiplies set 1 while the next stage's step 0 reads set 0
    read_frags(s ^ 1, 0, a0, b0);
    mma(a1, b1);
    if constexpr (SCHED == 1) {
#pragma unroll
      for (int q = 0; q < NRD; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x020, NCH / NRD, 0);  // fills
      }
      __builtin_amdgcn_sched_group_barrier(0x008, FM * FN - NRD, 0);
    }
    if constexpr (SCHED != 0) __builtin_amdgcn_sched_barrier(0);
  }
  __builtin_amdgcn_s_waitcnt(0x3f70);  // the last (unused) fills land before LDS is reused

  // ---- the store, in FM rounds. Round r parks every wave's fragment row r (fp32, 64
  // rows x BN columns: rows 32 wm + (l & 31), columns wn TN + 32 j + 8 g + 4 (l >> 5) for
  // run g) in an LDS slab; then each thread takes 8 consecutive columns of 8 slab rows,
  // runs the epilogue on them in registers and stores them as one 16-byte (8 x bf16) or
  // 32-byte (fp32) row piece. The epilogue is a rolled loop, so it costs no code per
  // accumulator and no registers beside the K loop's.
  constexpr int SR = BN * 4 + 16;  // slab row stride, bytes
  static_assert(64 * SR <= 2 * STAGE, "slab");
  const int orow = tid >> 5;        // slab rows orow + 8 q
  const int oc8 = (tid & 31) * 8;   // this thread's 8 columns of the slab (BN = 256)
  float* out32 = (float*)p.c + (int64_t)split * p.split_stride;
  // The row operands of the fused form depend on the column alone: loaded once.
  const Fused& e = p.ep;
  const bool fused = !PAIR && e.form == HKX_EP_FUSED;
  const int nq = n0 + oc8;
  const bool hi_ok = nq + 4 < p.N;  // N % 4 == 0: the second run of four is in or out whole
  f32x4 rs0 = {1.f, 1.f, 1.f, 1.f}, rs1 = rs0, ra0 = {0.f, 0.f, 0.f, 0.f}, ra1 = ra0;
  if (fused && nq < p.N) {
    if (e.rs.p) { rs0 = ld_row(e.rs, nq); if (hi_ok) rs1 = ld_row(e.rs, nq + 4); }
    if (e.ra.p) { ra0 = ld_row(e.ra, nq); if (hi_ok) ra1 = ld_row(e.ra, nq + 4); }
  }
#pragma unroll  // acc[r] must be a static index: the accumulators live in AGPRs
  for (int r = 0; r < FM; ++r) {
    __syncthreads();  // the K loop's (or the last round's) reads of LDS are done
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *(f32x4*)(smem + (wm * 32 + rf) * SR + (wn * TN + 32 * j + 8 * g + 4 * h) * 4) =
            f32x4{acc[r][j][4 * g], acc[r][j][4 * g + 1], acc[r][j][4 * g + 2],
                  acc[r][j][4 * g + 3]};
    __syncthreads();
    if (PAIR && oc8 >= BN / 2) continue;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int sr = orow + 8 * q;
      const int m = m0 + (sr >> 5) * TM + 32 * r + (sr & 31);
      const uint8_t* src = smem + sr * SR;
      const int n = nq;
      if (m >= p.M || n >= p.N) continue;
      f32x4 v0, v1;
      if constexpr (PAIR) {
        // slab columns are fragments: gate in even 32-column blocks, up in odd ones
        const int vb = (oc8 >> 5) * 64 + (oc8 & 31);
        const f32x4 g0 = *(const f32x4*)(src + vb * 4), g1 = *(const f32x4*)(src + vb * 4 + 16);
        const f32x4 u0 = *(const f32x4*)(src + (vb + 32) * 4);
        const f32x4 u1 = *(const f32x4*)(src + (vb + 32) * 4 + 16);
        if constexpr (MODE == kPairWs) {
          float* o = out32 + (int64_t)m * p.ldc;
          *(f32x4*)(o + n) = g0;
          *(f32x4*)(o + p.N + n) = u0;
          if (hi_ok) {
            *(f32x4*)(o + n + 4) = g1;
            *(f32x4*)(o + p.N + n + 4) = u1;
          }
          continue;
        }
        v0 = silu_mul4(g0, u0);
        v1 = silu_mul4(g1, u1);
      } else {
        v0 = *(const f32x4*)(src + oc8 * 4);
        v1 = *(const f32x4*)(src + oc8 * 4 + 16);
        if (fused) {
          if (e.cs.p) {
            const float sc = ld_col(e.cs, m);
            v0 *= sc;
            v1 *= sc;
          }
          v0 = v0 * rs0 * e.cmul + ra0;
          v1 = v1 * rs1 * e.cmul + ra1;
          if (e.ta.p) {
            v0 += ld_tile(e.ta, m, n);
            if (hi_ok) v1 += ld_tile(e.ta, m, n + 4);
          }
          v0 = act4(e.act, v0 + e.cadd);
          v1 = act4(e.act, v1 + e.cadd);
        }
      }
      if constexpr (MODE == kStoreF32) {
        float* o = out32 + (int64_t)m * p.ldc + n;
        *(f32x4*)o = v0;
        if (hi_ok) *(f32x4*)(o + 4) = v1;
      } else {
        uint8_t* dst = (uint8_t*)p.c + ((int64_t)m * p.ldc + n) * OB;
        const u32x2 w0 = pack4<OB>(p.c_dt, v0), w1 = pack4<OB>(p.c_dt, v1);
        if constexpr (OB == 2) {
          if (p.c_aligned && hi_ok) {
            *(i32x4*)dst = i32x4{(int)w0.x, (int)w0.y, (int)w1.x, (int)w1.y};
          } else {
            *(u32x2*)dst = w0;
            if (hi_ok) *(u32x2*)(dst + 8) = w1;
          }
        } else {
          *(uint32_t*)dst = w0.x;
          if (hi_ok) *(uint32_t*)(dst + 4) = w1.x;
        }
      }
    }
  }
}

}  // namespace hkx
