// The persistent 256 x 256 MFMA GEMM for gfx950: 8 waves in two groups of four (one wave of
// each group a SIMD), each wave a 64 x 128 block of C (128 fp32 accumulators a lane). One
// workgroup a CU walks its tiles (every gridDim.x-th, XCD-aware numbering, grouped raster)
// with one continuous LDS pipeline across tile boundaries.
//
// Why this schedule:
// * Ping-pong. The groups are one phase apart: while one issues a half-stage's MFMAs at raised
//   priority, the other reads the next half-stage's fragments from LDS and issues fills; a
//   barrier of all 8 waves ends every phase. A single wave's ds_read_b128 stream runs at a
//   quarter of the LDS's rate on gfx950, so one wave a SIMD cannot both feed a 128 x 128
//   block and keep its MFMAs busy; two waves taking turns can.
// * Fill latency. K advances in half-stages (64 bytes of every row) through a ring of four
//   32 KB buffers. Half-stage u + 3 is filled into the buffer u - 1 used, once every wave is
//   past u - 1's reads: three half-stages (~6 phases) to hide the L2 / MALL / HBM latency.
// * MFMA: bf16 as v_mfma_f32_16x16x32_bf16 (4 x 8 fragments of 16 x 16 a wave; one k-step is
//   a half-stage), fp8 e4m3 as v_mfma_scale_f32_32x32x64_f8f6f4 (2 x 4 fragments of 32 x 32).
//   B's fragment is the first operand, so a lane ends with runs of four consecutive columns
//   of one row of C. The MX form passes each lane's E8M0 byte for its fragment row and 32-K
//   block as the MFMA's scales.
// * Tile boundaries cost nothing in the pipeline: the fills of the next tile's first
//   half-stages are in flight while this tile's last k-steps run and its epilogue is
//   applied; the epilogue goes from the accumulators straight to global memory (no LDS
//   staging, no barrier), and the next tile's first k-step starts from zero accumulators.
// * Stores: lanes that hold neighbouring four-column runs trade them with
//   v_permlane16_swap (16 x 16 fragments) or v_permlane32_swap (32 x 32), so each lane
//   writes 16 contiguous bytes (eight bf16 columns) and a wave writes whole 64-byte pieces
//   of rows.
// * The epilogue's vector operands (column scale, row scale, row add) go global -> LDS by
//   the same DMA as the fills, double-buffered by tile parity, at the tile's start; a TILE
//   operand (residual) is read from global memory in the epilogue.
//
// Fills: wave w's instruction i moves rows 128 (i % 2) + 16 w + [0, 16) of a half-stage's A
// (i < 2) or B (i >= 2) rows; lane l writes bytes 16 l of that 1 KB (row + l / 4, physical
// chunk l % 4). A row's four 16-byte chunks are stored XOR-swizzled by bits 3 and 4 of the
// row (chunk c at c ^ swz4(r)), so the fragment reads -- 16 rows of four chunks, or 32 rows
// of one -- are conflict-free; the swizzle is applied on the global side.
//
// Ragged M and N edges read zeros through the buffer resources' bounds; stores are
// predicated on n < N and dropped past M by the store's buffer bounds (the host sends
// N % 8 != 0, an unaligned C or a C of 4 GiB or more elsewhere).
#pragma once

#include "hkx_tile.hpp"

namespace hkx {

typedef float f32x16 __attribute__((ext_vector_type(16)));

// s_waitcnt operands (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8)
constexpr int wait_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
constexpr int wait_vm_lgkm0(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4); }

// v_permlane32_swap: lanes 32-63 of a trade places with lanes 0-31 of b.
HKX_DEV void swap32(uint32_t& a, uint32_t& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
  a = r[0];
  b = r[1];
}

// v_permlane16_swap: the odd 16-lane rows of a trade places with the even rows of b.
HKX_DEV void swap16(uint32_t& a, uint32_t& b) {
  const auto r = __builtin_amdgcn_permlane16_swap(a, b, false, false);
  a = r[0];
  b = r[1];
}

// Epilogue operand forms of the ring kernel (compile time).
constexpr int kEpNone = 0;     // act(acc)
constexpr int kEpBias = 1;     // act(acc + ra[n]), ra bf16
constexpr int kEpDeq = 2;      // act(acc cs[m] rs[n]), cs and rs fp32
constexpr int kEpDeqBias = 3;  // act(acc cs[m] rs[n] + ra[n]), cs and rs fp32, ra bf16
constexpr int kEpGeneric = 4;  // the whole fused form with run-time types and output type
constexpr int kEpTile = 5;     // act(acc + ra[n] + ta[m][n]), ra (optional) and ta bf16 (quadrant kernel)

// FP8: 0 bf16 operands; 1 fp8 e4m3 x e4m3; 2 e5m2 x e5m2; 3 A e4m3 x B e5m2; 4 A e5m2 x B
// e4m3 (TileArgs::ab_fmt). The scaled MFMA takes its first operand's format (here B's, as
// B's fragment goes first) in cbsz and its second's (A's) in blgp: 0 e4m3, 1 e5m2.
template <int FP8, int MODE, int ACT, int EPF, bool MX = false>
__global__ void __launch_bounds__(512, 1) ring_kernel(const TileArgs p) {
  constexpr int FMT_B = (FP8 == 2 || FP8 == 3) ? 1 : 0;
  constexpr int FMT_A = (FP8 == 2 || FP8 == 4) ? 1 : 0;
  constexpr int BM = 256, BN = 256;
  constexpr int FR = FP8 ? 32 : 16;           // fragment edge
  constexpr int FM = 64 / FR, FN = 128 / FR;  // fragments of a wave's 64 x 128
  constexpr int HS = 512 * 64;                 // one half-stage buffer
  constexpr int NBUF = 4;
  constexpr int EPO = NBUF * HS;  // epilogue operands: [tile parity][cs, rs, ra][256 slots]
  // MX scales: [chunk % 3][512 rows] of 16 bytes, a chunk the E8M0 bytes of 8 half-stages
  // (16 blocks of 32 K) of every A and B row of the tile
  constexpr int SCO = EPO + 2 * 3 * 1024;
  constexpr int SMEM = SCO + (MX ? 3 * 512 * 16 : 0);
  static_assert(!MX || FP8, "MX scales go with fp8 operands");
  constexpr bool PAIR = (MODE == kPair16 || MODE == kPairWs);
  constexpr int OUTW = PAIR ? BN / 2 : BN;
  static_assert(!(PAIR && FP8) && !(MODE == kStore8 && PAIR), "modes");
  static_assert(SMEM <= 160 * 1024, "LDS");
  using Frag = typename std::conditional<FP8 != 0, i32x8, bf16x8>::type;
  using Acc = typename std::conditional<FP8 != 0, f32x16, f32x4>::type;

  __shared__ __attribute__((aligned(16))) uint8_t smem[SMEM];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2;  // the ping-pong group: a SIMD holds waves w and w + 4
  const int wm = (wave >> 1) & 1, wn = wave & 1;
  const int row0 = grp * 128 + wm * 64, col0 = wn * 128;  // the wave's block of the tile

  const int total = p.tiles_m * p.tiles_n;
  const int G = gridDim.x;
  const int my_tiles = (total - (int)blockIdx.x + G - 1) / G;
  const int split = blockIdx.y;
  const int kt0 = split * p.kt_split;
  const int nkt = min(p.kt_split, p.kt_total - kt0);
  const int hpt = 2 * nkt;        // half-stages (= k-steps) a tile
  const int nu = my_tiles * hpt;  // half-stages of this workgroup

  // tile (m0, n0) of this workgroup's lt-th tile: XCD-chunked renumbering (the hardware
  // deals workgroup ids round-robin over the 8 XCDs), then a grouped raster of wgm tile
  // rows, so the tiles in flight on one XCD share A and B panels in its L2
  auto tile_at = [&](int lt, int& m0, int& n0) {
    const int v = (int)blockIdx.x + lt * G;
    int L = v;
    if ((total & 7) == 0) L = (L & 7) * (total >> 3) + (L >> 3);
    const int per = p.wgm * p.tiles_n;
    const int gi = L / per;
    const int first = gi * p.wgm;
    const int gm = min(p.tiles_m - first, p.wgm);
    const int in = L - gi * per;
    m0 = (first + in % gm) * BM;
    n0 = (in / gm) * OUTW;
  };

  // (Code inside the tile loop takes the lane index fresh from mbcnt, through an empty asm,
  // so the per-lane values it derives are recomputed there instead of being hoisted out of
  // the loop and held -- or spilled -- in registers across it.)
  auto opaque_lane = [&]() {
    int l = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    asm volatile("" : "+v"(l));
    return l;
  };

  // ---- fills. Instruction i of a wave moves rows 128 i + 16 wave + l / 4: the swizzle
  // (bits 3-4 of the row) is the same for every i, so a fill's global offset is one per-lane
  // base (for A, for B) plus i times a uniform row step, added in the scalar offset.
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a, p.a_bytes);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.b, p.b_bytes);
  uint32_t fa = 0, fb = 0;
  const uint32_t sa_step = 128u * p.lda_b, sb_step = (PAIR ? 64u : 128u) * p.ldb_b;
  int f_lt = 0, f_kv = 0, f_u = 0;  // the next fill: local tile, half-stage in it, global
  const __amdgpu_buffer_rsrc_t rsa = make_rsrc(MX ? p.sa : nullptr, MX ? p.sa_bytes : 0u);
  const __amdgpu_buffer_rsrc_t rsb = make_rsrc(MX ? p.sb : nullptr, MX ? p.sb_bytes : 0u);
  uint32_t fsa = 0, fsb = 0;  // this lane's scale row (MX)
  // MX scale chunks a tile; chunks rotate through three LDS buffers across tiles too. A
  // chunk's buffer is refilled three chunks later, three half-stages before that chunk's
  // first read, so at least 2 + 2 - 3 half-stages after the old chunk's last one (every
  // chunk is 2 half-stages or more): with two buffers a 2-half-stage chunk (the end of
  // K = 1152) let the refill land under the other group's last reads.
  const int cpt = (hpt + 7) >> 3;
  auto fill_tile = [&](int lt) {
    int m0, n0;
    tile_at(lt, m0, n0);
    const int ln = opaque_lane();
    if constexpr (MX) {
      fsa = (uint32_t)(m0 + 64 * (wave & 3) + ln) * p.sa_ld;
      fsb = (uint32_t)(n0 + 64 * (wave & 3) + ln) * p.sb_ld;
    }
    const int r = 16 * wave + (ln >> 2);  // row of instruction 0 (A), 2 (B, less 256)
    const uint32_t ch = (uint32_t)(((ln & 3) ^ swz4(r)) << 4);
    fa = (uint32_t)(m0 + r) * p.lda_b + ch;
    int brow;
    if constexpr (PAIR) {
      // B tile row 16 f + x is row x of fragment f: the gate (even f) or up (odd f) row of
      // output column n0 + 16 (f / 2) + x; instruction i adds 8 fragments (64 B rows)
      brow = n0 + (wave >> 1) * 16 + (ln >> 2) + ((wave & 1) ? p.pair_off : 0);
    } else {
      brow = n0 + r;
    }
    fb = (uint32_t)brow * p.ldb_b + ch;
  };
  // Issues this wave's share of the next half-stage. Past the last one it fetches the
  // last again (into a buffer nothing reads), so every wait count stays the same.
  auto fill_next = [&]() {
    const uint32_t so = __builtin_amdgcn_readfirstlane((uint32_t)(kt0 * 128 + f_kv * 64));
    uint8_t* base = smem + (f_u & (NBUF - 1)) * HS + wave * 1024;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      buf_load16_lds(i < 2 ? ra : rb, base + i * 8192, i < 2 ? fa : fb,
                     so + (uint32_t)(i & 1) * (i < 2 ? sa_step : sb_step));
    if constexpr (MX) {
      // every 8th half-stage of a tile, after its operands: the scales of the 8 from it on
      // (16 bytes of E8M0 a row, blocks 2 uk .. 2 uk + 15), lane l of wave w for row
      // 64 w + l (A rows, then B). Issued after the half-stage's own fills, it is done
      // whenever they are, before that half-stage is read; one more load only makes the
      // waits count stricter.
      if ((f_kv & 7) == 0) {
        const uint32_t uk = (uint32_t)(2 * kt0 + f_kv);
        const int chunk = f_lt * cpt + (f_kv >> 3);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(wave < 4 ? rsa : rsb,
            (__attribute__((address_space(3))) void*)(smem + SCO + (chunk % 3) * 8192 + wave * 1024),
            16, wave < 4 ? fsa : fsb, __builtin_amdgcn_readfirstlane(2u * uk), 0, 0);
      }
    }
    ++f_u;
    if (f_u < nu) {
      if (++f_kv == hpt) {
        f_kv = 0;
        fill_tile(++f_lt);
      }
    }
  };

  // ---- the epilogue's vector operands of local tile lt, into LDS slots (tile parity).
  // A vector operand's slot e holds element e of the tile's rows (cs) or columns (rs, ra):
  // a 32-bit load of the aligned pair that contains it, for 16-bit types (the host sends a
  // 16-bit column operand here only with unit stride, so a slot's half is e's parity). A
  // broadcast operand (stride 0) is one value, read once.
  const Fused& e = p.ep;
  const bool fused = !PAIR && e.form == HKX_EP_FUSED;
  const bool cs_vec = fused && e.cs.p && e.cs.ld, rs_vec = fused && e.rs.p && e.rs.ld,
             ra_vec = fused && e.ra.p && e.ra.ld;
  const float cs_sc = (fused && e.cs.p && !e.cs.ld) ? ld1(e.cs.p, e.cs.dt, 0) * e.cmul : e.cmul;
  const float rs_sc = (fused && e.rs.p && !e.rs.ld) ? ld1(e.rs.p, e.rs.dt, 0) : 1.0f;
  const float ra_sc = (fused && e.ra.p && !e.ra.ld) ? ld1(e.ra.p, e.ra.dt, 0) : 0.0f;
  auto vec_rsrc = [&](const Opnd& o, int n) {
    return make_rsrc(o.p, (uint32_t)n * (o.dt == HKX_FP32 ? 4u : 2u));
  };
  const __amdgpu_buffer_rsrc_t rcs = vec_rsrc(e.cs, cs_vec ? (int)((int64_t)(p.M - 1) * e.cs.ld + 1) : 0);
  const __amdgpu_buffer_rsrc_t rrs = vec_rsrc(e.rs, rs_vec ? p.N : 0);
  const __amdgpu_buffer_rsrc_t rra = vec_rsrc(e.ra, ra_vec ? p.N : 0);
  auto slot_load = [&](__amdgpu_buffer_rsrc_t r, int dt, int64_t idx, uint8_t* dst) {
    const uint32_t off = dt == HKX_FP32 ? (uint32_t)idx * 4u : (uint32_t)(idx & ~1LL) * 2u;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 4,
                                             off, 0, 0, 0);
  };
  auto ep_load = [&](int lt) {
    if (!(cs_vec || rs_vec || ra_vec)) return;
    int m0, n0;
    tile_at(lt, m0, n0);
    uint8_t* base = smem + EPO + (lt & 1) * 3072 + (wave & 3) * 256;
    const int el = 64 * (wave & 3) + opaque_lane();  // this lane's row (cs) or column (rs, ra)
    if (grp == 0) {
      if (cs_vec) slot_load(rcs, e.cs.dt, (int64_t)(m0 + el) * e.cs.ld, base);
      if (rs_vec) slot_load(rrs, e.rs.dt, n0 + el, base + 1024);
    } else {
      if (ra_vec) slot_load(rra, e.ra.dt, n0 + el, base + 2048);
    }
  };

  // ---- fragment reads. 16 x 16 bf16: lane l reads row l % 16 of a fragment, chunk l / 16
  // (a 16-row fragment's swizzle bit 4 is the fragment's parity: rdo[1] serves the odd
  // ones). 32 x 32 fp8: lane l reads row l % 32, chunks l / 32 and 2 + l / 32: the scaled
  // MFMA takes a lane's bytes 0-15 as K block 0 of its 64 and bytes 16-31 as block 1 (the
  // scale of block b coming from the lanes l / 32 = b), so lane half h holds K [16 h, +16)
  // of each 32-K block.
  uint32_t rdo[2];
  {
    const int rf = lane & (FR - 1), h = lane / FR;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int lc = FP8 ? (2 * q + h) : h;
      const int sw = swz4(FP8 ? rf : rf + 16 * q);
      rdo[q] = rf * 64 + ((lc ^ sw) << 4);
    }
  }
  constexpr int FB = FR * 64;  // bytes of a fragment's rows in a buffer
  const int a_off = row0 * 64, b_off = (BM + col0) * 64;
  // MX: lanes l / 32 = h give the scale of 32-K block h of the MFMA's 64 for their fragment
  // row. Half-stage k of a tile (k % 8 = r in its chunk) has blocks 2 r and 2 r + 1 of the
  // chunk: byte 2 (r & 1) + h of dword r / 2 of the row's 16 bytes, shifted down to byte 0,
  // the MFMA's scale select.
  uint32_t sfa[FM], sfb[FN];
  const int sc_sh = 8 * (lane >> 5);
  auto read_scales = [&](int lt, int k) {
    if constexpr (MX) {
      const int r = k & 7;
      const uint32_t* sc =
          (const uint32_t*)(smem + SCO + ((lt * cpt + (k >> 3)) % 3) * 8192) + (r >> 1);
      const int rf = lane & 31, sh = sc_sh + 16 * (r & 1);
#pragma unroll
      for (int j = 0; j < FN; ++j) sfb[j] = sc[4 * (BM + col0 + 32 * j + rf)] >> sh;
#pragma unroll
      for (int i = 0; i < FM; ++i) sfa[i] = sc[4 * (row0 + 32 * i + rf)] >> sh;
    }
  };
  auto read_frags = [&](int u, int lt, int k, Frag (&af)[FM], Frag (&bf)[FN]) {
    const uint8_t* s = smem + (u & (NBUF - 1)) * HS;
    read_scales(lt, k);
    if constexpr (FP8) {
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const i32x4 lo = *(const i32x4*)(s + b_off + j * FB + rdo[0]);
        const i32x4 hi = *(const i32x4*)(s + b_off + j * FB + rdo[1]);
        bf[j] = i32x8{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
      }
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const i32x4 lo = *(const i32x4*)(s + a_off + i * FB + rdo[0]);
        const i32x4 hi = *(const i32x4*)(s + a_off + i * FB + rdo[1]);
        af[i] = i32x8{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
      }
    } else {
#pragma unroll
      for (int j = 0; j < FN; ++j) bf[j] = *(const bf16x8*)(s + b_off + j * FB + rdo[j & 1]);
#pragma unroll
      for (int i = 0; i < FM; ++i) af[i] = *(const bf16x8*)(s + a_off + i * FB + rdo[i & 1]);
    }
  };

  Acc acc[FM][FN];
  auto mma = [&](const Frag (&af)[FM], const Frag (&bf)[FN], auto zero) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const Acc c = decltype(zero)::value ? Acc{} : acc[i][j];
        if constexpr (MX)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bf[j], af[i], c, 0, 0, 0,
                                                                     (int)sfb[j], 0, (int)sfa[i]);
        else if constexpr (FP8)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bf[j], af[i], c, FMT_B,
                                                                     FMT_A, 0, 0, 0, 0);
        else
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf[j], af[i], c, 0, 0, 0);
      }
  };
  // ---- the epilogue of local tile lt, from the accumulators. EPF fixes the operand form
  // at compile time (the hot forms are straight-line code with no dtype branches).
  auto epilogue = [&](int lt) {
    int m0, n0;
    tile_at(lt, m0, n0);
    const uint32_t* eo = (const uint32_t*)(smem + EPO + (lt & 1) * 3072);
    const int ln = opaque_lane();
    const int rf = ln & (FR - 1), h = ln / FR;
    // element (row m, column n) of C: byte offset in a buffer resource bounded by M rows,
    // so rows past M are dropped by the hardware; columns past N are masked
    constexpr uint32_t EB = (MODE == kStoreF32 || MODE == kPairWs) ? 4u : (MODE == kStore8 ? 1u : 2u);
    const uint32_t row_b = (uint32_t)p.ldc * EB;
    const __amdgpu_buffer_rsrc_t rc = make_rsrc(
        (uint8_t*)p.c + (int64_t)split * p.split_stride * 4, (uint32_t)p.M * row_b);
    // the fused form on a run of four columns: tile row ml, tile column cl
    auto apply = [&](f32x4 v, int ml, int cl, float cs) -> f32x4 {
      if constexpr (EPF == kEpBias) {
        return act4c<ACT>(0, v + slot4(eo + 512 + cl, HKX_BF16));
      } else if constexpr (EPF == kEpDeq) {
        return act4c<ACT>(0, v * (__builtin_bit_cast(f32x4, *(const i32x4*)(eo + 256 + cl)) * cs));
      } else if constexpr (EPF == kEpDeqBias) {
        return act4c<ACT>(0, v * (__builtin_bit_cast(f32x4, *(const i32x4*)(eo + 256 + cl)) * cs) +
                                 slot4(eo + 512 + cl, HKX_BF16));
      } else if constexpr (EPF == kEpGeneric) {
        if (!fused) return v;
        const f32x4 rs = rs_vec ? slot4(eo + 256 + cl, e.rs.dt) : f32x4{rs_sc, rs_sc, rs_sc, rs_sc};
        const f32x4 rad = ra_vec ? slot4(eo + 512 + cl, e.ra.dt) : f32x4{ra_sc, ra_sc, ra_sc, ra_sc};
        v = v * (rs * cs) + rad;
        if (e.ta.p) v += ld_tile(e.ta, min(m0 + ml, p.M - 1), min(n0 + cl, p.N - 4));
        return act4(e.act, v + e.cadd);
      } else {
        return act4c<ACT>(0, v);
      }
    };
    auto col_scale = [&](int ml) -> float {
      if constexpr (EPF == kEpDeq || EPF == kEpDeqBias) return __builtin_bit_cast(float, eo[ml]);
      if constexpr (EPF == kEpGeneric) return cs_vec ? slot1(eo, ml, e.cs.dt) * e.cmul : cs_sc;
      return 1.0f;
    };
    auto run = [&](int i, int j, int g) -> f32x4 {
      if constexpr (FP8)
        return f32x4{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
      else
        return acc[i][j];
    };
    constexpr int OB = (MODE == kStore8) ? 1 : 2;
    const int cdt = (EPF == kEpGeneric || OB == 1) ? p.c_dt : HKX_BF16;
    // 16 output bytes (or 8 for an 8-bit C) at tile row ml, tile column n (8 columns)
    auto put = [&](int ml, int n, uint32_t x0, uint32_t y0, uint32_t x1, uint32_t y1) {
      if (n0 + n >= p.N) return;
      const uint32_t off = (uint32_t)(m0 + ml) * row_b + (uint32_t)(n0 + n) * EB;
      if constexpr (OB == 2)
        __builtin_amdgcn_raw_buffer_store_b128(i32x4{(int)x0, (int)y0, (int)x1, (int)y1}, rc, off, 0, 0);
      else
        __builtin_amdgcn_raw_buffer_store_b64(u32x2{x0, x1}, rc, off, 0, 0);
    };

    if constexpr (MODE == kStoreF32 || MODE == kPairWs) {
      // fp32: each run of four columns is one 16-byte store
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int ml = row0 + FR * i + rf;
        const float cs = col_scale(ml);
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int g = 0; g < FR / 8; ++g) {
            const int cl = col0 + FR * j + (FP8 ? 8 * g + 4 * h : 4 * h);
            f32x4 v = run(i, j, g);
            int n;
            if constexpr (MODE == kPairWs) {
              const int fv = wn * FN + j;  // 16-row fragment: gate (even) or up (odd)
              n = (fv >> 1) * 16 + 4 * h;
              if (n0 + n >= p.N) continue;
              n += (fv & 1) ? p.N : 0;
            } else {
              v = apply(v, ml, cl, cs);
              n = cl;
              if (n0 + n >= p.N) continue;
            }
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, v), rc,
                                                   (uint32_t)(m0 + ml) * row_b + (uint32_t)(n0 + n) * 4u, 0, 0);
          }
        }
      }
    } else if constexpr (FP8) {
      // 32 x 32: lanes l and l + 32 hold columns 8 g + [0, 4) and + [4, 8) of runs 2 t and
      // 2 t + 1; after the swap lane l holds 16 t + [0, 8), lane l + 32 16 t + [8, 16)
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int ml = row0 + 32 * i + rf;
        const float cs = col_scale(ml);
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            const int c0 = col0 + 32 * j + 16 * t;
            const u32x2 w0 = pack4<OB>(cdt, apply(run(i, j, 2 * t), ml, c0 + 4 * h, cs));
            const u32x2 w1 = pack4<OB>(cdt, apply(run(i, j, 2 * t + 1), ml, c0 + 8 + 4 * h, cs));
            uint32_t x0 = w0.x, x1 = w1.x, y0 = w0.y, y1 = w1.y;
            swap32(x0, x1);
            if constexpr (OB == 2) swap32(y0, y1);
            put(ml, c0 + 8 * h, x0, y0, x1, y1);
          }
        }
      }
    } else {
      // 16 x 16: lane l (row l % 16, quarter q = l / 16) holds columns 4 q + [0, 4) of each
      // fragment. Fragments a and b = a + 1 (or, paired, the silu-mul results of two
      // gate/up pairs) trade quarters: after the swap quarter q holds columns
      // 8 (q / 2) + [0, 8) of fragment a (q even) or b (q odd).
      const int q = h;
      // a bias is the same for the FM row fragments: read and widened once a column
      [[maybe_unused]] f32x4 bias_v[FN];
      if constexpr (EPF == kEpBias && !PAIR) {
#pragma unroll
        for (int j = 0; j < FN; ++j) bias_v[j] = slot4(eo + 512 + col0 + 16 * j + 4 * q, HKX_BF16);
      }
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int ml = row0 + 16 * i + rf;
        const float cs = col_scale(ml);
#pragma unroll
        for (int j = 0; j < FN; j += PAIR ? 4 : 2) {
          __builtin_amdgcn_sched_barrier(0);
          f32x4 va, vb;
          int ca;  // output tile column of fragment a's first column
          if constexpr (PAIR) {
            va = silu_mul4(run(i, j, 0), run(i, j + 1, 0));
            vb = silu_mul4(run(i, j + 2, 0), run(i, j + 3, 0));
            ca = ((wn * FN + j) >> 1) * 16;
          } else if constexpr (EPF == kEpBias) {
            ca = col0 + 16 * j;
            va = act4c<ACT>(0, run(i, j, 0) + bias_v[j]);
            vb = act4c<ACT>(0, run(i, j + 1, 0) + bias_v[j + 1]);
          } else {
            ca = col0 + 16 * j;
            va = apply(run(i, j, 0), ml, ca + 4 * q, cs);
            vb = apply(run(i, j + 1, 0), ml, ca + 16 + 4 * q, cs);
          }
          const u32x2 wa = pack4<OB>(cdt, va), wb = pack4<OB>(cdt, vb);
          uint32_t x0 = wa.x, x1 = wb.x, y0 = wa.y, y1 = wb.y;
          swap16(x0, x1);
          if constexpr (OB == 2) swap16(y0, y1);
          put(ml, ca + 16 * (q & 1) + 8 * (q >> 1), x0, y0, x1, y1);
        }
      }
    }
  };

  // ---- the K loop. Phases are separated by barriers of all 8 waves; group 1 starts one
  // barrier late (and group 0 ends with one extra), so the groups alternate:
  //   phase 2u + grp:     read half-stage u into registers, fill half-stage u + 3
  //   phase 2u + grp + 1: the MFMAs of half-stage u (at raised priority)
  // Before every barrier a wave waits for its reads and for all but its newest 8 vector
  // memory operations (the fills of the two newest half-stages, or stores after an
  // epilogue, which only makes the wait longer): the fills of half-stage v were issued
  // in phase 2 (v - 3) + grp and have landed at the barrier before phase 2 v, where group 0
  // reads v. Buffer u % 4 is refilled (with u + 4) in phase 2 (u + 1) + grp, after both
  // groups read it in phases 2u and 2u + 1.
  Frag af[FM], bf[FN];
  fill_tile(0);
  ep_load(0);
  fill_next();
  fill_next();
  fill_next();
  __builtin_amdgcn_s_waitcnt(wait_vm(8));  // this wave's share of half-stage 0 landed
  __builtin_amdgcn_s_barrier();
  if (grp == 1) __builtin_amdgcn_s_barrier();
  int u = 0;
  for (int lt = 0; lt < my_tiles; ++lt) {
    for (int k = 0; k < hpt; ++k, ++u) {
      // memory phase
      read_frags(u, lt, k, af, bf);
      if (k == 0 && lt + 1 < my_tiles) ep_load(lt + 1);
      fill_next();
      __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(8));
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      // matrix phase; a tile's first half-stage starts from zero accumulators
      __builtin_amdgcn_s_setprio(1);
      if (k == 0) mma(af, bf, std::true_type{});
      else mma(af, bf, std::false_type{});
      __builtin_amdgcn_s_setprio(0);
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(wait_vm(8));
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
    }
    epilogue(lt);
  }
  if (grp == 0) __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_s_waitcnt(wait_vm(0));  // no fill lands in LDS after the exit
}

}  // namespace hkx
