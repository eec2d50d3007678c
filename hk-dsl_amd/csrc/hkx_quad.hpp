// The quadrant ring GEMM kernel: bf16 C (M, N) = act(A . B^T (+ bias)) on 256 x 256 tiles,
// one persistent workgroup of 8 waves a CU, fills of whole 128-byte lines.
//
// Replaces, for bf16 operands and a 16-bit C with no epilogue or a bias and an activation,
// the reference's pp kernel (python/hk/ops/gemm_cdna.py:57-586, HipKittens' 256 x 256 x 64
// eight-wave ping-pong); the ring kernel (hkx_ring.hpp) takes every other form.
//
// * Quadrants. A tile's A rows are two halves of 128 (A0, A1), its B rows likewise (B0,
//   B1). Wave w of the 2 x 4 grid (r, c) = (w / 4, w % 4) owns rows 64 r + 128 i and
//   columns 32 c + 128 j of the tile for i, j in {0, 1}: four 64 x 32 accumulator blocks,
//   one per (A half i, B half j). So each half of A or B is read by all eight waves in one
//   phase and is free for its next fill right after.
// * K-tiles of 64 (whole 128-byte lines of a row). LDS holds two K-tile slots of four
//   quarters (A0, A1, B0, B1), 16 KB each. A quarter is 16 blocks of 1 KB, block b the 8
//   rows 8 b ..: its first 512 bytes K 0-31 of the 8 rows (64 bytes a row), the second K
//   32-63. One fill instruction moves one block: lanes l and l + 32 fetch the two halves
//   of row l % 32 / 4's line, so every request is a whole line, and the 64-byte K-halves
//   keep the bank pattern of 64-byte rows (16-byte chunk c of row r at c ^ swz4(r)).
// * Phases. Per K-tile t, two phases, each: LDS reads into registers, fills, a barrier,
//   the MFMAs of two blocks (32 v_mfma_f32_16x16x32_bf16, 16 fp8 16 x 16 x 128, or 8 MX
//   32 x 32 x 64), a barrier:
//     1: read A0(t), B0(t);      fill A1(t + 1), B1(t + 2);   math (0, 0), (0, 1)
//     2: read A1(t), B1(t + 1);  fill B0, A0 of t + 2;         math (1, 0), (1, 1)
//   (the MX form reads B1(t) in phase 1 and fills B1(t + 2) in phase 2 with B0 and A0).
//   A quarter is refilled only in a phase after both groups read it (group 1 runs one
//   barrier behind group 0, so its reads of phase k land under group 0's MFMAs of phase
//   k); each fill is about three phases ahead of its first read. Before each barrier a
//   wave waits for all but its 8 newest fill instructions: in issue order the four
//   quarters after the one the next phase reads. (Four phases of one block each, the
//   reference's pp order, ran 3-7% slower: twice the barriers for the same MFMAs.)
// * Tiles follow one another without a break in the fills (K-tile indices run on across
//   the workgroup's tiles); the epilogue stores from the accumulators after the tile's
//   last phase. A tile's bias reaches LDS by DMA during the tile before it (three slots
//   by tile), so the epilogue's reads wait for no fill.
//
// The MX form (fp8 with E8M0 block scales, bf16 C): each K-tile's 4 scale bytes a row reach
// LDS with the B0 fill of every 4th K-tile, 16 bytes a row, through three rotating buffers;
// lane group g of a 16 x 16 x 128 MFMA passes its fragment row's byte for 32-K block g.
//
// The paired form (C = silu(gate) * up, B's gate and up rows pair_off apart) reads 64 gate
// and 64 up rows a B quarter, so a wave's two 16-row B fragments of a block are the gate
// and up rows of the same 16 C columns; a tile is 128 C columns.
//
// Ragged M and N read zeros through the operands' buffer bounds; C's stores are dropped
// past M by its buffer bound and predicated on n < N (N % 8 == 0).
#pragma once

#include <type_traits>

#include "hkx_ring.hpp"

namespace hkx {

template <int ACT, int EPF, bool PAIR = false, bool FP8 = false, bool MX = false, int BM = 256,
          bool SHARE = false>
__global__ void __launch_bounds__(512, 1) quad_kernel(const TileArgs p) {
  constexpr int BN = PAIR ? 128 : 256;  // BN: C columns of a tile
  static_assert(BM == 256 || (BM == 128 && !FP8 && !MX), "128-row tiles: bf16 only");
  // SHARE: K split over blockIdx.y, each split's fp32 sums stored as they are (a later pass
  // adds the splits in order and applies the epilogue)
  static_assert(!SHARE || (BM == 256 && !PAIR && !MX && EPF == kEpNone && ACT == HKX_ACT_NONE),
                "fp32 shares: 256-row tiles, unpaired, no epilogue");
  constexpr int NI = BM / 128;          // A halves of a tile
  constexpr int QPS = NI + 2;           // quarters a K-tile slot: the A halves, B0, B1
  constexpr int NSL = NI == 2 ? 2 : 3;  // K-tile slots
  constexpr int QB = 128 * 128;         // one quarter: 128 rows x 128 bytes
  constexpr int EPV = NSL * QPS * QB;   // then the epilogue's vectors: [tile % 3][cs, rs, ra][1 KB]
  // MX: in their place, E8M0 scale chunks [chunk % 3][512 rows: A, then B][16 bytes]; a chunk
  // the scales of 4 K-tiles (16 blocks of 32 K) of every row of the tile
  constexpr int SCO = EPV;
  constexpr int SMEM = EPV + (MX ? 3 * 8192 : 3 * 3 * 1024);
  static_assert(!MX || (FP8 && EPF == kEpNone), "MX scales go with fp8 operands, no epilogue");
  static_assert(FP8 ? (EPF == kEpNone || EPF == kEpDeq || EPF == kEpDeqBias) && ACT == HKX_ACT_NONE
                    : (EPF == kEpNone || EPF == kEpBias || EPF == kEpTile), "forms");
  static_assert(!PAIR || (!FP8 && EPF == kEpNone && ACT == HKX_ACT_NONE), "the paired form is silu * up");
  static_assert(SMEM <= 160 * 1024, "LDS");

  // Fragments are 16 x 16: bf16 on v_mfma_f32_16x16x32_bf16, fp8 (plain and MX) on
  // v_mfma_scale_f32_16x16x128_f8f6f4, the K-tile's 128 bytes in one MFMA. The fp8 16 x 16 x 128
  // MFMA runs 9% more flops than 32 x 32 x 64 on random operands under the board's power
  // limit (4.34 against 3.97 PFLOP/s, a register-only loop on one box), for the same operand
  // registers, accumulators and LDS reads a K-tile.
  constexpr int KH = FP8 ? 1 : 2;  // MFMA K-steps a fragment a K-tile

  __shared__ __attribute__((aligned(16))) uint8_t smem[SMEM];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2;  // the ping-pong group and the wave's grid row
  const int wc = wave & 3;

  const int total = p.tiles_m * p.tiles_n;
  const int G = gridDim.x;
  const int my_tiles = (total - (int)blockIdx.x + G - 1) / G;
  const int kt0 = SHARE ? (int)blockIdx.y * p.kt_split : 0;  // this split's first K-tile
  const int nkt = SHARE ? min(p.kt_split, p.kt_total - kt0) : p.kt_total;  // K-tiles a tile
  const int nu = my_tiles * nkt;  // K-tiles of this workgroup

  // tile (m0, n0) of local tile lt: the ring kernel's XCD-chunked grouped raster
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
    n0 = (in / gm) * BN;
  };

  // ---- fills. Instruction k (0, 1) of wave w moves block 2 w + k of a quarter (rows
  // 16 w + 8 k + [0, 8)); lane l fetches row 16 w + 8 k + l % 32 / 4, K-half l / 32, its
  // 16-byte chunk (l % 4) ^ swz4(row) -- swz4 of those rows is (w & 1) | (k << 1).
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a, p.a_bytes);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.b, p.b_bytes);
  // Paired (gate | up, B has 2N rows): B tile row 16 F + x is row x of the gate (F even) or
  // up (F odd) block of C columns 16 (F / 2) ..: quarter h's row 16 w + x, F = 8 h + w, is
  // B row n0 + 64 h + 16 (w / 2) + x (+ pair_off for odd w).
  uint32_t lrow[2], lrow_b[2], lch[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    lrow[k] = (uint32_t)(16 * wave + 8 * k + (lane & 31) / 4);
    lrow_b[k] = PAIR ? (uint32_t)(16 * (wave >> 1) + 8 * k + (lane & 31) / 4 +
                                  ((wave & 1) ? p.pair_off : 0))
                     : lrow[k];
    lch[k] = (uint32_t)(64 * (lane >> 5) + 16 * ((lane & 3) ^ ((wave & 1) | (k << 1))));
  }
  // Two fill streams walk the workgroup's K-tiles: one a K-tile ahead (A1 of t + 1), one
  // two ahead (B0, A0, B1 of t + 2); each keeps its K-tile's index, position in its tile
  // and tile origin. Past the last K-tile a stream stays on it: its fills fetch the same
  // bytes again into the slot that K-tile already holds.
  struct Stream {
    int g, t, lt, m0, n0;
  };
  auto stream_at = [&](int g0) {
    Stream s{0, 0, 0, 0, 0};
    s.g = min(g0, nu - 1);
    s.lt = s.g / nkt;
    s.t = s.g - s.lt * nkt;
    tile_at(s.lt, s.m0, s.n0);
    return s;
  };
  auto advance = [&](Stream& s) {
    if (s.g + 1 >= nu) return;
    ++s.g;
    if (++s.t == nkt) {
      s.t = 0;
      tile_at(++s.lt, s.m0, s.n0);
    }
  };
  // quarter q (0 A0, 1 A1, 2 B0, 3 B1) of slot sl
  auto slot_of = [](int g) { return NSL == 2 ? (g & 1) : g % NSL; };
  auto quarter = [&](int sl, int q) { return smem + (sl * QPS + (q < 2 ? q : NI + q - 2)) * QB; };
  // quarter q of stream s's K-tile into its slot
  auto fill = [&](int q, const Stream& s) {
    const bool isb = q >= 2;
    const uint32_t ld = isb ? p.ldb_b : p.lda_b;
    const uint32_t row0 = (uint32_t)((isb ? s.n0 : s.m0) + (isb && PAIR ? 64 : 128) * (q & 1));
    const uint32_t so = __builtin_amdgcn_readfirstlane(row0 * ld + (uint32_t)(kt0 + s.t) * 128u);
    uint8_t* base = quarter(slot_of(s.g), q) + wave * 2048;
#pragma unroll
    for (int k = 0; k < 2; ++k)
      buf_load16_lds(isb ? rb : ra, base + k * 1024, (isb ? lrow_b[k] : lrow[k]) * ld + lch[k], so);
  };

  // ---- MX scales: with the B0 fill of a chunk's first K-tile, wave w moves 16 bytes of each
  // of rows 64 w + [0, 64) (A rows, then B) -- the chunk's 16 blocks -- into buffer
  // (chunk) % 3. A chunk is read at its K-tiles' first phases; its buffer is refilled three
  // chunks on, at the earliest a K-tile after its last read.
  const int cpt = (nkt + 3) >> 2;  // chunks a tile
  const __amdgpu_buffer_rsrc_t rsc = make_rsrc(MX ? (wave < 4 ? p.sa : p.sb) : nullptr,
                                               MX ? (wave < 4 ? p.sa_bytes : p.sb_bytes) : 0u);
  auto scale_fill = [&](const Stream& st) {
    if constexpr (MX) {
      if (st.t & 3) return;
      const int chunk = st.lt * cpt + (st.t >> 2);
      const uint32_t row = (uint32_t)((wave < 4 ? st.m0 : st.n0) + 64 * (wave & 3) + lane);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rsc, (__attribute__((address_space(3))) void*)(smem + SCO + (chunk % 3) * 8192 + wave * 1024), 16,
          row * (wave < 4 ? p.sa_ld : p.sb_ld), __builtin_amdgcn_readfirstlane((uint32_t)st.t * 4u), 0, 0);
    }
  };

  // ---- the epilogue's vectors of local tile lt by 16-byte DMA into slot lt % 3: the row
  // scale (256 fp32, wave 0), the column scale (256 fp32, wave 1), the bias (256 bf16, wave
  // 2; lanes 32-63 read past the tile's 512 bytes into the slot's spare half). Three slots:
  // the DMA of tile lt + 1, at tile lt's first phase, runs while group 1 may still read
  // tile lt - 1's.
  // kEpTile: the bias is optional (absent, its DMA reads zeros from an empty buffer)
  constexpr bool bias = EPF == kEpBias || EPF == kEpDeqBias || EPF == kEpTile;
  constexpr bool deq = EPF == kEpDeq || EPF == kEpDeqBias;
  const Fused& e = p.ep;
  const __amdgpu_buffer_rsrc_t rvec = make_rsrc(
      wave == 0 ? (deq ? e.cs.p : nullptr) : wave == 1 ? (deq ? e.rs.p : nullptr) : (bias ? e.ra.p : nullptr),
      wave == 0 ? (deq ? (uint32_t)p.M * 4u : 0u)
                : wave == 1 ? (deq ? (uint32_t)p.N * 4u : 0u) : (bias && e.ra.p ? (uint32_t)p.N * 2u : 0u));
  // a scale of one value (stride 0) is read once here, before any fill (a read after the
  // fills would wait for all of them), and has no DMA
  const bool cs_bc = deq && e.cs.ld == 0, rs_bc = deq && e.rs.ld == 0;
  [[maybe_unused]] const float cs0 = cs_bc ? ld1(e.cs.p, HKX_FP32, 0) : 1.0f;
  [[maybe_unused]] const float rs0 = rs_bc ? ld1(e.rs.p, HKX_FP32, 0) : 1.0f;
  auto vec_load = [&](int lt) {
    if (wave > 2 || (wave < 2 && !deq) || (wave == 2 && !bias)) return;
    if ((wave == 0 && cs_bc) || (wave == 1 && rs_bc)) return;
    int m0, n0;
    tile_at(lt, m0, n0);
    const uint32_t so = wave == 0 ? (uint32_t)m0 * 4u : wave == 1 ? (uint32_t)n0 * 4u : (uint32_t)n0 * 2u;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rvec, (__attribute__((address_space(3))) void*)(smem + EPV + (lt % 3) * 3072 + wave * 1024), 16,
        (uint32_t)lane * 16u, __builtin_amdgcn_readfirstlane(so), 0, 0);
  };

  // ---- fragment reads. Lane l reads row l % 16 of a 16-row fragment, 16-byte chunk l / 16
  // of a K-half; a fragment of quarter rows r0.. (r0 % 16 == 0) at K-half s sits at
  // r0 * 128 + s * 512 + rdo[(r0 >> 4) & 1]. bf16 (16 x 16 x 32) takes one K-half an MFMA;
  // fp8 (16 x 16 x 128) the chunk of both, the MFMA taking a lane's bytes 0-15 as K
  // 16 (l / 16) + [0, 16) and bytes 16-31 as K 64 + 16 (l / 16) + [0, 16) -- so lane group
  // l / 16 holds half of each of the K-tile's 32-K blocks l / 16 / 2 and 2 + l / 16 / 2, and
  // the MX form's scale of 32-K block b comes from lane group b.
  uint32_t rdo[2];
  {
    const int rr = lane & 15, q = lane >> 4;
#pragma unroll
    for (int par = 0; par < 2; ++par)
      rdo[par] = (uint32_t)((rr >> 3) * 1024 + (rr & 7) * 64 + ((q ^ (par | ((rr >> 3) << 1))) << 4));
  }
  constexpr int NA = 4, NB = 2;  // 16-row fragments of a block's 64 A rows and 32 B rows
  using Frag = typename std::conditional<FP8, i32x8, bf16x8>::type;
  // [fragment][K-half]; bfn: B1 of the next K-tile (see the K loop)
  Frag af[NA][2], bf0[NB][2], bf1[NB][2], bfn[NB][2];
  auto frag_at = [&](const uint8_t* s, int r0, int h, int par) -> Frag {
    if constexpr (FP8) {
      // 16 x 16 x 128: the bf16 fragment's 16-byte chunk of both K-halves, so lane l holds
      // K 16 (l / 16) + [0, 16) and 64 + 16 (l / 16) + [0, 16) of row l % 16 -- in A and B
      // alike, which is all a dot product needs of the K order
      const i32x4 lo = *(const i32x4*)(s + r0 * 128 + rdo[par]);
      const i32x4 hi = *(const i32x4*)(s + r0 * 128 + 512 + rdo[par]);
      return i32x8{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
    } else {
      return *(const bf16x8*)(s + r0 * 128 + h * 512 + rdo[par]);
    }
  };
  auto read_a = [&](int slot, int i) {
    const uint8_t* s = quarter(slot, i);
#pragma unroll
    for (int f = 0; f < NA; ++f)
#pragma unroll
      for (int h = 0; h < KH; ++h) af[f][h] = frag_at(s, grp * 64 + (64 / NA) * f, h, f & 1);
  };
  auto read_b = [&](int slot, int j, Frag (&bf)[NB][2]) {
    const uint8_t* s = quarter(slot, 2 + j);
#pragma unroll
    for (int g = 0; g < NB; ++g)
#pragma unroll
      for (int h = 0; h < KH; ++h) bf[g][h] = frag_at(s, wc * 32 + 16 * g, h, g & 1);
  };

  // MX: the E8M0 dword of each of this lane's fragment rows for the K-tile (its 4 blocks,
  // byte b for 32-K block b), read at the K-tile's first phase and shifted down by lane group
  // (l / 16) bytes, so every lane's byte 0 is the scale of the block its group supplies
  [[maybe_unused]] uint32_t sca[2][4], scb[2][2];  // [A half][fragment], [B half][fragment]
  const int sc_sh = 8 * (lane >> 4);
  auto read_scales = [&](int lt, int t) {
    if constexpr (MX) {
      const uint32_t* sc = (const uint32_t*)(smem + SCO + ((lt * cpt + (t >> 2)) % 3) * 8192) + (t & 3);
      const int rf = lane & 15;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int f = 0; f < 4; ++f) sca[i][f] = sc[4 * (128 * i + 64 * grp + 16 * f + rf)] >> sc_sh;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int g = 0; g < 2; ++g) scb[j][g] = sc[4 * (256 + 128 * j + 32 * wc + 16 * g + rf)] >> sc_sh;
    }
  };

  using Acc = f32x4;
  Acc acc[NI][2][NA][NB];  // [A half][B half][row fragment][column fragment]
  auto math = [&](int i, int j, const Frag (&bf)[NB][2], bool zero) {
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int h = 0; h < KH; ++h)
#pragma unroll
      for (int f = 0; f < NA; ++f)
#pragma unroll
        for (int g = 0; g < NB; ++g) {
          const Acc c = (zero && h == 0) ? Acc{} : acc[i][j][f][g];
          if constexpr (MX)
            acc[i][j][f][g] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                bf[g][h], af[f][h], c, 0, 0, 0, (int)scb[j][g], 0, (int)sca[i][f]);
          else if constexpr (FP8)
            acc[i][j][f][g] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bf[g][h], af[f][h], c, 0, 0, 0,
                                                                               0, 0, 0);
          else
            acc[i][j][f][g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf[g][h], af[f][h], c, 0, 0, 0);
        }
    __builtin_amdgcn_s_setprio(0);
  };

  // ---- the epilogue of local tile lt from the accumulators. Lane l (row l % 16, quarter
  // q = l / 16) holds columns 4 q + [0, 4) of each 16-column fragment; the two fragments
  // of a 32-column block trade quarters (v_permlane16_swap) so each lane stores 16
  // contiguous bytes.
  const uint32_t row_b = (uint32_t)p.ldc * (SHARE ? 4u : 2u);
  const __amdgpu_buffer_rsrc_t rc = make_rsrc(
      SHARE ? (const void*)((const float*)p.c + (int64_t)blockIdx.y * p.split_stride) : p.c,
      (uint32_t)p.M * row_b);
  auto store_c = [&](i32x4 v, bool in_n, uint32_t off) {
    if (in_n) __builtin_amdgcn_raw_buffer_store_b128(v, rc, off, 0, 0);
  };
  auto epilogue = [&](int lt) {
    int m0, n0;
    tile_at(lt, m0, n0);
    const uint8_t* ev = smem + EPV + (lt % 3) * 3072;  // cs, rs, ra
    if constexpr (SHARE) {
      // the split's fp32 sums, 16 bytes a lane (16 x 16 fragments; the split form is never
      // MX): lane (rf, q) holds row rf, columns 4 q + [0, 4) of each fragment
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int f = 0; f < NA; ++f)
#pragma unroll
            for (int g = 0; g < NB; ++g) {
              __builtin_amdgcn_sched_barrier(0);
              const int ml = 128 * i + 64 * grp + 16 * f + (lane & 15);
              const int n = n0 + 128 * j + 32 * wc + 16 * g + 4 * (lane >> 4);
              store_c(__builtin_bit_cast(i32x4, acc[i][j][f][g]), n < p.N,
                      (uint32_t)(m0 + ml) * row_b + (uint32_t)n * 4u);
            }
      return;
    }
    const int rf = lane & 15, q = lane >> 4;
    // fp8 dequant: this lane's row scales [i][f] (row 128 i + 64 grp + 16 f + rf) and the
    // column scales of its columns [j][g] (as the bias), read once a tile
    [[maybe_unused]] float rsc[NI][4];
    [[maybe_unused]] f32x4 csc[2][2];
    if constexpr (deq) {
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int f = 0; f < 4; ++f) rsc[i][f] = cs_bc ? cs0 : ((const float*)ev)[128 * i + 64 * grp + 16 * f + rf];
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          const int col = 128 * j + 32 * wc + 16 * g + 4 * q;
          csc[j][g] = rs_bc ? f32x4{rs0, rs0, rs0, rs0} : *(const f32x4*)(ev + 1024 + col * 4);
        }
    }
    [[maybe_unused]] f32x4 bv[2][2];
    if constexpr (bias) {
      const uint32_t* bs = (const uint32_t*)(ev + 2048);
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          const int col = 128 * j + 32 * wc + 16 * g + 4 * q;  // even: a whole word pair
          bv[j][g] = unpack_bf16x4(*(const u32x2*)(bs + col / 2));
        }
    }
    if constexpr (PAIR) {
      // fragment 0 of a block holds the gate rows, fragment 1 the up rows of C columns
      // 64 j + 16 c + [0, 16): lane l's four at 4 q. Row fragments f = 2 p and 2 p + 1 then
      // trade 16-lane rows (v_permlane16_swap), so a lane holds 8 columns: lanes 0-15 the
      // columns 0-7 of fragment 2 p's rows, 16-31 those of 2 p + 1's, 32-47 and 48-63
      // columns 8-15 of each; one 16-byte store covers 32 rows x 32 bytes (a 33 MB burst of
      // C: 2.9 TB/s, against 2.5 for the 8-byte stores of 16 rows x 32 bytes)
      const int n = 64 * 0 + 16 * wc + 8 * (lane >> 5);
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int fp = 0; fp < 2; ++fp) {
            __builtin_amdgcn_sched_barrier(0);
            u32x2 wa = pack4<2>(HKX_BF16, silu_mul4(acc[i][j][2 * fp][0], acc[i][j][2 * fp][1]));
            u32x2 wb = pack4<2>(HKX_BF16, silu_mul4(acc[i][j][2 * fp + 1][0], acc[i][j][2 * fp + 1][1]));
            uint32_t ax = wa.x, ay = wa.y, bx = wb.x, by = wb.y;
            swap16(ax, bx);
            swap16(ay, by);
            const int nn = 64 * j + n;
            const int ml = 128 * i + 64 * grp + 32 * fp + 16 * ((lane >> 4) & 1) + rf;
            store_c(i32x4{(int)ax, (int)ay, (int)bx, (int)by}, n0 + nn < p.N,
                    (uint32_t)(m0 + ml) * row_b + (uint32_t)(n0 + nn) * 2u);
          }
      return;
    }
    // kEpTile: this lane's 128 values of the tile operand (bf16 rows of stride ta.ld, 16-byte
    // aligned), all loaded before the first store so one memory latency covers them: for
    // fragment (i, j, f), row 128 i + 64 grp + 16 f + rf, columns ca + 4 q and ca + 16 + 4 q
    // (+ [0, 4)); rows past M read zeros through the buffer bound and are never stored
    [[maybe_unused]] u32x2 tv[NI][2][4][2];
    if constexpr (EPF == kEpTile) {
      const uint32_t tb = (uint32_t)e.ta.ld * 2u;
      const __amdgpu_buffer_rsrc_t rt = make_rsrc(e.ta.p, (uint32_t)p.M * tb);
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int f = 0; f < 4; ++f)
#pragma unroll
            for (int g = 0; g < 2; ++g) {
              const int col = n0 + 128 * j + 32 * wc + 16 * g + 4 * q;
              const int row = m0 + 128 * i + 64 * grp + 16 * f + rf;
              tv[i][j][f][g] = __builtin_bit_cast(
                  u32x2, __builtin_amdgcn_raw_buffer_load_b64(rt, (uint32_t)row * tb + (uint32_t)col * 2u, 0, 0));
            }
    }
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int ca = 128 * j + 32 * wc;  // the block's first column
#pragma unroll
        for (int f = 0; f < 4; ++f) {
          __builtin_amdgcn_sched_barrier(0);
          f32x4 va = acc[i][j][f][0], vb = acc[i][j][f][1];
          if constexpr (deq) {
            va = va * (csc[j][0] * rsc[i][f]);
            vb = vb * (csc[j][1] * rsc[i][f]);
          }
          if constexpr (bias) {
            va += bv[j][0];
            vb += bv[j][1];
          }
          if constexpr (EPF == kEpTile) {
            va += unpack_bf16x4(tv[i][j][f][0]);
            vb += unpack_bf16x4(tv[i][j][f][1]);
          }
          va = act4c<ACT>(0, va);
          vb = act4c<ACT>(0, vb);
          const u32x2 wa = pack4<2>(HKX_BF16, va), wb = pack4<2>(HKX_BF16, vb);
          uint32_t x0 = wa.x, x1 = wb.x, y0 = wa.y, y1 = wb.y;
          swap16(x0, x1);
          swap16(y0, y1);
          const int n = ca + 16 * (q & 1) + 8 * (q >> 1);
          const int ml = 128 * i + 64 * grp + 16 * f + rf;
          store_c(i32x4{(int)x0, (int)y0, (int)x1, (int)y1}, n0 + n < p.N,
                  (uint32_t)(m0 + ml) * row_b + (uint32_t)(n0 + n) * 2u);
        }
      }
  };

  // ---- the K loop. Before the first phase: K-tile 0 whole and K-tile 1 but A1, in the
  // order the steady state issues them (B0, B1, A0 of t + 2 in phase 2 of t, A1 of t + 1
  // in phase 1 of t).
  auto sync_mem = [&]() {  // before a math phase: this wave's LDS reads landed
    __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(8));
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
  };
  auto sync_math = [&]() {  // before a memory phase: the quarters it reads landed everywhere
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(wait_vm(8));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
  };
  if constexpr (NI == 1) {
    // 128-row tiles: one phase a K-tile (read A0, B0, B1; math (0, 0), (0, 1)) through three
    // slots. Phase t fills K-tile t + 2 into the slot of K-tile t - 1, which group 0 read a
    // phase and group 1 a barrier before; each fill lands three to four barriers ahead of its
    // first read. A wave issues 6 fill instructions a phase, so before each barrier it waits
    // for all but its 6 newest: those of K-tile t + 2.
    auto sync6 = [&](bool lds) {
      __builtin_amdgcn_sched_barrier(0);
      if (lds) __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(6));
      else __builtin_amdgcn_s_waitcnt(wait_vm(6));
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
    };
    vec_load(0);
    Stream s2 = stream_at(0);
#pragma unroll
    for (int r = 0; r < 2; ++r) {  // K-tiles 0 and 1, in steady-state order
      fill(2, s2);
      fill(3, s2);
      fill(0, s2);
      advance(s2);
    }
    __builtin_amdgcn_s_waitcnt(wait_vm(6));  // K-tile 0
    __builtin_amdgcn_s_barrier();
    if (grp == 1) __builtin_amdgcn_s_barrier();
    int g = 0;
    for (int lt = 0; lt < my_tiles; ++lt) {
      for (int t = 0; t < nkt; ++t, ++g) {
        const int slot = slot_of(g);
        const bool z = t == 0;
        read_a(slot, 0);
        read_b(slot, 0, bf0);
        read_b(slot, 1, bf1);
        if (t == 0 && lt + 1 < my_tiles) vec_load(lt + 1);
        fill(2, s2);
        fill(3, s2);
        fill(0, s2);
        advance(s2);
        sync6(true);
        math(0, 0, bf0, z);
        math(0, 1, bf1, z);
        sync6(false);
      }
      epilogue(lt);
    }
  } else {
  // Without MX, phase 2 also reads B1 of the next K-tile (into the other of bf1 / bfn, the
    // two alternating by K-tile) and B1's fill moves to phase 1, two K-tiles ahead: each phase
    // then reads 12 fragments and issues 4 fills, where phase 1 read 16 and issued 2 (config 2
    // 1-3% faster). Every quarter is still refilled only after both groups read it and about
    // three phases before its first read, and the fills keep the order of their reads, so the
    // waits stay "all but the newest 8". The MX form keeps B1 in phase 1: its scales leave
    // no registers for the second B1 set.
    constexpr bool B1N = !MX;
    vec_load(0);
    Stream s1 = stream_at(0), s2 = stream_at(0);
#pragma unroll
    for (int r = 0; r < 2; ++r) {  // K-tile 0 whole, then K-tile 1 but A1, in steady-state order
      if constexpr (B1N) fill(3, s2);
      fill(2, s2);
      scale_fill(s2);
      if constexpr (!B1N) fill(3, s2);
      fill(0, s2);
      if (r == 0) {
        fill(1, s1);
        advance(s1);
      }
      advance(s2);
    }
    __builtin_amdgcn_s_waitcnt(wait_vm(8));  // A0, B0 and B1 of K-tile 0
    __builtin_amdgcn_s_barrier();
    if constexpr (B1N) {  // B1 of K-tile 0, read by every wave before any refill of it
      read_b(0, 1, bf1);
      __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(8));
      __builtin_amdgcn_s_barrier();
    }
    if (grp == 1) __builtin_amdgcn_s_barrier();
    // K-tile t of local tile lt, the workgroup's g-th: b1 holds its B1 fragments, nb1 takes
    // the next K-tile's (B1N)
    // Group 1 runs a tile's epilogue before the barrier that ends its last math phase, not
    // after it: the two groups' epilogues then overlap (one group's VALU work under the
    // other's stores), where group 0's epilogue used to hold group 1 at that barrier for the
    // epilogue's whole length (config 5 1.2%, config 2 0.6% faster, same box). Nothing in
    // between reads LDS but the epilogue's own vector slot, which no fill of that interval
    // touches. (The MX form keeps the plain order: the early epilogue made it 9-14% slower,
    // same box, 2048-8192 rows.)
    constexpr bool EARLY = !MX;
    auto ktile = [&](int lt, int t, int g, Frag (&b1)[NB][2], Frag (&nb1)[NB][2]) {
      const int slot = g & 1;
      const bool z = t == 0;
      const bool last_g1 = EARLY && grp == 1 && t == nkt - 1;
      // phase 1
      read_a(slot, 0);
      read_b(slot, 0, bf0);
      if constexpr (!B1N) read_b(slot, 1, b1);
      read_scales(lt, t);
      if (t == 0 && lt + 1 < my_tiles) vec_load(lt + 1);
      fill(1, s1);
      advance(s1);
      if constexpr (B1N) fill(3, s2);
      sync_mem();
      math(0, 0, bf0, z);
      math(0, 1, b1, z);
      sync_math();
      // phase 2
      read_a(slot, 1);
      if constexpr (B1N) read_b(slot ^ 1, 1, nb1);
      fill(2, s2);
      scale_fill(s2);
      if constexpr (!B1N) fill(3, s2);
      fill(0, s2);
      advance(s2);
      sync_mem();
      math(1, 0, bf0, z);
      math(1, 1, b1, z);
      if (!last_g1) sync_math();
    };
    int g = 0;
    for (int lt = 0; lt < my_tiles; ++lt) {
      if constexpr (B1N) {
        int t = 0;
        for (; t + 1 < nkt; t += 2, g += 2) {
          ktile(lt, t, g, bf1, bfn);
          ktile(lt, t + 1, g + 1, bfn, bf1);
        }
        if (t < nkt) {  // an odd count: the last K-tile, and the next tile's B1 back in bf1
          ktile(lt, t, g++, bf1, bfn);
#pragma unroll
          for (int f = 0; f < NB; ++f)
#pragma unroll
            for (int h = 0; h < 2; ++h) bf1[f][h] = bfn[f][h];
        }
      } else {
        for (int t = 0; t < nkt; ++t, ++g) ktile(lt, t, g, bf1, bf1);
      }
      epilogue(lt);
      if (EARLY && grp == 1) sync_math();  // its last math phase's barrier, after the epilogue
    }
  }
  if (grp == 0) __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_s_waitcnt(wait_vm(0));  // no fill lands in LDS after the exit
}

}  // namespace hkx
