// The LDS-tiled MFMA GEMM for gfx950: C tile (BM x BN) = epilogue(A . B^T), 8 waves.
//
// Replaces the reference's gfx950 GEMM kernels (python/hk/ops/gemm_cdna.py:57-586, the
// 256x256 pingpong, and python/hk/ops/gemm_cdna_dp.py:30-243, the small-grid blocks and
// their split-K shares) with one hand-written kernel template:
//
// * Operands: A (M, K) and B (N, K), both K-contiguous. One stage of the K loop is one
//   128-byte slice of every row -- 64 bf16 or 128 fp8 elements -- so bf16 and fp8 share
//   the LDS layout and the loader, and differ only in the MFMA.
// * Loads: 16-byte raw buffer loads (a buffer resource per operand bounds them: rows past
//   M or N read 0), each wave instruction 8 whole 128-byte row slices, coalesced.
// * LDS: two stages of (BM + BN) x 128 bytes. A row's eight 16-byte chunks are stored
//   XOR-swizzled (chunk c of row r at c ^ swz(r % 16)), so the MFMA operand reads --
//   16 rows, one chunk each -- hit distinct banks. The loader writes the swizzle: thread
//   t's chunk lands at byte 16 t of its 8 KB slab, which is a plain, conflict-free store.
// * MFMA: v_mfma_f32_16x16x32_bf16 (bf16) or v_mfma_f32_16x16x128_f8f6f4 (fp8 e4m3),
//   with B's fragment as the first operand, so each lane's four accumulators are four
//   consecutive columns of one row of C -- the layout the epilogue loads and the store
//   packs want (a bias is one 8-byte load, a bf16 result one 8-byte write).
// * Waves: WM x (8 / WM), each a (BM / WM) x (BN * WM / 8) sub-tile of 16 x 16 fragments.
// * Epilogue: applied to the fp32 accumulators in registers, converted once, staged
//   through LDS and stored as 16-byte rows of C (fp32 C and split-K shares are stored
//   from registers, 16 bytes a lane).
// * Blocks: an XCD-aware renumbering (workgroup ids go round-robin over the 8 XCDs;
//   consecutive logical tiles are put on one XCD so they share its L2), then a grouped
//   raster of `wgm` tile rows.
#pragma once

#include "hkx_device.hpp"

namespace hkx {

struct TileArgs {
  const void* a;
  const void* b;
  void* c;             // C, or the fp32 shares (MODE kStoreF32 / kPairWs)
  uint32_t a_bytes;    // bounds of A and B for the buffer resources
  uint32_t b_bytes;
  uint32_t lda_b;      // row strides in bytes
  uint32_t ldb_b;
  int64_t ldc;         // elements
  int64_t split_stride;  // elements between split shares (0: C itself)
  int32_t M, N;        // C's shape (the paired form: N output columns, B has 2N rows)
  int32_t kt_total;    // 128-byte K stages in all
  int32_t kt_split;    // per split (blockIdx.y)
  int32_t tiles_m, tiles_n, wgm;
  int32_t pair_off;    // B rows from a gate row to its up row (paired form)
  int32_t c_dt;
  int32_t c_aligned;   // C's rows are 16-byte aligned: whole-chunk stores
  Fused ep;
  // MX block scales (the ring kernel's MX form): E8M0 bytes, one a row and 32 K, row
  // strides in bytes; bounds in bytes for the buffer resources
  const uint8_t* sa;
  const uint8_t* sb;
  uint32_t sa_ld, sb_ld;
  uint32_t sa_bytes, sb_bytes;
  // fp8 operand formats: 1 e4m3 x e4m3, 2 e5m2 x e5m2, 3 A e4m3 x B e5m2, 4 A e5m2 x B e4m3
  // (0 for bf16); formats past 1 run on the ring kernel only
  int32_t ab_fmt;
  // A K split finished in the kernel (MODE kStoreF32 with split shares): one arrival
  // counter a tile (blockIdx.x), zero before the call and left at zero; the last split to
  // arrive sums the shares into fin_c (row stride fin_ldc, type fin_dt) with fin_ep.
  // cnt == nullptr: the shares stay for the reduction pass.
  int32_t* cnt;
  void* fin_c;
  int64_t fin_ldc;
  int32_t fin_dt;
  Fused fin_ep;
};

// How a tile leaves the kernel.
constexpr int kStore16 = 0;   // 16-bit C, through LDS staging
constexpr int kStore8 = 1;    // 8-bit C (int8, fp8), through LDS staging
constexpr int kStoreF32 = 2;  // fp32 C or fp32 split shares, from registers
constexpr int kPair16 = 3;    // silu(gate) * up, 16-bit C, through LDS staging
constexpr int kPairWs = 4;    // gate and up fp32 shares, (M, 2N) per split

HKX_DEV int swz(int j) { return (j ^ (j >> 3)) & 7; }

// A split share's four fp32 values, stored and loaded through a buffer resource over the
// split's share with the device-scope coherence bit (sc1, cache policy 16): coherent
// across the XCDs' L2s without a cache-wide fence, which a workgroup's finish of a split
// cannot afford (a device-scope fence writes back and invalidates the whole L2). Byte
// offsets from the share's start, which the host keeps under 4 GiB.
constexpr int kCpolSc1 = 16;

HKX_DEV void share_store4(__amdgpu_buffer_rsrc_t r, uint32_t off, f32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, v), r, off, 0, kCpolSc1);
}

HKX_DEV f32x4 share_load4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCpolSc1));
}

// After a workgroup stored its split's share of tile `tile` (rows m0.., columns n0.. of
// a BM x OW tile; NT threads): its arrival at the tile's counter, and, if it is the last
// of the gridDim.y splits, the tile's finish -- the shares summed in split order (the
// reduction pass's order, so the result does not depend on which split arrives last),
// the fused epilogue, the store, and the counter back to zero for the next call. Every
// thread of the workgroup calls it. The reference finishes its stream-K and decode splits
// the same way (python/hk/ops/gemm_cdna.py:421-496, python/hk/ops/decode_gemm.py:155-170).
// The finish's sums and stores with S (a compile-time split count, or 0: run time) shares:
// each thread takes groups tid, tid + NT, ... of four columns and issues the loads of up to
// 16 share pieces before adding any (so it waits a memory latency per 16 loads, not one a
// group: issued group by group, the finish of a 64 x 128 tile split 4 ways cost 9 us).
template <int BM, int OW, int NT, int S>
HKX_DEV void finish_sums(const TileArgs& p, __amdgpu_buffer_rsrc_t r, uint32_t sb, int m0, int n0) {
  constexpr int IT = BM * OW / 4 / NT;  // groups a thread
  constexpr int SS = S > 0 ? S : 1;
  constexpr int CH = S == 0 ? 1 : ((16 / SS) < 1 ? 1 : ((16 / SS) > IT ? IT : 16 / SS));
  const int splits = S > 0 ? S : (int)gridDim.y;
  for (int base = 0; base < IT; base += CH) {
    f32x4 x[CH][SS];
    uint32_t off[CH];
    bool ok[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int q = (int)threadIdx.x + (base + c) * NT;
      const int row = q / (OW / 4), c4 = q - row * (OW / 4);
      const int m = m0 + row, n = n0 + 4 * c4;
      ok[c] = base + c < IT && m < p.M && n < p.N;
      off[c] = ((uint32_t)m * (uint32_t)p.ldc + (uint32_t)n) * 4u;
      if constexpr (S > 0) {
#pragma unroll
        for (int s = 0; s < S; ++s) x[c][s] = ok[c] ? share_load4(r, off[c] + (uint32_t)s * sb) : f32x4{};
      }
    }
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      if (!ok[c]) continue;
      f32x4 v;
      if constexpr (S > 0) {
        v = x[c][0];
#pragma unroll
        for (int s = 1; s < S; ++s) v += x[c][s];
      } else {
        v = share_load4(r, off[c]);
        for (int s = 1; s < splits; ++s) v += share_load4(r, off[c] + (uint32_t)s * sb);
      }
      const int q = (int)threadIdx.x + (base + c) * NT;
      const int row = q / (OW / 4), c4 = q - row * (OW / 4);
      const int m = m0 + row, n = n0 + 4 * c4;
      v = fused_apply(p.fin_ep, v, m, n, true);
      store4(p.fin_c, p.fin_dt, (int64_t)m * p.fin_ldc + n, v);
    }
  }
}

template <int BM, int OW, int NT>
HKX_DEV void finish_split(const TileArgs& p, int tile, int m0, int n0, int* last) {
  __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0): this wave's share stores performed
  __syncthreads();
  if (threadIdx.x == 0)
    *last = __hip_atomic_fetch_add(p.cnt + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
            (int)gridDim.y - 1;
  __syncthreads();
  if (!*last) return;
  // (the host keeps all the shares, splits x split_stride floats, under 4 GiB)
  const uint32_t sb = (uint32_t)p.split_stride * 4u;
  const __amdgpu_buffer_rsrc_t r = make_rsrc(p.c, sb * (uint32_t)gridDim.y);
  switch (gridDim.y) {
    case 2: finish_sums<BM, OW, NT, 2>(p, r, sb, m0, n0); break;
    case 3: finish_sums<BM, OW, NT, 3>(p, r, sb, m0, n0); break;
    case 4: finish_sums<BM, OW, NT, 4>(p, r, sb, m0, n0); break;
    case 8: finish_sums<BM, OW, NT, 8>(p, r, sb, m0, n0); break;
    default: finish_sums<BM, OW, NT, 0>(p, r, sb, m0, n0); break;
  }
  if (threadIdx.x == 0) __hip_atomic_store(p.cnt + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The swizzle of rows of four 16-byte chunks (64-byte half-stage rows): chunk c of row r is
// stored at c ^ swz4(r), bits 4 and 3 of the row, which makes the fragment reads of 32
// rows with one chunk each conflict-free.
HKX_DEV int swz4(int r) { return ((r >> 4) & 1) | ((r >> 2) & 2); }

template <int BM, int BN, int WM, bool FP8, int MODE>
__global__ void __launch_bounds__(512, 1) tile_kernel(const TileArgs p) {
  constexpr int WN = 8 / WM;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 16, FN = TN / 16;
  constexpr int ROWS = BM + BN;
  constexpr int NCH = ROWS / 64;  // 16-byte chunks a thread loads per stage
  constexpr int NA = BM / 64;     // of which from A
  constexpr int STAGE = ROWS * 128;
  constexpr bool PAIR = (MODE == kPair16 || MODE == kPairWs);
  constexpr bool STAGED = (MODE == kStore16 || MODE == kStore8 || MODE == kPair16);
  constexpr int OB = (MODE == kStore8) ? 1 : 2;
  constexpr int OUTW = PAIR ? BN / 2 : BN;  // C columns a tile covers
  constexpr int RS = OUTW * OB + 16;        // staging row stride, bytes
  constexpr int STAGING = STAGED ? BM * RS : 0;
  constexpr int SMEM = (2 * STAGE > STAGING) ? 2 * STAGE : STAGING;
  static_assert(WM * WN == 8 && TM % 16 == 0 && TN % 16 == 0, "wave tiling");
  static_assert(BM % 64 == 0 && BN % 64 == 0, "loader tiling");
  static_assert(!PAIR || FN % 2 == 0, "the paired form needs gate/up fragment pairs");
  static_assert(SMEM <= 160 * 1024, "LDS");

  __shared__ __attribute__((aligned(16))) uint8_t smem[SMEM];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;

  // ---- which tile: XCD-chunked renumbering, then a grouped raster
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

  // ---- loader: chunk i of thread t is row (t >> 3) + 64 i of the stage, physical
  // chunk t & 7, which holds logical chunk (t & 7) ^ swz(row & 15) of that row
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a, p.a_bytes);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.b, p.b_bytes);
  const int lrow = tid >> 3;
  const uint32_t lch16 = (uint32_t)(((tid & 7) ^ swz(lrow & 15)) << 4);
  uint32_t voff[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int r = lrow + 64 * i;
    if (i < NA) {
      voff[i] = (uint32_t)(m0 + r) * p.lda_b + lch16;
    } else {
      const int v = r - BM;
      int brow;
      if constexpr (PAIR) {
        const int fv = v >> 4;
        brow = n0 + (fv >> 1) * 16 + (v & 15) + ((fv & 1) ? p.pair_off : 0);
      } else {
        brow = n0 + v;
      }
      voff[i] = (uint32_t)brow * p.ldb_b + lch16;
    }
  }

  // ---- fragment reads: lane l reads row l % 16 of a fragment, k-slot l / 16
  const int rf = lane & 15, kq = lane >> 4;
  const int sw = swz(rf);
  uint32_t rdo0, rdo1;
  if constexpr (FP8) {  // one k-step of 128: the lane's 32 bytes are chunks 2kq, 2kq+1
    rdo0 = rf * 128 + (((2 * kq) ^ sw) << 4);
    rdo1 = rf * 128 + (((2 * kq + 1) ^ sw) << 4);
  } else {  // two k-steps of 32: chunk kq, then 4 + kq
    rdo0 = rf * 128 + ((kq ^ sw) << 4);
    rdo1 = rf * 128 + (((4 + kq) ^ sw) << 4);
  }
  const int a_base = wm * TM * 128;
  const int b_base = (BM + wn * TN) * 128;

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  i32x4 st[NCH];
  auto gload = [&](int kt) {
    const uint32_t so = (uint32_t)(kt0 + kt) * 128u;
#pragma unroll
    for (int i = 0; i < NCH; ++i) st[i] = buf_load16(i < NA ? ra : rb, voff[i], so);
  };
  auto swrite = [&](int s) {
    uint8_t* base = smem + s * STAGE + tid * 16;
#pragma unroll
    for (int i = 0; i < NCH; ++i) *(i32x4*)(base + i * 8192) = st[i];
  };
  auto compute = [&](int s) {
    const uint8_t* sa = smem + s * STAGE + a_base;
    const uint8_t* sb = smem + s * STAGE + b_base;
    if constexpr (FP8) {
      i32x8 bfr[FN], afr[FM];
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        i32x4 lo = *(const i32x4*)(sb + j * 2048 + rdo0);
        i32x4 hi = *(const i32x4*)(sb + j * 2048 + rdo1);
        bfr[j] = i32x8{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
      }
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        i32x4 lo = *(const i32x4*)(sa + i * 2048 + rdo0);
        i32x4 hi = *(const i32x4*)(sa + i * 2048 + rdo1);
        afr[i] = i32x8{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
      }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
              bfr[j], afr[i], acc[i][j], 0, 0, 0, 0, 0, 0);
    } else {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const uint32_t ro = ks ? rdo1 : rdo0;
        bf16x8 bfr[FN], afr[FM];
#pragma unroll
        for (int j = 0; j < FN; ++j) bfr[j] = *(const bf16x8*)(sb + j * 2048 + ro);
#pragma unroll
        for (int i = 0; i < FM; ++i) afr[i] = *(const bf16x8*)(sa + i * 2048 + ro);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bfr[j], afr[i], acc[i][j], 0, 0, 0);
      }
    }
  };

  // ---- the K loop: stage kt is computed while kt + 1 sits in LDS and kt + 2 in registers
  gload(0);
  swrite(0);
  __syncthreads();
  if (nkt > 1) gload(1);
  for (int kt = 0; kt < nkt; ++kt) {
    compute(kt & 1);
    if (kt + 1 < nkt) swrite((kt + 1) & 1);
    __syncthreads();
    if (kt + 2 < nkt) gload(kt + 2);
  }

  // ---- the store. Lane l holds, for fragment (i, j), C[m][n .. n + 3]:
  const int mw = wm * TM + rf;       // + 16 i
  const int nw = wn * TN + 4 * kq;   // + 16 j
  if constexpr (MODE == kStoreF32) {
    float* out = (float*)p.c + (int64_t)split * p.split_stride;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int m = m0 + mw + 16 * i;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int n = n0 + nw + 16 * j;
        if (m < p.M && n < p.N) {
          f32x4 v = fused_apply(p.ep, acc[i][j], m, n, true);
          *(f32x4*)(out + (int64_t)m * p.ldc + n) = v;
        }
      }
    }
  } else if constexpr (MODE == kPairWs) {
    float* out = (float*)p.c + (int64_t)split * p.split_stride;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int m = m0 + mw + 16 * i;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int fv = wn * FN + j;
        const int oc = n0 + (fv >> 1) * 16 + 4 * kq;
        if (m < p.M && oc < p.N)
          *(f32x4*)(out + (int64_t)m * p.ldc + oc + ((fv & 1) ? p.N : 0)) = acc[i][j];
      }
    }
  } else {
    // epilogue in registers, one conversion, into the staging tile
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int ml = mw + 16 * i;
      const int m = m0 + ml;
      if constexpr (MODE == kPair16) {
#pragma unroll
        for (int j = 0; j < FN; j += 2) {
          const int ocl = ((wn * FN + j) >> 1) * 16 + 4 * kq;
          f32x4 v = silu_mul4(acc[i][j], acc[i][j + 1]);
          *(u32x2*)(smem + ml * RS + ocl * 2) = pack4<2>(p.c_dt, v);
        }
      } else {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int nl = nw + 16 * j;
          f32x4 v = fused_apply(p.ep, acc[i][j], m, n0 + nl, m < p.M);
          u32x2 w = pack4<OB>(p.c_dt, v);
          if constexpr (OB == 2)
            *(u32x2*)(smem + ml * RS + nl * 2) = w;
          else
            *(uint32_t*)(smem + ml * RS + nl) = w.x;
        }
      }
    }
    __syncthreads();
    constexpr int CPR = OUTW * OB / 16;  // 16-byte chunks a row
    constexpr int EPC = 16 / OB;         // elements a chunk
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
          for (int e = 0; e < cnt; ++e) dst[e] = src[e];
        }
      }
    }
  }
}

}  // namespace hkx
