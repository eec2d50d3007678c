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
  // kDecArrive: the shares' buffer (c is C) and one arrival counter a block of rows
  float* ws;
  int32_t* cnt;
};

// s_waitcnt vmcnt(n) (gfx9 encoding: bits 3:0 and 15:14; expcnt and lgkmcnt left alone)
constexpr int wait_vm_dec(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

constexpr int kDecOut = 0;     // C with the fused epilogue
constexpr int kDecWs = 1;      // fp32 shares, (M, N) per split
constexpr int kDecPair = 2;    // silu(gate) * up into C
constexpr int kDecPairWs = 3;  // gate and up fp32 shares, (M, 2N) per split
constexpr int kDecArrive = 4;  // fp32 shares, the last split of a block sums them into C

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

  if constexpr (MODE == kDecArrive) {
    // This split's share of the block, then one arrival at the block's counter; the last of
    // the gridDim.y splits to arrive sums the shares in split order (so the result does not
    // depend on the order of arrival), applies the epilogue, stores C and sets the counter
    // back to zero for the next call (the reference's decode split finishes the same way,
    // python/hk/ops/decode_gemm.py:155-170). The shares are written and read as device-scope
    // relaxed atomics (coherent across the XCDs' L2s by themselves), and each wave waits for
    // its share stores before the barrier that precedes the arrival: a device-scope fence
    // instead writes back and invalidates the whole L2, and with hundreds of workgroups
    // arriving it made the call 5-100x slower.
    __shared__ int last;
    for (int f = wave; f < NF; f += NW) {
      f32x4 s = red[0][f][lane];
#pragma unroll
      for (int w2 = 1; w2 < NW; ++w2) s += red[w2][f][lane];
      const int i = f / FN, j = f - i * FN;
      const int m = i * 16 + rf, n = n0 + j * 16 + 4 * kq;
      if (m < p.M && n < p.N) {
        float* dst = p.ws + (int64_t)split * p.split_stride + (int64_t)m * p.N + n;
#pragma unroll
        for (int e = 0; e < 4; ++e) __hip_atomic_store(dst + e, s[e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    __builtin_amdgcn_s_waitcnt(wait_vm_dec(0));  // this wave's share stores performed
    __syncthreads();
    if (tid == 0)
      last = __hip_atomic_fetch_add(p.cnt + blockIdx.x, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
             (int)gridDim.y - 1;
    __syncthreads();
    if (!last) return;
    for (int f = wave; f < NF; f += NW) {
      const int i = f / FN, j = f - i * FN;
      const int m = i * 16 + rf, n = n0 + j * 16 + 4 * kq;
      if (m < p.M && n < p.N) {
        float* w0 = p.ws + (int64_t)m * p.N + n;
        f32x4 s;
#pragma unroll
        for (int e = 0; e < 4; ++e) s[e] = __hip_atomic_load(w0 + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (int s2 = 1; s2 < (int)gridDim.y; ++s2) {
          float* src = w0 + (int64_t)s2 * p.split_stride;
#pragma unroll
          for (int e = 0; e < 4; ++e) s[e] += __hip_atomic_load(src + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        store4(p.c, p.c_dt, (int64_t)m * p.ldc + n, fused_apply(p.ep, s, m, n, true));
      }
    }
    if (tid == 0) __hip_atomic_store(p.cnt + blockIdx.x, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else if constexpr (!PAIR) {
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


// The streaming decode GEMM: one workgroup a CU walks its share of the 16-row blocks of W
// (a consecutive run of them), for M <= 32 (MF = 1 or 2 16-token fragments; two from
// K = 2048 up), unpaired, no split, K a multiple of 1024: CPB chunks of 1024 a block
// (CPB = 1..4), or, with CPB = 0, K / 1024 of them read at run time (K past 4096).
//
// * W goes HBM -> LDS by non-temporal buffer loads (`buffer_load_dwordx4 ... lds`, read
//   once, kept out of the caches), each instruction 1 KB
//   of one row, contiguous -- the access a pure streaming read reaches HBM's ceiling with --
//   in chunks of 16 rows x 1024 K (32 KB) through a ring of four: chunk q + 3 is in flight
//   while chunk q is multiplied. A row's 128 16-byte pieces are stored XOR-swizzled by the
//   row (piece c at c ^ (r % 16)), applied on the global side, so the MFMA fragment reads
//   (16 rows, one piece each) are conflict-free.
// * X is the same for every block: wave w owns the 128-element group w of every chunk, and
//   loads its share of X (CPB groups of 16 or 32 rows) into registers once, a chunk's share
//   with the first block's fill of the chunk before it (all of X up front cost 1 us of
//   20 at M = 16, K = 4096); past K = 4096 it is streamed with the chunks instead (two
//   chunks ahead, three register slots). Above M = 8 it arrives as whole 128-byte lines
//   and is shuffled into the MFMA layout before the chunk's MFMAs (see xload / xperm).
//   Each step issues its X loads before its fill, so the waits, which count loads in issue
//   order, wait for exactly the chunk and the X they need (the compiler's own order put X
//   after the fill, which made the register waits take the next chunk's fill too: 0.4 us
//   at M = 16).
// * v_mfma_f32_16x16x32_bf16 with W's fragment first; the 8 waves' partial sums of a block
//   meet in LDS (double-buffered by block parity with one fragment, one buffer with two),
//   and wave 0 sums, applies the epilogue and
//   stores after the next chunk's barrier, under the other waves' MFMAs. The epilogue's
//   common form (a bf16 bias, an activation) reads its bias with one LDS read a lane; a
//   wait it had on a tile operand's direct load, and element-by-element vector reads,
//   cost 0.6-0.9 us a call with a bias before.
// The stream kernel's epilogue forms: kStreamEpFast -- an activation of acc times broadcast
// scales (or none) plus an optional bf16 bias of unit stride, 4-byte aligned, N even --
// reads its bias with one 8-byte LDS read a lane; kStreamEpGeneric reads every vector
// operand element by element in any dtype and stride.
constexpr int kStreamEpFast = 0;
constexpr int kStreamEpGeneric = 1;

template <int CPB, int EPF, int MF>
__global__ void __launch_bounds__(512) stream_kernel(const DecodeArgs p) {
  constexpr int NW = 8;
  constexpr int CH = 16 * 2048;  // a chunk: 16 rows x 2 KB
  constexpr int NR = 4;          // ring slots
  // then the partial sums: [block parity][wave][fragment][lane], 16 B each -- two parities
  // with one 16-token fragment, one with two (a block's partial sums are read at the next
  // block's first chunk and rewritten at its end, a barrier later: two fragments take only
  // K of 2048 and up)
  constexpr int NPAR = MF == 1 ? 2 : 1;
  constexpr int RED = NR * CH;
  constexpr int EPV = RED + NPAR * NW * MF * 64 * 16;  // then the epilogue's vectors: [block % 3][cs, rs, ra][64 slots]
  // then the tile operand's values of a block: [block % 3][row < 32][16 columns], up to 64
  // bytes a row
  constexpr int TOFF = EPV + 3 * 3 * 256;
  constexpr int TSLOT = 32 * 64;
  __shared__ __attribute__((aligned(16))) uint8_t ring[TOFF + 3 * TSLOT];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rf = lane & 15, kq = lane >> 4;
  const int nb = (p.N + 15) / 16;
  const int G = gridDim.x;
  if ((int)blockIdx.x >= nb) return;
  // a workgroup's blocks are consecutive (blocks [bstart, bstart + my_blocks)), and it
  // walks each block's K chunks starting from chunk (blockIdx.x / 8) % cpb, so the first
  // reads of X by the CUs of one XCD (workgroups blockIdx.x, + 8, + 16, ...) spread over
  // its chunks (measured 0.3-0.6 us faster at M = 16 than blocks strided by the grid and
  // every workgroup starting on chunk 0, and 0.1-0.2 us faster than a rotation by
  // blockIdx.x % cpb, which starts all the CUs of an XCD on one chunk)
  const int bstart = (int)(((int64_t)blockIdx.x * nb) / G);
  const int my_blocks = (int)((((int64_t)blockIdx.x + 1) * nb) / G) - bstart;
  auto block_of = [&](int j) { return bstart + j; };
  const int cpb = CPB ? CPB : p.g_total / 8;  // chunks a block
  const int rot = ((int)blockIdx.x >> 3) % cpb;
  auto kchunk = [&](int c) { const int r = c + rot; return r >= cpb ? r - cpb : r; };
  const int nq = my_blocks * cpb;             // chunks of this workgroup

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
  // With X streamed (CPB = 0) a fill past the last chunk is still issued, out of range (it
  // reads nothing and writes a slot no one reads again: chunk q - 4's, done before the
  // barrier that precedes it), so every wave issues the same loads on every path: the
  // compiler's own waits for X count the loads after X on the path with the fewest, and with
  // fills skipped at the end they had drained the ring before every chunk's MFMAs (1.1-1.6
  // us of 19.7-24 at the down projections' K). With X held (loaded in the first block only)
  // such a drain comes once a launch; there the fills stop at the end (issuing them
  // measured 0.2-0.6 us slower at M = 8-16 on 12288 and 28672 rows of W and 0.4-0.7 us
  // slower on 1536 and 4096 rows, in interleaved same-box runs).
  constexpr bool kAllFills = CPB == 0;
  auto fill = [&](int q) {
    if (!kAllFills && q >= nq) return;  // past the end: nothing (the waits count what was issued)
    const bool live = q < nq;
    const int jb = live ? q / cpb : 0, kc = live ? kchunk(q - jb * cpb) : 0;
    const int bi = block_of(jb);
    const uint32_t so = live ? __builtin_amdgcn_readfirstlane((uint32_t)bi * 16u * p.ldb_b + (uint32_t)kc * 2048u) : 0u;
    const uint32_t oob = live ? 0u : 0x80000000u;
    uint8_t* slot = ring + (q & (NR - 1)) * CH;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 2 * wave + (i >> 1), h = i & 1;
      buf_load16_lds<kNonTemporal>(rw, slot + r * 2048 + h * 1024, fv[i] + oob, so);
    }
  };
  // The epilogue's vector operands of block j (row scale per token m, column scale and
  // column add per output n) go global -> LDS by 4-byte DMA from wave 0, one block ahead,
  // so they land under the waits the fills already have: a direct load in the epilogue
  // would wait for every fill in flight (loads complete in order). Slot s of a vector
  // holds the aligned 32-bit word that contains element s of the block (its 16-bit half
  // picked by the element's address). Broadcast operands (stride 0) are read once.
  const Fused& e = p.ep;
  const bool fused = e.form == HKX_EP_FUSED;
  const bool cs_vec = fused && e.cs.p && e.cs.ld, rs_vec = fused && e.rs.p && e.rs.ld,
             ra_vec = fused && e.ra.p && e.ra.ld;
  // the tile operand (generic form only): a block's 16 columns of rows 0 .. M - 1 (32 or 64
  // bytes a row), by 16-byte DMA where its rows start 16-byte aligned (32 or 16 rows an
  // instruction), else by 4-byte DMA (8 or 4 rows an instruction)
  const bool ta_on = fused && e.ta.p;
  const uint32_t ta_eb = ta_on && e.ta.dt == HKX_FP32 ? 4u : 2u;
  const int ta_dpr = 4 * (int)ta_eb;  // dwords a row of the block
  const bool ta_w16 = ta_on && ((uintptr_t)e.ta.p & 15) == 0 && (e.ta.ld * ta_eb) % 16 == 0;
  const int ta_pb = ta_w16 ? 16 : 4;               // bytes a lane moves
  const int ta_ppr = ta_dpr * 4 / ta_pb;           // lanes a row
  const int ta_rpi = 64 / ta_ppr;                  // rows a DMA instruction
  const int ta_n = ta_on ? (min(p.M, 16 * MF) + ta_rpi - 1) / ta_rpi : 0;
  const float cs_sc = (fused && e.cs.p && !e.cs.ld) ? ld1(e.cs.p, e.cs.dt, 0) * e.cmul : e.cmul;
  const float rs_sc = (fused && e.rs.p && !e.rs.ld) ? ld1(e.rs.p, e.rs.dt, 0) : 1.0f;
  const float ra_sc = (fused && e.ra.p && !e.ra.ld) ? ld1(e.ra.p, e.ra.dt, 0) : 0.0f;
  auto ep_load = [&](int j) {
    if (wave != 0 || !(cs_vec || rs_vec || ra_vec || ta_on)) return;
    const int bi = block_of(j);
    uint8_t* base = ring + EPV + (j % 3) * 768;
    const int l = lane;
    constexpr uint32_t kOut = 0x7fffffffu;  // past every buffer's end: reads nothing
    // the tile operand's rows of the block into its slot
    auto tile_load = [&]() {
      const uint32_t rowb = (uint32_t)e.ta.ld * ta_eb;
      const __amdgpu_buffer_rsrc_t rt = make_rsrc(e.ta.p, (uint32_t)p.M * rowb);
      uint8_t* tslot = ring + TOFF + (j % 3) * TSLOT;
      for (int r = 0; r < ta_n; ++r) {
        const int row = r * ta_rpi + l / ta_ppr, d = l % ta_ppr;
        const uint32_t off =
            row < p.M ? (uint32_t)row * rowb + (uint32_t)bi * 16u * ta_eb + (uint32_t)(d * ta_pb) : kOut;
        auto* dst = (__attribute__((address_space(3))) void*)(tslot + r * ta_rpi * ta_dpr * 4);
        if (ta_w16) __builtin_amdgcn_raw_ptr_buffer_load_lds(rt, dst, 16, off, 0, 0, 0);
        else __builtin_amdgcn_raw_ptr_buffer_load_lds(rt, dst, 4, off, 0, 0, 0);
      }
    };
    if constexpr (EPF == kStreamEpFast) {
      // the block's 16 bf16 bias values: 8 lanes of one dword each, contiguous in LDS
      if (ra_vec)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            make_rsrc(e.ra.p, (uint32_t)p.N * 2u), (__attribute__((address_space(3))) void*)(base + 512), 4,
            lane < 8 ? (uint32_t)(bi * 32 + 4 * lane) : 0x7fffffffu, 0, 0, 0);
      if (ta_on) tile_load();
      return;
    }
    // the word of element idx, from the operand's address rounded down to 4 bytes (the
    // bound rounded up: a dword only partly inside a buffer reads as zero)
    auto load = [&](const Opnd& o, int64_t elems, bool ok, int64_t idx, uint8_t* dst) {
      const uintptr_t a = (uintptr_t)o.p, al = a & ~(uintptr_t)3;
      const uint32_t eb = o.dt == HKX_FP32 ? 4u : 2u;
      const uint32_t byte = (uint32_t)(a - al) + (uint32_t)idx * eb;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          make_rsrc((const void*)al, ((uint32_t)(a - al) + (uint32_t)elems * eb + 3u) & ~3u),
          (__attribute__((address_space(3))) void*)dst, 4, ok ? (byte & ~3u) : kOut, 0, 0, 0);
    };
    const int n = bi * 16 + l;
    if (cs_vec)
      load(e.cs, (int64_t)(p.M - 1) * e.cs.ld + 1, l < 16 * MF && l < p.M, (int64_t)l * e.cs.ld, base);
    if (rs_vec) load(e.rs, p.N, l < 16 && n < p.N, n, base + 256);
    if (ra_vec) load(e.ra, p.N, l < 16 && n < p.N, n, base + 512);
    if (ta_on) tile_load();
  };
  // which half of its word a 16-bit element is in (from its address)
  auto hi_half = [](const Opnd& o, int64_t idx) {
    return ((((uintptr_t)o.p >> 1) + (uint64_t)idx) & 1) != 0;
  };
  auto word_val = [](uint32_t w, int dt, bool hi) {
    if (dt == HKX_FP32) return __builtin_bit_cast(float, w);
    const uint32_t h = hi ? (w >> 16) : (w & 0xffffu);
    return dt == HKX_FP16 ? (float)__builtin_bit_cast(_Float16, (uint16_t)h) : bf16_to_f32(h);
  };
  auto vec4 = [&](const uint32_t* s, const Opnd& o, int n) {
    return f32x4{word_val(s[0], o.dt, hi_half(o, n)), word_val(s[1], o.dt, hi_half(o, n + 1)),
                 word_val(s[2], o.dt, hi_half(o, n + 2)), word_val(s[3], o.dt, hi_half(o, n + 3))};
  };
  f32x4 acc[MF];
#pragma unroll
  for (int f = 0; f < MF; ++f) acc[f] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto red_at = [&](int j, int w2, int f) {  // a lane's 16 bytes of the partial sums
    return (uint32_t)(RED + ((((MF == 1 ? j & 1 : 0) * NW + w2) * MF + f) * 64 + lane) * 16);
  };
  // the MFMAs of this wave's group of chunk q (its slot landed and visible)
  auto mma = [&](int q, const i32x4 (&xc)[MF][4]) {
    const uint32_t slot = (uint32_t)(q & (NR - 1)) * CH;
    i32x4 w[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int piece = 16 * wave + kq + 4 * s;  // global piece of the row in this chunk
      w[s] = ds_read16(slot + rf * 2048 + ((piece ^ rf) << 4));
    }
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int f = 0; f < MF; ++f)
        acc[f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, w[s]),
                                                         __builtin_bit_cast(bf16x8, xc[f][s]), acc[f], 0, 0, 0);
  };
  // block j of this workgroup (its partial sums at parity j & 1 with one fragment)
  auto finish = [&](int j) {
    const int bi = block_of(j);
#pragma unroll 1
    for (int f = 0; f < MF; ++f) {
    i32x4 part[NW];
#pragma unroll
    for (int w2 = 0; w2 < NW; ++w2) part[w2] = ds_read16(red_at(j, w2, f));
    f32x4 sum = __builtin_bit_cast(f32x4, part[0]);
#pragma unroll
    for (int w2 = 1; w2 < NW; ++w2) sum += __builtin_bit_cast(f32x4, part[w2]);
    const int m = 16 * f + rf, n = bi * 16 + 4 * kq;
    if (EPF == kStreamEpFast && fused) {
      const uint8_t* eo = ring + EPV + (j % 3) * 768;
      const f32x4 ra = ra_vec ? unpack_bf16x4(*(const u32x2*)(eo + 512 + 8 * kq))
                              : f32x4{ra_sc, ra_sc, ra_sc, ra_sc};
      const float sc = cs_sc * rs_sc;
      // (the fast form's tile operand is bf16, 32 bytes a row of the block)
      const f32x4 tv = ta_on ? unpack_bf16x4(*(const u32x2*)(ring + TOFF + (j % 3) * TSLOT + m * 32 + 8 * kq))
                             : f32x4{0.f, 0.f, 0.f, 0.f};
      sum = act4(e.act, sum * f32x4{sc, sc, sc, sc} + ra + tv + e.cadd);
    } else if (fused) {
      const uint32_t* eo = (const uint32_t*)(ring + EPV + (j % 3) * 768);
      const float cs = cs_vec ? word_val(eo[m], e.cs.dt, hi_half(e.cs, (int64_t)m * e.cs.ld)) * e.cmul
                              : cs_sc;
      const f32x4 rs = rs_vec ? vec4(eo + 64 + 4 * kq, e.rs, n) : f32x4{rs_sc, rs_sc, rs_sc, rs_sc};
      const f32x4 ra = ra_vec ? vec4(eo + 128 + 4 * kq, e.ra, n) : f32x4{ra_sc, ra_sc, ra_sc, ra_sc};
      f32x4 tv = f32x4{0.f, 0.f, 0.f, 0.f};
      if (ta_on) {  // from LDS (a direct load would make wave 0 wait for every fill in flight)
        const uint8_t* ts = ring + TOFF + (j % 3) * TSLOT + m * ta_dpr * 4;
        if (e.ta.dt == HKX_FP32) tv = *(const f32x4*)(ts + 16 * kq);
        else {
          const u32x2 w = *(const u32x2*)(ts + 8 * kq);
          tv = e.ta.dt == HKX_FP16 ? unpack_f16x4(w) : unpack_bf16x4(w);
        }
      }
      sum = act4(e.act, sum * (rs * cs) + ra + tv + e.cadd);
    }
    if (m < p.M && n < p.N) store4(p.c, p.c_dt, (int64_t)m * p.ldc + n, sum);
    }
  };

  // X for chunk k (its group of this wave) goes to registers by loads issued just before
  // the fill of chunk k + 1: x0 f0 x1 f1 f2, then step q issues x(q + 2) and f(q + 3). X is
  // loaded for every step with CPB = 0 (streamed; past the last chunk too, like the fills,
  // into a register slot no one reads), for the first CPB chunks with CPB > 0 (held across
  // the walk; a workgroup has at least CPB chunks).
  auto has_x = [&](int k) { return CPB == 0 || k < CPB; };
  // chunk q and its X landed, and every wave is done with chunk q - 1, whose slot the fill
  // of q + 3 takes: in issue order the loads after x(q) and f(q) are f(q + 1), x(q + 1) and
  // f(q + 2), 4 a wave each where they are issued (anything issued later only makes the wait
  // stricter); lgkmcnt(0) as well
  // wave 0's epilogue-vector DMAs of the step before (ep_load) are among them too
  const int nvec = EPF == kStreamEpFast ? (int)ra_vec + ta_n
                                        : (int)cs_vec + (int)rs_vec + (int)ra_vec + ta_n;
  auto wait_chunk = [&](int q, bool ep_before) {
    const int n = (kAllFills ? 8 : 4 * ((q + 1 < nq) + (q + 2 < nq))) + 4 * MF * has_x(q + 1) +
                  (ep_before && wave == 0 ? nvec : 0);
    switch (n) {
#define HKX_WAIT_CASE(N) case N: __builtin_amdgcn_s_waitcnt(wait_vm_dec(N) & ~(15 << 8)); break;
      HKX_WAIT_CASE(1) HKX_WAIT_CASE(2) HKX_WAIT_CASE(3) HKX_WAIT_CASE(4) HKX_WAIT_CASE(5)
      HKX_WAIT_CASE(6) HKX_WAIT_CASE(7) HKX_WAIT_CASE(8) HKX_WAIT_CASE(9) HKX_WAIT_CASE(10)
      HKX_WAIT_CASE(11) HKX_WAIT_CASE(12) HKX_WAIT_CASE(13) HKX_WAIT_CASE(14) HKX_WAIT_CASE(15)
      HKX_WAIT_CASE(16) HKX_WAIT_CASE(17) HKX_WAIT_CASE(18) HKX_WAIT_CASE(19) HKX_WAIT_CASE(20)
      HKX_WAIT_CASE(21) HKX_WAIT_CASE(22) HKX_WAIT_CASE(23) HKX_WAIT_CASE(24) HKX_WAIT_CASE(25)
      HKX_WAIT_CASE(26) HKX_WAIT_CASE(27) HKX_WAIT_CASE(28) HKX_WAIT_CASE(29) HKX_WAIT_CASE(30)
      HKX_WAIT_CASE(31)
#undef HKX_WAIT_CASE
      default: __builtin_amdgcn_s_waitcnt(wait_vm_dec(0) & ~(15 << 8)); break;
    }
  };
  auto block_done = [&](int j) {
#pragma unroll
    for (int f = 0; f < MF; ++f) {
      ds_write16(red_at(j, wave, f), __builtin_bit_cast(i32x4, acc[f]));
      acc[f] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  // This wave's share of X for chunk c (K group 8 c + wave: 16 rows x 256 bytes) in four
  // loads of whole 128-byte lines: load i brings rows 8 (i & 1) + [0, 8), line i >> 1 of
  // the group, lane l row l / 8 and piece l % 8 of the line (consecutive lanes along a
  // line). In the MFMA layout -- lane l holding row l % 16 -- a load asks for 64 bytes of
  // 16 lines: measured 0.4-0.5 us slower at M = 16 (lines with the row in the low lane
  // bits were no faster either).
  // (with two 16-token fragments, fragment f the rows 16 f + [0, 16)). Up to M = 8 the loads
  // are in the MFMA layout instead (lane l: row l % 16, 16 bytes at 16 (l / 16) + 64 i):
  // there X is a few KB a CU, rows past M read nothing, and the shuffle below would only
  // add its latency to every chunk of the first block (1-2 us at M = 1 on the shapes whose
  // workgroups have one block).
  const bool xlines = MF == 2 || p.M > 8;
  auto xload = [&](int c, i32x4 (&dst)[MF][4]) {
#pragma unroll
    for (int f = 0; f < MF; ++f)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t off = xlines ? (uint32_t)(16 * f + (lane >> 3) + 8 * (i & 1)) * p.lda_b +
                                          (uint32_t)(lane & 7) * 16 + (i >> 1) * 128
                                    : (uint32_t)rf * p.lda_b + kq * 16 + i * 64;
        dst[f][i] = buf_load16(rx, off, (uint32_t)(8 * kchunk(c) + wave) * 256u);
      }
  };
  // ... then into the MFMA layout, just before the chunk's MFMAs: k-step s = 2 h + e of lane
  // (rf, kq) takes row rf, piece 4 s + kq of the group, which load 2 h + rf / 8 holds at
  // lane 8 (rf % 8) + 4 e + kq. Loads 2 h (a) and 2 h + 1 (b) first trade 4-lane halves
  // (DPP row shifts by 4): m0 keeps a's pieces 0-3 of each row in place with b's beside
  // them (lanes 8 r + 4 + k), m1 a's pieces 4-7 in place with b's beside them (lanes
  // 8 r + k); then one ds_bpermute a dword. (Two ds_bpermutes a dword and a select, or the
  // shuffle moved off the path to the MFMAs, measured slower.)
  const int xsrc0 = 4 * (8 * (rf & 7) + kq + 4 * (rf >> 3)), xsrc1 = 4 * (8 * (rf & 7) + kq + 4 * (rf < 8));
  const bool hi4 = (lane & 4) != 0;
  auto xperm = [&](i32x4 (&vv)[MF][4]) {
    if (!xlines) return;
#pragma unroll
    for (int f = 0; f < MF; ++f) {
    i32x4 (&v)[4] = vv[f];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const int a = v[2 * h][d], b = v[2 * h + 1][d];
        const int bs = __builtin_amdgcn_update_dpp(0, b, 0x114, 0xf, 0xf, false);  // row_shr:4
        const int bl = __builtin_amdgcn_update_dpp(0, b, 0x104, 0xf, 0xf, false);  // row_shl:4
        const int m0 = hi4 ? bs : a, m1 = hi4 ? a : bl;
        v[2 * h][d] = __builtin_amdgcn_ds_bpermute(xsrc0, m0);
        v[2 * h + 1][d] = __builtin_amdgcn_ds_bpermute(xsrc1, m1);
      }
    }
  };

  if constexpr (CPB > 0) {
    // X held in registers for the whole walk, its chunks loaded with the first block's
    // fills, so a workgroup starts on 32 KB of X rather than all of it
    i32x4 x[CPB][MF][4];
    ep_load(0);
    xload(0, x[0]);
    __builtin_amdgcn_sched_barrier(0);
    fill(0);
    if (CPB > 1) xload(1, x[CPB > 1 ? 1 : 0]);
    __builtin_amdgcn_sched_barrier(0);
    fill(1);
    fill(2);
    for (int j = 0; j < my_blocks; ++j) {
#pragma unroll
      for (int c = 0; c < CPB; ++c) {
        const int q = j * CPB + c;
        // the step before issued ep_load(j) when it was the first chunk of block j - 1
        wait_chunk(q, (CPB == 1 ? c == 0 && j >= 1 : c == 1) && (CPB == 1 || j + 1 < my_blocks));
        __builtin_amdgcn_s_barrier();
        if (c == 0 && j + 1 < my_blocks) ep_load(j + 1);  // older than the fills of q + 3 on
        if (c + 2 < CPB && j == 0) xload(c + 2, x[c + 2 < CPB ? c + 2 : 0]);
        __builtin_amdgcn_sched_barrier(0);  // X before the fill: the waits count in that order
        fill(q + 3);
        if (c == 0 && j > 0 && wave == 0) finish(j - 1);
        if (j == 0) xperm(x[c]);  // (X is held in registers from the first block on)
        mma(q, x[c]);
      }
      block_done(j);
    }
  } else {
    // K past 4096: X streamed with the chunks through three register slots (the loop is
    // unrolled by three so every slot is a fixed register set)
    i32x4 xs[3][MF][4];
    auto xnext = [&](int q, i32x4 (&dst)[MF][4]) {
      if (has_x(q)) xload(q % cpb, dst);
    };
    ep_load(0);
    xnext(0, xs[0]);
    fill(0);
    xnext(1, xs[1]);
    fill(1);
    fill(2);
    auto step = [&](int q, i32x4 (&xc)[MF][4], i32x4 (&xn)[MF][4]) {
      const int j = q / cpb, c = q - j * cpb;
      wait_chunk(q, c == 1 && j + 1 < my_blocks);
      __builtin_amdgcn_s_barrier();
      if (c == 0 && j + 1 < my_blocks) ep_load(j + 1);
      xnext(q + 2, xn);
      fill(q + 3);
      if (c == 0 && j > 0 && wave == 0) finish(j - 1);
      xperm(xc);
      mma(q, xc);
      if (c == cpb - 1) block_done(j);
    };
    for (int q = 0; q < nq; q += 3) {
      step(q, xs[0], xs[2]);
      if (q + 1 < nq) step(q + 1, xs[1], xs[0]);
      if (q + 2 < nq) step(q + 2, xs[2], xs[1]);
    }
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the last partial sums written
  __builtin_amdgcn_s_barrier();
  if (wave == 0) finish(my_blocks - 1);
  __builtin_amdgcn_s_waitcnt(wait_vm_dec(0));  // no fill lands in LDS after the exit
}

}  // namespace hkx
