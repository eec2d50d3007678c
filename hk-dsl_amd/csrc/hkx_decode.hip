// Decode GEMM kernels: 4, 8 or 16 waves, 16 or 32 rows of W a workgroup, 1 or 2
// 16-token fragments, every store mode; the stream kernel; and the whole-row kernel, defined
// here (it is launched from this file only).
#include "hkx_launch.hpp"

namespace hkx {

// Groups in flight per wave: as many as the wave's share of the register file holds
// beside the accumulators (16 VGPRs a fragment a group, for W's and for X's).
constexpr int decode_unroll(int waves, int fn, int mf) {
  const int budget = 512 / (waves / 4 > 0 ? waves / 4 : 1);
  const int u = (budget - 48) / (16 * (fn + mf));
  return u < 1 ? 1 : (u > 4 ? 4 : u);
}

template <int NW, int FN, int MF>
static hipError_t launch_nw(const DecodeArgs& a, int mode, dim3 grid, hipStream_t s) {
  constexpr int U = decode_unroll(NW, FN, MF);
  const dim3 block(NW * 64);
  switch (mode) {
    case kDecOut: hipLaunchKernelGGL((decode_kernel<NW, FN, MF, U, kDecOut>), grid, block, 0, s, a); break;
    case kDecWs: hipLaunchKernelGGL((decode_kernel<NW, FN, MF, U, kDecWs>), grid, block, 0, s, a); break;
    case kDecArrive: hipLaunchKernelGGL((decode_kernel<NW, FN, MF, U, kDecArrive>), grid, block, 0, s, a); break;
    case kDecPair:
      if constexpr (FN % 2 == 0) { hipLaunchKernelGGL((decode_kernel<NW, FN, MF, U, kDecPair>), grid, block, 0, s, a); break; }
      return hipErrorInvalidValue;
    case kDecPairWs:
      if constexpr (FN % 2 == 0) { hipLaunchKernelGGL((decode_kernel<NW, FN, MF, U, kDecPairWs>), grid, block, 0, s, a); break; }
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int NW>
static hipError_t launch_fn(const DecodeArgs& a, int fn, int mf, int mode, dim3 grid, hipStream_t s) {
  if (fn == 1) return mf == 1 ? launch_nw<NW, 1, 1>(a, mode, grid, s) : launch_nw<NW, 1, 2>(a, mode, grid, s);
  return mf == 1 ? launch_nw<NW, 2, 1>(a, mode, grid, s) : launch_nw<NW, 2, 2>(a, mode, grid, s);
}

hipError_t launch_decode(const DecodeArgs& a, int waves, int fn, int mf, int mode, dim3 grid,
                         hipStream_t s) {
  if (waves == 4) return launch_fn<4>(a, fn, mf, mode, grid, s);
  if (waves == 8) return launch_fn<8>(a, fn, mf, mode, grid, s);
  return launch_fn<16>(a, fn, mf, mode, grid, s);
}

// Whether the stream kernel's fast epilogue form takes the call's epilogue: no vector
// scales (broadcast ones are fine), a bias -- if any -- bf16 of unit stride, 4-byte
// aligned, N even; a tile operand -- if any -- bf16 with 16-byte aligned rows.
static bool stream_fast(const DecodeArgs& a) {
  const Fused& e = a.ep;
  if (e.form != HKX_EP_FUSED) return true;
  if ((e.cs.p && e.cs.ld) || (e.rs.p && e.rs.ld)) return false;
  if (e.ta.p && (e.ta.dt != HKX_BF16 || ((uintptr_t)e.ta.p & 15) || (e.ta.ld * 2) % 16)) return false;
  if (e.ra.p && e.ra.ld)
    return e.ra.dt == HKX_BF16 && e.ra.ld == 1 && ((uintptr_t)e.ra.p & 3) == 0 && a.N % 2 == 0;
  return true;
}

bool stream_takes(const DecodeArgs& a, int splits, bool pair) {
  const int groups = a.g_total;  // 128-element K groups
  // a tile operand reaches LDS by 4-byte DMA: bf16, fp16 or fp32, rows 4-byte aligned, byte
  // offsets within 32 bits
  const Opnd& t = a.ep.ta;
  if (a.ep.form == HKX_EP_FUSED && t.p) {
    const int eb = t.dt == HKX_FP32 ? 4 : 2;
    if ((t.dt != HKX_BF16 && t.dt != HKX_FP16 && t.dt != HKX_FP32) || ((uintptr_t)t.p & 3) ||
        (t.ld * eb) % 4 || (int64_t)a.M * t.ld * eb >= (1LL << 32))
      return false;
  }
  // two 16-token fragments (M 17-32) keep one buffer of partial sums, which needs two chunks
  // a block (K of 2048 and up)
  return splits == 1 && !pair && groups % 8 == 0 && groups <= 256 &&
         (a.M <= 16 || (a.M <= 32 && groups >= 16));
}

template <int EPF, int MF>
static hipError_t launch_stream_ep(const DecodeArgs& a, dim3 grid, hipStream_t s) {
  const dim3 block(512);
  switch (a.g_total / 8) {
    case 1:
      if constexpr (MF == 1) { hipLaunchKernelGGL((stream_kernel<1, EPF, MF>), grid, block, 0, s, a); break; }
      return hipErrorInvalidValue;  // (stream_takes sends no such call)
    case 2: hipLaunchKernelGGL((stream_kernel<2, EPF, MF>), grid, block, 0, s, a); break;
    case 3: hipLaunchKernelGGL((stream_kernel<3, EPF, MF>), grid, block, 0, s, a); break;
    case 4: hipLaunchKernelGGL((stream_kernel<4, EPF, MF>), grid, block, 0, s, a); break;
    default: hipLaunchKernelGGL((stream_kernel<0, EPF, MF>), grid, block, 0, s, a); break;
  }
  return hipGetLastError();
}

// The whole-row decode GEMM: K = 4096, M <= 4, the fast epilogue form without a tile
// operand. A chunk is 4 whole rows of W (32 KB, contiguous when W's rows are), and the
// workgroups take chunks strided by the grid (workgroup g: chunks g, g + G, ...), so at any
// moment the GPU streams one contiguous window of W. A load-only kernel read W 1.2 us
// faster (of 16.7) this way than in the stream kernel's chunks of 16 rows x 2 KB, which
// the 16-row MFMA fragment otherwise needs.
//
// The MFMA still takes 16 rows: a chunk's 16 pseudo-rows are (row r, K quarter s), i = 4 r
// + s, and X enters as 16 columns (token t, quarter s'), 4 t + s', so one
// v_mfma_f32_16x16x32_bf16 a k-step covers every quarter of 4 rows for 4 tokens, and the
// products wanted are those with s = s' (a lane's component l % 4 of its D fragment),
// summed over the quad of lanes 4 t + [0, 4) by two DPP adds. X is the same for every chunk:
// each wave loads its share (k-steps 4 w .. 4 w + 3 of each quarter) into registers once.
// Past M = 4 (two or four 4-token blocks of X, an MFMA each a k-step) the form measured
// slower than the stream kernel (M = 16: 22.8 against 18.6 us at 12288 x 4096): every chunk
// spans all of K, so a workgroup needs all of X (up to 128 KB) before its first chunk, where
// the stream kernel spreads it over its first block's chunks (without the X loads: 19.8 us).
//
// LDS: a ring of four 32 KB chunk slots (chunk q + 3 in flight while q is multiplied), row r
// at 8 KB r, its 16-byte piece P holding global piece P ^ (4 r + P / 128) (XOR within the
// quarter, applied on the global side of the DMA), so the 16 lanes of one k-group reading
// (r, s) pairs hit 16 different banks. Partial sums: the 8 waves' quad sums of a group of 4
// chunks, double-buffered by group parity; wave 0 adds them, applies the epilogue and stores
// after the next group's first barrier, under the other waves' MFMAs.
__global__ void __launch_bounds__(512) rows_kernel(const DecodeArgs p) {
  constexpr int NW = 8;
  constexpr int CH = 32768;  // a chunk: 4 rows x 8 KB
  constexpr int NR = 4;      // ring slots
  constexpr int GC = 4;      // chunks a group (one reduction and epilogue a group)
  constexpr int RED = NR * CH;
  // then the bias words, three slots by group: [group % 3][256 B]. A slot is 256 bytes, not
  // the 32 its 8 values take, because the DMA runs on all 64 lanes of wave 0 and each lane,
  // in range or not, writes its dword at 4 * lane
  constexpr int EPV = RED + 2 * NW * GC * 64;
  constexpr int EPS = 256;
  __shared__ __attribute__((aligned(16))) uint8_t ring[EPV + 3 * EPS];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nck = (p.N + 3) / 4;
  const int G = gridDim.x;
  const int g = blockIdx.x;
  if (g >= nck) return;
  const int nq = (nck - g + G - 1) / G;  // this workgroup's chunks: g + q G
  auto chunk_of = [&](int q) { return g + q * G; };

  const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.b, p.b_bytes);
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.a, p.a_bytes);

  // fills: wave w moves half of row w / 2 of a chunk, 1 KB an instruction; the chunk's
  // offset goes in the per-lane offset, so rows past N read zero through the bound
  uint32_t fv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = wave >> 1, P = (wave & 1) * 256 + i * 64 + lane;
    fv[i] = (uint32_t)r * p.ldb_b + (uint32_t)((P ^ (4 * r + (P >> 7))) << 4);
  }
  // Past the last chunk a fill is still issued, out of range (it reads nothing and writes a
  // slot no one reads again: chunk q - 4's, done before the barrier that precedes it), so
  // every wave issues the same loads on every path: the compiler's own waits for X, which
  // count the loads after X on the path with the fewest, then never drain the ring.
  auto fill = [&](int q) {
    const uint32_t base = q < nq ? (uint32_t)chunk_of(q) * 4u * p.ldb_b : 0x80000000u;
    uint8_t* slot = ring + (q & (NR - 1)) * CH + (wave >> 1) * 8192 + (wave & 1) * 4096;
#pragma unroll
    for (int i = 0; i < 4; ++i) buf_load16_lds<kNonTemporal>(rw, slot + i * 1024, fv[i] + base, 0);
  };

  const Fused& e = p.ep;
  const bool fused = e.form == HKX_EP_FUSED;
  const bool ra_vec = fused && e.ra.p && e.ra.ld;
  // broadcast operands read (and their product formed) before any fill is issued: a use
  // after the fills would wait for every fill in flight (loads complete in order)
  const float cs_sc = (fused && e.cs.p) ? ld1(e.cs.p, e.cs.dt, 0) * e.cmul : (fused ? e.cmul : 1.0f);
  const float rs_sc = (fused && e.rs.p) ? ld1(e.rs.p, e.rs.dt, 0) : 1.0f;
  const float ra_sc = (fused && e.ra.p && !e.ra.ld) ? ld1(e.ra.p, e.ra.dt, 0) : 0.0f;
  const float sc = cs_sc * rs_sc;
  const float add0 = ra_sc + e.cadd;
  __builtin_amdgcn_sched_barrier(0);
  // group j's bias words (bf16 of unit stride, 4-byte aligned, N even): chunk c's 4 values
  // as 2 dwords at 8 c, by 4-byte DMA from 8 lanes of wave 0, a group ahead
  auto ep_load = [&](int j) {
    if (wave != 0 || !ra_vec) return;
    const int q = GC * j + (lane >> 1);
    const uint32_t off = lane < 8 && q < nq ? (uint32_t)(chunk_of(q) * 8 + 4 * (lane & 1)) : 0x7fffffffu;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(make_rsrc(e.ra.p, (uint32_t)p.N * 2u),
                                             (__attribute__((address_space(3))) void*)(ring + EPV + (j % 3) * EPS),
                                             4, off, 0, 0, 0);
  };
  const int nvec = ra_vec ? 1 : 0;

  // X: k-step t of this wave (4 w + t of each quarter): lane l holds token (l % 16) / 4,
  // quarter l % 4, the 8 values at 8 (l / 16) of the k-step (tokens past M read zero)
  i32x4 xr[4];
  {
    const int tl = (lane & 15) >> 2, sq = lane & 3, kq = lane >> 4;
#pragma unroll
    for (int t = 0; t < 4; ++t)
      xr[t] = buf_load16(rx, (uint32_t)tl * p.lda_b + sq * 2048 + (4 * wave + t) * 64 + kq * 16, 0);
  }
  // the A fragment's LDS offsets within a slot: lane l reads pseudo-row l % 16 = (r, s),
  // piece 128 s + 4 k + l / 16 of row r for k-step k
  uint32_t wa[4];
  {
    const int r = (lane & 15) >> 2, sq = lane & 3, kq = lane >> 4;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int gp = 128 * sq + 4 * (4 * wave + t) + kq;
      wa[t] = (uint32_t)(r * 8192 + ((gp ^ (4 * r + sq)) << 4));
    }
  }
  f32x4 acc[GC];
#pragma unroll
  for (int c = 0; c < GC; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto mma = [&](int q, f32x4& a) {
    const uint8_t* slot = ring + (q & (NR - 1)) * CH;
    i32x4 w[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) w[t] = *(const i32x4*)(slot + wa[t]);
#pragma unroll
    for (int t = 0; t < 4; ++t)
      a = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, w[t]),
                                                  __builtin_bit_cast(bf16x8, xr[t]), a, 0, 0, 0);
  };
  auto red_at = [&](int par, int w2, int c) {
    return (uint32_t)(RED + (((par * NW + w2) * GC + c) * 64));
  };
  // a group's quad sums: lane l's component l % 4 is row l / 16 of the chunk, token
  // (l % 16) / 4, quarter l % 4; the quad's four quarters summed, one lane of the quad
  // writes the float at (l / 4) % 16
  auto group_done = [&](int j) {
    const int sel = lane & 3;
#pragma unroll
    for (int c = 0; c < GC; ++c) {
        const f32x4 a = acc[c];
        float x = sel == 0 ? a.x : sel == 1 ? a.y : sel == 2 ? a.z : a.w;
        x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0xb1, 0xf, 0xf, false));  // quad_perm [1,0,3,2]
        x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x4e, 0xf, 0xf, false));  // quad_perm [2,3,0,1]
        if (sel == 0) *(float*)(ring + red_at(j & 1, wave, c) + (lane >> 2) * 4) = x;
        acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  // group j's outputs (wave 0): lane l is chunk l / 16 of the group, row (l / 4) % 4 of the
  // chunk, token l % 4
  auto finish = [&](int j) {
    const int c = lane >> 4, r = (lane >> 2) & 3, tl = lane & 3;
    const int q = GC * j + c;
    const int n = 4 * chunk_of(q) + r;
    const bool ok_n = q < nq && n < p.N;
    float add = add0;
    if (ra_vec) add = bf16_to_f32(*(const uint16_t*)(ring + EPV + (j % 3) * EPS + 8 * c + 2 * r)) + e.cadd;
    {
      float v = 0.f;
#pragma unroll
      for (int w2 = 0; w2 < NW; ++w2) v += *(const float*)(ring + red_at(j & 1, w2, c) + (lane & 15) * 4);
      const int m = tl;
      if (fused) v = act4(e.act, f32x4{v * sc + add, 0.f, 0.f, 0.f}).x;
      if (ok_n && m < p.M) {
        const int64_t idx = (int64_t)m * p.ldc + n;
        if (p.c_dt == HKX_BF16) ((uint16_t*)p.c)[idx] = (uint16_t)(pack_bf16x2(v, 0.f) & 0xffffu);
        else if (p.c_dt == HKX_FP16) ((uint16_t*)p.c)[idx] = (uint16_t)(pack_f16x2(v, 0.f) & 0xffffu);
        else if (p.c_dt == HKX_FP32) ((float*)p.c)[idx] = v;
        else if (p.c_dt == HKX_FP8E4M3) ((uint8_t*)p.c)[idx] = (uint8_t)f32_to_e4m3(v);
        else ((uint8_t*)p.c)[idx] = (uint8_t)f32_to_i8(v);
      }
    }
  };
  // chunk q landed (with X before it) and every wave is done with chunk q - 1, whose slot
  // the fill of q + 3 takes: the loads issued after f(q) are f(q + 1) and f(q + 2), 4 a wave
  // each, and, on wave 0 at the group's second chunk, the bias DMA of the next group;
  // lgkmcnt(0) as well
  auto wait_chunk = [&](bool ep_before) {
    if (ep_before && wave == 0 && nvec) __builtin_amdgcn_s_waitcnt(wait_vm_dec(9) & ~(15 << 8));
    else __builtin_amdgcn_s_waitcnt(wait_vm_dec(8) & ~(15 << 8));
  };

  ep_load(0);
  __builtin_amdgcn_sched_barrier(0);  // the bias and X before the fills: the waits count in order
  fill(0);
  fill(1);
  fill(2);
  const int ngr = (nq + GC - 1) / GC;
  for (int j = 0; j < ngr; ++j) {
#pragma unroll
    for (int c = 0; c < GC; ++c) {
      const int q = GC * j + c;
      if (q < nq) {
        wait_chunk(c == 1 && GC * (j + 1) < nq);
        __builtin_amdgcn_s_barrier();
        if (c == 0 && GC * (j + 1) < nq) ep_load(j + 1);  // older than the fill of q + 3
        __builtin_amdgcn_sched_barrier(0);
        fill(q + 3);
        if (c == 0 && j > 0 && wave == 0) finish(j - 1);
        mma(q, acc[c]);
      }
    }
    group_done(j);
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the last partial sums written
  __builtin_amdgcn_s_barrier();
  if (wave == 0) finish(ngr - 1);
  __builtin_amdgcn_s_waitcnt(wait_vm_dec(0));  // no fill lands in LDS after the exit
}

// The whole-row decode GEMM in short workgroups: the rows kernel's chunks, MFMA form and
// epilogue, but each workgroup takes CPW consecutive chunks (CPW x 32 KB of W, contiguous)
// and ends, so the grid is N / (4 CPW) workgroups, two (CPW = 2) or four (CPW = 1) resident
// on a CU at once, and the dispatcher hands a CU its next workgroup when one ends: the
// chunks even out over a CU's lifetime instead of being fixed at launch. All of a
// workgroup's fills are issued at its start (X, then on wave 0 the bias values, then the
// chunks in order), chunk j is multiplied once its fills land, and wave 0 sums the waves'
// quad sums, applies the epilogue and stores after the last.
template <int CPW>
__global__ void __launch_bounds__(512) rowsq_kernel(const DecodeArgs p) {
  constexpr int NW = 8;
  constexpr int CH = 32768;  // a chunk: 4 rows x 8 KB
  constexpr int RED = CPW * CH;
  __shared__ __attribute__((aligned(16))) uint8_t ring[RED + NW * CPW * 64];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nck = (p.N + 3) / 4;
  const int c0 = blockIdx.x * CPW;  // this workgroup's first chunk
  if (c0 >= nck) return;

  const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.b, p.b_bytes);
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.a, p.a_bytes);
  uint32_t fv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = wave >> 1, P = (wave & 1) * 256 + i * 64 + lane;
    fv[i] = (uint32_t)r * p.ldb_b + (uint32_t)((P ^ (4 * r + (P >> 7))) << 4);
  }
  // chunks past N (the last workgroup's second) are filled out of range: they read zeros
  // and are never stored, and every wave issues the same loads
  auto fill = [&](int j) {
    const uint32_t base = c0 + j < nck ? (uint32_t)(c0 + j) * 4u * p.ldb_b : 0x80000000u;
    uint8_t* slot = ring + j * CH + (wave >> 1) * 8192 + (wave & 1) * 4096;
#pragma unroll
    for (int i = 0; i < 4; ++i) buf_load16_lds<kNonTemporal>(rw, slot + i * 1024, fv[i] + base, 0);
  };

  const Fused& e = p.ep;
  const bool fused = e.form == HKX_EP_FUSED;
  const bool ra_vec = fused && e.ra.p && e.ra.ld;
  const float cs_sc = (fused && e.cs.p) ? ld1(e.cs.p, e.cs.dt, 0) * e.cmul : (fused ? e.cmul : 1.0f);
  const float rs_sc = (fused && e.rs.p) ? ld1(e.rs.p, e.rs.dt, 0) : 1.0f;
  const float ra_sc = (fused && e.ra.p && !e.ra.ld) ? ld1(e.ra.p, e.ra.dt, 0) : 0.0f;
  const float sc = cs_sc * rs_sc;
  const float add0 = ra_sc + e.cadd;

  // X, as the rows kernel holds it: lane l token (l % 16) / 4, quarter l % 4, k-steps
  // 4 w .. 4 w + 3 of each quarter
  i32x4 xr[4];
  {
    const int tl = (lane & 15) >> 2, sq = lane & 3, kq = lane >> 4;
#pragma unroll
    for (int t = 0; t < 4; ++t)
      xr[t] = buf_load16(rx, (uint32_t)tl * p.lda_b + sq * 2048 + (4 * wave + t) * 64 + kq * 16, 0);
  }
  // wave 0, lane l: the bias of chunk l / 16's row (l / 4) % 4 (bf16, unit stride)
  const int fc = lane >> 4, fr = (lane >> 2) & 3, ftl = lane & 3;
  const int fn = 4 * (c0 + fc) + fr;
  const bool f_ok = fc < CPW && c0 + fc < nck && fn < p.N;
  // (one buffer load on every lane of every wave, out of range where unused: a load under
  // a branch gets a wait of its own at the branch's end, before the fills)
  const uint16_t bias_w = __builtin_amdgcn_raw_buffer_load_b16(
      make_rsrc(ra_vec ? e.ra.p : nullptr, ra_vec ? (uint32_t)p.N * 2u : 0u),
      f_ok && wave == 0 ? (uint32_t)fn * 2u : 0x7ffffff0u, 0, 0);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < CPW; ++j) fill(j);

  uint32_t wa[4];
  {
    const int r = (lane & 15) >> 2, sq = lane & 3, kq = lane >> 4;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int gp = 128 * sq + 4 * (4 * wave + t) + kq;
      wa[t] = (uint32_t)(r * 8192 + ((gp ^ (4 * r + sq)) << 4));
    }
  }
  f32x4 acc[CPW];
#pragma unroll
  for (int j = 0; j < CPW; ++j) {
    // chunk j's fills landed in every wave (the newer chunks' 4 a wave may still run)
    if (j == CPW - 1) __builtin_amdgcn_s_waitcnt(wait_vm_dec(0) & ~(15 << 8));
    else if (CPW - 1 - j == 1) __builtin_amdgcn_s_waitcnt(wait_vm_dec(4) & ~(15 << 8));
    else if (CPW - 1 - j == 2) __builtin_amdgcn_s_waitcnt(wait_vm_dec(8) & ~(15 << 8));
    else __builtin_amdgcn_s_waitcnt(wait_vm_dec(12) & ~(15 << 8));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    const uint8_t* slot = ring + j * CH;
    i32x4 w[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) w[t] = *(const i32x4*)(slot + wa[t]);
    f32x4 a = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 4; ++t)
      a = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, w[t]),
                                                  __builtin_bit_cast(bf16x8, xr[t]), a, 0, 0, 0);
    acc[j] = a;
  }
  // the quad sums (lane l's component l % 4: row l / 16 of the chunk, token (l % 16) / 4,
  // quarter l % 4), one float a (row, token) at (l / 4) % 16 of the wave's slot
  {
    const int sel = lane & 3;
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      const f32x4 a = acc[j];
      float x = sel == 0 ? a.x : sel == 1 ? a.y : sel == 2 ? a.z : a.w;
      x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0xb1, 0xf, 0xf, false));
      x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x4e, 0xf, 0xf, false));
      if (sel == 0) *(float*)(ring + RED + (wave * CPW + j) * 64 + (lane >> 2) * 4) = x;
    }
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  if (wave != 0 || fc >= CPW) return;
  // lane l: chunk l / 16, row (l / 4) % 4, token l % 4
  float v = 0.f;
#pragma unroll
  for (int w2 = 0; w2 < NW; ++w2) v += *(const float*)(ring + RED + (w2 * CPW + fc) * 64 + (lane & 15) * 4);
  if (fused) v = act4(e.act, f32x4{v * sc + (ra_vec ? bf16_to_f32(bias_w) + e.cadd : add0), 0.f, 0.f, 0.f}).x;
  if (f_ok && ftl < p.M) {
    const int64_t idx = (int64_t)ftl * p.ldc + fn;
    if (p.c_dt == HKX_BF16) ((uint16_t*)p.c)[idx] = (uint16_t)(pack_bf16x2(v, 0.f) & 0xffffu);
    else if (p.c_dt == HKX_FP16) ((uint16_t*)p.c)[idx] = (uint16_t)(pack_f16x2(v, 0.f) & 0xffffu);
    else if (p.c_dt == HKX_FP32) ((float*)p.c)[idx] = v;
    else if (p.c_dt == HKX_FP8E4M3) ((uint8_t*)p.c)[idx] = (uint8_t)f32_to_e4m3(v);
    else ((uint8_t*)p.c)[idx] = (uint8_t)f32_to_i8(v);
  }
}

// The per-wave whole-row decode GEMM: K = 512 KS (KS = 2 or 4: K = 1024 or 2048), M <= 2
// (M <= 3 at K = 1024), the fast epilogue form without a tile operand. The workgroups take chunks of 8
// consecutive rows of W strided over the grid (workgroup g: chunks g, g + G, ...), and wave w
// takes row w of each: it streams its own rows into its own two LDS slots (a row is 2K
// bytes, one DMA instruction a KB), so no wave waits for another -- there is no barrier in
// the kernel. A row's whole K goes through one MFMA chain: the 16 rows of the MFMA are the
// row's 16 K segments (K / 16 each), and X enters as 16 columns, the same 16 segments of one
// token, so the row's dot product with the token is the trace of the 16 x 16 result -- the
// sum of one component in each of 16 lanes. Each row's result (the epilogue applied) waits in
// the lane of its index; all of a wave's rows are stored at the end, after its last fill
// (a store among the fills would enter the waits, which count loads and stores together).
// Against the whole-row kernel above, this removes the per-chunk barrier and the cross-wave
// sums of each group (and their tail after the last chunk). Measured on one box against the
// kernels that take these calls otherwise (graph replays over four rotated weights): at K =
// 1024 and 2048, M <= 2, 5-20% faster (12288 x 1024 at M = 1: 7.76 -> 6.23 us; 24576 x 2048:
// 18.16 -> 16.45); at K = 4096 (KS = 8, 160 KB of LDS) level at M = 1 and up to 10% slower from
// M = 2 and at N past 12288 -- there the whole-row kernel above stays. With more tokens each
// row's MFMA chains and trace sums lengthen the walk, and only two rows a wave are in flight.
//
// LDS: wave w's slots at 2 w RB and (2 w + 1) RB, RB = 2K bytes. A row's 16-byte pieces are
// XOR-swizzled within each 256-byte block by the block's segment (applied on the global side
// of the DMA), so the 16 lanes reading one k-step of the 16 segments hit 16 different banks.
template <int KS>
__device__ __forceinline__ uint32_t roww_swz(uint32_t piece) {  // physical <-> logical piece
  const uint32_t h = piece >> 4;  // its 256-byte block
  const uint32_t f = KS == 8 ? (h >> 1) & 15u : (KS == 4 ? h & 15u : h & 7u);
  return piece ^ f;
}

template <int KS>
__global__ void __launch_bounds__(512) roww_kernel(const DecodeArgs p) {
  constexpr int RB = KS * 1024;  // a row's bytes (K = 512 KS bf16)
  constexpr int MT = 4;          // tokens at most
  constexpr int XOFF = 16 * RB;  // then X: MT rows of RB bytes, laid out as W's rows
  __shared__ __attribute__((aligned(16))) uint8_t ring[XOFF + MT * RB];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nck = (p.N + 7) / 8;
  const int G = gridDim.x, g = blockIdx.x;
  if (g >= nck) return;  // (no barrier anywhere below)
  const int nq = (nck - g + G - 1) / G;  // rows of this wave: 8 (g + q G) + wave
  auto row_of = [&](int q) { return 8 * (g + q * G) + wave; };

  const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.b, p.b_bytes);
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.a, p.a_bytes);
  const Fused& e = p.ep;
  const bool fused = e.form == HKX_EP_FUSED;
  const bool ra_vec = fused && e.ra.p && e.ra.ld;
  const float cs_sc = (fused && e.cs.p) ? ld1(e.cs.p, e.cs.dt, 0) * e.cmul : (fused ? e.cmul : 1.0f);
  const float rs_sc = (fused && e.rs.p) ? ld1(e.rs.p, e.rs.dt, 0) : 1.0f;
  const float ra_sc = (fused && e.ra.p && !e.ra.ld) ? ld1(e.ra.p, e.ra.dt, 0) : 0.0f;
  const float sc = cs_sc * rs_sc;
  const float add0 = ra_sc + e.cadd;

  // the fragment offsets within a slot: lane l reads segment l % 16, k-group l / 16
  uint32_t fo[KS];
#pragma unroll
  for (int k = 0; k < KS; ++k)
    fo[k] = roww_swz<KS>((uint32_t)((lane & 15) * 4 * KS + k * 4 + (lane >> 4))) * 16u;
  // the DMA's per-lane global offsets: instruction u's lane fills physical piece 64 u + l
  uint32_t dv[KS];
#pragma unroll
  for (int u = 0; u < KS; ++u) dv[u] = roww_swz<KS>((uint32_t)(64 * u + lane)) * 16u;
  // Row q into slot q & 1; past the last row the fill is still issued, out of range (it reads
  // nothing and writes a slot already read), so every step waits for the same count.
  auto fill = [&](int q) {
    const uint32_t base = q < nq ? (uint32_t)row_of(q) * p.ldb_b : 0x80000000u;
    uint8_t* slot = ring + (2 * wave + (q & 1)) * RB;
#pragma unroll
    for (int u = 0; u < KS; ++u) buf_load16_lds<kNonTemporal>(rw, slot + u * 1024, dv[u] + base, 0);
  };
  // the biases of this wave's rows, row q's in lane q, loaded with X before the first fill
  // (a load in the loop would make the compiler wait for every fill in flight)
  float bias_l = 0.f;
  if (ra_vec && lane < nq && row_of(lane) < p.N) bias_l = ld1(e.ra.p, HKX_BF16, row_of(lane));
  // the rows' results, row q's in lane q (token t in res[t])
  float res[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) res[t] = 0.f;
  const bool diag = ((lane & 15) >> 2) == (lane >> 4);  // lanes holding a trace element
  // X: staged once a workgroup, by wave 0's DMA, in W's row layout (its M rows; rows past M
  // read zero), so each wave reads its fragments from LDS rather than from L2 -- every wave
  // loading all of X measured 1.3-1.6x slower at M = 4. Then each wave's X fragments (token
  // t, lane l: segment l % 16, k-group l / 16, k-step k) go to registers for the whole walk.
  if (wave == 0) {
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int u = 0; u < KS; ++u)
        buf_load16_lds(rx, ring + XOFF + t * RB + u * 1024, dv[u] + (uint32_t)t * p.lda_b, 0);
  }
  __builtin_amdgcn_sched_barrier(0);  // X before the fills: the waits count in order
  fill(0);
  fill(1);
  // X landed (wave 0's DMA, older than its fills); a bare barrier: __syncthreads() would
  // also wait for every fill in flight
  if (wave == 0) __builtin_amdgcn_s_waitcnt(wait_vm_dec(2 * KS));
  __builtin_amdgcn_s_barrier();
  i32x4 xr[MT][KS];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int k = 0; k < KS; ++k)
      xr[t][k] = t < p.M ? *(const i32x4*)(ring + XOFF + t * RB + fo[k]) : i32x4{0, 0, 0, 0};
  for (int q = 0; q < nq; ++q) {
    // row q landed (the KS loads of row q + 1 may still be in flight); lgkmcnt(0)
    __builtin_amdgcn_s_waitcnt(wait_vm_dec(KS) & ~(15 << 8));
    const float add = ra_vec ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, bias_l), q)) + e.cadd
                             : add0;
    const uint8_t* slot = ring + (2 * wave + (q & 1)) * RB;
    i32x4 w[KS];
#pragma unroll
    for (int k = 0; k < KS; ++k) w[k] = *(const i32x4*)(slot + fo[k]);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the slot is read
    __builtin_amdgcn_sched_barrier(0);
    fill(q + 2);
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      if (t < p.M) {
        f32x4 a = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < KS; ++k)
          a = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, w[k]),
                                                      __builtin_bit_cast(bf16x8, xr[t][k]), a, 0, 0, 0);
        // the trace: lane l holds D[4 (l / 16) + c][l % 16]; the diagonal is component l % 4
        // of the lanes with (l % 16) / 4 == l / 16 (lanes 0-3, 20-23, 40-43, 60-63)
        const int sel = lane & 3;
        float x = diag ? (sel == 0 ? a.x : sel == 1 ? a.y : sel == 2 ? a.z : a.w) : 0.f;
        x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0xb1, 0xf, 0xf, false));
        x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x4e, 0xf, 0xf, false));
        const float v =
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 0)) +
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 20)) +
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 40)) +
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 60));
        float o = v * sc + add;
        if (fused) o = act4(e.act, f32x4{o, 0.f, 0.f, 0.f}).x;
        res[t] = lane == q ? o : res[t];
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(wait_vm_dec(0));  // every fill landed (none lands after the exit)
  // the stores: lane q holds row q's results
  if (lane < nq) {
    const int n = row_of(lane);
    if (n < p.N) {
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        if (t < p.M) {
          const int64_t idx = (int64_t)t * p.ldc + n;
          const float v = res[t];
          if (p.c_dt == HKX_BF16) ((uint16_t*)p.c)[idx] = (uint16_t)(pack_bf16x2(v, 0.f) & 0xffffu);
          else if (p.c_dt == HKX_FP16) ((uint16_t*)p.c)[idx] = (uint16_t)(pack_f16x2(v, 0.f) & 0xffffu);
          else if (p.c_dt == HKX_FP32) ((float*)p.c)[idx] = v;
          else if (p.c_dt == HKX_FP8E4M3) ((uint8_t*)p.c)[idx] = (uint8_t)f32_to_e4m3(v);
          else ((uint8_t*)p.c)[idx] = (uint8_t)f32_to_i8(v);
        }
      }
    }
  }
}

// Whether the per-wave whole-row kernel takes a call: K = 1024 (M <= 3) or 2048 (M <= 2), the
// fast epilogue form without a tile operand, 64 or fewer rows a wave (results wait one a
// lane: N <= 131072 on 256 workgroups), row offsets within 31 bits.
bool roww_takes(const DecodeArgs& a, int grid) {
  const bool tile = a.ep.form == HKX_EP_FUSED && a.ep.ta.p;
  const int ks = a.g_total / 4;  // 128-element groups / 4 = K / 512
  const int nck = (a.N + 7) / 8;
  return ((ks == 2 && a.M <= 3) || (ks == 4 && a.M <= 2)) && a.g_total % 4 == 0 &&
         stream_fast(a) && !tile && (nck + grid - 1) / grid <= 64 &&
         (int64_t)a.N * a.ldb_b < (1LL << 31);
}

hipError_t launch_roww(const DecodeArgs& a, dim3 grid, hipStream_t s) {
  switch (a.g_total / 4) {
    case 2: hipLaunchKernelGGL(roww_kernel<2>, grid, dim3(512), 0, s, a); break;
    case 4: hipLaunchKernelGGL(roww_kernel<4>, grid, dim3(512), 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Whether the whole-row kernels take a call the stream kernel takes: K = 4096, M <= 4, the
// fast epilogue form without a tile operand; N up to 32768, and at M <= 2 (the short
// workgroups of one chunk) any N whose W spans less than 2 GiB (chunk offsets and the
// out-of-range fill offset within 31 bits). At the LM heads' N the short workgroups beat the
// stream kernel at M = 1 (151936 x 4096: 177.7 against 189.2 us, 7.0 TB/s; 128256: 150.3
// against 156.4; 65536: 75.3 against 82.3, one box) and tie or win at M = 2; from M = 3
// (two chunks a workgroup, or the persistent kernel) they lose there (151936 at M = 4:
// 194.2 against 189.5), so those stay at N <= 32768.
bool rows_takes(const DecodeArgs& a) {
  const bool tile = a.ep.form == HKX_EP_FUSED && a.ep.ta.p;
  const bool n_ok = a.M <= 2 ? (int64_t)a.N * a.ldb_b < (1LL << 31) : a.N <= 32768;
  return a.g_total == 32 && a.M <= 4 && n_ok && stream_fast(a) && !tile;
}

// The whole-row form a call runs: short workgroups of one chunk at M <= 2 and of two at
// M = 3, and at M = 4 up to N = 8192; the persistent rows_kernel at M = 4 past that, where
// each short workgroup's own copy of X (at M = 4 as many bytes as a chunk of W) costs more
// than the dispatcher's balancing gains. Measured on one box, graph replays over four
// rotated weights, K = 4096 (persistent -> short, us): N = 12288 M = 1 16.95 -> 16.18, M = 2
// 17.01 -> 16.65, M = 4 17.15 -> 19.50 (one chunk) / 17.61 (two); N = 28672 M = 1 36.68 ->
// 34.32; N = 6144 M = 4 10.63 -> 9.93 (two); N = 4096 M = 3 8.07 -> 7.21 (two).
hipError_t launch_rows(const DecodeArgs& a, dim3 grid, hipStream_t s) {
  const int nck = (a.N + 3) / 4;
  if (a.M <= 2)
    hipLaunchKernelGGL(rowsq_kernel<1>, dim3(nck), dim3(512), 0, s, a);
  else if (a.M == 3 || a.N <= 8192)
    hipLaunchKernelGGL(rowsq_kernel<2>, dim3((nck + 1) / 2), dim3(512), 0, s, a);
  else
    hipLaunchKernelGGL(rows_kernel, grid, dim3(512), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_stream(const DecodeArgs& a, dim3 grid, hipStream_t s) {
  if (a.M > 16)
    return stream_fast(a) ? launch_stream_ep<kStreamEpFast, 2>(a, grid, s)
                          : launch_stream_ep<kStreamEpGeneric, 2>(a, grid, s);
  return stream_fast(a) ? launch_stream_ep<kStreamEpFast, 1>(a, grid, s)
                        : launch_stream_ep<kStreamEpGeneric, 1>(a, grid, s);
}

}  // namespace hkx
