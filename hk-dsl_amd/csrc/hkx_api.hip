#include <algorithm>
// The C ABI of libhkx.so (include/hkx.h): argument checks, the plan of launches for a
// call, and the launches on the caller's stream. Stateless and reentrant; the only
// state is each thread's last error message.
//
// A call is the launches hk.templates.gemm's prepare() makes for a plan
// (python/hk/templates/gemm.py:577-665): one GEMM kernel that carries the epilogue, or
// a GEMM kernel that stores fp32 shares and a reduction that sums them in order and
// runs the epilogue once (gemm.py:500-502; python/hk/ops/gemm_cdna_dp.py:295-324).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "hkx.h"
#include "hkx_launch.hpp"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int elem_bytes(int dt) {
  switch (dt) {
    case HKX_BF16:
    case HKX_FP16: return 2;
    case HKX_FP32: return 4;
    case HKX_FP8E4M3:
    case HKX_FP8E5M2:
    case HKX_FP8_E4M3_E5M2:
    case HKX_FP8_E5M2_E4M3:
    case HKX_INT8: return 1;
    default: return 0;
  }
}

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

// A call resolved: which kernel, its shape parameters, how C leaves it.
struct Plan {
  int kernel;     // HKX_KERNEL_TILE / _DECODE
  int tile_m, tile_n, wm;
  int schedule;   // HKX_TILE_RING: ring_kernel, _PINGPONG: pp_kernel, _W4: tile4_kernel,
                  // _W8: tile_kernel
  int variant;
  int waves, fn, mf;  // decode
  int splits;     // effective (no empty split)
  int kunits;     // TILE: 128-byte K stages; DECODE: 128-element K groups
  int kper;       // units per split
  bool pair;
  bool via_ws;    // fp32 shares / sum to ws, then the reduction
  size_t ws_bytes;
  // HKX_RING_STREAMK: columns [0, sk_cut) in whole waves of ring tiles, the rest of N on
  // ring tiles split sk_splits ways over K (sk_kper units each) into the workspace
  int sk_cut, sk_splits, sk_kper;
  // DECODE split over K, unpaired, not a program: the counters it can finish with (one a
  // block of rows), and whether this call does (counters given)
  int ncnt;
  bool arrive;
};

int cu_count();
int wave_cut(int m, int n, int outw);

bool tile_shape_ok(int bm, int bn) {
  return (bm == 256 && bn == 256) || (bm == 128 && bn == 256) || (bm == 64 && bn == 256) ||
         (bm == 128 && bn == 128) || (bm == 256 && bn == 128) || (bm == 64 && bn == 128);
}

int wave_rows(int bm, int bn) {  // waves along M for a tile shape
  if (bm == 64) return 1;
  if (bm == 256 && bn == 128) return 4;
  return 2;
}

// The choice hkx_gemm makes for HKX_KERNEL_AUTO; the Python layer (hk.ops.gemm_cdna.route)
// normally passes an explicit one.
bool e5m2_pair(int dt) {
  return dt == HKX_FP8E5M2 || dt == HKX_FP8_E4M3_E5M2 || dt == HKX_FP8_E5M2_E4M3;
}

// The tile kernels' operand-format code (TileArgs::ab_fmt) of an ab_dtype.
int fmt_of(int dt) {
  switch (dt) {
    case HKX_FP8E4M3: return 1;
    case HKX_FP8E5M2: return 2;
    case HKX_FP8_E4M3_E5M2: return 3;
    case HKX_FP8_E5M2_E4M3: return 4;
    default: return 0;
  }
}

void auto_choose(const HkxGemmArgs* a, int* kernel, int* bm, int* bn, int* splits) {
  const int m = a->m, n = a->n;
  const bool pair = a->ep.form == HKX_EP_SILU_MUL;
  if (m <= 32 && a->ab_dtype == HKX_BF16 && (a->k % 128) == 0) {
    *kernel = HKX_KERNEL_DECODE;
    *bm = 0; *bn = 0;
    const int per_wg = pair ? 16 : 16;
    const int wgs = (n + per_wg - 1) / per_wg;
    *splits = wgs >= 512 ? 1 : (wgs >= 128 ? 4 : 8);
    return;
  }
  *kernel = HKX_KERNEL_TILE;
  *bm = m <= 64 ? 64 : (m <= 128 ? 128 : 256);
  *bn = 256;
  const int outw = pair ? *bn / 2 : *bn;
  const long tiles = (long)((m + *bm - 1) / *bm) * ((n + outw - 1) / outw);
  const int kunits = a->k * elem_bytes(a->ab_dtype) / 128;
  int s = 1;
  while (tiles * s * 2 <= 256 && kunits / (s * 2) >= 8) s *= 2;
  *splits = s;
}

int check_operand(const HkxOperand& o, int i) {
  if (!o.ptr) return fail(HKX_ERR_ARG, "epilogue operand %d: null pointer", i);
  if (o.kind != HKX_ROW && o.kind != HKX_COL && o.kind != HKX_TILE)
    return fail(HKX_ERR_ARG, "epilogue operand %d: kind %d is not ROW, COL or TILE", i, o.kind);
  const int eb = (o.dtype == HKX_BF16 || o.dtype == HKX_FP16) ? 2 : (o.dtype == HKX_FP32 ? 4 : 0);
  if (!eb)
    return fail(HKX_ERR_DTYPE, "epilogue operand %d: dtype %d; operands are bf16, fp16 or fp32", i,
                o.dtype);
  const size_t vec = 4 * eb;  // four elements are loaded at once
  if (o.kind == HKX_ROW && o.ld != 0 && !aligned(o.ptr, vec))
    return fail(HKX_ERR_SHAPE, "epilogue operand %d: a row vector must be %zu-byte aligned", i, vec);
  if (o.kind == HKX_TILE && (!aligned(o.ptr, vec) || (o.ld * eb) % vec || o.ld < 0))
    return fail(HKX_ERR_SHAPE,
                "epilogue operand %d: a tile operand must be %zu-byte aligned, rows too", i, vec);
  if (o.kind == HKX_COL && (o.ld < 0 || !aligned(o.ptr, eb)))
    return fail(HKX_ERR_SHAPE, "epilogue operand %d: a column vector needs a row stride >= 0", i);
  return HKX_OK;
}

int check_epilogue(const HkxEpilogue& ep) {
  if (ep.nops < 0 || ep.nops > HKX_MAX_OPERANDS)
    return fail(HKX_ERR_ARG, "epilogue: %d operands (at most %d)", ep.nops, HKX_MAX_OPERANDS);
  for (int i = 0; i < ep.nops; ++i) {
    int rc = check_operand(ep.ops[i], i);
    if (rc) return rc;
  }
  switch (ep.form) {
    case HKX_EP_NONE:
    case HKX_EP_SILU_MUL: return HKX_OK;
    case HKX_EP_FUSED: {
      const int idx[4] = {ep.col_scale, ep.row_scale, ep.row_add, ep.tile_add};
      const int kind[4] = {HKX_COL, HKX_ROW, HKX_ROW, HKX_TILE};
      const char* what[4] = {"col_scale", "row_scale", "row_add", "tile_add"};
      for (int s = 0; s < 4; ++s) {
        if (idx[s] < -1 || idx[s] >= ep.nops)
          return fail(HKX_ERR_ARG, "fused epilogue: %s names operand %d of %d", what[s], idx[s],
                      ep.nops);
        if (idx[s] >= 0 && ep.ops[idx[s]].kind != kind[s])
          return fail(HKX_ERR_ARG, "fused epilogue: %s is operand %d, of the wrong kind", what[s],
                      idx[s]);
      }
      if (ep.act < HKX_ACT_NONE || ep.act > HKX_ACT_RELU)
        return fail(HKX_ERR_ARG, "fused epilogue: activation %d", ep.act);
      return HKX_OK;
    }
    case HKX_EP_PROGRAM: {
      if (ep.nins < 0 || ep.nins > HKX_MAX_INSTR)
        return fail(HKX_ERR_ARG, "epilogue program: %d instructions (at most %d)", ep.nins,
                    HKX_MAX_INSTR);
      if (ep.out_reg < 0 || ep.out_reg >= HKX_MAX_REGS)
        return fail(HKX_ERR_ARG, "epilogue program: output register %d", ep.out_reg);
      for (int i = 0; i < ep.nins; ++i) {
        const HkxInstr& I = ep.ins[i];
        if (I.op >= HKX_NUM_OPS || I.dst >= HKX_MAX_REGS || I.a >= HKX_MAX_REGS ||
            I.b >= HKX_MAX_REGS || I.c >= HKX_MAX_REGS)
          return fail(HKX_ERR_ARG, "epilogue program: instruction %d is malformed", i);
        if (I.op == HKX_OP_LOAD && I.a >= ep.nops)
          return fail(HKX_ERR_ARG, "epilogue program: instruction %d loads operand %d of %d", i,
                      I.a, ep.nops);
      }
      return HKX_OK;
    }
    default: return fail(HKX_ERR_ARG, "epilogue form %d", ep.form);
  }
}

int make_plan(const HkxGemmArgs* a, Plan* p) {
  if (!a) return fail(HKX_ERR_ARG, "null args");
  if (!a->a || !a->b || !a->c) return fail(HKX_ERR_ARG, "A, B and C must be device pointers");
  if (a->m < 1 || a->k < 1 || a->n < 1)
    return fail(HKX_ERR_SHAPE, "M=%d, N=%d, K=%d; nothing to multiply", a->m, a->n, a->k);
  if (a->ab_dtype != HKX_BF16 && a->ab_dtype != HKX_FP8E4M3 && !e5m2_pair(a->ab_dtype))
    return fail(HKX_ERR_DTYPE, "A and B are bf16, fp8-e4m3 or an e5m2 pair (dtype %d)",
                a->ab_dtype);
  const int ob = elem_bytes(a->c_dtype);
  if (!ob || a->c_dtype > HKX_INT8) return fail(HKX_ERR_DTYPE, "C dtype %d", a->c_dtype);
  const int eb = elem_bytes(a->ab_dtype);
  const int kstep = 128 / eb;
  if (a->k % kstep || a->n % 4)
    return fail(HKX_ERR_SHAPE, "K=%d must be a multiple of %d and N=%d of 4; M may be anything",
                a->k, kstep, a->n);
  if (a->lda < a->k || a->ldb < a->k || a->ldc < a->n)
    return fail(HKX_ERR_SHAPE, "row strides lda=%lld ldb=%lld ldc=%lld are below K / N",
                (long long)a->lda, (long long)a->ldb, (long long)a->ldc);
  if (!aligned(a->a, 16) || !aligned(a->b, 16) || (a->lda * eb) % 16 || (a->ldb * eb) % 16)
    return fail(HKX_ERR_SHAPE, "A and B need 16-byte aligned rows (base and row stride)");
  if (!aligned(a->c, 4 * ob) || a->ldc % 4)
    return fail(HKX_ERR_SHAPE, "C needs %d-byte alignment and a row stride a multiple of 4",
                4 * ob);
  const bool pair = a->ep.form == HKX_EP_SILU_MUL;
  const long long brows = pair ? 2LL * a->n : a->n;
  if ((long long)a->m * a->lda * eb >= (1LL << 32) || brows * a->ldb * eb >= (1LL << 32))
    return fail(HKX_ERR_SHAPE, "A or B spans 4 GiB or more; split the call");
  int rc = check_epilogue(a->ep);
  if (rc) return rc;

  int kernel = a->kernel, bm = a->tile_m, bn = a->tile_n, splits = a->splits;
  if (kernel == HKX_KERNEL_AUTO) auto_choose(a, &kernel, &bm, &bn, &splits);
  if (splits < 1) splits = 1;
  if (e5m2_pair(a->ab_dtype) && pair)
    return fail(HKX_ERR_ARG, "the paired silu-and-mul epilogue is not built for e5m2 operands "
                "(bf16 and fp8-e4m3 only)");
  if (e5m2_pair(a->ab_dtype) &&
      (kernel != HKX_KERNEL_TILE || bm != 256 || bn != 256 ||
       (a->tile_schedule != HKX_TILE_RING && a->tile_schedule != HKX_TILE_AUTO) || a->variant))
    return fail(HKX_ERR_ARG, "e5m2 operands run on the 256x256 ring tile kernel "
                "(kernel TILE, tile 256x256, schedule ring or auto, variant 0)");
  p->kernel = kernel;
  p->pair = pair;
  if (kernel == HKX_KERNEL_TILE) {
    if (!tile_shape_ok(bm, bn))
      return fail(HKX_ERR_ARG, "tile %dx%d: 256x256, 128x256, 64x256, 128x128, 256x128 or 64x128",
                  bm, bn);
    p->tile_m = bm;
    p->tile_n = bn;
    p->wm = wave_rows(bm, bn);
    const bool four_ok = (bn == 256 && (bm == 256 || bm == 128 || bm == 64)) ||
                         (bn == 128 && (bm == 128 || bm == 64));
    const bool eight_ok = !(bm == 64 && bn == 128);
    const bool pp_ok = bn == 256 && bm == 256;
    int sc = a->tile_schedule;
    if (sc == HKX_TILE_AUTO) sc = pp_ok ? HKX_TILE_RING : (four_ok ? HKX_TILE_W4 : HKX_TILE_W8);
    if (sc != HKX_TILE_PINGPONG && sc != HKX_TILE_W4 && sc != HKX_TILE_W8 && sc != HKX_TILE_RING)
      return fail(HKX_ERR_ARG, "tile_schedule %d", a->tile_schedule);
    // RING at 128 x 256: the quadrant kernel's 128-row form (where it takes the call; else
    // the 4-wave kernel), no variant bits
    const bool q128 = bm == 128 && bn == 256;
    if (sc == HKX_TILE_RING && !pp_ok && !q128)
      return fail(HKX_ERR_ARG, "the ring tile kernel takes 256x256 tiles (128x256: its quadrant form)");
    if (sc == HKX_TILE_RING && q128 && a->variant)
      return fail(HKX_ERR_ARG, "variant %d: the 128x256 quadrant form has none", a->variant);
    if (sc == HKX_TILE_W4 && !four_ok)
      return fail(HKX_ERR_ARG, "the 4-wave tile kernel takes 256x256, 128x256, 64x256, 128x128 "
                  "or 64x128 tiles");
    if (sc == HKX_TILE_W8 && !eight_ok)
      return fail(HKX_ERR_ARG, "the 8-wave tile kernel takes 256x256, 128x256, 64x256, 128x128 "
                  "or 256x128 tiles");
    if (sc == HKX_TILE_PINGPONG && !pp_ok)
      return fail(HKX_ERR_ARG, "the ping-pong tile kernel takes 256x256 tiles");
    if (sc == HKX_TILE_RING ? (a->variant & ~(HKX_RING_WAVESPLIT | HKX_RING_STREAMK | HKX_RING_HALFSTAGE)) != 0 ||
                                  (a->variant & HKX_RING_WAVESPLIT && a->variant & HKX_RING_STREAMK)
                            : (a->variant & ~(HKX_PP_MFMA32 | HKX_PP_ONE_TILE)) != 0 ||
                                  (a->variant && sc != HKX_TILE_PINGPONG))
      return fail(HKX_ERR_ARG, "variant %d", a->variant);
    p->schedule = sc;
    p->variant = a->variant;
    p->kunits = a->k * eb / 128;
  } else if (kernel == HKX_KERNEL_DECODE) {
    if (a->ab_dtype != HKX_BF16) return fail(HKX_ERR_DTYPE, "the decode kernel takes bf16");
    if (a->m > 32) return fail(HKX_ERR_SHAPE, "the decode kernel takes M <= 32 (M=%d)", a->m);
    if (a->k % 128) return fail(HKX_ERR_SHAPE, "the decode kernel takes K a multiple of 128");
    p->waves = a->decode_waves ? a->decode_waves : 8;
    const int rows = a->decode_rows ? a->decode_rows : (pair ? 32 : 16);
    if (p->waves != 4 && p->waves != 8 && p->waves != 16)
      return fail(HKX_ERR_ARG, "decode waves %d: 4, 8 or 16", p->waves);
    if (rows != 16 && rows != 32) return fail(HKX_ERR_ARG, "decode rows %d: 16 or 32", rows);
    if (pair && rows != 32) return fail(HKX_ERR_ARG, "the paired decode kernel takes 32 rows");
    p->fn = rows / 16;
    p->mf = a->m <= 16 ? 1 : 2;
    p->kunits = a->k / 128;
    if (a->variant & ~HKX_DEC_STREAM) return fail(HKX_ERR_ARG, "decode variant %d", a->variant);
    p->variant = a->variant;
  } else {
    return fail(HKX_ERR_ARG, "kernel %d", kernel);
  }
  if (splits > p->kunits) splits = p->kunits;
  p->kper = (p->kunits + splits - 1) / splits;
  p->splits = (p->kunits + p->kper - 1) / p->kper;

  // Shares (or one fp32 sum) go through the workspace when the K sum is split, when
  // the epilogue is a program, or when a paired C is not 16-bit (tile kernel).
  const bool program = a->ep.form == HKX_EP_PROGRAM;
  bool ws = p->splits > 1 || program;
  if (pair && kernel == HKX_KERNEL_TILE && ob != 2) ws = true;
  p->via_ws = ws;
  const long long wcols = pair ? 2LL * a->n : a->n;
  p->ws_bytes = ws ? (size_t)p->splits * a->m * wcols * sizeof(float) : 0;
  p->sk_cut = p->sk_splits = p->sk_kper = 0;
  if (kernel == HKX_KERNEL_TILE && p->schedule == HKX_TILE_RING &&
      (p->variant & HKX_RING_STREAMK) && !ws) {
    // the rest of N past the whole waves, split over K so that its tiles fill the CUs
    // (at least 4 K units a split, at most 8 splits)
    const int outw = pair ? p->tile_n / 2 : p->tile_n;
    const int cut = wave_cut(a->m, a->n, outw);
    if (cut < a->n) {
      const int rest = a->n - cut;
      const int tiles = ((a->m + 255) / 256) * ((rest + outw - 1) / outw);
      int sk = std::max(1, std::min({cu_count() / tiles, p->kunits / 4, 8}));
      const int kper = (p->kunits + sk - 1) / sk;
      sk = (p->kunits + kper - 1) / kper;
      p->sk_cut = cut;
      p->sk_splits = sk;
      p->sk_kper = kper;
      if (sk > 1) {
        p->ws_bytes = (size_t)sk * a->m * (pair ? 2LL * rest : rest) * sizeof(float);
        ws = true;
      }
    }
  }
  p->ncnt = 0;
  p->arrive = false;
  // the 4-wave tile kernel (which runs every split call of the W4 schedule and of the
  // ring schedule's 128-row tiles) finishes its split itself: a counter a tile
  // (a share's byte offsets fit 32 bits)
  const bool tile4_split = kernel == HKX_KERNEL_TILE && p->splits > 1 && !pair && !program &&
                           p->sk_splits == 0 && (long long)p->splits * a->m * a->n * 4 < (1LL << 32) &&
                           (p->schedule == HKX_TILE_W4 || (p->schedule == HKX_TILE_RING && p->tile_m == 128));
  if (tile4_split) {
    p->ncnt = ((a->m + p->tile_m - 1) / p->tile_m) * ((a->n + p->tile_n - 1) / p->tile_n);
    if (a->counters) {
      if (a->counters_len < p->ncnt || !aligned(a->counters, 4))
        return fail(HKX_ERR_WORKSPACE, "this plan needs %d 4-byte aligned arrival counters "
                    "(counters_len %lld)", p->ncnt, (long long)a->counters_len);
      p->arrive = true;
    }
  }
  if (kernel == HKX_KERNEL_DECODE && p->splits > 1 && !pair && !program) {
    p->ncnt = (a->n + 16 * p->fn - 1) / (16 * p->fn);
    if (a->counters) {
      if (a->counters_len < p->ncnt || !aligned(a->counters, 4))
        return fail(HKX_ERR_WORKSPACE, "this plan needs %d 4-byte aligned arrival counters "
                    "(counters_len %lld)", p->ncnt, (long long)a->counters_len);
      p->arrive = true;
    }
  }
  if (ws && (!a->ws || a->ws_bytes < p->ws_bytes || !aligned(a->ws, 16)))
    return fail(HKX_ERR_WORKSPACE, "this plan needs a 16-byte aligned fp32 workspace of %zu bytes",
                p->ws_bytes);
  return HKX_OK;
}

hkx::Fused make_fused(const HkxEpilogue& ep) {
  hkx::Fused f{};
  f.form = ep.form == HKX_EP_FUSED ? HKX_EP_FUSED : HKX_EP_NONE;
  f.cmul = 1.0f;
  if (ep.form != HKX_EP_FUSED) return f;
  auto opnd = [&](int i) {
    hkx::Opnd o{};
    if (i >= 0) {
      o.p = ep.ops[i].ptr;
      o.ld = ep.ops[i].ld;
      o.dt = ep.ops[i].dtype;
      o.kind = ep.ops[i].kind;
    }
    return o;
  };
  f.cs = opnd(ep.col_scale);
  f.rs = opnd(ep.row_scale);
  f.ra = opnd(ep.row_add);
  f.ta = opnd(ep.tile_add);
  f.cmul = ep.cmul;
  f.cadd = ep.cadd;
  f.act = ep.act;
  return f;
}

int launched(hipError_t e, const char* what) {
  if (e != hipSuccess)
    return fail(HKX_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return HKX_OK;
}

// Tile rows of the grouped raster: consecutive tiles go down a group of this many tile
// rows, then on to the next column. With the XCD-chunked numbering each XCD's share of a
// 4096 x 12288 call is then 8 x 12 tiles (A and B panels: 40 MB) rather than 4 x 24 (56 MB).
constexpr int kWgmRows = 8;

int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// The columns of N whose 256 x 256 tiles fill whole waves of one-a-CU workgroups at M's
// tile rows (0 where one wave takes more than N has): the reference's wave_cut
// (python/hk/ops/gemm_cdna.py:923-930).
int wave_cut(int m, int n, int outw) {
  const int mb = (m + 255) / 256, cus = cu_count();
  if (mb > cus) return 0;
  const int per = cus / mb;
  return (n / outw / per) * per * outw;
}

hipError_t tile_dispatch(const Plan& p, const hkx::TileArgs& t, bool fp8, int mode, dim3 grid,
                         hipStream_t s) {
  const int bm = p.tile_m, bn = p.tile_n;
  // The ring kernel: one workgroup a CU (a split's share of them) walking its tiles. A call
  // it does not take (an unaligned C, N % 8 != 0, a strided 16-bit column scale) runs on
  // the ping-pong kernel, which takes every 256 x 256 call.
  if (t.ab_fmt > 1) {  // e5m2 pairs: the ring kernel only (make_plan and hkx_gemm checked)
    dim3 g = grid;
    g.x = std::min<unsigned>(g.x, (unsigned)std::max(1, cu_count() / (int)grid.y));
    return hkx::launch_ring(t, fp8, mode, g, s);
  }
  if (p.schedule == HKX_TILE_RING && bm == 128) {  // the 128-row quadrant form, or the 4-wave kernel
    if (grid.y == 1 && hkx::quad128_takes(t, fp8, mode)) {
      dim3 g = grid;
      g.x = std::min<unsigned>(g.x, (unsigned)cu_count());
      return hkx::launch_quad128(t, mode, g, s);
    }
    return hkx::launch_tile4<128, 256>(t, fp8, mode, grid, s);
  }
  if (p.schedule == HKX_TILE_RING && hkx::ring_takes(t, fp8, mode)) {
    dim3 g = grid;
    g.x = std::min<unsigned>(g.x, (unsigned)std::max(1, cu_count() / (int)grid.y));
    // the quadrant kernel: one pass, or a K split into fp32 shares
    if (!(p.variant & HKX_RING_HALFSTAGE) && (grid.y == 1 || mode == hkx::kStoreF32) &&
        hkx::quad_takes(t, fp8, mode))
      return hkx::launch_quad(t, fp8, mode, g, s);
    return hkx::launch_ring(t, fp8, mode, g, s);
  }
  if (p.schedule == HKX_TILE_RING) return hkx::launch_pp(t, fp8, mode, true, grid, s);
  if (p.schedule == HKX_TILE_PINGPONG) {
    dim3 g = grid;
    if (!(p.variant & HKX_PP_ONE_TILE)) g.x = std::min<unsigned>(g.x, (unsigned)cu_count());
    return hkx::launch_pp(t, fp8, mode, !(p.variant & HKX_PP_MFMA32), g, s);
  }
  if (p.schedule == HKX_TILE_W4) {
    if (bn == 128) {
      if (bm == 128) return hkx::launch_tile4<128, 128>(t, fp8, mode, grid, s);
      return hkx::launch_tile4<64, 128>(t, fp8, mode, grid, s);
    }
    if (bm == 256) return hkx::launch_tile4<256, 256>(t, fp8, mode, grid, s);
    if (bm == 128) return hkx::launch_tile4<128, 256>(t, fp8, mode, grid, s);
    return hkx::launch_tile4<64, 256>(t, fp8, mode, grid, s);
  }
  if (bm == 256 && bn == 256) return hkx::launch_tile<256, 256, 2>(t, fp8, mode, grid, s);
  if (bm == 128 && bn == 256) return hkx::launch_tile<128, 256, 2>(t, fp8, mode, grid, s);
  if (bm == 64 && bn == 256) return hkx::launch_tile<64, 256, 1>(t, fp8, mode, grid, s);
  if (bm == 128 && bn == 128) return hkx::launch_tile<128, 128, 2>(t, fp8, mode, grid, s);
  return hkx::launch_tile<256, 128, 4>(t, fp8, mode, grid, s);
}

// The fp32 workspace of hkx_gemm_noalloc: a file-scope device array, so a call needs no
// allocation. Each GPU the library runs on holds its own copy (HKX_NOALLOC_SCRATCH_BYTES)
// until the process ends. In host code `scratch` names a host-side stand-in, not device
// memory: the kernels get the per-device address hipGetSymbolAddress returns.
__device__ __align__(256) unsigned char scratch[HKX_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// This device's copy of `scratch` (looked up once per device, that device current).
int scratch_for_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(HKX_ERR_LAUNCH, "gemm_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(HKX_ERR_ARG, "gemm_noalloc: device %d", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(HKX_ERR_LAUNCH, "gemm_noalloc: hipGetSymbolAddress(scratch) on device %d: %s",
                  dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return HKX_OK;
}

}  // namespace

extern "C" {

int hkx_abi_version(void) { return HKX_ABI_VERSION; }

void hkx_abi_sizes(size_t out[4]) {
  out[0] = sizeof(HkxOperand);
  out[1] = sizeof(HkxInstr);
  out[2] = sizeof(HkxEpilogue);
  out[3] = sizeof(HkxGemmArgs);
}

const char* hkx_last_error(void) { return g_err.c_str(); }

size_t hkx_gemm_workspace(const HkxGemmArgs* args) {
  // Plan a copy that carries an ample (never dereferenced) workspace, so the
  // workspace check passes and only the size comes back.
  Plan p{};
  if (!args) return 0;
  HkxGemmArgs a = *args;
  a.ws = (void*)(uintptr_t)256;  // any aligned non-null pointer: only the size is wanted
  a.ws_bytes = (size_t)-1;
  if (make_plan(&a, &p) != HKX_OK) return 0;
  return p.ws_bytes;
}

size_t hkx_gemm_counters(const HkxGemmArgs* args) {
  Plan p{};
  if (!args) return 0;
  HkxGemmArgs a = *args;
  a.ws = (void*)(uintptr_t)256;
  a.ws_bytes = (size_t)-1;
  a.counters = nullptr;
  a.counters_len = 0;
  if (make_plan(&a, &p) != HKX_OK) return 0;
  return (size_t)p.ncnt;
}

int hkx_gemm_check(const HkxGemmArgs* args) {
  Plan p{};
  g_err.clear();
  return make_plan(args, &p);
}

int hkx_gemm(const HkxGemmArgs* args, void* stream) {
  Plan p{};
  g_err.clear();
  int rc = make_plan(args, &p);
  if (rc) return rc;
  const HkxGemmArgs& a = *args;
  hipStream_t s = (hipStream_t)stream;
  const bool fp8 = a.ab_dtype != HKX_BF16;
  const int eb = elem_bytes(a.ab_dtype);
  const int ob = elem_bytes(a.c_dtype);
  const long long wcols = p.pair ? 2LL * a.n : a.n;
  const hkx::Fused fused = make_fused(a.ep);
  const bool program = a.ep.form == HKX_EP_PROGRAM;

  if (p.kernel == HKX_KERNEL_TILE) {
    hkx::TileArgs t{};
    t.ab_fmt = fmt_of(a.ab_dtype);
    t.a = a.a;
    t.b = a.b;
    t.a_bytes = (uint32_t)((long long)a.m * a.lda * eb);
    t.b_bytes = (uint32_t)((p.pair ? 2LL : 1LL) * a.n * a.ldb * eb);
    t.lda_b = (uint32_t)(a.lda * eb);
    t.ldb_b = (uint32_t)(a.ldb * eb);
    t.M = a.m;
    t.N = a.n;
    t.kt_total = p.kunits;
    t.kt_split = p.kper;
    const int outw = p.pair ? p.tile_n / 2 : p.tile_n;
    t.tiles_m = (a.m + p.tile_m - 1) / p.tile_m;
    t.tiles_n = (a.n + outw - 1) / outw;
    t.wgm = kWgmRows;
    t.pair_off = a.n;
    t.c_dt = a.c_dtype;
    const dim3 grid(t.tiles_m * t.tiles_n, p.splits);
    int mode;
    if (p.via_ws) {
      t.c = a.ws;
      t.ldc = wcols;
      t.split_stride = (int64_t)a.m * wcols;
      t.c_dt = HKX_FP32;
      t.ep = hkx::Fused{};
      t.ep.form = HKX_EP_NONE;
      mode = p.pair ? hkx::kPairWs : hkx::kStoreF32;
      if (p.arrive) {  // the last split of each tile finishes it into C
        t.cnt = a.counters;
        t.fin_c = a.c;
        t.fin_ldc = a.ldc;
        t.fin_dt = a.c_dtype;
        t.fin_ep = fused;
      }
    } else {
      t.c = a.c;
      t.ldc = a.ldc;
      t.split_stride = 0;
      t.c_aligned = aligned(a.c, 16) && (a.ldc * ob) % 16 == 0;
      t.ep = fused;
      if (p.pair) mode = hkx::kPair16;
      else if (ob == 2) mode = hkx::kStore16;
      else if (ob == 1) mode = hkx::kStore8;
      else mode = hkx::kStoreF32;
    }
    if (t.ab_fmt > 1 && !hkx::ring_takes(t, fp8, mode))
      return fail(HKX_ERR_SHAPE, "e5m2 operands run on the ring kernel, which needs C's rows "
                  "16-byte aligned and N a multiple of 8");
    // The columns from c0 on as a call of their own: B's rows, C's columns and the
    // per-column epilogue operands (vectors and tiles; broadcasts stay) from column c0.
    auto from_col = [&](const hkx::TileArgs& t0, int c0) {
      hkx::TileArgs r = t0;
      r.b = (const uint8_t*)a.b + (int64_t)c0 * a.ldb * eb;
      r.b_bytes = (uint32_t)((p.pair ? 2LL * a.n - c0 : (long long)a.n - c0) * a.ldb * eb);
      r.c = (uint8_t*)a.c + (int64_t)c0 * elem_bytes(a.c_dtype);
      r.c_aligned = aligned(r.c, 16) && (a.ldc * ob) % 16 == 0;
      r.N = a.n - c0;
      r.tiles_n = (r.N + outw - 1) / outw;
      for (hkx::Opnd* o : {&r.ep.rs, &r.ep.ra, &r.ep.ta})
        if (o->p && ((o->kind == HKX_ROW && o->ld) || o->kind == HKX_TILE))
          o->p = (const uint8_t*)o->p + (int64_t)c0 * elem_bytes(o->dt);
      return r;
    };
    const int cut = (p.variant & HKX_RING_WAVESPLIT) && !p.via_ws ? wave_cut(a.m, a.n, outw)
                    : p.sk_cut;
    if (cut < a.n && ((p.variant & HKX_RING_WAVESPLIT) ? cut > 0 : p.sk_splits > 0)) {
      if (cut > 0) {  // whole waves of 256 x 256 tiles on the ring kernel
        hkx::TileArgs t1 = t;
        t1.N = cut;
        t1.tiles_n = cut / outw;
        rc = launched(tile_dispatch(p, t1, fp8, mode, dim3(t1.tiles_m * t1.tiles_n), s),
                      "tile GEMM (whole waves)");
        if (rc) return rc;
      }
      hkx::TileArgs t2 = from_col(t, cut);
      if (p.variant & HKX_RING_WAVESPLIT) {  // the rest on 128 x 256 tiles
        t2.tiles_m = (a.m + 127) / 128;
        Plan p2 = p;
        p2.schedule = HKX_TILE_W4;
        p2.tile_m = 128;
        p2.tile_n = 256;
        rc = launched(tile_dispatch(p2, t2, fp8, mode, dim3(t2.tiles_m * t2.tiles_n), s),
                      "tile GEMM (the rest of N)");
        if (rc) return rc;
      } else if (p.sk_splits == 1) {  // the rest on ring tiles, one pass
        rc = launched(tile_dispatch(p, t2, fp8, mode, dim3(t2.tiles_m * t2.tiles_n), s),
                      "tile GEMM (the rest of N)");
        if (rc) return rc;
      } else {  // the rest split over K: fp32 shares, then their sum and the epilogue
        const long long wc2 = p.pair ? 2LL * t2.N : t2.N;
        hkx::TileArgs t3 = t2;
        t3.c = a.ws;
        t3.ldc = wc2;
        t3.split_stride = (int64_t)a.m * wc2;
        t3.c_dt = HKX_FP32;
        t3.ep = hkx::Fused{};
        t3.ep.form = HKX_EP_NONE;
        t3.kt_split = p.sk_kper;
        Plan p3 = p;
        p3.splits = p.sk_splits;
        rc = launched(tile_dispatch(p3, t3, fp8, p.pair ? hkx::kPairWs : hkx::kStoreF32,
                                    dim3(t3.tiles_m * t3.tiles_n, p.sk_splits), s),
                      "tile GEMM (the rest of N, split over K)");
        if (rc) return rc;
        hkx::ReduceArgs r{};
        r.ws = (const float*)a.ws;
        r.split_stride = (int64_t)a.m * wc2;
        r.ws_ld = wc2;
        r.c = t2.c;
        r.ldc = a.ldc;
        r.splits = p.sk_splits;
        r.M = a.m;
        r.N = t2.N;
        r.c_dt = a.c_dtype;
        r.pair = p.pair;
        r.f = t2.ep;
        const dim3 rg(((t2.N + 3) / 4 + 255) / 256, a.m < 65535 ? a.m : 65535);
        rc = launched(hkx::launch_reduce(r, a.ep, false, rg, s), "reduction (the rest of N)");
        if (rc) return rc;
      }
    } else {
      rc = launched(tile_dispatch(p, t, fp8, mode, grid, s), "tile GEMM");
      if (rc) return rc;
    }
  } else {
    hkx::DecodeArgs d{};
    d.a = a.a;
    d.b = a.b;
    d.a_bytes = (uint32_t)((long long)a.m * a.lda * eb);
    d.b_bytes = (uint32_t)((p.pair ? 2LL : 1LL) * a.n * a.ldb * eb);
    d.lda_b = (uint32_t)(a.lda * eb);
    d.ldb_b = (uint32_t)(a.ldb * eb);
    d.M = a.m;
    d.N = a.n;
    d.g_total = p.kunits;
    d.g_split = p.kper;
    d.pair_off = a.n;
    d.c_dt = a.c_dtype;
    const int outw = p.pair ? 8 * p.fn : 16 * p.fn;
    const dim3 grid((a.n + outw - 1) / outw, p.splits);
    int mode;
    if (p.arrive) {  // shares in ws; the last split of a block finishes it into C
      d.c = a.c;
      d.ldc = a.ldc;
      d.ep = fused;
      d.ws = (float*)a.ws;
      d.split_stride = (int64_t)a.m * a.n;
      d.cnt = a.counters;
      mode = hkx::kDecArrive;
    } else if (p.via_ws) {
      d.c = a.ws;
      d.ldc = p.pair ? a.n * 2LL : a.n;
      d.split_stride = (int64_t)a.m * wcols;
      d.c_dt = HKX_FP32;
      d.ep.form = HKX_EP_NONE;
      mode = p.pair ? hkx::kDecPairWs : hkx::kDecWs;
    } else {
      d.c = a.c;
      d.ldc = a.ldc;
      d.ep = fused;
      mode = p.pair ? hkx::kDecPair : hkx::kDecOut;
    }
    const int gw = std::min((a.n + 7) / 8, cu_count());
    if ((p.variant & HKX_DEC_STREAM) && hkx::stream_takes(d, p.splits, p.pair) && hkx::roww_takes(d, gw)) {
      rc = launched(hkx::launch_roww(d, dim3(gw), s), "decode GEMM");
    } else if ((p.variant & HKX_DEC_STREAM) && hkx::stream_takes(d, p.splits, p.pair) && hkx::rows_takes(d)) {
      const dim3 g(std::min((a.n + 3) / 4, cu_count()));
      rc = launched(hkx::launch_rows(d, g, s), "decode GEMM");
    } else if ((p.variant & HKX_DEC_STREAM) && hkx::stream_takes(d, p.splits, p.pair)) {
      const dim3 g(std::min((a.n + 15) / 16, cu_count()));
      rc = launched(hkx::launch_stream(d, g, s), "decode GEMM");
    } else {
      rc = launched(hkx::launch_decode(d, p.waves, p.fn, p.mf, mode, grid, s), "decode GEMM");
    }
    if (rc) return rc;
  }

  if (p.via_ws && !p.arrive) {
    hkx::ReduceArgs r{};
    r.ws = (const float*)a.ws;
    r.split_stride = (int64_t)a.m * wcols;
    r.ws_ld = wcols;
    r.c = a.c;
    r.ldc = a.ldc;
    r.splits = p.splits;
    r.M = a.m;
    r.N = a.n;
    r.c_dt = a.c_dtype;
    r.pair = p.pair;
    r.f = fused;
    const dim3 grid(((a.n + 3) / 4 + 255) / 256, a.m < 65535 ? a.m : 65535);
    rc = launched(hkx::launch_reduce(r, a.ep, program, grid, s), "reduction");
    if (rc) return rc;
  }
  return HKX_OK;
}

int hkx_gemm_noalloc(const HkxGemmArgs* args, void* stream) {
  g_err.clear();
  if (!args) return fail(HKX_ERR_ARG, "gemm_noalloc: args is NULL");
  HkxGemmArgs a = *args;
  a.ws = nullptr;
  a.ws_bytes = 0;
  a.counters = nullptr;  // a K split is summed by its second launch, from the scratch
  a.counters_len = 0;
  const size_t need = hkx_gemm_workspace(&a);
  if (need > (size_t)HKX_NOALLOC_SCRATCH_BYTES)
    return fail(HKX_ERR_WORKSPACE,
                "gemm_noalloc: this plan needs %zu bytes of workspace; the no-allocation entry "
                "point has %zu (call hkx_gemm with a workspace, or split the call)",
                need, (size_t)HKX_NOALLOC_SCRATCH_BYTES);
  if (need) {
    int rc = scratch_for_current_device(&a.ws);
    if (rc) return rc;
    a.ws_bytes = HKX_NOALLOC_SCRATCH_BYTES;
  }
  return hkx_gemm(&a, stream);
}

// The MX GEMM's K split: where its 256 x 256 tiles fill less than half the CUs, up to 8
// splits of at least 8 k-tiles (1024 K) each, so the tiles times the splits stay within
// the CUs; none where an fp32 share would span 4 GiB. (Shorter splits lost more to the
// shares' round trip than they gained: K = 1152 and 1280 ran slower split in two.)
static int mx_splits(int32_t m, int32_t n, int32_t k) {
  if (m < 1 || n < 1 || k < 128 || k % 128) return 1;
  const int tiles = ((m + 255) / 256) * ((n + 255) / 256);
  const int cu = cu_count();
  if (2 * tiles > cu || (long long)((m + 255) / 256) * 256 * n * 4 >= (1LL << 32)) return 1;
  const int s = std::min(std::min(cu / tiles, (k / 128) / 8), 8);
  if (s < 2) return 1;
  const int kper = (k / 128 + s - 1) / s;  // no empty last split
  return (k / 128 + kper - 1) / kper;
}

size_t hkx_mx_gemm_workspace(int32_t m, int32_t n, int32_t k) {
  const int s = mx_splits(m, n, k);
  return s > 1 ? (size_t)s * (size_t)m * (size_t)n * 4u : 0;
}

int hkx_mx_gemm(const void* a, int64_t lda, const void* b, int64_t ldb, const uint8_t* sa,
                int64_t sa_ld, const uint8_t* sb, int64_t sb_ld, void* c, int64_t ldc, int32_t m,
                int32_t n, int32_t k, void* ws, size_t ws_bytes, void* stream) {
  g_err.clear();
  if (!a || !b || !c || !sa || !sb) return fail(HKX_ERR_ARG, "mx_gemm: a null pointer");
  if (m < 1 || n < 1 || k < 1) return fail(HKX_ERR_SHAPE, "mx_gemm: M=%d N=%d K=%d", m, n, k);
  if (k % 128 || n % 8)
    return fail(HKX_ERR_SHAPE, "mx_gemm: K=%d must be a multiple of 128 and N=%d of 8", k, n);
  if (lda < k || ldb < k || ldc < n || sa_ld < k / 32 || sb_ld < k / 32)
    return fail(HKX_ERR_SHAPE, "mx_gemm: row strides below K, N or K/32");
  if (!aligned(a, 16) || !aligned(b, 16) || lda % 16 || ldb % 16)
    return fail(HKX_ERR_SHAPE, "mx_gemm: A and B need 16-byte aligned rows");
  if (!aligned(c, 16) || (ldc * 2) % 16)
    return fail(HKX_ERR_SHAPE, "mx_gemm: C (bf16) needs 16-byte aligned rows");
  if (!aligned(sa, 4) || !aligned(sb, 4) || sa_ld % 4 || sb_ld % 4)
    return fail(HKX_ERR_SHAPE, "mx_gemm: the scales need 4-byte aligned rows");
  // 32-bit byte offsets, C's computed for every row of the last 256-row tile (rows past M
  // included, whose offsets must not wrap round into C's first rows)
  if ((long long)m * lda >= (1LL << 32) || (long long)n * ldb >= (1LL << 32) ||
      (long long)((m + 255) / 256) * 256 * ldc * 2 >= (1LL << 32))
    return fail(HKX_ERR_SHAPE, "mx_gemm: A, B or C spans 4 GiB or more; split the call");
  hkx::TileArgs t{};
  t.a = a;
  t.b = b;
  t.c = c;
  t.a_bytes = (uint32_t)((long long)m * lda);
  t.b_bytes = (uint32_t)((long long)n * ldb);
  t.lda_b = (uint32_t)lda;
  t.ldb_b = (uint32_t)ldb;
  t.ldc = ldc;
  t.M = m;
  t.N = n;
  t.kt_total = t.kt_split = k / 128;
  t.tiles_m = (m + 255) / 256;
  t.tiles_n = (n + 255) / 256;
  t.wgm = kWgmRows;
  t.pair_off = n;
  t.c_dt = HKX_BF16;
  t.c_aligned = 1;
  t.ep.form = HKX_EP_NONE;
  t.ep.cmul = 1.0f;
  t.sa = sa;
  t.sb = sb;
  t.sa_ld = (uint32_t)sa_ld;
  t.sb_ld = (uint32_t)sb_ld;
  t.sa_bytes = (uint32_t)((long long)m * sa_ld);
  t.sb_bytes = (uint32_t)((long long)n * sb_ld);
  const int splits = mx_splits(m, n, k);
  const hipStream_t s = (hipStream_t)stream;
  if (splits == 1) {
    const dim3 g(std::min(t.tiles_m * t.tiles_n, cu_count()));
    // the quadrant kernel (whole-line fills) where it takes the call, else the ring's MX form
    if (hkx::quad_takes(t, true, hkx::kStore16)) return launched(hkx::launch_quad_mx(t, g, s), "mx GEMM");
    return launched(hkx::launch_ring_mx(t, false, g, s), "mx GEMM");
  }
  const size_t need = hkx_mx_gemm_workspace(m, n, k);
  if (!ws || ws_bytes < need || !aligned(ws, 16))
    return fail(HKX_ERR_WORKSPACE, "mx_gemm: needs %zu bytes of 16-byte aligned workspace, got %zu",
                need, ws ? ws_bytes : (size_t)0);
  // split s of K into fp32 share s (M x N, row stride N), one tile a workgroup
  hkx::TileArgs tw = t;
  tw.c = ws;
  tw.ldc = n;
  tw.split_stride = (int64_t)m * n;
  tw.c_dt = HKX_FP32;
  tw.kt_split = (k / 128 + splits - 1) / splits;
  int rc = launched(hkx::launch_ring_mx(tw, true, dim3(t.tiles_m * t.tiles_n, splits), s),
                    "mx GEMM (split over K)");
  if (rc) return rc;
  hkx::ReduceArgs r{};
  r.ws = (const float*)ws;
  r.split_stride = (int64_t)m * n;
  r.ws_ld = n;
  r.c = c;
  r.ldc = ldc;
  r.splits = splits;
  r.M = m;
  r.N = n;
  r.c_dt = HKX_BF16;
  r.pair = 0;
  r.f = t.ep;
  HkxEpilogue none{};
  none.form = HKX_EP_NONE;
  const dim3 rg(((n + 3) / 4 + 255) / 256, m < 65535 ? m : 65535);
  return launched(hkx::launch_reduce(r, none, false, rg, s), "mx GEMM (sum of the splits)");
}

int hkx_mx_quant(const void* x, int64_t ldx, void* q, int64_t ldq, uint8_t* s, int64_t lds,
                 int32_t m, int32_t k, void* stream) {
  g_err.clear();
  if (!x || !q || !s) return fail(HKX_ERR_ARG, "mx_quant: a null pointer");
  if (m < 0 || k < 0 || k % 32) return fail(HKX_ERR_SHAPE, "mx_quant: K=%d, a multiple of 32", k);
  if (ldx < k || ldq < k || lds < k / 32) return fail(HKX_ERR_SHAPE, "mx_quant: row strides");
  if (!aligned(x, 16) || ldx % 8 || !aligned(q, 8) || ldq % 8)
    return fail(HKX_ERR_SHAPE, "mx_quant: x needs 16-byte and q 8-byte aligned rows");
  if (m == 0 || k == 0) return HKX_OK;
  return launched(hkx::launch_mx_quant(x, ldx, q, ldq, s, lds, m, k, (hipStream_t)stream),
                  "mx quant");
}

int hkx_scaled_mm(const void* a, int64_t lda, const void* b, int64_t ldb, const float* scale_a,
                  int64_t sa_ld, const float* scale_b, int32_t sb_per_channel, const void* bias,
                  void* c, int64_t ldc, int32_t m, int32_t n, int32_t k, void* ws,
                  size_t ws_bytes, void* stream) {
  HkxGemmArgs g;
  memset(&g, 0, sizeof g);
  g.a = a;
  g.b = b;
  g.c = c;
  g.lda = lda;
  g.ldb = ldb;
  g.ldc = ldc;
  g.m = m;
  g.n = n;
  g.k = k;
  g.ab_dtype = HKX_FP8E4M3;
  g.c_dtype = HKX_BF16;
  g.kernel = HKX_KERNEL_AUTO;
  g.splits = 1;
  g.ws = ws;
  g.ws_bytes = ws_bytes;
  HkxEpilogue& ep = g.ep;
  ep.form = HKX_EP_FUSED;
  ep.act = HKX_ACT_NONE;
  ep.cmul = 1.0f;
  ep.col_scale = ep.row_scale = ep.row_add = ep.tile_add = -1;
  if (!scale_a || !scale_b) return fail(HKX_ERR_ARG, "scaled_mm: scale_a and scale_b are required");
  ep.ops[0] = HkxOperand{scale_a, HKX_COL, HKX_FP32, sa_ld};
  ep.ops[1] = HkxOperand{scale_b, HKX_ROW, HKX_FP32, sb_per_channel ? 1 : 0};
  ep.col_scale = 0;
  ep.row_scale = 1;
  ep.nops = 2;
  if (bias) {
    ep.ops[2] = HkxOperand{bias, HKX_ROW, HKX_BF16, 1};
    ep.row_add = 2;
    ep.nops = 3;
  }
  return hkx_gemm(&g, stream);
}

}  // extern "C"
