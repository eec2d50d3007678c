/*
 * hkx.h -- the C ABI of libhkx.so: GEMM with a fused epilogue on MI355X (gfx950).
 *
 * C = epilogue(A . B^T accumulated in fp32), A (M, K) and B (N, K) K-contiguous
 * (F.linear's layout), bf16 x bf16 or fp8-e4m3 x fp8-e4m3, C (M, N) in bf16, fp16,
 * fp32, int8 or fp8-e4m3.
 *
 * Plain pointers and sizes only; no torch types. Every pointer is a device pointer
 * on the current HIP device; every launch goes on the stream passed in. The library
 * allocates nothing and never synchronizes: a caller that needs a workspace asks
 * hkx_gemm_workspace() for its size and passes it in (HkxGemmArgs.ws).
 *
 * What each entry point replaces in the reference (vivienfanghuagood/hk-dsl 0.9.24):
 *
 *   hkx_gemm            the launches hk.templates.gemm prepares for a plan, one
 *                       `kern(a, b, c, *extra, *ep_tensors, **consts)` per Step
 *                       (python/hk/templates/gemm.py:577-665, launch convention
 *                       python/hk/ops/_epilogue.py:28-43), which end in
 *                       hipModuleLaunchKernel on the caller's stream
 *                       (mlir/python/HKLaunch.c:1-25, python/hk/runtime/codeobj.py:265-276).
 *                       The kernels it runs replace gemm_cdna.gemm_kernel
 *                       (python/hk/ops/gemm_cdna.py:57-586), gemm_cdna_dp.gemm_kernel and
 *                       its split-K shares (python/hk/ops/gemm_cdna_dp.py:30-243),
 *                       reduce_epilogue_kernel (gemm_cdna_dp.py:295-324, 361-383) and
 *                       decode_gemm_kernel (python/hk/ops/decode_gemm.py:37-180).
 *   hkx_scaled_mm       hk.ops.gemm.scaled_mm's launch (python/hk/ops/gemm.py:884-975):
 *                       bf16 (A . B^T) * scale_a * scale_b (+ bias), fp8 operands.
 *   hkx_mx_gemm         hk.ops.mxfp8.gemm / gemm_pp's launch (python/hk/ops/mxfp8.py:64-110,
 *                       gemm_cdna.gemm_kernel with mx=True, python/hk/ops/gemm_cdna.py:82-94):
 *                       bf16 C = (sa . A)(sb . B)^T, fp8-e4m3 operands with OCP MX E8M0
 *                       scales, one byte a row and 32 K.
 *   hkx_mx_quant        hk.ops.mxfp8.quant's launch (python/hk/ops/mxfp8.py:605-660): bf16
 *                       rows to fp8-e4m3 with an E8M0 scale a 32-column block, AITER's
 *                       per_1x32 rule (python/hk/mx.py:17-31), the scales in the OCP
 *                       layout the MX GEMM reads.
 *   hkx_gemm_workspace  gemm_cdna_dp.scratch_for / decode_gemm.scratch_for
 *                       (gemm_cdna_dp.py:330-338, decode_gemm.py:283-298): the size of
 *                       the fp32 share buffer a plan needs (the caller allocates it).
 *   hkx_mx_gemm_workspace  the same for hkx_mx_gemm's split-K shares (this build splits
 *                       K across workgroups where the reference's MX kernel runs few tiles
 *                       unsplit, python/hk/ops/mxfp8.py:64-110).
 *   hkx_last_error      the message the reference raises in Python (ValueError /
 *                       TypeError texts of templates/gemm.py:770-803).
 */
#ifndef HKX_H_
#define HKX_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HKX_ABI_VERSION 4

/* Status codes. */
#define HKX_OK 0
#define HKX_ERR_SHAPE 1       /* a shape / stride / alignment the kernels do not take */
#define HKX_ERR_DTYPE 2       /* an element type the kernels do not take */
#define HKX_ERR_WORKSPACE 3   /* ws missing or smaller than hkx_gemm_workspace() */
#define HKX_ERR_LAUNCH 4      /* hipLaunchKernel failed; hkx_last_error() has hipGetErrorString */
#define HKX_ERR_ARG 5         /* a malformed argument (epilogue program, operand, null pointer) */

/* Element types. */
#define HKX_BF16 0
#define HKX_FP16 1
#define HKX_FP32 2
#define HKX_FP8E4M3 3 /* OCP e4m3 (float8_e4m3fn): max 448, no inf */
#define HKX_INT8 4
/* fp8 operand pairs with e5m2 (OCP float8_e5m2: max 57344, inf and nan), as ab_dtype only;
 * they run on the 256 x 256 ring tile kernel: */
#define HKX_FP8E5M2 5        /* A and B e5m2 */
#define HKX_FP8_E4M3_E5M2 6  /* A e4m3, B e5m2 (e.g. activations against a gradient) */
#define HKX_FP8_E5M2_E4M3 7  /* A e5m2, B e4m3 */

/* Epilogue operand kinds: what an operand is against C (M, N) -- templates/gemm.py:116-135. */
#define HKX_ROW 1  /* (N,) or (1, N): one value per column of C (a bias, a per-channel scale) */
#define HKX_COL 2  /* (M, 1): one value per row (a per-token scale); ld = its row stride */
#define HKX_TILE 3 /* (M, N): one per element (a residual); ld = its row stride */

/* Epilogue forms. */
#define HKX_EP_NONE 0     /* C = acc */
#define HKX_EP_FUSED 1    /* C = act(acc * col_scale[m] * row_scale[n] * cmul + row_add[n] + tile_add[m,n] + cadd) */
#define HKX_EP_PROGRAM 2  /* C = the register program below, run once per element on the fp32 sum */
#define HKX_EP_SILU_MUL 3 /* C[:, j] = silu(acc[:, j]) * acc[:, N + j]; B is (2N, K), gate rows then up rows */

/* Activations of the fused form. */
#define HKX_ACT_NONE 0
#define HKX_ACT_GELU_TANH 1
#define HKX_ACT_SILU 2
#define HKX_ACT_RELU 3

/* Program opcodes: dst <- f(a, b, c); registers are fp32, R0 starts as the accumulator. */
#define HKX_OP_MOV 0    /* dst = r[a] */
#define HKX_OP_LOAD 1   /* dst = operand a at this element (by its kind), as fp32 */
#define HKX_OP_CONST 2  /* dst = imm */
#define HKX_OP_ROW 3    /* dst = the element's row of C */
#define HKX_OP_COL 4    /* dst = the element's column of C, plus col0 */
#define HKX_OP_ADD 5
#define HKX_OP_SUB 6
#define HKX_OP_MUL 7
#define HKX_OP_DIV 8
#define HKX_OP_MAX 9
#define HKX_OP_MIN 10
#define HKX_OP_EXP 11
#define HKX_OP_EXP2 12
#define HKX_OP_LOG 13
#define HKX_OP_LOG2 14
#define HKX_OP_ABS 15
#define HKX_OP_RELU 16
#define HKX_OP_GELU 17  /* tanh approximation */
#define HKX_OP_SILU 18
#define HKX_OP_SQRT 19
#define HKX_OP_RSQRT 20
#define HKX_OP_NEG 21
#define HKX_OP_STEP 22  /* 1 where r[a] > 0, else 0 */
#define HKX_OP_SELLE 23 /* dst = r[a] <= 0 ? r[b] : r[c] */
#define HKX_OP_M 24     /* dst = M (C's rows) */
#define HKX_OP_TANH 25
#define HKX_OP_SIGMOID 26
#define HKX_OP_SQUARE 27 /* dst = r[a] * r[a] */
#define HKX_NUM_OPS 28

#define HKX_MAX_OPERANDS 8
#define HKX_MAX_INSTR 64
#define HKX_MAX_REGS 16

typedef struct HkxOperand {
  const void* ptr; /* device pointer */
  int32_t kind;    /* HKX_ROW / HKX_COL / HKX_TILE */
  int32_t dtype;   /* HKX_BF16 / HKX_FP16 / HKX_FP32 */
  int64_t ld;      /* COL, TILE: row stride in elements. ROW: 1 (a vector) or 0 (one value
                      broadcast to every column) */
} HkxOperand;

typedef struct HkxInstr {
  uint8_t op, dst, a, b, c, pad0, pad1, pad2;
  float imm;
} HkxInstr;

typedef struct HkxEpilogue {
  int32_t form; /* HKX_EP_* */
  /* HKX_EP_FUSED: operand indices into ops[] (-1 = absent), the activation, constants. */
  int32_t act;
  int32_t col_scale, row_scale, row_add, tile_add;
  float cmul, cadd;
  /* HKX_EP_PROGRAM */
  int32_t nins;
  int32_t out_reg;
  int32_t col0; /* added to HKX_OP_COL (a launch on a column slice of a larger C) */
  int32_t nops;
  HkxOperand ops[HKX_MAX_OPERANDS];
  HkxInstr ins[HKX_MAX_INSTR];
} HkxEpilogue;

/* Kernel families (HkxGemmArgs.kernel). */
#define HKX_KERNEL_AUTO 0
#define HKX_KERNEL_TILE 1   /* LDS-tiled MFMA GEMM, tile_m x tile_n blocks, optional split-K */
#define HKX_KERNEL_DECODE 2 /* skinny-M weight-streaming GEMM (M <= 32), optional split-K */

/* Tile kernel schedules (HkxGemmArgs.tile_schedule). */
#define HKX_TILE_AUTO 0
#define HKX_TILE_PINGPONG 1 /* 8 waves, two a SIMD taking turns at the MFMA; 256 x 256 only */
#define HKX_TILE_W4 2       /* 4 waves, one a SIMD (2 x 2, 32 x 32 MFMAs), up to four LDS
                               stages; 256, 128 or 64 x 256 and 128 or 64 x 128 */
#define HKX_TILE_W8 3       /* 8 waves, register-staged fills, 16 x 16 MFMAs; every tile
                               shape but 64 x 128 */
#define HKX_TILE_RING 4     /* 8 waves taking turns at the MFMA, one workgroup a CU walking its
                               tiles through one LDS ring, epilogue stored from registers;
                               256 x 256 only, C rows 16-byte aligned, N % 8 == 0 */

/* HKX_TILE_PINGPONG variant bits (HkxGemmArgs.variant; 0 = the default). */
#define HKX_PP_MFMA32 1   /* 32 x 32 MFMA fragments (the fp8 and paired forms always use them) */
#define HKX_PP_ONE_TILE 2 /* one tile a workgroup, instead of a grid of one workgroup a CU */

/* HKX_TILE_RING variant bits. */
#define HKX_RING_WAVESPLIT 4 /* the columns whose 256 x 256 tiles make whole waves of the CUs
                                on the ring kernel, the rest of N on the 4-wave kernel's
                                128 x 256 tiles (two launches; no split over K) -- the
                                reference's ppw candidate (gemm_cdna.py:834-835, 923-930) */
#define HKX_RING_STREAMK 8   /* the whole waves likewise on the ring kernel, the rest of N on
                                ring tiles split over K so that they fill the CUs (fp32 shares
                                in the workspace, then one pass that sums them in split order
                                and applies the epilogue) -- the reference's dp+sk stream-K
                                mode (gemm_cdna.py:421-496, 635-729) without its in-kernel
                                fix-up; hkx_gemm_workspace() sizes the shares */
#define HKX_RING_HALFSTAGE 16 /* every form on the half-stage ring kernel. Without it a call the
                                 quadrant kernel takes runs there (bf16 operands and C, no
                                 split, no epilogue or a bf16 bias and an activation): each
                                 wave's output spread over the tile's four 128 x 128 quadrants,
                                 whole 128-byte lines a fill -- the reference's pp schedule
                                 (gemm_cdna.py:57-586). Combines with the two bits above */

/* HKX_KERNEL_DECODE variant bits. */
#define HKX_DEC_STREAM 1  /* one workgroup a CU streaming W (M <= 16, or M <= 32 from K =
                             2048; K a multiple of 1024 up to 32768, no split, unpaired): in
                             blocks of 16 rows, or, with no residual and no vector scale, in
                             chunks of whole rows -- 4 rows at K = 4096, M <= 4, N <= 32768
                             or at M <= 2 any N with W under 2 GiB (one or two chunks a short
                             workgroup at M <= 3, and at M = 4 up to N = 8192; else strided
                             over one workgroup a CU); 8 rows, one
                             a wave, at K = 1024 (M <= 3) and K = 2048 (M <= 2); other calls
                             take the blocked kernel */

typedef struct HkxGemmArgs {
  const void* a; /* (M, K), row stride lda elements */
  const void* b; /* (N, K) -- (2N, K) for HKX_EP_SILU_MUL -- row stride ldb elements */
  void* c;       /* (M, N), row stride ldc elements */
  int64_t lda, ldb, ldc;
  int32_t m, n, k;
  int32_t ab_dtype; /* HKX_BF16, HKX_FP8E4M3 (both operands), or an e5m2 pair code */
  int32_t c_dtype;  /* HKX_BF16 / HKX_FP16 / HKX_FP32 / HKX_INT8 / HKX_FP8E4M3 */
  int32_t kernel;   /* HKX_KERNEL_* */
  int32_t tile_m;   /* TILE: 64, 128 or 256 (256 x 128 on W8 only, 64 x 128 on W4 only) */
  int32_t tile_n;   /* TILE: 128 or 256 */
  int32_t splits;   /* >= 1; > 1 stores fp32 shares to ws and sums them in order */
  int32_t tile_schedule; /* TILE: HKX_TILE_*; AUTO = RING for 256 x 256 tiles it takes,
                            else PINGPONG for 256 x 256, else W4 where the tile takes it,
                            else W8 */
  int32_t variant;  /* TILE, PINGPONG: HKX_PP_* bits (for tuning); DECODE: HKX_DEC_* bits */
  int32_t decode_waves; /* DECODE: waves per workgroup (4, 8 or 16); 0 = default */
  int32_t decode_rows;  /* DECODE: W rows per workgroup (16 or 32); 0 = default */
  void* ws;         /* fp32 workspace, hkx_gemm_workspace() bytes */
  size_t ws_bytes;
  HkxEpilogue ep;
  /* A split over K finished in the kernel: int32 arrival counters, hkx_gemm_counters() of
     them, all zero before the first call. With them the blocked decode kernel (one counter
     a block of rows) and the 4-wave tile kernel (one a tile) finish the split themselves:
     each workgroup stores its fp32 share and arrives at its counter, and the last to arrive
     sums the shares in split order (as the second launch does, so the result is the same),
     applies the epilogue and sets the counter back to zero -- one launch. NULL: the shares
     are summed by a second launch. Measured on MI355X, the decode finish costs what the
     second launch does, the tile finish 4-10 us more a call at M = 16-128 (its last
     arrivers' chain of share stores, arrival and share loads is all tail); hk's Python
     layer passes counters for decode splits only. Calls that overlap in time on one GPU
     must not share counters. */
  int32_t* counters;
  int64_t counters_len;
} HkxGemmArgs;

/* Library identity. */
int hkx_abi_version(void);
/* sizeof(HkxOperand), sizeof(HkxInstr), sizeof(HkxEpilogue), sizeof(HkxGemmArgs) into
 * out[0..3]: lets a binding check its struct layouts against the library's. */
void hkx_abi_sizes(size_t out[4]);
/* The message of the last failed call on this thread ("" if none). */
const char* hkx_last_error(void);

/* Bytes of fp32 workspace hkx_gemm needs for these args (0 if none). Resolves
 * HKX_KERNEL_AUTO the way hkx_gemm does. Host-only, needs no GPU. */
size_t hkx_gemm_workspace(const HkxGemmArgs* args);

/* int32 arrival counters hkx_gemm uses for these args (0 if the plan has no in-kernel
 * arrival): the blocked decode kernel or the 4-wave tile kernel split over K, unpaired,
 * fused or no epilogue (the tile kernel: all the shares under 4 GiB). Replaces
 * the counter half of decode_gemm.scratch_for (python/hk/ops/decode_gemm.py:283-298), whose
 * kernel arrives at cnt[b] and whose last arriver sums, finishes and resets it (:155-170).
 * Host-only, needs no GPU. */
size_t hkx_gemm_counters(const HkxGemmArgs* args);

/* Checks args (HKX_OK or an error code, message in hkx_last_error) without launching.
 * Host-only, needs no GPU. */
int hkx_gemm_check(const HkxGemmArgs* args);

/* Launch the plan for args on stream (a hipStream_t; NULL = the null stream).
 * Returns HKX_OK or an error code; hkx_last_error() says why. */
int hkx_gemm(const HkxGemmArgs* args, void* stream);

/* hkx_gemm with no workspace argument and no allocation: the plan's fp32 workspace (split-K
 * shares, a register program's sum) is a static device array of the library,
 * HKX_NOALLOC_SCRATCH_BYTES on each GPU it runs on, held until the process ends. args->ws
 * and args->ws_bytes are ignored. A plan that needs more than that fails with
 * HKX_ERR_WORKSPACE (nothing launched). Calls no hipMalloc / hipFree; every kernel writes
 * each scratch byte it reads in the same call, so nothing needs clearing between calls.
 * Every call on one GPU shares that GPU's array: two calls that overlap in time on one GPU
 * (other streams, or graphs replayed concurrently) race on it -- serialise them.
 * No counterpart in the reference: it is for callers that cannot allocate (code under
 * HIP-graph capture, serving loops and harnesses that forbid hipMalloc). */
#define HKX_NOALLOC_SCRATCH_BYTES (64u << 20)
int hkx_gemm_noalloc(const HkxGemmArgs* args, void* stream);

/* bf16 C = (A . B^T) * scale_a * scale_b (+ bias), A (M, K) and B (N, K) fp8-e4m3,
 * scale_a fp32 with sa_ld 0 (one value for all rows: per-tensor) or its row
 * stride (per-token, (M, 1)); scale_b fp32, sb_per_channel 0 (one value) or 1
 * ((N,), per-channel); bias bf16 (N,) or NULL. Row strides in elements. */
int hkx_scaled_mm(const void* a, int64_t lda, const void* b, int64_t ldb,
                  const float* scale_a, int64_t sa_ld, const float* scale_b,
                  int32_t sb_per_channel, const void* bias, void* c, int64_t ldc,
                  int32_t m, int32_t n, int32_t k, void* ws, size_t ws_bytes,
                  void* stream);

/* bf16 C = (sa . A)(sb . B)^T: A (M, K) and B (N, K) fp8-e4m3, sa (M, K/32) and sb
 * (N, K/32) E8M0 bytes (scale 2^(s - 127) for its row and 32 K), row strides lda, ldb,
 * ldc in elements and sa_ld, sb_ld in bytes. K a multiple of 128, N of 8; sa and sb
 * 4-byte aligned with sa_ld, sb_ld multiples of 4 and >= K/32; C's rows 16-byte aligned.
 * M any. Where the 256 x 256 tiles fill less than half the CUs and K is 2048 or more, K is
 * split over workgroups (1024 K or more each, at most 8) into fp32 shares in ws (hkx_mx_gemm_workspace() bytes; HKX_ERR_WORKSPACE if
 * smaller), summed in split order by a second pass. */
int hkx_mx_gemm(const void* a, int64_t lda, const void* b, int64_t ldb, const uint8_t* sa,
                int64_t sa_ld, const uint8_t* sb, int64_t sb_ld, void* c, int64_t ldc,
                int32_t m, int32_t n, int32_t k, void* ws, size_t ws_bytes, void* stream);

/* Bytes of fp32 workspace hkx_mx_gemm needs at M x N x K (0 if it runs in one pass). */
size_t hkx_mx_gemm_workspace(int32_t m, int32_t n, int32_t k);

/* x bf16 (M, K) -> q fp8-e4m3 (M, K) and s (M, K/32) E8M0 bytes: per 32-column block,
 * e = ceil(log2(amax / 448)) with amax >= 2^-126, q = x / 2^e rounded to nearest even,
 * s = clamp(e + 127, 0, 254). K a multiple of 32; row strides in elements (bytes for
 * q and s). */
int hkx_mx_quant(const void* x, int64_t ldx, void* q, int64_t ldq, uint8_t* s, int64_t lds,
                 int32_t m, int32_t k, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HKX_H_ */
