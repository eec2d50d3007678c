// The split-K reduction, and the pass that runs an epilogue program.
//
// Replaces reduce_epilogue_kernel / strip_reduce_kernel (python/hk/ops/gemm_cdna_dp.py:
// 295-324, 361-383): C = epilogue(sum over splits of the fp32 shares), the shares added
// in split order (so a result is reproducible run to run) and the epilogue run once on
// the sum -- never on a share, since an epilogue need not be linear.
//
// The same kernel is the "separate pass" the reference falls back to for an epilogue
// that does not fit beside its GEMM's registers (templates/gemm.py:616-634): here that
// is any epilogue not of the fused form, written as a register program (include/hkx.h,
// HKX_OP_*) and interpreted four columns a thread. Its registers live in LDS, one
// private 16-byte slot per thread and register, so the program's register numbers can
// be run-time values without spilling.
#pragma once

#include "hkx_device.hpp"

namespace hkx {

struct ReduceArgs {
  const float* ws;
  int64_t split_stride;  // elements between shares
  int64_t ws_ld;         // row stride of a share (N, or 2N paired)
  void* c;
  int64_t ldc;
  int32_t splits;
  int32_t M, N;
  int32_t c_dt;
  int32_t pair;
  Fused f;
};

HKX_DEV f32x4 prog_load(const HkxOperand& o, int m, int n) {
  if (o.kind == HKX_ROW) {
    if (o.ld == 0) {
      float s = ld1(o.ptr, o.dtype, 0);
      return f32x4{s, s, s, s};
    }
    return ld4(o.ptr, o.dtype, n);
  }
  if (o.kind == HKX_COL) {
    float s = ld1(o.ptr, o.dtype, (int64_t)m * o.ld);
    return f32x4{s, s, s, s};
  }
  return ld4(o.ptr, o.dtype, (int64_t)m * o.ld + n);
}

template <int NT>
HKX_DEV f32x4 run_program(const HkxEpilogue& ep, f32x4 acc, int m, int n, int M,
                          f32x4 (*R)[NT], int t) {
  R[0][t] = acc;
  for (int pc = 0; pc < ep.nins; ++pc) {
    const HkxInstr I = ep.ins[pc];
    const f32x4 a = R[I.a][t];
    const f32x4 b = R[I.b][t];
    f32x4 r;
    switch (I.op) {
      case HKX_OP_MOV: r = a; break;
      case HKX_OP_LOAD: r = prog_load(ep.ops[I.a], m, n); break;
      case HKX_OP_CONST: r = f32x4{I.imm, I.imm, I.imm, I.imm}; break;
      case HKX_OP_ROW: r = f32x4{(float)m, (float)m, (float)m, (float)m}; break;
      case HKX_OP_COL: {
        const float c0 = (float)(n + ep.col0);
        r = f32x4{c0, c0 + 1.0f, c0 + 2.0f, c0 + 3.0f};
        break;
      }
      case HKX_OP_M: r = f32x4{(float)M, (float)M, (float)M, (float)M}; break;
      case HKX_OP_ADD: r = a + b; break;
      case HKX_OP_SUB: r = a - b; break;
      case HKX_OP_MUL: r = a * b; break;
      case HKX_OP_DIV: r = a / b; break;
      case HKX_OP_MAX:
        r = f32x4{__builtin_fmaxf(a.x, b.x), __builtin_fmaxf(a.y, b.y), __builtin_fmaxf(a.z, b.z),
                  __builtin_fmaxf(a.w, b.w)};
        break;
      case HKX_OP_MIN:
        r = f32x4{__builtin_fminf(a.x, b.x), __builtin_fminf(a.y, b.y), __builtin_fminf(a.z, b.z),
                  __builtin_fminf(a.w, b.w)};
        break;
      case HKX_OP_EXP:
        r = f32x4{__builtin_amdgcn_exp2f(a.x * kLog2e), __builtin_amdgcn_exp2f(a.y * kLog2e),
                  __builtin_amdgcn_exp2f(a.z * kLog2e), __builtin_amdgcn_exp2f(a.w * kLog2e)};
        break;
      case HKX_OP_EXP2:
        r = f32x4{__builtin_amdgcn_exp2f(a.x), __builtin_amdgcn_exp2f(a.y),
                  __builtin_amdgcn_exp2f(a.z), __builtin_amdgcn_exp2f(a.w)};
        break;
      case HKX_OP_LOG:
        r = f32x4{__builtin_amdgcn_logf(a.x) * kLn2, __builtin_amdgcn_logf(a.y) * kLn2,
                  __builtin_amdgcn_logf(a.z) * kLn2, __builtin_amdgcn_logf(a.w) * kLn2};
        break;
      case HKX_OP_LOG2:
        r = f32x4{__builtin_amdgcn_logf(a.x), __builtin_amdgcn_logf(a.y),
                  __builtin_amdgcn_logf(a.z), __builtin_amdgcn_logf(a.w)};
        break;
      case HKX_OP_ABS:
        r = f32x4{__builtin_fabsf(a.x), __builtin_fabsf(a.y), __builtin_fabsf(a.z),
                  __builtin_fabsf(a.w)};
        break;
      case HKX_OP_RELU: r = act4(HKX_ACT_RELU, a); break;
      case HKX_OP_GELU: r = act4(HKX_ACT_GELU_TANH, a); break;
      case HKX_OP_SILU: r = act4(HKX_ACT_SILU, a); break;
      case HKX_OP_SQRT:
        r = f32x4{__builtin_sqrtf(a.x), __builtin_sqrtf(a.y), __builtin_sqrtf(a.z),
                  __builtin_sqrtf(a.w)};
        break;
      case HKX_OP_RSQRT:
        r = f32x4{__builtin_amdgcn_rsqf(a.x), __builtin_amdgcn_rsqf(a.y),
                  __builtin_amdgcn_rsqf(a.z), __builtin_amdgcn_rsqf(a.w)};
        break;
      case HKX_OP_NEG: r = -a; break;
      case HKX_OP_STEP:
        r = f32x4{a.x > 0.f ? 1.f : 0.f, a.y > 0.f ? 1.f : 0.f, a.z > 0.f ? 1.f : 0.f,
                  a.w > 0.f ? 1.f : 0.f};
        break;
      case HKX_OP_SELLE: {
        const f32x4 c = R[I.c][t];
        r = f32x4{a.x <= 0.f ? b.x : c.x, a.y <= 0.f ? b.y : c.y, a.z <= 0.f ? b.z : c.z,
                  a.w <= 0.f ? b.w : c.w};
        break;
      }
      case HKX_OP_TANH: r = f32x4{tanh_f(a.x), tanh_f(a.y), tanh_f(a.z), tanh_f(a.w)}; break;
      case HKX_OP_SIGMOID:
        r = f32x4{sigmoid(a.x), sigmoid(a.y), sigmoid(a.z), sigmoid(a.w)};
        break;
      case HKX_OP_SQUARE: r = a * a; break;
      default: r = a; break;
    }
    R[I.dst][t] = r;
  }
  return R[ep.out_reg][t];
}

// The shares of 4 columns at src, summed in split order. Up to 8 splits the count is a
// compile-time constant (one straight-line body each), so every share's load is issued
// before the first add and a thread waits one memory latency, not one a split (a loop of
// load-then-add waited after each load: 5 us for 8 MB of shares at M = 128).
template <int S>
HKX_DEV f32x4 sum_splits_n(const float* src, int64_t stride) {
  f32x4 x[S];
#pragma unroll
  for (int s = 0; s < S; ++s) x[s] = *(const f32x4*)(src + s * stride);
  f32x4 v = x[0];
#pragma unroll
  for (int s = 1; s < S; ++s) v += x[s];
  return v;
}

HKX_DEV f32x4 sum_splits(const float* src, int splits, int64_t stride) {
  switch (splits) {
    case 1: return *(const f32x4*)src;
    case 2: return sum_splits_n<2>(src, stride);
    case 3: return sum_splits_n<3>(src, stride);
    case 4: return sum_splits_n<4>(src, stride);
    case 5: return sum_splits_n<5>(src, stride);
    case 6: return sum_splits_n<6>(src, stride);
    case 7: return sum_splits_n<7>(src, stride);
    case 8: return sum_splits_n<8>(src, stride);
    default: break;
  }
  f32x4 v = *(const f32x4*)src;
  for (int s = 1; s < splits; ++s) v += *(const f32x4*)(src + s * stride);
  return v;
}

template <bool PROGRAM>
__global__ void __launch_bounds__(256) reduce_kernel(const ReduceArgs p, const HkxEpilogue ep) {
  constexpr int NR = PROGRAM ? HKX_MAX_REGS : 1;
  __shared__ f32x4 R[NR][256];
  const int t = threadIdx.x;
  const int n = (blockIdx.x * 256 + t) * 4;
  if (n >= p.N) return;  // no barrier follows: each thread's registers are its own
  for (int m = blockIdx.y; m < p.M; m += gridDim.y) {
    const float* src = p.ws + (int64_t)m * p.ws_ld + n;
    f32x4 v = sum_splits(src, p.splits, p.split_stride);
    if (p.pair) {
      f32x4 u = sum_splits(src + p.N, p.splits, p.split_stride);
      v = silu_mul4(v, u);
    } else if constexpr (PROGRAM) {
      v = run_program<256>(ep, v, m, n, p.M, R, t);
    } else {
      v = fused_apply(p.f, v, m, n, true);
    }
    store4(p.c, p.c_dt, (int64_t)m * p.ldc + n, v);
  }
}

}  // namespace hkx
