// Device-side building blocks shared by every hkx kernel: vector types, buffer
// loads, element conversions, the epilogue operand loads and the two epilogue
// evaluators (the fused form, run in registers at the store, and the register
// program, run by the reduction kernel).
//
// The epilogue semantics follow hk.templates.gemm (python/hk/templates/gemm.py):
// operands are loaded in their layout and converted to fp32 (:212-226), the
// tanh-GELU is the exp2 form of :814-837 (a reciprocal where it squares a rsqrt), silu is x * sigmoid(x) (:845-847).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hkx.h"

#define HKX_DEV __device__ __forceinline__

namespace hkx {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- raw buffer loads
//
// A buffer resource bounds every access: an offset at or past `bytes` reads 0.
// The GEMM kernels lean on that for the rows of A past M and of B past N, so a
// ragged edge needs no clamping and no branch in the K loop.

constexpr int kRsrcWord3 = 0x00020000;  // gfx9 data format: 32-bit, raw

HKX_DEV __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           kRsrcWord3);
}

template <int AUX = 0>
HKX_DEV i32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, AUX));
}

// 16 bytes a lane from global memory straight into LDS: lane l's bytes land at
// lds + 16 l (the LDS base is wave-uniform; it goes in M0).
// AUX is the cache policy: kNonTemporal marks a stream read once (kept out of the caches).
constexpr int kNonTemporal = 2;
template <int AUX = 0>
HKX_DEV void buf_load16_lds(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16,
                                           voff, soff, 0, AUX);
}

// ---------------------------------------------------------------- conversions

HKX_DEV float bf16_to_f32(uint32_t bits16) { return __builtin_bit_cast(float, bits16 << 16); }

HKX_DEV f32x4 unpack_bf16x4(u32x2 w) {
  f32x4 r;
  r.x = __builtin_bit_cast(float, w.x << 16);
  r.y = __builtin_bit_cast(float, w.x & 0xffff0000u);
  r.z = __builtin_bit_cast(float, w.y << 16);
  r.w = __builtin_bit_cast(float, w.y & 0xffff0000u);
  return r;
}

HKX_DEV f32x4 unpack_f16x4(u32x2 w) {
  f32x4 r;
  r.x = (float)__builtin_bit_cast(_Float16, (uint16_t)(w.x & 0xffff));
  r.y = (float)__builtin_bit_cast(_Float16, (uint16_t)(w.x >> 16));
  r.z = (float)__builtin_bit_cast(_Float16, (uint16_t)(w.y & 0xffff));
  r.w = (float)__builtin_bit_cast(_Float16, (uint16_t)(w.y >> 16));
  return r;
}

// Round to nearest even (the hardware's conversion on gfx950: v_cvt_pk_bf16_f32).
// two floats to a packed pair, round to nearest even (one v_cvt_pk_* for the pair)
HKX_DEV uint32_t pack_bf16x2(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2_t));
}

HKX_DEV uint32_t pack_f16x2(float a, float b) {
  typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, f16x2_t));
}

// fp32 -> OCP e4m3 (float8_e4m3fn), round to nearest even, saturating at +-448
// (where torch's cast gives NaN; hk's quantizing store saturates -- templates/gemm.py:883-888).
// NaN stays NaN (0x7f). Written from the format's definition: bias 7, 3 mantissa
// bits, subnormals m * 2^-9.
HKX_DEV uint32_t f32_to_e4m3(float x) {
  uint32_t u = __builtin_bit_cast(uint32_t, x);
  uint32_t sign = (u >> 24) & 0x80u;
  float ax = __builtin_fabsf(x);
  if (ax != ax) return sign | 0x7fu;
  ax = __builtin_fminf(ax, 448.0f);
  uint32_t code;
  if (ax < 0.015625f) {  // below the smallest normal, 2^-6: a multiple of 2^-9
    code = (uint32_t)__builtin_rintf(ax * 512.0f);  // 8 carries into the first normal
  } else {
    int e = (int)((__builtin_bit_cast(uint32_t, ax) >> 23) & 0xff) - 127;  // -6 .. 8
    float scaled = __builtin_ldexpf(ax, 3 - e);                            // [8, 16)
    uint32_t m = (uint32_t)__builtin_rintf(scaled) - 8u;                    // 0 .. 8
    code = ((uint32_t)(e + 7) << 3) + m;                                    // m == 8 carries
  }
  return sign | code;
}

HKX_DEV uint32_t f32_to_i8(float x) {
  float r = __builtin_rintf(x);
  r = __builtin_fminf(__builtin_fmaxf(r, -128.0f), 127.0f);
  if (x != x) r = 0.0f;
  return (uint32_t)((int32_t)r) & 0xffu;
}

// ---------------------------------------------------------------- epilogue operands

struct Opnd {
  const void* p;  // nullptr: absent
  int64_t ld;
  int32_t dt;
  int32_t kind;
};

// 4 consecutive elements from element index idx, as fp32 (idx a multiple of 4 for
// 16-bit loads to be 8-byte aligned; the host checks alignment).
HKX_DEV f32x4 ld4(const void* p, int32_t dt, int64_t idx) {
  if (dt == HKX_BF16) return unpack_bf16x4(*(const u32x2*)((const uint16_t*)p + idx));
  if (dt == HKX_FP16) return unpack_f16x4(*(const u32x2*)((const uint16_t*)p + idx));
  return *(const f32x4*)((const float*)p + idx);
}

HKX_DEV float ld1(const void* p, int32_t dt, int64_t idx) {
  if (dt == HKX_BF16) return bf16_to_f32(((const uint16_t*)p)[idx]);
  if (dt == HKX_FP16) return (float)__builtin_bit_cast(_Float16, ((const uint16_t*)p)[idx]);
  return ((const float*)p)[idx];
}

// A ROW operand at columns n..n+3 (ld 0: one value for every column).
HKX_DEV f32x4 ld_row(const Opnd& o, int n) {
  if (o.ld == 0) {
    float s = ld1(o.p, o.dt, 0);
    return f32x4{s, s, s, s};
  }
  return ld4(o.p, o.dt, n);
}

HKX_DEV float ld_col(const Opnd& o, int m) { return ld1(o.p, o.dt, (int64_t)m * o.ld); }

HKX_DEV f32x4 ld_tile(const Opnd& o, int m, int n) {
  return ld4(o.p, o.dt, (int64_t)m * o.ld + n);
}

// ---------------------------------------------------------------- pointwise math

// tanh-GELU as x * sigmoid(2u), u = sqrt(2/pi)(x + 0.044715 x^3):
// sigmoid(2u) = 1 / (1 + 2^(x (A x^2 + B))) -- one v_exp_f32 and one v_rcp_f32 (the
// reference squares a v_rsq_f32 instead, templates/gemm.py:814-837: one more multiply).
// At x -> -inf the power is +inf and its reciprocal 0, so the product stays finite.
constexpr float kGeluB = -2.0f * 1.4426950408889634f * 0.7978845608028654f;
constexpr float kGeluA = kGeluB * 0.044715f;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

HKX_DEV float gelu_tanh(float x) {
  float q = x * x;
  q = __builtin_fmaf(q, kGeluA, kGeluB);
  q *= x;
  q = __builtin_amdgcn_exp2f(q);
  return x * __builtin_amdgcn_rcpf(1.0f + q);
}

// silu(x) = x * sigmoid(x) = x / (1 + e^-x); at x -> -inf, e^-x -> inf and the
// reciprocal -> 0, so the product stays finite.
HKX_DEV float silu(float x) {
  float e = __builtin_amdgcn_exp2f(-x * kLog2e);
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}

HKX_DEV float sigmoid(float x) {
  float e = __builtin_amdgcn_exp2f(-x * kLog2e);
  return __builtin_amdgcn_rcpf(1.0f + e);
}

HKX_DEV float tanh_f(float x) {
  // tanh(x) = 2 sigmoid(2x) - 1, with |x| large saturating through the reciprocal.
  return 2.0f * sigmoid(2.0f * x) - 1.0f;
}

// The activation as a template parameter (ACT < 0: chosen at run time, act4 below).
template <int ACT>
HKX_DEV f32x4 act4c(int act, f32x4 v);

HKX_DEV f32x4 act4(int act, f32x4 v) {
  if (act == HKX_ACT_GELU_TANH) {
    v.x = gelu_tanh(v.x); v.y = gelu_tanh(v.y); v.z = gelu_tanh(v.z); v.w = gelu_tanh(v.w);
  } else if (act == HKX_ACT_SILU) {
    v.x = silu(v.x); v.y = silu(v.y); v.z = silu(v.z); v.w = silu(v.w);
  } else if (act == HKX_ACT_RELU) {
    v.x = __builtin_fmaxf(v.x, 0.0f); v.y = __builtin_fmaxf(v.y, 0.0f);
    v.z = __builtin_fmaxf(v.z, 0.0f); v.w = __builtin_fmaxf(v.w, 0.0f);
  }
  return v;
}

template <int ACT>
HKX_DEV f32x4 act4c(int act, f32x4 v) {
  if constexpr (ACT < 0) return act4(act, v);
  else return act4(ACT, v);
}

// ---------------------------------------------------------------- the fused form
//
// C = act(acc * col_scale[m] * row_scale[n] * cmul + row_add[n] + tile_add[m, n] + cadd)
// -- bias, the activations, per-token x per-channel dequant, a residual -- and
// silu(gate) * up for the paired form. Every branch is on a kernel argument, so it
// is uniform: the wave takes it or skips it whole.

struct Fused {
  Opnd cs, rs, ra, ta;
  float cmul, cadd;
  int32_t act;
  int32_t form;  // HKX_EP_NONE / HKX_EP_FUSED / HKX_EP_SILU_MUL
};

// v: C[m, n..n+3] as fp32; mvalid: m < M (rows past M load nothing; their values are
// never stored).
HKX_DEV f32x4 fused_apply(const Fused& e, f32x4 v, int m, int n, bool mvalid) {
  if (e.form != HKX_EP_FUSED) return v;
  if (e.cs.p) {
    float s = mvalid ? ld_col(e.cs, m) : 0.0f;
    v *= s;
  }
  if (e.rs.p) v *= ld_row(e.rs, n);
  v *= e.cmul;
  if (e.ra.p) v += ld_row(e.ra, n);
  if (e.ta.p && mvalid) v += ld_tile(e.ta, m, n);
  v += e.cadd;
  return act4(e.act, v);
}

// Four epilogue operand values from LDS slots (one 32-bit slot per element: an fp32
// value, or a 16-bit value in the low (even element) or high (odd element) half).
HKX_DEV f32x4 slot4(const uint32_t* s, int dt) {
  const i32x4 w = *(const i32x4*)s;
  if (dt == HKX_FP32) return __builtin_bit_cast(f32x4, w);
  const u32x2 pk = u32x2{((uint32_t)w.x & 0xffffu) | ((uint32_t)w.y & 0xffff0000u),
                         ((uint32_t)w.z & 0xffffu) | ((uint32_t)w.w & 0xffff0000u)};
  return dt == HKX_FP16 ? unpack_f16x4(pk) : unpack_bf16x4(pk);
}

HKX_DEV float slot1(const uint32_t* s, int e, int dt) {
  const uint32_t w = s[e];
  if (dt == HKX_FP32) return __builtin_bit_cast(float, w);
  const uint32_t h = (e & 1) ? (w >> 16) : (w & 0xffffu);
  return dt == HKX_FP16 ? (float)__builtin_bit_cast(_Float16, (uint16_t)h) : bf16_to_f32(h);
}

HKX_DEV f32x4 silu_mul4(f32x4 g, f32x4 u) {
  return f32x4{silu(g.x) * u.x, silu(g.y) * u.y, silu(g.z) * u.z, silu(g.w) * u.w};
}

// ---------------------------------------------------------------- stores of 4 elements

// Stores C[m, n..n+3] (converted to dt) at element index idx of c.
HKX_DEV void store4(void* c, int32_t dt, int64_t idx, f32x4 v) {
  if (dt == HKX_BF16) {
    *(u32x2*)((uint16_t*)c + idx) = u32x2{pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w)};
  } else if (dt == HKX_FP16) {
    *(u32x2*)((uint16_t*)c + idx) = u32x2{pack_f16x2(v.x, v.y), pack_f16x2(v.z, v.w)};
  } else if (dt == HKX_FP32) {
    *(f32x4*)((float*)c + idx) = v;
  } else if (dt == HKX_FP8E4M3) {
    uint32_t w = f32_to_e4m3(v.x) | (f32_to_e4m3(v.y) << 8) | (f32_to_e4m3(v.z) << 16) |
                 (f32_to_e4m3(v.w) << 24);
    *(uint32_t*)((uint8_t*)c + idx) = w;
  } else {
    uint32_t w = f32_to_i8(v.x) | (f32_to_i8(v.y) << 8) | (f32_to_i8(v.z) << 16) |
                 (f32_to_i8(v.w) << 24);
    *(uint32_t*)((uint8_t*)c + idx) = w;
  }
}

// The same four elements packed for an output of OB bytes an element: 8 bytes
// (two dwords) for 16-bit, 4 bytes (x) for 8-bit.
template <int OB>
HKX_DEV u32x2 pack4(int32_t dt, f32x4 v) {
  if constexpr (OB == 2) {
    if (dt == HKX_FP16) return u32x2{pack_f16x2(v.x, v.y), pack_f16x2(v.z, v.w)};
    return u32x2{pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w)};
  } else {
    if (dt == HKX_FP8E4M3)
      return u32x2{f32_to_e4m3(v.x) | (f32_to_e4m3(v.y) << 8) | (f32_to_e4m3(v.z) << 16) |
                       (f32_to_e4m3(v.w) << 24),
                   0u};
    return u32x2{f32_to_i8(v.x) | (f32_to_i8(v.y) << 8) | (f32_to_i8(v.z) << 16) |
                     (f32_to_i8(v.w) << 24),
                 0u};
  }
}

}  // namespace hkx
