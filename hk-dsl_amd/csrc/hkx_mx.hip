// MX quantization of bf16 rows: fp8 e4m3 values with an E8M0 scale a 32-column block.
//
// The rule is AITER's per_1x32 (restated from python/hk/mx.py:17-31): for each block,
// amax = max |x| (at least 2^-126), e = ceil(log2(amax / 448)) -- computed exactly as
// floor(log2 amax) - 8, plus one where amax > 448 * 2^e --, q = x / 2^e clamped to +-448 and
// rounded to the nearest even e4m3, scale byte clamp(e + 127, 0, 254). The block's largest
// value lands at or below 448, so nothing is clamped but a rounding at the top.
//
// One thread a 16-byte piece (8 values) of a row; the 4 threads of a 32-column block are
// consecutive lanes and meet with two xor-shuffles. x / 2^e is an exact power-of-two
// scaling (ldexp), which the division also is, so the result is bit for bit the same.
#include "hkx_device.hpp"
#include "hkx_launch.hpp"

namespace hkx {

__global__ void __launch_bounds__(256) mx_quant_kernel(const uint16_t* x, int64_t ldx, uint8_t* q,
                                                       int64_t ldq, uint8_t* sc, int64_t lds,
                                                       int m, int k8) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = (int64_t)m * k8;
  const bool ok = t < total;  // whole 4-thread groups are in or out (k8 % 4 == 0)
  const int64_t row = ok ? t / k8 : 0;
  const int g = ok ? (int)(t - row * k8) : 0;
  float v[8];
  float amax = 0.0f;
  if (ok) {
    const i32x4 w = *(const i32x4*)(x + row * ldx + 8 * g);
    const uint32_t ws[4] = {(uint32_t)w.x, (uint32_t)w.y, (uint32_t)w.z, (uint32_t)w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __builtin_bit_cast(float, ws[i] << 16);
      v[2 * i + 1] = __builtin_bit_cast(float, ws[i] & 0xffff0000u);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = __builtin_fmaxf(amax, __builtin_fabsf(v[i]));
  }
  amax = __builtin_fmaxf(amax, __shfl_xor(amax, 1));
  amax = __builtin_fmaxf(amax, __shfl_xor(amax, 2));
  if (!ok) return;
  amax = __builtin_fmaxf(amax, 0x1p-126f);
  int e = (int)((__builtin_bit_cast(uint32_t, amax) >> 23) & 0xff) - 127 - 8;
  if (amax > __builtin_ldexpf(448.0f, e)) e += 1;
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float r = __builtin_ldexpf(v[i], -e);
    r = __builtin_fminf(__builtin_fmaxf(r, -448.0f), 448.0f);
    const uint32_t b = f32_to_e4m3(r);
    if (i < 4) lo |= b << (8 * i);
    else hi |= b << (8 * (i - 4));
  }
  *(u32x2*)(q + row * ldq + 8 * g) = u32x2{lo, hi};
  if ((g & 3) == 0) sc[row * lds + g / 4] = (uint8_t)min(max(e + 127, 0), 254);
}

hipError_t launch_mx_quant(const void* x, int64_t ldx, void* q, int64_t ldq, uint8_t* sc,
                           int64_t lds, int m, int k, hipStream_t s) {
  const int k8 = k / 8;
  const int64_t total = (int64_t)m * k8;
  const dim3 grid((unsigned)((total + 255) / 256));
  hipLaunchKernelGGL(mx_quant_kernel, grid, dim3(256), 0, s, (const uint16_t*)x, ldx,
                     (uint8_t*)q, ldq, sc, lds, m, k8);
  return hipGetLastError();
}

}  // namespace hkx
