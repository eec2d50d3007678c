// MX quantization of bf16 rows: fp8 e4m3 values with an E8M0 scale a 32-column block.
//
// The rule is AITER's per_1x32 (restated from python/hk/mx.py:17-31): for each block,
// amax = max |x| (at least 2^-126), e = ceil(log2(amax / 448)) -- computed exactly as
// floor(log2 amax) - 8, plus one where amax > 448 * 2^e --, q = x / 2^e clamped to +-448 and
// rounded to the nearest even e4m3, scale byte clamp(e + 127, 0, 254). The block's largest
// value lands at or below 448, so nothing is clamped but a rounding at the top.
//
// A workgroup 512 consecutive 16-byte pieces (8 values) of the row-major piece index, each
// thread two of them 256 apart, both loaded before either is quantized; a piece's row is a
// 32-bit division wherever the index fits in 32 bits. The 4 threads of a 32-column block are
// consecutive lanes and meet with two xor-shuffles. x / 2^e is an exact power-of-two scaling
// (ldexp), which the division also is, so the result is bit for bit the same.
#include "hkx_device.hpp"
#include "hkx_launch.hpp"

namespace hkx {

template <typename IDX>
__global__ void __launch_bounds__(256) mx_quant_kernel(const uint16_t* x, int64_t ldx, uint8_t* q,
                                                       int64_t ldq, uint8_t* sc, int64_t lds,
                                                       int m, int k8) {
  const IDX total = (IDX)m * (IDX)k8;
  const IDX p0 = (IDX)blockIdx.x * 512 + threadIdx.x;
  i32x4 w[2];
  IDX row[2];
  int g[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {  // whole 4-thread groups are in or out (k8 % 4 == 0)
    const IDX p = p0 + 256 * u;
    const bool ok = p < total;
    row[u] = ok ? p / (IDX)k8 : 0;
    g[u] = ok ? (int)(p - row[u] * (IDX)k8) : k8;
    w[u] = ok ? *(const i32x4*)(x + (int64_t)row[u] * ldx + 8 * g[u]) : i32x4{0, 0, 0, 0};
  }
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    float v[8];
    const uint32_t ws[4] = {(uint32_t)w[u].x, (uint32_t)w[u].y, (uint32_t)w[u].z, (uint32_t)w[u].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __builtin_bit_cast(float, ws[i] << 16);
      v[2 * i + 1] = __builtin_bit_cast(float, ws[i] & 0xffff0000u);
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = __builtin_fmaxf(amax, __builtin_fabsf(v[i]));
    amax = __builtin_fmaxf(amax, __shfl_xor(amax, 1));
    amax = __builtin_fmaxf(amax, __shfl_xor(amax, 2));
    if (g[u] >= k8) continue;
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
    *(u32x2*)(q + (int64_t)row[u] * ldq + 8 * g[u]) = u32x2{lo, hi};
    if ((g[u] & 3) == 0)
      sc[(int64_t)row[u] * lds + g[u] / 4] = (uint8_t)min(max(e + 127, 0), 254);
  }
}

hipError_t launch_mx_quant(const void* x, int64_t ldx, void* q, int64_t ldq, uint8_t* sc,
                           int64_t lds, int m, int k, hipStream_t s) {
  const int k8 = k / 8;
  const int64_t total = (int64_t)m * k8;
  const dim3 grid((unsigned)((total + 511) / 512));
  if (total + 512 < (int64_t)1 << 32)  // a 32-bit row division wherever the index fits
    hipLaunchKernelGGL(mx_quant_kernel<uint32_t>, grid, dim3(256), 0, s, (const uint16_t*)x,
                       ldx, (uint8_t*)q, ldq, sc, lds, m, k8);
  else
    hipLaunchKernelGGL(mx_quant_kernel<uint64_t>, grid, dim3(256), 0, s, (const uint16_t*)x,
                       ldx, (uint8_t*)q, ldq, sc, lds, m, k8);
  return hipGetLastError();
}

}  // namespace hkx
