// Measured ceilings of this GPU, the denominators the roofline fractions are also
// reported against (the reference measures its own the same way: a register-only MFMA
// loop and an HBM read past the Infinity Cache -- tools/cdna-probes/peaks.hip:1-17).
//
//   hkxp_mfma(dtype, waves_per_cu, iters, stream) -> launches the MFMA loop
//   hkxp_read(ptr, bytes, out, stream)            -> launches the HBM read
//   hkxp_clock(out, iters, stream)                -> shader clock ticks vs the 100 MHz
//                                                    real-time counter, under MFMA load
#include <hip/hip_runtime.h>
#include <type_traits>
#include <stdint.h>

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

// CH independent 32x32 accumulators a wave, operands in registers: the MFMA pipe's rate.
template <bool FP8, int CH = 4>
__global__ void __launch_bounds__(256) mfma_loop(float* out, int iters) {
  f32x16 acc[CH] = {};
  const int l = threadIdx.x;
  bf16x8 a = {(__bf16)(l * 1e-3f), (__bf16)1.f, (__bf16)0.5f, (__bf16)0.25f, (__bf16)1.f,
              (__bf16)2.f, (__bf16)3.f, (__bf16)4.f};
  i32x8 f = {l, 1, 2, 3, 4, 5, 6, 7};
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      if constexpr (FP8)
        acc[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f, f, acc[j], 0, 0, 0, 0, 0, 0);
      else
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, a, acc[j], 0, 0, 0);
    }
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < CH; ++j) s += acc[j][0] + acc[j][15];
  if (s == 1234.5f) out[blockIdx.x] = s;  // keeps the loop alive
}

// The same loop on operands of random bits (bf16: random sign and mantissa, exponent in
// [2^-7, 2^8); fp8 e4m3: random bytes with the exponent's top bit clear, so no NaN), four
// operand sets rotated so that consecutive MFMAs see different data: the MFMA rate when
// the datapath toggles as it does on real tensors, which draws more power than the
// constant operands above and so runs at a lower clock under the board's power limit.
__device__ inline uint32_t mix32(uint32_t x) {
  x ^= x >> 16; x *= 0x7feb352dU; x ^= x >> 15; x *= 0x846ca68bU; x ^= x >> 16;
  return x;
}
// W16: the 16 x 16 instructions the GEMM kernels issue (v_mfma_f32_16x16x32_bf16,
// v_mfma_scale_f32_16x16x128_f8f6f4), 8 accumulators a wave; else the 32 x 32 ones, 4. On
// random operands the 16 x 16 forms run the more flops under the power limit (bf16 about 3%,
// fp8 about 9%), so they set the ceiling.
template <bool FP8, bool W16 = false, int CH = W16 ? 8 : 4>
__global__ void __launch_bounds__(256) mfma_rand_loop(float* out, int iters) {
  using Acc = typename std::conditional<W16, f32x4, f32x16>::type;
  Acc acc[CH] = {};
  const uint32_t seed = (uint32_t)(blockIdx.x * 256 + threadIdx.x) * 0x9E3779B9u;
  i32x4 ab[8];   // bf16: 4 A and 4 B operand sets
  i32x8 fb[8];   // fp8
#pragma unroll
  for (int u = 0; u < 8; ++u)
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      const uint32_t r = mix32(seed + 8 * u + d);
      // bf16 pair: sign and mantissa random, exponent 120-135
      const uint32_t h0 = (r & 0x807f) | ((120 + ((r >> 8) & 15)) << 7);
      const uint32_t h1 = ((r >> 16) & 0x807f) | ((120 + ((r >> 24) & 15)) << 7);
      if (d < 4) ab[u][d] = (int)(h0 | (h1 << 16));
      fb[u][d] = (int)(r & 0xbfbfbfbfu);
    }
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int j = 0; j < CH; ++j) {
        if constexpr (FP8 && W16)
          acc[j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(fb[u], fb[4 + ((u + j) & 3)], acc[j], 0, 0, 0,
                                                                    0, 0, 0);
        else if constexpr (FP8)
          acc[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fb[u], fb[4 + ((u + j) & 3)], acc[j], 0, 0, 0,
                                                                   0, 0, 0);
        else if constexpr (W16)
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ab[u]),
                                                           __builtin_bit_cast(bf16x8, ab[4 + ((u + j) & 3)]),
                                                           acc[j], 0, 0, 0);
        else
          acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, ab[u]),
                                                           __builtin_bit_cast(bf16x8, ab[4 + ((u + j) & 3)]),
                                                           acc[j], 0, 0, 0);
      }
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < CH; ++j) s += acc[j][0] + acc[j][3];
  if (s == 1234.5f) out[blockIdx.x] = s;
}

// The GEMM kernels' instruction, v_mfma_f32_16x16x32_bf16, issued back to back by every
// wave: CH independent 16x16 accumulators a wave. Written as inline asm so the compiler
// keeps the accumulators in place (its own code for this loop shuffles them between
// register files every iteration). With one wave a SIMD this is the rate of a schedule
// whose MFMAs come from one wave at a time (the ping-pong GEMMs' math phases).
template <int CH>
__global__ void __launch_bounds__(256) mfma_issue_loop(float* out, int iters) {
  typedef float f32x4v __attribute__((ext_vector_type(4)));
  f32x4v acc[CH];
#pragma unroll
  for (int j = 0; j < CH; ++j) acc[j] = f32x4v{0.f, 0.f, 0.f, 0.f};
  const int l = threadIdx.x;
  bf16x8 a = {(__bf16)(l * 1e-3f), (__bf16)1.f, (__bf16)0.5f, (__bf16)0.25f, (__bf16)1.f,
              (__bf16)2.f, (__bf16)3.f, (__bf16)4.f};
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int j = 0; j < CH; ++j)
      asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(acc[j]) : "v"(a), "v"(a));
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < CH; ++j) s += acc[j][0];
  if (s == 1234.5f) out[blockIdx.x] = s;
}

__global__ void __launch_bounds__(256) read_kernel(const i32x4* p, size_t n16, int* out) {
  i32x4 acc = {0, 0, 0, 0};
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride * 4) {
    i32x4 v0 = __builtin_nontemporal_load(p + i);
    i32x4 v1 = i + stride < n16 ? __builtin_nontemporal_load(p + i + stride) : i32x4{0, 0, 0, 0};
    i32x4 v2 = i + 2 * stride < n16 ? __builtin_nontemporal_load(p + i + 2 * stride) : i32x4{0, 0, 0, 0};
    i32x4 v3 = i + 3 * stride < n16 ? __builtin_nontemporal_load(p + i + 3 * stride) : i32x4{0, 0, 0, 0};
    acc ^= v0 ^ v1 ^ v2 ^ v3;
  }
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x12345678) out[0] = 1;
}

// HBM read in 64 KB chunks strided over the grid: each thread keeps 8 loads of 16 bytes in
// flight (chunk c of workgroup g: c = g + i G), non-temporal (NT = 1) or plain.
template <int NT>
__global__ void __launch_bounds__(512) read_chunks_kernel(const i32x4* p, size_t n16, int* out) {
  constexpr int U = 8;
  const size_t per = (size_t)U * 512;  // 16-byte pieces a chunk
  i32x4 acc = {0, 0, 0, 0};
  for (size_t c = blockIdx.x; c * per < n16; c += gridDim.x) {
    const size_t base = c * per + threadIdx.x;
    i32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const size_t i = base + (size_t)u * 512;
      if (NT) v[u] = i < n16 ? __builtin_nontemporal_load(p + i) : i32x4{0, 0, 0, 0};
      else v[u] = i < n16 ? p[i] : i32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u];
  }
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x12345678) out[0] = 1;
}

__global__ void __launch_bounds__(256) clock_kernel(unsigned long long* out, int iters) {
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
  f32x16 acc[4] = {};
  bf16x8 a = {(__bf16)1.f, (__bf16)1.f, (__bf16)1.f, (__bf16)1.f, (__bf16)1.f, (__bf16)1.f,
              (__bf16)1.f, (__bf16)1.f};
  for (int i = 0; i < iters; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, a, acc[j], 0, 0, 0);
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
  if (threadIdx.x == 0) {
    out[2 * blockIdx.x] = t1 - t0;
    out[2 * blockIdx.x + 1] = r1 - r0;
  }
  if (acc[0][0] == 1234.5f) out[0] = 0;
}

// LDS read bandwidth: every wave reads 16 bytes a lane per ds_read_b128, `iters` x 16
// reads. pattern 0: lane l reads bytes 16 l of a 1 KB slab (conflict-free); pattern 1:
// the GEMM kernels' fragment read, row l & 31 of 128-byte rows, chunk (2 (i & 3) +
// (l >> 5)) ^ swz(l & 15).
__global__ void __launch_bounds__(256) lds_read_kernel(float* out, int iters, int pattern) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[65536];
  const int t = threadIdx.x, l = t & 63, w = t >> 6;
  for (int i = t; i < 65536 / 16; i += 256) ((i32x4*)lds)[i] = i32x4{i, i + 1, i + 2, i + 3};
  __syncthreads();
  i32x4 acc = {0, 0, 0, 0};
  unsigned off[4];
  for (int q = 0; q < 4; ++q) {
    if (pattern == 0) {
      off[q] = (unsigned)(w * 4096 + q * 1024 + l * 16);
    } else {
      const int r = l & 31, j = r & 15, sw = (j ^ (j >> 3)) & 7;
      off[q] = (unsigned)(w * 16384 + r * 128 + (((2 * q + (l >> 5)) ^ sw) << 4));
    }
  }
  for (int it = 0; it < iters; ++it) {
    unsigned z = (unsigned)(it & 3) << 14;
    asm volatile("" : "+v"(z));  // an offset the compiler cannot see through: no hoisting
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const i32x4 v = *(const i32x4*)(lds + ((off[q & 3] + ((q >> 2) << 12) + z) & 65535));
      acc ^= v;
    }
  }
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x7777777) out[blockIdx.x] = 1.f;
}

extern "C" {

int hkxp_lds(int pattern, int blocks, int iters, float* out, void* stream) {
  hipLaunchKernelGGL(lds_read_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, out, iters,
                     pattern);
  return (int)hipGetLastError();
}


int hkxp_mfma16(int blocks, int iters, float* out, void* stream) {
  hipLaunchKernelGGL((mfma_loop<false, 16>), dim3(blocks), dim3(256), 0, (hipStream_t)stream, out, iters);
  return (int)hipGetLastError();
}

int hkxp_mfma_issue(int blocks, int iters, float* out, void* stream) {
  hipLaunchKernelGGL((mfma_issue_loop<8>), dim3(blocks), dim3(256), 0, (hipStream_t)stream, out, iters);
  return (int)hipGetLastError();
}

int hkxp_mfma(int fp8, int blocks, int iters, float* out, void* stream) {
  if (fp8)
    hipLaunchKernelGGL(mfma_loop<true>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, out, iters);
  else
    hipLaunchKernelGGL(mfma_loop<false>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, out, iters);
  return (int)hipGetLastError();
}

int hkxp_mfma_rand(int fp8, int blocks, int iters, float* out, void* stream) {
  if (fp8)
    hipLaunchKernelGGL(mfma_rand_loop<true>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, out, iters);
  else
    hipLaunchKernelGGL(mfma_rand_loop<false>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, out, iters);
  return (int)hipGetLastError();
}

int hkxp_mfma_rand16(int fp8, int blocks, int iters, float* out, void* stream) {
  if (fp8)
    hipLaunchKernelGGL((mfma_rand_loop<true, true>), dim3(blocks), dim3(256), 0, (hipStream_t)stream, out, iters);
  else
    hipLaunchKernelGGL((mfma_rand_loop<false, true>), dim3(blocks), dim3(256), 0, (hipStream_t)stream, out, iters);
  return (int)hipGetLastError();
}

int hkxp_read(const void* p, size_t bytes, int* out, void* stream) {
  hipLaunchKernelGGL(read_kernel, dim3(256 * 16), dim3(256), 0, (hipStream_t)stream,
                     (const i32x4*)p, bytes / 16, out);
  return (int)hipGetLastError();
}

// variant 0: read_kernel; 1: 64 KB chunks, non-temporal; 2: 64 KB chunks, plain loads
int hkxp_read_v(int variant, const void* p, size_t bytes, int blocks, int* out, void* stream) {
  if (variant == 0)
    hipLaunchKernelGGL(read_kernel, dim3(256 * 16), dim3(256), 0, (hipStream_t)stream,
                       (const i32x4*)p, bytes / 16, out);
  else if (variant == 1)
    hipLaunchKernelGGL(read_chunks_kernel<1>, dim3(blocks), dim3(512), 0, (hipStream_t)stream,
                       (const i32x4*)p, bytes / 16, out);
  else
    hipLaunchKernelGGL(read_chunks_kernel<0>, dim3(blocks), dim3(512), 0, (hipStream_t)stream,
                       (const i32x4*)p, bytes / 16, out);
  return (int)hipGetLastError();
}

int hkxp_clock(unsigned long long* out, int blocks, int iters, void* stream) {
  hipLaunchKernelGGL(clock_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, out, iters);
  return (int)hipGetLastError();
}

}  // extern "C"
