// FP16-weight matrix-vector kernels (the lm_head variant, kernels.rs:543-586).
//
//  * f16_generic_kernel: any m, any alignment, any number of tokens; one wave
//    per (token, row).
//  * f16_gemv_fast_kernel: one token; each wave owns kRows consecutive rows and
//    its lanes stream 16-byte chunks (8 weights) of all kRows rows together
//    (non-temporal loads), so every activation chunk loaded from cache feeds
//    kRows rows.  Weights are widened exactly to fp32 and accumulated in
//    fp32.
#include "common.hpp"

namespace hypno {

__global__ void __launch_bounds__(256)
f16_generic_kernel(float* __restrict__ y, const uint8_t* __restrict__ w,
                   const float* __restrict__ x, const float* __restrict__ bias, size_t n, size_t m,
                   size_t batch) {
  const size_t wave = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (wave >= n * batch) return;  // wave-uniform
  const size_t t = wave / n;
  const size_t r = wave - t * n;
  const uint8_t* row = w + r * m * 2;
  const float* xt = x + t * m;
  float acc = 0.0f;
  for (size_t k = lane; k < m; k += 64) {
    const uint32_t bits = (uint32_t)row[2 * k] | ((uint32_t)row[2 * k + 1] << 8);
    acc = fmaf(f16_bits_to_f32(bits), xt[k], acc);
  }
  acc = wave_sum(acc);
  if (lane == 0) y[t * n + r] = acc + (bias ? bias[r] : 0.0f);
}

hipError_t launch_f16_generic(float* y, const uint8_t* w, const float* x, const float* bias,
                              size_t n, size_t m, size_t batch, hipStream_t s) {
  const size_t waves = n * batch;
  if (waves == 0) return hipSuccess;
  const size_t grid = (waves + 3) / 4;
  hipLaunchKernelGGL(f16_generic_kernel, dim3((unsigned)grid), dim3(256), 0, s, y, w, x, bias, n,
                     m, batch);
  return hipGetLastError();
}

constexpr int kF16Rows = 4;

bool f16_gemv_fast_ok(const uint8_t* w, size_t n, size_t m) {
  if (m == 0 || m % 8 != 0 || n == 0 || n > (size_t)0x7FFFFFFF) return false;
  return ((uintptr_t)w & 15) == 0;
}

__global__ void __launch_bounds__(256)
f16_gemv_fast_kernel(float* __restrict__ y, const uint8_t* __restrict__ w,
                     const float* __restrict__ x, const float* __restrict__ bias, int n, int m) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int row0 = wave * kF16Rows;
  if (row0 >= n) return;  // wave-uniform
  const int chunks = m / 8;
  const float4* xv = reinterpret_cast<const float4*>(x);
  const uint4* wr[kF16Rows];
  int nrows = n - row0 < kF16Rows ? n - row0 : kF16Rows;
#pragma unroll
  for (int r = 0; r < kF16Rows; r++)
    wr[r] = reinterpret_cast<const uint4*>(w + (size_t)(row0 + (r < nrows ? r : 0)) * m * 2);
  float acc[kF16Rows];
#pragma unroll
  for (int r = 0; r < kF16Rows; r++) acc[r] = 0.0f;
  // Weights are read once: non-temporal loads (measured on the lm_head, 1.05
  // GB: 159 us per call against 177 with ordinary loads and the loop
  // unrolled twice).
#pragma unroll 1
  for (int c = lane; c < chunks; c += 64) {
    const float4 xa = xv[2 * c];
    const float4 xb = xv[2 * c + 1];
    const float xs[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
    for (int r = 0; r < kF16Rows; r++) {
      const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wr[r]) + c);
      const uint32_t u[4] = {v[0], v[1], v[2], v[3]};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        acc[r] = fmaf(f16_bits_to_f32(u[j] & 0xFFFFu), xs[2 * j], acc[r]);
        acc[r] = fmaf(f16_bits_to_f32(u[j] >> 16), xs[2 * j + 1], acc[r]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < kF16Rows; r++) {
    const float v = wave_sum(acc[r]);
    if (lane == 0 && r < nrows) y[row0 + r] = v + (bias ? bias[row0 + r] : 0.0f);
  }
}

hipError_t launch_f16_gemv_fast(float* y, const uint8_t* w, const float* x, const float* bias,
                                size_t n, size_t m, int num_cus, hipStream_t s) {
  (void)num_cus;
  const size_t waves = (n + kF16Rows - 1) / kF16Rows;
  const size_t grid = (waves + 3) / 4;
  hipLaunchKernelGGL(f16_gemv_fast_kernel, dim3((unsigned)grid), dim3(256), 0, s, y, w, x, bias,
                     (int)n, (int)m);
  return hipGetLastError();
}

}  // namespace hypno
