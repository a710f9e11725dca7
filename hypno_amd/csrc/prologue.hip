// The decode step's neighbours of the GEMV as device kernels: RMS norm
// (kernels.rs:592-625) and silu(gate) * up (transformer.rs:446-449,
// turbo.rs:235-237).  The streaming GEMV applies both as prologues of its
// activation staging (gemv_q4_0.hip); these stand-alone kernels serve the
// other paths (any K, batched rows) and the C ABI's hypno_hip_rms_norm_dev /
// hypno_hip_silu_mul_dev.
#include "common.hpp"

namespace hypno {

namespace {

constexpr int kNormThreads = 256;

// One work-group per row.  Sum of squares: per-thread FMA chains, wave sums,
// then the waves' sums in a fixed order.  Elements below n - n % 8 are
// x * inv_rms * w, the last n % 8 are x / sqrt(mean + eps) * w, the two forms
// of kernels.rs:611-616.
__global__ void __launch_bounds__(kNormThreads)
rms_norm_rows_kernel(float* out, const float* x, const float* __restrict__ weight, size_t n,
                     float eps) {
  __shared__ float wsum[kNormThreads / 64];
  const size_t row = blockIdx.x;
  const float* xr = x + row * n;
  float* orow = out + row * n;
  const int t = threadIdx.x;
  float ss = 0.0f;
  for (size_t i = t; i < n; i += kNormThreads) ss = fmaf(xr[i], xr[i], ss);
  ss = wave_sum(ss);
  if ((t & 63) == 0) wsum[t >> 6] = ss;
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int w = 0; w < kNormThreads / 64; w++) tot += wsum[w];
  const float mean = tot / (float)n;
  const float root = sqrtf(mean + eps);
  const float inv = 1.0f / root;
  const size_t n8 = n - n % 8;
  // Every read of the row happens before any write (out may alias x): the
  // sum above is complete (barrier), and each element below is read and
  // written by the same thread.
  for (size_t i = t; i < n; i += kNormThreads) {
    const float v = xr[i];
    orow[i] = i < n8 ? v * inv * weight[i] : v / root * weight[i];
  }
}

__global__ void __launch_bounds__(256)
silu_mul_kernel(float* out, const float* gate, const float* __restrict__ up, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x) {
    const float g = gate[i];
    out[i] = g / (1.0f + expf(-g)) * up[i];
  }
}

}  // namespace

hipError_t launch_rms_norm(float* out, const float* x, const float* weight, size_t n,
                           size_t rows, float eps, hipStream_t s) {
  if (n == 0 || rows == 0) return hipSuccess;
  hipLaunchKernelGGL(rms_norm_rows_kernel, dim3((unsigned)rows), dim3(kNormThreads), 0, s, out, x,
                     weight, n, eps);
  return hipGetLastError();
}

hipError_t launch_silu_mul(float* out, const float* gate, const float* up, size_t n,
                           hipStream_t s) {
  if (n == 0) return hipSuccess;
  size_t grid = (n + 255) / 256;
  if (grid > 4096) grid = 4096;
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)grid), dim3(256), 0, s, out, gate, up, n);
  return hipGetLastError();
}

}  // namespace hypno
