// Q4_0 and Q8_0 block codecs on the device: the quantizers that produce
// hypno's packed weights and the dequantizers, bit-exact with the reference
// CPU code.
#include "common.hpp"

namespace hypno {

// Q4_0Block::quantize (quant.rs:49-71), one thread per 32-element block.
// amax folds |v| with fmaxf (NaN ignored, like f32::max); s = amax/7 in f32
// with IEEE division (1.0 for an all-zero block); d = f16 RNE(s);
// q = clamp(round_half_away(v / s), -8, 7) with NaN -> 0.
__global__ void __launch_bounds__(256)
quantize_q4_0_kernel(uint8_t* __restrict__ out, const float* __restrict__ src, size_t n_blocks) {
  const size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= n_blocks) return;
  const float* v = src + b * kBlockElems;
  float vals[kBlockElems];
  float max_abs = 0.0f;
#pragma unroll
  for (int i = 0; i < kBlockElems; i++) {
    vals[i] = v[i];
    max_abs = fmaxf(max_abs, fabsf(vals[i]));
  }
  const float scale = max_abs > 0.0f ? max_abs / 7.0f : 1.0f;
  const uint16_t d = __builtin_bit_cast(uint16_t, (_Float16)scale);
  uint8_t* o = out + b * kBlockBytes;
  o[0] = (uint8_t)(d & 0xFF);
  o[1] = (uint8_t)(d >> 8);
#pragma unroll
  for (int i = 0; i < 16; i++) {
    uint32_t nib[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const float r = roundf(vals[2 * i + j] / scale);
      int q = 0;
      if (r == r) q = (int)fminf(fmaxf(r, -8.0f), 7.0f);
      nib[j] = (uint32_t)(q + 8) & 0x0Fu;
    }
    o[2 + i] = (uint8_t)(nib[0] | (nib[1] << 4));
  }
}

// Q4_0Block::dequantize (quant.rs:25-34): element 2i = (lo - 8) * d,
// element 2i+1 = (hi - 8) * d.  The product of an integer in [-8, 7] and an
// fp16 value is exact in fp32, so the output is bit-exact.
__global__ void __launch_bounds__(256)
dequantize_q4_0_kernel(float* __restrict__ out, const uint8_t* __restrict__ q, size_t n_blocks) {
  const size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= n_blocks) return;
  const uint8_t* blk = q + b * kBlockBytes;
  const float scale = f16_bits_to_f32((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
  float* o = out + b * kBlockElems;
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const uint32_t byte = blk[2 + i];
    o[2 * i] = (float)((int)(byte & 0x0F) - 8) * scale;
    o[2 * i + 1] = (float)((int)(byte >> 4) - 8) * scale;
  }
}

// quantize_f32_to_q8_0 (quant.rs:177-191), one thread per block: amax as for
// Q4_0; d = f16 RNE(amax / 127) (1.0 for an all-zero block); unlike Q4_0 each
// value is divided by the ROUNDED scale f32(d); q = clamp(round_half_away(v /
// f32(d)), -127, 127) with NaN -> 0 and +-inf -> +-127 (Rust's saturating
// cast); byte = q + 128.
__global__ void __launch_bounds__(256)
quantize_q8_0_kernel(uint8_t* __restrict__ out, const float* __restrict__ src, size_t n_blocks) {
  const size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= n_blocks) return;
  const float* v = src + b * kBlockElems;
  float vals[kBlockElems];
  float max_abs = 0.0f;
#pragma unroll
  for (int i = 0; i < kBlockElems; i++) {
    vals[i] = v[i];
    max_abs = fmaxf(max_abs, fabsf(vals[i]));
  }
  const _Float16 dh = (_Float16)(max_abs > 0.0f ? max_abs / 127.0f : 1.0f);
  const uint16_t d = __builtin_bit_cast(uint16_t, dh);
  const float scale = (float)dh;
  uint8_t* o = out + b * kQ8BlockBytes;
  o[0] = (uint8_t)(d & 0xFF);
  o[1] = (uint8_t)(d >> 8);
#pragma unroll
  for (int i = 0; i < kBlockElems; i++) {
    const float r = roundf(vals[i] / scale);
    int q = 0;
    if (r == r) q = (int)fminf(fmaxf(r, -127.0f), 127.0f);
    o[2 + i] = (uint8_t)(q + 128);
  }
}

// Q8_0Block::dequantize (quant.rs:90-95): (u - 128) * d, exact in fp32.
__global__ void __launch_bounds__(256)
dequantize_q8_0_kernel(float* __restrict__ out, const uint8_t* __restrict__ q, size_t n_blocks) {
  const size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= n_blocks) return;
  const uint8_t* blk = q + b * kQ8BlockBytes;
  const float scale = f16_bits_to_f32((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
  float* o = out + b * kBlockElems;
#pragma unroll
  for (int i = 0; i < kBlockElems; i++) o[i] = (float)((int)blk[2 + i] - 128) * scale;
}

hipError_t launch_quantize_q8_0(uint8_t* out, const float* src, size_t n_blocks, hipStream_t s) {
  if (n_blocks == 0) return hipSuccess;
  const size_t grid = (n_blocks + 255) / 256;
  hipLaunchKernelGGL(quantize_q8_0_kernel, dim3((unsigned)grid), dim3(256), 0, s, out, src, n_blocks);
  return hipGetLastError();
}

hipError_t launch_dequantize_q8_0(float* out, const uint8_t* q, size_t n_blocks, hipStream_t s) {
  if (n_blocks == 0) return hipSuccess;
  const size_t grid = (n_blocks + 255) / 256;
  hipLaunchKernelGGL(dequantize_q8_0_kernel, dim3((unsigned)grid), dim3(256), 0, s, out, q, n_blocks);
  return hipGetLastError();
}

hipError_t launch_quantize_q4_0(uint8_t* out, const float* src, size_t n_blocks, hipStream_t s) {
  if (n_blocks == 0) return hipSuccess;
  const size_t grid = (n_blocks + 255) / 256;
  hipLaunchKernelGGL(quantize_q4_0_kernel, dim3((unsigned)grid), dim3(256), 0, s, out, src, n_blocks);
  return hipGetLastError();
}

hipError_t launch_dequantize_q4_0(float* out, const uint8_t* q, size_t n_blocks, hipStream_t s) {
  if (n_blocks == 0) return hipSuccess;
  const size_t grid = (n_blocks + 255) / 256;
  hipLaunchKernelGGL(dequantize_q4_0_kernel, dim3((unsigned)grid), dim3(256), 0, s, out, q, n_blocks);
  return hipGetLastError();
}

}  // namespace hypno
