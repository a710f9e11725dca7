// Q8_0 prefill (turbo.rs:334-341 dequantises the tensor to fp32 and runs one
// matmul_f32 per token).  Here, for M >= 16 tokens: the weights are expanded
// once per call to fp16 in a workspace and an fp16 MFMA GEMM runs on them
// (gemm_q4.hip: the register-streaming kernel up to 64 tokens, the DMA-fed
// one beyond), with the activations rounded to fp16 as on the other GEMM
// paths.
//
// Each row n is expanded as (u - 128) * (d / D_n), D_n = the row's largest
// |d|: every value then lies in [-128, 128], so none overflows fp16 (a plain
// (u - 128) * d would for |w| > 65504), and each weight is rounded to fp16
// once (relative 2^-11).  The GEMM's epilogue multiplies output column n by
// D_n and adds the bias.  A row whose largest |d| is 0 or not finite keeps
// D_n = 1.
#include "common.hpp"

namespace hypno {

namespace {

// out[g][8k + i] = fp16((u_{8k+i} - 128) * (d / D)), i < 8: quarter k of
// Q8_0 block g, read as four 2-byte loads (the block's bytes are 2-byte
// aligned) and written as one 16-byte store.
__device__ __forceinline__ void q8_0_quarter_to_f16(_Float16* __restrict__ out,
                                                    const uint8_t* __restrict__ w, size_t g, int k,
                                                    float D) {
  const uint8_t* blk = w + g * kQ8BlockBytes;
  const float d = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(blk));
  const float r = d / D;
  const uint16_t* q = reinterpret_cast<const uint16_t*>(blk + 2 + 8 * k);
  u32x4 o;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t two = q[i];
    const _Float16 lo = (_Float16)((float)((int)(two & 0xFFu) - 128) * r);
    const _Float16 hi = (_Float16)((float)((int)(two >> 8) - 128) * r);
    o[i] = (uint32_t)__builtin_bit_cast(uint16_t, lo) |
           ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
  }
  *reinterpret_cast<u32x4*>(out + g * kBlockElems + 8 * k) = o;  // 16-aligned
}

// One wave per weight row: D[row] = max |d| over the row's blocks (1 when
// that is 0 or not finite), then the row's blocks to fp16.  The row's bytes are read from HBM once: the conversion finds them
// in the caches the scale pass filled.
__global__ void __launch_bounds__(256)
q8_0_rows_to_f16_kernel(_Float16* __restrict__ out, float* __restrict__ D,
                        const uint8_t* __restrict__ w, size_t n, int bpr) {
  const size_t row = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (row >= n) return;  // wave-uniform
  const uint8_t* base = w + row * (size_t)bpr * kQ8BlockBytes;
  float mx = 0.0f;
  for (int b = lane; b < bpr; b += 64) {
    const uint8_t* blk = base + (size_t)b * kQ8BlockBytes;
    mx = fmaxf(mx, fabsf(f16_bits_to_f32((uint32_t)blk[0] | ((uint32_t)blk[1] << 8))));
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  const float dr = (mx > 0.0f && mx <= 3.0e38f) ? mx : 1.0f;
  if (lane == 0) D[row] = dr;
  // four lanes per block, consecutive lanes on consecutive 16-byte outputs
  for (int gi = lane; gi < 4 * bpr; gi += 64)
    q8_0_quarter_to_f16(out, w, row * (size_t)bpr + (gi >> 2), gi & 3, dr);
}

size_t round256(size_t b) { return (b + 255) / 256 * 256; }

bool mul_overflows_sz(size_t a, size_t b) { return a != 0 && b > SIZE_MAX / 2 / a; }

}  // namespace

bool q8_0_gemm_ok(size_t n, size_t m, size_t batch) {
  // The fp16 copy sits at the start of a 256-byte-aligned workspace (the
  // address passed only stands for that alignment); K a multiple of the
  // GEMM's 64-column stage, so rows hold whole blocks.
  return m % 64 == 0 && !mul_overflows_sz(n, m) &&
         f16_gemm_v2_ok(reinterpret_cast<const uint8_t*>((uintptr_t)256), n, m, batch);
}

// The fp16 GEMM for the expanded weights (16-byte aligned: the workspace
// start is 256-byte aligned): the register-streaming kernel up to 64 tokens
// (Mistral gate/up- and down-sized calls 6-8% faster at 16 and 64 tokens),
// the DMA-fed one beyond (2-3% faster at 128).
bool q8_0_use_stream(size_t n, size_t m, size_t batch) {
  return batch <= 64 &&
         f16_gemm_stream_ok(reinterpret_cast<const uint8_t*>((uintptr_t)256), nullptr, n, m, batch);
}
size_t q8_0_gemm_workspace_bytes(size_t batch, size_t n, size_t m, int num_cus) {
  return round256(n * m * 2) + round256(n * 4) +
         (q8_0_use_stream(n, m, batch) ? f16_gemm_stream_workspace_bytes(batch, n, m, num_cus)
                                       : f16_gemm_v2_workspace_bytes(batch, n, m, num_cus));
}

hipError_t launch_q8_0_gemm(float* y, const uint8_t* w, const float* x, const float* bias,
                            size_t n, size_t m, size_t batch, void* ws, int num_cus,
                            hipStream_t s) {
  uint8_t* base = static_cast<uint8_t*>(ws);
  _Float16* w16 = reinterpret_cast<_Float16*>(base);
  float* D = reinterpret_cast<float*>(base + round256(n * m * 2));
  void* gemm_ws = base + round256(n * m * 2) + round256(n * 4);
  const int bpr = (int)(m / kBlockElems);
  hipLaunchKernelGGL(q8_0_rows_to_f16_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, s, w16,
                     D, w, n, bpr);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  // the fp16 GEMM's epilogue multiplies output column n by D[n] and adds the bias
  if (q8_0_use_stream(n, m, batch))
    return launch_f16_gemm_stream(y, reinterpret_cast<const uint8_t*>(w16), x, bias, n, m, batch,
                                  gemm_ws, num_cus, s, D);
  return launch_f16_gemm_v2(y, reinterpret_cast<const uint8_t*>(w16), x, bias, n, m, batch,
                            gemm_ws, num_cus, s, D);
}

}  // namespace hypno
