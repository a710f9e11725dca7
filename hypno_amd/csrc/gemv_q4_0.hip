// Q4_0 matrix-vector kernels for gfx950.
//
//  * q4_0_generic_kernel: any m (blocks straddling rows), any alignment, short
//    weight buffers, bias, and any number of tokens.  One wave per
//    (token, row); lanes walk the row's overlapping blocks.  Semantics follow
//    matmul_q4_0_scalar (kernels.rs:362-400).
//  * q4_0_gemv_fast_kernel: the decode GEMV (one token).  A work-group owns a
//    fixed set of 64-element column ranges ("pairs" of two 18-byte blocks, 36
//    bytes each) and keeps the matching 64 activations in registers; it then
//    walks groups of rows.  Each step streams `rows*m/32*18` contiguous bytes
//    with 16-byte loads (rows are 16-byte aligned because m % 256 == 0),
//    stages them in LDS, and every thread decodes its 36-byte pair from LDS,
//    unpacks the nibbles in registers and accumulates in fp32.  Per-row sums
//    finish with wave shuffles (and an LDS hop when a row spans waves).
#include "common.hpp"

namespace hypno {

__global__ void __launch_bounds__(256)
q4_0_generic_kernel(float* __restrict__ y, const uint8_t* __restrict__ w, size_t w_len,
                    const float* __restrict__ x, const float* __restrict__ bias, size_t n,
                    size_t m, size_t batch) {
  const size_t wave = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (wave >= n * batch) return;  // wave-uniform
  const size_t t = wave / n;
  const size_t r = wave - t * n;
  const float* xt = x + t * m;
  float acc = 0.0f;
  if (m > 0) {
    const size_t row_start = r * m;
    const size_t row_end = row_start + m;
    const size_t first = row_start / kBlockElems;
    const size_t last = (row_end - 1) / kBlockElems;
    const size_t avail = w_len / kBlockBytes;  // blocks that fit (kernels.rs:374)
    const size_t stop = last + 1 < avail ? last + 1 : avail;
    for (size_t b = first + lane; b < stop; b += 64) {
      const uint8_t* blk = w + b * kBlockBytes;
      const float d = f16_bits_to_f32((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
      const size_t bs = b * kBlockElems;
      const size_t os = bs < row_start ? row_start - bs : 0;
      const size_t oe = bs + kBlockElems > row_end ? row_end - bs : kBlockElems;
      const size_t xo = bs > row_start ? bs - row_start : 0;
      for (size_t i = os; i < oe; i++) {
        const uint32_t byte = blk[2 + (i >> 1)];
        const uint32_t nib = (i & 1) ? (byte >> 4) : (byte & 0x0Fu);
        const float deq = (float)((int)nib - 8) * d;
        acc = fmaf(deq, xt[xo + (i - os)], acc);
      }
    }
  }
  acc = wave_sum(acc);
  if (lane == 0) y[t * n + r] = acc + (bias ? bias[r] : 0.0f);
}

hipError_t launch_q4_0_generic(float* y, const uint8_t* w, size_t w_len, const float* x,
                               const float* bias, size_t n, size_t m, size_t batch,
                               hipStream_t s) {
  const size_t waves = n * batch;
  if (waves == 0) return hipSuccess;
  const size_t grid = (waves + 3) / 4;  // 4 waves per 256-thread group
  hipLaunchKernelGGL(q4_0_generic_kernel, dim3((unsigned)grid), dim3(256), 0, s, y, w, w_len, x,
                     bias, n, m, batch);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Fast decode GEMV
// ---------------------------------------------------------------------------

// Work-group geometry for P = m/64 pairs per row: T threads, rps rows/step.
struct GemvGeom {
  int P, T, rps;
  bool shuffle;  // rows are power-of-two lane segments inside one wave
};

static int gcd_int(int a, int b) {
  while (b) {
    int t = a % b;
    a = b;
    b = t;
  }
  return a;
}

static GemvGeom gemv_geom(size_t m) {
  GemvGeom g;
  g.P = (int)(m / 64);
  if (g.P <= 64 && (g.P & (g.P - 1)) == 0) {
    g.T = 256;
    g.shuffle = true;
  } else {
    const int l = g.P / gcd_int(g.P, 64) * 64;  // lcm(P, 64)
    g.T = l <= 1024 ? l : ((g.P + 63) / 64) * 64;
    g.shuffle = false;
  }
  g.rps = g.T / g.P;
  return g;
}

bool q4_0_gemv_fast_ok(const uint8_t* w, size_t w_len, size_t n, size_t m) {
  if (m == 0 || m % 256 != 0 || m > 65536) return false;
  if (n == 0 || n > (size_t)0x7FFFFFFF) return false;
  if (((uintptr_t)w & 15) != 0) return false;
  return w_len / kBlockBytes >= n * (m / kBlockElems);
}

template <bool kShuffle>
__global__ void __launch_bounds__(1024)
q4_0_gemv_fast_kernel(float* __restrict__ y, const uint8_t* __restrict__ w,
                      const float* __restrict__ x, const float* __restrict__ bias, int n, int P,
                      int rps) {
  extern __shared__ __align__(16) uint8_t smem[];
  uint4* stage = reinterpret_cast<uint4*>(smem);
  const int T = blockDim.x;
  const int t = threadIdx.x;
  float* red = reinterpret_cast<float*>(smem + (size_t)rps * P * 36);

  const int p = t % P;
  const int rs = t / P;
  const bool active = rs < rps;

  // 64 activations of this thread's pair, and their two block sums (the -8
  // offset of every nibble is applied once per block as -8 * sum(x)).
  float xr[64];
  {
    const float4* xv = reinterpret_cast<const float4*>(x + (size_t)64 * p);
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const float4 v = xv[i];
      xr[4 * i + 0] = v.x;
      xr[4 * i + 1] = v.y;
      xr[4 * i + 2] = v.z;
      xr[4 * i + 3] = v.w;
    }
  }
  float xs0 = 0.0f, xs1 = 0.0f;
#pragma unroll
  for (int i = 0; i < 32; i++) {
    xs0 += xr[i];
    xs1 += xr[32 + i];
  }

  const size_t row_bytes = (size_t)P * 36;
  const int total_steps = (n + rps - 1) / rps;
  for (int step = blockIdx.x; step < total_steps; step += gridDim.x) {
    const int row0 = step * rps;
    const int rows = min(rps, n - row0);
    const int chunks = rows * P * 9 / 4;  // 16-byte chunks in this step
    const uint4* src = reinterpret_cast<const uint4*>(w + (size_t)row0 * row_bytes);
    for (int c = t; c < chunks; c += T) stage[c] = src[c];
    __syncthreads();

    float part = 0.0f;
    if (active && rs < rows) {
      const uint32_t* u = reinterpret_cast<const uint32_t*>(smem) + 9 * t;
      uint32_t d[9];
#pragma unroll
      for (int j = 0; j < 9; j++) d[j] = u[j];
      // block 0: bytes 0-1 scale, 2-17 nibbles; block 1: bytes 18-19, 20-35
      const float s0 = f16_bits_to_f32(d[0] & 0xFFFFu);
      const float s1 = f16_bits_to_f32(d[4] >> 16);
      float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint32_t q0 = __builtin_amdgcn_alignbit(d[j + 1], d[j], 16);
        a0 += dot8_nib(q0, xr + 8 * j);
        a1 += dot8_nib(d[5 + j], xr + 32 + 8 * j);
      }
      part = fmaf(s0, fmaf(-8.0f, xs0, a0), s1 * fmaf(-8.0f, xs1, a1));
    }

    if (kShuffle) {
      // P is a power of two <= 64: each row is an aligned segment of P lanes.
      for (int off = P >> 1; off > 0; off >>= 1) part += __shfl_xor(part, off, 64);
      if (active && rs < rows && p == 0)
        y[row0 + rs] = part + (bias ? bias[row0 + rs] : 0.0f);
      __syncthreads();
    } else {
      red[t] = part;
      __syncthreads();
      const int wv = t >> 6, lane = t & 63, nw = T >> 6;
      for (int r = wv; r < rows; r += nw) {  // wave-uniform loop
        float v = 0.0f;
        for (int q = lane; q < P; q += 64) v += red[r * P + q];
        v = wave_sum(v);
        if (lane == 0) y[row0 + r] = v + (bias ? bias[row0 + r] : 0.0f);
      }
      __syncthreads();
    }
  }
}

hipError_t launch_q4_0_gemv_fast(float* y, const uint8_t* w, const float* x, const float* bias,
                                 size_t n, size_t m, int num_cus, hipStream_t s) {
  const GemvGeom g = gemv_geom(m);
  const int total_steps = (int)((n + g.rps - 1) / g.rps);
  const int per_cu = g.T <= 256 ? 4 : (g.T <= 512 ? 2 : 1);
  const int grid = total_steps < num_cus * per_cu ? total_steps : num_cus * per_cu;
  const size_t lds = (size_t)g.rps * g.P * 36 + (g.shuffle ? 0 : (size_t)g.T * 4);
  if (g.shuffle)
    hipLaunchKernelGGL(q4_0_gemv_fast_kernel<true>, dim3(grid), dim3(g.T), lds, s, y, w, x, bias,
                       (int)n, g.P, g.rps);
  else
    hipLaunchKernelGGL(q4_0_gemv_fast_kernel<false>, dim3(grid), dim3(g.T), lds, s, y, w, x,
                       bias, (int)n, g.P, g.rps);
  return hipGetLastError();
}

}  // namespace hypno
