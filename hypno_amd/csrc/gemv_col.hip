// Column-major Q4_0 matrix-vector product (kernels.rs:403-535, chosen when a
// model's metadata says weight_layout = col_major, loader.rs:166-168).
//
// Layout: W_col[k][j] for input index k < m and output j < n: each k owns a
// "column" of n outputs stored contiguously and quantised in Q4_0 blocks
// along j (nb = n / 32 blocks, floor: outputs past 32 * nb get only the
// bias, as in matmul_q4_0_col_scalar).  y[j] = sum_k W_col[k][j] * x[k] (+ bias).
// A block past the end of a short buffer contributes nothing
// (kernels.rs:522).  The reference's AVX2 form sums per-thread partial
// buffers, so its bits depend on the thread count; this one is fixed-order
// (deterministic) and checked against fp64.
//
// Each thread owns one block column b (32 outputs, 32 fp32 accumulators) and
// walks k: per k it reads the block (k, b) — consecutive threads read
// consecutive 18-byte blocks, as a 20-byte window when w is dword-aligned —
// and adds (nib - 8) * (d * x[k]) to its 32 accumulators.  Work-groups split
// k into ranges (and their waves interleave k within a range); each writes a
// partial plane, and a second kernel adds the planes in a fixed order
// (+ bias).
#include "common.hpp"

namespace hypno {

namespace {

constexpr int kColThreads = 256;

// Partial sums of the work-group's block columns over its k range.  The
// work-group's 256 threads are CW = 64, 128 or 256 column lanes times
// KW = 256 / CW interleaved k lanes (thread t: column t % CW, k lane t / CW);
// the KW partial sums of a column are added through LDS in k-lane order.
// `part` is [gridDim.y][nb * 32]; with one range it is y itself and the bias
// is added here.
template <bool kWindow>
__global__ void __launch_bounds__(kColThreads)
q4_0_col_kernel(float* __restrict__ part, const uint8_t* __restrict__ w, size_t avail_blocks,
                const float* __restrict__ x, const float* __restrict__ bias, int nb, int m,
                int k_per, int cw) {
  __shared__ __align__(16) float red[kColThreads * kBlockElems];
  const int kw = kColThreads / cw;
  const int cl = threadIdx.x % cw, kl = threadIdx.x / cw;
  const int b = blockIdx.x * cw + cl;
  const int k0 = blockIdx.y * k_per;
  const int k1 = min(m, k0 + k_per);
  const bool active = b < nb;
  float acc[kBlockElems];
#pragma unroll
  for (int i = 0; i < kBlockElems; i++) acc[i] = 0.0f;
  // Block (k, b) is valid when its index k * nb + b lies below avail_blocks
  // (and k lies in the range).  Loads are unconditional — an invalid block
  // reads block 0 and gets scale 0 — so the compiler can keep kDepth of them
  // in flight instead of waiting at a branch.
  constexpr int kDepth = 8;
  auto load = [&](int k, uint32_t* d) {
    const size_t g = (size_t)k * nb + b;
    const bool valid = active && k < k1 && g < avail_blocks;
    const uint8_t* blk = w + (valid ? g : 0) * kBlockBytes;
    if constexpr (kWindow) {
      // 20-byte window from the dword below the block (w is dword-aligned, so
      // block g starts at window byte 0 (g even) or 2 (g odd); an even
      // block's window reads 2 bytes of the next block, and the host takes
      // this path only when those bytes exist for the last valid block).
      const uint8_t* p = reinterpret_cast<const uint8_t*>((uintptr_t)blk & ~(uintptr_t)3);
      const u32x4 a = load_global<u32x4>(p);
      const uint32_t e = load_global<uint32_t>(p + 16);
      const bool odd = ((uintptr_t)blk & 2) != 0;
      const uint32_t v[5] = {a.x, a.y, a.z, a.w, e};
      const uint32_t sel = odd ? 0x07060504u : 0x05040302u;
      d[0] = odd ? v[0] >> 16 : v[0] & 0xFFFFu;
#pragma unroll
      for (int j = 0; j < 4; j++) d[1 + j] = __builtin_amdgcn_perm(v[j + 1], v[j], sel);
    } else {
      d[0] = (uint32_t)blk[0] | ((uint32_t)blk[1] << 8);
#pragma unroll
      for (int j = 0; j < 4; j++)
        d[1 + j] = (uint32_t)blk[2 + 4 * j] | ((uint32_t)blk[3 + 4 * j] << 8) |
                   ((uint32_t)blk[4 + 4 * j] << 16) | ((uint32_t)blk[5 + 4 * j] << 24);
    }
    if (!valid) d[0] = 0;  // scale 0: contributes nothing
  };
  for (int kb = k0 + kl; kb < k1; kb += kw * kDepth) {  // kl is wave-uniform
    uint32_t d[kDepth][5];
    float xk[kDepth];
#pragma unroll
    for (int r = 0; r < kDepth; r++) {
      const int k = kb + r * kw;
      load(k, d[r]);
      xk[r] = load_global<float>(x + (k < k1 ? k : k0));
    }
#pragma unroll
    for (int r = 0; r < kDepth; r++) {
      const float s = f16_bits_to_f32(d[r][0]) * xk[r];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint32_t q = d[r][1 + j];
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const uint32_t byte = (q >> (8 * i)) & 0xFFu;
          acc[8 * j + 2 * i] = fmaf((float)((int)(byte & 15u) - 8), s, acc[8 * j + 2 * i]);
          acc[8 * j + 2 * i + 1] =
              fmaf((float)((int)(byte >> 4) - 8), s, acc[8 * j + 2 * i + 1]);
        }
      }
    }
  }
  if (kw > 1) {
    float4* r4 = reinterpret_cast<float4*>(red + (size_t)threadIdx.x * kBlockElems);
#pragma unroll
    for (int i = 0; i < kBlockElems / 4; i++)
      r4[i] = make_float4(acc[4 * i], acc[4 * i + 1], acc[4 * i + 2], acc[4 * i + 3]);
    __syncthreads();
    if (kl != 0) return;
    for (int l = 1; l < kw; l++) {
      const float* o = red + (size_t)(l * cw + cl) * kBlockElems;
#pragma unroll
      for (int i = 0; i < kBlockElems; i++) acc[i] += o[i];
    }
  }
  if (!active) return;
  float* out = part + (size_t)blockIdx.y * nb * kBlockElems + (size_t)b * kBlockElems;
  if (gridDim.y == 1 && bias) {
#pragma unroll
    for (int i = 0; i < kBlockElems; i++) acc[i] += bias[b * kBlockElems + i];
  }
  if (((uintptr_t)part & 15) == 0) {  // uniform: b * 32 floats keeps the alignment
    float4* o4 = reinterpret_cast<float4*>(out);
#pragma unroll
    for (int i = 0; i < kBlockElems / 4; i++)
      o4[i] = make_float4(acc[4 * i], acc[4 * i + 1], acc[4 * i + 2], acc[4 * i + 3]);
  } else {
#pragma unroll
    for (int i = 0; i < kBlockElems; i++) out[i] = acc[i];
  }
}

// y[j] = sum of the planes (+ bias); j >= covered gets the bias only.  A
// work-group takes 32 outputs x 8 plane slices (slice s adds planes s, s + 8,
// ... in order); the 8 slice sums are then added in slice order through LDS,
// so the result is the same on every run.
constexpr int kRedOut = 32, kRedSlices = 8;

__global__ void __launch_bounds__(kRedOut * kRedSlices)
q4_0_col_reduce_kernel(float* __restrict__ y, const float* __restrict__ part,
                       const float* __restrict__ bias, size_t n, size_t covered, int planes) {
  __shared__ float red[kRedSlices][kRedOut];
  const int jo = threadIdx.x % kRedOut, sl = threadIdx.x / kRedOut;
  const size_t j = (size_t)blockIdx.x * kRedOut + jo;
  float s = 0.0f;
  if (j < covered) {
    int p = sl;
    for (; p + 3 * kRedSlices < planes; p += 4 * kRedSlices) {  // four loads in flight
      const float a0 = part[(size_t)p * covered + j];
      const float a1 = part[(size_t)(p + kRedSlices) * covered + j];
      const float a2 = part[(size_t)(p + 2 * kRedSlices) * covered + j];
      const float a3 = part[(size_t)(p + 3 * kRedSlices) * covered + j];
      s = (((s + a0) + a1) + a2) + a3;
    }
    for (; p < planes; p += kRedSlices) s += part[(size_t)p * covered + j];
  }
  red[sl][jo] = s;
  __syncthreads();
  if (sl != 0 || j >= n) return;
  float t = 0.0f;
#pragma unroll
  for (int q = 0; q < kRedSlices; q++) t += red[q][jo];
  y[j] = t + (bias ? bias[j] : 0.0f);
}

}  // namespace

// Column lanes per work-group: the block columns rounded up to a wave, at
// most the whole work-group.
static int col_lanes(int nb) {
  const int r = (nb + 63) / 64 * 64;
  return r < kColThreads ? (r == 192 ? kColThreads : r) : kColThreads;
}

// k ranges (partial planes): about two work-groups per CU, but at least 28 k
// per range, so the planes (ranges x n x 4 bytes) stay within about a
// quarter of the weight bytes (k x n x 0.5625).
static int col_ranges(int nb, size_t m, int num_cus) {
  const int gx = (nb + col_lanes(nb) - 1) / col_lanes(nb);
  long long r = (2LL * num_cus + gx - 1) / gx;
  const long long cap = (long long)(m / 28);
  if (r > cap) r = cap;
  return r < 1 ? 1 : (int)r;
}

size_t q4_0_col_workspace_bytes(size_t n, size_t m, int num_cus) {
  const int nb = (int)(n / kBlockElems);
  if (nb == 0 || m == 0) return 0;
  const int r = col_ranges(nb, m, num_cus);
  return r > 1 ? (size_t)r * nb * kBlockElems * sizeof(float) : 0;
}

hipError_t launch_q4_0_col(float* y, const uint8_t* w, size_t w_len, const float* x,
                           const float* bias, size_t n, size_t m, void* ws, int num_cus,
                           hipStream_t s) {
  const int nb = (int)(n / kBlockElems);
  const size_t covered = (size_t)nb * kBlockElems;
  const size_t avail = w_len / kBlockBytes;
  if (nb > 0 && m > 0 && avail > 0) {
    const int cw = col_lanes(nb);
    const int gx = (nb + cw - 1) / cw;
    const int ranges = col_ranges(nb, m, num_cus);
    const int k_per = (int)((m + ranges - 1) / ranges);
    const int gy = (int)((m + k_per - 1) / k_per);
    float* part = gy > 1 ? static_cast<float*>(ws) : y;
    // Windows need a dword-aligned w, and 2 readable bytes after the last
    // valid block when its index is even.
    const bool window =
        ((uintptr_t)w & 3) == 0 && (avail % 2 == 0 || w_len >= avail * kBlockBytes + 2);
    if (window)
      hipLaunchKernelGGL(q4_0_col_kernel<true>, dim3(gx, gy), dim3(kColThreads), 0, s, part, w,
                         avail, x, bias, nb, (int)m, k_per, cw);
    else
      hipLaunchKernelGGL(q4_0_col_kernel<false>, dim3(gx, gy), dim3(kColThreads), 0, s, part, w,
                         avail, x, bias, nb, (int)m, k_per, cw);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (gy == 1) {
      if (covered == n) return hipSuccess;  // y written, bias included
      // y[0, covered) holds the sums (+ bias); the tail gets the bias.
      const size_t tail = n - covered;
      hipLaunchKernelGGL(q4_0_col_reduce_kernel, dim3((unsigned)((tail + kRedOut - 1) / kRedOut)),
                         dim3(kRedOut * kRedSlices), 0, s, y + covered, nullptr,
                         bias ? bias + covered : nullptr, tail, (size_t)0, 0);
      return hipGetLastError();
    }
    hipLaunchKernelGGL(q4_0_col_reduce_kernel, dim3((unsigned)((n + kRedOut - 1) / kRedOut)),
                       dim3(kRedOut * kRedSlices), 0, s, y, part, bias, n, covered, gy);
    return hipGetLastError();
  }
  // No whole block, no input or no weight block: y = bias (or 0).
  hipLaunchKernelGGL(q4_0_col_reduce_kernel, dim3((unsigned)((n + kRedOut - 1) / kRedOut)),
                     dim3(kRedOut * kRedSlices), 0, s, y, nullptr, bias, n, (size_t)0, 0);
  return hipGetLastError();
}

}  // namespace hypno
