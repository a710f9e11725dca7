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
// Each lane owns one block column b (32 outputs, 32 fp32 accumulators) and a
// few rows k: per k it reads the block (k, b) — the 64 lanes of a wave read
// 64 consecutive 18-byte blocks, as 20-byte windows when w is dword-aligned —
// and adds (nib - 8) * (d * x[k]) to its 32 accumulators.  A work-group's
// waves interleave over a range of k and add their sums through LDS; each
// range writes a partial plane, and a second kernel adds the planes in a
// fixed order (+ bias).
#include "common.hpp"

namespace hypno {

namespace {

// Block (k, b) = block index g of w, valid when `valid` (k in range, b a
// block column) and g lies below avail_blocks.  Loads are unconditional — an
// invalid block reads block 0 and gets scale 0 — so the compiler can keep
// several in flight instead of waiting at a branch.  d[0] = scale bits,
// d[1..4] = the 16 nibble bytes.
template <bool kWindow>
__device__ __forceinline__ void col_block_load(const uint8_t* __restrict__ w, size_t g, bool valid,
                                               size_t avail_blocks, uint32_t (&d)[5]) {
  valid = valid && g < avail_blocks;
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
}

// acc[o] += (nib_o - 8) * (d * xk) for the block's 32 outputs (byte i of the
// nibbles holds outputs 2i (low nibble) and 2i + 1 (high)).  The nibbles
// become exact fp16 values nib - 8 two at a time (unpack8: dword j's outputs
// 8j + t and 8j + t + 4 share slot t), which the fp32 FMAs take as they are.
__device__ __forceinline__ void col_block_fma(const uint32_t (&d)[5], float xk,
                                              float (&acc)[kBlockElems], bool valid = true) {
  const float s = valid ? f16_bits_to_f32(d[0]) * xk : 0.0f;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const u32x4 r = unpack8(d[1 + j]);
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const uint32_t rt = r[t];  // (a bit_cast of the vector element itself reads element 0)
      const half2v h = __builtin_bit_cast(half2v, rt);
      acc[8 * j + t] = fmaf((float)h[0], s, acc[8 * j + t]);
      acc[8 * j + t + 4] = fmaf((float)h[1], s, acc[8 * j + t + 4]);
    }
  }
}

// KW waves of 64 block columns each, interleaved over k (wave v takes rows
// k0 + v, k0 + v + KW, ...), R rows per lane with all R loads in flight
// before any arithmetic, so a work-group covers KW * R rows and the whole
// matrix is in flight at about one work-group per CU.  With kWindow the
// loads are buffer loads of the 20-byte windows (32-bit offsets: the host
// takes this form only for w_len <= kColOob); an invalid block's offset lies
// past the range and reads zeros, and its scale term is 0.  Without it
// (w not dword-aligned, or larger than kColOob) the blocks are read byte by
// byte.  The KW partial sums of a block column meet in LDS (float4 slots,
// conflict-free) and are added in wave order.
constexpr uint32_t kColOob = 0xFFFFFFE0u;

template <int KW, int R, bool kWindow>
__global__ void __launch_bounds__(64 * KW)
q4_0_col_wide_kernel(float* __restrict__ part, const uint8_t* __restrict__ w, size_t avail_blocks,
                     uint32_t w_range, const float* __restrict__ x,
                     const float* __restrict__ bias, int nb, int m, int k_per, size_t part_tok) {
#if defined(__HIP_DEVICE_COMPILE__)  // (the buffer builtins exist only in the device pass)
  extern __shared__ __align__(16) float4 red4[];  // [KW][8][64]
  // token blockIdx.z: its x row and its planes (or its y row)
  x += (size_t)blockIdx.z * m;
  part += (size_t)blockIdx.z * part_tok;
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int b = blockIdx.x * 64 + lane;
  const int k0 = blockIdx.y * k_per;
  const int k1 = min(m, k0 + k_per);
  const bool active = b < nb;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(w), (short)0, (int)w_range, 0x00020000);
  float acc[kBlockElems];
#pragma unroll
  for (int i = 0; i < kBlockElems; i++) acc[i] = 0.0f;
  for (int kb = k0 + wv; kb < k1; kb += KW * R) {
    uint32_t d[R][5];
    float xk[R];
    bool val[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
      const int k = kb + r * KW;
      const size_t g = (size_t)k * nb + b;
      val[r] = active && k < k1 && g < avail_blocks;
      xk[r] = load_global<float>(x + (k < k1 ? k : k0));
      if constexpr (kWindow) {
        const uint32_t byte = (uint32_t)(g * kBlockBytes);
        const uint32_t off = val[r] ? (byte & ~3u) : kColOob;
        const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
        d[r][0] = a[0];
        d[r][1] = a[1];
        d[r][2] = a[2];
        d[r][3] = a[3];
        d[r][4] = __builtin_amdgcn_raw_buffer_load_b32(rs, off + 16, 0, 0);
      } else {
        col_block_load<false>(w, g, val[r], avail_blocks, d[r]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // every row's reads issued before the arithmetic
#pragma unroll
    for (int r = 0; r < R; r++) {
      uint32_t q[5];
      if constexpr (kWindow) {
        // block g starts at window byte 0 (g even) or 2 (g odd)
        const bool odd = (((uint32_t)(((size_t)(kb + r * KW) * nb + b) * kBlockBytes)) & 2u) != 0;
        const uint32_t sel = odd ? 0x07060504u : 0x05040302u;
        q[0] = odd ? d[r][0] >> 16 : d[r][0] & 0xFFFFu;
#pragma unroll
        for (int j = 0; j < 4; j++) q[1 + j] = __builtin_amdgcn_perm(d[r][j + 1], d[r][j], sel);
      } else {
#pragma unroll
        for (int j = 0; j < 5; j++) q[j] = d[r][j];
      }
      // an invalid block adds exactly nothing, whatever x[k] holds
      col_block_fma(q, val[r] ? xk[r] : 0.0f, acc, val[r]);
    }
  }
#pragma unroll
  for (int i = 0; i < kBlockElems / 4; i++)
    red4[(wv * 8 + i) * 64 + lane] =
        make_float4(acc[4 * i], acc[4 * i + 1], acc[4 * i + 2], acc[4 * i + 3]);
  __syncthreads();
  const int t = threadIdx.x;
  if (t >= 8 * 64) return;
  const int i = t >> 6, l = t & 63;
  float4 o[KW];  // every read issued before the adds
#pragma unroll
  for (int v = 0; v < KW; v++) o[v] = red4[(v * 8 + i) * 64 + l];
  float4 sum = o[0];
#pragma unroll
  for (int v = 1; v < KW; v++) {
    sum.x += o[v].x;
    sum.y += o[v].y;
    sum.z += o[v].z;
    sum.w += o[v].w;
  }
  const int bo = blockIdx.x * 64 + l;
  if (bo >= nb) return;
  if (gridDim.y == 1 && bias) {
    const float* bp = bias + (size_t)bo * kBlockElems + 4 * i;
    sum.x += bp[0];
    sum.y += bp[1];
    sum.z += bp[2];
    sum.w += bp[3];
  }
  float* out = part + (size_t)blockIdx.y * nb * kBlockElems + (size_t)bo * kBlockElems + 4 * i;
  if (((uintptr_t)part & 15) == 0) {
    *reinterpret_cast<float4*>(out) = sum;
  } else {
    out[0] = sum.x;
    out[1] = sum.y;
    out[2] = sum.z;
    out[3] = sum.w;
  }
#endif
}

// y[j] = sum of the planes (+ bias); j >= covered gets the bias only.  A
// work-group takes kRedOut outputs x kRedSlices plane slices (slice s adds
// planes s, s + kRedSlices, ... in order); the slice sums are then added in
// slice order through LDS, so the result is the same on every run.
constexpr int kRedOut = 32, kRedSlices = 8;

__global__ void __launch_bounds__(kRedOut * kRedSlices)
q4_0_col_reduce_kernel(float* __restrict__ y, const float* __restrict__ part,
                       const float* __restrict__ bias, size_t n, size_t covered, int planes,
                       size_t y_tok, size_t part_tok) {
  // token blockIdx.y: its y row and its planes
  y += (size_t)blockIdx.y * y_tok;
  if (part) part += (size_t)blockIdx.y * part_tok;
  __shared__ float red[kRedSlices][kRedOut];
  const int jo = threadIdx.x % kRedOut, sl = threadIdx.x / kRedOut;
  const size_t j = (size_t)blockIdx.x * kRedOut + jo;
  float s = 0.0f;
  if (j < covered) {
    int p = sl;
    for (; p + 7 * kRedSlices < planes; p += 8 * kRedSlices) {  // eight loads in flight
      float a[8];
#pragma unroll
      for (int u = 0; u < 8; u++) a[u] = part[(size_t)(p + u * kRedSlices) * covered + j];
#pragma unroll
      for (int u = 0; u < 8; u++) s += a[u];
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

// Geometry: KW waves x R rows per lane = k_per rows per work-group,
// the longest range of 64 (8 waves x 8 rows, 104 VGPRs, 64 KB of LDS: two
// work-groups per CU), 32 (16 waves x 2 rows, 128 KB of LDS) and 16 (8 x 2)
// that still gives every CU a work-group.  Longer ranges leave fewer partial
// planes (7.1 / k_per of the weight bytes).  Measured per call on the
// Mistral shapes (µs): 8 x 8 gate/up 15.6 and down 16.9 against 18.1 and
// 19.7 with 16 x 4 and 17.0 and 18.2 with 8 x 16 (162 VGPRs); q/o 9.3 with
// 16 x 2 against 9.9 with 8 x 4 and 11.0 with 8 x 2.

struct ColGeom {
  int gx, gy, k_per, kw, r;
};

static ColGeom col_geom(int nb, size_t m, int num_cus) {
  ColGeom g;
  g.gx = (nb + 63) / 64;
  static const int kForms[3][2] = {{8, 8}, {16, 2}, {8, 2}};  // (KW, R)
  int f = 0;
  while (f < 2 && (size_t)g.gx * ((m + kForms[f][0] * kForms[f][1] - 1) /
                                  (kForms[f][0] * kForms[f][1])) < (size_t)num_cus)
    f++;
  g.kw = kForms[f][0];
  g.r = kForms[f][1];
  const int rows = g.kw * g.r;
  // (grid y stays below 65536: longer ranges loop)
  const size_t steps = (m + rows - 1) / rows;
  g.k_per = rows * (int)((steps + 65534) / 65535);
  g.gy = (int)((m + g.k_per - 1) / g.k_per);
  return g;
}

size_t q4_0_col_workspace_bytes(size_t n, size_t m, int num_cus) {
  const int nb = (int)(n / kBlockElems);
  if (nb == 0 || m == 0) return 0;
  const ColGeom g = col_geom(nb, m, num_cus);
  return g.gy > 1 ? (size_t)g.gy * nb * kBlockElems * sizeof(float) : 0;
}

template <int KW, int R, bool kWindow>
static hipError_t launch_col_wide(const ColGeom& g, float* part, const uint8_t* w, size_t avail,
                                  uint32_t w_range, const float* x, const float* bias, int nb,
                                  int m, int tokens, size_t part_tok, hipStream_t s) {
  constexpr int lds = KW * 8 * 64 * (int)sizeof(float4);
  const void* k = reinterpret_cast<const void*>(q4_0_col_wide_kernel<KW, R, kWindow>);
  hipError_t e = set_lds_limit(k, lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((q4_0_col_wide_kernel<KW, R, kWindow>), dim3(g.gx, g.gy, tokens),
                     dim3(64 * KW), lds, s, part, w, avail, w_range, x, bias, nb, m, g.k_per,
                     part_tok);
  return hipGetLastError();
}

template <bool kWindow>
static hipError_t launch_col_main(const ColGeom& g, float* part, const uint8_t* w, size_t avail,
                                  uint32_t w_range, const float* x, const float* bias, int nb,
                                  int m, int tokens, size_t part_tok, hipStream_t s) {
  if (g.r == 8)
    return launch_col_wide<8, 8, kWindow>(g, part, w, avail, w_range, x, bias, nb, m, tokens,
                                          part_tok, s);
  if (g.kw == 16)
    return launch_col_wide<16, 2, kWindow>(g, part, w, avail, w_range, x, bias, nb, m, tokens,
                                           part_tok, s);
  return launch_col_wide<8, 2, kWindow>(g, part, w, avail, w_range, x, bias, nb, m, tokens,
                                        part_tok, s);
}

hipError_t launch_q4_0_col(float* y, const uint8_t* w, size_t w_len, const float* x,
                           const float* bias, size_t n, size_t m, int tokens, void* ws,
                           int num_cus, hipStream_t s) {
  const int nb = (int)(n / kBlockElems);
  const size_t covered = (size_t)nb * kBlockElems;
  const size_t avail = w_len / kBlockBytes;
  const unsigned red_n = (unsigned)((n + kRedOut - 1) / kRedOut);
  if (nb > 0 && m > 0 && avail > 0) {
    const ColGeom g = col_geom(nb, m, num_cus);
    float* part = g.gy > 1 ? static_cast<float*>(ws) : y;
    // a token's planes in the workspace, or its y row when y is written directly
    const size_t part_tok = g.gy > 1 ? (size_t)g.gy * covered : n;
    // Windows need a dword-aligned w, 2 readable bytes after the last valid
    // block when its index is even, and 32-bit offsets.
    const bool window = ((uintptr_t)w & 3) == 0 && w_len <= kColOob &&
                        (avail % 2 == 0 || w_len >= avail * kBlockBytes + 2);
    const uint32_t range = (uint32_t)(w_len < kColOob ? w_len : kColOob);
    hipError_t e = window ? launch_col_main<true>(g, part, w, avail, range, x, bias, nb, (int)m,
                                                  tokens, part_tok, s)
                          : launch_col_main<false>(g, part, w, avail, range, x, bias, nb, (int)m,
                                                   tokens, part_tok, s);
    if (e != hipSuccess) return e;
    if (g.gy == 1) {
      if (covered == n) return hipSuccess;  // y written, bias included
      // y[0, covered) holds the sums (+ bias); the tail gets the bias.
      const size_t tail = n - covered;
      hipLaunchKernelGGL(q4_0_col_reduce_kernel,
                         dim3((unsigned)((tail + kRedOut - 1) / kRedOut), (unsigned)tokens),
                         dim3(kRedOut * kRedSlices), 0, s, y + covered, nullptr,
                         bias ? bias + covered : nullptr, tail, (size_t)0, 0, n, (size_t)0);
      return hipGetLastError();
    }
    hipLaunchKernelGGL(q4_0_col_reduce_kernel, dim3(red_n, (unsigned)tokens),
                       dim3(kRedOut * kRedSlices), 0, s, y, part, bias, n, covered, g.gy, n,
                       part_tok);
    return hipGetLastError();
  }
  // No whole block, no input or no weight block: y = bias (or 0).
  hipLaunchKernelGGL(q4_0_col_reduce_kernel, dim3(red_n, (unsigned)tokens),
                     dim3(kRedOut * kRedSlices), 0, s, y, nullptr, bias, n, (size_t)0, 0, n,
                     (size_t)0);
  return hipGetLastError();
}

}  // namespace hypno
