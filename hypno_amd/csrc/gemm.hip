// Batched-prefill GEMM on CDNA4 MFMA: Y[M][N] = X[M][K] . W[N][K]^T (+ bias).
//
// X (fp32) is first rounded to fp16 into a workspace padded to a multiple of
// the 128-row tile.  For Q4_0 weights each 8-column group of X is stored in
// the order [0,4,1,5,2,6,3,7], which is the order in which one packed nibble
// dword unpacks into fp16 pairs (see unpack_nib8); both MFMA operands then
// list the same columns in the same slots.
//
// Q4_0 path: per 64-column K step the work-group stages X (fp16) and the
// packed weight bytes in LDS, expands every weight row's two blocks into
// exact fp16 integers (nibble - 8) plus one fp32 scale per (row, block), and
// each wave runs v_mfma_f32_16x16x32_f16 once per 32-column block (K = 32 is
// exactly one Q4_0 block) with a zero accumulator; the block partial is then
// scaled by the fp32 block scale into the fp32 accumulators.
//
// FP16 path: the same tiling with the fp16 weights copied to LDS as-is and
// the MFMA accumulating directly across K (there is no per-block scale).
#include "common.hpp"

namespace hypno {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 128;    // rows of X per work-group
constexpr int kBN = 128;    // rows of W per work-group
constexpr int kBK = 64;     // K per step (two Q4_0 blocks)
constexpr int kLdsRow = 72; // halves per LDS row: 64 + 8 padding (144 B)

static size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

size_t gemm_workspace_bytes(size_t batch, size_t m) { return round_up(batch, kBM) * m * 2; }

bool q4_0_gemm_ok(const uint8_t* w, size_t w_len, size_t n, size_t m, size_t batch) {
  if (m == 0 || m % kBK != 0 || n == 0 || batch == 0) return false;
  if (((uintptr_t)w & 3) != 0) return false;
  if (n > (size_t)0x7FFFFFFF || m > (size_t)0x7FFFFFFF || batch > (size_t)0x7FFFFFFF) return false;
  return w_len / kBlockBytes >= n * (m / kBlockElems);
}

bool f16_gemm_ok(const uint8_t* w, size_t n, size_t m, size_t batch) {
  if (m == 0 || m % kBK != 0 || n == 0 || batch == 0) return false;
  if (((uintptr_t)w & 15) != 0) return false;
  return n <= (size_t)0x7FFFFFFF && m <= (size_t)0x7FFFFFFF && batch <= (size_t)0x7FFFFFFF;
}

// X fp32 [M][K] -> Xh fp16 [Mp][K], zero rows M..Mp-1.  One thread per
// 8-column group; kPermute applies the nibble-unpack column order.
template <bool kPermute>
__global__ void __launch_bounds__(256)
x_to_f16_kernel(uint4* __restrict__ xh, const float* __restrict__ x, int M, int Mp, int K) {
  const size_t groups = (size_t)K / 8;
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (size_t)Mp * groups) return;
  const size_t row = idx / groups;
  const size_t g = idx - row * groups;
  float v[8];
  if (row < (size_t)M) {
    const float* src = x + row * K + g * 8;
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = src[i];
  } else {
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = 0.0f;
  }
  constexpr int perm_q4[8] = {0, 4, 1, 5, 2, 6, 3, 7};
  uint32_t packed[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int a = kPermute ? perm_q4[2 * j] : 2 * j;
    const int b = kPermute ? perm_q4[2 * j + 1] : 2 * j + 1;
    const uint32_t lo = __builtin_bit_cast(uint16_t, (_Float16)v[a]);
    const uint32_t hi = __builtin_bit_cast(uint16_t, (_Float16)v[b]);
    packed[j] = lo | (hi << 16);
  }
  xh[idx] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
}

// One packed nibble dword (elements e0..e7, byte i = e[2i] | e[2i+1] << 4)
// -> 8 exact fp16 values (e - 8) in slot order e0,e4,e1,e5,e2,e6,e3,e7.
// (0x6400 | n) is the fp16 value 1024 + n; subtracting 1032 is exact.
__device__ __forceinline__ uint4 unpack_nib8(uint32_t dw) {
  typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
  const half2_t off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
  uint32_t r[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint32_t bits = ((dw >> (4 * j)) & 0x000F000Fu) | 0x64006400u;
    half2_t h = __builtin_bit_cast(half2_t, bits);
    h = h + off;
    r[j] = __builtin_bit_cast(uint32_t, h);
  }
  return make_uint4(r[0], r[1], r[2], r[3]);
}

template <bool kQ4>
__global__ void __launch_bounds__(256, 2)
gemm_kernel(float* __restrict__ y, const uint8_t* __restrict__ w, const uint4* __restrict__ xh,
            const float* __restrict__ bias, int M, int N, int K) {
  __shared__ __align__(16) _Float16 As[kBM * kLdsRow];
  __shared__ __align__(16) _Float16 Bs[kBN * kLdsRow];
  __shared__ __align__(16) uint32_t Bq[kBN * 9];  // raw Q4_0 bytes: 2 blocks per row
  __shared__ float Sc[2][kBN];                     // fp32 block scales

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;  // 2x2 waves, 64x64 each
  const int m0 = blockIdx.y * kBM;
  const int n0 = blockIdx.x * kBN;
  const size_t row_bytes = kQ4 ? (size_t)K / 32 * 18 : (size_t)K * 2;
  const int kgroups = K / 8;  // uint4 per X row

  floatx4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  const int frag_row = lane & 15;
  const int frag_k = (lane >> 4) * 8;

  for (int k0 = 0; k0 < K; k0 += kBK) {
    // --- stage X: 128 rows x 64 halves = 1024 uint4, 4 per thread
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int c = t + 256 * i;
      const int row = c >> 3, col = c & 7;
      const uint4 v = xh[(size_t)(m0 + row) * kgroups + k0 / 8 + col];
      *reinterpret_cast<uint4*>(&As[row * kLdsRow + col * 8]) = v;
    }
    if (kQ4) {
      // --- stage packed W: 128 rows x 36 bytes = 1152 dwords
      const size_t kb_off = (size_t)(k0 / 32) * 18;
#pragma unroll
      for (int i = 0; i < 5; i++) {
        const int c = t + 256 * i;
        if (c < kBN * 9) {
          const int row = c / 9, j = c - row * 9;
          uint32_t v = 0;
          if (n0 + row < N)
            v = *reinterpret_cast<const uint32_t*>(w + (size_t)(n0 + row) * row_bytes + kb_off +
                                                   4 * j);
          Bq[c] = v;
        }
      }
      __syncthreads();
      // --- expand: thread -> (row n, block kb)
      {
        const int n = t & 127, kb = t >> 7;
        const uint32_t* q = Bq + n * 9;
        float sc;
        uint32_t dw[4];
        if (kb == 0) {
          sc = f16_bits_to_f32(q[0] & 0xFFFFu);
#pragma unroll
          for (int j = 0; j < 4; j++) dw[j] = __builtin_amdgcn_alignbit(q[j + 1], q[j], 16);
        } else {
          sc = f16_bits_to_f32(q[4] >> 16);
#pragma unroll
          for (int j = 0; j < 4; j++) dw[j] = q[5 + j];
        }
        Sc[kb][n] = sc;
#pragma unroll
        for (int j = 0; j < 4; j++)
          *reinterpret_cast<uint4*>(&Bs[n * kLdsRow + kb * 32 + j * 8]) = unpack_nib8(dw[j]);
      }
    } else {
      // --- stage fp16 W: 128 rows x 64 halves = 1024 uint4
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int c = t + 256 * i;
        const int row = c >> 3, col = c & 7;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (n0 + row < N)
          v = *reinterpret_cast<const uint4*>(w + (size_t)(n0 + row) * row_bytes +
                                              (size_t)(k0 + col * 8) * 2);
        *reinterpret_cast<uint4*>(&Bs[row * kLdsRow + col * 8]) = v;
      }
    }
    __syncthreads();

    // --- MFMA: one 16x16x32 per (16-row X tile, 16-row W tile, 32-col block)
#pragma unroll
    for (int kb = 0; kb < 2; kb++) {
      half8 a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; i++)
        a[i] = *reinterpret_cast<const half8*>(
            &As[(wm * 64 + i * 16 + frag_row) * kLdsRow + kb * 32 + frag_k]);
#pragma unroll
      for (int j = 0; j < 4; j++)
        b[j] = *reinterpret_cast<const half8*>(
            &Bs[(wn * 64 + j * 16 + frag_row) * kLdsRow + kb * 32 + frag_k]);
      if (kQ4) {
        float sc[4];
#pragma unroll
        for (int j = 0; j < 4; j++) sc[j] = Sc[kb][wn * 64 + j * 16 + frag_row];
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
          for (int j = 0; j < 4; j++) {
            const floatx4 part = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                a[i], b[j], floatx4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; r++) acc[i][j][r] = fmaf(sc[j], part[r], acc[i][j][r]);
          }
      } else {
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
          for (int j = 0; j < 4; j++)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j], 0, 0, 0);
      }
    }
    __syncthreads();
  }

  // --- epilogue: lane holds D[4*(lane/16)+r][lane%16] of each 16x16 tile
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int n = n0 + wn * 64 + j * 16 + (lane & 15);
    if (n >= N) continue;
    const float bv = bias ? bias[n] : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int mrow = m0 + wm * 64 + i * 16 + (lane >> 4) * 4 + r;
        if (mrow < M) y[(size_t)mrow * N + n] = acc[i][j][r] + bv;
      }
  }
}

static hipError_t launch_x_prepass(const float* x, size_t batch, size_t m, void* ws, bool permute,
                                   hipStream_t s) {
  const size_t mp = round_up(batch, kBM);
  const size_t work = mp * (m / 8);
  const size_t grid = (work + 255) / 256;
  if (permute)
    hipLaunchKernelGGL(x_to_f16_kernel<true>, dim3((unsigned)grid), dim3(256), 0, s,
                       (uint4*)ws, x, (int)batch, (int)mp, (int)m);
  else
    hipLaunchKernelGGL(x_to_f16_kernel<false>, dim3((unsigned)grid), dim3(256), 0, s,
                       (uint4*)ws, x, (int)batch, (int)mp, (int)m);
  return hipGetLastError();
}

hipError_t launch_q4_0_gemm(float* y, const uint8_t* w, const float* x, const float* bias,
                            size_t n, size_t m, size_t batch, void* ws, hipStream_t s) {
  hipError_t e = launch_x_prepass(x, batch, m, ws, true, s);
  if (e != hipSuccess) return e;
  const dim3 grid((unsigned)((n + kBN - 1) / kBN), (unsigned)(round_up(batch, kBM) / kBM));
  hipLaunchKernelGGL(gemm_kernel<true>, grid, dim3(256), 0, s, y, w, (const uint4*)ws, bias,
                     (int)batch, (int)n, (int)m);
  return hipGetLastError();
}

hipError_t launch_f16_gemm(float* y, const uint8_t* w, const float* x, const float* bias,
                           size_t n, size_t m, size_t batch, void* ws, hipStream_t s) {
  hipError_t e = launch_x_prepass(x, batch, m, ws, false, s);
  if (e != hipSuccess) return e;
  const dim3 grid((unsigned)((n + kBN - 1) / kBN), (unsigned)(round_up(batch, kBM) / kBM));
  hipLaunchKernelGGL(gemm_kernel<false>, grid, dim3(256), 0, s, y, w, (const uint4*)ws, bias,
                     (int)batch, (int)n, (int)m);
  return hipGetLastError();
}

}  // namespace hypno
