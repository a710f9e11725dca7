// Q4_0 prefill GEMM for shapes the main kernel (gemm_q4.hip) does not take
// (K % 64 == 0 but K % 256 != 0, 4-byte-aligned weights), and the fp16
// activation pre-passes shared with gemm_q4.hip:
// Y[M][N] = X[M][K] . W[N][K]^T (+ bias).
//
// Pre-pass: X (fp32) is rounded to fp16 into a workspace padded to a multiple
// of the 128-row tile, each row scaled by a power of two (undone in the
// epilogue) so that no token's magnitude takes it out of fp16's normal range.  For
// Q4_0 weights each 8-column group is stored in the order [0,4,1,5,2,6,3,7],
// the order in which one packed nibble dword unpacks into fp16 pairs (see
// unpack_nib8), so both MFMA operands list the same columns in the same
// slots.  When the GEMM splits K in two, the pre-pass also zeroes Y.
//
// Main kernel: a 256-thread work-group computes a 128 x 128 tile of Y with
// 2 x 2 waves of 64 x 64.  K advances in steps of 64 (two Q4_0 blocks)
// through two LDS buffers: while the waves compute step s from one buffer,
// the global loads of step s+1 are already in flight into registers, and are
// then written to the other buffer (one barrier per step).
//   Each thread takes one (row, block) of the step's 128 x 2 weight
//   blocks, loads its 20-byte window (the 64 threads of a wave read
//   contiguous memory), expands the 32 nibbles to exact fp16 integers
//   (nibble - 8) into LDS, and stores the fp32 scale.  Every 32-column block
//   is one v_mfma_f32_16x16x32_f16 with a zero accumulator per 16 x 16 tile;
//   the partial is multiplied by the block's fp32 scale into fp32
//   accumulators.
// Split-K: when the tile grid has fewer than two work-groups per CU, K is
// split in two and the halves are added into the zeroed Y with atomics (two
// addends onto zero: the sum is the same in either order).
#include "common.hpp"

namespace hypno {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 128;     // rows of X per work-group
constexpr int kBN = 128;     // rows of W per work-group
constexpr int kBK = 64;      // K per step (two Q4_0 blocks)
constexpr int kLdsRow = 72;  // halves per LDS row: 64 + 8 padding (144 bytes)
constexpr int kTileHalves = kBM * kLdsRow;

static size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

size_t gemm_workspace_bytes(size_t batch, size_t m) {
  const size_t mp = round_up(batch, kBM);
  return round_up(mp * m * 2, 256) + mp * 4;
}

int* gemm_x_exponents(void* ws, size_t batch, size_t m) {
  return reinterpret_cast<int*>(static_cast<uint8_t*>(ws) +
                                round_up(round_up(batch, kBM) * m * 2, 256));
}

bool q4_0_gemm_ok(const uint8_t* w, size_t w_len, size_t n, size_t m, size_t batch) {
  if (m == 0 || m % kBK != 0 || n == 0 || batch == 0) return false;
  if (((uintptr_t)w & 3) != 0) return false;
  if (n > (size_t)0x7FFFFFFF || m > (size_t)0x7FFFFFFF || batch > (size_t)0x7FFFFFFF) return false;
  return w_len / kBlockBytes >= n * (m / kBlockElems);
}

// X fp32 [M][K] -> Xh fp16 [Mp][K] with per-row exponents (x_row_to_f16),
// one work-group per row; optionally zero Y (grid-stride over all of them).
template <bool kPermute>
__global__ void __launch_bounds__(256)
x_rows_to_f16_kernel(u32x4* __restrict__ xh, int* __restrict__ xexp, const float* __restrict__ x,
                     int M, int K, float* __restrict__ y_zero, size_t y_elems) {
  if (y_zero) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < y_elems; i += stride)
      y_zero[i] = 0.0f;
  }
  x_row_to_f16<kPermute>(xh, xexp, x, M, K, (int)blockIdx.x);
}

// One packed nibble dword (elements e0..e7, byte i = e[2i] | e[2i+1] << 4)
// -> 8 exact fp16 values (e - 8) in slot order e0,e4,e1,e5,e2,e6,e3,e7.
// (0x6400 | n) is the fp16 value 1024 + n; subtracting 1032 is exact.
__device__ __forceinline__ u32x4 unpack_nib8(uint32_t dw) {
  typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
  const half2_t off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
  u32x4 r;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint32_t bits = ((dw >> (4 * j)) & 0x000F000Fu) | 0x64006400u;
    half2_t h = __builtin_bit_cast(half2_t, bits);
    h = h + off;
    r[j] = __builtin_bit_cast(uint32_t, h);
  }
  return r;
}

// Global loads of one K step held in registers until they are written to LDS.
struct StepRegs {
  u32x4 a[4];  // X: 4 x 16 bytes
  u32x4 b;  // W: this thread's 20-byte window (16 + 4 bytes)
  uint32_t bw;
};

__global__ void __launch_bounds__(256, 2)
gemm_kernel(float* __restrict__ y, const uint8_t* __restrict__ w, const u32x4* __restrict__ xh,
            const int* __restrict__ xexp, const float* __restrict__ bias, int M, int N, int K,
            int ksplit) {
  extern __shared__ __align__(16) uint8_t smem[];
  // LDS: 2 x {A tile, B tile} fp16 + 2 x scales [2 blocks][128]
  _Float16* As0 = reinterpret_cast<_Float16*>(smem);
  const size_t buf_bytes = (size_t)2 * kTileHalves * 2 + 2 * kBN * 4;

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * kBM;
  const int n0 = blockIdx.x * kBN;
  const int kz = blockIdx.z;
  const int k_len = K / ksplit;
  const int k_begin = kz * k_len;
  const int steps = k_len / kBK;
  const size_t row_bytes = (size_t)K / 32 * 18;
  const int kgroups = K / 8;

  // Q4_0 staging role: (row, block) of the step's 128 x 2 blocks
  const int qrow = t & 127, qkb = t >> 7;
  const bool qvalid = n0 + qrow < N;
  const uint8_t* qrow_ptr = w + (size_t)(qvalid ? n0 + qrow : 0) * row_bytes;
  const bool qodd = (qkb & 1) != 0;  // odd block: starts 2 bytes into its window
  const uint32_t sel_q = qodd ? 0x07060504u : 0x05040302u;
  const uint32_t sh_d = qodd ? 16u : 0u;

  auto load_step = [&](int s, StepRegs& r) {
    const int k0 = k_begin + s * kBK;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int c = t + 256 * i;
      const int row = c >> 3, col = c & 7;
      r.a[i] = load_global<u32x4>(xh + (size_t)(m0 + row) * kgroups + k0 / 8 + col);
    }
    const size_t boff = (size_t)(k0 / 32 + qkb) * 18;
    const uint8_t* p = qrow_ptr + (boff & ~(size_t)3);
    r.b = load_global<u32x4>(p);
    r.bw = load_global<uint32_t>(p + 16);
  };

  auto store_step = [&](int buf, const StepRegs& r) {
    _Float16* As = As0 + (size_t)buf * (buf_bytes / 2);
    _Float16* Bs = As + kTileHalves;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int c = t + 256 * i;
      const int row = c >> 3, col = c & 7;
      *reinterpret_cast<u32x4*>(&As[row * kLdsRow + col * 8]) = r.a[i];
    }
    float* Sc = reinterpret_cast<float*>(Bs + kTileHalves);
    const uint32_t d[5] = {r.b.x, r.b.y, r.b.z, r.b.w, r.bw};
    Sc[qkb * kBN + qrow] = qvalid ? f16_bits_to_f32(d[0] >> sh_d) : 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t q = __builtin_amdgcn_perm(d[j + 1], d[j], sel_q);
      *reinterpret_cast<u32x4*>(&Bs[qrow * kLdsRow + qkb * 32 + j * 8]) = unpack_nib8(q);
    }
  };

  floatx4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  const int frag_row = lane & 15;
  const int frag_k = (lane >> 4) * 8;

  auto compute_step = [&](int buf) {
    const _Float16* As = As0 + (size_t)buf * (buf_bytes / 2);
    const _Float16* Bs = As + kTileHalves;
    const float* Sc = reinterpret_cast<const float*>(Bs + kTileHalves);
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
      float sc[4];
#pragma unroll
      for (int j = 0; j < 4; j++) sc[j] = Sc[kb * kBN + wn * 64 + j * 16 + frag_row];
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const floatx4 part = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              a[i], b[j], floatx4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 4; r++) acc[i][j][r] = fmaf(sc[j], part[r], acc[i][j][r]);
        }
    }
  };

  StepRegs regs;
  load_step(0, regs);
  store_step(0, regs);
  __syncthreads();
  for (int s = 0; s < steps; s++) {
    const bool more = s + 1 < steps;
    if (more) load_step(s + 1, regs);
    compute_step(s & 1);
    if (more) store_step((s + 1) & 1, regs);
    __syncthreads();
  }

  // Epilogue: lane holds D[4*(lane/16)+r][lane%16] of each 16x16 tile.
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int n = n0 + wn * 64 + j * 16 + (lane & 15);
    if (n >= N) continue;
    const float bv = (bias && kz == 0) ? bias[n] : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int mrow = m0 + wm * 64 + i * 16 + (lane >> 4) * 4 + r;
        if (mrow >= M) continue;
        float* dst = y + (size_t)mrow * N + n;
        const float v = ldexpf(acc[i][j][r], xexp[mrow]);
        if (ksplit == 1)
          *dst = v + bv;
        else
          atomicAdd(dst, v + bv);
      }
  }
}

// Two K halves when the tile grid leaves CUs idle and K allows it.
static int pick_ksplit(size_t tiles, size_t m, int num_cus) {
  if (tiles < (size_t)num_cus * 2 && m % (2 * kBK) == 0) return 2;
  return 1;
}

static hipError_t launch_x_prepass(const float* x, size_t batch, size_t m, void* ws, bool permute,
                                   float* y_zero, size_t y_elems, hipStream_t s) {
  const size_t mp = round_up(batch, kBM);
  int* xexp = gemm_x_exponents(ws, batch, m);
  if (permute)
    hipLaunchKernelGGL(x_rows_to_f16_kernel<true>, dim3((unsigned)mp), dim3(256), 0, s,
                       (u32x4*)ws, xexp, x, (int)batch, (int)m, y_zero, y_elems);
  else
    hipLaunchKernelGGL(x_rows_to_f16_kernel<false>, dim3((unsigned)mp), dim3(256), 0, s,
                       (u32x4*)ws, xexp, x, (int)batch, (int)m, y_zero, y_elems);
  return hipGetLastError();
}

hipError_t launch_x_rows_f16(const float* x, size_t batch, size_t rows, size_t m, void* xh,
                            int* xexp, bool permute, hipStream_t s) {
  if (permute)
    hipLaunchKernelGGL(x_rows_to_f16_kernel<true>, dim3((unsigned)rows), dim3(256), 0, s,
                       (u32x4*)xh, xexp, x, (int)batch, (int)m, nullptr, (size_t)0);
  else
    hipLaunchKernelGGL(x_rows_to_f16_kernel<false>, dim3((unsigned)rows), dim3(256), 0, s,
                       (u32x4*)xh, xexp, x, (int)batch, (int)m, nullptr, (size_t)0);
  return hipGetLastError();
}

hipError_t launch_x_f16_permuted(const float* x, size_t batch, size_t m, void* ws,
                                 hipStream_t s) {
  return launch_x_prepass(x, batch, m, ws, true, nullptr, 0, s);
}

hipError_t launch_x_f16_plain(const float* x, size_t batch, size_t m, void* ws, hipStream_t s) {
  return launch_x_prepass(x, batch, m, ws, false, nullptr, 0, s);
}

hipError_t launch_q4_0_gemm(float* y, const uint8_t* w, const float* x, const float* bias,
                            size_t n, size_t m, size_t batch, void* ws, int num_cus,
                            hipStream_t s) {
  const size_t tiles_n = (n + kBN - 1) / kBN;
  const size_t tiles_m = round_up(batch, kBM) / kBM;
  const int ksplit = pick_ksplit(tiles_n * tiles_m, m, num_cus);
  hipError_t e = launch_x_prepass(x, batch, m, ws, true, ksplit > 1 ? y : nullptr,
                                  ksplit > 1 ? n * batch : 0, s);
  if (e != hipSuccess) return e;
  const size_t lds = 2 * ((size_t)2 * kTileHalves * 2 + 2 * kBN * 4);
  e = set_lds_limit(reinterpret_cast<const void*>(gemm_kernel), (int)lds);
  if (e != hipSuccess) return e;
  const dim3 grid((unsigned)tiles_n, (unsigned)tiles_m, (unsigned)ksplit);
  hipLaunchKernelGGL(gemm_kernel, grid, dim3(256), lds, s, y, w, (const u32x4*)ws,
                     (const int*)gemm_x_exponents(ws, batch, m), bias, (int)batch, (int)n, (int)m,
                     ksplit);
  return hipGetLastError();
}

}  // namespace hypno
