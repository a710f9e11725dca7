// Q4_0 matmul for a few tokens (2 <= M <= 64): Y[M][N] = X[M][K] . W[N][K]^T.
//
// This regime is bound by the weight stream (3.6 M flop per weight byte at
// most 228 flop/B, below the ~310 flop/B ridge), so the kernel streams every
// Q4_0 block of W exactly once and does the arithmetic on the matrix cores:
//
//  * A work-group owns 16 rows of W (one MFMA column tile); its W waves split
//    K into W equal ranges and their fp32 partial sums are added through LDS
//    in wave order at the end (deterministic, no atomics).
//  * Each lane loads the 4 nibble bytes it feeds to v_mfma_f32_16x16x32_f16
//    (row lane & 15, nibble dword lane >> 4 of the block) plus the block's
//    fp16 scale straight from global memory, two blocks at a time, a few
//    block pairs ahead in registers.  The nibbles become exact fp16
//    (nib - 8) in registers; the block's partial is scaled in fp32.
//  * Activations come from a pre-pass as MFMA A-operand rows (fp16, columns
//    permuted per group of 8 to the unpack order):
//      - M <= 16 ("split"): token t is scaled by a power of two s_t so that
//        max|x_t| s_t lies in [2^14, 2^15), and stored as hi = fp16(x s_t)
//        in row t and lo = fp16(x s_t - hi) in row Mh + t.  hi + lo equals
//        x s_t to about 2^-22 relative, the products with the exact integer
//        weights are exact in fp32, and y_t = (acc_hi + acc_lo) / s_t: an
//        fp32-accurate result, as the GEMV path gives.
//      - 16 < M <= 64: one fp16 row per token (the prefill GEMM's rounding).
//
// Requirements (q4_0_skinny_ok): K % (64 * waves) == 0, w 4-byte aligned,
// w holds N whole rows.
#include "common.hpp"

namespace hypno {

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// Eight nibbles (byte i of q = e[2i] | e[2i+1] << 4) -> eight exact fp16
// values e - 8 in slot order e0,e4,e1,e5,e2,e6,e3,e7 (0x6400 | n = 1024 + n,
// 0x6400 | n << 4 = 1024 + 16 n).
__device__ __forceinline__ half8 unpack8h(uint32_t q) {
  const half2v lo_off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
  const half2v hi_mul = {(_Float16)0.0625f, (_Float16)0.0625f};
  const half2v hi_off = {(_Float16)-72.0f, (_Float16)-72.0f};
  const uint32_t q8 = q >> 8;
  u32x4 r;
  r[0] = __builtin_bit_cast(uint32_t,
                            __builtin_bit_cast(half2v, (q & 0x000F000Fu) | 0x64006400u) + lo_off);
  r[1] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(
      __builtin_bit_cast(half2v, (q & 0x00F000F0u) | 0x64006400u), hi_mul, hi_off));
  r[2] = __builtin_bit_cast(uint32_t,
                            __builtin_bit_cast(half2v, (q8 & 0x000F000Fu) | 0x64006400u) + lo_off);
  r[3] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(
      __builtin_bit_cast(half2v, (q8 & 0x00F000F0u) | 0x64006400u), hi_mul, hi_off));
  return __builtin_bit_cast(half8, r);
}

__device__ __forceinline__ uint32_t pack2h(float a, float b) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)a) |
         ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)b) << 16);
}

// Pre-pass: X fp32 [M][K] -> A rows fp16 [rows][K] (+ 1/s_t per token).
// One work-group per hi row r < Mh: token r's hi row (and lo row Mh + r when
// split), or zero rows for r >= M.
__global__ void __launch_bounds__(256)
x_skinny_kernel(uint8_t* __restrict__ xa, float* __restrict__ inv_s, const float* __restrict__ x,
                int M, int K, int Mh, int split) {
  __shared__ float red[4];
  const int r = blockIdx.x;
  const int t = threadIdx.x;
  u32x4* hi_row = reinterpret_cast<u32x4*>(xa + (size_t)r * K * 2);
  u32x4* lo_row = reinterpret_cast<u32x4*>(xa + (size_t)(Mh + r) * K * 2);
  const int groups = K / 8;
  if (r >= M) {
    for (int g = t; g < groups; g += 256) {
      hi_row[g] = u32x4{0u, 0u, 0u, 0u};
      if (split) lo_row[g] = u32x4{0u, 0u, 0u, 0u};
    }
    return;
  }
  const float* xr = x + (size_t)r * K;
  float s = 1.0f;
  if (split) {
    uint32_t mb = 0;  // largest |x| by bit pattern (NaN/inf compare above finite)
    for (int i = t; i < K; i += 256) mb = max(mb, __float_as_uint(xr[i]) & 0x7FFFFFFFu);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mb = max(mb, (uint32_t)__shfl_xor((int)mb, o, 64));
    if ((t & 63) == 0) red[t >> 6] = __uint_as_float(mb);
    __syncthreads();
    const float amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    // s = 2^(15 - e) with amax < 2^e, so amax * s < 2^15; zero, inf and NaN
    // rows keep s = 1 (their products propagate as the reference's would)
    if (amax > 0.0f && amax < __builtin_inff())
      s = ldexpf(1.0f, min(15 - __builtin_amdgcn_frexp_expf(amax), 126));
    if (t == 0) inv_s[r] = 1.0f / s;
  }
  constexpr int perm[8] = {0, 4, 1, 5, 2, 6, 3, 7};
  for (int g = t; g < groups; g += 256) {
    const float4 a0 = load_global<float4>(xr + 8 * g);
    const float4 a1 = load_global<float4>(xr + 8 * g + 4);
    const float v[8] = {a0.x * s, a0.y * s, a0.z * s, a0.w * s,
                        a1.x * s, a1.y * s, a1.z * s, a1.w * s};
    u32x4 h, l;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float p = v[perm[2 * j]], q = v[perm[2 * j + 1]];
      h[j] = pack2h(p, q);
      if (split) {
        const float ph = (float)(_Float16)p, qh = (float)(_Float16)q;
        l[j] = pack2h(p - ph, q - qh);
      }
    }
    hi_row[g] = h;
    if (split) lo_row[g] = l;
  }
}

struct SkinnyArgs {
  float* y;
  const uint8_t* w;
  const uint8_t* xa;
  const float* inv_s;
  const float* bias;
  int M, N, K;
  int Mh;     // row offset of the lo rows (split), else 0
  int split;
};

// One block pair (2p, 2p+1) of one 16-row tile, as loaded by this lane.
template <int MF>
struct Pair {
  uint32_t e0, e1, es;  // even block: 8 bytes around the nibble dword, scale dword
  uint32_t on, os;      // odd block: nibble dword, scale dword
  u32x4 xe[MF], xo[MF]; // A operands of the two blocks
};

template <int MF, int W>
__global__ void __launch_bounds__(64 * W) q4_0_skinny_kernel(const SkinnyArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int lr = lane & 15, lq = lane >> 4;
  const int K = a.K;
  const int nblk = K / 32 / W;  // blocks per wave (even)
  const int n = blockIdx.x * 16 + lr;
  const bool nvalid = n < a.N;
  const size_t w_row = (size_t)(K / 32) * 18;
  const uint8_t* wr = a.w + (size_t)(nvalid ? n : a.N - 1) * w_row + (size_t)wave * nblk * 18;
  const size_t x_row = (size_t)K * 2;
  const uint8_t* xr = a.xa + (size_t)lr * x_row + ((size_t)wave * nblk * 32 + 8 * lq) * 2;

  auto load = [&](int p) -> Pair<MF> {
    Pair<MF> r;
    const uint8_t* b = wr + (size_t)p * 36;  // even block start (4-byte aligned)
    r.e0 = load_global<uint32_t>(b + 4 * lq);
    r.e1 = load_global<uint32_t>(b + 4 * lq + 4);
    r.es = load_global<uint32_t>(b);
    r.on = load_global<uint32_t>(b + 20 + 4 * lq);
    r.os = load_global<uint32_t>(b + 16);
    const uint8_t* xp = xr + (size_t)p * 128;
#pragma unroll
    for (int m = 0; m < MF; m++) {
      r.xe[m] = load_global<u32x4>(xp + (size_t)m * 16 * x_row);
      r.xo[m] = load_global<u32x4>(xp + (size_t)m * 16 * x_row + 64);
    }
    return r;
  };

  floatx4 acc[MF];
#pragma unroll
  for (int m = 0; m < MF; m++) acc[m] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  // `live` is false for the padding pairs past the end (their scales are
  // zeroed, so they add nothing).
  auto compute = [&](const Pair<MF>& r, bool live) {
    const half8 be = unpack8h(__builtin_amdgcn_perm(r.e1, r.e0, 0x05040302u));
    const half8 bo = unpack8h(r.on);
    const bool v = nvalid && live;
    const float se = v ? f16_bits_to_f32(r.es & 0xFFFFu) : 0.0f;
    const float so = v ? f16_bits_to_f32(r.os >> 16) : 0.0f;
#pragma unroll
    for (int m = 0; m < MF; m++) {
      const floatx4 pe = __builtin_amdgcn_mfma_f32_16x16x32_f16(
          __builtin_bit_cast(half8, r.xe[m]), be, floatx4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
      const floatx4 po = __builtin_amdgcn_mfma_f32_16x16x32_f16(
          __builtin_bit_cast(half8, r.xo[m]), bo, floatx4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; i++) acc[m][i] = fmaf(so, po[i], fmaf(se, pe[i], acc[m][i]));
    }
  };

  // Ring of four pairs with static slot names and no early exit (an exit
  // lets the compiler sink each load down to its use, which serialises the
  // stream): while pair p is computed, pairs p+1..p+3 are in flight and pair
  // p+4 is requested into the slot just freed.  The pair count is padded to
  // a multiple of four; requests past the end re-read pair 0 (in bounds).
  const int np = nblk / 2;
  auto nxt = [&](int p) { return p < np ? p : 0; };
  Pair<MF> ra = load(0);
  __builtin_amdgcn_sched_barrier(0);
  Pair<MF> rb = load(nxt(1));
  __builtin_amdgcn_sched_barrier(0);
  Pair<MF> rc = load(nxt(2));
  __builtin_amdgcn_sched_barrier(0);
  Pair<MF> rd = load(nxt(3));
  __builtin_amdgcn_sched_barrier(0);
  // Scheduling barriers keep each request after the compute before it (the
  // scheduler would otherwise hoist requests, and the in-order load counter
  // would then make each compute wait for younger requests too).
  for (int p = 0; p < np; p += 4) {
    compute(ra, true);
    __builtin_amdgcn_sched_barrier(0);
    ra = load(nxt(p + 4));
    __builtin_amdgcn_sched_barrier(0);
    compute(rb, p + 1 < np);
    __builtin_amdgcn_sched_barrier(0);
    rb = load(nxt(p + 5));
    __builtin_amdgcn_sched_barrier(0);
    compute(rc, p + 2 < np);
    __builtin_amdgcn_sched_barrier(0);
    rc = load(nxt(p + 6));
    __builtin_amdgcn_sched_barrier(0);
    compute(rd, p + 3 < np);
    __builtin_amdgcn_sched_barrier(0);
    rd = load(nxt(p + 7));
    __builtin_amdgcn_sched_barrier(0);
  }

  // Wave partials -> LDS; wave 0 adds them in wave order and stores.
  float* red = reinterpret_cast<float*>(smem);
  if (wave > 0) {
#pragma unroll
    for (int m = 0; m < MF; m++)
#pragma unroll
      for (int i = 0; i < 4; i++) red[(((wave - 1) * MF + m) * 4 + i) * 64 + lane] = acc[m][i];
  }
  __syncthreads();
  if (wave != 0) return;
  for (int v = 1; v < W; v++)
#pragma unroll
    for (int m = 0; m < MF; m++)
#pragma unroll
      for (int i = 0; i < 4; i++) acc[m][i] += red[(((v - 1) * MF + m) * 4 + i) * 64 + lane];
  // lane holds A rows 16m + 4*lq + i of column n
  const float bv = (a.bias && nvalid) ? a.bias[n] : 0.0f;
  if (a.split) {
    if (MF == 1) {  // hi rows 0..7 in lanes lq 0-1, lo rows 8..15 in lanes lq 2-3
#pragma unroll
      for (int i = 0; i < 4; i++) acc[0][i] += __shfl_down(acc[0][i], 32, 64);
      if (lq < 2 && nvalid) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int tkn = 4 * lq + i;
          if (tkn < a.M) a.y[(size_t)tkn * a.N + n] = acc[0][i] * a.inv_s[tkn] + bv;
        }
      }
    } else {  // hi frags 0 .. MF/2-1, lo frags MF/2 .. MF-1
#pragma unroll
      for (int m = 0; m < MF / 2; m++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int tkn = 16 * m + 4 * lq + i;
          if (nvalid && tkn < a.M)
            a.y[(size_t)tkn * a.N + n] = (acc[m][i] + acc[m + MF / 2][i]) * a.inv_s[tkn] + bv;
        }
    }
  } else {
#pragma unroll
    for (int m = 0; m < MF; m++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int tkn = 16 * m + 4 * lq + i;
        if (nvalid && tkn < a.M) a.y[(size_t)tkn * a.N + n] = acc[m][i] + bv;
      }
  }
}

// Waves per work-group (K split): enough waves overall to cover the chip.
int skinny_waves(size_t n, size_t m, int num_cus) {
  const size_t tiles = (n + 15) / 16;
  int w = 2;
  while (w < 8 && tiles * (size_t)w < (size_t)num_cus * 8 && m % (64 * (size_t)w * 2) == 0) w *= 2;
  return m % (64 * (size_t)w) == 0 ? w : 0;
}

struct SkinnyShape {
  int mf;      // A operand frags (16 rows each)
  int split;   // hi/lo rows
  int rows;    // A rows written by the pre-pass
  int mh;      // lo row offset
};

SkinnyShape skinny_shape(size_t batch) {
  SkinnyShape s;
  if (batch <= 8) {
    s.mf = 1; s.split = 1; s.mh = 8;
  } else if (batch <= 16) {
    s.mf = 2; s.split = 1; s.mh = 16;
  } else if (batch <= 32) {
    s.mf = 2; s.split = 0; s.mh = 32;
  } else {
    s.mf = 4; s.split = 0; s.mh = 64;
  }
  s.rows = 16 * s.mf;
  return s;
}

template <int MF>
hipError_t launch_mf(int w, const SkinnyArgs& a, int grid, hipStream_t s) {
  const size_t lds = (size_t)(w - 1) * MF * 4 * 64 * 4;
  switch (w) {
    case 2:
      hipLaunchKernelGGL((q4_0_skinny_kernel<MF, 2>), dim3(grid), dim3(128), lds, s, a);
      break;
    case 4:
      hipLaunchKernelGGL((q4_0_skinny_kernel<MF, 4>), dim3(grid), dim3(256), lds, s, a);
      break;
    default:
      hipLaunchKernelGGL((q4_0_skinny_kernel<MF, 8>), dim3(grid), dim3(512), lds, s, a);
      break;
  }
  return hipGetLastError();
}

}  // namespace

bool q4_0_skinny_ok(const uint8_t* w, size_t w_len, size_t n, size_t m, size_t batch, int num_cus) {
  if (batch < 2 || batch > 64 || n == 0 || m == 0) return false;
  if (((uintptr_t)w & 3) != 0) return false;
  if (n > (size_t)0x7FFFFFFF || m > (size_t)0x7FFFFFF) return false;
  if (skinny_waves(n, m, num_cus) == 0) return false;
  return w_len / kBlockBytes >= n * (m / kBlockElems);
}

size_t skinny_workspace_bytes(size_t batch, size_t m) {
  const SkinnyShape sh = skinny_shape(batch);
  return (size_t)sh.rows * m * 2 + 64 * 4;
}

hipError_t launch_q4_0_skinny(float* y, const uint8_t* w, const float* x, const float* bias,
                              size_t n, size_t m, size_t batch, void* ws, int num_cus,
                              hipStream_t s) {
  const SkinnyShape sh = skinny_shape(batch);
  uint8_t* xa = static_cast<uint8_t*>(ws);
  float* inv_s = reinterpret_cast<float*>(xa + (size_t)sh.rows * m * 2);
  const int hi_rows = sh.split ? sh.mh : sh.rows;
  hipLaunchKernelGGL(x_skinny_kernel, dim3(hi_rows), dim3(256), 0, s, xa, inv_s, x, (int)batch,
                     (int)m, sh.mh, sh.split);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  SkinnyArgs a;
  a.y = y;
  a.w = w;
  a.xa = xa;
  a.inv_s = inv_s;
  a.bias = bias;
  a.M = (int)batch;
  a.N = (int)n;
  a.K = (int)m;
  a.Mh = sh.mh;
  a.split = sh.split;
  const int grid = (int)((n + 15) / 16);
  const int wv = skinny_waves(n, m, num_cus);
  switch (sh.mf) {
    case 1: return launch_mf<1>(wv, a, grid, s);
    case 2: return launch_mf<2>(wv, a, grid, s);
    default: return launch_mf<4>(wv, a, grid, s);
  }
}

}  // namespace hypno
