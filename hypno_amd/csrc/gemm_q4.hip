// Q4_0 batched-prefill GEMM for gfx950: Y[M][N] = X[M][K] . W[N][K]^T (+ bias)
// with W in hypno's Q4_0 blocks (quant.rs:10-22) and X rounded to fp16.
//
// The integer nibbles (nib - 8) go to the matrix cores as exact fp16 values;
// each 32-column block is one v_mfma_f32_16x16x32_f16 into a zeroed
// accumulator, and the block's partial sum is scaled by the block's fp32
// scale into fp32 accumulators (acc += d * partial).  That scale FMA is one
// VALU op per output per block -- as much issue time as the MFMA itself -- so
// the kernel is organised to keep VALU work besides it small and to overlap
// it with the matrix pipe:
//
//  * Work-group = 512 threads (8 waves) on a 128 x 128 tile of Y; one
//    work-group per CU, two waves per SIMD.  Waves 0-3 and 4-7 form two
//    K-groups: each stage holds 128 columns of K (four Q4_0 blocks) and
//    K-group g multiplies blocks 2g and 2g+1 of it, with its four waves in a
//    2 x 2 grid of 64 x 64 sub-tiles (4 x 4 MFMA tiles per wave).  At the end
//    K-group 1 hands its accumulators to K-group 0 through LDS (a fixed-order
//    sum: deterministic, no atomics, no zeroed output).
//  * Activations: a pre-pass rounds X to fp16 once, permuting each group of 8
//    columns into the order in which the nibble unpack below emits weights.
//    Each stage's 128 x 128 fp16 X tile is copied straight into LDS with
//    global_load_lds_dwordx4 (no registers, no VALU); the source address of
//    each lane is chosen so that 16-byte chunk c of row r lands in slot
//    c ^ (r & 15) of that row (conflict-free MFMA operand reads).
//  * Weights: each thread fetches one block (a 20-byte window: dwordx4 +
//    dword) two stages ahead into registers, and one stage ahead expands it
//    into LDS as exact fp16 (nib - 8) with two and-or ops and one packed fp16
//    op per pair of weights, plus the block's fp32 scale.  The expansion is
//    done once per work-group and shared by all 128 rows of X.
//  * Two LDS stages (A tile, B tile, scales = 66 KB each) alternate; one
//    barrier per stage.
//
// Requirements (checked by q4_0_gemm_v3_ok): K % 128 == 0, w 4-byte aligned,
// w holds N whole rows.  Tiles at the N and M edges are handled by clamping
// the rows read (their scale is zeroed) and not storing rows/columns past
// the edge.
#include "common.hpp"

namespace hypno {

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int BM = 128;
constexpr int BN = 128;
constexpr int BK = 128;                      // four Q4_0 blocks per stage
constexpr int kThreads = 512;
constexpr int kRowBytes = BK * 2;            // one LDS tile row: 128 fp16
constexpr int kTileBytes = BM * kRowBytes;   // 32 KB
constexpr int kScaleBytes = (BK / 32) * BN * 4;
constexpr int kStageBytes = 2 * kTileBytes + kScaleBytes;
constexpr int kLdsBytes = 2 * kStageBytes;   // 132 KB (< 160 KB)

// Byte offset of 16-byte chunk c of tile row r (XOR-swizzled by the row).
__device__ __forceinline__ uint32_t tile_off(int r, int c) {
  return (uint32_t)(r * kRowBytes + ((c ^ (r & 15)) << 4));
}

// Eight nibbles (byte i of q = e[2i] | e[2i+1] << 4) -> eight exact fp16
// values e - 8 in slot order e0,e4,e1,e5,e2,e6,e3,e7.  0x6400 | n is the fp16
// value 1024 + n and 0x6400 | n << 4 is 1024 + 16n; one packed fp16 add or
// fma maps either to n - 8 exactly.
__device__ __forceinline__ u32x4 unpack8(uint32_t q) {
  const half2v lo_off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
  const half2v hi_mul = {(_Float16)0.0625f, (_Float16)0.0625f};
  const half2v hi_off = {(_Float16)-72.0f, (_Float16)-72.0f};
  const uint32_t q8 = q >> 8;
  const uint32_t p0 = (q & 0x000F000Fu) | 0x64006400u;   // e0, e4
  const uint32_t p1 = (q & 0x00F000F0u) | 0x64006400u;   // e1, e5 (x16)
  const uint32_t p2 = (q8 & 0x000F000Fu) | 0x64006400u;  // e2, e6
  const uint32_t p3 = (q8 & 0x00F000F0u) | 0x64006400u;  // e3, e7 (x16)
  u32x4 r;
  r[0] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, p0) + lo_off);
  r[1] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(
                                          __builtin_bit_cast(half2v, p1), hi_mul, hi_off));
  r[2] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, p2) + lo_off);
  r[3] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(
                                          __builtin_bit_cast(half2v, p3), hi_mul, hi_off));
  return r;
}

struct Raw {  // one thread's 20-byte window of one stage
  u32x4 a;
  uint32_t b;
};

struct Args {
  float* y;
  const uint8_t* w;
  const uint8_t* xh;  // fp16 [Mp][K], columns permuted per group of 8
  const float* bias;
  int M, N, K;
  int tiles_m, tiles_n;
  int xcd_map;        // 1: blockIdx -> tile mapping groups tiles per XCD
};

__global__ void __launch_bounds__(kThreads, 1) q4_0_gemm_v3_kernel(const Args a) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int kgrp = wave >> 2;
  const int wm = (wave >> 1) & 1;
  const int wn = wave & 1;
  const int lr = lane & 15;
  const int lq = lane >> 4;

  // Tile of this work-group.  Work-groups are dispatched round-robin over the
  // 8 XCDs; with xcd_map, XCD x gets a contiguous range of tiles in
  // (n-tile, m-tile) order, so the m-tiles that share a weight tile run on
  // the same XCD and share its L2.
  int tile = blockIdx.x;
  const int ntiles = a.tiles_m * a.tiles_n;
  if (a.xcd_map) tile = (tile & 7) * (ntiles >> 3) + (tile >> 3);
  const int m0 = (tile % a.tiles_m) * BM;
  const int n0 = (tile / a.tiles_m) * BN;
  const int K = a.K;
  const int steps = K / BK;
  const size_t x_row = (size_t)K * 2;
  const size_t w_row = (size_t)(K / 32) * 18;

  // --- activation copy (LDS DMA): wave w, instruction i fills LDS segment
  // i*8 + w (rows 4*seg .. 4*seg+3 of the tile, 1 KB); lane -> row
  // 4*seg + lq, physical chunk lr, i.e. logical chunk lr ^ (row & 15).
  const int arow0 = 4 * wave + lq;               // row for i = 0 (row & 15 same for all i)
  const int achunk = lr ^ (arow0 & 15);
  const uint8_t* xsrc = a.xh + (size_t)(m0 + arow0) * x_row + achunk * 16;
  auto copy_a = [&](int s, int buf) {
    const uint8_t* src = xsrc + (size_t)s * BK * 2;
    uint8_t* dst = smem + buf * kStageBytes + wave * 1024;
#pragma unroll
    for (int i = 0; i < 4; i++)
      __builtin_amdgcn_global_load_lds(
          (const void*)(src + (size_t)i * 32 * x_row),
          (__attribute__((address_space(3))) void*)(dst + i * 8 * 1024), 16, 0, 0);
  };

  // --- weight fetch: thread -> (row br, block bb) of the stage
  const int br = t >> 2, bb = t & 3;
  const bool bvalid = n0 + br < a.N;
  const uint8_t* wsrc = a.w + (size_t)(bvalid ? n0 + br : a.N - 1) * w_row + ((18 * bb) & ~3);
  const bool bodd = (bb & 1) != 0;  // block starts 2 bytes into its window
  const uint32_t sel = bodd ? 0x07060504u : 0x05040302u;
  const uint32_t dsh = bodd ? 16u : 0u;
  auto fetch_b = [&](int s) -> Raw {
    const uint8_t* p = wsrc + (size_t)s * (BK / 32) * 18;
    Raw r;
    r.a = load_global<u32x4>(p);
    r.b = load_global<uint32_t>(p + 16);
    return r;
  };
  auto expand_b = [&](const Raw& r, int buf) {
    uint8_t* bt = smem + buf * kStageBytes + kTileBytes;
    float* sc = reinterpret_cast<float*>(smem + buf * kStageBytes + 2 * kTileBytes);
    const uint32_t d[5] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b};
    sc[((bb * 2 + (br >> 6)) * 16 + (br & 15)) * 4 + ((br & 63) >> 4)] =
        bvalid ? f16_bits_to_f32((d[0] >> dsh) & 0xFFFFu) : 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t q = __builtin_amdgcn_perm(d[j + 1], d[j], sel);
      *reinterpret_cast<u32x4*>(bt + tile_off(br, 4 * bb + j)) = unpack8(q);
    }
  };

  floatx4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  // One stage for this wave: its two blocks kb = 2*kgrp, 2*kgrp + 1.  The
  // operands of the second block are read from LDS before the first block's
  // MFMAs start.  MFMA q = 4i + j; its partial is scaled in after MFMA
  // q + kLag has been issued, so the FMAs do not wait on the matrix pipe and
  // at most kLag + 1 partials are live.  Hard scheduling barriers keep this
  // order (the default scheduler would issue all 32 MFMAs first).
  struct Frags {
    half8 a[4], b[4];
    floatx4 sc;
  };
  auto read_frags = [&](int buf, int kb) -> Frags {
    const uint8_t* at = smem + buf * kStageBytes;
    const uint8_t* bt = at + kTileBytes;
    const uint8_t* st = at + 2 * kTileBytes;
    const int c = ((4 * kb + lq) ^ lr) << 4;
    Frags f;
#pragma unroll
    for (int i = 0; i < 4; i++)
      f.a[i] = *reinterpret_cast<const half8*>(at + (wm * 64 + 16 * i + lr) * kRowBytes + c);
#pragma unroll
    for (int j = 0; j < 4; j++)
      f.b[j] = *reinterpret_cast<const half8*>(bt + (wn * 64 + 16 * j + lr) * kRowBytes + c);
    f.sc = *reinterpret_cast<const floatx4*>(st + ((kb * 2 + wn) * 16 + lr) * 16);
    return f;
  };
  constexpr int kLag = 3;
  auto mma_block = [&](Frags f) {
    floatx4 part[16];
#pragma unroll
    for (int q = 0; q < 16 + kLag; q++) {
      if (q < 16)
        part[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(f.a[q >> 2], f.b[q & 3],
                                                         floatx4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
      if (q >= kLag) {
        const int u = q - kLag;
#pragma unroll
        for (int r = 0; r < 4; r++)
          acc[u >> 2][u & 3][r] = fmaf(f.sc[u & 3], part[u][r], acc[u >> 2][u & 3][r]);
        // Order MFMA q+1 after these FMAs: its A operand passes through an
        // (empty) statement that also takes the accumulator just written.
        if (q + 1 < 16) asm volatile("" : "+v"(f.a[(q + 1) >> 2]), "+v"(acc[u >> 2][u & 3]));
      }
    }
  };
  auto compute = [&](int buf) {
    const Frags f0 = read_frags(buf, 2 * kgrp);
    const Frags f1 = read_frags(buf, 2 * kgrp + 1);
    __builtin_amdgcn_sched_barrier(0);
    mma_block(f0);
    mma_block(f1);
  };

  // Prologue: stage 0 in LDS buffer 0, stage 1's weights in registers.
  Raw raw0 = fetch_b(0);
  Raw raw1 = raw0;
  if (steps > 1) raw1 = fetch_b(1);
  copy_a(0, 0);
  expand_b(raw0, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  // Stage s: start the copy of stage s+1's activations into the other buffer
  // and the fetch of stage s+2's weights, compute stage s, expand stage s+1's
  // weights (fetched a stage ago), then wait for everything and barrier.
  // Unrolled by two so the register double buffer has static names.
  for (int s = 0; s < steps; s += 2) {
    {
      const bool more = s + 1 < steps;
      if (more) copy_a(s + 1, 1);
      if (s + 2 < steps) raw0 = fetch_b(s + 2);
      compute(0);
      if (more) expand_b(raw1, 1);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      if (!more) break;
    }
    {
      const bool more = s + 2 < steps;
      if (more) copy_a(s + 2, 0);
      if (s + 3 < steps) raw1 = fetch_b(s + 3);
      compute(1);
      if (more) expand_b(raw0, 0);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    }
  }

  // K-group 1 -> LDS -> K-group 0 adds (fixed order) and stores.
  float* red = reinterpret_cast<float*>(smem);
  const int wig = wave & 3;
  if (kgrp == 1) {
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) red[((wig * 64 + (i * 4 + j) * 4 + r) * 64) + lane] = acc[i][j][r];
  }
  __syncthreads();
  if (kgrp == 0) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int n = n0 + wn * 64 + 16 * j + lr;
      const bool nok = n < a.N;
      const float bv = (a.bias && nok) ? a.bias[n] : 0.0f;
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const float v = acc[i][j][r] + red[((wig * 64 + (i * 4 + j) * 4 + r) * 64) + lane];
          const int m = m0 + wm * 64 + 16 * i + 4 * lq + r;
          if (nok && m < a.M) a.y[(size_t)m * a.N + n] = v + bv;
        }
    }
  }
}

}  // namespace

bool q4_0_gemm_v3_ok(const uint8_t* w, size_t w_len, size_t n, size_t m, size_t batch) {
  if (m == 0 || m % BK != 0 || n == 0 || batch == 0) return false;
  if (((uintptr_t)w & 3) != 0) return false;
  if (n > (size_t)0x7FFFFFFF || m > (size_t)0x7FFFFFF || batch > (size_t)0x7FFFFFFF) return false;
  const size_t tiles = ((n + BN - 1) / BN) * ((batch + BM - 1) / BM);
  if (tiles > (size_t)0x7FFFFFFF) return false;
  return w_len / kBlockBytes >= n * (m / kBlockElems);
}

hipError_t launch_q4_0_gemm_v3(float* y, const uint8_t* w, const float* x, const float* bias,
                               size_t n, size_t m, size_t batch, void* ws, int num_cus,
                               hipStream_t s) {
  (void)num_cus;
  hipError_t e = launch_x_f16_permuted(x, batch, m, ws, s);
  if (e != hipSuccess) return e;
  static bool attr_set = false;
  if (!attr_set) {
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(q4_0_gemm_v3_kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  Args a;
  a.y = y;
  a.w = w;
  a.xh = static_cast<const uint8_t*>(ws);
  a.bias = bias;
  a.M = (int)batch;
  a.N = (int)n;
  a.K = (int)m;
  a.tiles_m = (int)((batch + BM - 1) / BM);
  a.tiles_n = (int)((n + BN - 1) / BN);
  const int tiles = a.tiles_m * a.tiles_n;
  a.xcd_map = (tiles % 8) == 0 ? 1 : 0;
  hipLaunchKernelGGL(q4_0_gemm_v3_kernel, dim3(tiles), dim3(kThreads), kLdsBytes, s, a);
  return hipGetLastError();
}

}  // namespace hypno
