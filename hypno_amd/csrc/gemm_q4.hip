// Q4_0 batched-prefill GEMM for gfx950: Y[M][N] = X[M][K] . W[N][K]^T (+ bias)
// with W in hypno's Q4_0 blocks (quant.rs:10-22) and X rounded to fp16.
//
// Two ways to apply the per-block scale d, one kernel template:
//
//  * kFold (M >= 256, or >= 128 for W up to 64 MB): each weight goes to the
//    matrix cores as fp16 (nib - 8) * (d / D_n), with D_n a power of two
//    just above the largest |d| of weight row n (the pre-pass that converts
//    X, q4_0_prepass_kernel, also writes that exponent): every such value
//    lies in (-8, 8), so none overflows fp16; the MFMAs accumulate straight
//    into fp32 accumulators across blocks, and the output column is
//    multiplied by D_n at the end (exact: a power of two).  Each weight is
//    rounded to fp16 once (relative 2^-11).
//  * exact (smaller M, where the pre-pass's extra read of W costs more than
//    folding saves): the integer nibbles go to the matrix cores as exact fp16
//    values, each block is one MFMA into a zeroed accumulator, and the
//    block's partial sum is scaled by d into the fp32 accumulators
//    (acc += d * partial) -- one VALU FMA per output per block, as much issue
//    time as the MFMA itself.
//
//  * Work-group = 512 threads (8 waves) on a 128 x 128 tile of Y, one per CU,
//    two waves per SIMD.  A stage is 64 columns of K (two Q4_0 blocks); waves
//    0-3 (K-group 0) multiply block 0 of every stage and waves 4-7 block 1,
//    each wave a 64 x 64 sub-tile (4 x 4 MFMA tiles).  At the end K-group 1
//    hands its accumulators to K-group 0 through LDS (fixed-order sum:
//    deterministic, no atomics, no zeroed output).
//  * Global reads run kPrefetch = 4 stages ahead, three VMEM instructions
//    per wave and stage, so one s_waitcnt vmcnt(3) per stage waits for
//    precisely the data the next stage needs:
//      - X: two LDS DMAs (global_load_lds_dwordx4) per wave into a 4-slot
//        ring.  A pre-pass rounds X to fp16 once, permuting each group of 8
//        columns into the order the nibble unpack emits weights.  Each
//        stage's 128 x 64 tile lands with 16-byte chunk c of row r in slot
//        c ^ ((r >> 1) & 7) (conflict-free MFMA operand reads).
//      - W: one 12-byte register read per thread (global_load_dwordx3 from
//        asm, so the compiler adds no waits of its own): a quarter of one
//        row's 36 stage bytes -- a block's scale and 8 nibble bytes, or the
//        other 8 -- in a two-deep register double buffer.
//  * Two stages ahead, every thread unpacks its 16 nibbles into exact fp16
//    (nib - 8) with one and-or op and one packed fp16 op per pair of weights,
//    and either multiplies them by fp16(d / D_n) (kFold: one packed fp16 op
//    per pair) or writes the block scale as fp32 beside them, into a 2-slot
//    B ring in LDS.  The expansion is shared by all 128 rows of X.
//  * Each MFMA operand register is reloaded from LDS for the next stage
//    right after its last MFMA of this stage, so LDS latency hides behind
//    the matrix work.  One barrier per stage.
//  * Tile grids under 3/4 of the CUs split K over blockIdx.y into fp32
//    partial planes that split_k_reduce_kernel adds in split order (+ bias).
//  * Work-groups go round-robin over the 8 XCDs; the tile order gives each
//    XCD a contiguous range of tiles, so the M-tiles sharing a W tile share
//    an L2.
//
// Requirements (q4_0_gemm_v3_ok): K % 256 == 0 (rows of W start on 16-byte
// boundaries), w 16-byte aligned, w holds N whole rows.  Rows past N read
// row N-1 with a zero scale; rows/columns past M/N are not stored.
#include <algorithm>

#include "common.hpp"

namespace hypno {

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int BM = 128;
constexpr int BN = 128;
constexpr int BK = 64;          // two Q4_0 blocks per stage
constexpr int kThreads = 512;
constexpr int kPrefetch = 4;    // stages of DMA in flight ahead of the compute
constexpr int kARing = kPrefetch;       // stage s+1 read while s+2..s+4 land
constexpr int kBRing = 2;               // stage s+1 read while s+2 is written
constexpr int kRowBytes = BK * 2;           // 128 B: one fp16 tile row
constexpr int kTileBytes = BM * kRowBytes;  // 16 KB
constexpr int kScaleBytes = 2 * BN * 4;     // 1 KB (exact variant)
constexpr int kOffA = 0;
constexpr int kOffB = kOffA + kARing * kTileBytes;
constexpr int kOffS = kOffB + kBRing * kTileBytes;
constexpr int kLdsBytes = kOffS + kBRing * kScaleBytes;  // 98 KB (< 160 KB)
// The folded-scale variant runs from kFoldMinBatch tokens, and from
// kFoldMinBatchSmallW when W is at most kFoldSmallWBytes (its pre-pass reads
// every block scale, i.e. all of W once more; for a 295 MB lm_head at 128
// tokens that costs more than folding saves, for a 33 MB matrix it does not).
constexpr size_t kFoldMinBatch = 256;
constexpr size_t kFoldMinBatchSmallW = 128;
constexpr size_t kFoldSmallWBytes = (size_t)64 << 20;
static_assert(kLdsBytes <= 160 * 1024, "LDS budget");
static_assert(4 * 64 * 64 * 4 <= kARing * kTileBytes, "K-group reduction fits in the A ring");

// End of stage s: every wave waits until all but its three newest global
// reads (the two X DMAs of stage s+4 and the W read of stage s+4) have
// landed -- vmcnt counts this wave's outstanding reads in issue order, three
// per stage -- and its LDS writes are done; then the work-group meets at the
// barrier.  One asm statement with a memory clobber: the compiler neither
// moves LDS accesses across it nor adds the vmcnt(0) that a fence-based
// __syncthreads() would (which would drain the prefetch ring).
static_assert(kPrefetch == 4, "stage_barrier's vmcnt(3) is one stage of reads");
__device__ __forceinline__ void stage_barrier() {
  asm volatile("s_waitcnt vmcnt(3) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// 12-byte global read into registers (global_load_dwordx3), an ordinary
// load: the compiler tracks the registers it fills and places the wait for
// them before their first use (the weight unpack a stage later), counting
// the LDS DMAs issued in between.
__device__ __forceinline__ u32x3 global_load_w(const uint8_t* p) { return load_global<u32x3>(p); }

// Byte offset of 16-byte chunk c (0..7) of tile row r.
__device__ __forceinline__ uint32_t tile_off(int r, int c) {
  return (uint32_t)(r * kRowBytes + ((c ^ ((r >> 1) & 7)) << 4));
}

// One wave-wide 16-byte-per-lane DMA: lane i's 16 bytes at `src` land at
// lds_wave_base + 16 * i.
__device__ __forceinline__ void dma16(const void* src, uint8_t* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds_wave_base,
                                   16, 0, 0);
}

struct Args {
  float* y;
  const uint8_t* w;
  const uint8_t* xh;  // fp16 [Mp][K], columns permuted per group of 8
  const float* bias;
  int M, N, K;
  int tiles_m, tiles_n;
  int xcd_map;        // 1: blockIdx -> tile mapping groups tiles per XCD
  int splits;         // K split over blockIdx.y; > 1: fp32 partials to `part`
  float* part;        // [splits][M][N] partial sums (splits > 1)
  const int* rowexp;  // [N]: D_n = 2^rowexp[n] (kFold)
  const int* xexp;    // [Mp]: row m of xh holds X row m times 2^-xexp[m]
};

// One launch before the folded-scale GEMM.  Work-groups [0, Mp) round X to
// fp16, one row each (x_row_to_f16, permuted, per-row exponents); the rest
// write rowexp[n] = e with 2^(e-1) <= max |d| < 2^e over weight row n's
// blocks (0 when that maximum is 0 or not finite), one wave per row, its
// scale loads four deep.
__global__ void __launch_bounds__(256)
q4_0_prepass_kernel(u32x4* __restrict__ xh, int* __restrict__ xexp, const float* __restrict__ x,
                    int M, int Mp, int K, int* __restrict__ rowexp,
                    const uint8_t* __restrict__ w, int n) {
  if ((int)blockIdx.x < Mp) {
    x_row_to_f16<true>(xh, xexp, x, M, K, (int)blockIdx.x);
    return;
  }
  const int row = (int)(((blockIdx.x - Mp) * blockDim.x + threadIdx.x) >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= n) return;  // wave-uniform
  const int bpr = K / kBlockElems;
  const uint8_t* base = w + (size_t)row * bpr * kBlockBytes;
  float mx = 0.0f;
  for (int b0 = lane; b0 < bpr; b0 += 256) {
    float d[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int b = b0 + 64 * u;
      const uint8_t* blk = base + (size_t)b * kBlockBytes;
      d[u] = b < bpr ? f16_bits_to_f32((uint32_t)blk[0] | ((uint32_t)blk[1] << 8)) : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < 4; u++) mx = fmaxf(mx, fabsf(d[u]));
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  int e = 0;
  if (mx > 0.0f && mx <= 3.0e38f) frexpf(mx, &e);
  if (lane == 0) rowexp[row] = e;
}

template <bool kFold>
__global__ void __launch_bounds__(kThreads, 1) q4_0_gemm_v3_kernel(const Args a) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
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
  // This work-group's K range: stages [s0, s0 + steps) of gsteps (even
  // bounds; the ring code runs on local stage numbers, addresses use s0 + s).
  const int gsteps = a.K / BK;
  const int z = blockIdx.y;
  const int s0 = (int)((long long)gsteps * z / a.splits) & ~1;
  const int s1 = z == a.splits - 1 ? gsteps : (int)((long long)gsteps * (z + 1) / a.splits) & ~1;
  const int steps = s1 - s0;
  const size_t x_row = (size_t)a.K * 2;
  const size_t w_row = (size_t)(a.K / 32) * 18;

  // --- X DMA: wave w, instruction i fills rows 64i + 8w .. +7 (1 KB); lane
  // -> row 64i + 8w + (lane >> 3), slot lane & 7 = logical chunk
  // (lane & 7) ^ ((row >> 1) & 7), and (row >> 1) & 7 does not depend on i.
  const int xr = 8 * wave + (lane >> 3);
  const int xc = (lane & 7) ^ ((xr >> 1) & 7);
  const uint8_t* xsrc = a.xh + (size_t)(m0 + xr) * x_row + xc * 16;
  auto issue = [&](int s) {  // X DMA of stage min(s, steps-1) into the ring slot of s
    const int sc = s < steps ? s : steps - 1;
    uint8_t* adst = smem + kOffA + (s % kARing) * kTileBytes + wave * 1024;
    const uint8_t* asrc = xsrc + (size_t)(s0 + sc) * kRowBytes;
    dma16(asrc, adst);
    dma16(asrc + 64 * x_row, adst + 8 * 1024);
  };

  // --- expansion role: thread -> row er, block eb of the stage, half eh.
  // Its 12 bytes of a stage are read straight into registers: for eb = 0 the
  // block's scale and first 8 nibble bytes, or the last 8; for eb = 1 the
  // same 2 bytes later (the block starts 18 bytes into the stage's 36), so
  // the dword-aligned read starts at 16 + 8 eh and ends at most at the row's
  // end.
  // The four threads of a row are lanes 4k..4k+3; lanes 4k+4..4k+7 take a
  // row whose swizzle differs in its low bit (k's two low bits swapped), so
  // every 8 lanes of a 16-byte LDS write cover all eight chunk slots of the
  // 128-byte row stride (no bank conflict).
  const int erk = (t >> 2) & 15;
  const int er = (t >> 6) * 16 + ((erk & 12) | ((erk & 1) << 1) | ((erk >> 1) & 1));
  const int eb = (t >> 1) & 1, eh = t & 1;
  const bool evalid = n0 + er < a.N;
  const uint32_t esel = eb ? 0x07060504u : 0x05040302u;  // block at byte 0 / 2 mod 4
  const uint8_t* erow = a.w + (size_t)min(n0 + er, a.N - 1) * w_row + 16 * eb + 8 * eh;
  const uint32_t boff0 = tile_off(er, 4 * eb + 2 * eh);
  const uint32_t boff1 = tile_off(er, 4 * eb + 2 * eh + 1);
  const uint32_t soff = (((eb * 2 + (er >> 6)) * 16 + (er & 15)) * 4 + ((er & 63) >> 4)) * 4;
  const int eexp = (kFold && evalid) ? a.rowexp[n0 + er] : 0;
  using RawW = u32x3;
  auto raw_load = [&](int s) -> RawW {  // stage min(s, steps-1) of this range
    const int g = s0 + (s < steps ? s : steps - 1);
    return global_load_w(erow + (size_t)g * 36);
  };
  struct Expanded {
    u32x4 lo, hi;
    float scale;  // exact variant
  };
  auto expand_unpack = [&](const RawW& r) -> Expanded {
    if constexpr (!kFold) {
      Expanded e;
      e.lo = unpack8(__builtin_amdgcn_perm(r.y, r.x, esel));
      e.hi = unpack8(__builtin_amdgcn_perm(r.z, r.y, esel));
      const uint32_t dbits = (r.x >> (eb ? 16 : 0)) & 0xFFFFu;
      e.scale = evalid ? f16_bits_to_f32(dbits) : 0.0f;  // used by the eh = 0 thread
      return e;
    }
    // fp16(d / D_n): exact while d / D_n is a normal fp16 number (d is fp16,
    // D_n a power of two); rows past N get 0.  Only the eh = 0 thread's words
    // hold the block's scale; its eh = 1 partner (the next lane) takes it
    // with a DPP lane move (quad_perm 0,0,2,2).
    const uint32_t own = (r.x >> (eb ? 16 : 0)) & 0xFFFFu;
    const uint32_t dbits = (uint32_t)__builtin_amdgcn_mov_dpp((int)own, 0xA0, 0xF, 0xF, false);
    const _Float16 h = evalid ? (_Float16)ldexpf(f16_bits_to_f32(dbits), -eexp) : (_Float16)0.0f;
    const half2v hh = {h, h};
    const u32x4 lo = unpack8(__builtin_amdgcn_perm(r.y, r.x, esel));
    const u32x4 hi = unpack8(__builtin_amdgcn_perm(r.z, r.y, esel));
    // (__builtin_bit_cast of a vector element reads element 0 under this
    // compiler, so each word is copied to a scalar first.)
    Expanded e;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t wl = lo[i], wh = hi[i];
      e.lo[i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, wl) * hh);
      e.hi[i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, wh) * hh);
    }
    e.scale = 0.0f;
    return e;
  };
  auto expand_write = [&](int s, const Expanded& e) {
    uint8_t* bt = smem + kOffB + (s % kBRing) * kTileBytes;
    *reinterpret_cast<u32x4*>(bt + boff0) = e.lo;
    *reinterpret_cast<u32x4*>(bt + boff1) = e.hi;
    if constexpr (!kFold) {
      if (eh == 0)
        *reinterpret_cast<float*>(smem + kOffS + (s % kBRing) * kScaleBytes + soff) = e.scale;
    }
  };
  auto expand = [&](int s, const RawW& r) { expand_write(s, expand_unpack(r)); };

  // MFMA operands of this wave's block (kb = kgrp) of one stage: one
  // register set for A and one for B, each operand reloaded in place for the
  // next stage right after its last MFMA of this stage; the block scales
  // (exact variant) are double-buffered.
  const uint32_t fchunk = ((4 * kgrp + lq) ^ ((lr >> 1) & 7)) << 4;
  const uint32_t fa_off = (wm * 64 + lr) * kRowBytes + fchunk;
  const uint32_t fb_off = (wn * 64 + lr) * kRowBytes + fchunk;
  const uint32_t fs_off = ((kgrp * 2 + wn) * 16 + lr) * 16;
  auto a_addr = [&](int s, int i) -> uint32_t {
    return (uint32_t)(kOffA + (s % kARing) * kTileBytes) + fa_off + i * 16 * kRowBytes;
  };
  auto b_addr = [&](int s, int j) -> uint32_t {
    return (uint32_t)(kOffB + (s % kBRing) * kTileBytes) + fb_off + j * 16 * kRowBytes;
  };
  auto read_sc = [&](int s) -> floatx4 {
    return *reinterpret_cast<const floatx4*>(smem + kOffS + (s % kBRing) * kScaleBytes + fs_off);
  };

  floatx4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  // Exact variant, stage s's MFMAs.  MFMA q = 4i + j; its partial is scaled in after MFMA
  // q + kLag has been issued, so the FMAs do not wait on the matrix pipe and
  // at most kLag + 2 partials are live.  The order is pinned by one empty
  // asm statement per step (the default schedule would issue all MFMAs first
  // and hold every partial at once, or scale a partial right behind its own
  // MFMA and stall): statement q comes after MFMA q (it reads partial q),
  // after the FMAs of partial q - kLag - 1 (it passes that accumulator
  // through), and before the FMAs of partial q - kLag and MFMA q + 1 (it
  // passes their operands through).  The scheduling groups then place up to
  // six VALU ops after each MFMA -- the scale FMAs plus the weight unpack.
  // A operand i is reloaded for stage `nx` right after MFMA 4i+3 and B
  // operand j right after MFMA 12+j, from one base address per tile that
  // also passes through the statements (which orders the loads); the
  // unpacked weights of stage `xs` (W words `rw`) go to LDS early.
  constexpr int kLag = 3;
  auto mma_exact = [&](half8 (&fa)[4], half8 (&fb)[4], const floatx4& sc, int nx, const RawW& rw,
                 int xs) {
    floatx4 part[16];
    uint32_t abase = a_addr(nx, 0);
    uint32_t bbase = b_addr(nx, 0);
#pragma unroll
    for (int q = 0; q < 16 + kLag; q++) {
      const int u = q - kLag;
      if (q < 16) {
        part[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[q >> 2], fb[q & 3],
                                                         floatx4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
        const int i1 = (q + 1 < 16) ? (q + 1) >> 2 : 3;
        if (u >= 1)
          asm volatile("" : "+v"(fa[i1]), "+v"(part[u]), "+v"(acc[(u - 1) >> 2][(u - 1) & 3]),
                       "+v"(abase), "+v"(bbase) : "v"(part[q]));
        else if (u == 0)
          asm volatile("" : "+v"(fa[i1]), "+v"(part[u]), "+v"(abase), "+v"(bbase)
                       : "v"(part[q]));
        else
          asm volatile("" : "+v"(fa[i1]), "+v"(abase), "+v"(bbase) : "v"(part[q]));
        if ((q & 3) == 3)
          fa[q >> 2] = *reinterpret_cast<const half8*>(smem + abase + (q >> 2) * 16 * kRowBytes);
        if (q >= 12)
          fb[q & 3] = *reinterpret_cast<const half8*>(smem + bbase + (q & 3) * 16 * kRowBytes);
      }
      if (u >= 0) {
#pragma unroll
        for (int r = 0; r < 4; r++)
          acc[u >> 2][u & 3][r] = fmaf(sc[u & 3], part[u][r], acc[u >> 2][u & 3][r]);
      }
      if (q == 2) expand_write(xs, expand_unpack(rw));
      if (q < 16) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
    }
  };

  // Folded variant, stage s's MFMAs, each accumulating into its own
  // accumulator.  A operand i is reloaded for stage `nx` after MFMA 4i+3 and
  // B operand j after MFMA 12+j (the reloads read the other ring slot, so
  // their order against the MFMAs is free); the unpacked weights of stage
  // `xs` (W words `rw`) go to LDS.  The compiler schedules all of it: asm
  // statements pinning the reloads behind their MFMAs, and scheduling groups
  // pinning three VALU ops after each MFMA, were each 1-3% slower.
  auto mma_fold = [&](half8 (&fa)[4], half8 (&fb)[4], int nx, const RawW& rw, int xs) {
    uint32_t abase = a_addr(nx, 0);
    uint32_t bbase = b_addr(nx, 0);
#pragma unroll
    for (int q = 0; q < 16; q++) {
      acc[q >> 2][q & 3] =
          __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[q >> 2], fb[q & 3], acc[q >> 2][q & 3], 0, 0, 0);
      if ((q & 3) == 3)
        fa[q >> 2] = *reinterpret_cast<const half8*>(smem + abase + (q >> 2) * 16 * kRowBytes);
      if (q >= 12)
        fb[q & 3] = *reinterpret_cast<const half8*>(smem + bbase + (q & 3) * 16 * kRowBytes);
      if (q == 2) expand_write(xs, expand_unpack(rw));

    }
  };

  // Prologue: X DMA of stages 0..3 and W reads of stages 0..3, all landed;
  // B tiles of stages 0 and 1; operands of stage 0.
  issue(0);
  issue(1);
  issue(2);
  issue(3);
  RawW r0 = raw_load(0), r1 = raw_load(1);
  RawW rwa = raw_load(2), rwb = raw_load(3);
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier"  // all of it landed
               ::: "memory");
  expand(0, r0);
  expand(1, r1);
  stage_barrier();
  half8 fa[4], fb[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    fa[i] = *reinterpret_cast<const half8*>(smem + a_addr(0, i));
    fb[i] = *reinterpret_cast<const half8*>(smem + b_addr(0, i));
  }
  floatx4 sc0 = {}, sc1 = {};
  if constexpr (!kFold) sc0 = read_sc(0);
  stage_barrier();

  // Stage s (operands of s and W words of s+2 already in registers): LDS
  // read of stage s+1's scales (exact variant); MFMAs of stage s with the
  // reloads of stage
  // s+1's operands and the unpack/writes of stage s+2's B tile woven in; X
  // DMA of stage s+4 and W read of stage s+4 (into the register slot just
  // used); then wait for everything but stage s+4's reads, and barrier.
  // Unrolled by two so the register double buffers have static names (steps
  // is even).
  // Past the end (the last two stages) the reloads and expansions run
  // anyway, on stale data into slots no later stage reads: the loop body
  // has no branches, so the scheduler keeps the reads where they are issued.
  // The stage's global reads are issued after its MFMAs (a scheduling
  // barrier keeps them there).
  for (int s = 0; s < steps; s += 2) {
    if constexpr (kFold) {
      mma_fold(fa, fb, s + 1, rwa, s + 2);
    } else {
      sc1 = read_sc(s + 1);
      mma_exact(fa, fb, sc0, s + 1, rwa, s + 2);
    }
    __builtin_amdgcn_sched_barrier(0);
    issue(s + kPrefetch);
    rwa = raw_load(s + 4);
    stage_barrier();
    if constexpr (kFold) {
      mma_fold(fa, fb, s + 2, rwb, s + 3);
    } else {
      sc0 = read_sc(s + 2);
      mma_exact(fa, fb, sc1, s + 2, rwb, s + 3);
    }
    __builtin_amdgcn_sched_barrier(0);
    issue(s + 1 + kPrefetch);
    rwb = raw_load(s + 5);
    stage_barrier();
  }
  // The trailing reads (re-loads of the last stage) land before their
  // registers and LDS slots are reused.
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");

  // K-group 1 -> LDS -> K-group 0 adds (fixed order) and stores.
  float* red = reinterpret_cast<float*>(smem + kOffA);
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
    // Output column n is scaled by D_n = 2^rowexp[n] (kFold) and row m by
    // 2^xexp[m] (both exact).  Split K: this range's sum goes to its partial
    // plane, the bias is added by the reduction.
    float* dst = a.splits > 1 ? a.part + (size_t)z * a.M * a.N : a.y;
    const float* bias = a.splits > 1 ? nullptr : a.bias;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int n = n0 + wn * 64 + 16 * j + lr;
      const bool nok = n < a.N;
      const float bv = (bias && nok) ? bias[n] : 0.0f;
      const int en = (kFold && nok) ? a.rowexp[n] : 0;
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int m = m0 + wm * 64 + 16 * i + 4 * lq + r;
          const float v = ldexpf(acc[i][j][r] + red[((wig * 64 + (i * 4 + j) * 4 + r) * 64) + lane],
                                 en + a.xexp[m]);
          if (nok && m < a.M) dst[(size_t)m * a.N + n] = v + bv;
        }
    }
  }
}

// ---------------------------------------------------------------------------
// Folded-scale GEMM on 256 x 128 tiles (q4_0_gemm_v4_kernel), for grids
// of such tiles that fill the GPU.  The same operands, layouts and
// arithmetic as q4_0_gemm_v3_kernel<true>, with every wave on a 64 x 64
// sub-tile over both blocks of a stage (32 MFMAs per stage instead of 16)
// and 256 rows of X sharing each expanded weight tile: per MFMA, half the
// barriers, half the weight expansion (VALU and LDS writes) and half the
// weight reads.
//
//  * 8 waves: wave w covers rows 64 (w >> 1) .. +63, columns 64 (w & 1) .. +63.
//  * X: LDS DMA into a 3-slot ring of 32 KB (256 rows x 64 K), two stages
//    ahead, four VMEM instructions per wave and stage; chunk c of row r at
//    c ^ ((r >> 1) & 7), as in the 128-row kernel.
//  * W: the 128-row tile's stage bytes read into registers three stages
//    ahead (one 12-byte read per thread), unpacked and scaled one stage ahead
//    into a 2-slot fp16 B ring.
//  * Stage s: block 0's operands are read from LDS right after the barrier
//    that opens the stage, block 1's during block 0's MFMAs; then stage
//    s + 1's B tile is written, the wave waits for all but its newest five
//    global reads (stage s + 2's X DMAs and stage s + 3's W words) and meets
//    the work-group at the barrier.
// ---------------------------------------------------------------------------
constexpr int kV4BM = 256;
constexpr int kV4XRing = 3;
constexpr int kV4BRing = 2;
constexpr int kV4XTile = kV4BM * kRowBytes;                   // 32 KB
constexpr int kV4OffB = kV4XRing * kV4XTile;                  // 96 KB
constexpr int kV4Lds = kV4OffB + kV4BRing * kTileBytes;       // 128 KB
static_assert(kV4Lds <= 160 * 1024, "LDS budget");

__global__ void __launch_bounds__(kThreads, 1) q4_0_gemm_v4_kernel(const Args a) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = wave >> 1;
  const int wn = wave & 1;
  const int lr = lane & 15;
  const int lq = lane >> 4;

  int tile = blockIdx.x;
  const int ntiles = a.tiles_m * a.tiles_n;
  if (a.xcd_map) tile = (tile & 7) * (ntiles >> 3) + (tile >> 3);
  const int m0 = (tile % a.tiles_m) * kV4BM;
  const int n0 = (tile / a.tiles_m) * BN;
  // This work-group's K range: stages [s0, s0 + steps) of gsteps (even
  // bounds; the ring code runs on local stage numbers, addresses use s0 + s).
  const int gsteps = a.K / BK;
  const int z = blockIdx.y;
  const int s0 = (int)((long long)gsteps * z / a.splits) & ~1;
  const int s1 = z == a.splits - 1 ? gsteps : (int)((long long)gsteps * (z + 1) / a.splits) & ~1;
  const int steps = s1 - s0;
  const size_t x_row = (size_t)a.K * 2;
  const size_t w_row = (size_t)(a.K / 32) * 18;

  // X DMA: instruction i of wave w fills rows 64 i + 8 w .. +7 (1 KB);
  // lane -> row 64 i + 8 w + (lane >> 3), slot lane & 7 = logical chunk
  // (lane & 7) ^ ((row >> 1) & 7) ((row >> 1) & 7 does not depend on i).
  const int xr = 8 * wave + (lane >> 3);
  const int xc = (lane & 7) ^ ((xr >> 1) & 7);
  const uint8_t* xsrc = a.xh + (size_t)(m0 + xr) * x_row + xc * 16;
  auto issue = [&](int s) {  // X DMA of stage min(s, steps-1) into the ring slot of s
    const int sc = s < steps ? s : steps - 1;
    uint8_t* adst = smem + (s % kV4XRing) * kV4XTile + wave * 1024;
    const uint8_t* asrc = xsrc + (size_t)(s0 + sc) * kRowBytes;
#pragma unroll
    for (int i = 0; i < 4; i++) dma16(asrc + (size_t)(64 * i) * x_row, adst + i * 8 * 1024);
  };

  // Expansion role, as in q4_0_gemm_v3_kernel: thread -> row er, block eb of
  // the stage, half eh of the block's nibbles.
  const int erk = (t >> 2) & 15;
  const int er = (t >> 6) * 16 + ((erk & 12) | ((erk & 1) << 1) | ((erk >> 1) & 1));
  const int eb = (t >> 1) & 1, eh = t & 1;
  const bool evalid = n0 + er < a.N;
  const uint32_t esel = eb ? 0x07060504u : 0x05040302u;
  const uint8_t* erow = a.w + (size_t)min(n0 + er, a.N - 1) * w_row + 16 * eb + 8 * eh;
  const uint32_t boff0 = tile_off(er, 4 * eb + 2 * eh);
  const uint32_t boff1 = tile_off(er, 4 * eb + 2 * eh + 1);
  const int eexp = evalid ? a.rowexp[n0 + er] : 0;
  using RawW = u32x3;
  auto raw_load = [&](int s) -> RawW {
    return global_load_w(erow + (size_t)(s0 + (s < steps ? s : steps - 1)) * 36);
  };
  // This thread's 16 weights of a stage as fp16 (nib - 8)·(d / D_n), and
  // their store into the stage's B ring slot.
  auto expand_regs = [&](const RawW& r, u32x4& elo, u32x4& ehi) {
    const uint32_t own = (r.x >> (eb ? 16 : 0)) & 0xFFFFu;
    const uint32_t dbits = (uint32_t)__builtin_amdgcn_mov_dpp((int)own, 0xA0, 0xF, 0xF, false);
    const _Float16 h = evalid ? (_Float16)ldexpf(f16_bits_to_f32(dbits), -eexp) : (_Float16)0.0f;
    const half2v hh = {h, h};
    const u32x4 lo = unpack8(__builtin_amdgcn_perm(r.y, r.x, esel));
    const u32x4 hi = unpack8(__builtin_amdgcn_perm(r.z, r.y, esel));
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t wl = lo[i], wh = hi[i];
      elo[i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, wl) * hh);
      ehi[i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, wh) * hh);
    }
  };
  auto expand_store = [&](int s, const u32x4& elo, const u32x4& ehi) {
    uint8_t* bt = smem + kV4OffB + (s % kV4BRing) * kTileBytes;
    *reinterpret_cast<u32x4*>(bt + boff0) = elo;
    *reinterpret_cast<u32x4*>(bt + boff1) = ehi;
  };

  // MFMA operands of block kb of stage s.
  auto load_ops = [&](int s, int kb, half8 (&fa)[4], half8 (&fb)[4]) {
    const uint32_t chunk = ((4 * kb + lq) ^ ((lr >> 1) & 7)) << 4;
    const uint8_t* xt = smem + (s % kV4XRing) * kV4XTile + (wm * 64 + lr) * kRowBytes + chunk;
    const uint8_t* wt = smem + kV4OffB + (s % kV4BRing) * kTileBytes + (wn * 64 + lr) * kRowBytes +
                        chunk;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      fa[i] = *reinterpret_cast<const half8*>(xt + i * 16 * kRowBytes);
      fb[i] = *reinterpret_cast<const half8*>(wt + i * 16 * kRowBytes);
    }
  };

  floatx4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  auto mma = [&](const half8 (&fa)[4], const half8 (&fb)[4]) {
#pragma unroll
    for (int q = 0; q < 16; q++)
      acc[q >> 2][q & 3] =
          __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[q >> 2], fb[q & 3], acc[q >> 2][q & 3], 0, 0, 0);
  };

  // Prologue: X of stages 0 and 1 and the W words of stages 0 and 1 landed,
  // stage 0's B tile written, stage 2's W words in flight.
  issue(0);
  issue(1);
  RawW r0 = raw_load(0), ra = raw_load(1);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  {
    u32x4 elo, ehi;
    expand_regs(r0, elo, ehi);
    expand_store(0, elo, ehi);
  }
  RawW rb = raw_load(2);
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

  // Stage s.  At its top (just past the barrier): X of s and s+1 landed, B
  // tile of s visible, the W words of s+1 in registers (landed) and those of
  // s+2 issued one stage earlier.
  //  - operand reads of both blocks of s, with stage s+1's weights unpacked
  //    between them (VALU work that hides the reads' latency; a scheduling
  //    barrier keeps the MFMAs after it);
  //  - block 0's MFMAs, then the B tile of s+1 stored (into the slot of
  //    s-1) and the X DMA of stage s+2 issued (into the slot of s-1: every
  //    wave finished reading stage s-1's operands before the barrier), then
  //    block 1's MFMAs;
  //  - the W words of s+3 into the registers just expanded;
  //  - wait for all but this stage's five reads (so X of s+1 and the W words
  //    of s+2 have landed; those registers pass through the statement, so
  //    nothing reads them before it) and for the LDS writes; barrier.
  // Unrolled by two so the W registers keep static names: a register that a
  // read issued from asm is still filling is never copied (steps is even).
  auto stage = [&](int s, RawW& rx) {
    half8 fa0[4], fb0[4], fa1[4], fb1[4];
    u32x4 elo, ehi;
    load_ops(s, 0, fa0, fb0);
    expand_regs(rx, elo, ehi);
    load_ops(s, 1, fa1, fb1);
    __builtin_amdgcn_sched_barrier(0);
    mma(fa0, fb0);
    expand_store(s + 1, elo, ehi);
    issue(s + 2);
    mma(fa1, fb1);
    rx = raw_load(s + 3);
  };
  for (int s = 0; s < steps; s += 2) {
    stage(s, ra);
    asm volatile("s_waitcnt vmcnt(5) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    stage(s + 1, rb);
    asm volatile("s_waitcnt vmcnt(5) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  }
  // The trailing reads (re-reads of the last stage) land before the
  // work-group's LDS is released.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // Output column n scaled by D_n = 2^rowexp[n], row m by 2^xexp[m] (exact).
  // Split K: this range's sum goes to its partial plane, the bias is added
  // by the reduction.
  float* dst = a.splits > 1 ? a.part + (size_t)z * a.M * a.N : a.y;
  const float* bias = a.splits > 1 ? nullptr : a.bias;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int n = n0 + wn * 64 + 16 * j + lr;
    const bool nok = n < a.N;
    const float bv = (bias && nok) ? bias[n] : 0.0f;
    const int en = nok ? a.rowexp[n] : 0;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int m = m0 + wm * 64 + 16 * i + 4 * lq + r;
        if (nok && m < a.M) dst[(size_t)m * a.N + n] = ldexpf(acc[i][j][r], en + a.xexp[m]) + bv;
      }
  }
}

// Y = sum of the K-split partial planes in split order (+ bias): a fixed
// order, so results do not depend on which work-group finished first.
__global__ void __launch_bounds__(256)
split_k_reduce_kernel(float* __restrict__ y, const float* __restrict__ part,
                      const float* __restrict__ bias, size_t mn, int n, int splits) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= mn) return;
  float v = part[i];
  for (int z = 1; z < splits; z++) v += part[(size_t)z * mn + i];
  y[i] = v + (bias ? bias[i % n] : 0.0f);
}

// ---------------------------------------------------------------------------
// FP16 weights: Y[M][N] = X[M][K] . W[N][K]^T with W fp16 (kernels.rs:571-586
// per token).  No per-block scale, so the MFMAs accumulate straight into
// their accumulators; at the BASELINE sizes (lm_head, M = 128: 2 bytes per
// weight against 256 flop) the kernel is bound by the weight stream, so it
// keeps many bytes in flight: a 128 x 64 NW tile per work-group of 2 NW
// waves (64 x 64 each), stages of 64 K, and an LDS ring fed by DMA, W
// non-temporal (read once), X cached (shared by all N tiles).  Both tiles use
// the layout of the Q4_0 kernel's X tile (chunk c of row r in slot
// c ^ ((r >> 1) & 7)), so the operand reads of 16 rows hit 16 bank groups.
// Geometry: NW waves along N (BN = 64 NW), two along M (128 rows).
template <int NW>
struct F16Geom {
  static constexpr int kWaves = 2 * NW;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kBN = 64 * NW;
  static constexpr int kXBytes = kTileBytes;            // 128 rows x 128 bytes
  static constexpr int kWBytes = kBN * kRowBytes;
  static constexpr int kSlot = kXBytes + kWBytes;
  static constexpr int kRing = NW == 2 ? 4 : 3;
  static constexpr int kLds = kRing * kSlot;           // 128 KB / 144 KB
  static constexpr int kXDma = kXBytes / 1024 / kWaves;  // per wave and stage
  static constexpr int kWDma = kWBytes / 1024 / kWaves;
  static_assert(kLds <= 160 * 1024, "LDS budget");
};
constexpr int kF16NW = 4;  // 128 x 256 tiles

struct F16Args {
  float* y;
  const uint8_t* w;   // fp16 [N][K]
  const uint8_t* xh;  // fp16 [Mp][K]
  const float* bias;
  int M, N, K;
  int tiles_m, tiles_n;
  int xcd_map;
  int splits;
  float* part;
  const float* colscale;  // optional: output column n multiplied by colscale[n]
  const int* xexp;        // [Mp]: row m of xh holds X row m times 2^-xexp[m]
  uint32_t w_bytes, xh_bytes, xe_bytes;  // buffer ranges (streaming kernel)
};

__device__ __forceinline__ void dma16_nt(const void* src, uint8_t* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds_wave_base,
                                   16, 0, 2);
}

template <int NW>
__global__ void __launch_bounds__(F16Geom<NW>::kThreads, 1) f16_gemm_v2_kernel(const F16Args a) {
  using G = F16Geom<NW>;
  extern __shared__ __align__(16) uint8_t smem[];
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = wave / NW, wn = wave % NW;
  const int lr = lane & 15, lq = lane >> 4;

  int tile = blockIdx.x;
  const int ntiles = a.tiles_m * a.tiles_n;
  if (a.xcd_map) tile = (tile & 7) * (ntiles >> 3) + (tile >> 3);
  const int m0 = (tile % a.tiles_m) * BM;
  const int n0 = (tile / a.tiles_m) * G::kBN;
  const int gsteps = a.K / BK;
  const int z = blockIdx.y;
  const int s0 = (int)((long long)gsteps * z / a.splits);
  const int steps = (int)((long long)gsteps * (z + 1) / a.splits) - s0;
  const size_t row_bytes = (size_t)a.K * 2;

  // DMA i of a tile fills rows 8 (kWaves i + wave) .. + 7: lane -> row
  // 8 (kWaves i + wave) + (lane >> 3), slot lane & 7 holding logical chunk
  // (lane & 7) ^ ((row >> 1) & 7) ((row >> 1) & 7 does not depend on i).
  const int dr = 8 * wave + (lane >> 3);
  const int dc = (lane & 7) ^ ((dr >> 1) & 7);
  const uint8_t* xsrc = a.xh + (size_t)(m0 + dr) * row_bytes + dc * 16;
  const uint8_t* wsrc[G::kWDma];
#pragma unroll
  for (int i = 0; i < G::kWDma; i++)
    wsrc[i] = a.w + (size_t)min(n0 + 8 * G::kWaves * i + dr, a.N - 1) * row_bytes + dc * 16;
  auto issue = [&](int s) {  // stage min(s, steps - 1) into ring slot s % kRing
    const int sc = s < steps ? s : steps - 1;
    const size_t koff = (size_t)(s0 + sc) * kRowBytes;
    uint8_t* slot = smem + (s % G::kRing) * G::kSlot + wave * 1024;
#pragma unroll
    for (int i = 0; i < G::kXDma; i++)
      dma16(xsrc + (size_t)8 * G::kWaves * i * row_bytes + koff, slot + i * 1024 * G::kWaves);
#pragma unroll
    for (int i = 0; i < G::kWDma; i++)
      dma16_nt(wsrc[i] + koff, slot + G::kXBytes + i * 1024 * G::kWaves);
  };

  floatx4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  for (int s = 0; s < G::kRing - 1; s++) issue(s);
  for (int s = 0; s < steps; s++) {
    // stage s landed (all but the newest kRing - 2 stages), everyone done
    // with stage s - 1, whose slot the next request reuses
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier"
                 : : "n"((G::kXDma + G::kWDma) * (G::kRing - 2)) : "memory");
    issue(s + G::kRing - 1);
    const uint8_t* xt = smem + (s % G::kRing) * G::kSlot;
    const uint8_t* wt = xt + G::kXBytes;
#pragma unroll
    for (int kh = 0; kh < 2; kh++) {
      half8 fa[4], fb[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        fa[i] = *reinterpret_cast<const half8*>(xt + tile_off(wm * 64 + 16 * i + lr, 4 * kh + lq));
        fb[i] = *reinterpret_cast<const half8*>(wt + tile_off(wn * 64 + 16 * i + lr, 4 * kh + lq));
      }
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" : : : "memory");  // trailing re-loads landed

  // acc[i][j][r]: row m0 + wm 64 + 16 i + 4 lq + r, column n0 + wn 64 + 16 j + lr
  float* out = a.splits > 1 ? a.part + (size_t)z * a.M * a.N : a.y;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int n = n0 + wn * 64 + 16 * j + lr;
    if (n >= a.N) continue;
    const float bv = (a.splits == 1 && a.bias) ? a.bias[n] : 0.0f;
    const float cs = a.colscale ? a.colscale[n] : 1.0f;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int m = m0 + wm * 64 + 16 * i + 4 * lq + r;
        if (m < a.M) out[(size_t)m * a.N + n] = ldexpf(acc[i][j][r], a.xexp[m]) * cs + bv;
      }
  }
}

// ---------------------------------------------------------------------------
// FP16 weights, up to 128 tokens: the weight stream is the bound (2 bytes per
// weight against 2 M flop), so W never passes through LDS and no barrier
// waits on it.  A work-group of NW waves (8 or 16) owns 32 NW columns of W
// (wave w: columns 32 w .. 32 w + 31, two MFMA column tiles) and all 16 MT
// rows of X;
// K streams in stages of 64.  Each wave loads its 32 rows' 128-byte stage
// segments straight from HBM into registers (non-temporal: read once), P
// stages ahead, as whole lines: 8 rows x 128 bytes per instruction (reading
// the MFMA operand shape directly, 16 rows x 64 bytes per instruction, ran
// the weight stream 20-25% slower); at its use the wave passes the stage
// through its own LDS area (swizzled rows, no barrier: a wave's LDS accesses
// run in order) into MFMA B operands.  X (16 MT rows x 128 bytes a stage,
// shared by the 8 waves) moves in groups of P stages: a group is loaded
// into registers one group ahead and written into one half of a 2 P-slot
// LDS ring while the other half is read; one barrier per group orders those
// writes and reads (it waits on LDS only; one per stage held every wave to
// the slowest wave's weights, stage by stage).  Every wait on a global read
// is the compiler's own, before the register's first use: with stage j's W
// issued P stages before its use, the P later stages stay in flight.  The
// loads are buffer loads issued
// on every iteration (stages past the range aim past the buffer and read
// zeros without touching memory), so the count of reads in flight is the
// same on every path and the compiler's waits stay exact.
constexpr uint32_t kFsOob = 0xFFFFFFF0u;  // an offset past every buffer range

// Hi/lo rows for the streaming kernel at 2..15 tokens: token r < M becomes
// hi = fp16(x 2^sh) in row r and lo = fp16(x 2^sh - hi) in row 16 + r (sh as
// in x_row_to_f16: the row's largest |x| 2^sh lies in [2^14, 2^15); 0 for a
// zero row or one holding inf or NaN), xexp[r] = -sh; rows r >= M are zero.
// hi + lo is x 2^sh to about 2^-22 of the row's largest value and its
// products with fp16 weights are exact in fp32, so the sum of the two rows'
// dot products is as accurate as an fp32 GEMV (where hi is not finite, lo is
// 0: the product keeps its inf or NaN).  One 256-thread work-group per hi
// row (16); natural column order; x 16-byte aligned, K % 8 == 0.
__global__ void __launch_bounds__(256)
x_rows_hilo_kernel(u32x4* __restrict__ xh, int* __restrict__ xexp, const float* __restrict__ x,
                   int M, int K) {
  __shared__ uint32_t red[4];
  const int r = blockIdx.x, t = threadIdx.x, groups = K / 8;
  u32x4* hi = xh + (size_t)r * groups;
  u32x4* lo = xh + (size_t)(16 + r) * groups;
  if (r >= M) {
    for (int g = t; g < groups; g += 256) hi[g] = lo[g] = u32x4{0u, 0u, 0u, 0u};
    if (t == 0) xexp[r] = 0;
    return;
  }
  const float4* src = reinterpret_cast<const float4*>(x + (size_t)r * K);
  uint32_t mb = 0;  // largest |x| by bit pattern (inf and NaN above every finite value)
  for (int g = t; g < groups; g += 256) {
    const float4 a = src[2 * g], b = src[2 * g + 1];
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int i = 0; i < 8; i++) mb = max(mb, __float_as_uint(v[i]) & 0x7FFFFFFFu);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mb = max(mb, (uint32_t)__shfl_xor((int)mb, off, 64));
  if ((t & 63) == 0) red[t >> 6] = mb;
  __syncthreads();
  mb = max(max(red[0], red[1]), max(red[2], red[3]));
  const float amax = __uint_as_float(mb);
  int sh = 0;
  if (amax > 0.0f && amax < __builtin_inff()) sh = 15 - __builtin_amdgcn_frexp_expf(amax);
  for (int g = t; g < groups; g += 256) {
    const float4 a = src[2 * g], b = src[2 * g + 1];
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    u32x4 h, l;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float p = ldexpf(v[2 * j], sh), q = ldexpf(v[2 * j + 1], sh);
      const _Float16 ph = (_Float16)p, qh = (_Float16)q;
      const float pl = __builtin_isfinite((float)ph) ? p - (float)ph : 0.0f;
      const float ql = __builtin_isfinite((float)qh) ? q - (float)qh : 0.0f;
      h[j] = (uint32_t)__builtin_bit_cast(uint16_t, ph) |
             ((uint32_t)__builtin_bit_cast(uint16_t, qh) << 16);
      l[j] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)pl) |
             ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)ql) << 16);
    }
    hi[g] = h;
    lo[g] = l;
  }
  if (t == 0) xexp[r] = -sh;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t fs_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// HL: rows 0..15 hold the tokens' hi rows and 16..31 their lo rows (MT = 2);
// token t's output is the sum of rows t and 16 + t.
template <int MT, int P, bool HL, int NW>
__global__ void __launch_bounds__(64 * NW, 1) f16_gemm_stream_kernel(const F16Args a) {
  static_assert(!HL || MT == 2, "hi/lo rows: two row tiles");
  constexpr int kRows = 16 * MT;
  constexpr int kSlotBytes = kRows * kRowBytes;  // one X stage
  constexpr int kChunks = kRows * 8;             // its 16-byte chunks
  constexpr int kThr = 64 * NW;
  constexpr int kXPer = (kChunks + kThr - 1) / kThr;  // per thread
  extern __shared__ __align__(16) uint8_t xs[];  // X ring (2 P slots), then the W areas
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int lr = lane & 15, lq = lane >> 4;
  const int n0 = blockIdx.x * 32 * NW + 32 * wave;
  const int gsteps = a.K / BK;
  const int z = blockIdx.y;
  const int s0 = (int)((long long)gsteps * z / a.splits);
  const int steps = (int)((long long)gsteps * (z + 1) / a.splits) - s0;
  const uint32_t row_bytes = (uint32_t)a.K * 2;
  // W read i of a stage: row n0 + 8 i + (lane >> 3) (past N: row N - 1,
  // never stored), 16-byte piece lane & 7 of its 128-byte segment; it lands
  // in the wave's LDS area at tile_off(8 i + (lane >> 3), lane & 7)
  const __amdgpu_buffer_rsrc_t wrs = fs_rsrc(a.w, a.w_bytes);
  uint8_t* wl = xs + 2 * P * kSlotBytes + wave * 32 * kRowBytes;
  uint32_t wo[4], wlo[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int r = 8 * i + (lane >> 3);
    wo[i] = (uint32_t)min(n0 + r, a.N - 1) * row_bytes + (uint32_t)s0 * kRowBytes +
            16 * (lane & 7);
    wlo[i] = tile_off(r, lane & 7);
  }
  // X chunk q = t + 512 i of a stage: row q >> 3, chunk q & 7 (threads past
  // the chunks read zeros and store nothing)
  const __amdgpu_buffer_rsrc_t xrs = fs_rsrc(a.xh, a.xh_bytes);
  uint32_t xg[kXPer], xo[kXPer];
  bool xv[kXPer];
#pragma unroll
  for (int i = 0; i < kXPer; i++) {
    const int q = t + kThr * i;
    xv[i] = q < kChunks;
    const int row = xv[i] ? q >> 3 : 0;
    xg[i] = xv[i] ? (uint32_t)row * row_bytes + (uint32_t)s0 * kRowBytes + 16 * (q & 7) : kFsOob;
    xo[i] = tile_off(row, q & 7);
  }
  u32x4 wr[P][4];
  u32x4 xr[P][kXPer];
  auto load_w = [&](int s, u32x4(&d)[4]) {  // non-temporal: read once
    const bool in = s < steps;
#pragma unroll
    for (int i = 0; i < 4; i++)
      d[i] = __builtin_amdgcn_raw_buffer_load_b128(
          wrs, in ? wo[i] + (uint32_t)s * kRowBytes : kFsOob, 0, 2);
  };
  auto load_x = [&](int s, u32x4(&d)[kXPer]) {
    const bool in = s < steps;
#pragma unroll
    for (int i = 0; i < kXPer; i++)
      d[i] = __builtin_amdgcn_raw_buffer_load_b128(
          xrs, in && xv[i] ? xg[i] + (uint32_t)s * kRowBytes : kFsOob, 0, 0);
  };
  // Threads past the chunks store their zeros into their wave's W area,
  // which compute() rewrites before reading (no branch around the stores).
  auto store_x = [&](int slot, const u32x4(&d)[kXPer]) {
#pragma unroll
    for (int i = 0; i < kXPer; i++) {
      uint8_t* dst = xv[i] ? xs + slot * kSlotBytes + xo[i] : wl + 16 * lane;
      *reinterpret_cast<u32x4*>(dst) = d[i];
    }
  };
  auto barrier = [&]() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" : : : "memory"); };

  floatx4 acc[MT][2];
#pragma unroll
  for (int i = 0; i < MT; i++)
#pragma unroll
    for (int c = 0; c < 2; c++) acc[i][c] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  auto compute = [&](int slot, const u32x4(&w)[4]) {
    const uint8_t* xt = xs + slot * kSlotBytes;
#pragma unroll
    for (int i = 0; i < 4; i++) *reinterpret_cast<u32x4*>(wl + wlo[i]) = w[i];
    // B operand of column tile c: row 16 c + lr, K 32 kh + 8 lq
    half8 bw[2][2];
#pragma unroll
    for (int c = 0; c < 2; c++)
#pragma unroll
      for (int kh = 0; kh < 2; kh++)
        bw[c][kh] = *reinterpret_cast<const half8*>(wl + tile_off(16 * c + lr, 4 * kh + lq));
#pragma unroll
    for (int kh = 0; kh < 2; kh++) {
      const half8 b0 = bw[0][kh];
      const half8 b1 = bw[1][kh];
#pragma unroll
      for (int i = 0; i < MT; i++) {
        const half8 av = *reinterpret_cast<const half8*>(xt + tile_off(16 * i + lr, 4 * kh + lq));
        acc[i][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, b0, acc[i][0], 0, 0, 0);
        acc[i][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, b1, acc[i][1], 0, 0, 0);
      }
    }
  };

  // Stage j's W in wr[j % P], its X in xr[j % P] until written to slot j & 1.
  // Group g: X in ring half g & 1 (slots P (g & 1) + u), W of stage j in
  // wr[j % P].  The prologue ends in the loop's own issue order (the next
  // group's X, then W stage by stage), so the loop's waits hold from its
  // start; group 0's X comes first, into registers of its own.
  {
    u32x4 x0[P][kXPer];
#pragma unroll
    for (int u = 0; u < P; u++) load_x(u, x0[u]);
#pragma unroll
    for (int u = 0; u < P; u++) load_x(P + u, xr[u]);
#pragma unroll
    for (int u = 0; u < P; u++) load_w(u, wr[u]);
#pragma unroll
    for (int u = 0; u < P; u++) store_x(u, x0[u]);
  }
  barrier();
  // Whole groups (no exit inside the unrolled group, so every path has the
  // same reads in flight): stages past the range multiply zero X by zero W.
  const int groups = (steps + P - 1) / P;
  for (int g = 0; g < groups; g++) {
    const int h = g & 1;
#pragma unroll
    for (int u = 0; u < P; u++) store_x(P * (1 - h) + u, xr[u]);  // group g + 1
#pragma unroll
    for (int u = 0; u < P; u++) load_x(P * (g + 2) + u, xr[u]);
    // the reads go out where they stand (the scheduler would sink them to
    // the group's end, and the next group's first wait would then drain them)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < P; u++) {
      const int s = P * g + u;
      compute(P * h + u, wr[u]);
      load_w(s + P, wr[u]);
      __builtin_amdgcn_sched_barrier(0);
    }
    barrier();
  }

  // acc[i][c][r]: row 16 i + 4 lq + r, column n0 + 16 c + lr.  The row
  // exponents, bias and column scales are read together before any store.
  const __amdgpu_buffer_rsrc_t ers = fs_rsrc(a.xexp, a.xe_bytes);
  u32x4 ex[MT];
#pragma unroll
  for (int i = 0; i < MT; i++)
    ex[i] = __builtin_amdgcn_raw_buffer_load_b128(ers, (uint32_t)(16 * i + 4 * lq) * 4u, 0, 0);
  float bv[2], cs[2];
#pragma unroll
  for (int c = 0; c < 2; c++) {
    const int n = min(n0 + 16 * c + lr, a.N - 1);
    bv[c] = (a.splits == 1 && a.bias) ? a.bias[n] : 0.0f;
    cs[c] = a.colscale ? a.colscale[n] : 1.0f;
  }
  float* out = a.splits > 1 ? a.part + (size_t)z * a.M * a.N : a.y;
  if constexpr (HL) {
#pragma unroll
    for (int c = 0; c < 2; c++) {
      const int n = n0 + 16 * c + lr;
      if (n >= a.N) continue;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int m = 4 * lq + r;
        if (m < a.M)
          out[(size_t)m * a.N + n] =
              ldexpf(acc[0][c][r] + acc[1][c][r], (int)ex[0][r]) * cs[c] + bv[c];
      }
    }
    return;
  }
#pragma unroll
  for (int c = 0; c < 2; c++) {
    const int n = n0 + 16 * c + lr;
    if (n >= a.N) continue;
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int m = 16 * i + 4 * lq + r;
        if (m < a.M)
          out[(size_t)m * a.N + n] = ldexpf(acc[i][c][r], (int)ex[i][r]) * cs[c] + bv[c];
      }
  }
}

// K splits: when the tile grid leaves CUs idle, each tile's K range is cut
// into `splits` pieces (each at least kMinSplitStages stages) so the grid
// nearly fills the chip.
constexpr int kMinSplitStages = 8;
int pick_splits(size_t tiles, size_t m, int num_cus) {
  const size_t stages = m / BK;
  if (tiles == 0) return 1;
  if (tiles * 4 >= (size_t)num_cus * 3) return 1;
  size_t s = (size_t)num_cus / tiles;
  if (s > stages / kMinSplitStages) s = stages / kMinSplitStages;
  return s < 2 ? 1 : (int)s;
}

size_t round256(size_t v) { return (v + 255) / 256 * 256; }

}  // namespace

// Workspace of the Q4_0 GEMM: fp16 X, then the K-split partial planes (if
// any), then the row exponents.
size_t gemm_v3_workspace_bytes(size_t batch, size_t n, size_t m, int num_cus) {
  const size_t tiles = ((n + BN - 1) / BN) * ((batch + BM - 1) / BM);
  const size_t mp = (batch + BM - 1) / BM * BM;
  const size_t tiles4 = ((n + BN - 1) / BN) * ((mp + kV4BM - 1) / kV4BM);
  const int splits = std::max(pick_splits(tiles, m, num_cus), pick_splits(tiles4, m, num_cus));
  const size_t xb = round256(gemm_workspace_bytes(batch, m));
  const size_t pb = splits > 1 ? round256((size_t)splits * batch * n * 4) : 0;
  return xb + pb + round256(n * 4);
}

bool q4_0_gemm_v3_ok(const uint8_t* w, size_t w_len, size_t n, size_t m, size_t batch) {
  if (m == 0 || m % 256 != 0 || n == 0 || batch == 0) return false;
  if (((uintptr_t)w & 15) != 0) return false;
  if (n > (size_t)0x7FFFFFFF || m > (size_t)0x7FFFFFF || batch > (size_t)0x7FFFFFFF) return false;
  const size_t tiles = ((n + BN - 1) / BN) * ((batch + BM - 1) / BM);
  if (tiles > (size_t)0x7FFFFFFF) return false;
  return w_len / kBlockBytes >= n * (m / kBlockElems);
}

size_t f16_gemm_v2_workspace_bytes(size_t batch, size_t n, size_t m, int num_cus) {
  const size_t tiles = ((n + F16Geom<kF16NW>::kBN - 1) / F16Geom<kF16NW>::kBN) *
                       ((batch + BM - 1) / BM);
  const int splits = pick_splits(tiles, m, num_cus);
  const size_t xb = round256(gemm_workspace_bytes(batch, m));
  return splits > 1 ? xb + (size_t)splits * batch * n * 4 : xb;
}

bool f16_gemm_v2_ok(const uint8_t* w, size_t n, size_t m, size_t batch) {
  if (m == 0 || m % BK != 0 || n == 0 || batch == 0) return false;
  if (((uintptr_t)w & 15) != 0) return false;
  if (n > (size_t)0x7FFFFFFF || m > (size_t)0x7FFFFFF || batch > (size_t)0x7FFFFFFF) return false;
  const size_t tiles = ((n + BN - 1) / BN) * ((batch + BM - 1) / BM);
  return tiles <= (size_t)0x7FFFFFFF;
}

hipError_t launch_f16_gemm_v2(float* y, const uint8_t* w, const float* x, const float* bias,
                              size_t n, size_t m, size_t batch, void* ws, int num_cus,
                              hipStream_t s, const float* colscale) {
  using G = F16Geom<kF16NW>;
  hipError_t e = launch_x_f16_plain(x, batch, m, ws, s);
  if (e != hipSuccess) return e;
  e = set_lds_limit(reinterpret_cast<const void*>(f16_gemm_v2_kernel<kF16NW>), G::kLds);
  if (e != hipSuccess) return e;
  F16Args a;
  a.y = y;
  a.w = w;
  a.xh = static_cast<const uint8_t*>(ws);
  a.bias = bias;
  a.M = (int)batch;
  a.N = (int)n;
  a.K = (int)m;
  a.tiles_m = (int)((batch + BM - 1) / BM);
  a.tiles_n = (int)((n + G::kBN - 1) / G::kBN);
  const int tiles = a.tiles_m * a.tiles_n;
  a.xcd_map = (tiles % 8) == 0 ? 1 : 0;
  a.splits = pick_splits((size_t)tiles, m, num_cus);
  a.part = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) +
                                    round256(gemm_workspace_bytes(batch, m)));
  a.colscale = colscale;
  a.xexp = gemm_x_exponents(ws, batch, m);
  hipLaunchKernelGGL(f16_gemm_v2_kernel<kF16NW>, dim3(tiles, a.splits), dim3(G::kThreads), G::kLds,
                     s, a);
  e = hipGetLastError();
  if (e != hipSuccess || a.splits == 1) return e;
  const size_t mn = batch * n;
  hipLaunchKernelGGL(split_k_reduce_kernel, dim3((unsigned)((mn + 255) / 256)), dim3(256), 0, s, y,
                     a.part, bias, mn, (int)n, a.splits);
  return hipGetLastError();
}

// The streaming FP16 GEMM (2..128 tokens; hi/lo rows below 16): same
// workspace layout as the DMA-fed kernel (fp16 X rows, exponents, K-split
// planes over 256-column tiles).
namespace {
constexpr int kFsP = 4;  // stages of W and X in registers ahead of their use
// Waves per work-group (32 columns each): as many as the tile height leaves
// registers for — 16 up to 32 tokens (four waves per SIMD), 12 up to 64
// (three) — where those wider tiles alone cover three quarters of the CUs;
// else 8.  More reads in flight per CU: lm_head at 4-32 tokens 160-167 us
// per call with 16 against 212-247 with 8, at 48-64 tokens 226-231 with 12
// against 240-244 (16 waves there spill registers: 326 us); on the Mistral
// shapes the wider tiles leave too few work-groups (10-30% slower).
int f16_stream_waves(size_t n, size_t batch, int num_cus) {
  const int nw = batch <= 32 ? 16 : batch <= 64 ? 12 : 8;
  const size_t bn = 32 * (size_t)nw;
  return (n + bn - 1) / bn * 4 >= (size_t)num_cus * 3 ? nw : 8;
}
int f16_stream_splits(size_t n, size_t m, size_t batch, int num_cus) {
  const size_t bn = 32 * (size_t)f16_stream_waves(n, batch, num_cus);
  return pick_splits((n + bn - 1) / bn, m, num_cus);
}
template <int MT, bool HL, int NW>
hipError_t launch_fs_w(const F16Args& a, dim3 grid, hipStream_t s) {
  constexpr int lds = 2 * kFsP * 16 * MT * kRowBytes + NW * 32 * kRowBytes;
  static_assert(lds <= 160 * 1024, "LDS budget");
  const void* k = reinterpret_cast<const void*>(f16_gemm_stream_kernel<MT, kFsP, HL, NW>);
  hipError_t e = set_lds_limit(k, lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((f16_gemm_stream_kernel<MT, kFsP, HL, NW>), grid, dim3(64 * NW), lds, s, a);
  return hipGetLastError();
}
template <int MT, bool HL = false>
hipError_t launch_fs(const F16Args& a, int nw, dim3 grid, hipStream_t s) {
  if constexpr (MT <= 2)
    if (nw == 16) return launch_fs_w<MT, HL, 16>(a, grid, s);
  if constexpr (MT == 4)
    if (nw == 12) return launch_fs_w<MT, HL, 12>(a, grid, s);
  return launch_fs_w<MT, HL, 8>(a, grid, s);
}
}  // namespace

bool f16_gemm_stream_ok(const uint8_t* w, const float* x, size_t n, size_t m, size_t batch) {
  if (batch < 2 || batch > 128 || m == 0 || m % BK != 0 || n == 0) return false;
  if (((uintptr_t)w & 15) != 0) return false;
  if (batch < 16 && ((uintptr_t)x & 15) != 0) return false;  // the hi/lo pre-pass reads float4
  // 32-bit buffer offsets, with kFsOob past every valid one
  return n <= (size_t)0x7FFFFFFF && m <= (size_t)0x7FFFFFF && 2 * n * m <= 0xFFFFFF00ull &&
         (size_t)128 * m * 2 <= 0xFFFFFF00ull;
}

size_t f16_gemm_stream_workspace_bytes(size_t batch, size_t n, size_t m, int num_cus) {
  const int splits = f16_stream_splits(n, m, batch, num_cus);
  const size_t xb = round256(gemm_workspace_bytes(batch, m));
  return splits > 1 ? xb + (size_t)splits * batch * n * 4 : xb;
}

hipError_t launch_f16_gemm_stream(float* y, const uint8_t* w, const float* x, const float* bias,
                                  size_t n, size_t m, size_t batch, void* ws, int num_cus,
                                  hipStream_t s, const float* colscale) {
  hipError_t e;
  if (batch < 16) {
    hipLaunchKernelGGL(x_rows_hilo_kernel, dim3(16), dim3(256), 0, s, static_cast<u32x4*>(ws),
                       gemm_x_exponents(ws, batch, m), x, (int)batch, (int)m);
    e = hipGetLastError();
  } else {
    e = launch_x_f16_plain(x, batch, m, ws, s);
  }
  if (e != hipSuccess) return e;
  F16Args a{};
  a.y = y;
  a.w = w;
  a.xh = static_cast<const uint8_t*>(ws);
  a.bias = bias;
  a.M = (int)batch;
  a.N = (int)n;
  a.K = (int)m;
  const int nw = f16_stream_waves(n, batch, num_cus);
  a.splits = f16_stream_splits(n, m, batch, num_cus);
  a.part = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) +
                                    round256(gemm_workspace_bytes(batch, m)));
  a.colscale = colscale;
  a.xexp = gemm_x_exponents(ws, batch, m);
  const size_t mp = (batch + 127) / 128 * 128;  // the pre-pass's padded rows
  a.w_bytes = (uint32_t)(2 * n * m);
  a.xh_bytes = (uint32_t)(mp * m * 2);
  a.xe_bytes = (uint32_t)(mp * 4);
  const size_t bn = 32 * (size_t)nw;
  const dim3 grid((unsigned)((n + bn - 1) / bn), (unsigned)a.splits);
  if (batch < 16)
    e = launch_fs<2, true>(a, nw, grid, s);
  else if (batch == 16)
    e = launch_fs<1>(a, nw, grid, s);
  else if (batch <= 32)
    e = launch_fs<2>(a, nw, grid, s);
  else if (batch <= 64)
    e = launch_fs<4>(a, nw, grid, s);
  else
    e = launch_fs<8>(a, nw, grid, s);
  if (e != hipSuccess || a.splits == 1) return e;
  const size_t mn = batch * n;
  hipLaunchKernelGGL(split_k_reduce_kernel, dim3((unsigned)((mn + 255) / 256)), dim3(256), 0, s, y,
                     a.part, bias, mn, (int)n, a.splits);
  return hipGetLastError();
}

hipError_t launch_q4_0_gemm_v3(float* y, const uint8_t* w, const float* x, const float* bias,
                               size_t n, size_t m, size_t batch, void* ws, int num_cus,
                               hipStream_t s) {
  hipError_t e;
  for (const void* k : {reinterpret_cast<const void*>(q4_0_gemm_v3_kernel<true>),
                        reinterpret_cast<const void*>(q4_0_gemm_v3_kernel<false>)}) {
    e = set_lds_limit(k, kLdsBytes);
    if (e != hipSuccess) return e;
  }
  const size_t wbytes = n * (m / kBlockElems) * kBlockBytes;
  const bool fold = gemm_folded() &&
                    (batch >= kFoldMinBatch ||
                     (batch >= kFoldMinBatchSmallW && wbytes <= kFoldSmallWBytes));
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
  a.splits = pick_splits((size_t)tiles, m, num_cus);
  a.part = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) +
                                    round256(gemm_workspace_bytes(batch, m)));
  int* rowexp = reinterpret_cast<int*>(
      static_cast<uint8_t*>(ws) + gemm_v3_workspace_bytes(batch, n, m, num_cus) - round256(n * 4));
  a.rowexp = rowexp;
  a.xexp = gemm_x_exponents(ws, batch, m);
  if (fold) {
    const size_t mp = (batch + BM - 1) / BM * BM;
    hipLaunchKernelGGL(q4_0_prepass_kernel, dim3((unsigned)mp + (unsigned)((n + 3) / 4)),
                       dim3(256), 0, s, static_cast<u32x4*>(ws), gemm_x_exponents(ws, batch, m), x,
                       (int)batch, (int)mp, (int)m, rowexp, w, (int)n);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    // 256-row tiles when the fp16 X rows (Mp, a multiple of 128) cover whole
    // 256-row tiles, the grid (K split by the same rule) fills three
    // quarters of the CUs, and it needs no K-split reduction that the
    // 128-row grid would not (the reduction launch costs more than the
    // larger tiles save on a small grid).
    const size_t tiles4 = (mp / kV4BM) * (size_t)a.tiles_n;  // 0 when mp < 256
    const int splits4 = tiles4 ? pick_splits(tiles4, m, num_cus) : 1;
    if (tiles4 && mp % kV4BM == 0 && tiles4 * (size_t)splits4 * 4 >= (size_t)num_cus * 3 &&
        (splits4 == 1 || a.splits > 1)) {
      if ((e = set_lds_limit(reinterpret_cast<const void*>(q4_0_gemm_v4_kernel), kV4Lds)) !=
          hipSuccess)
        return e;
      a.tiles_m = (int)(mp / kV4BM);
      a.xcd_map = (tiles4 % 8) == 0 ? 1 : 0;
      a.splits = splits4;
      hipLaunchKernelGGL(q4_0_gemm_v4_kernel, dim3((unsigned)tiles4, a.splits), dim3(kThreads),
                         kV4Lds, s, a);
    } else {
      hipLaunchKernelGGL(q4_0_gemm_v3_kernel<true>, dim3(tiles, a.splits), dim3(kThreads),
                         kLdsBytes, s, a);
    }
  } else {
    if ((e = launch_x_f16_permuted(x, batch, m, ws, s)) != hipSuccess) return e;
    hipLaunchKernelGGL(q4_0_gemm_v3_kernel<false>, dim3(tiles, a.splits), dim3(kThreads),
                       kLdsBytes, s, a);
  }
  e = hipGetLastError();
  if (e != hipSuccess || a.splits == 1) return e;
  const size_t mn = batch * n;
  hipLaunchKernelGGL(split_k_reduce_kernel, dim3((unsigned)((mn + 255) / 256)), dim3(256), 0, s, y,
                     a.part, bias, mn, (int)n, a.splits);
  return hipGetLastError();
}

}  // namespace hypno
