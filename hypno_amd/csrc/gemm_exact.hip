// Q4_0 batched-prefill GEMM in the exact-nibble arithmetic, for gfx950:
// Y[M][N] = X[M][K] . W[N][K]^T (+ bias), W in hypno's Q4_0 blocks
// (quant.rs:10-22), X rounded to fp16 (each row scaled by a power of two
// first, undone exactly on output).  Every block b of output column n
// contributes d[n][b] * P, where P = sum over the block's 32 columns of
// (nib - 8) * x is one v_mfma_f32_16x16x32_f16 on the exact integer nibbles
// (fp16 values -8..7) into a zeroed accumulator, and the fp32 scale is
// applied by one VALU FMA per output and block: acc += d * P
// (kernels.rs:292-349 semantics, one block at a time; turbo.rs:306-333 per
// token).
//
// What bounds it on gfx950: per 16x16x32 MFMA (16 cycles of the matrix
// pipe) the scale costs 4 wave64 fp32 FMAs, and a wave's VALU instructions
// and MFMA issues share one issue port per SIMD.  Measured on the MI355X
// with independent MFMAs and k VALU ops each (two waves per SIMD, no
// memory): k = 0 runs the matrix pipe at 93% of 2.5 PF, k = 4 at 61%, and
// every further op costs ~1.9 ns per MFMA per SIMD.  So the design spends as
// few VALU ops per MFMA beyond the four FMAs as it can:
//
//  * Work-group = 8 waves (two per SIMD) on a BM x 128 tile of Y; wave w
//    owns output columns 16w..16w+15 for all BM = 16 MT rows (MT M-tiles).
//    A wave expands only its own weights, in registers: per block each lane
//    unpacks the 8 nibbles it feeds to the MFMA (one 16-column x 32-K B
//    operand: 9 VALU ops, v_perm for the even block's 2-byte offset) and
//    converts its column's scale (1 op); that B operand then serves all MT
//    MFMAs of the block.  No barrier waits on another wave's weights.
//  * W: each wave DMAs its own 16 rows' 36 bytes of a stage (two blocks)
//    into its own LDS ring (three 4-byte-per-lane buffer_load ... lds, the
//    stage offset a scalar, so addresses cost no VALU), kWRing stages deep,
//    and reads its lanes' words back from there; only the wave's own load
//    counter orders that ring.
//  * X: the fp16 rows (permuted per group of 8 columns into the order the
//    unpack emits weights, as x_row_to_f16 writes them) reach a 4-slot LDS
//    ring by DMA (buffer_load ... lds, scalar stage offset), three stages
//    ahead; 16-byte chunk c of row r sits in slot c ^ ((r >> 1) & 7), so the
//    16 rows of an MFMA operand read hit distinct banks.  One barrier per
//    stage (64 K): it publishes the X slot two stages ahead.
//  * The A operands of block 0 of the next stage are read during block 1's
//    MFMAs, so no stage starts on an LDS read.
//  * The K range of a tile can be cut into pieces (splits): each piece
//    writes an fp32 partial plane and split_k_reduce-style summation in
//    split order finishes (fixed order: deterministic).
//
// Requirements (q4_0_gemm_exact_ok): K % 256 == 0, w 4-byte aligned and
// holding N whole rows, W and the fp16 X under 4 GB (32-bit buffer offsets).
#include <algorithm>

#include "common.hpp"

namespace hypno {

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kEWaves = 8;
constexpr int kEThreads = 64 * kEWaves;
constexpr int kEBN = 16 * kEWaves;  // 128 output columns per work-group
constexpr int kEStageK = 64;        // two Q4_0 blocks per stage
constexpr int kERowBytes = kEStageK * 2;
// Per M-tiles per wave (MT): X stages resident in LDS (the ring, kRing slots
// of BM x 128 bytes) and the per-wave W ring (kWRing slots of 768 bytes:
// 16 rows x 36 bytes of a stage, rounded up to three 256-byte DMAs).
template <int MT>
struct ExactGeom {
  static constexpr int kRing = MT == 16 ? 4 : MT == 8 ? 6 : 8;
  static constexpr int kWRing = MT == 16 ? 4 : MT == 8 ? 8 : 16;
  static constexpr int kXLds = kRing * 16 * MT * kERowBytes;
  static constexpr int kWSlot = 768;
  static constexpr int kSpare = kXLds + kEWaves * kWRing * kWSlot;  // 1 KB (BM < 64)
  static constexpr int kLds = kSpare + (MT < 4 ? 1024 : 0);
  static_assert(kLds <= 160 * 1024, "LDS budget");
  static_assert(kWRing >= kRing, "the stage wait below counts X(s+2) as the newer read");
};

struct ExactArgs {
  float* y;
  const uint8_t* w;
  const uint8_t* xh;  // fp16 [Mp][K], columns permuted per group of 8
  const float* bias;
  const int* xexp;    // [Mp]: row m of xh holds X row m times 2^-xexp[m]
  float* part;        // [splits][M][N] partial planes (splits > 1)
  uint32_t w_bytes;   // W bytes (buffer range)
  uint32_t x_bytes;   // xh bytes (buffer range: rows past Mp read zeros)
  uint32_t xe_bytes;  // xexp bytes (rows past Mp read 0)
  uint32_t y_bytes;   // M x N x 4: the range of Y and of each partial plane
  int M, N, K;
  int tiles_m, tiles_n;
  int xcd_map;
  int splits;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// A stage's W words of one lane (row n, quarter q = lane >> 4 of the block's
// nibbles): the even block starts at byte 0 of the 36-byte stage, the odd one
// at byte 18.
struct RawW {
  uint32_t e0, e1;  // bytes 4q .. 4q+7: the even block's nibble bytes 4q..4q+3 at offset 2
  uint32_t d;       // bytes 0..3: the even block's scale in the low half
  uint32_t x4;      // bytes 16..19: the odd block's scale in the high half
  uint32_t o;       // bytes 20+4q .. 23+4q: the odd block's nibble bytes 4q..4q+3
};

template <int MT>
__global__ void __launch_bounds__(kEThreads, 1) q4_0_gemm_exact_kernel(const ExactArgs a) {
#if defined(__HIP_DEVICE_COMPILE__)  // (the buffer builtins exist only in the device pass)
  constexpr int BM = 16 * MT;
  using G = ExactGeom<MT>;
  constexpr int kERing = G::kRing;
  constexpr int kWRing = G::kWRing;
  constexpr int kTile = BM * kERowBytes;  // one stage of X in LDS
  // X DMA instructions per wave and stage; below 64 rows the waves past the
  // tile's 8-row groups re-read its last group into a spare LDS chunk, so
  // every wave issues the same count.
  constexpr int kDx = BM >= 64 ? BM / 64 : 1;
  extern __shared__ __align__(16) uint8_t smem[];
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int lr = lane & 15;
  const int lq = lane >> 4;

  // Tile of this work-group; with xcd_map the 8 XCDs (work-groups go round
  // robin over them) each get a contiguous range of tiles in (n-tile,
  // m-tile) order, so the m-tiles sharing W rows share an L2.
  int tile = blockIdx.x;
  const int ntiles = a.tiles_m * a.tiles_n;
  if (a.xcd_map) tile = (tile & 7) * (ntiles >> 3) + (tile >> 3);
  const int m0 = (tile % a.tiles_m) * BM;
  const int n0 = (tile / a.tiles_m) * kEBN;
  // K range of this piece: stages [s0, s0 + steps).
  const int gsteps = a.K / kEStageK;
  const int z = blockIdx.y;
  const int s0 = (int)((long long)gsteps * z / a.splits);
  const int s1 = (int)((long long)gsteps * (z + 1) / a.splits);
  const int steps = s1 - s0;

  // --- X DMA: instruction i of wave w fills rows 8 (8 i + w) .. +7 of the
  // slot; lane -> row 8 (8 i + w) + (lane >> 3), slot chunk lane & 7, which
  // holds logical chunk (lane & 7) ^ ((row >> 1) & 7).
  const __amdgpu_buffer_rsrc_t xrs = rsrc(a.xh, a.x_bytes);
  const uint32_t x_row = (uint32_t)a.K * 2;
  uint32_t xvoff[kDx];
#pragma unroll
  for (int i = 0; i < kDx; i++) {
    const int grp = min(8 * i + wave, BM / 8 - 1);
    const int row = 8 * grp + (lane >> 3);
    const int c = (lane & 7) ^ ((row >> 1) & 7);
    xvoff[i] = (uint32_t)(m0 + row) * x_row + (uint32_t)c * 16u;
  }
  auto issue_x = [&](int s) {  // stage min(s, steps - 1) into the slot of s
    const int sc = s < steps ? s : steps - 1;
    const int soff = (s0 + sc) * kERowBytes;
    uint8_t* slot = smem + (s % kERing) * kTile;
#pragma unroll
    for (int i = 0; i < kDx; i++) {
      const int grp = 8 * i + wave;
      uint8_t* dst = grp < BM / 8 ? slot + 8 * grp * kERowBytes : smem + G::kSpare;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          xrs, (__attribute__((address_space(3))) void*)dst, 16, xvoff[i], soff, 0, 0);
    }
  };

  // --- W: each wave DMAs its own 16 rows' 36 stage bytes into its own ring
  // (three 4-byte-per-lane DMAs: lane L of the 192 -> row min(L / 9, 15),
  // dword L % 9, the 48 surplus lanes re-reading row 15's last dword into
  // the slot's tail) and reads them back per lane; no other wave touches
  // the ring, so only this wave's own load counter orders it.
  const int ncol = n0 + 16 * wave + lr;
  const bool nvalid = ncol < a.N;
  const __amdgpu_buffer_rsrc_t wrs = rsrc(a.w, a.w_bytes);
  const uint32_t w_row = (uint32_t)(a.K / kBlockElems * kBlockBytes);
  uint32_t wvoff[3];
#pragma unroll
  for (int i = 0; i < 3; i++) {
    const int l = 64 * i + lane;
    const int r = l < 144 ? l / 9 : 15;
    const int c = l < 144 ? l % 9 : 8;
    wvoff[i] = (uint32_t)min(n0 + 16 * wave + r, a.N - 1) * w_row + 4u * (uint32_t)c;
  }
  uint8_t* const wring = smem + G::kXLds + wave * kWRing * G::kWSlot;
  auto issue_w = [&](int s) {  // stage min(s, steps - 1) into the slot of s
    const int sc = s < steps ? s : steps - 1;
    const int soff = (s0 + sc) * 36;
    uint8_t* slot = wring + (s % kWRing) * G::kWSlot;
#pragma unroll
    for (int i = 0; i < 3; i++)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          wrs, (__attribute__((address_space(3))) void*)(slot + 256 * i), 4, wvoff[i], soff, 0,
          0);
  };
  auto read_w = [&](int s) -> RawW {
    const uint32_t* p =
        reinterpret_cast<const uint32_t*>(wring + (s % kWRing) * G::kWSlot + lr * 36);
    RawW r;
    r.e0 = p[lq];
    r.e1 = p[lq + 1];
    r.d = p[0];
    r.x4 = p[4];
    r.o = p[5 + lq];
    return r;
  };

  // --- A operands: block kb of the slot of stage s, M-tile i: row 16 i + lr,
  // logical chunk 4 kb + lq ((row >> 1) & 7 = (lr >> 1) & 7 for every i).
  const uint32_t aoff0 = (uint32_t)lr * kERowBytes + (((0 + lq) ^ ((lr >> 1) & 7)) << 4);
  const uint32_t aoff1 = (uint32_t)lr * kERowBytes + (((4 + lq) ^ ((lr >> 1) & 7)) << 4);
  auto read_a = [&](int s, int kb, half8 (&fa)[MT]) {
    const uint8_t* base = smem + (s % kERing) * kTile + (kb ? aoff1 : aoff0);
#pragma unroll
    for (int i = 0; i < MT; i++)
      fa[i] = *reinterpret_cast<const half8*>(base + i * 16 * kERowBytes);
  };

  floatx4 acc[MT];
#pragma unroll
  for (int i = 0; i < MT; i++) acc[i] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  // B operand of a block, unpacked in steps that the slot schedule below
  // spreads over the MFMAs (the arithmetic of unpack8: eight nibbles of q
  // -> eight exact fp16 values nib - 8 in the order e0,e4,e1,e5,e2,e6,e3,e7,
  // which is the order x_row_to_f16 permutes each group of 8 columns into),
  // and the block's scale as fp32 (0 past N).
  struct Unp {
    uint32_t q, q8, p0, p1, p2, p3;
    u32x4 r;
    float d;
  };
  auto unp_step = [&](Unp& u, int k, uint32_t dbits) {
    const half2v lo_off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    const half2v hi_mul = {(_Float16)0.0625f, (_Float16)0.0625f};
    const half2v hi_off = {(_Float16)-72.0f, (_Float16)-72.0f};
    if (k == 0) {
      u.p0 = and_or(u.q, 0x000F000Fu, 0x64006400u);
      u.p1 = and_or(u.q, 0x00F000F0u, 0x64006400u);
    } else if (k == 1) {
      u.q8 = u.q >> 8;
      u.p2 = and_or(u.q8, 0x000F000Fu, 0x64006400u);
    } else if (k == 2) {
      u.p3 = and_or(u.q8, 0x00F000F0u, 0x64006400u);
      u.r[0] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, u.p0) + lo_off);
    } else if (k == 3) {
      u.r[1] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(
                                                __builtin_bit_cast(half2v, u.p1), hi_mul, hi_off));
      u.r[2] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, u.p2) + lo_off);
    } else if (k == 4) {
      u.r[3] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(
                                                __builtin_bit_cast(half2v, u.p3), hi_mul, hi_off));
      u.d = f16_bits_to_f32(dbits);
    } else if (k == 5) {
      u.d = nvalid ? u.d : 0.0f;
    }
  };

  // Prologue: X of stages 0..R-2 and W of stages 0..P-1 in flight (R =
  // kRing, P = kWRing); X and W of stages 0 and 1 landed (all but the last
  // 3 (P - 2) reads) and published; A operands of stage 0 block 0, the W
  // words of stage 0 and its even block's B operand.
  for (int i = 0; i < kERing - 1; i++) issue_x(i);
  for (int i = 0; i < kWRing; i++) issue_w(i);
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(3 * (kWRing - 2)) : "memory");
  half8 fa[MT], fx;
  read_a(0, 0, fa);
  RawW wc = read_w(0);
  Unp ue;
  ue.q = __builtin_amdgcn_perm(wc.e1, wc.e0, 0x05040302u);
#pragma unroll
  for (int k = 0; k < 6; k++) unp_step(ue, k, wc.d & 0xFFFFu);
  half8 fbe = __builtin_bit_cast(half8, ue.r);
  float de = ue.d;

  // Stage s = 2 MT MFMA slots, block 0 (slots 0..MT-1, operand fa[i] times
  // fbe, scale de) then block 1 (fa[i] times the odd block's fbo, scale
  // dod).  Slot j issues, in this order (a scheduling barrier between slots
  // keeps it):
  //  - MFMA j into a zeroed partial;
  //  - the reload of the A register that MFMA j-1 read, with the operand of
  //    the next block (block 1 of s, then block 0 of s+1), MT slots before
  //    its use;
  //  - the four scale FMAs of partial j-kLag (of the previous stage's last
  //    slots for j < kLag), kLag MFMAs after it, so they wait on nothing;
  //  - one or two ops of the next block's unpack (odd block of s during
  //    block 0, even block of s+1 during block 1).
  // Then stage s's W words of s+1 were read at slot 0; after the slots: the
  // X DMA of stage s+R-1 into the slot of s-1 (every wave is past the
  // barrier that ended stage s-1, so none reads it any more), the W DMA of
  // stage s+P into the slot of s (whose words this wave already holds), and
  // the wait for X and W of s+2 and the barrier.  X(s+2) went out in stage
  // s+3-R and W(s+2) earlier (P >= R), so the wait leaves outstanding that
  // stage's 3 W DMAs and R-3 whole stages of kDx + 3; in the first stages,
  // where the prologue issued them, more reads follow them than that.
  constexpr int kLag = 2;
  constexpr int kStageWait = 3 + (kERing - 3) * (kDx + 3);
  static_assert(kStageWait <= 3 * (kWRing - 2) + kDx + 3 && 3 * kWRing + kERing * kDx < 64,
                "vmcnt");
  // The unpack's steps spread over a block's slots (1..MT-1, or slot 0 when
  // MT = 1): step k of the odd block's 6 in slot kFirst + k * kSl / 6, the
  // even block's perm and 6 steps likewise over 7.
  constexpr int kFirst = MT >= 2 ? 1 : 0;
  constexpr int kSl = MT >= 2 ? MT - 1 : 1;
  // Partials of the last kLag slots are scaled in the next stage's first
  // slots, each with the scale of its own block.
  floatx4 carry[kLag];
  float dcar[kLag];
#pragma unroll
  for (int k = 0; k < kLag; k++) {
    carry[k] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    dcar[k] = 0.0f;
  }
  const uint8_t* abase0 = smem + aoff0;
  const uint8_t* abase1 = smem + aoff1;
  for (int s = 0; s < steps; s++) {
    const RawW wn = read_w(s + 1);
    const uint8_t* a1 = abase1 + (s % kERing) * kTile;        // block 1 of s
    const uint8_t* a0 = abase0 + ((s + 1) % kERing) * kTile;  // block 0 of s+1
    Unp uo, un;
    uo.q = wc.o;
    half8 fbo;
    float dod = 0.0f;
    floatx4 pr[2 * MT];
#pragma unroll
    for (int j = 0; j < 2 * MT; j++) {
      const int kb = j / MT, i = j % MT;
      pr[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16((MT == 1 && kb) ? fx : fa[i], kb ? fbo : fbe,
                                                     floatx4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
      if constexpr (MT == 1) {  // one slot per block: block 1's operand has its own register
        if (j == 0) fx = *reinterpret_cast<const half8*>(a1);
        if (j == 1) fa[0] = *reinterpret_cast<const half8*>(a0);
      } else if (j >= 1) {
        const int pj = j - 1;
        fa[pj % MT] = *reinterpret_cast<const half8*>((pj < MT ? a1 : a0) +
                                                      (pj % MT) * 16 * kERowBytes);
      }
      if (j >= kLag) {
        const int u = j - kLag;
        const float d = u < MT ? de : dod;
#pragma unroll
        for (int r = 0; r < 4; r++) acc[u % MT][r] = fmaf(d, pr[u][r], acc[u % MT][r]);
      } else {
        const int t = (2 * MT - kLag + j) % MT;
#pragma unroll
        for (int r = 0; r < 4; r++) acc[t][r] = fmaf(dcar[j], carry[j][r], acc[t][r]);
      }
#pragma unroll
      for (int k = 0; k < 6; k++)
        if (kb == 0 && i == kFirst + k * kSl / 6) unp_step(uo, k, wc.x4 >> 16);
      if (kb == 0 && i == MT - 1) {
        fbo = __builtin_bit_cast(half8, uo.r);
        dod = uo.d;
      }
      if (kb == 1 && i == kFirst) un.q = __builtin_amdgcn_perm(wn.e1, wn.e0, 0x05040302u);
#pragma unroll
      for (int k = 0; k < 6; k++)
        if (kb == 1 && i == kFirst + (k + 1) * kSl / 7) unp_step(un, k, wn.d & 0xFFFFu);
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (MT > 1) fa[MT - 1] = *reinterpret_cast<const half8*>(a0 + (MT - 1) * 16 * kERowBytes);
#pragma unroll
    for (int k = 0; k < kLag; k++) {
      carry[k] = pr[2 * MT - kLag + k];
      dcar[k] = 2 * MT - kLag + k < MT ? de : dod;
    }
    // The X DMAs go out before the W DMAs (the wait below counts on it).
    asm volatile("" ::: "memory");
    issue_x(s + kERing - 1);
    asm volatile("" ::: "memory");
    issue_w(s + kWRing);
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(kStageWait) : "memory");
    wc = wn;
    fbe = __builtin_bit_cast(half8, un.r);
    de = un.d;
  }
#pragma unroll
  for (int k = 0; k < kLag; k++) {
    const int t = (2 * MT - kLag + k) % MT;
#pragma unroll
    for (int r = 0; r < 4; r++) acc[t][r] = fmaf(dcar[k], carry[k][r], acc[t][r]);
  }
  // Every DMA into LDS (the trailing re-reads included) has landed before
  // the work-group's LDS is released.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // Output row m = m0 + 16 i + 4 lq + r, column ncol: scaled back by
  // 2^xexp[m] (exact).  The exponents of a lane's 4 MT rows come in MT
  // 16-byte reads issued together; Y goes out through a buffer whose range
  // is M x N, so rows past M drop out of range and lanes past N aim past
  // it (no per-element branch or wait).  K pieces write their partial plane
  // instead; the reduction adds the bias.
  const __amdgpu_buffer_rsrc_t ers = rsrc(a.xexp, a.xe_bytes);
  u32x4 ex[MT];
#pragma unroll
  for (int i = 0; i < MT; i++)
    ex[i] = __builtin_amdgcn_raw_buffer_load_b128(ers, (uint32_t)(m0 + 16 * i + 4 * lq) * 4u, 0, 0);
  float* dst = a.splits > 1 ? a.part + (size_t)z * a.M * a.N : a.y;
  const __amdgpu_buffer_rsrc_t yrs = rsrc(dst, a.y_bytes);
  const float bv = (nvalid && a.bias && a.splits == 1) ? a.bias[ncol] : 0.0f;
#pragma unroll
  for (int i = 0; i < MT; i++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const uint32_t m = (uint32_t)(m0 + 16 * i + 4 * lq + r);
      const uint32_t off = nvalid ? (m * (uint32_t)a.N + (uint32_t)ncol) * 4u : 0xFFFFFFF0u;
      const float v = ldexpf(acc[i][r], (int)ex[i][r]) + bv;
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), yrs, off, 0, 0);
    }
#endif
}

__global__ void __launch_bounds__(256)
exact_split_reduce_kernel(float* __restrict__ y, const float* __restrict__ part,
                          const float* __restrict__ bias, size_t mn, int n, int splits) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= mn) return;
  float v = part[i];
  for (int z = 1; z < splits; z++) v += part[(size_t)z * mn + i];
  y[i] = v + (bias ? bias[i % n] : 0.0f);
}

// X fp32 [M][K] -> fp16 [Mp][K] for the kernel above, one work-group of 256
// threads per row, in one read of the row: each thread holds its groups of
// 8 columns (group g = t + 256 u, u < kXGroups) in registers while the row's
// largest |x| is found, then writes them scaled by 2^sh (sh puts that
// maximum in [2^14, 2^15); 0 for an all-zero row or one holding inf or NaN,
// the same rule as x_row_to_f16) and rounded to fp16, each group permuted to
// the unpack order e0,e4,e1,e5,e2,e6,e3,e7; xexp[row] = -sh.  Rows M..Mp-1
// are written as zeros.  K <= 256 * 8 * kXGroups.
constexpr int kXGroups = 8;
__global__ void __launch_bounds__(256)
x_rows_f16_onepass_kernel(u32x4* __restrict__ xh, int* __restrict__ xexp,
                          const float* __restrict__ x, int M, int K) {
  __shared__ uint32_t red[4];
  const int row = blockIdx.x;
  const int t = threadIdx.x;
  const int groups = K / 8;
  u32x4* dst = xh + (size_t)row * groups;
  if (row >= M) {
    for (int g = t; g < groups; g += 256) dst[g] = u32x4{0u, 0u, 0u, 0u};
    if (t == 0) xexp[row] = 0;
    return;
  }
  const float4* src = reinterpret_cast<const float4*>(x + (size_t)row * K);
  float4 v[kXGroups][2];
  uint32_t mb = 0;  // largest |x| by bit pattern (inf and NaN above every finite value)
#pragma unroll
  for (int u = 0; u < kXGroups; u++) {
    const int g = t + 256 * u;
    if (g < groups) {
      v[u][0] = load_global<float4>(src + 2 * g);
      v[u][1] = load_global<float4>(src + 2 * g + 1);
    }
  }
#pragma unroll
  for (int u = 0; u < kXGroups; u++) {
    if (t + 256 * u < groups) {
      const float e[8] = {v[u][0].x, v[u][0].y, v[u][0].z, v[u][0].w,
                          v[u][1].x, v[u][1].y, v[u][1].z, v[u][1].w};
#pragma unroll
      for (int i = 0; i < 8; i++) mb = max(mb, __float_as_uint(e[i]) & 0x7FFFFFFFu);
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mb = max(mb, (uint32_t)__shfl_xor((int)mb, off, 64));
  if ((t & 63) == 0) red[t >> 6] = mb;
  __syncthreads();
  mb = max(max(red[0], red[1]), max(red[2], red[3]));
  const float amax = __uint_as_float(mb);
  int sh = 0;
  if (amax > 0.0f && amax < __builtin_inff()) sh = 15 - __builtin_amdgcn_frexp_expf(amax);
  constexpr int perm[8] = {0, 4, 1, 5, 2, 6, 3, 7};
#pragma unroll
  for (int u = 0; u < kXGroups; u++) {
    const int g = t + 256 * u;
    if (g < groups) {
      const float e[8] = {v[u][0].x, v[u][0].y, v[u][0].z, v[u][0].w,
                          v[u][1].x, v[u][1].y, v[u][1].z, v[u][1].w};
      u32x4 packed;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint32_t lo = __builtin_bit_cast(uint16_t, (_Float16)ldexpf(e[perm[2 * j]], sh));
        const uint32_t hi = __builtin_bit_cast(uint16_t, (_Float16)ldexpf(e[perm[2 * j + 1]], sh));
        packed[j] = lo | (hi << 16);
      }
      dst[g] = packed;
    }
  }
  if (t == 0) xexp[row] = -sh;
}

size_t rup(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Geometry chosen for a shape: M-tiles per wave and K pieces.
struct ExactPlan {
  int mt;
  int tiles_m, tiles_n;
  int splits;
};

// Tile height and K pieces by a cost model of this kernel on the MI355X
// (microseconds, measured): a stage of 64 K costs 0.40 / 0.45 / 0.57 / 0.79
// / 1.22 on tiles of 16 / 32 / 64 / 128 / 256 rows (a B operand serves MT
// MFMAs), a round of work-groups (one per CU) ~3 more to fill and drain;
// K pieces add the reduction launch (~2.5) and its read of every partial
// plane (~4 TB/s).
ExactPlan exact_plan(size_t batch, size_t n, size_t m, int num_cus) {
  const size_t tn = (n + kEBN - 1) / kEBN;
  const size_t steps = m / kEStageK;
  ExactPlan best{8, 1, (int)tn, 1};
  double best_cost = 1e300;
  for (int mt : {1, 2, 4, 8, 16}) {
    if (mt > 1 && (size_t)16 * (mt / 2) >= batch) break;  // taller tiles than the rows
    const size_t tm = (batch + 16 * mt - 1) / (16 * mt);
    const size_t tiles = tm * tn;
    const double stage_us = mt == 16 ? 1.22 : mt == 8 ? 0.79 : mt == 4 ? 0.57 : mt == 2 ? 0.45 : 0.40;
    for (size_t sp = 1; sp <= std::min<size_t>(steps, 64); sp++) {
      const size_t wgs = tiles * sp;
      const size_t rounds = (wgs + num_cus - 1) / num_cus;
      double cost = (double)rounds * ((double)((steps + sp - 1) / sp) * stage_us + 3.0);
      if (sp > 1) cost += 2.5 + (double)sp * (double)(batch * n * 4) / 4.0e6;
      if (cost < best_cost * 0.999) {
        best_cost = cost;
        best = ExactPlan{mt, (int)tm, (int)tn, (int)sp};
      }
      if (rounds > 1 && sp > 1) break;  // more pieces only add rounds
    }
  }
  return best;
}

}  // namespace

bool q4_0_gemm_exact_ok(const uint8_t* w, size_t w_len, size_t n, size_t m, size_t batch) {
  if (m == 0 || m % 256 != 0 || n == 0 || batch == 0) return false;
  if (((uintptr_t)w & 3) != 0) return false;
  if (n > (size_t)0x7FFFFFFF || m > (size_t)0x7FFFFFF || batch > (size_t)0x7FFFFFFF) return false;
  const size_t wbytes = n * (m / kBlockElems) * kBlockBytes;
  if (wbytes >= ((size_t)1 << 32)) return false;
  if (rup(batch, 256) * m * 2 >= ((size_t)1 << 32)) return false;
  // Output offsets (row m < M + 256) stay below 2^32 - 16 (the lanes past N
  // aim at 2^32 - 16).
  if ((batch + 256) * n * 4 >= ((size_t)1 << 32) - 16) return false;
  return w_len >= wbytes;
}

size_t q4_0_gemm_exact_workspace_bytes(size_t batch, size_t n, size_t m, int num_cus) {
  const ExactPlan p = exact_plan(batch, n, m, num_cus);
  const size_t xb = rup(gemm_workspace_bytes(batch, m), 256);
  return p.splits > 1 ? xb + (size_t)p.splits * batch * n * 4 : xb;
}

hipError_t launch_q4_0_gemm_exact(float* y, const uint8_t* w, const float* x, const float* bias,
                                  size_t n, size_t m, size_t batch, void* ws, int num_cus,
                                  hipStream_t s) {
  hipError_t e;
  if (m <= (size_t)256 * 8 * kXGroups && ((uintptr_t)x & 15) == 0) {
    hipLaunchKernelGGL(x_rows_f16_onepass_kernel, dim3((unsigned)rup(batch, 128)), dim3(256), 0, s,
                       static_cast<u32x4*>(ws), gemm_x_exponents(ws, batch, m), x, (int)batch,
                       (int)m);
    e = hipGetLastError();
  } else {
    e = launch_x_f16_permuted(x, batch, m, ws, s);
  }
  if (e != hipSuccess) return e;
  const ExactPlan p = exact_plan(batch, n, m, num_cus);
  ExactArgs a;
  a.y = y;
  a.w = w;
  a.xh = static_cast<const uint8_t*>(ws);
  a.bias = bias;
  a.xexp = gemm_x_exponents(ws, batch, m);
  a.part = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) +
                                    rup(gemm_workspace_bytes(batch, m), 256));
  a.w_bytes = (uint32_t)(n * (m / kBlockElems) * kBlockBytes);
  a.x_bytes = (uint32_t)(rup(batch, 128) * m * 2);
  a.xe_bytes = (uint32_t)(rup(batch, 128) * 4);
  a.y_bytes = (uint32_t)(batch * n * 4);
  a.M = (int)batch;
  a.N = (int)n;
  a.K = (int)m;
  a.tiles_m = p.tiles_m;
  a.tiles_n = p.tiles_n;
  const int tiles = p.tiles_m * p.tiles_n;
  a.xcd_map = (tiles % 8) == 0 ? 1 : 0;
  a.splits = p.splits;
  auto go = [&](auto kernel, int lds) -> hipError_t {
    hipError_t le = set_lds_limit(reinterpret_cast<const void*>(kernel), lds);
    if (le != hipSuccess) return le;
    hipLaunchKernelGGL(kernel, dim3(tiles, p.splits), dim3(kEThreads), lds, s, a);
    return hipSuccess;
  };
  switch (p.mt) {
    case 16: e = go(q4_0_gemm_exact_kernel<16>, ExactGeom<16>::kLds); break;
    case 8: e = go(q4_0_gemm_exact_kernel<8>, ExactGeom<8>::kLds); break;
    case 4: e = go(q4_0_gemm_exact_kernel<4>, ExactGeom<4>::kLds); break;
    case 2: e = go(q4_0_gemm_exact_kernel<2>, ExactGeom<2>::kLds); break;
    default: e = go(q4_0_gemm_exact_kernel<1>, ExactGeom<1>::kLds); break;
  }
  if (e != hipSuccess) return e;
  if ((e = hipGetLastError()) != hipSuccess || p.splits == 1) return e;
  const size_t mn = batch * n;
  hipLaunchKernelGGL(exact_split_reduce_kernel, dim3((unsigned)((mn + 255) / 256)), dim3(256), 0,
                     s, y, a.part, bias, mn, (int)n, p.splits);
  return hipGetLastError();
}

}  // namespace hypno
