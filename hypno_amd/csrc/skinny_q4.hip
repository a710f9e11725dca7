// Q4_0 matmul for a few tokens (2 <= M <= 64): Y[M][N] = X[M][K] . W[N][K]^T.
//
// This regime is bound by the weight stream (2 M flop per weight byte, at
// most 228 flop/B, below the ~310 flop/B ridge), so the kernel reads every
// Q4_0 block of W exactly once, in coalesced 16-byte pieces of contiguous
// row segments, and does the arithmetic on the matrix cores:
//
//  * A work-group owns 64 rows of W (16 on matrices too small for 64-row
//    tiles to fill the GPU) and a range of K; K streams through LDS
//    in stages of 256 (8 blocks): DMA (global_load_lds) of the stage's
//    activation rows and W row segments into a ring of LDS slots, one
//    barrier per stage.  Its 16 (4) waves form 4 (1) row groups (16 rows,
//    one MFMA column tile each) x 4 K-groups (block pair kg of every stage):
//    up to four waves per SIMD, so their unpacking overlaps the others'
//    waits; at the end K-groups 1-3 hand their sums to K-group 0 through LDS
//    (added in K-group order: deterministic).
//  * Lane (n, g) of a wave takes nibble quarter g of row n's block from LDS
//    (4 bytes), turns it into exact fp16 (nib - 8) in registers and feeds
//    v_mfma_f32_16x16x32_f16; the block's partial is scaled in fp32.
//  * Small tile grids split K over blockIdx.y; the fp32 partials are added in
//    split order by a second kernel (deterministic, no atomics).
//  * Activations come from a pre-pass as MFMA A-operand rows (fp16, columns
//    permuted per group of 8 to the unpack order):
//      - M <= 16 ("split"): each stage (256 K) of token t is scaled by a
//        power of two s so that its max |x| s lies in [2^14, 2^15), and
//        stored as hi = fp16(x s) in row t and lo = fp16(x s - hi) in row
//        Mh + t.  hi + lo equals x s to about 2^-22 relative, the products
//        with the exact integer weights are exact in fp32, and every stage
//        adds (acc_hi + acc_lo) / s to y_t: an fp32-accurate result, as the
//        GEMV path gives.  (Per-stage scales keep the pre-pass one pass over
//        X with a work-group per stage.)
//      - 16 < M <= 64: one fp16 row per token (the prefill GEMM's rounding),
//        scaled by a power of two per token (x_row_to_f16) that the epilogue
//        undoes.
//    On 16-row tiles whose K is split into ranges of at most 8 stages (up to
//    8 tokens), each work-group converts its own stages the same way into
//    LDS instead (no pre-pass launch).
//
// Requirements (q4_0_skinny_ok): K % 256 == 0, w 16-byte aligned (row
// segments of a stage are then 16-byte aligned), W and X under 4 GB, w
// holds N whole rows.
#include "common.hpp"

namespace hypno {

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t pack2h(float a, float b) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)a) |
         ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)b) << 16);
}

// The pre-pass arithmetic for lane gi's 8 columns of one token's stage
// (32-lane groups): s = 2^(15 - e) with max |x| < 2^e over the group, so
// max |x| s < 2^15 (zero, inf and NaN stages keep s = 1: their products
// propagate as the reference's would); hi = fp16(x s), lo = fp16(x s - hi),
// columns permuted per group of 8 to the unpack order.
struct StagePieces {
  u32x4 h, l;
  float inv;
};
__device__ __forceinline__ StagePieces split_stage8(const float (&v)[8]) {
  uint32_t mb = 0;  // largest |x| of the stage by bit pattern (NaN and inf above finite)
#pragma unroll
  for (int k = 0; k < 8; k++) mb = max(mb, __float_as_uint(v[k]) & 0x7FFFFFFFu);
  // over the 32 lanes: DPP quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror,
  // row_mirror (all 16 lanes of a row), then the other row of the group
  mb = max(mb, (uint32_t)__builtin_amdgcn_mov_dpp((int)mb, 0xB1, 0xF, 0xF, false));
  mb = max(mb, (uint32_t)__builtin_amdgcn_mov_dpp((int)mb, 0x4E, 0xF, 0xF, false));
  mb = max(mb, (uint32_t)__builtin_amdgcn_mov_dpp((int)mb, 0x141, 0xF, 0xF, false));
  mb = max(mb, (uint32_t)__builtin_amdgcn_mov_dpp((int)mb, 0x140, 0xF, 0xF, false));
  mb = max(mb, (uint32_t)__shfl_xor((int)mb, 16, 64));
  const float amax = __uint_as_float(mb);
  float sc = 1.0f;
  if (amax > 0.0f && amax < __builtin_inff())
    sc = ldexpf(1.0f, min(15 - __builtin_amdgcn_frexp_expf(amax), 126));
  float w8[8];
#pragma unroll
  for (int k = 0; k < 8; k++) w8[k] = v[k] * sc;
  constexpr int perm[8] = {0, 4, 1, 5, 2, 6, 3, 7};
  StagePieces r;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const float pp = w8[perm[2 * j]], qq = w8[perm[2 * j + 1]];
    r.h[j] = pack2h(pp, qq);
    const float ph = (float)(_Float16)pp, qh = (float)(_Float16)qq;
    r.l[j] = pack2h(pp - ph, qq - qh);
  }
  r.inv = 1.0f / sc;
  return r;
}

// Pre-pass: X fp32 [M][K] -> A rows fp16 [rows][K], in stages of 256 K
// (the main kernel's stage), plus 1/s per token and stage when split.
// 32 lanes per (row, stage): lane i converts K elements 8i .. 8i+7 of the
// stage.  Grid: (stages / 8 rounded up, hi rows); rows r >= M are zero.
__global__ void __launch_bounds__(256)
x_skinny_kernel(uint8_t* __restrict__ xa, float* __restrict__ inv_s, const float* __restrict__ x,
                int M, int K, int Mh, int split) {
  const int r = blockIdx.y;
  const int t = threadIdx.x;
  const int c = blockIdx.x * 8 + (t >> 5);  // stage
  const int gi = t & 31;
  const int stages = K / 256;
  if (c >= stages) return;  // whole 32-lane groups
  const size_t g = (size_t)c * 32 + gi;     // group of 8 along the row
  u32x4* hi_row = reinterpret_cast<u32x4*>(xa + (size_t)r * K * 2);
  u32x4* lo_row = reinterpret_cast<u32x4*>(xa + (size_t)(Mh + r) * K * 2);
  if (r >= M) {
    hi_row[g] = u32x4{0u, 0u, 0u, 0u};
    if (split) {
      lo_row[g] = u32x4{0u, 0u, 0u, 0u};
      if (gi == 0) inv_s[(size_t)c * Mh + r] = 1.0f;
    }
    return;
  }
  const float* xr = x + (size_t)r * K + 8 * g;
  const float4 a0 = load_global<float4>(xr);
  const float4 a1 = load_global<float4>(xr + 4);
  const float v[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
  if (split) {
    const StagePieces q = split_stage8(v);
    hi_row[g] = q.h;
    lo_row[g] = q.l;
    if (gi == 0) inv_s[(size_t)c * Mh + r] = q.inv;
    return;
  }
  constexpr int perm[8] = {0, 4, 1, 5, 2, 6, 3, 7};
  u32x4 h;
#pragma unroll
  for (int j = 0; j < 4; j++) h[j] = pack2h(v[perm[2 * j]], v[perm[2 * j + 1]]);
  hi_row[g] = h;
}

// Stage geometry.  A stage is 256 K (8 Q4_0 blocks) of every row and token:
// a row's 144 bytes of a stage start 16-byte aligned (rows are K/32*18 =
// multiples of 144 bytes when K % 256 == 0), so they move as nine 16-byte
// pieces.
constexpr int kSkKGroups = 4;                  // waves per row group, a quarter of a stage's blocks each
constexpr int kSkRowBytes = 144;               // W bytes of one row and stage
constexpr int kSkRowPieces = kSkRowBytes / 16;  // 9
constexpr int kSkWDma = (16 * kSkRowPieces + 63) / 64;  // 3 DMAs per wave and stage
constexpr int kSkWBytes = 1024 * kSkWDma;      // LDS per wave and stage (W)
constexpr int kSkXRowBytes = 512;              // fp16 A-row bytes of one stage
constexpr int kSkStageK = 256;

// RW row groups (16 W rows each) per work-group: 4, or 1 where 64-row tiles
// would leave the GPU short of work-groups.
template <int MF, int RW>
struct SkGeom {
  static constexpr int kWaves = RW * kSkKGroups;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kRows = 16 * MF;                      // A rows
  static constexpr int kXBytes = kRows * kSkXRowBytes;       // X chunk per stage
  static constexpr int kXTot = kXBytes / 1024;               // X DMAs per stage (8/16/32)
  static constexpr int kXDma = kXTot >= kWaves ? kXTot / kWaves : 1;  // per issuing wave
  static constexpr int kSlot = kXBytes + RW * kSkWBytes;
  static constexpr int kRing = MF == 4 ? 3 : 4;              // stages in LDS
  static constexpr int kLds = kRing * kSlot;                 // 80 / 112 / 132 KB
  // Per wave and stage: kXDma X DMAs (waves below kXTot / kXDma) and W DMA
  // i from K-group i of the row group (i < 3; the third carries the 16 rows'
  // last pieces and, when split, the 1/s table).
  static_assert(kSkWDma == 3, "W DMA split between the K-groups");
  static_assert(kLds <= 160 * 1024, "LDS budget");
  static_assert((kRing - 2) * (kXDma + 1) <= 63, "vmcnt range");
  static_assert(kXDma * kWaves >= kXTot, "every X piece has a wave");
  static_assert(kWaves * MF * 4 * 64 * 4 <= kLds, "K-group hand-over fits the ring");
};

// Wait until at most N of this wave's global reads are outstanding and its
// LDS accesses are done, then meet the work-group.  (One asm statement with a
// memory clobber: the compiler adds no wait of its own, and no LDS access
// moves across it.)
template <int N>
__device__ __forceinline__ void wait_reads_barrier() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"(N) : "memory");
}

// One wave-wide DMA of 16 bytes per lane: lane i's 16 bytes at `src` land at
// lds_wave_base + 16 i.
__device__ __forceinline__ void dma16(const void* src, uint8_t* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds_wave_base,
                                   16, 0, 0);
}

struct SkinnyArgs {
  float* y;
  float* part;        // [splits][M][N] partial sums when splits > 1
  const uint8_t* w;
  const uint8_t* xa;
  const float* x;     // fp32 activations (read by the kernel itself with INX)
  const float* inv_s;
  const int* xexp;    // without SPLIT: token t's row holds x_t times 2^-xexp[t]
  const float* bias;
  int M, N, K;
  int split;          // hi/lo rows
  int splits;         // K ranges over blockIdx.y
};

// A work-group owns 16 RW rows of W (wave w: rows 16 (w % RW) .. + 15, one
// MFMA column tile) and a range of whole stages of K; stages stream through
// a ring of LDS slots:
//  * X: the stage's 16 MF A rows (512 bytes each), DMA'd by all waves, 16-byte
//    pieces XOR-swizzled by row (piece c of row r at c ^ (r & 15)) so the
//    A-operand reads of 16 rows hit 16 different bank groups;
//  * W: each wave DMAs its own 16 rows x 144 bytes, row after row (row
//    stride 144 bytes = 36 dwords: 16 rows land in 16 different bank groups),
//    as 16-byte pieces of contiguous row segments (coalesced reads).
// One barrier per stage, after the wait for that stage's DMAs.  The MFMA B
// operand of lane (n, g) for a block is its quarter g (4 nibble bytes) of
// row n; it becomes exact fp16 (nib - 8) in registers, and the block's
// partial is scaled in fp32.
// INX (one A fragment, hi/lo rows, K split into ranges of at most
// kInxStages stages): the work-group converts its own stages of X (fp32)
// into the hi/lo rows and 1/s, the x_skinny_kernel arithmetic, straight
// into an LDS region ahead of the ring, instead of a pre-pass launch; the
// ring then carries W only.
constexpr int kInxStages = 8;

template <int MF, bool SPLIT, int RW, bool INX>
__global__ void __launch_bounds__((SkGeom<MF, RW>::kThreads)) q4_0_skinny_kernel(const SkinnyArgs a) {
  using G = SkGeom<MF, RW>;
  static_assert(!INX || (MF == 1 && SPLIT), "in-kernel X: one fragment, hi/lo rows");
  // INX: converted stage ls at ls * kXStride (A rows, then 16 floats of 1/s);
  // the ring follows at kXOff with slots of W only.
  constexpr int kXStride = G::kXBytes + 64;
  constexpr int kXOff = INX ? kInxStages * kXStride : 0;
  constexpr int kSlotB = INX ? RW * kSkWBytes : G::kSlot;
  extern __shared__ __align__(16) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rw = wave % RW;  // row group: W rows 16 rw .. 16 rw + 15 of the tile
  const int kg = wave / RW;  // K-group: blocks 2 kg, 2 kg + 1 of every stage
  const bool xact = !INX && wave * G::kXDma < G::kXTot;  // this wave DMAs X pieces
  const int n16 = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16 * RW + 16 * rw;  // this wave's first W row
  const int gsteps = a.K / kSkStageK;
  const int z = blockIdx.y;
  const int s0 = (int)((long long)gsteps * z / a.splits);
  const int steps = (int)((long long)gsteps * (z + 1) / a.splits) - s0;
  const size_t w_row = (size_t)(a.K / 32) * 18;
  const size_t x_row = (size_t)a.K * 2;

  // W DMA i, lane -> piece p = 64 i + lane of the row group's 16 x 9 pieces:
  // row p / 9, piece p % 9 (lanes past 144 are idle).  Rows past N re-read
  // row N - 1 (their outputs are not stored).  K-group i issues DMA i
  // (i < 3); K-group 3 none.
  uint32_t woff[kSkWDma];
#pragma unroll
  for (int i = 0; i < kSkWDma; i++) {
    const int p = 64 * i + lane;
    const int rr = p < 16 * kSkRowPieces ? p / kSkRowPieces : 0;
    const int row = min(n0 + rr, a.N - 1);
    woff[i] = (uint32_t)((size_t)row * w_row + 16 * (p % kSkRowPieces));
  }
  // The last W DMA has 16 W lanes; with SPLIT, the next Mh / 4 lanes bring the
  // stage's 1/s of the hi rows (Mh floats) to byte 2304 of the wave's W area.
  constexpr int kWLast = 16 * kSkRowPieces - 64 * (kSkWDma - 1);
  constexpr int kMh = MF == 1 ? 8 : 16;
  constexpr int kInvOff = 16 * kSkRowPieces * 16;  // 2304
  const int w_active = kWLast + (SPLIT && !INX ? kMh / 4 : 0);
  const bool inv_lane = SPLIT && !INX && lane >= kWLast;
  // X DMA i of this wave (0..15; only waves below kXTot / kXDma issue any)
  // covers pieces p = 64 (wave * kXDma + i) + lane of the chunk: row p / 32,
  // slot p % 32 holding logical piece (p % 32) ^ (row & 15).
  uint32_t xoff[G::kXDma];
#pragma unroll
  for (int i = 0; i < G::kXDma; i++) {
    const int p = 64 * (wave * G::kXDma + i) + lane;
    const int r = p >> 5;
    xoff[i] = (uint32_t)((size_t)r * x_row + 16 * ((p & 31) ^ (r & 15)));
  }
  // Stage s (clamped to the last one: the trailing requests re-read it into
  // slots no later stage reads) into ring slot s % kRing.
  auto issue = [&](int s) {
    const int gs = s0 + (s < steps ? s : steps - 1);
    uint8_t* slot = smem + kXOff + (s % G::kRing) * kSlotB;
    const uint8_t* xsrc = a.xa + (size_t)gs * kSkXRowBytes;
    if (xact) {
#pragma unroll
      for (int i = 0; i < G::kXDma; i++) dma16(xsrc + xoff[i], slot + (wave * G::kXDma + i) * 1024);
    }
    const uint8_t* wsrc = a.w + (size_t)gs * kSkRowBytes;
    uint8_t* wdst = slot + (INX ? 0 : G::kXBytes) + rw * kSkWBytes;
    if (kg == 0) {
      dma16(wsrc + woff[0], wdst);
    } else if (kg == 1) {
      dma16(wsrc + woff[1], wdst + 1024);
    } else if (kg == 2) {
      const uint8_t* last = wsrc + woff[kSkWDma - 1];
      if (inv_lane)
        last = reinterpret_cast<const uint8_t*>(a.inv_s + (size_t)gs * kMh + 4 * (lane - kWLast));
      if (lane < w_active) dma16(last, wdst + (kSkWDma - 1) * 1024);
    }
  };

  floatx4 acc[MF];
#pragma unroll
  for (int f = 0; f < MF; f++) acc[f] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  // All LDS operands of a stage are read first (one wait), then the four
  // block pairs are unpacked and multiplied.
  auto compute = [&](int slot_i, int ls) {
    floatx4 st_[MF];
#pragma unroll
    for (int f = 0; f < MF; f++) st_[f] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    floatx4(&st)[MF] = SPLIT ? st_ : acc;  // stage sums (SPLIT) or the totals
    // A rows and (SPLIT) 1/s of the stage; its W area
    const uint8_t* xs = INX ? smem + ls * kXStride : smem + slot_i * G::kSlot;
    const uint8_t* ws = INX ? smem + kXOff + slot_i * kSlotB : xs + G::kXBytes;
    const uint32_t* wr = reinterpret_cast<const uint32_t*>(ws + rw * kSkWBytes +
                                                           n16 * kSkRowBytes);
    // this K-group's block pairs jp = 2 kg, 2 kg + 1 of the stage: blocks 2 jp
    // (byte 36 jp of the row) and 2 jp + 1 (byte 36 jp + 18)
    constexpr int kJp = 1;
    uint32_t qe0[kJp], qe1[kJp], qo[kJp], se_bits[kJp], so_bits[kJp];
#pragma unroll
    for (int jj = 0; jj < kJp; jj++) {
      const int jp = kg + jj;
      const uint32_t* q = wr + 9 * jp;
      qe0[jj] = q[g];
      qe1[jj] = q[g + 1];
      qo[jj] = q[5 + g];
      se_bits[jj] = q[0];
      so_bits[jj] = q[4];
    }
    half8 xe[MF][kJp], xo[MF][kJp];
#pragma unroll
    for (int f = 0; f < MF; f++) {
      const uint8_t* xr = xs + (16 * f + n16) * kSkXRowBytes;  // A row of this lane
#pragma unroll
      for (int jj = 0; jj < kJp; jj++) {
        const int jp = kg + jj;
        xe[f][jj] = *reinterpret_cast<const half8*>(xr + (((8 * jp + g) ^ n16) << 4));
        xo[f][jj] = *reinterpret_cast<const half8*>(xr + (((8 * jp + 4 + g) ^ n16) << 4));
      }
    }
#pragma unroll
    for (int jp = 0; jp < kJp; jp++) {
      const half8 be = __builtin_bit_cast(
          half8, unpack8(__builtin_amdgcn_perm(qe1[jp], qe0[jp], 0x05040302u)));
      const half8 bo = __builtin_bit_cast(half8, unpack8(qo[jp]));
      const float se = f16_bits_to_f32(se_bits[jp] & 0xFFFFu);
      const float so = f16_bits_to_f32(so_bits[jp] >> 16);
#pragma unroll
      for (int f = 0; f < MF; f++) {
        const floatx4 pe = __builtin_amdgcn_mfma_f32_16x16x32_f16(
            xe[f][jp], be, floatx4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
        const floatx4 po = __builtin_amdgcn_mfma_f32_16x16x32_f16(
            xo[f][jp], bo, floatx4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; i++) st[f][i] = fmaf(so, po[i], fmaf(se, pe[i], st[f][i]));
      }
    }
    // SPLIT: this lane's tokens (4 g + i, hi and lo alike; g mod 2 when the hi
    // and lo rows share one frag) were scaled by s of this stage.
    if (SPLIT) {
      const uint8_t* ip = INX ? xs + G::kXBytes : ws + rw * kSkWBytes + kInvOff;
      const floatx4 inv =
          *reinterpret_cast<const floatx4*>(ip + 16 * (MF == 1 ? (g & 1) : g));
#pragma unroll
      for (int f = 0; f < MF; f++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[f][i] = fmaf(st[f][i], inv[i], acc[f][i]);
    }
  };

  if constexpr (INX) {
    // (token t < 8, local stage ls) pairs, 32 lanes each: lane gi takes
    // columns 8 gi .. 8 gi + 7 of the stage.  All x reads go out first, then
    // the ring's first W DMAs, then the conversion (which waits on the x
    // reads only).
    constexpr int kGroups = G::kThreads / 32;
    constexpr int kRounds = (kMh * kInxStages + kGroups - 1) / kGroups;
    const int gi = threadIdx.x & 31;
    const int pairs = kMh * steps;
    float v[kRounds][8];
#pragma unroll
    for (int r = 0; r < kRounds; r++) {
      const int p = (int)(threadIdx.x >> 5) + r * kGroups;
      const int t = p % kMh, ls = p / kMh;
      if (p < pairs && t < a.M) {
        const float* xp = a.x + (size_t)t * a.K + (size_t)(s0 + ls) * kSkStageK + 8 * gi;
        const float4 v0 = load_global<float4>(xp);
        const float4 v1 = load_global<float4>(xp + 4);
        v[r][0] = v0.x; v[r][1] = v0.y; v[r][2] = v0.z; v[r][3] = v0.w;
        v[r][4] = v1.x; v[r][5] = v1.y; v[r][6] = v1.z; v[r][7] = v1.w;
      } else {
#pragma unroll
        for (int k = 0; k < 8; k++) v[r][k] = 0.0f;
      }
    }
    for (int s = 0; s < G::kRing - 1; s++) issue(s);
#pragma unroll
    for (int r = 0; r < kRounds; r++) {
      const int p = (int)(threadIdx.x >> 5) + r * kGroups;
      if (p < pairs) {  // whole 32-lane groups
        const int t = p % kMh, ls = p / kMh;
        const StagePieces q = split_stage8(v[r]);
        uint8_t* xs = smem + ls * kXStride;
        const int rh = t, rl = kMh + t;  // hi and lo A rows; piece gi at slot gi ^ (row & 15)
        *reinterpret_cast<u32x4*>(xs + rh * kSkXRowBytes + ((gi ^ (rh & 15)) << 4)) = q.h;
        *reinterpret_cast<u32x4*>(xs + rl * kSkXRowBytes + ((gi ^ (rl & 15)) << 4)) = q.l;
        if (gi == 0) reinterpret_cast<float*>(xs + G::kXBytes)[t] = q.inv;
      }
    }
  } else {
    for (int s = 0; s < G::kRing - 1; s++) issue(s);
  }
  for (int s = 0; s < steps; s++) {
    // stage s landed (each wave waits for its own DMAs), slot of s-1 free
    // this wave's reads per stage: X pieces (xact) + one W DMA (K-groups 0-2)
    if (xact) {
      if (kg < 3)
        wait_reads_barrier<(G::kRing - 2) * (G::kXDma + 1)>();
      else
        wait_reads_barrier<(G::kRing - 2) * G::kXDma>();
    } else {
      if (kg < 3)
        wait_reads_barrier<(G::kRing - 2) * 1>();
      else
        wait_reads_barrier<0>();
    }
    issue(s + G::kRing - 1);
    compute(s % G::kRing, s);
  }
  // Trailing DMAs landed and every wave is done with the ring; then K-group 1
  // hands its sums to K-group 0 through LDS (a fixed order: deterministic).
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" : : : "memory");
  float* red = reinterpret_cast<float*>(smem) + ((size_t)(kg * RW + rw) * MF * 4) * 64 + lane;
  if (kg > 0) {
#pragma unroll
    for (int f = 0; f < MF; f++)
#pragma unroll
      for (int i = 0; i < 4; i++) red[(f * 4 + i) * 64] = acc[f][i];
  }
  __syncthreads();
  if (kg > 0) return;
#pragma unroll
  for (int g2 = 1; g2 < kSkKGroups; g2++)
#pragma unroll
    for (int f = 0; f < MF; f++)
#pragma unroll
      for (int i = 0; i < 4; i++) acc[f][i] += red[((size_t)g2 * RW * MF * 4 + (f * 4 + i)) * 64];

  // lane holds A rows 16 f + 4 g + i of W row n
  const int n = n0 + n16;
  const bool nvalid = n < a.N;
  float* out = a.splits > 1 ? a.part + (size_t)z * a.M * a.N : a.y;
  const float bv = (a.splits == 1 && a.bias && nvalid) ? a.bias[n] : 0.0f;
  if (SPLIT) {
    if (MF == 1) {  // hi rows 0..7 in lanes g 0-1, lo rows 8..15 in lanes g 2-3
#pragma unroll
      for (int i = 0; i < 4; i++) acc[0][i] += __shfl_down(acc[0][i], 32, 64);
      if (g < 2 && nvalid) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int tkn = 4 * g + i;
          if (tkn < a.M) out[(size_t)tkn * a.N + n] = acc[0][i] + bv;
        }
      }
    } else {  // hi frags 0 .. MF/2-1, lo frags MF/2 .. MF-1
#pragma unroll
      for (int f = 0; f < MF / 2; f++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int tkn = 16 * f + 4 * g + i;
          if (nvalid && tkn < a.M)
            out[(size_t)tkn * a.N + n] = (acc[f][i] + acc[f + MF / 2][i]) + bv;
        }
    }
  } else {
    // The exponents of this lane's 4 MF tokens, all read before any is used
    // (rows past M hold 0: the activation rows are padded).
    u32x4 ex[MF];
#pragma unroll
    for (int f = 0; f < MF; f++) ex[f] = load_global<u32x4>(a.xexp + 16 * f + 4 * g);
#pragma unroll
    for (int f = 0; f < MF; f++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int tkn = 16 * f + 4 * g + i;
        if (nvalid && tkn < a.M) out[(size_t)tkn * a.N + n] = ldexpf(acc[f][i], (int)ex[f][i]) + bv;
      }
  }
}

// y = sum of the split partials in split order (+ bias): deterministic.
__global__ void __launch_bounds__(256)
skinny_reduce_kernel(float* __restrict__ y, const float* __restrict__ part,
                     const float* __restrict__ bias, int M, int N, int splits) {
  const size_t mn = (size_t)M * N;
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= mn) return;
  // Eight planes' loads go out together, then the adds run in split order
  // (a loop of load-then-add waits a full memory latency per plane).
  float v = 0.0f;
  for (int z0 = 0; z0 < splits; z0 += 8) {
    float a[8];
#pragma unroll
    for (int k = 0; k < 8; k++) a[k] = z0 + k < splits ? part[(size_t)(z0 + k) * mn + i] : 0.0f;
#pragma unroll
    for (int k = 0; k < 8; k++)
      if (z0 + k < splits) v += a[k];
  }
  if (bias) v += bias[i % N];
  y[i] = v;
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

// Row groups per work-group: 64-row tiles (4) when they alone cover three
// quarters of the CUs.  Otherwise 16-row tiles (1) give four times the
// work-groups before any K split, and each re-reads the activation stages
// from L2: 2 N K MF bytes in all, against the reduction launch and the
// shallow K ranges a split of 64-row tiles costs.  Measured on the
// Mistral-7B shapes, the 16-row tiles win up to 64 MiB of such reads (q/o
// up to 32 tokens, k/v up to 64) and lose beyond (q/o at 64 tokens: 134 MB;
// down, K = 14336: 117 MB from 2 tokens on).
int skinny_rw(size_t n, size_t m, size_t batch, int num_cus) {
  if (((n + 63) / 64) * 4 >= (size_t)num_cus * 3) return 4;
  const size_t xbytes = 2 * n * m * (size_t)skinny_shape(batch).mf;
  return xbytes <= ((size_t)64 << 20) ? 1 : 4;
}

// K ranges per row tile: none when the row tiles alone cover three quarters
// of the CUs (a split costs a reduction launch), else about `target`
// work-groups in all: two per CU for single-fragment tiles, one otherwise
// (measured on 16-row k/v tiles: 8 splits at M = 8 8.5 µs per call against
// 9.4 with 12, 4 splits at M = 16 9.4 against 9.7 with 8), at most one range
// per stage.
int skinny_splits(size_t n, size_t m, size_t batch, int num_cus) {
  const SkinnyShape sh = skinny_shape(batch);
  const int rw = skinny_rw(n, m, batch, num_cus);
  const size_t rows = 16 * (size_t)rw;
  const size_t tiles = (n + rows - 1) / rows;
  const size_t per_cu = sh.mf == 1 ? 2 : 1;
  const size_t target = (size_t)num_cus * per_cu;
  size_t sp = tiles * 4 >= (size_t)num_cus * 3 ? 1 : (target + tiles / 2) / tiles;
  const size_t gsteps = m / kSkStageK;
  if (sp < 1) sp = 1;
  if (sp > gsteps) sp = gsteps;
  return (int)sp;
}

template <int MF, bool SPLIT, int RW, bool INX = false>
hipError_t launch_mf(const SkinnyArgs& a, dim3 grid, hipStream_t s) {
  using G = SkGeom<MF, RW>;
  constexpr int kInxLds = kInxStages * (G::kXBytes + 64) + G::kRing * RW * kSkWBytes;
  constexpr int lds = INX ? kInxLds : G::kLds;
  static_assert(lds <= 160 * 1024 && G::kWaves * MF * 4 * 64 * 4 <= lds, "LDS budget");
  hipError_t e = set_lds_limit(
      reinterpret_cast<const void*>(q4_0_skinny_kernel<MF, SPLIT, RW, INX>), lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((q4_0_skinny_kernel<MF, SPLIT, RW, INX>), grid, dim3(G::kThreads), lds, s, a);
  return hipGetLastError();
}

template <int MF, bool SPLIT>
hipError_t launch_rw(const SkinnyArgs& a, int rw, dim3 grid, hipStream_t s) {
  return rw == 4 ? launch_mf<MF, SPLIT, 4>(a, grid, s) : launch_mf<MF, SPLIT, 1>(a, grid, s);
}

}  // namespace

bool q4_0_skinny_ok(const uint8_t* w, size_t w_len, size_t n, size_t m, size_t batch, int num_cus) {
  (void)num_cus;
  if (batch < 2 || batch > 64 || n == 0 || m == 0) return false;
  if (m % kSkStageK != 0 || ((uintptr_t)w & 15) != 0) return false;
  // 32-bit piece offsets within W and X
  if (n * (m / kBlockElems) * kBlockBytes > 0xFFFFFFFFull || 64 * m * 2 > 0xFFFFFFFFull) return false;
  if (n > (size_t)0x7FFFFFFF || m > (size_t)0x7FFFFFF) return false;
  return w_len / kBlockBytes >= n * (m / kBlockElems);
}

static size_t round256(size_t v) { return (v + 255) / 256 * 256; }

// Workspace: A rows, the split mode's 1/s table, the plain mode's per-token
// exponents (64 ints), the K-split partial planes.
size_t skinny_workspace_bytes(size_t batch, size_t n, size_t m, int num_cus) {
  const SkinnyShape sh = skinny_shape(batch);
  const int sp = skinny_splits(n, m, batch, num_cus);
  size_t b = round256((size_t)sh.rows * m * 2) + round256(m / kSkStageK * 16 * 4) + 256;
  if (sp > 1) b += (size_t)sp * batch * n * 4;
  return b;
}

hipError_t launch_q4_0_skinny(float* y, const uint8_t* w, const float* x, const float* bias,
                              size_t n, size_t m, size_t batch, void* ws, int num_cus,
                              hipStream_t s) {
  const SkinnyShape sh = skinny_shape(batch);
  uint8_t* xa = static_cast<uint8_t*>(ws);
  float* inv_s = reinterpret_cast<float*>(xa + round256((size_t)sh.rows * m * 2));
  int* xexp = reinterpret_cast<int*>(reinterpret_cast<uint8_t*>(inv_s) +
                                     round256(m / kSkStageK * 16 * 4));
  float* part = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(xexp) + 256);
  hipError_t e;
  const int sp = skinny_splits(n, m, batch, num_cus);
  const size_t gsteps = m / kSkStageK;
  // 16-row tiles whose K is split into ranges of a few stages: the kernel
  // converts its own stages of X (no pre-pass launch).  Measured on the
  // Mistral shapes at 5-8 tokens: k/v (16-row tiles, 2 stages per range) 7.7
  // against 8.5 us per call; down (64-row tiles, 7 stages per range) 2.5 us
  // slower, so 64-row tiles keep the pre-pass.
  const int rw = skinny_rw(n, m, batch, num_cus);
  const bool inx = sh.split && sh.mf == 1 && sp > 1 && rw == 1 &&
                   (gsteps + sp - 1) / sp <= (size_t)kInxStages && ((uintptr_t)x & 15) == 0;
  if (inx) {
    e = hipSuccess;
  } else if (sh.split) {
    const int stages = (int)(m / kSkStageK);
    hipLaunchKernelGGL(x_skinny_kernel, dim3((unsigned)((stages + 7) / 8), (unsigned)sh.mh),
                       dim3(256), 0, s, xa, inv_s, x, (int)batch, (int)m, sh.mh, sh.split);
    e = hipGetLastError();
  } else {
    e = launch_x_rows_f16(x, batch, (size_t)sh.rows, m, xa, xexp, true, s);
  }
  if (e != hipSuccess) return e;
  SkinnyArgs a;
  a.y = y;
  a.part = part;
  a.w = w;
  a.xa = xa;
  a.x = x;
  a.inv_s = inv_s;
  a.xexp = xexp;
  a.bias = bias;
  a.M = (int)batch;
  a.N = (int)n;
  a.K = (int)m;
  a.split = sh.split;
  a.splits = sp;
  const dim3 grid((unsigned)((n + 16 * rw - 1) / (16 * rw)), (unsigned)sp);
  if (inx)
    e = launch_mf<1, true, 1, true>(a, grid, s);
  else if (sh.mf == 1)
    e = launch_rw<1, true>(a, rw, grid, s);
  else if (sh.mf == 2)
    e = sh.split ? launch_rw<2, true>(a, rw, grid, s) : launch_rw<2, false>(a, rw, grid, s);
  else
    e = launch_rw<4, false>(a, rw, grid, s);
  if (e != hipSuccess || sp == 1) return e;
  const size_t mn = batch * n;
  hipLaunchKernelGGL(skinny_reduce_kernel, dim3((unsigned)((mn + 255) / 256)), dim3(256), 0, s, y,
                     part, bias, (int)batch, (int)n, sp);
  return hipGetLastError();
}

}  // namespace hypno
