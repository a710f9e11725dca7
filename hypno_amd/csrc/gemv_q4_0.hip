// Q4_0 and Q8_0 matrix-vector kernels for gfx950.
//
//  * q4_0_generic_kernel: any m (blocks straddling rows), any alignment, short
//    weight buffers, bias, and any number of tokens.  One wave per
//    (token, row); lanes walk the row's overlapping blocks.  Semantics follow
//    matmul_q4_0_scalar (kernels.rs:362-400).
//  * q4_0_gemv_jobs_kernel: the decode GEMV (one token) over one job or a
//    table of independent jobs in a single launch.  See the comment above it.
//  * q8_0_generic_kernel / q8_0_gemv_jobs_kernel: the same for Q8_0 weights
//    (ops.rs:33-36 semantics: dequantised rows, fp32 accumulation); the
//    streaming kernel is the Q4_0 one instantiated for 34-byte blocks.
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

// Q8_0 for any shape: ops.rs:33-36 dequantises the tensor and runs matmul_f32
// over the flattened rows [r*m, (r+1)*m) (kernels.rs:234-241), so a block
// may straddle two rows.  One wave per (token, row); lanes take the row's
// elements in strides of 64.  The caller guarantees the buffer holds all
// n*m elements (a shorter one is a panic in the reference).
__global__ void __launch_bounds__(256)
q8_0_generic_kernel(float* __restrict__ y, const uint8_t* __restrict__ w,
                    const float* __restrict__ x, const float* __restrict__ bias, size_t n,
                    size_t m, size_t batch) {
  const size_t wave = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (wave >= n * batch) return;  // wave-uniform
  const size_t t = wave / n;
  const size_t r = wave - t * n;
  const float* xt = x + t * m;
  float acc = 0.0f;
  for (size_t j = lane; j < m; j += 64) {
    const size_t e = r * m + j;
    const uint8_t* blk = w + (e / kBlockElems) * kQ8BlockBytes;
    const float d = f16_bits_to_f32((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
    acc = fmaf((float)((int)blk[2 + e % kBlockElems] - 128) * d, xt[j], acc);
  }
  acc = wave_sum(acc);
  if (lane == 0) y[t * n + r] = acc + (bias ? bias[r] : 0.0f);
}

hipError_t launch_q8_0_generic(float* y, const uint8_t* w, const float* x, const float* bias,
                               size_t n, size_t m, size_t batch, hipStream_t s) {
  const size_t waves = n * batch;
  if (waves == 0) return hipSuccess;
  const size_t grid = (waves + 3) / 4;
  hipLaunchKernelGGL(q8_0_generic_kernel, dim3((unsigned)grid), dim3(256), 0, s, y, w, x, bias, n,
                     m, batch);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Streaming decode GEMV over a table of jobs (one token, m % 256 == 0)
//
// A row of m weights is B = m/32 blocks of 18 bytes.  A work-group of T
// threads treats rps = T/B consecutive rows of a job (T blocks, contiguous in
// memory) as one step; thread t owns block t % B of row t / B in every step
// of that job, so its 32 activations stay in registers while the job lasts.
// T is a multiple of lcm(B, 64) for every job of the launch, so every lane
// has a block.
//
// The steps of all jobs form one global sequence; each work-group takes a
// contiguous range of it (possibly spanning jobs).  The 64 blocks a wave owns
// in a step are one contiguous 1152-byte span; LDS DMA copies it into the
// wave's own ring of two or three step slots in LDS (one 1 KB and one
// 128-byte non-temporal piece, so every cache line is read by exactly one
// instruction), running ahead across job boundaries, and each lane reads its
// block back as the 20-byte window [18 lane & ~3, +20) of the span.  The
// ring is private to the wave, so no barrier orders it: a wave waits only
// for its own oldest DMAs.  A block starts at byte 0 or 2 of its window:
// three window dwords and one lane-dependent byte permute give its nibble
// dwords (in an order the activation digits follow); nib ^ 8 read
// as a signed i4 is nib - 8, and v_dot8_i32_i4
// multiplies eight of them with eight i4 digits of the block's activations
// (the limbs below) into an exact int32 sum; the limb sums combine into one
// fp32 value that the block scale d and the block's exponent scale.  Each
// step, DPP row shifts add the partials of
// aligned 8-lane groups (a row is B/8 whole groups), and the group sums of S
// steps are parked in LDS; after one barrier one thread per row adds its
// groups in a fixed order (deterministic) and writes y.  Activations are
// restaged (coalesced, through LDS with an XOR swizzle) only when the job
// changes.
//
// Bounds: the DMAs read through a buffer resource sized to the step's valid
// bytes, so nothing past a job's last row is read (out-of-range dwords
// arrive as zeros, in rows that are never written).
// ---------------------------------------------------------------------------

// Activations as exact integer limbs.  For each block of 32 activations let
// e be the exponent of its largest |x| (amax < 2^e).  m = rint(x * 2^(18-e))
// has |m| <= 2^18, and m + kDigitBias (kDigitBias = sum_l 8 * 16^l) lies in
// [0, 16^5), so m = sum_l 16^l * (u_l - 8) with u_l its base-16 digits; the
// signed digit u_l - 8 is stored as the i4 value u_l ^ 8.  The dot product of
// a block with (nib - 8) is then 2^(e-18) * sum_l 16^l * D_l with D_l an
// exact integer dot product of i4 values (|D_l| <= 32 * 64).  The only
// rounding besides fp32 arithmetic on the block result is that of x to m: at
// most 2^-19 of the block's largest |x| (a normwise error near 1e-6 on
// N(0,1) activations, against the 1e-4 bound), for 20 dot instructions per
// block.
//
// Q8_0 blocks (34 bytes: fp16 d, then 32 bytes u = q + 128) use the same
// scheme with signed base-256 digits: m = rint(x * 2^(22-e)), |m| <= 2^22,
// m + 0x808080 in [0, 2^24) split into three bytes u_l, the digit u_l - 128
// stored as the i8 value u_l ^ 0x80; v_dot4_i32_i8 multiplies four
// (u - 128) weights (u ^ 0x80 read as i8) with four digits, 24 dot
// instructions per block, x rounded to 2^-23 of the block's largest |x|.
template <int F>
struct Fmt;
template <>
struct Fmt<kFmtQ4_0> {
  static constexpr int kBytes = 18;       // block bytes
  static constexpr int kLimbs = 5;        // digits of x
  static constexpr int kLimbDwords = 4;   // dwords per block per digit plane
  static constexpr int kMantBits = 18;
  static constexpr int kDigitBias = 0x88888;
};
template <>
struct Fmt<kFmtQ8_0> {
  static constexpr int kBytes = 34;
  static constexpr int kLimbs = 3;
  static constexpr int kLimbDwords = 8;
  static constexpr int kMantBits = 22;
  static constexpr int kDigitBias = 0x808080;
};
constexpr int kBadExp = -100000;  // block with inf or NaN activations

static int gcd_int(int a, int b) {
  while (b) {
    int t = a % b;
    a = b;
    b = t;
  }
  return a;
}

static int lcm_int(int a, int b) { return a / gcd_int(a, b) * b; }

// Threads needed so that every lane owns a block of a row with B blocks.
static int job_threads(int B) {
  const int l = lcm_int(B, 64);
  return l <= 1024 ? l : -1;
}

// T: the threads per work-group (a multiple of Tbase up to 1024); 0 picks
// Tbase doubled up to at least 256.
static void finish_geometry(GemvGroupGeom& g, int T = 0) {
  g.T = T > 0 ? T : g.Tbase;
  while (T <= 0 && g.T < 256 && 2 * g.T <= 1024) g.T *= 2;
  g.W = g.T / 64;
  g.S = 64 / g.rows;  // steps per partial-sum chunk, per x row
  const size_t loop = (size_t)g.S * (g.T / 8) * 4 * g.rows;  // 8-lane group partials
  // activation digits and exponents, then one float per wave (prologue sums)
  const size_t digits = g.fmt == kFmtQ8_0 ? 4 * Fmt<kFmtQ8_0>::kLimbs * 8
                                          : 4 * Fmt<kFmtQ4_0>::kLimbs * 4;
  const size_t xs = (size_t)g.maxB * (digits + 4) + 4 * (size_t)g.W;
  g.ring_off = ((xs > loop ? xs : loop) + 15) & ~(size_t)15;
  // Each wave's ring of weight spans (64 blocks per step) follows: three
  // steps deep when two work-groups still share a CU, else two.
  const size_t span = 64 * (size_t)(g.fmt == kFmtQ8_0 ? Fmt<kFmtQ8_0>::kBytes : kBlockBytes);
  g.ring = 2 * (g.ring_off + (size_t)g.W * 3 * span) <= 160 * 1024 ? 3 : 2;
  g.lds = g.ring_off + (size_t)g.W * g.ring * span;
}

static const size_t kMaxLds = 160 * 1024;  // gfx950 LDS per work-group

bool gemv_group_add(GemvGroupGeom& g, size_t m) {
  if (m == 0 || m % 256 != 0 || m > 65536) return false;
  const int B = (int)(m / 32);
  const int T = job_threads(B);
  if (T < 0) return false;
  GemvGroupGeom t = g;
  t.Tbase = t.Tbase ? lcm_int(t.Tbase, T) : T;
  if (t.Tbase > 1024) return false;
  t.maxB = t.maxB > B ? t.maxB : B;
  finish_geometry(t);
  if (t.lds > kMaxLds) return false;
  g = t;
  return true;
}

// Work-groups a launch runs at most, per CU, by the staging rule below
// (launch_q4_0_gemv_group): every work-group stages the whole x, so each
// should stream at least about twice that in weights.
static long long gemv_per_cu(const GemvGroupGeom& g, long long wbytes, int num_cus) {
  const long long stage = 4LL * kBlockElems * g.maxB * (g.pro ? 2 : 1);
  const long long ws = wbytes / (2 * stage);
  const long long per = (ws + num_cus / 2) / num_cus;
  return per > 1 ? per : 1;
}

void gemv_group_widen(GemvGroupGeom& g, const int* n, const int* B, int count, int num_cus) {
  const int bytes = g.fmt == kFmtQ8_0 ? Fmt<kFmtQ8_0>::kBytes : kBlockBytes;
  long long wbytes = 0;
  for (int i = 0; i < count; i++) wbytes += (long long)n[i] * B[i] * bytes;
  if (gemv_per_cu(g, wbytes, num_cus) > 1) return;
  int top = g.Tbase;
  while (2 * top <= 1024) top *= 2;
  for (int T = top; T > g.T; T /= 2) {
    long long steps = 0;
    for (int i = 0; i < count; i++) {
      const int rps = T / B[i];
      steps += (n[i] + rps - 1) / rps;
    }
    if (steps < num_cus) continue;
    GemvGroupGeom t = g;
    finish_geometry(t, T);
    if (t.lds > kMaxLds) continue;
    g = t;
    return;
  }
}

bool q4_0_gemv_fast_ok(const uint8_t* w, size_t w_len, size_t n, size_t m) {
  if (n == 0 || n > (size_t)0x3FFFFFFF) return false;
  if (((uintptr_t)w & 15) != 0) return false;
  GemvGroupGeom g;
  if (!gemv_group_add(g, m)) return false;
  return w_len / kBlockBytes >= n * (m / kBlockElems);
}

bool q8_0_gemv_fast_ok(const uint8_t* w, size_t w_len, size_t n, size_t m) {
  if (n == 0 || n > (size_t)0x3FFFFFFF) return false;
  if (((uintptr_t)w & 15) != 0) return false;
  GemvGroupGeom g;
  g.fmt = kFmtQ8_0;
  if (!gemv_group_add(g, m)) return false;
  return w_len / Fmt<kFmtQ8_0>::kBytes >= n * (m / kBlockElems);
}

// Prefetch cursor (work-group uniform): the job the ring is reading and the
// address of the next step to fetch.
struct RingCursor {
  const uint8_t* next;  // first byte of the next step to fetch
  int bps;              // bytes per step = rps * B * block bytes
  int end;              // one past the job's last global step
  int last_units;       // blocks in the job's last (possibly partial) step
  int j;
};

__device__ __forceinline__ int job_steps(const GemvJob& J) { return (J.n + J.rps - 1) / J.rps; }

// Raw buffer resource over [base, base + bytes) for dword accesses (word 3:
// 32-bit data format); loads at offsets past `bytes` return zeros, checked
// per dword.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}

// LDS DMA, non-temporal: 16 bytes per lane from rs at byte offset voff to
// LDS dst + 16 * lane (dst wave-uniform).
__device__ __forceinline__ void lds_dma16_nt(__amdgpu_buffer_rsrc_t rs, uint8_t* dst,
                                             uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)dst, 16,
                                           voff, 0, 0, 2);
}

// First product of a v_dot8_i32_i4 chain, in the form with an inline zero
// accumulator (no register to clear first).
__device__ __forceinline__ int sdot8_first(uint32_t a, uint32_t b) {
  int r;
  asm("v_dot8_i32_i4 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

// PRO: some job of the launch has a prologue (a separate instantiation, so
// launches without one keep the smaller staging code and register budget).
// The launch's leading kernel arguments, preloaded into SGPRs (the build
// preloads this file's first 11 arguments: these, in this order, 14 SGPRs):
// the launch shape and the first job's streaming fields.  aux0 is null
// unless job 0 has a prologue.
struct GemvHead {
  int total_steps, grid, T, ring_off, njobs, n0, B0, rps0;
  const uint8_t* w0;
  const float* x0;
  const float* aux0;
};

// MR: rows of x (consecutive, K floats apart) multiplied by the same weights
// in one pass (y rows n floats apart); only with one plain Q4_0 job.
template <int F, bool PRO, int R, int MR = 1>
__device__ __forceinline__ void gemv_jobs_body(const GemvHead& H, const GemvLaunch& L) {
  static_assert(MR == 1 || !PRO, "several rows: no prologue");
  using FT = Fmt<F>;
  constexpr int kLimbs = FT::kLimbs;
  constexpr int kLD = FT::kLimbDwords;
  constexpr int kMantBits = FT::kMantBits;
  constexpr int kDigitBias = FT::kDigitBias;
  extern __shared__ __align__(16) uint8_t smem[];
  const int T = H.T;
  const int t = threadIdx.x;
  const int G = H.total_steps;
  const uint32_t gd = (uint32_t)H.grid, gb = blockIdx.x;
  const bool narrow = (uint32_t)G <= 0xFFFFFFFFu / gd;  // G * gd fits 32 bits
  const int s_begin = narrow ? (int)((uint32_t)G * gb / gd)
                             : (int)((unsigned long long)G * gb / gd);
  const int s_end = narrow ? (int)((uint32_t)G * (gb + 1) / gd)
                           : (int)((unsigned long long)G * (gb + 1) / gd);
  if (s_begin >= s_end) return;  // whole work-group

  // Jobs come from the launch's arguments (up to kGemvInline of them), else
  // from the device table.
  const bool inl = H.njobs <= kGemvInline;
  auto get = [&](int j) -> GemvJob {
    return inl ? L.inl[j] : load_const<GemvJob>(L.jobs + j);
  };
  auto cursor_of = [&](const GemvJob& J, int j, int g) {
    const int steps = job_steps(J);
    RingCursor c;
    c.bps = J.rps * J.B * FT::kBytes;
    c.next = J.w + (size_t)(g - J.step0) * c.bps;
    c.end = J.step0 + steps;
    c.last_units = (J.n - (steps - 1) * J.rps) * J.B;
    c.j = j;
    return c;
  };
  auto cursor_at = [&](int j, int g) { return cursor_of(get(j), j, g); };
  // First job of this work-group's range (binary search on step0).
  int j0 = 0;
  if (inl) {
    // step0 rises with the job: j0 counts the later jobs starting at or
    // before s_begin (constant indices, so the loads go out together)
#pragma unroll
    for (int k = 1; k < kGemvInline; k++) j0 += (k < H.njobs && L.inl[k].step0 <= s_begin) ? 1 : 0;
  } else {
    int lo = 0, hi = H.njobs - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (load_const<int>(&L.jobs[mid].step0) <= s_begin)
        lo = mid;
      else
        hi = mid - 1;
    }
    j0 = lo;
  }
  // The first job's activations (and prologue operand), element groups
  // i = t + p T for p < kPre, are read now, before anything waits on memory:
  // their latency runs alongside the weight ring's first fetches.
  constexpr int kPre = 2;
  GemvJob J0;
  if (inl) {  // constant indices again: no load waits on j0
    J0 = L.inl[0];
#pragma unroll
    for (int k = 1; k < kGemvInline; k++)
      if (k == j0) J0 = L.inl[k];
  } else {
    J0 = load_const<GemvJob>(L.jobs + j0);
  }
  // What the first reads need, from the preloaded head for job 0 (a uniform
  // branch: that path waits on no argument memory)
  GemvJob F0;
  const float* aux_first;
  if (j0 == 0) {
    F0.w = H.w0;
    F0.x = H.x0;
    F0.n = H.n0;
    F0.B = H.B0;
    F0.rps = H.rps0;
    F0.step0 = 0;
    aux_first = H.aux0;
  } else {
    F0 = J0;
    aux_first = J0.pro != kProNone ? J0.aux : nullptr;
  }
  float xpre[kPre][8], apre[kPre][8] = {};
  auto load8 = [&](const float4* p, int i, float* o) __attribute__((always_inline)) {
    const float4 v0 = load_global<float4>(p + 2 * i);
    const float4 v1 = load_global<float4>(p + 2 * i + 1);
    o[0] = v0.x; o[1] = v0.y; o[2] = v0.z; o[3] = v0.w;
    o[4] = v1.x; o[5] = v1.y; o[6] = v1.z; o[7] = v1.w;
  };
#pragma unroll
  for (int p = 0; p < kPre; p++) {
    const int i = t + p * T;
    if (i < F0.B * 4) {
      load8(reinterpret_cast<const float4*>(F0.x), i, xpre[p]);
      if (PRO && aux_first != nullptr) load8(reinterpret_cast<const float4*>(aux_first), i, apre[p]);
    }
  }

  // The weights stream through a ring of R step spans per wave in LDS, filled
  // by LDS DMA: each wave owns blocks [64w, 64w + 64) of every step, i.e. the
  // span of 64 * kBytes contiguous bytes at 64w * kBytes, fetched as whole
  // 1 KB pieces plus one 128-byte piece (every cache line read by one
  // instruction, non-temporal).  The DMAs go through a buffer resource whose
  // size is the step's valid bytes (0 past the work-group's range), so a
  // partial last step or the ring's run-out past s_end reads zeros instead
  // of memory beyond the job; the range check is per dword and valid bytes
  // are a multiple of 4.  The job table is read only when the ring crosses
  // into the next job.
  constexpr int kSpan = 64 * FT::kBytes;
  constexpr int kFull = kSpan / 1024;        // whole 1 KB pieces per span
  static_assert(kSpan - kFull * 1024 == 128, "span = whole KBs + 128 bytes");
  constexpr int kDmaPerStep = kFull + 1;
  const int lane = t & 63;
  const int wv = __builtin_amdgcn_readfirstlane(t >> 6);  // wave-uniform
  uint8_t* ring = smem + H.ring_off + (size_t)wv * (R * kSpan);
  RingCursor pc = cursor_of(F0, j0, s_begin);
  int pg = s_begin;  // next step the ring fetches
  const uint8_t* wsafe = pc.next;
  const uint32_t dma_off = (uint32_t)(wv * kSpan + 16 * lane);
  auto issue = [&](int slot) {
    const uint8_t* base = wsafe;
    int nrec = 0;
    if (pg < s_end) {
      if (pg == pc.end) pc = cursor_at(pc.j + 1, pg);
      base = pc.next;
      nrec = pg == pc.end - 1 ? pc.last_units * FT::kBytes : pc.bps;
      pc.next += pc.bps;
    }
    pg++;
    const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(base, nrec);
    uint8_t* dst = ring + slot * kSpan;
#pragma unroll
    for (int k = 0; k < kFull; k++) lds_dma16_nt(rs, dst + 1024 * k, dma_off + 1024 * k);
    if (lane < 8) lds_dma16_nt(rs, dst + 1024 * kFull, dma_off + 1024 * kFull);
  };
  // Window start inside a wave's span: the lane's block at byte kBytes *
  // lane, rounded down to a dword (a block starts at byte 0 or 2 of its
  // window; the span's last block has an odd lane, so its window ends with
  // the span).
  const uint32_t win = (uint32_t)(FT::kBytes * lane) & ~3u;
#pragma unroll
  for (int k = 0; k < R; k++) issue(k);

  // Byte selectors for v_perm_b32: a block starts at byte 0 (t even) or 2
  // (t odd) of its window; weight dword j is bytes [2+4j, 6+4j) of the block
  // (Q8_0), and (Q4_0) the permute of window dwords 0 and 4 gives nibble
  // bytes {0, 1, 14, 15} (t even) or 12-15 (t odd).
  const bool odd = (t & 1) != 0;
  const uint32_t sel_q = odd ? 0x07060504u : 0x05040302u;
  const uint32_t sh_d = odd ? 16u : 0u;

  // [S][T/8] sums of 8-lane groups (a row of B blocks is B/8 whole groups
  // because B % 8 == 0); aliases the activation staging area.
  float* part = reinterpret_cast<float*>(smem);
  const int T8 = __builtin_amdgcn_readfirstlane(T >> 3);

  // State of the job being computed (work-group uniform except the limbs).
  GemvJob J = get(j0);
  int cj = j0;
  int seg_end = s_begin;  // end of this work-group's steps of job cj
  int c0 = s_begin;       // first step of the open partial-sum chunk
  u32x4 xl[MR][kLimbs * kLD / 4];  // this lane's block column of each x row as digit planes
  int xe[MR] = {};       // its exponent: x = 2^xe * sum_k base^k * digit_k
  float xnan[MR] = {};   // NaN when the block holds a non-finite activation

  // Sum the parked partials of steps [c0, c1) into y (one thread per row, in
  // a fixed order).  Row starts in `part` are 16-byte aligned when B8 % 4 == 0
  // and 8-byte aligned when B8 is even (T8 is a multiple of 8), so the reads
  // are vectorised with independent partial sums.  The bias branch is
  // uniform and kept apart: a bias load waited for in the common path would
  // also wait for every ring DMA in flight.
  auto row_sum = [&](const float* pr, int B8) -> float {
    if ((B8 & 3) == 0) {
      float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
      const float4* p4 = reinterpret_cast<const float4*>(pr);
#pragma unroll 4
      for (int q = 0; q < (B8 >> 2); q++) {
        const float4 v = p4[q];
        a0 += v.x; a1 += v.y; a2 += v.z; a3 += v.w;
      }
      return (a0 + a1) + (a2 + a3);
    }
    if ((B8 & 1) == 0) {
      float a0 = 0.0f, a1 = 0.0f;
      const float2* p2 = reinterpret_cast<const float2*>(pr);
#pragma unroll 1
      for (int q = 0; q < (B8 >> 1); q++) {
        const float2 v = p2[q];
        a0 += v.x; a1 += v.y;
      }
      return a0 + a1;
    }
    float a0 = 0.0f;
    for (int q = 0; q < B8; q++) a0 += pr[q];
    return a0;
  };
  auto flush = [&](int c1) {
    __syncthreads();
    const int rps = J.rps, B8 = J.B >> 3;
    const int row0 = (c0 - J.step0) * rps;
    const int nrows = min((c1 - c0) * rps, J.n - row0);
#pragma unroll
    for (int m = 0; m < MR; m++) {  // x row m's partials follow row m-1's S steps
      float* yr = J.y + (size_t)m * J.n + row0;
      const float* pm = part + m * L.S * T8;
      if (J.bias == nullptr) {
        for (int r = t; r < nrows; r += T) {
          const int sl = r / rps;
          yr[r] = row_sum(pm + sl * T8 + (r - sl * rps) * B8, B8);
        }
      } else {
        const float* br = J.bias + row0;
        for (int r = t; r < nrows; r += T) {
          const int sl = r / rps;
          yr[r] = row_sum(pm + sl * T8 + (r - sl * rps) * B8, B8) + br[r];
        }
      }
    }
    __syncthreads();
  };
  // Make job j current at global step g: convert its activations to i4 limbs
  // (cooperatively: thread i handles elements [8i, 8i+8) of x, four threads
  // per block), park them in LDS as [limb][block][4 dwords] plus one
  // exponent per block, and keep this lane's block column in registers.
  // A prologue first turns x into rms_norm(x) or silu(x) * up, element by
  // element in registers (the RMS sum: per-thread FMA chains, wave sums, then
  // the waves' sums in a fixed order, so every work-group gets the same
  // scale).
  auto enter = [&](int j, int g, bool first) __attribute__((always_inline)) {
    J = first ? J0 : get(j);
    cj = j;
    const int steps = job_steps(J);
    seg_end = min(s_end, J.step0 + steps);
    c0 = g;
    const int B = J.B;
    uint32_t* limbs = reinterpret_cast<uint32_t*>(smem);
    int* exps = reinterpret_cast<int*>(smem + (size_t)kLimbs * kLD * 4 * B);
    const float4* xv = reinterpret_cast<const float4*>(J.x);
    const float4* av = reinterpret_cast<const float4*>(J.aux);
    int row = 0;  // the x row being staged (xv points at it)
    // element group i's x (and prologue operand): from the registers read
    // at the start for the first job's first kPre rounds (of x row 0)
    auto get8 = [&](int i, int p, float* xs, float* as) __attribute__((always_inline)) {
      if (first && row == 0 && p < kPre) {
#pragma unroll
        for (int k = 0; k < 8; k++) {
          xs[k] = xpre[p][k];
          if (PRO) as[k] = apre[p][k];
        }
      } else {
        load8(xv, i, xs);
        if (PRO && J.pro != kProNone) load8(av, i, as);
      }
    };
    auto sumsq8 = [&](const float* xs, float ss) __attribute__((always_inline)) {
#pragma unroll
      for (int k = 0; k < 8; k++) ss = fmaf(xs[k], xs[k], ss);
      return ss;
    };
    // Sum of the work-group's partial sums in a fixed order; the last
    // barrier also orders the limb writes below after every wsum read.
    auto inv_rms_of = [&](float ss) __attribute__((always_inline)) {
      float* wsum = reinterpret_cast<float*>(exps + B);
      ss = wave_sum(ss);
      if ((t & 63) == 0) wsum[t >> 6] = ss;
      __syncthreads();
      float tot = 0.0f;
      for (int w = 0; w < (T >> 6); w++) tot += wsum[w];
      return 1.0f / sqrtf(tot / (float)(B * 32) + J.eps);
    };
    auto prologue = [&](float* xs, const float* as, float inv_rms) __attribute__((always_inline)) {
      if (J.pro == kProRmsNorm) {
#pragma unroll
        for (int k = 0; k < 8; k++) xs[k] = xs[k] * inv_rms * as[k];
      } else if (J.pro == kProSiluMul) {
#pragma unroll
        for (int k = 0; k < 8; k++) xs[k] = xs[k] / (1.0f + expf(-xs[k])) * as[k];
      }
    };
    // Group i (elements [8i, 8i+8)) -> i4 limbs and, for the block's first
    // group, the block exponent.  The four groups of a block are consecutive
    // lanes, all active together.
    auto convert = [&](int i, const float* xs) __attribute__((always_inline)) {
      // Largest |x| of the block by its bit pattern (ordered like the value
      // for non-negative floats; inf and NaN compare above every finite).
      uint32_t mb = 0;
#pragma unroll
      for (int k = 0; k < 8; k++) mb = max(mb, __float_as_uint(xs[k]) & 0x7FFFFFFFu);
      // the block's four lanes (a quad): DPP quad_perm [1,0,3,2], then [2,3,0,1]
      mb = max(mb, (uint32_t)__builtin_amdgcn_mov_dpp((int)mb, 0xB1, 0xF, 0xF, false));
      mb = max(mb, (uint32_t)__builtin_amdgcn_mov_dpp((int)mb, 0x4E, 0xF, 0xF, false));
      const int e = __builtin_amdgcn_frexp_expf(__uint_as_float(mb));  // amax < 2^e
      uint32_t u[8];
#pragma unroll
      for (int k = 0; k < 8; k++)
        u[k] = (uint32_t)((int)rintf(ldexpf(xs[k], kMantBits - e)) + kDigitBias);
      if constexpr (F == kFmtQ4_0) {
        // Plane l holds digit l (bits 4l..4l+3) of the 8 values, value k in
        // nibble k.  Per pair (u[2p], u[2p+1]): e_p bytes 0..2 = digits 0, 2,
        // 4 of both (low nibble the even value), o_p bytes 0..1 = digits 1,
        // 3; then v_perm_b32 gathers byte b of the four pairs into a plane.
        static_assert(kLimbs == 5, "five 4-bit digits");
        uint32_t e[4], o[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const uint32_t a = u[2 * q], b = u[2 * q + 1];
          e[q] = (a & 0x000F0F0Fu) | ((b & 0x000F0F0Fu) << 4);
          o[q] = ((a >> 4) & 0x00000F0Fu) | (b & 0x0000F0F0u);
        }
        // bytes [x0.b0, x1.b0, x0.b1, x1.b1] of (x1:x0), and the same of the
        // odd pair; then [lo.b0, lo.b1, hi.b0, hi.b1] / [lo.b2, lo.b3, hi.b2, hi.b3]
        const uint32_t ea = __builtin_amdgcn_perm(e[1], e[0], 0x05010400u);
        const uint32_t eb = __builtin_amdgcn_perm(e[3], e[2], 0x05010400u);
        const uint32_t ec = __builtin_amdgcn_perm(e[1], e[0], 0x0C0C0602u);
        const uint32_t ed = __builtin_amdgcn_perm(e[3], e[2], 0x0C0C0602u);
        const uint32_t oa = __builtin_amdgcn_perm(o[1], o[0], 0x05010400u);
        const uint32_t ob = __builtin_amdgcn_perm(o[3], o[2], 0x05010400u);
        const uint32_t plane[kLimbs] = {
            __builtin_amdgcn_perm(eb, ea, 0x05040100u), __builtin_amdgcn_perm(ob, oa, 0x05040100u),
            __builtin_amdgcn_perm(eb, ea, 0x07060302u), __builtin_amdgcn_perm(ob, oa, 0x07060302u),
            __builtin_amdgcn_perm(ed, ec, 0x05040100u)};
#pragma unroll
        for (int l = 0; l < kLimbs; l++) limbs[(l * B * 4) + i] = plane[l] ^ 0x88888888u;
      } else {
#pragma unroll
        for (int l = 0; l < kLimbs; l++) {
          uint32_t w0 = 0, w1 = 0;
#pragma unroll
          for (int k = 0; k < 4; k++) {
            w0 |= ((u[k] >> (8 * l)) & 255u) << (8 * k);
            w1 |= ((u[k + 4] >> (8 * l)) & 255u) << (8 * k);
          }
          limbs[(l * B * 8) + 2 * i] = w0 ^ 0x80808080u;
          limbs[(l * B * 8) + 2 * i + 1] = w1 ^ 0x80808080u;
        }
      }
      if ((i & 3) == 0) exps[i >> 2] = mb >= 0x7F800000u ? kBadExp : e - kMantBits;
    };
    float inv_rms = 1.0f;
    if (PRO && J.pro == kProRmsNorm) {
      float ss = 0.0f;
#pragma unroll
      for (int p = 0; p < kPre; p++) {
        const int i = t + p * T;
        if (i < B * 4) {
          float xs[8], as[8];
          get8(i, p, xs, as);
          ss = sumsq8(xs, ss);
        }
      }
      for (int i = t + kPre * T; i < B * 4; i += T) {
        float xs[8];
        load8(xv, i, xs);
        ss = sumsq8(xs, ss);
      }
      inv_rms = inv_rms_of(ss);
    }
    // whole 4-thread groups stay together (T is a multiple of 64)
    auto round = [&](int i, int p) __attribute__((always_inline)) {
      float xs[8], as[8];
      get8(i, p, xs, as);
      if constexpr (PRO) prologue(xs, as, inv_rms);
      convert(i, xs);
    };
    const int kb = t % B;
#pragma unroll
    for (int m = 0; m < MR; m++) {
      row = m;
      xv = reinterpret_cast<const float4*>(J.x + (size_t)m * B * kBlockElems);
#pragma unroll
      for (int p = 0; p < kPre; p++)
        if (t + p * T < B * 4) round(t + p * T, p);
      for (int i = t + kPre * T; i < B * 4; i += T) round(i, kPre);
      __syncthreads();
#pragma unroll
      for (int v = 0; v < kLimbs * kLD / 4; v++)  // plane v / (kLD / 4), piece v % (kLD / 4)
        xl[m][v] = *reinterpret_cast<const u32x4*>(limbs + (v / (kLD / 4)) * B * kLD + kb * kLD +
                                                   (v % (kLD / 4)) * 4);
      if constexpr (F == kFmtQ4_0) {
        // The step takes a block's nibble dwords as window dwords 1, 2, 3 and
        // one permute of dwords 0 and 4: nibble bytes 2-5, 6-9, 10-13 and
        // {0, 1, 14, 15} when the block starts at byte 0 of its window (even
        // t), bytes 0-3 .. 12-15 when it starts at byte 2 (odd t).  The digit
        // planes are put in the same byte order here, once per job (a dot
        // product does not depend on the order of its terms).
        const uint32_t s_main = odd ? 0x03020100u : 0x05040302u;
        const uint32_t s_last = odd ? 0x07060504u : 0x07060100u;
#pragma unroll
        for (int v = 0; v < kLimbs; v++) {
          const u32x4 a = xl[m][v];
          xl[m][v] = u32x4{__builtin_amdgcn_perm(a[1], a[0], s_main),
                           __builtin_amdgcn_perm(a[2], a[1], s_main),
                           __builtin_amdgcn_perm(a[3], a[2], s_main),
                           __builtin_amdgcn_perm(a[3], a[0], s_last)};
        }
      }
      const int ex = exps[kb];
      xe[m] = ex == kBadExp ? 0 : ex;
      xnan[m] = ex == kBadExp ? __builtin_nanf("") : 0.0f;
      __syncthreads();  // the region is the next row's, then partial space
    }
  };

  // One step: close the chunk / switch job when due (uniform branches), read
  // this lane's window from the step's slot, refill the slot with the step R
  // ahead, decode the block and park its 8-lane group sum.
  auto step = [&](int ss, int slot) {
    if (ss == seg_end) {
      flush(ss);
      enter(cj + 1, ss, false);
    } else if (ss == c0 + L.S) {
      flush(ss);
      c0 = ss;
    }
    // This slot's DMAs are the oldest of the R steps in flight (vector memory
    // operations complete in order; any younger load only makes the wait
    // longer).  Its window goes to registers, then the slot is refilled.
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"((R - 1) * kDmaPerStep) : "memory");
    const uint32_t* wp = reinterpret_cast<const uint32_t*>(ring + slot * kSpan + win);
    uint32_t d[FT::kBytes / 4 + 1];
#pragma unroll
    for (int k = 0; k < FT::kBytes / 4 + 1; k++) d[k] = wp[k];
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the slot is read out
    issue(slot);
    float partial[MR];
    {
      if constexpr (F == kFmtQ4_0) {
        const float scale = f16_bits_to_f32(d[0] >> sh_d);
        int acc[MR][kLimbs];
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const uint32_t q =
              (j < 3 ? d[j + 1] : __builtin_amdgcn_perm(d[4], d[0], sel_q)) ^ 0x88888888u;
#pragma unroll
          for (int m = 0; m < MR; m++)
#pragma unroll
            for (int l = 0; l < kLimbs; l++)
              acc[m][l] = j == 0 ? sdot8_first(q, xl[m][l][0])
                                 : __builtin_amdgcn_sdot8((int)q, (int)xl[m][l][j], acc[m][l], false);
        }
        // sum_l 16^l * D_l, exact in int32 (|sum| < 2^28), as a chain of
        // shift-adds (one instruction per limb), then one rounding to fp32.
#pragma unroll
        for (int m = 0; m < MR; m++) {
          int h = acc[m][kLimbs - 1];
#pragma unroll
          for (int l = kLimbs - 2; l >= 0; l--) {
            // one v_lshl_add_u32 per limb (the empty asm keeps the compiler
            // from re-associating the chain into separate shifts and adds)
            h = (int)(((uint32_t)h << 4) + (uint32_t)acc[m][l]);
            asm("" : "+v"(h));
          }
          // one rounding of d * h (xnan is +0 or NaN: the +0 turns a -0
          // product into +0, as a separate addition would), then the exact
          // power-of-two scale
          partial[m] = ldexpf(fmaf(scale, (float)h, xnan[m]), xe[m]);
        }
      } else {
        const float scale = f16_bits_to_f32(d[0] >> sh_d);
        int acc[MR][kLimbs] = {};
#pragma unroll
        for (int j = 0; j < 8; j++) {
          const uint32_t q = __builtin_amdgcn_perm(d[j + 1], d[j], sel_q) ^ 0x80808080u;
#pragma unroll
          for (int m = 0; m < MR; m++)
#pragma unroll
            for (int l = 0; l < kLimbs; l++)
              acc[m][l] = __builtin_amdgcn_sdot4((int)q, (int)xl[m][2 * l + (j >> 2)][j & 3],
                                                 acc[m][l], false);
        }
#pragma unroll
        for (int m = 0; m < MR; m++) {
          const int h = acc[m][2] * 256 + acc[m][1];
          const float r = fmaf((float)h, 256.0f, (float)acc[m][0]);
          partial[m] = ldexpf(fmaf(scale, r, xnan[m]), xe[m]);
        }
      }
    }
#pragma unroll
    for (int m = 0; m < MR; m++) {
      float ps = group8_sum(partial[m]);
      asm volatile("" : "+v"(ps));  // the last add stays a DPP add, ahead of the store's branch
      if ((t & 7) == 7) part[(m * L.S + (ss - c0)) * T8 + (t >> 3)] = ps;
    }
  };

  enter(j0, s_begin, true);
  int slot = 0;
  for (int ss = s_begin; ss < s_end; ss++) {
    step(ss, slot);
    slot = slot + 1 == R ? 0 : slot + 1;
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the ring's run-out DMAs
  flush(s_end);
}

#define GEMV_HEAD_PARAMS                                                                   \
  int total_steps, int grid, int T, int ring_off, int njobs, int n0, int B0, int rps0,      \
      const uint8_t *w0, const float *x0, const float *aux0
#define GEMV_HEAD_ARGS \
  GemvHead { total_steps, grid, T, ring_off, njobs, n0, B0, rps0, w0, x0, aux0 }

template <int R>
__global__ void __launch_bounds__(1024) q4_0_gemv_jobs_kernel(GEMV_HEAD_PARAMS, GemvLaunch L) {
  gemv_jobs_body<kFmtQ4_0, false, R>(GEMV_HEAD_ARGS, L);
}

template <int R>
__global__ void __launch_bounds__(1024) q4_0_gemv_jobs_pro_kernel(GEMV_HEAD_PARAMS, GemvLaunch L) {
  gemv_jobs_body<kFmtQ4_0, true, R>(GEMV_HEAD_ARGS, L);
}

template <int R>
__global__ void __launch_bounds__(1024) q8_0_gemv_jobs_kernel(GEMV_HEAD_PARAMS, GemvLaunch L) {
  gemv_jobs_body<kFmtQ8_0, false, R>(GEMV_HEAD_ARGS, L);
}

template <int R, int MR>
__global__ void __launch_bounds__(512) q4_0_gemv_rows_kernel(GEMV_HEAD_PARAMS, GemvLaunch L) {
  gemv_jobs_body<kFmtQ4_0, false, R, MR>(GEMV_HEAD_ARGS, L);
}

template <int R, int MR>
__global__ void __launch_bounds__(512) q8_0_gemv_rows_kernel(GEMV_HEAD_PARAMS, GemvLaunch L) {
  gemv_jobs_body<kFmtQ8_0, false, R, MR>(GEMV_HEAD_ARGS, L);
}

template <int R>
static const void* gemv_rows_kernel_r(int rows, int fmt) {
  if (fmt == kFmtQ8_0) {
    switch (rows) {
      case 2: return reinterpret_cast<const void*>(q8_0_gemv_rows_kernel<R, 2>);
      case 3: return reinterpret_cast<const void*>(q8_0_gemv_rows_kernel<R, 3>);
      case 4: return reinterpret_cast<const void*>(q8_0_gemv_rows_kernel<R, 4>);
      case 5: return reinterpret_cast<const void*>(q8_0_gemv_rows_kernel<R, 5>);
      case 6: return reinterpret_cast<const void*>(q8_0_gemv_rows_kernel<R, 6>);
      case 7: return reinterpret_cast<const void*>(q8_0_gemv_rows_kernel<R, 7>);
      default: return reinterpret_cast<const void*>(q8_0_gemv_rows_kernel<R, 8>);
    }
  }
  switch (rows) {
    case 2: return reinterpret_cast<const void*>(q4_0_gemv_rows_kernel<R, 2>);
    case 3: return reinterpret_cast<const void*>(q4_0_gemv_rows_kernel<R, 3>);
    default: return reinterpret_cast<const void*>(q4_0_gemv_rows_kernel<R, 4>);
  }
}

template <int R>
static const void* gemv_kernel_r(int which) {
  return which == 2   ? reinterpret_cast<const void*>(q8_0_gemv_jobs_kernel<R>)
         : which == 1 ? reinterpret_cast<const void*>(q4_0_gemv_jobs_pro_kernel<R>)
                      : reinterpret_cast<const void*>(q4_0_gemv_jobs_kernel<R>);
}

// Ring depths built: 2 and 3 for work-groups that share a CU, deeper ones for
// launches of at most one work-group per CU.
static const void* gemv_kernel(int which, int R) {
  switch (R) {
    case 8: return gemv_kernel_r<8>(which);
    case 6: return gemv_kernel_r<6>(which);
    case 4: return gemv_kernel_r<4>(which);
    case 3: return gemv_kernel_r<3>(which);
    default: return gemv_kernel_r<2>(which);
  }
}

hipError_t launch_q4_0_gemv_group(const GemvGroupGeom& g, const GemvJob* d_jobs,
                                  const GemvJob* h_jobs, int njobs, int total_steps, int num_cus,
                                  hipStream_t s) {
  const bool q8 = g.fmt == kFmtQ8_0;
  const int which = q8 ? 2 : (g.pro ? 1 : 0);
  const void* kern = gemv_kernel(which, g.ring);
  {
    hipError_t e = set_lds_limit(kern, (int)kMaxLds);
    if (e != hipSuccess) return e;
  }
  // As many work-groups as can be resident at once (registers and LDS).
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, g.T, g.lds) != hipSuccess ||
      per_cu < 1)
    per_cu = 1;
  int grid = total_steps < num_cus * per_cu ? total_steps : num_cus * per_cu;
  // Every work-group stages a job's whole x (4K bytes, and as much again for
  // a prologue operand) before streaming its rows, so each one should stream
  // at least about twice that in weights: for one matrix about n/14
  // work-groups.  Rounded to a whole number per CU (a partial round leaves
  // most CUs idle while a few run a second work-group), at least one per CU.
  // Measured on a TinyLlama decode step (88 small launches): 577 -> 543 us,
  // 669 -> 614 us with fused norms; 1x or 4x the staging bytes do worse.
  {
    const long long wbytes =
        (long long)total_steps * g.T * (q8 ? Fmt<kFmtQ8_0>::kBytes : kBlockBytes);
    const long long cap = gemv_per_cu(g, wbytes, num_cus) * num_cus;
    if (grid > cap) grid = (int)cap;
  }
  // At most one work-group per CU: LDS has room for a deeper ring, which
  // keeps more of the work-group's weights in flight (a small matrix's
  // stream is otherwise bound by the bytes each CU has in flight); up to one
  // slot per step the work-group streams.
  size_t lds = g.lds;
  if (grid <= num_cus) {
    const int per_wg = (total_steps + grid - 1) / grid;
    const size_t span = 64 * (size_t)(q8 ? Fmt<kFmtQ8_0>::kBytes : kBlockBytes);
    int R = g.ring;
    for (int cand : {4, 6, 8}) {
      if (R >= per_wg) break;
      if (g.ring_off + (size_t)g.W * cand * span > kMaxLds) break;
      R = cand;
    }
    if (R != g.ring) {
      kern = gemv_kernel(which, R);
      hipError_t e = set_lds_limit(kern, (int)kMaxLds);
      if (e != hipSuccess) return e;
      lds = g.ring_off + (size_t)g.W * R * span;
    }
  }
  GemvLaunch L;
  L.jobs = d_jobs;
  for (int i = 0; i < kGemvInline; i++) L.inl[i] = h_jobs[i < njobs ? i : 0];
  L.S = g.S;
  const GemvJob& J0 = h_jobs[0];
  using Kern = void (*)(int, int, int, int, int, int, int, int, const uint8_t*, const float*,
                        const float*, GemvLaunch);
  hipLaunchKernelGGL(reinterpret_cast<Kern>(const_cast<void*>(kern)), dim3(grid), dim3(g.T), lds, s,
                     total_steps, grid, g.T, (int)g.ring_off, njobs, J0.n, J0.B, J0.rps, J0.w, J0.x,
                     J0.pro != kProNone ? J0.aux : nullptr, L);
  return hipGetLastError();
}

static hipError_t launch_gemv_fast(int fmt, float* y, const uint8_t* w, const float* x,
                                   const float* bias, size_t n, size_t m, int num_cus,
                                   hipStream_t s) {
  GemvGroupGeom g;
  g.fmt = fmt;
  gemv_group_add(g, m);
  {
    const int nn = (int)n, BB = (int)(m / 32);
    gemv_group_widen(g, &nn, &BB, 1, num_cus);
  }
  GemvJob J;
  J.w = w;
  J.x = x;
  J.y = y;
  J.bias = bias;
  J.aux = nullptr;
  J.pro = kProNone;
  J.eps = 0.0f;
  J.n = (int)n;
  J.B = (int)(m / 32);
  J.rps = g.T / J.B;
  J.step0 = 0;
  const int steps = (J.n + J.rps - 1) / J.rps;
  return launch_q4_0_gemv_group(g, nullptr, &J, 1, steps, num_cus, s);
}

// Work-groups of 512 threads where the row length allows (twice the steps in
// flight per work-group of the 256 that the one-row geometry picks for
// K = 4096; the grid below then needs half the work-groups).
static bool rows_geometry(GemvGroupGeom& g, size_t m, size_t rows, int fmt) {
  if (rows < 2 || (int)rows > (fmt == kFmtQ8_0 ? kQ8GemvMaxRows : kGemvMaxRows)) return false;
  g.fmt = fmt;
  g.rows = (int)rows;
  if (!gemv_group_add(g, m) || g.T > 512) return false;
  if (g.T < 512 && 512 % g.Tbase == 0) {
    GemvGroupGeom t = g;
    finish_geometry(t, 512);
    if (t.lds <= kMaxLds) g = t;
  }
  return true;
}

bool q4_0_gemv_rows_ok(const uint8_t* w, size_t w_len, size_t n, size_t m, size_t rows) {
  GemvGroupGeom g;
  return q4_0_gemv_fast_ok(w, w_len, n, m) && rows_geometry(g, m, rows, kFmtQ4_0);
}

bool q8_0_gemv_rows_ok(const uint8_t* w, size_t w_len, size_t n, size_t m, size_t rows) {
  GemvGroupGeom g;
  return q8_0_gemv_fast_ok(w, w_len, n, m) && rows_geometry(g, m, rows, kFmtQ8_0);
}

static hipError_t launch_gemv_rows(int fmt, float* y, const uint8_t* w, const float* x,
                                   const float* bias, size_t n, size_t m, int rows, int num_cus,
                                   hipStream_t s) {
  GemvGroupGeom g;
  if (!rows_geometry(g, m, (size_t)rows, fmt)) return hipErrorInvalidValue;
  const int bbytes = fmt == kFmtQ8_0 ? Fmt<kFmtQ8_0>::kBytes : kBlockBytes;
  GemvJob J;
  J.w = w;
  J.x = x;
  J.y = y;
  J.bias = bias;
  J.aux = nullptr;
  J.pro = kProNone;
  J.eps = 0.0f;
  J.n = (int)n;
  J.B = (int)(m / 32);
  J.rps = g.T / J.B;
  J.step0 = 0;
  const int steps = (J.n + J.rps - 1) / J.rps;
  const void* kern =
      g.ring == 3 ? gemv_rows_kernel_r<3>(rows, fmt) : gemv_rows_kernel_r<2>(rows, fmt);
  {
    hipError_t e = set_lds_limit(kern, (int)kMaxLds);
    if (e != hipSuccess) return e;
  }
  // Every work-group converts all rows of x (rows x 16 KB at K = 4096), so,
  // as for one row, each should stream at least twice that in weights; at
  // most as many work-groups as are resident.
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, g.T, g.lds) != hipSuccess ||
      per_cu < 1)
    per_cu = 1;
  {
    const long long stage = 4LL * kBlockElems * g.maxB * rows;
    const long long ws = (long long)n * J.B * bbytes / (2 * stage);
    long long per = (ws + num_cus / 2) / num_cus;
    if (per < 1) per = 1;
    if (per < per_cu) per_cu = (int)per;
  }
  const int grid = steps < num_cus * per_cu ? steps : num_cus * per_cu;
  GemvLaunch L;
  L.jobs = nullptr;
  for (int i = 0; i < kGemvInline; i++) L.inl[i] = J;
  L.S = g.S;
  using Kern = void (*)(int, int, int, int, int, int, int, int, const uint8_t*, const float*,
                        const float*, GemvLaunch);
  hipLaunchKernelGGL(reinterpret_cast<Kern>(const_cast<void*>(kern)), dim3(grid), dim3(g.T), g.lds, s,
                     steps, grid, g.T, (int)g.ring_off, 1, J.n, J.B, J.rps, J.w, J.x,
                     static_cast<const float*>(nullptr), L);
  return hipGetLastError();
}

hipError_t launch_q4_0_gemv_rows(float* y, const uint8_t* w, const float* x, const float* bias,
                                 size_t n, size_t m, int rows, int num_cus, hipStream_t s) {
  return launch_gemv_rows(kFmtQ4_0, y, w, x, bias, n, m, rows, num_cus, s);
}

hipError_t launch_q8_0_gemv_rows(float* y, const uint8_t* w, const float* x, const float* bias,
                                 size_t n, size_t m, int rows, int num_cus, hipStream_t s) {
  return launch_gemv_rows(kFmtQ8_0, y, w, x, bias, n, m, rows, num_cus, s);
}

hipError_t launch_q4_0_gemv_fast(float* y, const uint8_t* w, const float* x, const float* bias,
                                 size_t n, size_t m, int num_cus, hipStream_t s) {
  return launch_gemv_fast(kFmtQ4_0, y, w, x, bias, n, m, num_cus, s);
}

hipError_t launch_q8_0_gemv_fast(float* y, const uint8_t* w, const float* x, const float* bias,
                                 size_t n, size_t m, int num_cus, hipStream_t s) {
  return launch_gemv_fast(kFmtQ8_0, y, w, x, bias, n, m, num_cus, s);
}

}  // namespace hypno
