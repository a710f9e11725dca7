// Q4_0 matrix-vector kernels for gfx950.
//
//  * q4_0_generic_kernel: any m (blocks straddling rows), any alignment, short
//    weight buffers, bias, and any number of tokens.  One wave per
//    (token, row); lanes walk the row's overlapping blocks.  Semantics follow
//    matmul_q4_0_scalar (kernels.rs:362-400).
//  * q4_0_gemv_jobs_kernel: the decode GEMV (one token) over one job or a
//    table of independent jobs in a single launch.  See the comment above it.
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
// contiguous range of it (possibly spanning jobs).  A lane loads its own
// block straight from HBM as the 20-byte window [18t & ~3, +20) (a 16-byte
// and a 4-byte load; the 64 lanes of a wave cover one contiguous 1152-byte
// span, so the loads coalesce), and keeps the next kDepth steps in flight in
// a register ring that runs across job boundaries.  A lane-dependent byte
// permute realigns the nibble dwords (a block starts at byte 0 or 2 of its
// window), the nibbles are converted in registers (v_cvt_f32_ubyte*), sum(nib
// * x) accumulates in fp32, and the block's scale is applied as
// d * (sum - 8 * sum(x)).  Per-block partials of S steps are parked in LDS;
// after one barrier each wave sums whole rows in a fixed order
// (deterministic) and writes y.  Activations are restaged (coalesced, through
// LDS with an XOR swizzle) only when the job changes.
//
// Bounds: a matrix of whole rows is a multiple of 144 bytes, so its last
// block starts 2 bytes past a dword boundary and its window ends exactly at
// the end of the matrix; every other window ends inside the next block.
// ---------------------------------------------------------------------------

constexpr int kDepth = 3;  // steps in flight per wave beyond the current one (the slot
                           // dispatch in the step loop is written out for 3)

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

static void finish_geometry(GemvGroupGeom& g) {
  g.T = g.Tbase;
  while (g.T < 256 && 2 * g.T <= 1024) g.T *= 2;
  g.W = g.T / 64;
  g.S = 32;
  const size_t loop = (size_t)g.S * (g.T / 8) * 4;  // 8-lane group partials
  const size_t xs = (size_t)g.maxB * 32 * 4;        // activations
  g.lds = xs > loop ? xs : loop;
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

bool q4_0_gemv_fast_ok(const uint8_t* w, size_t w_len, size_t n, size_t m) {
  if (n == 0 || n > (size_t)0x3FFFFFFF) return false;
  if (((uintptr_t)w & 15) != 0) return false;
  GemvGroupGeom g;
  if (!gemv_group_add(g, m)) return false;
  return w_len / kBlockBytes >= n * (m / kBlockElems);
}

// One ring slot: this lane's 20-byte window of one step.
struct Slot {
  u32x4 a;
  uint32_t b;
};

// Cached description of the job the prefetch ring is reading (uniform).
struct RingCursor {
  const uint8_t* w;
  int n, B, rps, step0, end, j;
};

__global__ void __launch_bounds__(1024)
q4_0_gemv_jobs_kernel(GemvLaunch L) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int T = blockDim.x;
  const int t = threadIdx.x;
  const int G = L.total_steps;
  const int s_begin = (int)((long long)G * blockIdx.x / gridDim.x);
  const int s_end = (int)((long long)G * (blockIdx.x + 1) / gridDim.x);
  if (s_begin >= s_end) return;  // whole work-group

  auto get = [&](int j) -> GemvJob {
    return L.njobs == 1 ? L.job0 : load_const<GemvJob>(L.jobs + j);
  };
  auto cursor = [&](int j) {
    const GemvJob J = get(j);
    RingCursor c;
    c.w = J.w;
    c.n = J.n;
    c.B = J.B;
    c.rps = J.rps;
    c.step0 = J.step0;
    c.end = J.step0 + (J.n + J.rps - 1) / J.rps;
    c.j = j;
    return c;
  };
  // First job of this work-group's range (binary search on step0).
  int j0 = 0;
  if (L.njobs > 1) {
    int lo = 0, hi = L.njobs - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (load_const<int>(&L.jobs[mid].step0) <= s_begin)
        lo = mid;
      else
        hi = mid - 1;
    }
    j0 = lo;
  }

  // Ring loads are unconditional (a lane with nothing to fetch re-reads the
  // first 20 bytes of a job's weights, always in bounds): a load under a
  // branch is waited for at once, which would serialise the ring.  The job
  // table is read only when the ring crosses into the next job.
  RingCursor pc = cursor(j0);
  const uint8_t* wsafe = pc.w;
  const uint32_t win = (uint32_t)(18 * t) & ~3u;  // window start inside a step
  auto issue = [&](int g) -> Slot {
    const uint8_t* p = wsafe;
    if (g < s_end) {
      if (g >= pc.end) pc = cursor(pc.j + 1);
      const int ls = g - pc.step0;
      const int vu = min(pc.rps, pc.n - ls * pc.rps) * pc.B;  // valid blocks in the step
      if (t < vu) p = pc.w + (size_t)ls * pc.rps * pc.B * 18 + win;
    }
    Slot r;
    r.a = load_global<u32x4>(p);
    r.b = load_global<uint32_t>(p + 16);
    return r;
  };
  Slot ring[kDepth];
#pragma unroll
  for (int d = 0; d < kDepth; d++) ring[d] = issue(s_begin + d);

  // Byte selectors for v_perm_b32: a block starts at byte 0 (t even) or 2
  // (t odd) of its window; nibble dword j is bytes [2+4j, 6+4j) of the block.
  const bool odd = (t & 1) != 0;
  const uint32_t sel_q = odd ? 0x07060504u : 0x05040302u;
  const uint32_t sh_d = odd ? 16u : 0u;

  // [S][T/8] sums of 8-lane groups (a row of B blocks is B/8 whole groups
  // because B % 8 == 0); aliases the activation staging area.
  float* part = reinterpret_cast<float*>(smem);
  const int T8 = T >> 3;

  int cj = j0;
  int s = s_begin;
  while (s < s_end) {
    const GemvJob J = get(cj);
    const int B = J.B, rps = J.rps, n = J.n;
    const int seg_end = min(s_end, J.step0 + (n + rps - 1) / rps);
    const int kb = t % B;

    // Activations of this job: coalesced copy to LDS (float4 q of block b is
    // stored at 8b + (q ^ (b & 7)), so the per-lane reads below do not
    // conflict), then this lane's 32 into registers.
    {
      float4* xs = reinterpret_cast<float4*>(smem);
      const float4* xv = reinterpret_cast<const float4*>(J.x);
      for (int i = t; i < B * 8; i += T) {
        const int b = i >> 3;
        xs[(b << 3) + ((i & 7) ^ (b & 7))] = load_global<float4>(xv + i);
      }
    }
    __syncthreads();
    float xr[32];
    {
      const float4* xs = reinterpret_cast<const float4*>(smem) + (kb << 3);
#pragma unroll
      for (int q = 0; q < 8; q++) {
        const float4 v = xs[q ^ (kb & 7)];
        xr[4 * q + 0] = v.x;
        xr[4 * q + 1] = v.y;
        xr[4 * q + 2] = v.z;
        xr[4 * q + 3] = v.w;
      }
    }
    // The -8 offset of every nibble is applied once per block as -8 * sum(x).
    float xsum = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) xsum += xr[i];
    const float m8xsum = -8.0f * xsum;
    __syncthreads();  // the activation region becomes partial space

    // One step: decode this lane's block from its ring slot, refill the slot
    // with step ss + kDepth (returned), park the partial.
    auto step = [&](int ss, int c0, const Slot sl) -> Slot {
      const Slot next = issue(ss + kDepth);
      const int vu = min(rps, n - (ss - J.step0) * rps) * B;
      float partial = 0.0f;
      if (t < vu) {
        const uint32_t d[5] = {sl.a.x, sl.a.y, sl.a.z, sl.a.w, sl.b};
        const float scale = f16_bits_to_f32(d[0] >> sh_d);
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++)
          acc += dot8_nib(__builtin_amdgcn_perm(d[j + 1], d[j], sel_q), xr + 8 * j);
        partial = scale * (acc + m8xsum);
      }
      partial = group8_sum(partial);
      if ((t & 7) == 7) part[(ss - c0) * T8 + (t >> 3)] = partial;
      return next;
    };

    for (int c0 = s; c0 < seg_end; c0 += L.S) {
      const int c1 = min(c0 + L.S, seg_end);
      // ring[k] holds step ss with (ss - s_begin) % kDepth == k: rotate by
      // value so the slot index stays a compile-time constant.
      for (int ss = c0; ss < c1; ss++) {
        const int k = (ss - s_begin) % kDepth;
        if (k == 0) ring[0] = step(ss, c0, ring[0]);
        else if (k == 1) ring[1] = step(ss, c0, ring[1]);
        else ring[2] = step(ss, c0, ring[2]);
      }
      __syncthreads();
      // One thread per row sums the row's B/8 group partials in a fixed order.
      const int row0 = (c0 - J.step0) * rps;
      const int nrows = min((c1 - c0) * rps, n - row0);
      const int B8 = B >> 3;
      for (int r = t; r < nrows; r += T) {
        const int sl = r / rps;
        const float* pr = part + sl * T8 + (r - sl * rps) * B8;
        float v = 0.0f;
        for (int q = 0; q < B8; q++) v += pr[q];
        J.y[row0 + r] = v + (J.bias ? J.bias[row0 + r] : 0.0f);
      }
      __syncthreads();
    }
    s = seg_end;
    cj++;
  }
}

static bool g_lds_attr_set = false;

hipError_t launch_q4_0_gemv_group(const GemvGroupGeom& g, const GemvJob* d_jobs,
                                  const GemvJob& job0, int njobs, int total_steps, int num_cus,
                                  hipStream_t s) {
  if (!g_lds_attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(q4_0_gemv_jobs_kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxLds);
    if (e != hipSuccess) return e;
    g_lds_attr_set = true;
  }
  // As many work-groups as can be resident at once (registers and LDS).
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &per_cu, reinterpret_cast<const void*>(q4_0_gemv_jobs_kernel), g.T, g.lds) !=
          hipSuccess ||
      per_cu < 1)
    per_cu = 1;
  const int grid = total_steps < num_cus * per_cu ? total_steps : num_cus * per_cu;
  GemvLaunch L;
  L.jobs = d_jobs;
  L.job0 = job0;
  L.njobs = njobs;
  L.total_steps = total_steps;
  L.S = g.S;
  hipLaunchKernelGGL(q4_0_gemv_jobs_kernel, dim3(grid), dim3(g.T), g.lds, s, L);
  return hipGetLastError();
}

hipError_t launch_q4_0_gemv_fast(float* y, const uint8_t* w, const float* x, const float* bias,
                                 size_t n, size_t m, int num_cus, hipStream_t s) {
  GemvGroupGeom g;
  gemv_group_add(g, m);
  GemvJob J;
  J.w = w;
  J.x = x;
  J.y = y;
  J.bias = bias;
  J.n = (int)n;
  J.B = (int)(m / 32);
  J.rps = g.T / J.B;
  J.step0 = 0;
  const int steps = (J.n + J.rps - 1) / J.rps;
  return launch_q4_0_gemv_group(g, nullptr, J, 1, steps, num_cus, s);
}

}  // namespace hypno
