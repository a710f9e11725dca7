// The steps either side of the decode path that read or write whole rows of
// a weight table or of the logits:
//
//  * embedding gather (transformer.rs:476-497, turbo.rs:38-66, with
//    q4_0_extract_row quant.rs:139-153 and q8_0_extract_row quant.rs:158-175):
//    out[t][0..hd) = row ids[t] of an FP32 / FP16 / Q8_0 / Q4_0 table,
//    dequantised bit-exactly, one work-group per token;
//  * next-token choice from the lm_head's logits: greedy argmax (one launch
//    of one work-group) and sample_token (run.rs:203-251) with its
//    XorShift64 generator (run.rs:267-278), in two launches: up to 64
//    work-groups over consecutive ranges of the logits (per-range argmax,
//    p_i, and per range either the top-k candidates or the top-p key-bin
//    masses), then one work-group for the rest.
//
// sample_token, as the reference defines it:
//   p_i = exp(l_i * (1 / temperature)) if temperature > 0, else l_i;
//   top_k (0 < k < n): p_i = 0 where p_i < the k-th largest p;
//   top_p (< 1): with S = sum_i p_i in index order (fp32), walk the p in
//     descending order adding p / S to an fp32 running sum; the p at which it
//     first exceeds top_p is the threshold (none: the largest fp32), and
//     p_i = 0 where p_i < threshold;
//   S = sum_i p_i (index order, fp32); S <= 0: the argmax of the logits;
//   otherwise r = next_f32() and the first i whose running sum of p_i / S
//   exceeds r (none: the argmax of the p).
// Argmax is Iterator::max_by with partial_cmp: the last of equal maxima, and a
// NaN is passed over by the comparisons (the result is the argmax of what
// follows the last NaN, or the NaN itself when it is the last element).
//
// Here: without top-k the sums and walks run over p itself (all n values in
// index order, zeros included, as the reference's loops). With top-k, the
// k-th largest p comes from a three-level radix select (11 + 11 + 10 bits of
// an order-preserving key) over the ranges' candidates, and the p left
// non-zero are compacted in index order: adding a zero changes no running sum
// (at most the sign of a zero sum, which no comparison sees), so the
// compacted list gives the same sums and crossings. The top-p walk sorts
// (stable LSD radix, four 8-bit passes; a rank pass for short lists) only the
// key bins from the top down to where their mass reaches top_p plus the fp32
// sums' margin. Every running sum reproduces the reference's sequential fp32
// additions exactly: integer prefix sums on the running sum's binade grid, in
// parallel, with one fp32 addition for each value the grid cannot take
// (acc_chunk).
// exp is computed in fp64 and rounded once to fp32 (the reference calls the
// platform's expf; the two agree except where a result lies within about
// 2^-29 of a rounding boundary).
#include "common.hpp"

namespace hypno {

namespace {

// --- embedding gather ---------------------------------------------------------------

struct EmbedArgs {
  float* out;            // [count][hd]
  const uint8_t* table;
  size_t table_len;
  const uint32_t* ids;   // [count], device; NULL: the single row id0
  size_t id0;
  int dtype;             // HYPNO_DTYPE_*
  size_t hd;
};

// One work-group per token; threads stride over the row's elements.  A row
// whose bytes are not all inside the table (a panic in the reference's
// slicing) is written as NaN.
__global__ void __launch_bounds__(256) embed_rows_kernel(const EmbedArgs a) {
  const size_t t = blockIdx.x;
  const size_t id = a.ids ? (size_t)a.ids[t] : a.id0;
  float* o = a.out + t * a.hd;
  const size_t hd = a.hd;
  if (a.dtype == 0 || a.dtype == 1) {  // FP32 / FP16: [start, start + hd)
    const size_t esz = a.dtype == 0 ? 4 : 2;
    // (id + 1) * hd <= table_len / esz, without a product that can wrap.
    const bool ok = id < a.table_len / esz / hd;
    for (size_t i = threadIdx.x; i < hd; i += 256) {
      float v = __builtin_nanf("");
      if (ok) {
        const size_t e = id * hd + i;
        v = a.dtype == 0 ? reinterpret_cast<const float*>(a.table)[e]
                         : f16_bits_to_f32(reinterpret_cast<const uint16_t*>(a.table)[e]);
      }
      o[i] = v;
    }
    return;
  }
  // Q8_0 / Q4_0: hd / 32 whole blocks per row (q*_extract_row), elements past
  // them stay 0.
  const size_t bb = a.dtype == 2 ? kQ8BlockBytes : kBlockBytes;
  const size_t bpr = hd / kBlockElems;
  const bool ok = bpr != 0 && id < a.table_len / bb / bpr;
  for (size_t i = threadIdx.x; i < hd; i += 256) {
    const size_t b = i / kBlockElems, j = i % kBlockElems;
    float v = 0.0f;
    if (b < bpr) {
      if (!ok) {
        v = __builtin_nanf("");
      } else {
        const uint8_t* blk = a.table + (id * bpr + b) * bb;
        const float d = f16_bits_to_f32((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
        if (a.dtype == 2) {
          v = (float)((int)blk[2 + j] - 128) * d;
        } else {
          const uint32_t byte = blk[2 + (j >> 1)];
          v = (float)((int)((j & 1) ? byte >> 4 : byte & 15u) - 8) * d;
        }
      }
    }
    o[i] = v;
  }
}

// --- argmax and sampling ------------------------------------------------------------

constexpr int kST = 1024;  // threads of a sampling work-group
constexpr int kSW = kST / 64;
constexpr int kMaxParts = 64;     // work-groups of the first sampling kernel
constexpr int kPartElems = 2048;  // at least this many logits per such work-group
constexpr int kBins1 = 2048;      // level-1 bins of the top-k radix select

// Order-preserving map of fp32 bit patterns to u32 (ascending key = ascending
// value, -0 just below +0) and back.
__device__ __forceinline__ uint32_t fkey(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float funkey(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}


// Argmax of one range of the logits: the last NaN in it (-1: none) and the
// best (value, index) over the elements after that NaN, the later index among
// equal values (bi = -1: nothing follows the NaN).
struct ArgPart {
  int ln;
  int bi;
  float bv;
  int pad;
};

struct SampleArgs {
  const float* logits;
  int n;
  int greedy_only;  // argmax of the logits, nothing else
  float temperature, inv_temp, top_p;
  int top_k;
  int parts;        // work-groups of the first kernel
  uint32_t* token;
  uint64_t* state;
  // workspace
  ArgPart* part;    // [parts]
  int* seg_cnt;     // [parts]: candidates of each range
  float* probs;     // n entries each from here on
  uint32_t* seg_idx;  // range g's candidates at [lo_g, lo_g + seg_cnt[g])
  float* seg_val;
  uint32_t* a_idx;
  float* a_val;
  double* range_mass;  // without top-k: [parts][kBins1] key-bin masses (planes 1-3)
  uint32_t* k0;
  uint32_t* k1;
};

constexpr int kChunk = 8192;  // floats of a sequential pass staged in LDS at a time

constexpr int kSortCap = 12288;  // keys a sort keeps in LDS

struct SampleShared {
  union {
    float chunk[kChunk];         // staged values of a sequential sum
    uint32_t sorta[kSortCap];    // an LDS sort's second buffer
  };
  uint32_t sortb[kSortCap];      // keys of an LDS sort, in and out
  double mass[kBins1];
  uint32_t hist[kBins1];
  uint32_t cnt[kSW][256];
  uint32_t base[256];
  uint32_t wsum[kSW];
  float fred[kSW];
  int ired[kSW];
  double dred[kSW];
  uint32_t u[4];
  float f[4];
  alignas(16) uint32_t acc_w[kSW];  // exact accumulation: per-wave increment totals
  alignas(16) int acc_ev[kSW];      // ... per-wave first event
  alignas(16) int acc_hit[kSW];     // ... per-wave first running sum above thr
  int acc_i[4];    // sequential batch: -, first sum above thr, next position; hit flag
  uint32_t acc_s;  // the running sum's bit pattern
};
static_assert(sizeof(SampleShared) <= 160 * 1024, "LDS of a work-group");

__device__ __forceinline__ uint32_t usat_add(uint32_t a, uint32_t b) {
  return __builtin_elementwise_add_sat(a, b);
}

// d = v / u rounded to the nearest integer for v >= +0 finite, on the grid
// u = 2^(E - 150) of exponent field E >= 1, with sc = 150 - E: v 2^sc is
// exact (a power-of-two scaling; an overflow to inf only where v / u >=
// 2^24, a result below 2^-126 only where v / u < 1/2: d = 0 either way); d
// >= 2^24 is returned as 2^24 (the sum leaves the binade whatever m is).
// tie: v / u is exactly halfway between two integers.
__device__ __forceinline__ uint32_t acc_increment(float v, int sc, bool& tie) {
  const float q = fminf(ldexpf(v, sc), 16777216.0f);  // NaN v: 2^24 (an event anyway)
  tie = __builtin_amdgcn_fractf(q) == 0.5f;
  return (uint32_t)__builtin_rintf(q);
}

// Inclusive scan of x over the wave (lane order), saturating at 2^32 - 1:
// sums over 1, 2, 4, 8 lanes within each row of 16, then each row takes the
// previous rows' total (row_bcast:15, row_bcast:31).
__device__ __forceinline__ uint32_t wave_scan_sat(uint32_t x) {
  x = usat_add(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xf, 0xf, false));
  x = usat_add(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xf, 0xf, false));
  x = usat_add(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xf, 0xf, false));
  x = usat_add(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xf, 0xf, false));
  x = usat_add(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x142, 0xa, 0xf, false));
  x = usat_add(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x143, 0xc, 0xf, false));
  return x;
}

// In the histogram hist[0..nbins), bins counted from the top: the bin holding
// the kk-th largest element (1-based) and kk within that bin.  nbins <= 2048.
__device__ void select_from_top(SampleShared& sh, int nbins, uint32_t kk, uint32_t* bin,
                                uint32_t* kin) {
  const int t = threadIdx.x;
  // thread t owns bins nbins-1-2t (higher) and nbins-2-2t
  const int b0 = nbins - 1 - 2 * t, b1 = b0 - 1;
  const uint32_t c0 = b0 >= 0 ? sh.hist[b0] : 0u, c1 = b1 >= 0 ? sh.hist[b1] : 0u;
  // inclusive scan over threads in order t = 0, 1, ... (DPP within the
  // wave, then the waves' totals)
  const int lane = t & 63;
  const uint32_t s = wave_scan_sat(c0 + c1);
  __syncthreads();
  if (lane == 63) sh.wsum[t >> 6] = s;
  __syncthreads();
  uint32_t before = 0;
  for (int w = 0; w < (t >> 6); w++) before += sh.wsum[w];
  const uint32_t incl = s + before, excl = incl - c0 - c1;
  if (excl < kk && kk <= incl) {
    if (kk <= excl + c0) {
      sh.u[0] = (uint32_t)b0;
      sh.u[1] = kk - excl;
    } else {
      sh.u[0] = (uint32_t)b1;
      sh.u[1] = kk - excl - c0;
    }
  }
  __syncthreads();
  *bin = sh.u[0];
  *kin = sh.u[1];
  __syncthreads();
}

// (value, index) pairs: a replaces b when it is larger, or equal with the
// larger index (Iterator::max_by keeps the last of equal maxima).
__device__ __forceinline__ bool arg_better(float av, int ai, float bv, int bi) {
  return ai >= 0 && (bi < 0 || av > bv || (av == bv && ai > bi));
}

// ArgPart of v(lo..hi), work-group wide; every thread gets the result.
template <typename V>
__device__ ArgPart argmax_part(int lo, int hi, V v, SampleShared& sh) {
  const int t = threadIdx.x;
  int ln = -1;
  for (int i = lo + t; i < hi; i += kST)
    if (__builtin_isnan(v(i))) ln = i;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ln = max(ln, __shfl_xor(ln, off, 64));
  __syncthreads();
  if ((t & 63) == 0) sh.ired[t >> 6] = ln;
  __syncthreads();
  ln = -1;
  for (int w = 0; w < kSW; w++) ln = max(ln, sh.ired[w]);
  float bv = 0.0f;
  int bi = -1;
  for (int i = (ln >= 0 ? ln + 1 : lo) + t; i < hi; i += kST) {
    const float x = v(i);
    if (bi < 0 || x >= bv) {  // ties: the later index (i grows per thread)
      bv = x;
      bi = i;
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(bv, off, 64);
    const int oi = __shfl_xor(bi, off, 64);
    if (arg_better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  __syncthreads();
  if ((t & 63) == 0) {
    sh.fred[t >> 6] = bv;
    sh.ired[t >> 6] = bi;
  }
  __syncthreads();
  bv = 0.0f;
  bi = -1;
  for (int w = 0; w < kSW; w++)
    if (arg_better(sh.fred[w], sh.ired[w], bv, bi)) {
      bv = sh.fred[w];
      bi = sh.ired[w];
    }
  __syncthreads();
  return ArgPart{ln, bi, bv, 0};
}

// Iterator::max_by(partial_cmp) over n values from the ArgParts of
// consecutive ranges covering them: the last of equal maxima after the last
// NaN, or that NaN if it is the last element; n == 0 gives 0.  Each range's
// best already excludes what precedes its own last NaN, and ranges before
// the range of the overall last NaN hold only indices below it.
__device__ uint32_t argmax_combine(const ArgPart* p, int parts, int n) {
  if (n == 0) return 0u;
  int ln = -1;
  for (int g = 0; g < parts; g++) ln = max(ln, p[g].ln);
  if (ln == n - 1) return (uint32_t)ln;
  float bv = 0.0f;
  int bi = -1;
  for (int g = 0; g < parts; g++)
    if (p[g].bi > ln && arg_better(p[g].bv, p[g].bi, bv, bi)) {
      bv = p[g].bv;
      bi = p[g].bi;
    }
  return (uint32_t)bi;
}

// Iterator::max_by over v(0..n) in one work-group.
template <typename V>
__device__ uint32_t argmax_fold(int n, V v, SampleShared& sh) {
  const ArgPart p = argmax_part(0, n, v, sh);
  return argmax_combine(&p, 1, n);
}

// Compact the elements i in [lo, hi) for which keep(i, x) holds, x = val(i),
// into (idx[], v[]) in index order (idx holds i); returns their count.  A
// work-group pass per kST elements: wave ballots give ranks, LDS the wave
// offsets.
template <typename V, typename K>
__device__ int compact_range(int lo, int hi, V val, K keep, uint32_t* idx, float* v,
                             SampleShared& sh) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const uint64_t lt = (1ull << lane) - 1ull;
  int L = 0;
  for (int b0 = lo; b0 < hi; b0 += kST) {
    const int i = b0 + t;
    const float x = i < hi ? val(i) : 0.0f;
    const bool kp = i < hi && keep(i, x);
    const uint64_t m = __ballot(kp);
    if (lane == 0) sh.wsum[wave] = (uint32_t)__popcll(m);
    __syncthreads();
    int off = L, tot = 0;
    for (int w = 0; w < kSW; w++) {
      const int c = (int)sh.wsum[w];
      if (w < wave) off += c;
      tot += c;
    }
    if (kp) {
      const int d = off + __popcll(m & lt);
      idx[d] = (uint32_t)i;
      v[d] = x;
    }
    L += tot;
    __syncthreads();
  }
  return L;
}

// Stable LSD radix sort of keys ascending, four 8-bit passes: with kLds,
// sh.sortb[0..L) (L <= kSortCap) through sh.sorta, else k0[0..L) in global
// memory through k1; the result is back where the keys were.  The four digit
// histograms come from one read of the keys (a key's digits do not depend on
// the order); then each pass takes the keys kST at a time (the next kST read
// while the current ones are placed): ranks within a wave from ballots over
// the digit's bits, across waves from per-wave digit counts, two barriers
// per kST keys.
template <bool kLds>
__device__ __forceinline__ void radix_sort_impl(uint32_t* g0, uint32_t* g1, int L,
                                                SampleShared& sh) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const uint64_t lt = (1ull << lane) - 1ull;
  if (L <= 1) return;
  uint32_t* k0 = kLds ? sh.sortb : g0;
  uint32_t* k1 = kLds ? sh.sorta : g1;
  // hist[256 p + d]: keys whose digit p is d
  for (int i = t; i < 4 * 256; i += kST) sh.hist[i] = 0;
  __syncthreads();
  {
    constexpr int kR = 8;
    for (int b0 = 0; b0 < L; b0 += kR * kST) {
      uint32_t k[kR];
#pragma unroll
      for (int u = 0; u < kR; u++) k[u] = k0[min(b0 + u * kST + t, L - 1)];
#pragma unroll
      for (int u = 0; u < kR; u++) {
        if (b0 + u * kST + t < L) {
#pragma unroll
          for (int p = 0; p < 4; p++) atomicAdd(&sh.hist[256 * p + ((k[u] >> (8 * p)) & 255u)], 1u);
        }
      }
    }
  }
  __syncthreads();
  // exclusive offsets within each histogram: thread t scans entry t of
  // histogram t / 256 (four waves per histogram)
  {
    const uint32_t c = sh.hist[t];
    const uint32_t inc = wave_scan_sat(c);
    if (lane == 63) sh.wsum[wave] = inc;
    __syncthreads();
    uint32_t off = 0;
    for (int w = wave & ~3; w < wave; w++) off += sh.wsum[w];
    sh.hist[t] = off + inc - c;
  }
  for (int pass = 0; pass < 4; pass++) {
    const int shb = 8 * pass;
    const uint32_t* src = (pass & 1) ? k1 : k0;
    uint32_t* dst = (pass & 1) ? k0 : k1;
    __syncthreads();  // the offsets, and the previous pass's keys, are complete
    if (t < 256) sh.base[t] = sh.hist[256 * pass + t];
    uint32_t key = src[min(t, L - 1)];
    for (int b0 = 0; b0 < L; b0 += kST) {
      const int i = b0 + t;
      const bool valid = i < L;
      const uint32_t cur = key;
      if (b0 + kST < L) key = src[min(b0 + kST + t, L - 1)];  // the next kST
      const uint32_t d = (cur >> shb) & 255u;
      uint64_t m = __ballot(valid);
#pragma unroll
      for (int b = 0; b < 8; b++) {
        const uint64_t bb = __ballot((d >> b) & 1u);
        m &= ((d >> b) & 1u) ? bb : ~bb;
      }
      const int rank = __popcll(m & lt);
      // this wave's digit counts (its own row: zeros, then the counts; one
      // wave's LDS writes land in order)
      for (int e = lane; e < 256; e += 64) sh.cnt[wave][e] = 0;
      if (valid && rank == 0) sh.cnt[wave][d] = (uint32_t)__popcll(m);
      __syncthreads();
      if (t < 256) {
        uint32_t c[kSW];
#pragma unroll
        for (int w = 0; w < kSW; w++) c[w] = sh.cnt[w][t];
        uint32_t run = sh.base[t];
#pragma unroll
        for (int w = 0; w < kSW; w++) {
          sh.cnt[w][t] = run;
          run += c[w];
        }
        sh.base[t] = run;
      }
      __syncthreads();
      if (valid) dst[sh.cnt[wave][d] + rank] = cur;
    }
  }
  __syncthreads();
}

__device__ void radix_sort_keys(uint32_t* k0, uint32_t* k1, int L, SampleShared& sh) {
  radix_sort_impl<false>(k0, k1, L, sh);
}

__device__ void radix_sort_lds(int L, SampleShared& sh) {
  radix_sort_impl<true>(nullptr, nullptr, L, sh);
}

constexpr int kRankSortMax = 256;  // lists sorted by one rank pass

// Sorts keys k0[0..L) ascending; returns where the result is: sh.sortb (the
// keys copied there, L <= kSortCap) or k0 (a global sort through k1).  Up to
// kRankSortMax keys: thread t takes key t and places it at its rank (the
// keys below it, and the equal ones before it).
__device__ const uint32_t* sort_keys(uint32_t* k0, uint32_t* k1, int L, SampleShared& sh) {
  if (L > kSortCap) {
    radix_sort_keys(k0, k1, L, sh);
    return k0;
  }
  const int t = threadIdx.x;
  if (L <= kRankSortMax) {
    const uint32_t k = t < L ? k0[t] : 0u;
    if (t < L) sh.sorta[t] = k;
    __syncthreads();
    if (t < L) {
      int rank = 0;
      for (int j = 0; j < L; j++) {
        const uint32_t o = sh.sorta[j];  // the same address across the wave
        rank += o < k || (o == k && j < t);
      }
      sh.sortb[rank] = k;
    }
    __syncthreads();
    return sh.sortb;
  }
  constexpr int kPer = kSortCap / kST;
  uint32_t v[kPer];
#pragma unroll
  for (int u = 0; u < kPer; u++) v[u] = k0[min(t + u * kST, max(L - 1, 0))];
#pragma unroll
  for (int u = 0; u < kPer; u++)
    if (t + u * kST < L) sh.sortb[t + u * kST] = v[u];
  __syncthreads();
  radix_sort_lds(L, sh);
  return sh.sortb;
}

// The k-th largest (1-based, 1 <= kk <= cnt) of the keys key(j), j in
// [0, cnt), by radix select: 11, 11 and 10 bits of the key, one histogram
// pass per level.  Up to kSelReg * kST keys are read once into registers;
// more are read again at each level.
constexpr int kSelReg = 4;

template <typename Key>
__device__ uint32_t kth_largest_key(int cnt, Key key, uint32_t kk, SampleShared& sh) {
  const int t = threadIdx.x;
  const bool reg = cnt <= kSelReg * kST;
  uint32_t kr[kSelReg];
  if (reg) {
#pragma unroll
    for (int u = 0; u < kSelReg; u++) kr[u] = key(min(t + u * kST, cnt - 1));  // in bounds
  }
  // f(k) for every key this thread owns
  auto each = [&](auto f) {
    if (reg) {
#pragma unroll
      for (int u = 0; u < kSelReg; u++)
        if (t + u * kST < cnt) f(kr[u]);
    } else {
      for (int j = t; j < cnt; j += kST) f(key(j));
    }
  };
  uint32_t b1, b2, b3;
  for (int i = t; i < 2048; i += kST) sh.hist[i] = 0;
  __syncthreads();
  each([&](uint32_t k) { atomicAdd(&sh.hist[k >> 21], 1u); });
  __syncthreads();
  select_from_top(sh, 2048, kk, &b1, &kk);
  for (int i = t; i < 2048; i += kST) sh.hist[i] = 0;
  __syncthreads();
  each([&](uint32_t k) {
    if ((k >> 21) == b1) atomicAdd(&sh.hist[(k >> 10) & 2047u], 1u);
  });
  __syncthreads();
  select_from_top(sh, 2048, kk, &b2, &kk);
  for (int i = t; i < 1024; i += kST) sh.hist[i] = 0;
  __syncthreads();
  const uint32_t pre = (b1 << 11) | b2;
  each([&](uint32_t k) {
    if ((k >> 10) == pre) atomicAdd(&sh.hist[k & 1023u], 1u);
  });
  __syncthreads();
  select_from_top(sh, 1024, kk, &b3, &kk);
  return (pre << 10) | b3;
}

// The reference's sequential fp32 loops (s = s + v in index order) are
// reproduced exactly, but mostly in parallel.  While s is finite and not
// negative, every float32 at or above s in its binade is m u for an integer
// m < 2^24 with u = 2^(E - 150), E = max(exponent field of s, 1); for v >= 0
// finite, s + v = (m + v/u) u, so fl(s + v) = (m + d) u with d = v/u rounded
// to the nearest integer -- as long as v/u is not exactly halfway between
// two integers (then the tie goes to the even m + d, which depends on m) and
// m + d < 2^24 (else the sum leaves the binade).  d comes from the bit
// patterns by integer shifts, exactly (no division, no subnormal flushing).
// So over a run of such values the running sums are m + prefix sums of the
// d: the work-group computes them with a scan, finds the first value that is
// an event (a tie, a crossing of 2^24, a negative, infinite or NaN value)
// and, for a walk, the first running sum above thr, takes the sums up to
// the event, and adds the event value with one float32 addition on thread
// 0, as the reference does.  Events are rare (a binade crossing each time
// the sum doubles, exact ties); when they come densely, or s itself is
// negative, infinite or NaN (or -0), thread 0 adds the next values one at a
// time.  The values are staged in LDS by the whole work-group, kChunk at a
// time; the quotients p / S of the walks are computed by the staging
// threads.

// Staging of x(b0 + j), j < len (1 <= len <= kChunk), into sh.chunk, in two
// halves so that the next chunk is read while the current one is added:
// each thread's kChunk / kST values are all read before any is stored, so
// the reads are in flight together.  Positions past len evaluate x at the
// last position (in bounds, unconditionally, so no read sits in a branch)
// and are not stored.
constexpr int kStagePer = kChunk / kST;
template <typename X>
__device__ __forceinline__ void load_chunk(X x, int b0, int len, float (&v)[kStagePer]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int u = 0; u < kStagePer; u++) v[u] = x(b0 + min(t + u * kST, len - 1));
}
__device__ __forceinline__ void store_chunk(const float (&v)[kStagePer], int len, SampleShared& sh) {
  const int t = threadIdx.x;
#pragma unroll
  for (int u = 0; u < kStagePer; u++) {
    const int j = t + u * kST;
    if (j < len) sh.chunk[j] = v[u];
  }
}

constexpr int kAccMinAdv = 32;  // a parallel pass advancing less: go one by one
constexpr int kAccSeq = 256;    // values thread 0 adds one by one then
constexpr int kRun = 32;        // ... read kRun at a time
constexpr int kAccPer = 8;      // consecutive values per thread in a parallel pass
static_assert(kAccPer * kST == kChunk, "a parallel pass covers a chunk");
constexpr uint32_t kTwo24 = 1u << 24;


// Bit pattern of m u on the grid of exponent field E (m < 2^24; m < 2^23
// only with E = 1, the subnormal range).
__device__ __forceinline__ uint32_t acc_bits(int E, uint32_t m) {
  return ((uint32_t)(E - 1) << 23) + m;
}

// s = s + sh.chunk[j] for j = 0 .. len-1 in order, float32, exactly as the
// sequential loop; with WALK, stops after the first j at which s > thr and
// returns that j (else -1).  s, thr and adv are the same in every thread;
// adv, carried from chunk to chunk, is how far the last parallel pass got
// (below kAccMinAdv, as at the start, thread 0 adds the next values one at
// a time).
template <bool WALK>
__device__ int acc_chunk(int len, float& s, float thr, int& adv, SampleShared& sh) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  int pos = 0;
  while (pos < len) {
    const uint32_t sb = __float_as_uint(s);
    const bool regular = (sb >> 31) == 0 && (sb >> 23) != 255u;  // +0 <= s < inf
    if (!regular || adv < kAccMinAdv) {
      // thread 0 adds the next values one at a time
      if (t == 0) {
        const int stop = min(len, pos + (regular ? kAccSeq : 64));
        int hit = -1, j = pos;
        float c = s;
        // runs of kRun values: the run's reads are all issued before its
        // additions; the first sum above thr is noted, the run finished
        for (; j + kRun <= stop && hit < 0; j += kRun) {
          float v[kRun];
#pragma unroll
          for (int u = 0; u < kRun; u++) v[u] = sh.chunk[j + u];
#pragma unroll
          for (int u = 0; u < kRun; u++) {
            c += v[u];
            if (WALK && hit < 0 && c > thr) hit = j + u;
          }
        }
        for (; j < stop && hit < 0; j++) {
          c += sh.chunk[j];
          if (WALK && c > thr) hit = j;
        }
        sh.acc_s = __float_as_uint(c);
        sh.acc_i[1] = hit;
        sh.acc_i[2] = j;
      }
      __syncthreads();
      s = __uint_as_float(sh.acc_s);
      const int hit = sh.acc_i[1];
      pos = sh.acc_i[2];
      __syncthreads();
      if (WALK && hit >= 0) return hit;
      adv = kAccMinAdv;
      if (s != s) return WALK ? -2 : -1;  // NaN: every later sum is NaN
      continue;
    }
    // Parallel pass over [pos, len): thread t takes the kAccPer values from
    // a0 + kAccPer t (a0 = pos rounded down to a multiple of kAccPer; values
    // outside [pos, len) count as 0).
    const int E = max((int)(sb >> 23), 1);
    const int sc = 150 - E;
    const uint32_t m0 = ((sb >> 23) ? 0x800000u : 0u) | (sb & 0x7FFFFFu);
    const int a0 = pos & ~(kAccPer - 1);
    const int lo = a0 + kAccPer * t;
    float v[kAccPer];
    if (lo < len) {  // in bounds: lo + kAccPer <= kChunk
      const float4* c4 = reinterpret_cast<const float4*>(sh.chunk + lo);
#pragma unroll
      for (int q = 0; q < kAccPer / 4; q++) {
        const float4 f = c4[q];
        v[4 * q] = f.x;
        v[4 * q + 1] = f.y;
        v[4 * q + 2] = f.z;
        v[4 * q + 3] = f.w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < kAccPer; e++) v[e] = 0.0f;
    }
    // values outside [pos, len) count as +0 (only thread 0 and the thread
    // holding position len have any)
    if (lo < pos || lo + kAccPer > len) {
#pragma unroll
      for (int e = 0; e < kAccPer; e++) v[e] = lo + e < pos || lo + e >= len ? 0.0f : v[e];
    }
    uint32_t d[kAccPer];
    bool ev[kAccPer];
    bool any_ev = false;
    uint32_t tot = 0;
#pragma unroll
    for (int e = 0; e < kAccPer; e++) {
      bool tie;
      const uint32_t de = acc_increment(v[e], sc, tie);
      // negative (or -0), infinite or NaN values, and ties, are events:
      // classes sNaN, qNaN, -inf, -normal, -subnormal, -0, +inf
      ev[e] = __builtin_amdgcn_classf(v[e], 0x23F) || tie;
      d[e] = ev[e] ? 0u : de;
      tot += d[e];  // <= 8 2^24
      any_ev = any_ev || ev[e];
    }
    const uint32_t inc = wave_scan_sat(tot);
    if (lane == 63) sh.acc_w[w] = inc;
    __syncthreads();
    // the waves before this one: their totals, read four at a time
    uint32_t woff = 0;
    const uint4* w4 = reinterpret_cast<const uint4*>(sh.acc_w);
#pragma unroll
    for (int q = 0; q < kSW / 4; q++) {
      const uint4 x = w4[q];
      woff = usat_add(woff, 4 * q < w ? x.x : 0u);
      woff = usat_add(woff, 4 * q + 1 < w ? x.y : 0u);
      woff = usat_add(woff, 4 * q + 2 < w ? x.z : 0u);
      woff = usat_add(woff, 4 * q + 3 < w ? x.w : 0u);
    }
    // this thread's running sums (exact while below 2^24): its first event
    // (an event value, or a sum reaching 2^24) and, for a walk, its first sum
    // above thr before that; run stops before the first of them.  The sums
    // only grow, so a thread with no event value whose last sum stays below
    // 2^24 (and, walking, at most thr) has neither; one starting at 2^24 or
    // more has its first value in range as its event.
    uint32_t run = usat_add(m0, usat_add(woff, inc - tot));
    const uint32_t last = usat_add(run, tot);
    int my_ev = len, my_hit = 0x7FFFFFFF;
    if (run >= kTwo24) {
      my_ev = max(lo, pos);
    } else if (any_ev || last >= kTwo24 ||
               (WALK && __uint_as_float(acc_bits(E, last)) > thr)) {
      bool stop = false;
#pragma unroll
      for (int e = 0; e < kAccPer; e++) {
        const uint32_t nr = usat_add(run, d[e]);
        const bool is_ev = !stop && (ev[e] || nr >= kTwo24);
        my_ev = is_ev ? lo + e : my_ev;
        stop = stop || is_ev;
        const bool is_hit = WALK && !stop && lo + e >= pos && lo + e < len &&
                            __uint_as_float(acc_bits(E, nr)) > thr;
        my_hit = is_hit ? lo + e : my_hit;
        run = stop ? run : nr;
        stop = stop || is_hit;
      }
    } else {
      run = last;
    }
    // the wave's first event and first hit: those of its lowest lane that
    // has one (the lanes' values are in index order)
    const uint64_t em = __ballot(my_ev < len);
    const uint64_t hm = WALK ? __ballot(my_hit != 0x7FFFFFFF) : 0ull;
    const int wev = em ? __builtin_amdgcn_readlane(my_ev, __builtin_ctzll(em)) : len;
    const int whit = hm ? __builtin_amdgcn_readlane(my_hit, __builtin_ctzll(hm)) : 0x7FFFFFFF;
    if (lane == 0) {
      sh.acc_ev[w] = wev;
      sh.acc_hit[w] = whit;
    }
    __syncthreads();
    int fe = len, fh = 0x7FFFFFFF;
    {
      const int4* e4 = reinterpret_cast<const int4*>(sh.acc_ev);
      const int4* h4 = reinterpret_cast<const int4*>(sh.acc_hit);
#pragma unroll
      for (int q = 0; q < kSW / 4; q++) {
        const int4 a = e4[q];
        fe = min(fe, min(min(a.x, a.y), min(a.z, a.w)));
        if (WALK) {
          const int4 b = h4[q];
          fh = min(fh, min(min(b.x, b.y), min(b.z, b.w)));
        }
      }
    }
    if (WALK && fh < fe) {
      __syncthreads();  // every thread read acc_i before it is reused
      return fh;
    }
    // The sum after the pass: the thread holding the first event adds the
    // event value to the running sum before it (one float32 addition); with
    // no event, the thread holding the last value has the sum.
    const int owner = fe < len ? fe : len - 1;
    if (owner >= lo && owner < lo + kAccPer) {
      if (fe < len) {
        const float c = __uint_as_float(acc_bits(E, run)) + sh.chunk[fe];
        sh.acc_s = __float_as_uint(c);
        sh.acc_i[2] = WALK && c > thr ? 1 : 0;
      } else {
        sh.acc_s = acc_bits(E, run);
        sh.acc_i[2] = 0;
      }
    }
    __syncthreads();
    s = __uint_as_float(sh.acc_s);
    if (WALK && sh.acc_i[2] != 0) {
      __syncthreads();  // every thread read acc_i before it is reused
      return fe;
    }
    adv = fe - pos;
    pos = fe < len ? fe + 1 : len;
    if (s != s) return WALK ? -2 : -1;
  }
  return -1;
}

// -0.0 + x(0) + x(1) + ... in index order, fp32 (Iterator::sum); every thread
// gets the result.
// on_chunk(len) runs on each staged chunk (sh.chunk[0..len)) before it is
// added; it may read the chunk, not change it.
template <typename X, typename F>
__device__ float seq_sum(int cnt, X x, SampleShared& sh, F on_chunk) {
  float s = -0.0f;
  int adv = 0;  // the first values one at a time
  if (cnt <= 0) return s;
  float v[kStagePer];
  load_chunk(x, 0, min(kChunk, cnt), v);
  for (int b0 = 0; b0 < cnt; b0 += kChunk) {
    const int len = min(kChunk, cnt - b0);
    store_chunk(v, len, sh);  // the previous chunk's reads ended at its last barrier
    __syncthreads();
    // the next chunk's values are read while this one is added
    if (b0 + kChunk < cnt) load_chunk(x, b0 + kChunk, min(kChunk, cnt - b0 - kChunk), v);
    on_chunk(len);
    acc_chunk<false>(len, s, 0.0f, adv, sh);  // its barriers follow on_chunk's reads
    if (s != s) return s;  // NaN stays NaN
  }
  return s;
}

template <typename X>
__device__ float seq_sum(int cnt, X x, SampleShared& sh) {
  return seq_sum(cnt, x, sh, [](int) {});
}

// The first j in [0, cnt) at which cum (0.0 + q(0) + ... + q(j), fp32, in
// order) exceeds thr (thread 0's value, the one every thread compares
// with); -1 if none.
template <typename Q>
__device__ int seq_cross(int cnt, Q q, float thr0, SampleShared& sh) {
  if (threadIdx.x == 0) sh.f[0] = thr0;
  __syncthreads();
  const float thr = sh.f[0];
  __syncthreads();
  float cum = 0.0f;
  int adv = 0;  // the first values one at a time
  if (cnt <= 0) return -1;
  float v[kStagePer];
  load_chunk(q, 0, min(kChunk, cnt), v);
  for (int b0 = 0; b0 < cnt; b0 += kChunk) {
    const int len = min(kChunk, cnt - b0);
    store_chunk(v, len, sh);  // the previous chunk's reads ended at its last barrier
    __syncthreads();
    if (b0 + kChunk < cnt) load_chunk(q, b0 + kChunk, min(kChunk, cnt - b0 - kChunk), v);
    const int hit = acc_chunk<true>(len, cum, thr, adv, sh);
    if (hit >= 0) return b0 + hit;
    if (hit == -2) return -1;  // cum is NaN: it exceeds nothing
  }
  return -1;
}

// Margin of the top-p bins: how far, relative to the total, the fp32 running
// sums of L values can stray from exact ones (2 (L + 2) 2^-24).
__device__ __forceinline__ double top_p_margin(int L) { return 2.0 * ((double)L + 2.0) * 0x1p-24; }

// Without top-k, top-p over a long list walks only the key bins from the
// top down to where their exact mass reaches top_p + margin of the total.
__device__ __forceinline__ bool top_bins_apply(const SampleArgs& a) {
  const bool use_k = a.top_k > 0 && a.top_k < a.n;
  return !use_k && a.top_p < 1.0f && a.n > kChunk && (double)a.top_p + top_p_margin(a.n) < 1.0;
}

// First kernel, `parts` work-groups over consecutive ranges [lo, hi) of the
// logits: each range's ArgPart; unless greedy, p_i for its elements, and
//  * with top-k, the range's candidates, in index order, at
//    [lo, lo + seg_cnt[g]) of seg_idx / seg_val: the elements whose key is at
//    least the range's own k-th largest key (every element of a range of at
//    most k), and every NaN: an element that top-k keeps is at least the
//    overall k-th largest p, and fewer than k elements in all (so in its
//    range) exceed it;
//  * without, when top_bins_apply, the range's mass (double) in each of the
//    kBins1 key bins, and in seg_cnt[g] whether any p is negative, infinite
//    or NaN (the bins are then not used).
__global__ void __launch_bounds__(kST) sample_parts_kernel(const SampleArgs a) {
  __shared__ SampleShared sh;
  const int t = threadIdx.x, g = blockIdx.x;
  const int lo = (int)((long long)a.n * g / a.parts);
  const int hi = (int)((long long)a.n * (g + 1) / a.parts);
  const ArgPart ap = argmax_part(lo, hi, [&](int i) { return a.logits[i]; }, sh);
  if (t == 0) a.part[g] = ap;
  if (a.greedy_only) return;
  const bool use_k = a.top_k > 0 && a.top_k < a.n;
  const bool bins = top_bins_apply(a);
  if (bins) {
    for (int i = t; i < kBins1; i += kST) sh.mass[i] = 0.0;
    __syncthreads();
  }
  const bool scale = a.temperature > 0.0f;
  int bad = 0;
  for (int i = lo + t; i < hi; i += kST) {
    const float l = a.logits[i];
    const float p = scale ? (float)exp((double)(l * a.inv_temp)) : l;
    a.probs[i] = p;
    if (bins) {
      bad |= !(p >= 0.0f && p < __builtin_inff());
      atomicAdd(&sh.mass[fkey(p) >> 21], (double)p);
    }
  }
  if (!use_k) {
    if (bins) {
      bad = __syncthreads_or(bad);
      static_assert(kBins1 == 2 * kST, "two bins per thread");
      reinterpret_cast<double2*>(a.range_mass)[(size_t)g * kST + t] =
          make_double2(sh.mass[2 * t], sh.mass[2 * t + 1]);
      if (t == 0) a.seg_cnt[g] = bad;
    }
    return;
  }
  __syncthreads();
  int cnt;
  {
    const uint32_t kth = hi - lo > a.top_k
                             ? kth_largest_key(hi - lo, [&](int j) { return fkey(a.probs[lo + j]); },
                                               (uint32_t)a.top_k, sh)
                             : 0u;
    cnt = compact_range(
        lo, hi, [&](int i) { return a.probs[i]; },
        [&](int, float x) { return fkey(x) >= kth || __builtin_isnan(x); }, a.seg_idx + lo,
        a.seg_val + lo, sh);
  }
  if (t == 0) a.seg_cnt[g] = cnt;
}

// Appends ~key of every staged value whose key is at least tkey to
// sh.sortb, in no particular order, counting in sh.u[3] (one LDS atomic per
// wave); keys past kSortCap are counted, not stored.
__device__ void gather_top_keys(int len, uint32_t tkey, SampleShared& sh) {
  const int t = threadIdx.x, lane = t & 63;
  const uint64_t lt = (1ull << lane) - 1ull;
  constexpr int kPer = kChunk / kST;
  uint32_t k[kPer];
  uint64_t m[kPer];
  uint32_t cnt = 0;
#pragma unroll
  for (int e = 0; e < kPer; e++) {
    const int j = t + e * kST;
    k[e] = j < len ? fkey(sh.chunk[j]) : 0u;
    m[e] = __ballot(j < len && k[e] >= tkey);
    cnt += (uint32_t)__popcll(m[e]);
  }
  if (cnt == 0) return;  // the whole wave
  uint32_t base = 0;
  if (lane == 0) base = atomicAdd(&sh.u[3], cnt);
  base = (uint32_t)__builtin_amdgcn_readfirstlane((int)base);
#pragma unroll
  for (int e = 0; e < kPer; e++) {
    const uint32_t at = base + (uint32_t)__popcll(m[e] & lt);
    if (((m[e] >> lane) & 1ull) && at < (uint32_t)kSortCap) sh.sortb[at] = ~k[e];
    base += (uint32_t)__popcll(m[e]);
  }
}

// Without top-k: the top key bin whose mass, added from the top down,
// reaches (top_p + margin) of the total, from the ranges' bin masses;
// -1 when a range held a negative, infinite or NaN p, or no bin reaches it
// (the double sums' order differs from a sequential one: any bin is a
// correct choice, it only decides how much is sorted before the fallback).
__device__ int top_mass_bin(const SampleArgs& a, SampleShared& sh) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  // bins 2t and 2t + 1 over the ranges, 16 ranges' loads in flight
  constexpr int kB = 16;
  const double2* rm = reinterpret_cast<const double2*>(a.range_mass);
  double m0 = 0.0, m1 = 0.0;
  for (int g0 = 0; g0 < a.parts; g0 += kB) {
    double2 v[kB];
#pragma unroll
    for (int u = 0; u < kB; u++) v[u] = rm[(size_t)min(g0 + u, a.parts - 1) * kST + t];
#pragma unroll
    for (int u = 0; u < kB; u++) {
      if (g0 + u < a.parts) {
        m0 += v[u].x;
        m1 += v[u].y;
      }
    }
  }
  const int bad = __syncthreads_or(t < a.parts ? a.seg_cnt[t] : 0);
  if (bad) return -1;
  sh.mass[2 * t] = m0;
  sh.mass[2 * t + 1] = m1;
  __syncthreads();
  // top-first: thread t owns bins 2047 - 2t, then 2046 - 2t
  const double c0 = sh.mass[kBins1 - 1 - 2 * t], c1 = sh.mass[kBins1 - 2 - 2 * t];
  double incl = c0 + c1;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const double o = __shfl_up(incl, off, 64);
    if (lane >= off) incl += o;
  }
  double excl = __shfl_up(incl, 1, 64);
  if (lane == 0) excl = 0.0;
  if (lane == 63) sh.dred[w] = incl;
  __syncthreads();
  double before = 0.0, tot = 0.0;
  for (int v = 0; v < kSW; v++) {
    const double d = sh.dred[v];
    if (v < w) before += d;
    tot += d;
  }
  const double need = ((double)a.top_p + top_p_margin(a.n)) * tot;
  const double a0 = before + excl + c0, a1 = a0 + c1;
  const int cand = a0 >= need ? 2 * t : a1 >= need ? 2 * t + 1 : 0x7FFFFFFF;
  // the first candidate from the top: that of the lowest such thread
  const uint64_t cm = __ballot(cand != 0x7FFFFFFF);
  const int wc = cm ? __builtin_amdgcn_readlane(cand, __builtin_ctzll(cm)) : 0x7FFFFFFF;
  if (lane == 0) sh.ired[w] = wc;
  __syncthreads();
  int first = 0x7FFFFFFF;
  for (int v = 0; v < kSW; v++) first = min(first, sh.ired[v]);
  __syncthreads();  // sh.ired / sh.dred read by all before reuse
  return first == 0x7FFFFFFF ? -1 : kBins1 - 1 - first;
}

// A work-group barrier that orders LDS only: __syncthreads() also waits for
// every global store in flight (a release), which a loop whose stores are
// read only after it ends need not pay at each step.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// The elements of p[0..n) not below thr (NaN included), in index order, to
// (ov, oi); returns their count.  Per pass thread t takes the kCP
// consecutive values from kCP t (all its reads in flight together): the
// kept count per thread, a DPP wave scan, the waves' totals through LDS.
// The kept values are placed in LDS at their list positions, then copied
// out contiguously (scattered global stores, one masked instruction per
// value slot, cost several times more); a pass keeping more than the LDS
// holds stores them directly.  Uses sh.sorta / sh.sortb.
constexpr int kCP = 32;
constexpr int kCStage = kSortCap;  // values a pass stages (sorta as floats, sortb)

__device__ int compact_kept(const float* p, int n, float thr, float* ov, uint32_t* oi,
                            SampleShared& sh) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  int base = 0;
  for (int c0 = 0; c0 < n; c0 += kCP * kST) {
    const int lo = c0 + kCP * t;
    float v[kCP];
    if (lo + kCP <= n) {
      const float4* p4 = reinterpret_cast<const float4*>(p + lo);  // p is 16-byte aligned
#pragma unroll
      for (int q = 0; q < kCP / 4; q++) {
        const float4 f = p4[q];
        v[4 * q] = f.x;
        v[4 * q + 1] = f.y;
        v[4 * q + 2] = f.z;
        v[4 * q + 3] = f.w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < kCP; e++) v[e] = lo + e < n ? p[lo + e] : 0.0f;
    }
    uint32_t km = 0;
#pragma unroll
    for (int e = 0; e < kCP; e++) km |= (lo + e < n && !(v[e] < thr)) ? 1u << e : 0u;
    const uint32_t cnt = (uint32_t)__popc(km);
    const uint32_t inc = wave_scan_sat(cnt);
    if (lane == 63) sh.acc_w[w] = inc;
    lds_barrier();  // the stores of the passes before may still be in flight
    uint32_t woff = 0, tot = 0;
    const uint4* w4 = reinterpret_cast<const uint4*>(sh.acc_w);
#pragma unroll
    for (int q = 0; q < kSW / 4; q++) {
      const uint4 x = w4[q];
      const uint32_t xs[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
      for (int k = 0; k < 4; k++) {
        woff += 4 * q + k < w ? xs[k] : 0u;
        tot += xs[k];
      }
    }
    if (tot <= (uint32_t)kCStage) {
      float* lv = reinterpret_cast<float*>(sh.sorta);
      uint32_t* li = sh.sortb;
      int q = (int)(woff + inc - cnt);
#pragma unroll
      for (int e = 0; e < kCP; e++) {
        if ((km >> e) & 1u) {
          lv[q] = v[e];
          li[q] = (uint32_t)(lo + e);
          q++;
        }
      }
      lds_barrier();
      for (int i = t; i < (int)tot; i += kST) {
        ov[base + i] = lv[i];
        oi[base + i] = li[i];
      }
    } else {
      int pos = base + (int)(woff + inc - cnt);
#pragma unroll
      for (int e = 0; e < kCP; e++) {
        if ((km >> e) & 1u) {
          ov[pos] = v[e];
          oi[pos] = (uint32_t)(lo + e);
          pos++;
        }
      }
    }
    base += (int)tot;
    lds_barrier();  // acc_w and the staging are read by all before the next pass
  }
  __syncthreads();  // the list is complete and visible
  return base;
}

// sample_token without top-k: the sums and walks run over p itself, all n
// values in index order, zeros included, as the reference's loops do
// (run.rs:203-251); the draw's index is the token.
__device__ void sample_no_topk(const SampleArgs& a, SampleShared& sh) {
  const int t = threadIdx.x;
  const int n = a.n;
  const float* p = a.probs;
  float thr_p = -__builtin_inff();
  if (a.top_p < 1.0f) {
    const int top = top_bins_apply(a) ? top_mass_bin(a, sh) : -1;
    const uint32_t tkey = (uint32_t)(top < 0 ? 0 : top) << 21;
    if (t == 0) {
      sh.u[2] = 0;
      sh.u[3] = 0;
    }
    __syncthreads();
    // the sum, gathering the keys of the top bins (into LDS) from its staged
    // chunks
    const float sum1 = seq_sum(n, [&](int j) { return p[j]; }, sh, [&](int len) {
      if (top >= 0) gather_top_keys(len, tkey, sh);
    });
    const int Lc = (int)sh.u[3];
    if (sum1 > 0.0f) {
      int at = -1;
      const uint32_t* keys = a.k0;
      if (top >= 0) {
        if (Lc <= kSortCap) {
          radix_sort_lds(Lc, sh);
          keys = sh.sortb;
        } else {  // too many for LDS: gathered again, into global memory
          for (int j = t; j < n; j += kST) {
            const uint32_t k = fkey(p[j]);
            if (k >= tkey) a.k0[atomicAdd(&sh.u[2], 1u)] = ~k;
          }
          __syncthreads();
          radix_sort_keys(a.k0, a.k1, Lc, sh);
        }
        at = seq_cross(Lc, [&](int j) { return funkey(~keys[j]) / sum1; }, a.top_p, sh);
      }
      if (at < 0) {  // every p, sorted
        for (int j = t; j < n; j += kST) a.k0[j] = ~fkey(p[j]);
        __syncthreads();
        radix_sort_keys(a.k0, a.k1, n, sh);
        keys = a.k0;
        at = seq_cross(n, [&](int j) { return funkey(~keys[j]) / sum1; }, a.top_p, sh);
      }
      thr_p = at >= 0 ? funkey(~keys[at]) : 3.40282347e+38f;
    }
    __syncthreads();  // sh.u[3] read by all before reuse
  }
  const float tp = thr_p;
  auto q = [&](int j) {
    const float x = p[j];
    return x < tp ? 0.0f : x;
  };
  // With a top-p threshold, the survivors (p not below it) in index order:
  // the zeros between them change neither the sum nor where the draw's
  // running sum crosses r, so both run over the short list.  The draw:
  // len values val(j), the token of position j tok(j); false when the sum
  // is not positive (the argmax of the logits is the token then) or the
  // walk does not cross.
  auto draw = [&](int len, auto val, auto tok) -> bool {
    const float sum2 = seq_sum(len, val, sh);
    if (sum2 <= 0.0f) {
      if (t == 0) *a.token = argmax_combine(a.part, a.parts, n);
      return true;
    }
    // r = next_f32(): xorshift 13, 7, 17, then the top 24 bits / 2^24
    float r = 0.0f;
    if (t == 0) {
      uint64_t x = *a.state;
      x ^= x << 13;
      x ^= x >> 7;
      x ^= x << 17;
      *a.state = x;
      r = (float)(x >> 40) / 16777216.0f;
    }
    // the first index whose running sum of p / S exceeds r (r < cum)
    const int at = seq_cross(len, [&](int j) { return val(j) / sum2; }, r, sh);
    if (at >= 0) {
      if (t == 0) *a.token = tok(at);
      return true;
    }
    return false;
  };
  bool done;
  if (thr_p > -__builtin_inff()) {
    const int Lb = compact_kept(p, n, tp, a.a_val, a.a_idx, sh);
    const float* bv = a.a_val;
    const uint32_t* bi = a.a_idx;
    done = draw(Lb, [&](int j) { return bv[j]; }, [&](int j) { return bi[j]; });
  } else {
    done = draw(n, [&](int j) { return p[j]; }, [&](int j) { return (uint32_t)j; });
  }
  if (done) return;
  const uint32_t am = argmax_fold(n, q, sh);
  if (t == 0) *a.token = am;
}

// Greedy argmax (Iterator::max_by over partial_cmp, as argmax_combine) in
// one work-group and one launch: each thread reads the 16-byte pieces
// r kST + t of the aligned body (coalesced, kB in flight), keeping the best
// (value, the later index on ties) and whether it met a NaN; thread 0 also
// takes the elements before the first 16-byte boundary and after the last.
// A NaN anywhere (rare) sends the work-group to the exact scan: the last
// NaN, then the best after it.
__global__ void __launch_bounds__(kST) argmax_one_kernel(const float* __restrict__ x, int n,
                                                         uint32_t* token) {
  __shared__ SampleShared sh;
  const int t = threadIdx.x, lane = t & 63;
  if (n <= 0) {
    if (t == 0) *token = 0u;
    return;
  }
  const uintptr_t addr = reinterpret_cast<uintptr_t>(x);
  const int head = min(n, (int)(((16u - (addr & 15u)) & 15u) >> 2));
  const int nv = (n - head) >> 2;  // 16-byte pieces
  const float4* x4 = reinterpret_cast<const float4*>(x + head);
  float bv = 0.0f;
  int bi = -1;
  int nan = 0;
  auto take = [&](float v, int i) {
    nan |= v != v;
    if (bi < 0 || v >= bv) {  // indices grow per thread: ties go to the later
      bv = v;
      bi = i;
    }
  };
  if (t == 0)
    for (int i = 0; i < head; i++) take(x[i], i);
  constexpr int kB = 16;
  for (int r0 = 0; r0 * kST < nv; r0 += kB) {
    float4 v[kB];
#pragma unroll
    for (int u = 0; u < kB; u++) v[u] = x4[min((r0 + u) * kST + t, nv - 1)];  // in bounds
#pragma unroll
    for (int u = 0; u < kB; u++) {
      const int p = (r0 + u) * kST + t;
      if (p < nv) {
        const int i = head + 4 * p;
        take(v[u].x, i);
        take(v[u].y, i + 1);
        take(v[u].z, i + 2);
        take(v[u].w, i + 3);
      }
    }
  }
  if (t == 0)
    for (int i = head + 4 * nv; i < n; i++) take(x[i], i);
  if (__syncthreads_or(nan)) {
    const ArgPart p = argmax_part(0, n, [&](int i) { return x[i]; }, sh);
    if (t == 0) *token = argmax_combine(&p, 1, n);
    return;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(bv, off, 64);
    const int oi = __shfl_xor(bi, off, 64);
    if (arg_better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if (lane == 0) {
    sh.fred[t >> 6] = bv;
    sh.ired[t >> 6] = bi;
  }
  __syncthreads();
  if (t == 0) {
    float fv = 0.0f;
    int fi = -1;
    for (int w = 0; w < kSW; w++)
      if (arg_better(sh.fred[w], sh.ired[w], fv, fi)) {
        fv = sh.fred[w];
        fi = sh.ired[w];
      }
    *token = (uint32_t)fi;
  }
}

// Second kernel, one work-group: the rest of sample_token.
__global__ void __launch_bounds__(kST) sample_token_kernel(const SampleArgs a) {
  __shared__ SampleShared sh;
  const int t = threadIdx.x;
  const int n = a.n;
  if (a.greedy_only) {
    if (t == 0) *a.token = argmax_combine(a.part, a.parts, n);
    return;
  }
  const bool use_k = a.top_k > 0 && a.top_k < n;
  if (!use_k) {
    sample_no_topk(a, sh);
    return;
  }
  // the ranges' candidate lists, concatenated in order (index order), into
  // k0 (indices) / k1 (values) for the top-k pass; the ranges' offsets by
  // one wave (lane g reads range g's count: parts <= 64), a DPP scan
  static_assert(kMaxParts <= 64, "one lane per range");
  if (t < 64) {
    const uint32_t c = t < a.parts ? (uint32_t)a.seg_cnt[t] : 0u;
    const uint32_t inc = wave_scan_sat(c);
    sh.cnt[0][t] = inc - c;
    if (t == 63) sh.u[2] = inc;
  }
  __syncthreads();
  const int C = (int)sh.u[2];
  uint32_t* cidx = a.k0;
  float* cval = reinterpret_cast<float*>(a.k1);
  // Element i of the concatenation is element i - off[g] of range g, g the
  // last range with off[g] <= i (a binary search over the range offsets);
  // each thread reads kPer elements before storing any, so the reads are in
  // flight together.
  {
    constexpr int kPer = 8;
    auto range_of = [&](int i) {
      int lo = 0, hi = a.parts - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if ((int)sh.cnt[0][mid] <= i)
          lo = mid;
        else
          hi = mid - 1;
      }
      return lo;
    };
    for (int base = 0; base < C; base += kPer * kST) {
      uint32_t vi[kPer];
      float vv[kPer];
      int dst[kPer];
#pragma unroll
      for (int u = 0; u < kPer; u++) {
        const int i = min(base + u * kST + t, C - 1);
        const int g = range_of(i);
        const int src = (int)((long long)n * g / a.parts) + (i - (int)sh.cnt[0][g]);
        vi[u] = a.seg_idx[src];
        vv[u] = a.seg_val[src];
        dst[u] = base + u * kST + t;
      }
#pragma unroll
      for (int u = 0; u < kPer; u++) {
        if (dst[u] < C) {
          cidx[dst[u]] = vi[u];
          cval[dst[u]] = vv[u];
        }
      }
    }
  }
  __syncthreads();
  // top_k: the k-th largest p; the non-zero p not below it, in index order
  // (zeros add nothing to the running sums)
  const float thr_k =
      funkey(kth_largest_key(C, [&](int j) { return fkey(cval[j]); }, (uint32_t)a.top_k, sh));
  const int L = compact_range(
      0, C, [&](int j) { return cval[j]; },
      [&](int, float x) { return !(x < thr_k) && x != 0.0f; }, a.a_idx, a.a_val, sh);
  for (int j = t; j < L; j += kST) a.a_idx[j] = a.k0[a.a_idx[j]];  // positions -> tokens
  __syncthreads();
  // top_p: walk the p in descending order (sorted keys)
  float thr_p = -__builtin_inff();
  int Lb = L;
  const float* bval = a.a_val;
  const uint32_t* bidx = a.a_idx;
  if (a.top_p < 1.0f) {
    const float sum1 = seq_sum(L, [&](int j) { return a.a_val[j]; }, sh);
    if (sum1 > 0.0f) {
      // The walk only reaches the largest p: for long lists, sort just the
      // bins (11 key bits) from the top down to where their exact mass
      // reaches top_p + margin of the total, the margin covering how far the
      // fp32 sums can stray from exact ones (2 (L + 2) 2^-24 relative);
      // failing that (top_p near 1, negative or non-finite p), or should the
      // walk not cross in them, all of the p.
      const double margin = top_p_margin(L);
      int at = -1;
      const uint32_t* keys = a.k0;  // the sorted keys: global, or LDS
      if (L > kChunk && (double)a.top_p + margin < 1.0) {
        for (int i = t; i < kBins1; i += kST) sh.mass[i] = 0.0;
        __syncthreads();
        int bad = 0;
        for (int j = t; j < L; j += kST) {
          const float x = a.a_val[j];
          bad |= !(x > 0.0f && x < __builtin_inff());
          atomicAdd(&sh.mass[fkey(x) >> 21], (double)x);
        }
        bad = __syncthreads_or(bad);
        if (t == 0) {
          int top = -1;
          if (!bad) {
            double tot = 0.0;
            for (int b = 0; b < kBins1; b++) tot += sh.mass[b];
            const double need = ((double)a.top_p + margin) * tot;
            double acc = 0.0;
            for (int b = kBins1 - 1; b >= 0; b--) {
              acc += sh.mass[b];
              if (acc >= need) {
                top = b;
                break;
              }
            }
          }
          sh.ired[0] = top;
        }
        __syncthreads();
        const int top = sh.ired[0];
        __syncthreads();
        if (top >= 0) {
          const uint32_t tkey = (uint32_t)top << 21;
          float* cv = reinterpret_cast<float*>(a.k0);
          const int Lc = compact_range(
              0, L, [&](int j) { return a.a_val[j]; },
              [&](int, float x) { return fkey(x) >= tkey; }, a.k1, cv, sh);
          for (int j = t; j < Lc; j += kST) a.k0[j] = ~fkey(cv[j]);  // descending
          __syncthreads();
          keys = sort_keys(a.k0, a.k1, Lc, sh);
          at = seq_cross(Lc, [&](int j) { return funkey(~keys[j]) / sum1; }, a.top_p, sh);
        }
      }
      if (at < 0) {
        for (int j = t; j < L; j += kST) a.k0[j] = ~fkey(a.a_val[j]);  // descending
        __syncthreads();
        keys = sort_keys(a.k0, a.k1, L, sh);
        at = seq_cross(L, [&](int j) { return funkey(~keys[j]) / sum1; }, a.top_p, sh);
      }
      thr_p = at >= 0 ? funkey(~keys[at]) : 3.40282347e+38f;
      // p < thr_p -> 0: keep the survivors of the index-ordered list, in
      // order (k0 / k1 reused as the second list's storage)
      uint32_t* b_idx = a.k1;
      float* b_val = reinterpret_cast<float*>(a.k0);
      const uint32_t* ai = a.a_idx;
      const float* av = a.a_val;
      __syncthreads();
      Lb = compact_range(
          0, L, [&](int j) { return av[j]; }, [&](int, float x) { return !(x < thr_p); }, b_idx,
          b_val, sh);
      // compact_range stored list positions; map them to token indices
      for (int j = t; j < Lb; j += kST) b_idx[j] = ai[b_idx[j]];
      __syncthreads();
      bval = b_val;
      bidx = b_idx;
    }
  }
  const float sum2 = seq_sum(Lb, [&](int j) { return bval[j]; }, sh);
  if (sum2 <= 0.0f) {
    if (t == 0) *a.token = argmax_combine(a.part, a.parts, n);
    return;
  }
  // r = next_f32(): xorshift 13, 7, 17, then the top 24 bits / 2^24
  float r = 0.0f;
  if (t == 0) {
    uint64_t x = *a.state;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *a.state = x;
    r = (float)(x >> 40) / 16777216.0f;
  }
  // the first token whose running sum of p / S exceeds r (r < cum)
  const int at = seq_cross(Lb, [&](int j) { return bval[j] / sum2; }, r, sh);
  if (at >= 0) {
    if (t == 0) *a.token = bidx[at];
    return;
  }
  const uint32_t am = argmax_fold(
      n,
      [&](int i) {
        float p = a.probs[i];
        p = p < thr_k ? 0.0f : p;
        return p < thr_p ? 0.0f : p;
      },
      sh);
  if (t == 0) *a.token = am;
}

}  // namespace

hipError_t launch_embed_rows(float* out, const uint8_t* table, size_t table_len, int dtype,
                             const uint32_t* ids, size_t id0, size_t count, size_t hd,
                             hipStream_t s) {
  EmbedArgs a{out, table, table_len, ids, id0, dtype, hd};
  hipLaunchKernelGGL(embed_rows_kernel, dim3((unsigned)count), dim3(256), 0, s, a);
  return hipGetLastError();
}

static size_t round_up256(size_t v) { return (v + 255) / 256 * 256; }

static int sample_parts(size_t n) {
  const size_t p = (n + kPartElems - 1) / kPartElems;
  return (int)(p < 1 ? 1 : p > (size_t)kMaxParts ? (size_t)kMaxParts : p);
}

size_t sample_workspace_bytes(size_t n, bool greedy) {
  const size_t head = round_up256(kMaxParts * sizeof(ArgPart)) + round_up256(kMaxParts * 4);
  if (greedy) return head;
  return head + 7 * round_up256(n * 4);
}

hipError_t launch_sample_token(uint32_t* token, uint64_t* state, const float* logits, size_t n,
                               float temperature, float top_p, size_t top_k, bool greedy,
                               void* ws, hipStream_t s) {
  SampleArgs a;
  a.logits = logits;
  a.n = (int)n;
  a.greedy_only = greedy ? 1 : 0;
  a.temperature = temperature;
  a.inv_temp = 1.0f / temperature;  // as the reference: 1.0 / temperature in f32
  a.top_p = top_p;
  a.top_k = top_k > 0x7FFFFFFFull ? 0x7FFFFFFF : (int)top_k;
  a.parts = sample_parts(n);
  a.token = token;
  a.state = state;
  if (greedy && (reinterpret_cast<uintptr_t>(logits) & 3u) == 0) {
    hipLaunchKernelGGL(argmax_one_kernel, dim3(1), dim3(kST), 0, s, logits, (int)n, token);
    return hipGetLastError();
  }
  uint8_t* w = static_cast<uint8_t*>(ws);
  const size_t parts_b = round_up256(kMaxParts * sizeof(ArgPart));
  const size_t plane = round_up256(n * 4);
  a.part = reinterpret_cast<ArgPart*>(w);
  a.seg_cnt = reinterpret_cast<int*>(w + parts_b);
  uint8_t* q = greedy ? nullptr : w + parts_b + round_up256(kMaxParts * 4);
  auto pl = [&](int i) { return q ? q + (size_t)i * plane : nullptr; };
  a.probs = reinterpret_cast<float*>(pl(0));
  a.seg_idx = reinterpret_cast<uint32_t*>(pl(1));
  a.seg_val = reinterpret_cast<float*>(pl(2));
  a.a_idx = reinterpret_cast<uint32_t*>(pl(3));
  a.a_val = reinterpret_cast<float*>(pl(4));
  a.k0 = reinterpret_cast<uint32_t*>(pl(5));
  a.k1 = reinterpret_cast<uint32_t*>(pl(6));
  // planes 1-3 (contiguous, 12 n bytes), unused without top-k, hold the
  // ranges' bin masses: parts * kBins1 * 8 <= (n / kPartElems + 1) * 16 KB,
  // within 12 n bytes whenever the bins are used (n > kChunk)
  a.range_mass = reinterpret_cast<double*>(pl(1));
  hipLaunchKernelGGL(sample_parts_kernel, dim3(a.parts), dim3(kST), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(sample_token_kernel, dim3(1), dim3(kST), 0, s, a);
  return hipGetLastError();
}

}  // namespace hypno
