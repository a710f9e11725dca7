// The steps either side of the decode path that read or write whole rows of
// a weight table or of the logits:
//
//  * embedding gather (transformer.rs:476-497, turbo.rs:38-66, with
//    q4_0_extract_row quant.rs:139-153 and q8_0_extract_row quant.rs:158-175):
//    out[t][0..hd) = row ids[t] of an FP32 / FP16 / Q8_0 / Q4_0 table,
//    dequantised bit-exactly, one work-group per token;
//  * next-token choice from the lm_head's logits: greedy argmax and
//    sample_token (run.rs:203-251) with its XorShift64 generator
//    (run.rs:267-278), in one single-work-group kernel.
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
// Here: the k-th largest p comes from a three-level radix select (11 + 11 +
// 10 bits of an order-preserving key, LDS histograms); the p left non-zero
// are compacted in index order (wave ballots) -- zeros add nothing to the
// running sums, so walking only the non-zero p gives the reference's fp32
// sums bit for bit; the top-p walk sorts them with a stable LSD radix sort
// (four 8-bit passes, wave-ballot ranks); the running sums are one lane's
// sequential fp32 additions and IEEE divisions, exactly the reference's.
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
    const bool ok = (id + 1) * hd <= a.table_len / esz;
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
  const bool ok = (id + 1) * bpr * bb <= a.table_len;
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

constexpr int kST = 1024;  // threads of the sampling work-group
constexpr int kSW = kST / 64;

// Order-preserving map of fp32 bit patterns to u32 (ascending key = ascending
// value, -0 just below +0) and back.
__device__ __forceinline__ uint32_t fkey(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float funkey(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

struct SampleArgs {
  const float* logits;
  int n;
  int greedy_only;  // argmax of the logits, nothing else
  float temperature, inv_temp, top_p;
  int top_k;
  uint32_t* token;
  uint64_t* state;
  // workspace, n entries each
  float* probs;
  uint32_t* a_idx;
  float* a_val;
  uint32_t* k0;
  uint32_t* k1;
};

constexpr int kChunk = 8192;  // floats of a sequential pass staged in LDS at a time

struct SampleShared {
  float chunk[kChunk];
  uint32_t hist[2048];
  uint32_t cnt[kSW][256];
  uint32_t base[256];
  uint32_t tot[256];
  uint32_t wsum[kSW];
  float fred[kSW];
  int ired[kSW];
  uint32_t u[4];
  float f[4];
};

// In the histogram hist[0..nbins), bins counted from the top: the bin holding
// the kk-th largest element (1-based) and kk within that bin.  nbins <= 2048.
__device__ void select_from_top(SampleShared& sh, int nbins, uint32_t kk, uint32_t* bin,
                                uint32_t* kin) {
  const int t = threadIdx.x;
  // thread t owns bins nbins-1-2t (higher) and nbins-2-2t
  const int b0 = nbins - 1 - 2 * t, b1 = b0 - 1;
  const uint32_t c0 = b0 >= 0 ? sh.hist[b0] : 0u, c1 = b1 >= 0 ? sh.hist[b1] : 0u;
  uint32_t s = c0 + c1;
  // inclusive scan over threads in order t = 0, 1, ... (wave, then waves)
  const int lane = t & 63;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t o = (uint32_t)__shfl_up((int)s, off, 64);
    if (lane >= off) s += o;
  }
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

// Iterator::max_by(partial_cmp) over v(0..n): the last of equal maxima after
// the last NaN (or that NaN if it is the last element); n == 0 gives 0.
template <typename V>
__device__ uint32_t argmax_fold(int n, V v, SampleShared& sh) {
  const int t = threadIdx.x;
  int ln = -1;  // last NaN
  for (int i = t; i < n; i += kST)
    if (__builtin_isnan(v(i))) ln = i;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ln = max(ln, __shfl_xor(ln, off, 64));
  __syncthreads();
  if ((t & 63) == 0) sh.ired[t >> 6] = ln;
  __syncthreads();
  ln = -1;
  for (int w = 0; w < kSW; w++) ln = max(ln, sh.ired[w]);
  if (n == 0) return 0u;
  if (ln == n - 1) return (uint32_t)ln;
  float bv = 0.0f;
  int bi = -1;
  for (int i = ln + 1 + t; i < n; i += kST) {
    const float x = v(i);
    if (bi < 0 || x >= bv) {  // ties: the later index (i grows per thread)
      bv = x;
      bi = i;
    }
  }
  // combine (value, index): larger value, then larger index
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(bv, off, 64);
    const int oi = __shfl_xor(bi, off, 64);
    if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi > bi))) {
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
  for (int w = 0; w < kSW; w++) {
    const float ov = sh.fred[w];
    const int oi = sh.ired[w];
    if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi > bi))) {
      bv = ov;
      bi = oi;
    }
  }
  __syncthreads();
  return (uint32_t)bi;
}

// Compact the elements i in [0, n) with val(i) != 0 (NaN counts) into
// (idx[], v[]) in index order; returns their count.
template <typename V>
__device__ int compact_nonzero(int n, V val, uint32_t* idx, float* v, SampleShared& sh) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const uint64_t lt = (1ull << lane) - 1ull;
  int L = 0;
  for (int b0 = 0; b0 < n; b0 += kST) {
    const int i = b0 + t;
    const float x = i < n ? val(i) : 0.0f;
    const bool nz = i < n && x != 0.0f;
    const uint64_t m = __ballot(nz);
    if (lane == 0) sh.wsum[wave] = (uint32_t)__popcll(m);
    __syncthreads();
    int off = L, tot = 0;
    for (int w = 0; w < kSW; w++) {
      const int c = (int)sh.wsum[w];
      if (w < wave) off += c;
      tot += c;
    }
    if (nz) {
      const int d = off + __popcll(m & lt);
      idx[d] = (uint32_t)i;
      v[d] = x;
    }
    L += tot;
    __syncthreads();
  }
  return L;
}

// Stable LSD radix sort of keys k0[0..L) ascending (four 8-bit passes through
// k1; the result is back in k0).  Ranks within a wave come from ballots over
// the digit's bits, across waves from per-digit counts in LDS.
__device__ void radix_sort_keys(uint32_t* k0, uint32_t* k1, int L, SampleShared& sh) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const uint64_t lt = (1ull << lane) - 1ull;
  if (L <= 1) return;
  for (int pass = 0; pass < 4; pass++) {
    const int sh_bits = 8 * pass;
    uint32_t* src = (pass & 1) ? k1 : k0;
    uint32_t* dst = (pass & 1) ? k0 : k1;
    if (t < 256) sh.hist[t] = 0;
    __syncthreads();
    for (int i = t; i < L; i += kST) atomicAdd(&sh.hist[(src[i] >> sh_bits) & 255u], 1u);
    __syncthreads();
    if (t == 0) {
      uint32_t run = 0;
      for (int d = 0; d < 256; d++) {
        sh.base[d] = run;
        run += sh.hist[d];
      }
    }
    __syncthreads();
    for (int b0 = 0; b0 < L; b0 += kST) {
      const int i = b0 + t;
      const bool valid = i < L;
      const uint32_t key = valid ? src[i] : 0u;
      const uint32_t d = (key >> sh_bits) & 255u;
      uint64_t m = __ballot(valid);
#pragma unroll
      for (int b = 0; b < 8; b++) {
        const uint64_t bb = __ballot((d >> b) & 1u);
        m &= ((d >> b) & 1u) ? bb : ~bb;
      }
      const int rank = __popcll(m & lt);
      for (int e = t; e < kSW * 256; e += kST) (&sh.cnt[0][0])[e] = 0;
      __syncthreads();
      if (valid && rank == 0) sh.cnt[wave][d] = (uint32_t)__popcll(m);
      __syncthreads();
      if (t < 256) {
        uint32_t run = 0;
        for (int w = 0; w < kSW; w++) {
          const uint32_t c = sh.cnt[w][t];
          sh.cnt[w][t] = run;
          run += c;
        }
        sh.tot[t] = run;
      }
      __syncthreads();
      if (valid) dst[sh.base[d] + sh.cnt[wave][d] + rank] = key;
      __syncthreads();
      if (t < 256) sh.base[t] += sh.tot[t];
      __syncthreads();
    }
  }
}

// One thread's in-order pass over x(0..cnt) (the reference's sequential fp32
// loops), the work-group staging kChunk values at a time in LDS: f(j, x_j)
// for j = 0, 1, ... until it returns true.  Returns that j, or -1.
template <typename X, typename F>
__device__ int seq_walk(int cnt, X x, F f, SampleShared& sh) {
  const int t = threadIdx.x;
  for (int b0 = 0; b0 < cnt; b0 += kChunk) {
    const int len = min(kChunk, cnt - b0);
    for (int j = t; j < len; j += kST) sh.chunk[j] = x(b0 + j);
    __syncthreads();
    if (t == 0) {
      int hit = -1;
      int j = 0;
      for (; j + 4 <= len; j += 4) {  // 16-byte LDS reads, in order
        const float4 q = *reinterpret_cast<const float4*>(&sh.chunk[j]);
        if (f(b0 + j, q.x)) { hit = b0 + j; break; }
        if (f(b0 + j + 1, q.y)) { hit = b0 + j + 1; break; }
        if (f(b0 + j + 2, q.z)) { hit = b0 + j + 2; break; }
        if (f(b0 + j + 3, q.w)) { hit = b0 + j + 3; break; }
      }
      if (hit < 0)
        for (; j < len; j++)
          if (f(b0 + j, sh.chunk[j])) { hit = b0 + j; break; }
      sh.ired[0] = hit;
    }
    __syncthreads();
    const int hit = sh.ired[0];
    __syncthreads();
    if (hit >= 0) return hit;
  }
  return -1;
}

__global__ void __launch_bounds__(kST) sample_token_kernel(const SampleArgs a) {
  __shared__ SampleShared sh;
  const int t = threadIdx.x;
  const int n = a.n;
  if (a.greedy_only) {
    const uint32_t am = argmax_fold(n, [&](int i) { return a.logits[i]; }, sh);
    if (t == 0) *a.token = am;
    return;
  }
  const bool use_k = a.top_k > 0 && a.top_k < n;
  const bool scale = a.temperature > 0.0f;

  // p_i, and the level-1 histogram of their keys for top-k
  if (use_k)
    for (int i = t; i < 2048; i += kST) sh.hist[i] = 0;
  __syncthreads();
  for (int i = t; i < n; i += kST) {
    const float l = a.logits[i];
    const float p = scale ? (float)exp((double)(l * a.inv_temp)) : l;
    a.probs[i] = p;
    if (use_k) atomicAdd(&sh.hist[fkey(p) >> 21], 1u);
  }
  __syncthreads();
  // top_k: the k-th largest p by radix select (11, 11, 10 bits of its key)
  float thr_k = -__builtin_inff();  // p < thr_k -> 0 (nothing when -inf)
  if (use_k) {
    uint32_t b1, b2, b3, kk;
    select_from_top(sh, 2048, (uint32_t)a.top_k, &b1, &kk);
    for (int i = t; i < 2048; i += kST) sh.hist[i] = 0;
    __syncthreads();
    for (int i = t; i < n; i += kST) {
      const uint32_t k = fkey(a.probs[i]);
      if ((k >> 21) == b1) atomicAdd(&sh.hist[(k >> 10) & 2047u], 1u);
    }
    __syncthreads();
    select_from_top(sh, 2048, kk, &b2, &kk);
    for (int i = t; i < 1024; i += kST) sh.hist[i] = 0;
    __syncthreads();
    const uint32_t pre = (b1 << 11) | b2;
    for (int i = t; i < n; i += kST) {
      const uint32_t k = fkey(a.probs[i]);
      if ((k >> 10) == pre) atomicAdd(&sh.hist[k & 1023u], 1u);
    }
    __syncthreads();
    select_from_top(sh, 1024, kk, &b3, &kk);
    thr_k = funkey((pre << 10) | b3);
  }
  auto eff1 = [&](int i) {
    const float p = a.probs[i];
    return p < thr_k ? 0.0f : p;
  };
  // the non-zero p in index order (zeros add nothing to the running sums)
  const int L = compact_nonzero(n, eff1, a.a_idx, a.a_val, sh);
  // fp32 sum in index order (thread 0 keeps it; the others only need the
  // branch outcomes, which are shared through LDS)
  auto seq_sum = [&](const float* v, int cnt) {
    float s = -0.0f;
    seq_walk(cnt, [&](int j) { return v[j]; }, [&](int, float x) { s += x; return false; }, sh);
    if (threadIdx.x == 0) sh.f[0] = s;
    __syncthreads();
    const float r = sh.f[0];
    __syncthreads();
    return r;
  };
  // top_p: walk the p in descending order (sorted keys, zeros skipped)
  float thr_p = -__builtin_inff();
  int Lb = L;
  const float* bval = a.a_val;
  const uint32_t* bidx = a.a_idx;
  if (a.top_p < 1.0f) {
    const float sum1 = seq_sum(a.a_val, L);
    if (sum1 > 0.0f) {
      for (int j = t; j < L; j += kST) a.k0[j] = ~fkey(a.a_val[j]);  // descending
      __syncthreads();
      radix_sort_keys(a.k0, a.k1, L, sh);
      float cum = 0.0f;
      const int at = seq_walk(
          L, [&](int j) { return funkey(~a.k0[j]); },
          [&](int, float p) {
            cum += p / sum1;
            return cum > a.top_p;
          },
          sh);
      thr_p = at >= 0 ? funkey(~a.k0[at]) : 3.40282347e+38f;
      // p < thr_p -> 0: keep the survivors of the index-ordered list, in
      // order (k0 / k1 reused as the second list's storage)
      uint32_t* b_idx = a.k1;
      float* b_val = reinterpret_cast<float*>(a.k0);
      const uint32_t* ai = a.a_idx;
      const float* av = a.a_val;
      __syncthreads();
      Lb = compact_nonzero(L, [&](int j) { return av[j] < thr_p ? 0.0f : av[j]; }, b_idx, b_val,
                           sh);
      // compact_nonzero stored list positions; map them to token indices
      for (int j = t; j < Lb; j += kST) b_idx[j] = ai[b_idx[j]];
      __syncthreads();
      bval = b_val;
      bidx = b_idx;
    }
  }
  const float sum2 = seq_sum(bval, Lb);
  if (sum2 <= 0.0f) {
    const uint32_t am = argmax_fold(n, [&](int i) { return a.logits[i]; }, sh);
    if (t == 0) *a.token = am;
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
  float cum = 0.0f;
  const int at = seq_walk(
      Lb, [&](int j) { return bval[j]; },
      [&](int, float p) {
        cum += p / sum2;
        return r < cum;
      },
      sh);
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

size_t sample_workspace_bytes(size_t n) { return 5 * ((n * 4 + 255) / 256 * 256) + 256; }

hipError_t launch_sample_token(uint32_t* token, uint64_t* state, const float* logits, size_t n,
                               float temperature, float top_p, size_t top_k, void* ws,
                               hipStream_t s) {
  SampleArgs a;
  a.logits = logits;
  a.n = (int)n;
  a.greedy_only = ws == nullptr;
  a.temperature = temperature;
  a.inv_temp = 1.0f / temperature;  // as the reference: 1.0 / temperature in f32
  a.top_p = top_p;
  a.top_k = top_k > 0x7FFFFFFFull ? 0x7FFFFFFF : (int)top_k;
  a.token = token;
  a.state = state;
  const size_t plane = (n * 4 + 255) / 256 * 256;
  uint8_t* w = static_cast<uint8_t*>(ws);
  a.probs = reinterpret_cast<float*>(w);
  a.a_idx = reinterpret_cast<uint32_t*>(w ? w + plane : nullptr);
  a.a_val = reinterpret_cast<float*>(w ? w + 2 * plane : nullptr);
  a.k0 = reinterpret_cast<uint32_t*>(w ? w + 3 * plane : nullptr);
  a.k1 = reinterpret_cast<uint32_t*>(w ? w + 4 * plane : nullptr);
  hipLaunchKernelGGL(sample_token_kernel, dim3(1), dim3(kST), 0, s, a);
  return hipGetLastError();
}

}  // namespace hypno
