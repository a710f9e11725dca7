// Shared device helpers and internal launcher declarations for the gfx950
// Q4_0 / FP16 matmul library.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <string>

namespace hypno {

// Native 4 x u32 vector: loads and stores of it are single instructions
// (HIP's uint4 struct copies lower to memcpy and can keep values in scratch).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));

// Load through the global address space (global_load_*, counted by vmcnt only;
// a generic pointer would give flat_load_*, which also holds lgkmcnt).  The
// address-space cast exists only in the device pass; the host pass never
// runs kernel bodies.
template <typename T>
__device__ __forceinline__ T load_global(const void* p) {
#if defined(__HIP_DEVICE_COMPILE__)
  return *reinterpret_cast<const __attribute__((address_space(1))) T*>(
      reinterpret_cast<uintptr_t>(p));
#else
  return *reinterpret_cast<const T*>(p);
#endif
}

// Streaming load (global_load_* nt): data read once, kept out of the caches'
// normal replacement; plain streaming reads of HBM run ~10% faster this way.
template <typename T>
__device__ __forceinline__ T load_global_nt(const void* p) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_nontemporal_load(reinterpret_cast<const __attribute__((address_space(1))) T*>(
      reinterpret_cast<uintptr_t>(p)));
#else
  return *reinterpret_cast<const T*>(p);
#endif
}

// Load of read-only, work-group-uniform data through the constant address
// space (scalar s_load_* when the address is uniform).
template <typename T>
__device__ __forceinline__ T load_const(const void* p) {
#if defined(__HIP_DEVICE_COMPILE__)
  return *reinterpret_cast<const __attribute__((address_space(4))) T*>(
      reinterpret_cast<uintptr_t>(p));
#else
  return *reinterpret_cast<const T*>(p);
#endif
}

constexpr int kBlockElems = 32;  // Q4_0 block: 32 weights (dtype.rs:40-45)
constexpr int kBlockBytes = 18;  // fp16 scale + 16 packed bytes (dtype.rs:48-54)
constexpr int kQ8BlockBytes = 34;  // Q8_0: fp16 scale + 32 bytes q + 128 (dtype.rs:50)

// f16 bits -> f32, exact (v_cvt_f32_f16).
__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits) {
  _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)bits);
  return (float)h;
}

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// (a & b) | c in one v_and_or_b32 (the compiler emits two ops when b and c
// are both literals).  VOP3 reads at most one SGPR here, so the mask b sits
// in a VGPR and c in an SGPR.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t b, uint32_t c) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "s"(c));
  return r;
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
  const uint32_t p0 = and_or(q, 0x000F000Fu, 0x64006400u);   // e0, e4
  const uint32_t p1 = and_or(q, 0x00F000F0u, 0x64006400u);   // e1, e5 (x16)
  const uint32_t p2 = and_or(q8, 0x000F000Fu, 0x64006400u);  // e2, e6
  const uint32_t p3 = and_or(q8, 0x00F000F0u, 0x64006400u);  // e3, e7 (x16)
  u32x4 r;
  r[0] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, p0) + lo_off);
  r[1] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(
                                          __builtin_bit_cast(half2v, p1), hi_mul, hi_off));
  r[2] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, p2) + lo_off);
  r[3] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(
                                          __builtin_bit_cast(half2v, p3), hi_mul, hi_off));
  return r;
}

// Row r of X fp32 [M][K] -> row r of Xh fp16 [Mp][K], scaled by 2^sh with sh
// chosen so that the row's largest |x| times 2^sh lies in [2^14, 2^15) (sh =
// 0 for an all-zero row or one holding inf or NaN), and xexp[r] = -sh: the
// consumer multiplies output row r by 2^xexp[r] (exact), so no token
// overflows fp16 or sinks into fp16 subnormals because of its magnitude.
// (Scaling by a power of two leaves the rounding of normal values unchanged.)
// Rows M..Mp-1 are zero.  Called by a whole 256-thread work-group per row;
// with kPermute each group of 8 columns goes in the Q4_0 nibble-unpack
// order e0,e4,e1,e5,e2,e6,e3,e7.  K % 8 == 0.
template <bool kPermute>
__device__ __forceinline__ void x_row_to_f16(u32x4* __restrict__ xh, int* __restrict__ xexp,
                                             const float* __restrict__ x, int M, int K, int r) {
  __shared__ uint32_t red[4];
  const int t = threadIdx.x;
  const int groups = K / 8;
  u32x4* dst = xh + (size_t)r * groups;
  if (r >= M) {
    for (int g = t; g < groups; g += 256) dst[g] = u32x4{0u, 0u, 0u, 0u};
    if (t == 0) xexp[r] = 0;
    return;
  }
  const float* src = x + (size_t)r * K;
  const bool al = ((uintptr_t)src & 15) == 0;
  auto load8 = [&](int g, float (&v)[8]) {
    const float* p = src + (size_t)g * 8;
    if (al) {
      const float4 a = load_global<float4>(p);
      const float4 b = load_global<float4>(p + 4);
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
      v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
      for (int i = 0; i < 8; i++) v[i] = p[i];
    }
  };
  uint32_t mb = 0;  // largest |x| by bit pattern (inf and NaN above every finite value)
  for (int g = t; g < groups; g += 256) {
    float v[8];
    load8(g, v);
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
  constexpr int perm_q4[8] = {0, 4, 1, 5, 2, 6, 3, 7};
  for (int g = t; g < groups; g += 256) {
    float v[8];
    load8(g, v);
    u32x4 packed;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int a = kPermute ? perm_q4[2 * j] : 2 * j;
      const int b = kPermute ? perm_q4[2 * j + 1] : 2 * j + 1;
      const uint32_t lo = __builtin_bit_cast(uint16_t, (_Float16)ldexpf(v[a], sh));
      const uint32_t hi = __builtin_bit_cast(uint16_t, (_Float16)ldexpf(v[b], sh));
      packed[j] = lo | (hi << 16);
    }
    dst[g] = packed;
  }
  if (t == 0) xexp[r] = -sh;
}

// Wave-wide sum (wave64) with xor butterflies; every lane gets the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Sum over aligned groups of 8 lanes with DPP row shifts (VALU only, no LDS):
// lane 8g+7 returns the sum of lanes 8g..8g+7 (other lanes: partial sums).
__device__ __forceinline__ float group8_sum(float v) {
  v += __builtin_amdgcn_update_dpp(0.0f, v, 0x111, 0xF, 0xF, true);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0.0f, v, 0x112, 0xF, 0xF, true);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0.0f, v, 0x114, 0xF, 0xF, true);  // row_shr:4
  return v;
}

// Dot product of 8 nibbles of one packed dword with 8 activations:
// byte i of `dw` holds element 2i (low nibble) and 2i+1 (high nibble);
// returns sum_j nib_j * x_j (nibbles in 0..15, the -8 offset is applied by
// the caller through the block's activation sum).
__device__ __forceinline__ float dot8_nib(uint32_t dw, const float* x) {
  uint32_t lo = dw & 0x0F0F0F0Fu;
  uint32_t hi = (dw >> 4) & 0x0F0F0F0Fu;
  // Opaque to the optimiser: otherwise it folds the byte masks into 4-bit
  // field extracts and loses v_cvt_f32_ubyte{1,2,3} (one op per nibble).
  asm volatile("" : "+v"(lo), "+v"(hi));
  float a = (float)(lo & 0xFFu) * x[0];
  a = fmaf((float)(hi & 0xFFu), x[1], a);
  a = fmaf((float)((lo >> 8) & 0xFFu), x[2], a);
  a = fmaf((float)((hi >> 8) & 0xFFu), x[3], a);
  a = fmaf((float)((lo >> 16) & 0xFFu), x[4], a);
  a = fmaf((float)((hi >> 16) & 0xFFu), x[5], a);
  a = fmaf((float)(lo >> 24), x[6], a);
  a = fmaf((float)(hi >> 24), x[7], a);
  return a;
}

// Launchers (all asynchronous on `stream`; return hipSuccess or the launch error).
hipError_t launch_quantize_q4_0(uint8_t* out, const float* src, size_t n_blocks, hipStream_t s);
hipError_t launch_dequantize_q4_0(float* out, const uint8_t* q, size_t n_blocks, hipStream_t s);

// Any shape / alignment / short buffer; one wave per (token, row).
hipError_t launch_q4_0_generic(float* y, const uint8_t* w, size_t w_len, const float* x,
                               const float* bias, size_t n, size_t m, size_t batch,
                               hipStream_t s);
// Streaming decode GEMV for one token.  Requires m % 256 == 0 (m <= 15360),
// lcm(m/64, 64) <= 1024, w 16-byte aligned, x 16-byte aligned,
// w_len >= n*m/32*18.
bool q4_0_gemv_fast_ok(const uint8_t* w, size_t w_len, size_t n, size_t m);
hipError_t launch_q4_0_gemv_fast(float* y, const uint8_t* w, const float* x, const float* bias,
                                 size_t n, size_t m, int num_cus, hipStream_t s);
// Q8_0 codec (codec.hip) and any-shape GEMV (gemv_q4_0.hip; requires the
// buffer to hold all n*m elements, as matmul_f32 does).
hipError_t launch_quantize_q8_0(uint8_t* out, const float* src, size_t n_blocks, hipStream_t s);
hipError_t launch_dequantize_q8_0(float* out, const uint8_t* q, size_t n_blocks, hipStream_t s);
hipError_t launch_q8_0_generic(float* y, const uint8_t* w, const float* x, const float* bias,
                               size_t n, size_t m, size_t batch, hipStream_t s);
// Q8_0 prefill through fp16 weights and the fp16 GEMM (gemm_q8_0.hip).
bool q8_0_gemm_ok(size_t n, size_t m, size_t batch);
size_t q8_0_gemm_workspace_bytes(size_t batch, size_t n, size_t m, int num_cus);
hipError_t launch_q8_0_gemm(float* y, const uint8_t* w, const float* x, const float* bias,
                            size_t n, size_t m, size_t batch, void* ws, int num_cus,
                            hipStream_t s);
// Q8_0 (34-byte blocks), same conditions with w_len >= n*m/32*34.
bool q8_0_gemv_fast_ok(const uint8_t* w, size_t w_len, size_t n, size_t m);
hipError_t launch_q8_0_gemv_fast(float* y, const uint8_t* w, const float* x, const float* bias,
                                 size_t n, size_t m, int num_cus, hipStream_t s);

// Step applied to a job's input vector while it is staged (values of
// HYPNO_HIP_PROLOGUE_* in include/hypno_hip.h).
constexpr int kProNone = 0;
constexpr int kProRmsNorm = 1;  // x * (1 / sqrt(mean(x^2) + eps)) * aux
constexpr int kProSiluMul = 2;  // x / (1 + exp(-x)) * aux

// One GEMV of a multi-job launch (device-side descriptor).
struct GemvJob {
  const uint8_t* w;
  const float* x;
  float* y;
  const float* bias;
  const float* aux;  // prologue operand (norm weight or up), [m]
  int n;      // rows
  int B;      // blocks per row = m / 32
  int rps;    // rows per step = T / B
  int step0;  // first global step of this job
  int pro;    // kPro*
  float eps;  // kProRmsNorm
};

// Weight block formats of the streaming GEMV.
constexpr int kFmtQ4_0 = 0;
constexpr int kFmtQ8_0 = 1;

// Work-group shape shared by the jobs of one launch.
struct GemvGroupGeom {
  int fmt = kFmtQ4_0;
  int Tbase = 0; // lcm over jobs of lcm(B, 64)
  int T = 0;     // threads: Tbase doubled up to at least 256 (when it fits)
  int W = 0;     // waves
  int S = 0;     // steps per partial-sum chunk
  int maxB = 0;  // largest B (activation staging size)
  int pro = 0;   // some job stages a prologue operand too
  int ring = 0;  // weight steps in flight per wave (LDS ring depth)
  int rows = 1;  // x rows per pass (the few-row kernels)
  size_t ring_off = 0;  // LDS offset of the weight rings
  size_t lds = 0;
};

// Few-row GEMV (2 <= rows <= kGemvMaxRows, Q4_0 or Q8_0): the streaming
// kernel with every weight block multiplied by `rows` consecutive x rows (K
// floats apart) in one pass; y rows n floats apart.  Work-groups of at most
// 512 threads.
constexpr int kGemvMaxRows = 4;  // Q4_0 rows per launch (then few-token MFMA)
// Q8_0 rows per launch: eight rows' digit planes fill 256 VGPRs; measured
// against launches of at most four (µs per call, 14336 x 4096): 5 tokens
// 27.4 against 33.8, 8 tokens 38.5 against 42.4, 15 tokens 70.7 against 79.6.
constexpr int kQ8GemvMaxRows = 8;
bool q4_0_gemv_rows_ok(const uint8_t* w, size_t w_len, size_t n, size_t m, size_t rows);
hipError_t launch_q4_0_gemv_rows(float* y, const uint8_t* w, const float* x, const float* bias,
                                 size_t n, size_t m, int rows, int num_cus, hipStream_t s);
bool q8_0_gemv_rows_ok(const uint8_t* w, size_t w_len, size_t n, size_t m, size_t rows);
hipError_t launch_q8_0_gemv_rows(float* y, const uint8_t* w, const float* x, const float* bias,
                                 size_t n, size_t m, int rows, int num_cus, hipStream_t s);

// A launch that the staging rule holds to at most one work-group per CU
// gets wider work-groups (more waves per CU streaming and computing): the
// largest T (a multiple of Tbase, up to 1024) that still gives every CU a
// step.  Jobs (n rows, B blocks per row) must take their rps / step0 after.
void gemv_group_widen(GemvGroupGeom& g, const int* n, const int* B, int count, int num_cus);

constexpr int kGemvInline = 4;  // jobs a launch carries in its arguments

// The job count, step count and ring offset travel in the preloaded scalar
// arguments ahead of this struct, not in it.
struct GemvLaunch {
  const GemvJob* jobs;           // device table when njobs > kGemvInline
  GemvJob inl[kGemvInline];      // the jobs when njobs <= kGemvInline
  int S;                         // steps per partial-sum chunk, per x row
};

// Adds a job with m columns to group g if the shared shape still fits.
bool gemv_group_add(GemvGroupGeom& g, size_t m);
// h_jobs: the first min(njobs, kGemvInline) jobs (host memory); d_jobs: all
// of them in device memory when njobs > kGemvInline.
hipError_t launch_q4_0_gemv_group(const GemvGroupGeom& g, const GemvJob* d_jobs,
                                  const GemvJob* h_jobs, int njobs, int total_steps, int num_cus,
                                  hipStream_t s);

// MFMA prefill GEMM.  Requires m % 64 == 0, w 4-byte aligned, w_len full.
// `xh` is a device workspace of gemm_q4_0_workspace_bytes(batch, m) bytes.
bool q4_0_gemm_ok(const uint8_t* w, size_t w_len, size_t n, size_t m, size_t batch);
// Bytes of the fp16 activation copy [round_up(batch, 128)][m] followed by its
// per-row exponents (x_row_to_f16), which gemm_x_exponents locates.
size_t gemm_workspace_bytes(size_t batch, size_t m);
int* gemm_x_exponents(void* ws, size_t batch, size_t m);
hipError_t launch_q4_0_gemm(float* y, const uint8_t* w, const float* x, const float* bias,
                            size_t n, size_t m, size_t batch, void* workspace, int num_cus,
                            hipStream_t s);

// X fp32 [batch][m] -> fp16 [round_up(batch,128)][m] workspace (zero pad
// rows, each row scaled by its power of two, exponents after the rows), each
// group of 8 columns permuted to the Q4_0 nibble-unpack order.
hipError_t launch_x_f16_permuted(const float* x, size_t batch, size_t m, void* ws,
                                 hipStream_t s);

// MFMA prefill GEMM, 512-thread 128x128 tiles with K-groups (gemm_q4.hip),
// weights rounded to fp16 after a per-row power-of-two normalisation.
// Requires m % 256 == 0, w 16-byte aligned, w_len full.
bool q4_0_gemm_v3_ok(const uint8_t* w, size_t w_len, size_t n, size_t m, size_t batch);
// Workspace of launch_q4_0_gemm_v3: the fp16 activations, the K-split
// partial planes when the tile grid is too small for the chip, the per-row
// scale exponents.
size_t gemm_v3_workspace_bytes(size_t batch, size_t n, size_t m, int num_cus);
hipError_t launch_q4_0_gemm_v3(float* y, const uint8_t* w, const float* x, const float* bias,
                               size_t n, size_t m, size_t batch, void* workspace, int num_cus,
                               hipStream_t s);

// MFMA prefill GEMM in the exact-nibble arithmetic (gemm_exact.hip): the
// integer nibbles as fp16 into the matrix cores, each block's partial sum
// scaled by its fp32 scale.  Requires m % 256 == 0, w 4-byte aligned, w_len
// full, W and the fp16 X under 4 GB.
bool q4_0_gemm_exact_ok(const uint8_t* w, size_t w_len, size_t n, size_t m, size_t batch);
size_t q4_0_gemm_exact_workspace_bytes(size_t batch, size_t n, size_t m, int num_cus);
hipError_t launch_q4_0_gemm_exact(float* y, const uint8_t* w, const float* x, const float* bias,
                                  size_t n, size_t m, size_t batch, void* workspace, int num_cus,
                                  hipStream_t s);

// A few tokens (2 <= batch <= 64): weight-streaming MFMA kernel (skinny_q4.hip).
bool q4_0_skinny_ok(const uint8_t* w, size_t w_len, size_t n, size_t m, size_t batch,
                    int num_cus);
size_t skinny_workspace_bytes(size_t batch, size_t n, size_t m, int num_cus);
hipError_t launch_q4_0_skinny(float* y, const uint8_t* w, const float* x, const float* bias,
                              size_t n, size_t m, size_t batch, void* workspace, int num_cus,
                              hipStream_t s);

// FP16 weights.
hipError_t launch_f16_generic(float* y, const uint8_t* w, const float* x, const float* bias,
                              size_t n, size_t m, size_t batch, hipStream_t s);
bool f16_gemv_fast_ok(const uint8_t* w, size_t n, size_t m);
hipError_t launch_f16_gemv_fast(float* y, const uint8_t* w, const float* x, const float* bias,
                                size_t n, size_t m, int num_cus, hipStream_t s);
// X fp32 [batch][m] -> `rows` (>= batch) fp16 rows at xh, per-row exponents
// at xexp (x_row_to_f16; permuted or natural column order).
hipError_t launch_x_rows_f16(const float* x, size_t batch, size_t rows, size_t m, void* xh,
                            int* xexp, bool permute, hipStream_t s);
// X -> fp16 [Mp][K] in natural column order, rows scaled as above
// (FP16-weight GEMM pre-pass).
hipError_t launch_x_f16_plain(const float* x, size_t batch, size_t m, void* ws, hipStream_t s);
// DMA-fed FP16-weight GEMM (gemm_q4.hip).
bool f16_gemm_v2_ok(const uint8_t* w, size_t n, size_t m, size_t batch);
size_t f16_gemm_v2_workspace_bytes(size_t batch, size_t n, size_t m, int num_cus);
hipError_t launch_f16_gemm_v2(float* y, const uint8_t* w, const float* x, const float* bias,
                              size_t n, size_t m, size_t batch, void* ws, int num_cus,
                              hipStream_t s,
                              const float* colscale = nullptr);
// Register-streaming FP16-weight GEMM for 2..128 tokens (gemm_q4.hip); below
// 16 tokens on hi/lo fp16 rows (fp32-accurate).
bool f16_gemm_stream_ok(const uint8_t* w, const float* x, size_t n, size_t m, size_t batch);
size_t f16_gemm_stream_workspace_bytes(size_t batch, size_t n, size_t m, int num_cus);
hipError_t launch_f16_gemm_stream(float* y, const uint8_t* w, const float* x, const float* bias,
                                  size_t n, size_t m, size_t batch, void* ws, int num_cus,
                                  hipStream_t s, const float* colscale = nullptr);

// Column-major Q4_0 (gemv_col.hip): y[n] = W_col[m][n]^T x[m] (+ bias) for
// `tokens` consecutive x rows (m floats apart) and y rows (n apart) in one
// main and one reduction launch; the workspace holds each token's split
// partial planes (q4_0_col_workspace_bytes per token; 0 bytes: none needed).
size_t q4_0_col_workspace_bytes(size_t n, size_t m, int num_cus);
hipError_t launch_q4_0_col(float* y, const uint8_t* w, size_t w_len, const float* x,
                           const float* bias, size_t n, size_t m, int tokens, void* ws,
                           int num_cus, hipStream_t s);

// Decode-step neighbours of the GEMV (prologue.hip).  rms_norm: `rows` rows
// of n, out may alias x; silu_mul: n elements, out may alias gate.
hipError_t launch_rms_norm(float* out, const float* x, const float* weight, size_t n,
                           size_t rows, float eps, hipStream_t s);
hipError_t launch_silu_mul(float* out, const float* gate, const float* up, size_t n,
                           hipStream_t s);

// Embedding rows (sample.hip): out[t][0..hd) = row ids[t] (or the single
// row id0 when ids is NULL) of an FP32 / FP16 / Q8_0 / Q4_0 table (dtype =
// HYPNO_DTYPE_*); rows outside the table are NaN.
hipError_t launch_embed_rows(float* out, const uint8_t* table, size_t table_len, int dtype,
                             const uint32_t* ids, size_t id0, size_t count, size_t hd,
                             hipStream_t s);
// Next token from n logits (sample.hip): the greedy argmax (greedy), or
// sample_token; two launches, with a workspace of
// sample_workspace_bytes(n, greedy).
size_t sample_workspace_bytes(size_t n, bool greedy);
hipError_t launch_sample_token(uint32_t* token, uint64_t* state, const float* logits, size_t n,
                               float temperature, float top_p, size_t top_k, bool greedy,
                               void* ws, hipStream_t s);

// Status reporting shared by the C ABI sources (api.cpp): record `msg` as the
// calling thread's last error and return `status`; hip_status maps a HIP error
// to ENOMEM / EDEVICE the same way.
int set_last_error(int status, const std::string& msg);
int hip_status(hipError_t e, const char* what);

// True when the caller asked for the exact-nibble GEMM arithmetic
// (hypno_hip_set_gemm_numerics(HYPNO_HIP_GEMM_EXACT)).
bool gemm_folded();

// Raises `kernel`'s dynamic-LDS limit to `bytes` on the current device, once
// per (kernel, device); safe to call from several threads (api.cpp).
hipError_t set_lds_limit(const void* kernel, int bytes);

}  // namespace hypno
