/*
 * hypno_hip.h — C ABI of the MI355X (gfx950) Q4_0 / FP16 matmul library.
 *
 * Drop-in for hypno's quantized matmul path.  Paths in citations are relative
 * to the hypno repository (crates/hypno/src/...).
 *
 * Conventions shared by every entry point:
 *   - Rows are the flattened ranges [r*m, (r+1)*m) of the row-major weight
 *     tensor, quantised in consecutive 32-element blocks (sft_convert.rs:261,
 *     quant.rs:108).  A Q4_0 block is 18 bytes: fp16 scale d (little-endian)
 *     then 16 bytes; byte i holds element 2i in its low nibble and element
 *     2i+1 in its high nibble; weight = (nibble - 8) * d (quant.rs:10-34).
 *     m need not be a multiple of 32: blocks then straddle rows
 *     (kernels.rs:362-400).
 *   - A weight buffer shorter than the tensor is not an error: a block whose
 *     18 bytes lie past w_len contributes nothing (kernels.rs:275-277, :374).
 *   - y is fully overwritten; bias may be NULL (kernels.rs:356).  y may not
 *     share memory with any input (EINVAL; Rust's &mut y rules it out too).
 *   - Arithmetic by path (M = tokens):
 *       Q4_0, M = 1, m % 256 == 0 (the streaming decode GEMV): each block of
 *         32 activations becomes exact integers of 19 significant bits
 *         relative to the block's largest |x| (rounding <= 2^-18 of that
 *         value), products with the nibbles are exact in int32, each block's
 *         sum is scaled by d in fp32 and blocks accumulate in fp32.  Other
 *         shapes: fp32 FMAs.  Bar: max|y - r| / max|r| <= 1e-4.
 *       Q4_0, M = 2 (M <= 4 when n * m <= 16M),
 *         m % 256 == 0: the
 *         streaming GEMV with every block multiplied by each token's row, in
 *         its arithmetic above (each token's y bit-identical to its M = 1
 *         result).  Otherwise M = 2..16: fp16 hi/lo activation pairs per
 *         256-column stage (to ~2^-22), exact nibble products on MFMA, fp32
 *         block scale; the same 1e-4 bar per token.
 *       Q4_0, M = 17..64, and M >= 65 (prefill GEMM): activations rounded to
 *         fp16 after a power-of-two scale per token (undone exactly on the
 *         output), fp32 accumulation on MFMA.  Weights: the exact integer
 *         nibbles (fp16 -8..7), each block's d applied to its partial sum in
 *         fp32.  Only under hypno_hip_set_gemm_numerics(HYPNO_HIP_GEMM_FOLDED)
 *         do the M >= 65 GEMMs from 256 tokens (from 128 when W is at most
 *         64 MB) instead feed each weight as fp16 (nibble - 8) * d / 2^E_n
 *         (one rounding, relative 2^-11; 2^E_n just above row n's largest
 *         |d|), faster on the largest shapes.  Bar:
 *         ||Y - R||_2 / ||R||_2 <= 2e-3.
 *       FP16: M = 1 fp32 FMAs; M = 2..15 each token as two fp16 rows, hi and
 *         lo (x 2^s = hi + lo to ~2^-22), on MFMA against the fp16 weights
 *         with fp32 accumulation (the 1e-4 bar per token; fp32 FMAs token by
 *         token if x is not 16-byte aligned); M >= 16 as the Q4_0 GEMM with
 *         fp16 weights.
 *       Q8_0: M < 16 each token's activations as three exact int8 digit
 *         planes per block (to 2^-23), each weight block read once for 2 to 8
 *         tokens; M >= 16 weights expanded once to fp16 (row-normalised,
 *         relative 2^-11) and the FP16 GEMM.
 *   - Every function returns a status (HYPNO_HIP_OK on success) and never
 *     aborts the process.  hypno_hip_last_error() describes the last failure
 *     on the calling thread.
 *   - All functions are thread-safe.  Device-pointer ("_dev") entry points are
 *     asynchronous on the given stream (NULL = the default stream).  Calls
 *     from several threads on one stream are serialised for the span of
 *     their launches (each stream has its own workspace); a call needing a
 *     larger workspace than its stream holds synchronises that stream first,
 *     so make the first call of each size before capturing a HIP graph.
 */
#ifndef HYPNO_HIP_H
#define HYPNO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HYPNO_HIP_ABI_VERSION 1

/* Status codes (errno-like values). */
#define HYPNO_HIP_OK 0
#define HYPNO_HIP_EINVAL 22   /* null pointer, bad shape or length, bad dtype */
#define HYPNO_HIP_ENOMEM 12   /* device or pinned-host allocation failed */
#define HYPNO_HIP_EDEVICE 5   /* HIP runtime / launch error, or no device */
#define HYPNO_HIP_ENOTSUP 95  /* dtype outside this path (FP32) */
#define HYPNO_HIP_ENOENT 2    /* no such file, tensor or metadata key */
#define HYPNO_HIP_EFILE 9     /* a file could not be opened, mapped or read */
#define HYPNO_HIP_EFORMAT 74  /* malformed .hypno file (format.rs:109-131) */

/* Weight dtypes: hypno's DType codes (dtype.rs:4-15). */
#define HYPNO_DTYPE_FP32 0u
#define HYPNO_DTYPE_FP16 1u
#define HYPNO_DTYPE_Q8_0 2u
#define HYPNO_DTYPE_Q4_0 3u

/* ABI version (HYPNO_HIP_ABI_VERSION of the built library). */
int hypno_hip_abi_version(void);

/* Static description of a status code. */
const char* hypno_hip_strerror(int status);

/* Detail of the last failure on the calling thread ("" if none). */
const char* hypno_hip_last_error(void);

/* Number of visible HIP devices (0 when there is none; never fails). */
int hypno_hip_device_count(void);

/* ---------------------------------------------------------------------------
 * Host-slice entry points: same arguments as the reference functions, with
 * the slice lengths the Rust signature carries made explicit.  Inputs are
 * host memory; they are staged to the current device, computed there, and y
 * is copied back before return.  A weight buffer registered with
 * hypno_hip_weight_register() is not uploaded again.
 * ------------------------------------------------------------------------- */

/* Replaces kernels::matmul_q4_0(y, w_q, x, bias, n, m) (kernels.rs:256).
 * y[n], w_q[w_len] (Q4_0 bytes), x[m], bias[n] or NULL. */
int hypno_hip_matmul_q4_0(float* y, const uint8_t* w_q, size_t w_len, const float* x,
                          const float* bias, size_t n, size_t m);

/* Replaces kernels::matmul_f16(y, w, x, bias, n, m) (kernels.rs:571).
 * w holds n*m fp16 values as little-endian bytes; w_len must be >= 2*n*m. */
int hypno_hip_matmul_f16(float* y, const uint8_t* w, size_t w_len, const float* x,
                         const float* bias, size_t n, size_t m);

/* Replaces the Q8_0 arm of ops::matmul_vec_auto (ops.rs:33-36): y = the
 * dequantised rows [r*m, (r+1)*m) of w_q (34-byte blocks: fp16 d, then 32
 * bytes u; weight = (u - 128) * d) times x, fp32 accumulation, + bias.  The
 * buffer must hold all n*m elements (EINVAL otherwise; the reference panics).
 * The reference dequantises the whole tensor to fp32 on every call; this one
 * streams the blocks. */
int hypno_hip_matmul_q8_0(float* y, const uint8_t* w_q, size_t w_len, const float* x,
                          const float* bias, size_t n, size_t m);

/* Replaces ops::matmul_vec_auto(y, w, dtype, x, bias, n, m) (ops.rs:25-38) for
 * FP16, Q4_0 and Q8_0; FP32 returns ENOTSUP. */
int hypno_hip_matmul_vec_auto(float* y, const uint8_t* w, size_t w_len, uint32_t dtype,
                              const float* x, const float* bias, size_t n, size_t m);

/* Replaces turbo::batch_matmul(y, w, dtype, x, n, dim, batch, false)
 * (turbo.rs:306-341) for FP16, Q4_0 and Q8_0: X[batch][dim] -> Y[batch][n] in
 * one device call instead of one GEMV per token.  No bias. */
int hypno_hip_batch_matmul(float* y, const uint8_t* w, size_t w_len, uint32_t dtype,
                           const float* x, size_t n, size_t dim, size_t batch);

/* Replaces kernels::matmul_q4_0_col(y, w_q, x, bias, n, m) (kernels.rs:414-535),
 * the kernel a col_major model uses (loader.rs:166-168): w_q holds W_col[m][n]
 * (for each input index k, n outputs in Q4_0 blocks along n; floor(n/32)
 * blocks per k, outputs past 32*floor(n/32) get only the bias), and
 * y[j] = sum_k W_col[k][j] * x[k] (+ bias).  Blocks past a short buffer
 * contribute nothing.  Fixed summation order (the reference's AVX2 form
 * depends on the thread count). */
int hypno_hip_matmul_q4_0_col(float* y, const uint8_t* w_q, size_t w_len, const float* x,
                              const float* bias, size_t n, size_t m);

/* Replaces ops::matmul_vec_col (ops.rs:41-51): Q4_0 -> the column-major
 * kernel, every other dtype as hypno_hip_matmul_vec_auto. */
int hypno_hip_matmul_vec_col(float* y, const uint8_t* w, size_t w_len, uint32_t dtype,
                             const float* x, const float* bias, size_t n, size_t m);

/* turbo::batch_matmul with col_major = true (turbo.rs:322-326): Q4_0 weights
 * are column-major, other dtypes as hypno_hip_batch_matmul. */
int hypno_hip_batch_matmul_col(float* y, const uint8_t* w, size_t w_len, uint32_t dtype,
                               const float* x, size_t n, size_t dim, size_t batch);

/* ---------------------------------------------------------------------------
 * Weight residency.  hypno hands the kernel zero-copy slices of a read-only
 * mmap (loader.rs:139-148).  Registering such a slice uploads it once; later
 * host-slice calls whose w pointer and length match use the device copy.
 * ------------------------------------------------------------------------- */

/* Upload [host, host+len) to the current device and remember it by pointer. */
int hypno_hip_weight_register(const uint8_t* host, size_t len);

/* Forget (and free) a registration; EINVAL if it was not registered. */
int hypno_hip_weight_unregister(const uint8_t* host);

/* ---------------------------------------------------------------------------
 * Device-pointer entry points (the serving path: inputs already in HBM).
 * All pointers are device memory; `stream` is a hipStream_t or NULL.
 * ------------------------------------------------------------------------- */

/* Y[batch][n] = X[batch][m] . W^T (+ bias) with Q4_0 W (kernels.rs:256 for
 * batch == 1; turbo.rs:306-333 semantics for batch > 1). */
int hypno_hip_matmul_q4_0_dev(float* y, const uint8_t* w_q, size_t w_len, const float* x,
                              const float* bias, size_t n, size_t m, size_t batch,
                              void* stream);

/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Same arguments, semantics and kernels as
 * hypno_hip_matmul_q4_0_dev, but the scratch memory those kernels use (fp16
 * activations, per-token exponents, split-K partial planes) is one fixed
 * array of HYPNO_HIP_NOALLOC_SCRATCH_BYTES per GPU, in the library's device
 * image, instead of the per-stream workspace: the call allocates nothing.
 * A call that would need more scratch (e.g. 2048 tokens at m = 16384) is
 * EINVAL before anything is launched.  Every call on one GPU shares that
 * array and nothing in it carries over between calls: calls that overlap on
 * one GPU (other streams, other threads) race, so serialise them. */
#define HYPNO_HIP_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int hypno_hip_matmul_q4_0_dev_noalloc(float* y, const uint8_t* w_q, size_t w_len,
                                      const float* x, const float* bias, size_t n, size_t m,
                                      size_t batch, void* stream);

/* Column-major Q4_0 on device pointers (semantics of
 * hypno_hip_matmul_q4_0_col; batch > 1: each token's product as
 * turbo.rs:322-326 computes it token by token, the tokens run in groups). */
int hypno_hip_matmul_q4_0_col_dev(float* y, const uint8_t* w_q, size_t w_len, const float* x,
                                  const float* bias, size_t n, size_t m, size_t batch,
                                  void* stream);

/* Same with FP16 W (kernels.rs:571; turbo.rs:316-320). */
int hypno_hip_matmul_f16_dev(float* y, const uint8_t* w, size_t w_len, const float* x,
                             const float* bias, size_t n, size_t m, size_t batch,
                             void* stream);

/* Q8_0 on device pointers (ops.rs:33-36 for batch == 1; turbo.rs:334-341
 * semantics for batch > 1).  batch >= 16 with m % 64 == 0 runs a prefill
 * GEMM on an fp16 expansion of the weights (rel-L2 <= 2e-3 of the exact
 * product); smaller batches (m % 256 == 0, x 16-byte aligned) read each
 * weight block once per 2 to 8 tokens, every token's row bit-identical to
 * its one-token call (normwise <= 1e-4); other shapes run token by token. */
int hypno_hip_matmul_q8_0_dev(float* y, const uint8_t* w_q, size_t w_len, const float* x,
                              const float* bias, size_t n, size_t m, size_t batch,
                              void* stream);

/* quantize_f32_to_q8_0 (quant.rs:177-191) on the device, bit-exact:
 * floor(n_elems/32) blocks written to out (34 bytes each). */
int hypno_hip_quantize_q8_0_dev(uint8_t* out, const float* src, size_t n_elems, void* stream);

/* dequantize_q8_0 (quant.rs:194-206) on the device, bit-exact:
 * floor(q_len/34) blocks -> 32 fp32 values each. */
int hypno_hip_dequantize_q8_0_dev(float* out, const uint8_t* q, size_t q_len, void* stream);

/* quantize_f32_to_q4_0 (quant.rs:108-117) on the device, bit-exact:
 * floor(n_elems/32) blocks written to out (18 bytes each). */
int hypno_hip_quantize_q4_0_dev(uint8_t* out, const float* src, size_t n_elems, void* stream);

/* dequantize_q4_0 (quant.rs:120-132) on the device, bit-exact:
 * floor(q_len/18) blocks -> 32 fp32 values each. */
int hypno_hip_dequantize_q4_0_dev(float* out, const uint8_t* q, size_t q_len, void* stream);

/* ---------------------------------------------------------------------------
 * Multi-GEMV plans (no counterpart in hypno, which calls matmul_q4_0 once per
 * weight matrix: transformer.rs:305-453).  A decode step streams many
 * independent Q4_0 GEMVs (q/k/v share one input, gate/up another); running
 * them as one launch removes the per-launch cost (about 1.6 us per kernel in
 * a HIP graph on MI355X) and keeps HBM busy across matrix boundaries.
 * Each descriptor has the semantics of hypno_hip_matmul_q4_0_dev with
 * batch = 1.  Jobs must be independent: no job's y may overlap any job's y,
 * x, w, bias or prologue aux (plan_create checks this: EINVAL).  Descriptors that the streaming kernel cannot take (m % 256 != 0,
 * unaligned pointers, short buffers) are run by the generic kernel in the
 * same plan.  A plan stores the pointers: update the x buffers in place and
 * run it again (it is safe to capture plan_run in a HIP graph).
 * ------------------------------------------------------------------------- */
typedef struct hypno_hip_gemv_desc {
  float* y;              /* [n] device */
  const uint8_t* w_q;    /* Q4_0 bytes, device */
  size_t w_len;
  const float* x;        /* [m] device */
  const float* bias;     /* [n] device or NULL */
  size_t n;
  size_t m;
} hypno_hip_gemv_desc;

typedef struct hypno_hip_gemv_plan hypno_hip_gemv_plan;

/* Validate `count` descriptors on the current device and build the plan
 * (uploads a small job table; the descriptors are copied). */
int hypno_hip_q4_0_gemv_plan_create(const hypno_hip_gemv_desc* descs, size_t count,
                                    hypno_hip_gemv_plan** plan);

/* Steps either side of the decode GEMV, applied to a plan job's input while
 * the GEMV stages it (no extra pass over HBM, no extra launch), or as
 * stand-alone device calls:
 *   RMS_NORM  x' = rms_norm_fused(x, aux, eps) (kernels.rs:592-625;
 *             transformer.rs:301,435 before q/k/v and gate/up)
 *   SILU_MUL  x' = silu(x) * aux, silu(v) = v / (1 + exp(-v))
 *             (transformer.rs:446-449, turbo.rs:235-237 before down)
 * aux is a device vector of m floats (the norm weight, or the up
 * projection's output).  x itself is not modified. */
#define HYPNO_HIP_PROLOGUE_NONE 0u
#define HYPNO_HIP_PROLOGUE_RMS_NORM 1u
#define HYPNO_HIP_PROLOGUE_SILU_MUL 2u

typedef struct hypno_hip_gemv_prologue {
  uint32_t kind;     /* HYPNO_HIP_PROLOGUE_* */
  const float* aux;  /* [m] device; NULL for NONE */
  float eps;         /* RMS_NORM: rms_norm_eps (transformer.rs:59) */
} hypno_hip_gemv_prologue;

/* plan_create with one prologue per descriptor (prologues may be NULL: none).
 * Jobs the streaming kernel cannot take run the prologue as a separate
 * kernel into a plan-owned buffer, then the generic GEMV. */
int hypno_hip_q4_0_gemv_plan_create_ex(const hypno_hip_gemv_desc* descs,
                                       const hypno_hip_gemv_prologue* prologues, size_t count,
                                       hypno_hip_gemv_plan** plan);

/* Run every GEMV of the plan on `stream` (usually one kernel launch). */
int hypno_hip_q4_0_gemv_plan_run(const hypno_hip_gemv_plan* plan, void* stream);

/* Number of kernel launches plan_run issues. */
int hypno_hip_q4_0_gemv_plan_launches(const hypno_hip_gemv_plan* plan);

/* Free the plan (waits for the device first). */
int hypno_hip_q4_0_gemv_plan_destroy(hypno_hip_gemv_plan* plan);

/* ops::rms_norm / rms_norm_in_place (ops.rs:52-61 -> kernels.rs:592-625) on
 * `rows` consecutive rows of n floats: out[r] = x[r] * inv_rms(x[r]) * weight.
 * out may equal x.  Device pointers. */
int hypno_hip_rms_norm_dev(float* out, const float* x, const float* weight, size_t n,
                           size_t rows, float eps, void* stream);

/* silu_in_place(gate) then gate *= up (transformer.rs:446-449): out[i] =
 * silu(gate[i]) * up[i] over n floats; out may equal gate.  Device pointers. */
int hypno_hip_silu_mul_dev(float* out, const float* gate, const float* up, size_t n,
                           void* stream);

/* How the Q4_0 prefill GEMM applies the block scales (no counterpart in
 * hypno, whose CPU kernel has one arithmetic).  AUTO (the default) and EXACT
 * feed the MFMAs the integer nibbles and apply each block's d to its partial
 * in fp32 (the arithmetic the reference's block-at-a-time dequantisation
 * implies); FOLDED opts into folding d into fp16 weights from 128-256 tokens
 * up, as described at the top of this file.  Process-wide; returns the
 * previous mode, or -EINVAL for an unknown one. */
#define HYPNO_HIP_GEMM_AUTO 0u
#define HYPNO_HIP_GEMM_EXACT 1u
#define HYPNO_HIP_GEMM_FOLDED 2u
int hypno_hip_set_gemm_numerics(uint32_t mode);

/* ---------------------------------------------------------------------------
 * Steps either side of the GEMVs that read whole rows: the token embedding
 * before the first layer, the next-token choice after the lm_head.  Device
 * pointers, asynchronous on `stream`.
 * ------------------------------------------------------------------------- */

/* q4_0_extract_row(q, row_idx, row_width) (quant.rs:139-153): out[0..row_width)
 * = row row_idx of a Q4_0 matrix of floor(row_width / 32) blocks per row,
 * dequantised bit-exactly; elements past those blocks are 0.  A row whose
 * blocks are not all inside q_len bytes (a panic in the reference) is
 * EINVAL. */
int hypno_hip_q4_0_extract_row_dev(float* out, const uint8_t* q, size_t q_len, size_t row_idx,
                                   size_t row_width, void* stream);

/* q8_0_extract_row (quant.rs:158-175): the same with 34-byte Q8_0 blocks. */
int hypno_hip_q8_0_extract_row_dev(float* out, const uint8_t* q, size_t q_len, size_t row_idx,
                                   size_t row_width, void* stream);

/* The token embedding of a decode step or a prefill batch (transformer.rs:
 * 476-497, turbo.rs:38-66): out[t][0..hd) = row ids[t] of the embedding table
 * (dtype FP32, FP16, Q8_0 or Q4_0; quantised rows as the extract functions
 * above), for `count` token ids already in device memory.  A row outside the
 * table (a panic in the reference) is written as NaN. */
int hypno_hip_embed_tokens_dev(float* out, const uint8_t* table, size_t table_len,
                               uint32_t dtype, const uint32_t* ids, size_t count, size_t hd,
                               void* stream);

/* Greedy next token: *index = the position of the largest of n logits, as
 * Iterator::max_by with partial_cmp picks it (run.rs:232-234): the last of
 * equal maxima, NaNs passed over by the comparisons; n = 0 gives 0.
 * `index` is device memory.  4-byte-aligned logits: one launch of one
 * work-group, no workspace; otherwise two launches and a small part of the
 * stream's workspace. */
int hypno_hip_argmax_dev(uint32_t* index, const float* logits, size_t n, void* stream);

/* sample_token(logits, temperature, top_p, top_k, rng) (run.rs:203-251) on
 * the device: temperature scaling, top-k, top-p and the draw, with the
 * reference's fp32 sums in its order, so the chosen token is the
 * reference's.  *rng_state (device) is its XorShift64 state (run.rs:267-278:
 * seed with max(seed, 1)); it advances by one step when a draw is made, as
 * the reference's does.  exp is evaluated in fp64 and rounded to fp32 (the
 * reference's libm expf agrees but for results within ~2^-29 of a rounding
 * boundary).  Logits must not hold NaN (the reference's sort is then not
 * total).  Two launches (per-range candidates over up to 64 work-groups,
 * then one work-group).  The sums, the top-p walk and the draw run in
 * parallel yet give the reference's sequential fp32 results bit for bit:
 * integer prefix sums on the running sum's binade grid, with one fp32 add for
 * each value that grid cannot hold; the top-p walk sorts only the top key
 * bins down to where their mass reaches top_p (plus the fp32 sums' margin).
 * Uses the stream's workspace (about 28 n bytes). */
int hypno_hip_sample_token_dev(uint32_t* token, uint64_t* rng_state, const float* logits,
                               size_t n, float temperature, float top_p, size_t top_k,
                               void* stream);

/* Block until all work this library queued on `stream` is done. */
int hypno_hip_stream_synchronize(void* stream);

/* ---------------------------------------------------------------------------
 * .hypno model files (format.rs, loader.rs).  Replaces HypnoModel
 * (loader.rs:20-169): the file is mapped read-only and its manifest parsed
 * with the reference's checks and errors; unless HOST_ONLY is given, every
 * tensor payload is then uploaded once to the current device, so decode and
 * prefill calls take device pointers straight from the model.  Host pointers
 * are the zero-copy mapping (what HypnoModel::get_tensor_data returns); the
 * device copy keeps each tensor's in-file alignment (64 bytes for files
 * written by hypno's converter).  Strings, shapes and both pointers stay
 * valid until hypno_hip_model_close.
 * Errors: ENOENT (file missing), EFILE (open / mmap / read failure),
 * EFORMAT (one per FormatError variant: bad magic, version, short buffer,
 * UTF-8, unknown dtype, tensor out of file bounds), ENOMEM / EDEVICE
 * (upload).  A tensor name whose bytes run past the end of the file is
 * EFORMAT here (the reference reads it unchecked, loader.rs:96-97).
 * ------------------------------------------------------------------------- */
typedef struct hypno_hip_model hypno_hip_model;

typedef struct hypno_hip_tensor_info {
  const char* name;       /* NUL-terminated UTF-8 */
  uint32_t dtype;         /* HYPNO_DTYPE_* (dtype.rs:4-15) */
  uint32_t ndim;
  const uint64_t* shape;  /* [ndim] (NULL when ndim == 0) */
  uint64_t offset;        /* absolute byte offset in the file */
  uint64_t data_len;      /* payload bytes */
  const uint8_t* host;    /* [data_len] in the read-only mapping */
  const uint8_t* device;  /* [data_len] on the model's device; NULL if host-only
                             or data_len == 0 */
} hypno_hip_tensor_info;

/* Parse and map only; no device is touched (tools, CPU-side checks). */
#define HYPNO_HIP_MODEL_HOST_ONLY 1u

/* HypnoModel::open (loader.rs:39-134), plus the upload to the current
 * device (pinned, pipelined: file reads overlap the host-to-device copies). */
int hypno_hip_model_open(const char* path, uint32_t flags, hypno_hip_model** model);

/* Unmap the file and free the device copy. */
int hypno_hip_model_close(hypno_hip_model* model);

/* The header fields (format.rs:13-24); any pointer may be NULL. */
int hypno_hip_model_header(const hypno_hip_model* model, uint32_t* version,
                           uint32_t* metadata_kv_count, uint32_t* tensor_count);

/* Metadata entry i in file order (HypnoManifest::metadata). */
int hypno_hip_model_metadata_at(const hypno_hip_model* model, size_t i, const char** key,
                                const char** value);

/* HypnoModel::get_metadata (loader.rs:158-163): first entry with this key;
 * ENOENT if none. */
int hypno_hip_model_metadata(const hypno_hip_model* model, const char* key, const char** value);

/* Tensor i in file order (HypnoManifest::tensors). */
int hypno_hip_model_tensor_at(const hypno_hip_model* model, size_t i,
                              hypno_hip_tensor_info* info);

/* HypnoModel::find_tensor / get_tensor_data (loader.rs:139-156): first tensor
 * with this name; ENOENT if none. */
int hypno_hip_model_find_tensor(const hypno_hip_model* model, const char* name,
                                hypno_hip_tensor_info* info);

/* HypnoModel::is_col_major (loader.rs:166-168): 1 if metadata
 * "weight_layout" is "col_major", else 0 (also for a NULL model). */
int hypno_hip_model_is_col_major(const hypno_hip_model* model);

#ifdef __cplusplus
}
#endif

#endif /* HYPNO_HIP_H */
