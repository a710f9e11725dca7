/*
 * q4_0_oracle.c — CPU restatement of hypno's Q4_0 / FP16 matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker and the CPU
 * baseline.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library (hypno_amd) never
 * links, calls or falls back to it.
 *
 * Every function cites the reference source it restates (paths relative to
 * the hypno repository root, crates/hypno/src/).  The reference is Rust and
 * cannot be built in this image (no rustc/cargo, no crate registry), so it is
 * restated here in C and pinned by the tests in tests/test_oracle.py against
 * the reference's own known-answer tests, IEEE definitions, numpy and
 * brute-force fp64 sums.
 *
 * Parity status per function (what pins it):
 *   orc_f16_to_f32      exact by definition; checked against numpy and F16C
 *   orc_f32_to_f16      IEEE RNE; checked against numpy float16 and F16C
 *   orc_quantize_q4_0   reference KATs quant.rs:213-237, sft_convert.rs:430-457,
 *                       hand-computed blocks (half-away rounding, clamp, f16 d)
 *   orc_dequantize_q4_0 closed form; hand-built blocks, nibble 0/8/15 cases
 *   orc_matmul_q4_0_*   fp64 brute force on the dequantized matrix, exact
 *                       integer-valued cases, straddling rows (K % 32 != 0),
 *                       short-buffer semantics, bias; the exact fp32 bits of
 *                       the AVX2 summation order are "parity unpinned" (only
 *                       running hypno could pin them)
 *   orc_matmul_f16_*    fp64 brute force; exact integer KAT (ops.rs:114-121)
 *   orc_batch_matmul    per-token equality with the GEMV; turbo.rs KATs
 *   orc_quantize_q8_0   no reference test covers Q8_0: hand-computed blocks
 *                       (divide by the rounded f16 scale, half-away ties,
 *                       clamp to +-127, zero / NaN / overflowing scales)
 *   orc_dequantize_q8_0 closed form (u - 128) * d, exact
 *   orc_matmul_q8_0     dequantize + matmul_f32_scalar order; fp64 brute
 *                       force and exact integer cases (the AVX2 / AVX-512
 *                       f32 orders are not restated: tolerance-based)
 *   orc_matmul_q4_0_col matmul_q4_0_col_scalar order; no reference test
 *                       checks it numerically: exact integer cases, fp64,
 *                       n % 32 != 0 tails and short buffers (the AVX2 form's
 *                       bits depend on the thread count: not restated)
 *   orc_rms_norm_*      reference KATs ops.rs:131-136, turbo.rs:716-735 (the
 *                       f64 batch_rms_norm within 1e-6 of the SIMD form),
 *                       turbo.rs:924-951; closed forms (constant rows, the
 *                       n % 8 tail's divide form) and an fp64 brute force
 *   orc_silu_mul        reference KAT turbo.rs:979-990; silu(v) - silu(-v) = v
 *                       and fp64 closed form
 *   orc_xorshift64_*    Marsaglia's published xorshift64 (13, 7, 17) sequence
 *                       from seed 88172645463325252; max(seed, 1) seeding
 *   orc_argmax          Iterator::max_by fold semantics: hand-built ties,
 *                       signed zeros and NaN positions
 *   orc_sample_token    hand-computed draws whose r lies well inside one
 *                       interval (exact decimal boundaries), top-k = 1 and
 *                       a tiny top-p reduce to the argmax, uniform logits
 *                       reduce to floor(r n), the sum <= 0 and never-crossed
 *                       top-p paths, and a float32 restatement in numpy
 *
 * Build: oracle/Makefile (gcc, -ffp-contract=off, no fast-math; the AVX2
 * kernels use target attributes so the library runs on any x86-64 host and
 * dispatches at run time like kernels.rs:256-265).
 */
#include <math.h>
#include <stdint.h>
#include <stddef.h>
#include <string.h>
#include <stdlib.h>
#ifdef _OPENMP
#include <omp.h>
#endif
#if defined(__x86_64__)
#include <immintrin.h>
#endif

#define Q4_BLOCK_ELEMS 32
#define Q4_BLOCK_BYTES 18

static int g_threads = 1;

/* Number of OpenMP threads the matmul kernels use (rayon pool size in
 * hypno: run.rs:56-59, bench.rs:20). */
void orc_set_threads(int n) { g_threads = n > 0 ? n : 1; }
int orc_get_threads(void) { return g_threads; }

/* ------------------------------------------------------------------------ */
/* half 2.7.1 f16 <-> f32 (third-party crate used at kernels.rs:297,376,561,  */
/* 583 and quant.rs:26,57).  to_f32 is exact; from_f32 is IEEE-754          */
/* round-to-nearest-even with overflow to infinity.                           */
/* ------------------------------------------------------------------------ */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            /* subnormal: man * 2^-24; normalise so bit 10 is the implicit 1 */
            int e = -1;
            do { man <<= 1; e++; } while (!(man & 0x400u));
            bits = sign | ((uint32_t)(112 - e) << 23) | ((man & 0x3FFu) << 13);
        }
    } else if (exp == 31) {
        /* inf, or NaN made quiet with its payload kept */
        bits = sign | 0x7F800000u | (man << 13) | (man ? 0x00400000u : 0u);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (exp == 0xFF) {
        if (man == 0) return (uint16_t)(sign | 0x7C00u);
        return (uint16_t)(sign | 0x7E00u | (man >> 13));
    }
    int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        /* f16 subnormal (or zero): units of 2^-24 */
        if (exp == 0) return (uint16_t)sign; /* f32 subnormal/zero < 2^-126 */
        uint32_t full = man | 0x800000u;
        int s = 126 - (int)exp; /* >= 14 */
        if (s > 24) return (uint16_t)sign;
        uint32_t hm = full >> s;
        uint32_t rem = full & ((1u << s) - 1u);
        uint32_t half = 1u << (s - 1);
        if (rem > half || (rem == half && (hm & 1u))) hm++;
        return (uint16_t)(sign | hm);
    }
    uint32_t hm = man >> 13;
    uint32_t rem = man & 0x1FFFu;
    uint32_t h = ((uint32_t)e << 10) + hm;
    if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) h++; /* carry may reach inf */
    return (uint16_t)(sign | h);
}

void orc_f16_to_f32_array(const uint16_t* src, float* dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = orc_f16_to_f32(src[i]);
}

void orc_f32_to_f16_array(const float* src, uint16_t* dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = orc_f32_to_f16(src[i]);
}

/* ------------------------------------------------------------------------ */
/* Q4_0 codec (quant.rs)                                                      */
/* ------------------------------------------------------------------------ */

/* Rust `f32 as i32` is a saturating cast with NaN -> 0. */
static int32_t sat_f32_to_i32(float r) {
    if (r != r) return 0;
    if (r >= 2147483648.0f) return INT32_MAX;
    if (r <= -2147483648.0f) return INT32_MIN;
    return (int32_t)r;
}

static int32_t clamp_i32(int32_t v, int32_t lo, int32_t hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}

/* Q4_0Block::quantize, quant.rs:49-71.
 * amax = fold(0, f32::max) over |v| (f32::max ignores NaN, like fmaxf);
 * s = amax/7 in f32 (1.0 when amax == 0); d = f16 RNE(s);
 * q = clamp(round_half_away(v / s), -8, 7) — divides by the unrounded s;
 * byte i = (q[2i]+8) | (q[2i+1]+8) << 4. */
void orc_quantize_block_q4_0(const float* src, uint8_t* out) {
    float max_abs = 0.0f;
    for (int i = 0; i < Q4_BLOCK_ELEMS; i++) max_abs = fmaxf(max_abs, fabsf(src[i]));
    float scale = max_abs > 0.0f ? max_abs / 7.0f : 1.0f;
    uint16_t d = orc_f32_to_f16(scale);
    out[0] = (uint8_t)(d & 0xFF);
    out[1] = (uint8_t)(d >> 8);
    for (int i = 0; i < 16; i++) {
        float v0 = src[2 * i];
        float v1 = src[2 * i + 1];
        int32_t q0 = clamp_i32(sat_f32_to_i32(roundf(v0 / scale)), -8, 7);
        int32_t q1 = clamp_i32(sat_f32_to_i32(roundf(v1 / scale)), -8, 7);
        uint8_t nib0 = (uint8_t)((q0 + 8) & 0x0F);
        uint8_t nib1 = (uint8_t)((q1 + 8) & 0x0F);
        out[2 + i] = (uint8_t)(nib0 | (nib1 << 4));
    }
}

/* quantize_f32_to_q4_0, quant.rs:108-117: floor(len/32) blocks; a trailing
 * partial block is dropped.  Returns the number of bytes written. */
size_t orc_quantize_q4_0(const float* src, size_t n, uint8_t* out) {
    size_t nb = n / Q4_BLOCK_ELEMS;
    for (size_t b = 0; b < nb; b++)
        orc_quantize_block_q4_0(src + b * Q4_BLOCK_ELEMS, out + b * Q4_BLOCK_BYTES);
    return nb * Q4_BLOCK_BYTES;
}

/* Q4_0Block::dequantize, quant.rs:25-34; dequantize_q4_0, quant.rs:120-132:
 * floor(q_len/18) blocks; element 2i = (lo(byte i) - 8) * d,
 * element 2i+1 = (hi(byte i) - 8) * d, computed in f32 (exact). */
size_t orc_dequantize_q4_0(const uint8_t* q, size_t q_len, float* out) {
    size_t nb = q_len / Q4_BLOCK_BYTES;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = q + b * Q4_BLOCK_BYTES;
        float scale = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
        for (int i = 0; i < 16; i++) {
            uint8_t byte = blk[2 + i];
            out[b * 32 + 2 * i] = (float)((int32_t)(byte & 0x0F) - 8) * scale;
            out[b * 32 + 2 * i + 1] = (float)((int32_t)((byte >> 4) & 0x0F) - 8) * scale;
        }
    }
    return nb * Q4_BLOCK_ELEMS;
}

static void deq_block(const uint8_t* blk, float* deq) {
    float scale = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
    for (int i = 0; i < 16; i++) {
        uint8_t byte = blk[2 + i];
        deq[2 * i] = (float)((int32_t)(byte & 0x0F) - 8) * scale;
        deq[2 * i + 1] = (float)((int32_t)((byte >> 4) & 0x0F) - 8) * scale;
    }
}

/* ------------------------------------------------------------------------ */
/* matmul_q4_0_scalar, kernels.rs:362-400.                                    */
/* Row r covers flattened elements [r*m, (r+1)*m); it walks the blocks that    */
/* overlap that range (blocks straddle rows when m % 32 != 0).  A block whose  */
/* 18 bytes do not fit in w_len ends the row (`break`, kernels.rs:374).        */
/* sum += deq*x in f32 without contraction; y = sum + (bias or 0.0).          */
/* ------------------------------------------------------------------------ */
static float row_q4_0_scalar(const uint8_t* w, size_t w_len, const float* x,
                             size_t row, size_t m) {
    size_t row_start = row * m;
    size_t row_end = row_start + m;
    size_t first_block = row_start / 32;
    size_t last_block = (row_end > 0 ? row_end - 1 : 0) / 32;
    float sum = 0.0f;
    float deq[32];
    for (size_t b = first_block; b <= last_block; b++) {
        size_t bo = b * Q4_BLOCK_BYTES;
        if (bo + Q4_BLOCK_BYTES > w_len) break;
        deq_block(w + bo, deq);
        size_t block_start = b * 32;
        size_t ov_start = block_start < row_start ? row_start - block_start : 0;
        size_t ov_end = block_start + 32 > row_end ? row_end - block_start : 32;
        size_t x_off = block_start > row_start ? block_start - row_start : 0;
        for (size_t i = ov_start; i < ov_end; i++) sum += deq[i] * x[x_off + (i - ov_start)];
    }
    return sum;
}

void orc_matmul_q4_0_scalar(float* y, const uint8_t* w, size_t w_len, const float* x,
                            const float* bias, size_t n, size_t m) {
    long long nn = (long long)n;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (long long r = 0; r < nn; r++) {
        float sum = row_q4_0_scalar(w, w_len, x, (size_t)r, m);
        y[r] = sum + (bias ? bias[r] : 0.0f);
    }
}

#if defined(__x86_64__)
/* hsum256, kernels.rs:169-178: lo128+hi128, then two horizontal adds. */
__attribute__((target("avx2,fma"))) static inline float hsum256(__m256 v) {
    __m128 hi = _mm256_extractf128_ps(v, 1);
    __m128 lo = _mm256_castps256_ps128(v);
    __m128 s = _mm_add_ps(lo, hi);
    s = _mm_hadd_ps(s, s);
    s = _mm_hadd_ps(s, s);
    return _mm_cvtss_f32(s);
}

/* matmul_q4_0_avx2, kernels.rs:270-359.  Same operation order: per full block
 * four 8-wide FMAs into acc0..acc3 over a scalar-dequantised stack buffer;
 * boundary blocks add deq*x into scalar_tail; at the end
 * ((acc0+acc1)+(acc2+acc3)) -> hsum256 -> + scalar_tail -> + bias. */
__attribute__((target("avx2,fma"))) static float row_q4_0_avx2(
    const uint8_t* w, size_t w_len, const float* x, size_t row, size_t m) {
    size_t row_start = row * m;
    size_t row_end = row_start + m;
    size_t first_block = row_start / 32;
    size_t last_block = (row_end > 0 ? row_end - 1 : 0) / 32;
    __m256 acc0 = _mm256_setzero_ps();
    __m256 acc1 = _mm256_setzero_ps();
    __m256 acc2 = _mm256_setzero_ps();
    __m256 acc3 = _mm256_setzero_ps();
    float scalar_tail = 0.0f;
    float deq[32];
    for (size_t b = first_block; b <= last_block; b++) {
        size_t bo = b * Q4_BLOCK_BYTES;
        if (bo + Q4_BLOCK_BYTES > w_len) break;
        deq_block(w + bo, deq);
        size_t block_start = b * 32;
        size_t ov_start = block_start < row_start ? row_start - block_start : 0;
        size_t ov_end = block_start + 32 > row_end ? row_end - block_start : 32;
        size_t x_off = block_start > row_start ? block_start - row_start : 0;
        if (ov_start == 0 && ov_end == 32) {
            __m256 dv0 = _mm256_loadu_ps(deq);
            __m256 dv1 = _mm256_loadu_ps(deq + 8);
            __m256 dv2 = _mm256_loadu_ps(deq + 16);
            __m256 dv3 = _mm256_loadu_ps(deq + 24);
            __m256 xv0 = _mm256_loadu_ps(x + x_off);
            __m256 xv1 = _mm256_loadu_ps(x + x_off + 8);
            __m256 xv2 = _mm256_loadu_ps(x + x_off + 16);
            __m256 xv3 = _mm256_loadu_ps(x + x_off + 24);
            acc0 = _mm256_fmadd_ps(dv0, xv0, acc0);
            acc1 = _mm256_fmadd_ps(dv1, xv1, acc1);
            acc2 = _mm256_fmadd_ps(dv2, xv2, acc2);
            acc3 = _mm256_fmadd_ps(dv3, xv3, acc3);
        } else {
            for (size_t i = ov_start; i < ov_end; i++)
                scalar_tail += deq[i] * x[x_off + (i - ov_start)];
        }
    }
    __m256 sum01 = _mm256_add_ps(acc0, acc1);
    __m256 sum23 = _mm256_add_ps(acc2, acc3);
    __m256 sumall = _mm256_add_ps(sum01, sum23);
    return hsum256(sumall) + scalar_tail;
}

__attribute__((target("avx2,fma"))) void orc_matmul_q4_0_avx2(
    float* y, const uint8_t* w, size_t w_len, const float* x, const float* bias,
    size_t n, size_t m) {
    size_t total_blocks = (n * m + 31) / 32;
    if (w_len < total_blocks * Q4_BLOCK_BYTES) {
        /* kernels.rs:275-277: a short buffer falls back to the scalar kernel */
        orc_matmul_q4_0_scalar(y, w, w_len, x, bias, n, m);
        return;
    }
    long long nn = (long long)n;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (long long r = 0; r < nn; r++) {
        float total = row_q4_0_avx2(w, w_len, x, (size_t)r, m);
        if (bias) total += bias[r];
        y[r] = total;
    }
}

/* matmul_f16_avx2_fma, kernels.rs:543-565: one 8-wide FMA accumulator over
 * F16C-converted weights, hsum256, scalar tail, + (bias or 0.0). */
__attribute__((target("avx2,fma,f16c"))) void orc_matmul_f16_avx2(
    float* y, const uint8_t* w, size_t w_len, const float* x, const float* bias,
    size_t n, size_t m) {
    (void)w_len;
    const uint16_t* w16 = (const uint16_t*)w;
    size_t m8 = m - (m % 8);
    long long nn = (long long)n;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (long long r = 0; r < nn; r++) {
        const uint16_t* row = w16 + (size_t)r * m;
        __m256 acc = _mm256_setzero_ps();
        for (size_t j = 0; j < m8; j += 8) {
            __m128i w128 = _mm_loadu_si128((const __m128i*)(row + j));
            __m256 wf = _mm256_cvtph_ps(w128);
            __m256 xv = _mm256_loadu_ps(x + j);
            acc = _mm256_fmadd_ps(wf, xv, acc);
        }
        float sum = hsum256(acc);
        for (size_t j = m8; j < m; j++) sum += orc_f16_to_f32(row[j]) * x[j];
        y[r] = sum + (bias ? bias[r] : 0.0f);
    }
}

/* Hardware F16C conversions, used only to cross-check orc_f32_to_f16 and
 * orc_f16_to_f32 in the tests (an implementation independent of the C code
 * above).  Round-to-nearest-even is requested explicitly. */
__attribute__((target("f16c"))) void orc_f32_to_f16_f16c(const float* src, uint16_t* dst, size_t n) {
    for (size_t i = 0; i < n; i++)
        dst[i] = (uint16_t)_cvtss_sh(src[i], _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
}
__attribute__((target("f16c"))) void orc_f16_to_f32_f16c(const uint16_t* src, float* dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = _cvtsh_ss(src[i]);
}

/* rms_norm_fused, AVX2 branch (kernels.rs:592-619): one 8-wide FMA chain
 * of v*v over the first n8 = n - n % 8 elements, hsum256, the tail's x*x
 * added one by one (no FMA), divided by n; the n8 elements become
 * (v * inv_rms) * w with inv_rms = 1 / sqrt(mean + eps), the tail
 * x / sqrt(mean + eps) * w.  In place. */
__attribute__((target("avx2,fma"))) void orc_rms_norm_avx2(float* x, const float* weight,
                                                           size_t n, float eps) {
    size_t n8 = n - (n % 8);
    __m256 sq = _mm256_setzero_ps();
    for (size_t i = 0; i < n8; i += 8) {
        __m256 v = _mm256_loadu_ps(x + i);
        sq = _mm256_fmadd_ps(v, v, sq);
    }
    float mean_sq = hsum256(sq);
    for (size_t i = n8; i < n; i++) mean_sq += x[i] * x[i];
    mean_sq /= (float)n;
    __m256 inv_rms = _mm256_set1_ps(1.0f / sqrtf(mean_sq + eps));
    for (size_t i = 0; i < n8; i += 8) {
        __m256 v = _mm256_loadu_ps(x + i);
        __m256 w = _mm256_loadu_ps(weight + i);
        _mm256_storeu_ps(x + i, _mm256_mul_ps(_mm256_mul_ps(v, inv_rms), w));
    }
    for (size_t i = n8; i < n; i++) x[i] = x[i] / sqrtf(mean_sq + eps) * weight[i];
}

int orc_have_avx2_fma(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
}
int orc_have_f16c(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("f16c");
}
#else
int orc_have_avx2_fma(void) { return 0; }
int orc_have_f16c(void) { return 0; }
void orc_rms_norm_scalar(float* x, const float* weight, size_t n, float eps);
void orc_rms_norm_avx2(float* x, const float* weight, size_t n, float eps) {
    orc_rms_norm_scalar(x, weight, n, eps);
}
void orc_matmul_q4_0_avx2(float* y, const uint8_t* w, size_t w_len, const float* x,
                          const float* bias, size_t n, size_t m) {
    orc_matmul_q4_0_scalar(y, w, w_len, x, bias, n, m);
}
void orc_matmul_f16_scalar(float* y, const uint8_t* w, size_t w_len, const float* x,
                           const float* bias, size_t n, size_t m);
void orc_matmul_f16_avx2(float* y, const uint8_t* w, size_t w_len, const float* x,
                         const float* bias, size_t n, size_t m) {
    orc_matmul_f16_scalar(y, w, w_len, x, bias, n, m);
}
#endif

/* matmul_f16 scalar fallback, kernels.rs:578-585. */
void orc_matmul_f16_scalar(float* y, const uint8_t* w, size_t w_len, const float* x,
                           const float* bias, size_t n, size_t m) {
    (void)w_len;
    const uint16_t* w16 = (const uint16_t*)w;
    long long nn = (long long)n;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (long long r = 0; r < nn; r++) {
        const uint16_t* row = w16 + (size_t)r * m;
        float s = 0.0f;
        for (size_t j = 0; j < m; j++) s += orc_f16_to_f32(row[j]) * x[j];
        y[r] = s + (bias ? bias[r] : 0.0f);
    }
}

/* matmul_q4_0 dispatch, kernels.rs:256-265: AVX2+FMA when present, else scalar. */
void orc_matmul_q4_0(float* y, const uint8_t* w, size_t w_len, const float* x,
                     const float* bias, size_t n, size_t m) {
    if (orc_have_avx2_fma())
        orc_matmul_q4_0_avx2(y, w, w_len, x, bias, n, m);
    else
        orc_matmul_q4_0_scalar(y, w, w_len, x, bias, n, m);
}

/* matmul_f16 dispatch, kernels.rs:571-586. */
void orc_matmul_f16(float* y, const uint8_t* w, size_t w_len, const float* x,
                    const float* bias, size_t n, size_t m) {
    if (orc_have_avx2_fma() && orc_have_f16c())
        orc_matmul_f16_avx2(y, w, w_len, x, bias, n, m);
    else
        orc_matmul_f16_scalar(y, w, w_len, x, bias, n, m);
}

/* turbo::batch_matmul Q4_0 / FP16 arms, turbo.rs:306-333: one GEMV per token,
 * X [batch][m] -> Y [batch][n], no bias.  dtype uses hypno's DType codes
 * (dtype.rs:4-15): 1 = FP16, 3 = Q4_0.  Returns 0, or -1 for another dtype. */
int orc_batch_matmul(float* y, const uint8_t* w, size_t w_len, int dtype, const float* x,
                     size_t n, size_t m, size_t batch) {
    for (size_t t = 0; t < batch; t++) {
        if (dtype == 3)
            orc_matmul_q4_0(y + t * n, w, w_len, x + t * m, NULL, n, m);
        else if (dtype == 1)
            orc_matmul_f16(y + t * n, w, w_len, x + t * m, NULL, n, m);
        else
            return -1;
    }
    return 0;
}

/* fp64 brute force: dequantise the whole flattened tensor (quant.rs:120-132),
 * then y[r] = sum_k w[r*m+k] * x[k] in double, + bias.  Elements beyond the
 * last whole block in w_len contribute nothing (kernels.rs:374). */
void orc_matmul_q4_0_f64(double* y, const uint8_t* w, size_t w_len, const float* x,
                         const float* bias, size_t n, size_t m) {
    size_t avail = (w_len / Q4_BLOCK_BYTES) * 32;
    long long nn = (long long)n;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (long long r = 0; r < nn; r++) {
        double s = 0.0;
        float deq[32];
        size_t cur_block = (size_t)-1;
        for (size_t k = 0; k < m; k++) {
            size_t e = (size_t)r * m + k;
            if (e >= avail) break;
            size_t b = e / 32;
            if (b != cur_block) { deq_block(w + b * Q4_BLOCK_BYTES, deq); cur_block = b; }
            s += (double)deq[e % 32] * (double)x[k];
        }
        y[r] = s + (bias ? (double)bias[r] : 0.0);
    }
}

void orc_matmul_f16_f64(double* y, const uint8_t* w, const float* x, const float* bias,
                        size_t n, size_t m) {
    const uint16_t* w16 = (const uint16_t*)w;
    long long nn = (long long)n;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (long long r = 0; r < nn; r++) {
        double s = 0.0;
        for (size_t k = 0; k < m; k++)
            s += (double)orc_f16_to_f32(w16[(size_t)r * m + k]) * (double)x[k];
        y[r] = s + (bias ? (double)bias[r] : 0.0);
    }
}

/* Sum of |w_rk * x_k| per row (the conditioning denominator for the
 * tolerance report). */
void orc_matmul_q4_0_absdot_f64(double* y, const uint8_t* w, size_t w_len, const float* x,
                                size_t n, size_t m) {
    size_t avail = (w_len / Q4_BLOCK_BYTES) * 32;
    long long nn = (long long)n;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (long long r = 0; r < nn; r++) {
        double s = 0.0;
        float deq[32];
        size_t cur_block = (size_t)-1;
        for (size_t k = 0; k < m; k++) {
            size_t e = (size_t)r * m + k;
            if (e >= avail) break;
            size_t b = e / 32;
            if (b != cur_block) { deq_block(w + b * Q4_BLOCK_BYTES, deq); cur_block = b; }
            s += fabs((double)deq[e % 32] * (double)x[k]);
        }
        y[r] = s;
    }
}

/* rms_norm_fused, scalar fallback (kernels.rs:621-624): sequential sum of
 * v*v, / n, inv_rms = 1 / sqrt(mean + eps), x * inv_rms * w.  In place. */
void orc_rms_norm_scalar(float* x, const float* weight, size_t n, float eps) {
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) sum += x[i] * x[i];
    float mean_sq = sum / (float)n;
    float inv_rms = 1.0f / sqrtf(mean_sq + eps);
    for (size_t i = 0; i < n; i++) x[i] = x[i] * inv_rms * weight[i];
}

/* ops::rms_norm_in_place -> kernels::rms_norm_fused (ops.rs:59-61,
 * kernels.rs:592-625): AVX2 when present, else scalar; `rows` rows of n. */
void orc_rms_norm(float* x, const float* weight, size_t n, size_t rows, float eps) {
    for (size_t r = 0; r < rows; r++) {
        if (orc_have_avx2_fma())
            orc_rms_norm_avx2(x + r * n, weight, n, eps);
        else
            orc_rms_norm_scalar(x + r * n, weight, n, eps);
    }
}

/* turbo::batch_rms_norm (turbo.rs:288-303): f64 sum of squares,
 * rms = (f32)sqrt(ss / dim + eps) in f64, inv = 1 / rms in f32,
 * out = inp * inv * w. */
void orc_batch_rms_norm(float* out, const float* inp, const float* weight, size_t dim,
                        size_t batch, float eps) {
    for (size_t r = 0; r < batch; r++) {
        const float* in = inp + r * dim;
        double ss = 0.0;
        for (size_t i = 0; i < dim; i++) ss += (double)in[i] * (double)in[i];
        float rms = (float)sqrt(ss / (double)dim + (double)eps);
        float inv = 1.0f / rms;
        for (size_t i = 0; i < dim; i++) out[r * dim + i] = in[i] * inv * weight[i];
    }
}

/* ops::silu_in_place then gate *= up (ops.rs:81-83, transformer.rs:446-449):
 * out[i] = (g / (1 + exp(-g))) * up[i] with libm expf (what Rust's f32::exp
 * calls on Linux). */
void orc_silu_mul(float* out, const float* gate, const float* up, size_t n) {
    for (size_t i = 0; i < n; i++) {
        float g = gate[i];
        float s = g / (1.0f + expf(-g));
        out[i] = s * up[i];
    }
}

/* ------------------------------------------------------------------------ */
/* Q8_0 (quant.rs:74-103, 176-206; ops.rs:33-36; turbo.rs:334-341)           */
/* ------------------------------------------------------------------------ */

#define Q8_BLOCK_BYTES 34

/* quantize_f32_to_q8_0, quant.rs:177-191: floor(len/32) blocks;
 * amax = fold(0, f32::max) over |v|; d = f16 RNE(amax / 127) (1.0 when
 * amax == 0); q = clamp(round_half_away(v / f32(d)), -127, 127) — divides by
 * the ROUNDED scale (unlike Q4_0); byte = q + 128. */
size_t orc_quantize_q8_0(const float* src, size_t n, uint8_t* out) {
    size_t nb = n / 32;
    for (size_t b = 0; b < nb; b++) {
        const float* v = src + b * 32;
        uint8_t* o = out + b * Q8_BLOCK_BYTES;
        float max_abs = 0.0f;
        for (int i = 0; i < 32; i++) max_abs = fmaxf(max_abs, fabsf(v[i]));
        uint16_t d = orc_f32_to_f16(max_abs > 0.0f ? max_abs / 127.0f : 1.0f);
        float scale = orc_f16_to_f32(d);
        o[0] = (uint8_t)(d & 0xFF);
        o[1] = (uint8_t)(d >> 8);
        for (int i = 0; i < 32; i++) {
            int32_t q = clamp_i32(sat_f32_to_i32(roundf(v[i] / scale)), -127, 127);
            o[2 + i] = (uint8_t)(q + 128);
        }
    }
    return nb * Q8_BLOCK_BYTES;
}

/* dequantize_q8_0, quant.rs:194-206 (Q8_0Block::dequantize, quant.rs:90-95):
 * floor(len/34) blocks; element i = (u_i - 128) * d in f32 (exact). */
size_t orc_dequantize_q8_0(const uint8_t* q, size_t q_len, float* out) {
    size_t nb = q_len / Q8_BLOCK_BYTES;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = q + b * Q8_BLOCK_BYTES;
        float scale = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
        for (int i = 0; i < 32; i++) out[b * 32 + i] = (float)((int32_t)blk[2 + i] - 128) * scale;
    }
    return nb * 32;
}

/* matmul_vec_auto's Q8_0 arm, ops.rs:33-36: dequantize_q8_0 then matmul_f32
 * in its scalar order (kernels.rs:234-241: s += w*x over the row, then
 * s + (bias or 0.0)); rows are the flattened ranges [r*m, (r+1)*m) of the
 * dequantised tensor.  Returns -1 (the reference panics) when the buffer
 * holds fewer than n*m elements, else 0. */
int orc_matmul_q8_0(float* y, const uint8_t* w, size_t w_len, const float* x, const float* bias,
                    size_t n, size_t m) {
    size_t avail = (w_len / Q8_BLOCK_BYTES) * 32;
    if (avail < n * m) return -1;
    float* deq = (float*)malloc((avail ? avail : 1) * sizeof(float));
    if (!deq) return -2;
    orc_dequantize_q8_0(w, w_len, deq);
    long long nn = (long long)n;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (long long r = 0; r < nn; r++) {
        const float* row = deq + (size_t)r * m;
        float s = 0.0f;
        for (size_t j = 0; j < m; j++) s += row[j] * x[j];
        y[r] = s + (bias ? bias[r] : 0.0f);
    }
    free(deq);
    return 0;
}

/* fp64 brute force of the same product (the tolerance reference). */
void orc_matmul_q8_0_f64(double* y, const uint8_t* w, size_t w_len, const float* x,
                         const float* bias, size_t n, size_t m) {
    (void)w_len;
    long long nn = (long long)n;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (long long r = 0; r < nn; r++) {
        double s = 0.0;
        for (size_t j = 0; j < m; j++) {
            size_t e = (size_t)r * m + j;
            const uint8_t* blk = w + (e / 32) * Q8_BLOCK_BYTES;
            double d = (double)orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
            s += (double)((int32_t)blk[2 + e % 32] - 128) * d * (double)x[j];
        }
        y[r] = s + (bias ? (double)bias[r] : 0.0);
    }
}

/* ------------------------------------------------------------------------ */
/* Column-major Q4_0 (kernels.rs:403-535)                                     */
/* ------------------------------------------------------------------------ */

/* matmul_q4_0_col_scalar, kernels.rs:506-535: y = 0; for each input index k,
 * blocks_per_col = n / 32 blocks of column k (byte offset k * nb * 18), each
 * adding deq * x[k] to y[32b + i] (i < n); a block past w_len ends column k
 * (and, offsets only growing, every later one); then y += bias. */
void orc_matmul_q4_0_col(float* y, const uint8_t* w, size_t w_len, const float* x,
                         const float* bias, size_t n, size_t m) {
    size_t nb = n / 32;
    size_t col_bytes = nb * Q4_BLOCK_BYTES;
    for (size_t i = 0; i < n; i++) y[i] = 0.0f;
    for (size_t k = 0; k < m; k++) {
        float xk = x[k];
        for (size_t b = 0; b < nb; b++) {
            size_t bo = k * col_bytes + b * Q4_BLOCK_BYTES;
            if (bo + Q4_BLOCK_BYTES > w_len) break;
            float scale = orc_f16_to_f32((uint16_t)(w[bo] | (w[bo + 1] << 8)));
            for (int i = 0; i < 16; i++) {
                uint8_t byte = w[bo + 2 + i];
                float v0 = (float)((int32_t)(byte & 0x0F) - 8) * scale;
                float v1 = (float)((int32_t)((byte >> 4) & 0x0F) - 8) * scale;
                size_t r = b * 32 + 2 * (size_t)i;
                if (r < n) y[r] += v0 * xk;
                if (r + 1 < n) y[r + 1] += v1 * xk;
            }
        }
    }
    if (bias)
        for (size_t i = 0; i < n; i++) y[i] += bias[i];
}

/* fp64 of the same sum (the tolerance reference). */
void orc_matmul_q4_0_col_f64(double* y, const uint8_t* w, size_t w_len, const float* x,
                             const float* bias, size_t n, size_t m) {
    size_t nb = n / 32;
    for (size_t i = 0; i < n; i++) y[i] = bias ? (double)bias[i] : 0.0;
    for (size_t k = 0; k < m; k++) {
        for (size_t b = 0; b < nb; b++) {
            size_t bo = (k * nb + b) * Q4_BLOCK_BYTES;
            if (bo + Q4_BLOCK_BYTES > w_len) break;
            double d = (double)orc_f16_to_f32((uint16_t)(w[bo] | (w[bo + 1] << 8)));
            for (int i = 0; i < 32; i++) {
                uint8_t byte = w[bo + 2 + i / 2];
                int q = (int)((i & 1) ? (byte >> 4) : (byte & 0x0F)) - 8;
                y[b * 32 + i] += (double)q * d * (double)x[k];
            }
        }
    }
}


/* ------------------------------------------------------------------------ */
/* Next-token choice after the lm_head (run.rs:203-278; serve.rs:279-312 is  */
/* the same code).                                                           */
/* ------------------------------------------------------------------------ */

/* XorShift64::next (run.rs:271-276): x ^= x << 13; x ^= x >> 7; x ^= x << 17.
 * The state is seeded with max(seed, 1) (run.rs:270). */
uint64_t orc_xorshift64_next(uint64_t* state) {
    uint64_t x = *state;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *state = x;
    return x;
}

/* XorShift64::next_f32 (run.rs:277): the top 24 bits over 2^24 (exact). */
float orc_xorshift64_next_f32(uint64_t* state) {
    return (float)(orc_xorshift64_next(state) >> 40) / 16777216.0f;
}

/* Iterator::max_by(|a, b| a.partial_cmp(b).unwrap_or(Equal)) over v[0..n),
 * returning the index (run.rs:232-234, :248-250): the fold keeps the current
 * element only when it compares Greater, so equal maxima resolve to the last
 * and a NaN (Equal to everything) takes over and hands over to the next.
 * Empty input: 0 (unwrap_or(0)). */
uint32_t orc_argmax(const float* v, size_t n) {
    size_t cur = 0;
    for (size_t i = 1; i < n; i++)
        if (!(v[cur] > v[i])) cur = i;
    return (uint32_t)cur;
}

typedef struct {
    size_t i;
    float v;
} orc_iv;

/* sort_unstable_by(|a, b| b.1.partial_cmp(&a.1).unwrap_or(Equal)): descending;
 * the order among equal values is immaterial (equal values add equal terms),
 * ties broken by index here only to make qsort's output reproducible. */
static int orc_cmp_desc(const void* pa, const void* pb) {
    const orc_iv* a = (const orc_iv*)pa;
    const orc_iv* b = (const orc_iv*)pb;
    if (b->v < a->v) return -1;
    if (b->v > a->v) return 1;
    return a->i < b->i ? -1 : (a->i > b->i ? 1 : 0);
}

/* The fp32 sum of probs in index order (probs.iter().sum(): a fold from
 * -0.0 in current Rust, 0.0 in older; only the sign of a zero sum differs,
 * which no later step can see). */
static float orc_sum_f32(const float* p, size_t n) {
    float s = -0.0f;
    for (size_t i = 0; i < n; i++) s += p[i];
    return s;
}

/* sample_token (run.rs:203-251), step by step.  exp is the platform's expf,
 * as Rust's f32::exp calls it. */
uint32_t orc_sample_token(const float* logits, size_t n, float temperature, float top_p,
                          size_t top_k, uint64_t* state) {
    float* probs = (float*)malloc((n ? n : 1) * sizeof(float));
    orc_iv* idx = (orc_iv*)malloc((n ? n : 1) * sizeof(orc_iv));
    uint32_t out;
    memcpy(probs, logits, n * sizeof(float));
    if (temperature > 0.0f) {
        const float inv_temp = 1.0f / temperature;
        for (size_t i = 0; i < n; i++) probs[i] = expf(probs[i] * inv_temp);
    }
    if (top_k > 0 && top_k < n) {
        for (size_t i = 0; i < n; i++) { idx[i].i = i; idx[i].v = probs[i]; }
        qsort(idx, n, sizeof(orc_iv), orc_cmp_desc);
        const float threshold = idx[top_k - 1].v;
        for (size_t i = 0; i < n; i++)
            if (probs[i] < threshold) probs[i] = 0.0f;
    }
    if (top_p < 1.0f) {
        for (size_t i = 0; i < n; i++) { idx[i].i = i; idx[i].v = probs[i]; }
        qsort(idx, n, sizeof(orc_iv), orc_cmp_desc);
        const float sum = orc_sum_f32(probs, n);
        if (sum > 0.0f) {
            float cumsum = 0.0f;
            float threshold = 3.40282347e+38f; /* f32::MAX */
            for (size_t j = 0; j < n; j++) {
                cumsum += idx[j].v / sum;
                if (cumsum > top_p) { threshold = idx[j].v; break; }
            }
            for (size_t i = 0; i < n; i++)
                if (probs[i] < threshold) probs[i] = 0.0f;
        }
    }
    const float sum = orc_sum_f32(probs, n);
    if (sum <= 0.0f) {
        out = orc_argmax(logits, n);
    } else {
        const float r = orc_xorshift64_next_f32(state);
        float cumsum = 0.0f;
        out = UINT32_MAX;
        for (size_t i = 0; i < n; i++) {
            cumsum += probs[i] / sum;
            if (r < cumsum) { out = (uint32_t)i; break; }
        }
        if (out == UINT32_MAX) out = orc_argmax(probs, n);
    }
    free(probs);
    free(idx);
    return out;
}
