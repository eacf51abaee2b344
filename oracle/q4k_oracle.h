/*
 * CPU ORACLE for the Q4_K matvec path -- TEST INFRASTRUCTURE ONLY.
 *
 * This library is the checker that the HIP kernels are compared against. Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it;
 * the product library (modgrad_amd/libmodgrad_q4k.so) never links or calls it.
 *
 * Every function restates one function of the reference
 * (rotkonetworks/modgrad, Rust) and cites the file:line it follows.
 * Floating-point code is compiled with -ffp-contract=off so that each
 * multiply and each subtract rounds separately, as Rust does.
 */
#ifndef MODGRAD_Q4K_ORACLE_H
#define MODGRAD_Q4K_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORQ_BLOCK_BYTES 144
#define ORQ_BLOCK_ELEMS 256

/* f16 helpers: crates/modgrad-device/src/kfd/gguf.rs:281-292 and :297-328 */
float orq_f16_to_f32(uint16_t h);
uint16_t orq_f32_to_f16(float f); /* truncating, as the reference does */

/* gguf.rs:334-342 and :349-358 */
void orq_get_scale_min_k4(int j, const uint8_t *scales, uint8_t *sc, uint8_t *m);
void orq_pack_scales_mins(const uint8_t sc[8], const uint8_t m[8], uint8_t scales[12]);

/* gguf.rs:364-404 -- canonical (ggml) element order. Writes n_blocks*256
 * floats, or fewer when out_len is smaller (the reference's bounds check). */
void orq_dequantize_row_q4_k(const uint8_t *data, float *out, size_t out_len,
                             size_t n_blocks);

/* gguf.rs:509-663 -- the reference's own quantizer (legacy sub-block order).
 * Returns bytes written, or 0 when n % 256 != 0 (the reference asserts). */
size_t orq_quantize_row_q4_k(const float *x, size_t n, uint8_t *out);
/* The same quantizer with the sub-block table of gguf.rs:601 given: offs[is]
 * is the first element of sub-block is ({0,32,..,224} is the one-line
 * canonical-order patch of that table). */
size_t orq_quantize_row_q4_k_offsets(const float *x, size_t n, uint8_t *out, const int *offs);

/* SimpleRng: crates/modgrad-compute/src/neuron.rs:1345-1367 */
typedef struct { uint64_t s; } orq_rng;
void orq_rng_init(orq_rng *r, uint64_t seed);
uint64_t orq_rng_next_u64(orq_rng *r);
float orq_rng_next_f32(orq_rng *r);
float orq_rng_next_normal(orq_rng *r);
/* Fill out[0..n) with scale * next_normal() (scale 1 -> plain normals). */
void orq_fill_normal(uint64_t seed, float scale, float *out, size_t n);

/* f64-accumulated dequant-dot GEMV:
 * crates/modgrad-device/examples/rocm_matvec_check.rs:38-47.
 * Row-aligned GGUF layout: row r at byte r*bpr*144, x has bpr*256 floats. */
void orq_gemv_f64(const uint8_t *w, const float *x, float *y, int out_dim, int bpr);
/* Same, and also returns sum_k |w_rk||x_k| per row (the tolerance scale). */
void orq_gemv_f64_abs(const uint8_t *w, const float *x, float *y, double *absdot,
                      int out_dim, int bpr);

/* Flat-stream layout (LinearResidentQuantized, neuron.rs:931-951 quantizes
 * the flattened [out x in] weight): element (r,c) is flat index r*K+c. */
void orq_gemv_flat_f64_abs(const uint8_t *w, const float *x, float *y,
                           double *absdot, int out_dim, int k_elems);

/* Batched: Y[b][r] = dequant(W)[r] . X[b], X is [B][K] row-major. */
void orq_gemv_batched_f64_abs(const uint8_t *w, const float *X, float *Y,
                              double *absdot, int out_dim, int bpr, int batch);

/* Prefill reference: C[m][r] = sum_k dequant(W)[r][k] * f16(A[m][k]), f64
 * accumulation, for the listed rows only (rows == NULL -> all). A holds IEEE
 * half bits. */
void orq_gemm_f16_f64(const uint8_t *w, const uint16_t *a_f16, float *c,
                      double *absdot, int out_dim, int bpr, int m_tokens,
                      const int *rows, int n_rows);

/* Q8_1 activation quantizer: kernels/matvec_q4k_dp4a.hip:29-50. Per 32-value
 * sub-block s < n/32: amax = max|x|, d = amax/127, id = amax > 0 ? 127/amax : 0
 * (non-finite id -> id = d = 0), q = clamp(rint(x*id), -127, 127) (round half
 * to even; a NaN product converts to 0, as the GPU's float->int conversion
 * does), xd[s] = d, xsum[s] = (float)sum q. */
void orq_quantize_q8_1(const float *x, int n, int8_t *xq, float *xd, float *xsum);

/* dp4a Q4_K matvec: kernels/matvec_q4k_dp4a.hip:52-106, evaluated in f64 with
 * the integer dots exact: y[r] = sum_s xd[s]*(dw*sc_s*isum_s - dmw*m_s*xsum[s]),
 * isum_s = sum of nibble*xq over the sub-block (canonical order); a
 * non-finite row result becomes 0 (the reference clamps it). absterm[r] =
 * sum_s |xd[s]|*(|dw*sc_s*isum_s| + |dmw*m_s*xsum[s]|), the scale of the
 * rounding any f32 evaluation of the same formula can add. */
void orq_gemv_q4k_dp4a_f64(const uint8_t *w, const int8_t *xq, const float *xd,
                           const float *xsum, int out_dim, int bpr, double *y,
                           double *absterm);

/* Q5_K (176 B / 256 values: d, dmin f16; scales[12]; qh[32]; ql[128]) and
 * Q6_K (210 B: ql[128]; qh[64]; int8 scales[16]; d f16) dequantizers:
 * gguf.rs:419-447 and :450-477. Canonical order. Same out_len bound as Q4_K. */
#define ORQ_Q5K_BYTES 176
#define ORQ_Q6K_BYTES 210
void orq_dequantize_row_q5_k(const uint8_t *data, float *out, size_t out_len, size_t n_blocks);
void orq_dequantize_row_q6_k(const uint8_t *data, float *out, size_t out_len, size_t n_blocks);

/* f64 dequant-dot GEMV for a row-aligned K-quant matrix of block size
 * block_bytes (144 = Q4_K, 176 = Q5_K, 210 = Q6_K): the reference's check
 * method (rocm_matvec_check.rs:38-47) with that format's dequantizer. */
void orq_gemv_kquant_f64_abs(int block_bytes, const uint8_t *w, const float *x, float *y,
                             double *absdot, int out_dim, int bpr);

/* Q6_K dp4a matvec: kernels/matvec_q6k_dp4a.hip (matvec_q6k_dp4a_kernel), in
 * f64 with exact integer dots: y[r] = sum_s xd[s]*d*(sc_lo*isum_lo +
 * sc_hi*isum_hi), the two 16-value halves of each 32-value sub-block s having
 * their own int8 scale; no xsum term (the q6 values are signed) and no
 * non-finite clamp. absterm as for orq_gemv_q4k_dp4a_f64. */
void orq_gemv_q6k_dp4a_f64(const uint8_t *w, const int8_t *xq, const float *xd, int out_dim,
                           int bpr, double *y, double *absterm);

/* Decode glue (kernels/rms_norm.hip:28-75, kernels/transformer_ops.hip:32-46).
 * orq_rms_norm: y[r][c] = (x[r][c] * rstd) * w[c], rstd = 1/sqrt(mean + eps);
 * the sum of squares in the reference kernel's order: thread t of 256 sums
 * fmaf(x, x, s) over c = t, t+256, ... (hipcc -O3 contracts `partial += v*v`),
 * then the pairwise tree t += t+128, t+64, ..., 1. The GPU's rsqrtf may
 * differ from 1/sqrtf by an ulp, so tests use a few-ulp bound.
 * orq_glu: out[i] = act(gate[i]) * up[i]; act 0 = gelu_tanh as the reference
 * writes it (the inner v + 0.044715*v*v*v contracted to one fma, as hipcc
 * does), act 1 = silu, v / (1 + exp(-v)). */
void orq_rms_norm(const float *x, const float *w, float *y, int rows, int hidden, float eps);
void orq_glu(const float *gate, const float *up, float *out, int n, int act);

/* CPU timing baseline: kfd::llm::matvec (llm.rs:468-534) with the fused
 * dequant-dot of llm.rs:684-806 (AVX-512 when the host has it, else scalar),
 * parallel over rows. threads <= 0 -> all cores. Returns 1 if AVX-512 used. */
int orq_cpu_matvec_q4k(const uint8_t *w, const float *x, float *y, int out_dim,
                       int bpr, int threads);
int orq_cpu_has_avx512(void);

/* The reference tests' smooth signal (gguf.rs:703-738). */
void orq_fill_smooth(float *out, size_t n);

#ifdef __cplusplus
}
#endif
#endif
