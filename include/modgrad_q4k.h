/*
 * modgrad_q4k -- MI355X (gfx950) Q4_K quantized matvec, C ABI.
 *
 * Drop-in for the Q4_K kernel ABI of rotkonetworks/modgrad: the first group of
 * entry points has exactly the names, argument order and types that the
 * reference's Rust host declares in its `unsafe extern "C"` block
 * (crates/modgrad-device/src/backend/rocm.rs:433-563), so that block links
 * against libmodgrad_q4k unchanged. The remaining entry points are additive.
 *
 * Conventions (kept from the reference, matvec_q4k.hip:110-124):
 *   - every pointer is a device pointer owned by the caller; launchers never
 *     allocate caller-visible memory and never synchronize;
 *   - reference-compatible launchers enqueue on the null stream; the *_ex
 *     variants take an explicit hipStream_t;
 *   - the return value is a hipError_t (0 = hipSuccess); non-positive sizes
 *     return hipErrorInvalidValue and enqueue nothing;
 *   - quantized weight bytes and int8 activations may start at any byte
 *     address, as the reference's byte-reading kernels allow (its engine
 *     packs tensors back to back, rocm_gemma.rs:214-215); the same kernels
 *     run at every offset. Float pointers need 4-byte alignment and f16
 *     pointers 2-byte (hipErrorInvalidValue otherwise).
 *
 * Q4_K super-block (144 bytes, 256 weights): +0 d:f16, +2 dmin:f16,
 * +4 scales[12] (6-bit scale/min pairs), +16 qs[128] (4-bit quants).
 * Element order is ggml's (canonical): position p of a block belongs to
 * sub-block p/32 and reads the low (p/32 even) or high nibble of
 * qs[32*(p/64) + p%32]; w = d*sc*q - dmin*m.
 */
#ifndef MODGRAD_Q4K_H
#define MODGRAD_Q4K_H

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------------------
 * Reference-compatible entry points
 * ------------------------------------------------------------------------ */

/* Replaces launch_dequant_q4k (decl rocm.rs:447-451, def
 * kernels/dequant_q4k.hip:147-157). Dequantizes n_blocks*144 bytes into
 * n_blocks*256 floats in canonical order, bit-identical to the reference host
 * dequantizer dequantize_row_q4_k (kfd/gguf.rs:364-404): each weight is
 * fl(fl(d*sc)*q) - fl(dmin*m), never fused. (The reference's own GPU kernel
 * writes the legacy all-low-then-all-high order instead; this one follows the
 * host spec.) n_blocks <= 0 -> hipErrorInvalidValue. */
hipError_t launch_dequant_q4k(const unsigned char *q4k, int n_blocks, float *fp32_out);

/* Replaces launch_matvec_q4k (decl rocm.rs:457-463, def
 * kernels/matvec_q4k.hip:111-124). y[r] = sum_k dequant(W)[r][k] * x[k],
 * W row-aligned: row r starts at byte r*blocks_per_row*144, x has
 * blocks_per_row*256 floats, y has out_dim floats. f32 accumulation;
 * |y - y_f64| <= 1e-4 * sum_k |w_rk||x_k| per row.
 * out_dim <= 0 or blocks_per_row <= 0 -> hipErrorInvalidValue. */
hipError_t launch_matvec_q4k(const unsigned char *w_q4, const float *x, float *y,
                             int out_dim, int blocks_per_row);

/* Replaces launch_quantize_q8_1 (decl rocm.rs:477, def
 * kernels/matvec_q4k_dp4a.hip:29-55): the int8 activations of the dp4a path.
 * For each of the n/32 sub-blocks s (trailing n%32 values are ignored, as in
 * the reference): xd[s] = amax/127, xq = clamp(rint(x*127/amax), -127, 127)
 * (round half to even), xsum[s] = sum of the 32 xq; amax = 0, or a scale whose
 * inverse is not finite, gives an all-zero sub-block. Bit-identical to the
 * reference. n < 32 -> hipErrorInvalidValue. */
hipError_t launch_quantize_q8_1(const float *x, signed char *xq, float *xd, float *xsum, int n);

/* Replaces launch_matvec_q4k_dp4a (decl rocm.rs:478-479, def
 * kernels/matvec_q4k_dp4a.hip:52-116): y[r] = sum over sub-blocks s of
 * xd[s]*(d*sc_s*isum_s - dmin*m_s*xsum[s]), isum_s = sum of nibble*xq over the
 * sub-block (exact integer dot, canonical order); a non-finite row result is
 * written as 0, as the reference does. xq/xd/xsum as produced by
 * launch_quantize_q8_1 for x of blocks_per_row*256 values. Its accuracy
 * against the f32 matvec is the int8 quantization's (the reference accepts
 * RMS-relative error < 0.02, examples/rocm_dp4a_check.rs:63). */
hipError_t launch_matvec_q4k_dp4a(const unsigned char *w, const signed char *xq, const float *xd,
                                  const float *xsum, float *y, int out_dim, int bpr);

/* Replace launch_matvec_q5k (decl rocm.rs:467-472, def kernels/matvec_q5k.hip)
 * and launch_matvec_q6k (decl rocm.rs:482-485, def kernels/matvec_q6k.hip):
 * the same matvec for Q5_K (176 B per 256 weights) and Q6_K (210 B) rows,
 * canonical order as dequantize_row_q5_k / dequantize_row_q6_k
 * (gguf.rs:419-477); same per-row tolerance as launch_matvec_q4k. */
hipError_t launch_matvec_q5k(const unsigned char *w_q5, const float *x, float *y, int out_dim,
                             int blocks_per_row);
hipError_t launch_matvec_q6k(const unsigned char *w_q6, const float *x, float *y, int out_dim,
                             int blocks_per_row);

/* Replaces launch_matvec_q6k_dp4a (decl rocm.rs:490-491, def
 * kernels/matvec_q6k_dp4a.hip): Q6_K rows on launch_quantize_q8_1's output,
 * y[r] = sum_s xd[s]*d*(sc_lo*isum_lo + sc_hi*isum_hi) over the two 16-value
 * halves of each sub-block (exact integer dots; xsum is not used, as in the
 * reference, and no non-finite clamp is applied). */
hipError_t launch_matvec_q6k_dp4a(const unsigned char *w, const signed char *xq, const float *xd,
                                  const float *xsum, float *y, int out_dim, int bpr);

/* ---------------------------------------------------------------------------
 * Additive entry points (no counterpart in the reference unless noted)
 * ------------------------------------------------------------------------ */

/* Layout of the weight bytes for launch_matvec_q4k_ex. */
#define MGQ_LAYOUT_ROWS 0 /* GGUF row-aligned: k_elems % 256 == 0 */
#define MGQ_LAYOUT_FLAT 1 /* flattened [out_dim x k_elems] tensor quantized as one
                             stream (LinearResidentQuantized, neuron.rs:931-951):
                             element (r,c) is flat index r*k_elems+c, in block
                             idx/256 at position idx%256; needs
                             out_dim*k_elems % 256 == 0 */

/* launch_matvec_q4k with an explicit stream and either layout. For
 * MGQ_LAYOUT_ROWS it computes the same function as launch_matvec_q4k with
 * blocks_per_row = k_elems/256. */
hipError_t launch_matvec_q4k_ex(const unsigned char *w_q4, const float *x, float *y,
                                int out_dim, int k_elems, int layout,
                                hipStream_t stream);

/* launch_quantize_q8_1 / launch_matvec_q4k_dp4a with an explicit stream. */
hipError_t launch_quantize_q8_1_ex(const float *x, signed char *xq, float *xd, float *xsum, int n,
                                   hipStream_t stream);
hipError_t launch_matvec_q4k_dp4a_ex(const unsigned char *w, const signed char *xq,
                                     const float *xd, const float *xsum, float *y, int out_dim,
                                     int bpr, hipStream_t stream);

/* launch_quantize_q8_1 followed by launch_matvec_q4k_dp4a, in one launch: the
 * matvec quantizes x (blocks_per_row*256 f32) to Q8_1 itself, with the same
 * steps as launch_quantize_q8_1, so y is bit-identical to the two-launch
 * sequence (rocm_gemma.rs:298-306) while x, xq, xd and xsum never go to
 * memory. hipErrorNotSupported when K exceeds the kernel's LDS staging. */
hipError_t launch_quantize_matvec_q4k_dp4a_ex(const unsigned char *w, const float *x, float *y,
                                              int out_dim, int bpr, hipStream_t stream);

/* launch_matvec_q5k / launch_matvec_q6k / launch_matvec_q6k_dp4a with an
 * explicit stream. */
hipError_t launch_matvec_q5k_ex(const unsigned char *w_q5, const float *x, float *y, int out_dim,
                                int blocks_per_row, hipStream_t stream);
hipError_t launch_matvec_q6k_ex(const unsigned char *w_q6, const float *x, float *y, int out_dim,
                                int blocks_per_row, hipStream_t stream);
hipError_t launch_matvec_q6k_dp4a_ex(const unsigned char *w, const signed char *xq,
                                     const float *xd, const float *xsum, float *y, int out_dim,
                                     int bpr, hipStream_t stream);

/* launch_dequant_q4k with an explicit stream. */
hipError_t launch_dequant_q4k_ex(const unsigned char *q4k, int n_blocks, float *fp32_out,
                                 hipStream_t stream);

/* Batched matvec for multi-sequence decode: Y[b][r] = dequant(W)[r] . X[b] for
 * b < batch (1..16). X is [batch][blocks_per_row*256] f32 row-major, Y is
 * [batch][out_dim] f32. Each super-block is decoded once and reused across
 * the batch (on the matrix cores, batch rows on the MFMA M dimension). Same
 * per-(b,r) tolerance as launch_matvec_q4k.
 * `workspace` is caller-owned device memory of at least
 * mgq_batched_workspace_bytes(blocks_per_row, batch) bytes, 16-byte aligned;
 * it holds X converted to matrix-core operands for the duration of the call,
 * so calls that may overlap need distinct workspaces. A smaller or null
 * workspace -> hipErrorInvalidValue. Y must not overlap X, W or the
 * workspace: for long K and few rows the call zeroes Y first and adds two
 * K-half partials into it (bit-identical from call to call). */
size_t mgq_batched_workspace_bytes(int blocks_per_row, int batch);
hipError_t launch_matvec_q4k_batched(const unsigned char *w_q4, const float *X, float *Y,
                                     int out_dim, int blocks_per_row, int batch,
                                     void *workspace, size_t workspace_bytes,
                                     hipStream_t stream);

/* No counterpart in the reference. launch_matvec_q4k_batched without a
 * workspace argument and without any device allocation, for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). The operand table lives in a fixed
 * MGQ_NOALLOC_SCRATCH_BYTES array of the library on each GPU (held until
 * the process ends; its device address is looked up once per device, by
 * mgq_prepare or the first call). Same results as launch_matvec_q4k_batched
 * with a workspace. Shapes whose workspace
 * (mgq_batched_workspace_bytes) exceeds the array return
 * hipErrorInvalidValue: up to blocks_per_row 451 for batch <= 8, 225 for
 * batch <= 16. Calls on one GPU share the array: calls that may overlap (on
 * unordered streams) race and must not be issued. */
#define MGQ_NOALLOC_SCRATCH_BYTES ((size_t)4 << 20)
hipError_t launch_matvec_q4k_batched_noalloc(const unsigned char *w_q4, const float *X, float *Y,
                                             int out_dim, int blocks_per_row, int batch,
                                             hipStream_t stream);

/* Prefill dequant-GEMM: C[m][r] = sum_k dequant(W)[r][k] * A[m][k] for
 * m < m_tokens, with A f16 [m_tokens][blocks_per_row*256] (IEEE half bits)
 * and C f32 [m_tokens][out_dim]. Weights are dequantized to f16 tiles and
 * multiplied on the gfx950 matrix cores with f32 accumulation. */
hipError_t launch_gemm_q4k_f16(const unsigned char *w_q4, const uint16_t *a_f16, float *c,
                               int out_dim, int blocks_per_row, int m_tokens,
                               hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Decode glue (kernels/rms_norm.hip, kernels/transformer_ops.hip) and its
 * fusion into the Q4_K matvec.
 * ------------------------------------------------------------------------- */

/* Replaces launch_rms_norm (decl rocm.rs:435-445, def kernels/rms_norm.hip:
 * 79-95): y[r][c] = x[r][c] * rstd * weight[c] for r < n rows of `hidden`,
 * rstd = 1/sqrt(mean(x[r]^2) + eps). The sum of squares follows the
 * reference kernel's order; the result matches it to an ulp of rsqrt.
 * hipErrorInvalidValue for n <= 0, hidden <= 0 or a null pointer. */
hipError_t launch_rms_norm(const float *x, const float *weight, float *y, int n, int hidden,
                           float eps);
hipError_t launch_rms_norm_ex(const float *x, const float *weight, float *y, int n, int hidden,
                              float eps, hipStream_t stream);

/* Replaces launch_geglu (decl rocm.rs:505, def kernels/transformer_ops.hip:
 * 32-46): out[i] = gelu_tanh(gate[i]) * up[i]. */
hipError_t launch_geglu(const float *gate, const float *up, float *out, int n);

/* GLU activations for launch_glu_ex / launch_matvec_q4k_glu_ex. */
#define MGQ_ACT_GELU_TANH 0 /* the reference's geglu */
#define MGQ_ACT_SILU 1      /* v * sigmoid(v) (SwiGLU); no counterpart in the reference */

/* out[i] = act(gate[i]) * up[i] on `stream`. */
hipError_t launch_glu_ex(const float *gate, const float *up, float *out, int n, int act,
                         hipStream_t stream);

/* Replaces launch_residual_add (decl rocm.rs:503, def kernels/
 * transformer_ops.hip:10-19): h[i] += x[i] for i < n. Also the bias add of
 * the resident linear layer (hipblasSgemv's beta = 1 on a bias-filled y,
 * rocm.rs:2000-2056). hipErrorInvalidValue for n <= 0 or a null pointer. */
hipError_t launch_residual_add(float *h, const float *x, int n);
hipError_t launch_residual_add_ex(float *h, const float *x, int n, hipStream_t stream);

/* Replaces launch_scale (decl rocm.rs:504, def kernels/transformer_ops.hip:
 * 21-30): h[i] *= s for i < n. hipErrorInvalidValue for n <= 0 or null h. */
hipError_t launch_scale(float *h, float s, int n);
hipError_t launch_scale_ex(float *h, float s, int n, hipStream_t stream);

/* Fused RMSNorm -> Q4_K matvec: y = W * rms_norm(x, norm_w, eps) for one
 * activation row of K = blocks_per_row*256, replacing the reference decode's
 * launch_rms_norm + launch_matvec_q4k pair (rocm_gemma.rs:439-440, 477-478).
 * Computed as rstd * (W * (x .* norm_w)): the matvec's activation staging
 * multiplies by norm_w and reduces sum(x^2) on the way, so the normalized
 * vector never goes to memory. Same per-row bound as launch_matvec_q4k
 * against the f64 matvec of the normalized vector. hipErrorNotSupported when
 * K exceeds the kernel's LDS staging (blocks_per_row > ~110). */
hipError_t launch_matvec_q4k_rmsnorm_ex(const unsigned char *w_q4, const float *x,
                                        const float *norm_w, float eps, float *y, int out_dim,
                                        int blocks_per_row, hipStream_t stream);

/* Fused RMSNorm -> Q6_K matvec: y = W * rms_norm(x, norm_w, eps), replacing
 * the reference decode's launch_rms_norm + launch_matvec_q6k pair where a
 * Q4_K_M model's Q6_K tensors follow a norm (attn_v on its 'more bits'
 * layers, the output matrix; rocm_gemma.rs:439-440 with the dtype dispatch
 * of rocm_gemma.rs:291-309). No counterpart in the reference as one call.
 * Computed as rstd * (W * (x .* norm_w)) on the matrix-core kernel, whose
 * activation staging multiplies by norm_w and reduces sum(x^2). Same per-row
 * bound as launch_matvec_q6k against the f64 matvec of the normalized
 * vector. Runs on the whole-row kernel only: hipErrorNotSupported unless w
 * is 16-byte aligned, out_dim * blocks_per_row * 210 is a multiple of 16 and
 * blocks_per_row <= 14 (K <= 3584); callers then keep the two launches. */
hipError_t launch_matvec_q6k_rmsnorm_ex(const unsigned char *w_q6, const float *x,
                                        const float *norm_w, float eps, float *y, int out_dim,
                                        int blocks_per_row, hipStream_t stream);

/* Fused gate/up matvec + GLU: y[i] = act(g[i]) * u[i] with g = W_gate * xn,
 * u = W_up * xn, xn = rms_norm(x, norm_w, eps) when norm_w is not null (else
 * xn = x). Replaces the reference FFN's launch_rms_norm + two
 * launch_matvec_q4k + launch_geglu (rocm_gemma.rs:477-481): one launch, and
 * gate/up never go to memory. W_gate and W_up are out_dim x blocks_per_row
 * row-aligned Q4_K. */
hipError_t launch_matvec_q4k_glu_ex(const unsigned char *w_gate, const unsigned char *w_up,
                                    const float *x, const float *norm_w, float eps, int act,
                                    float *y, int out_dim, int blocks_per_row,
                                    hipStream_t stream);

/* One matvec of a decode-step chain. */
typedef struct mgq_gemv_desc {
    const unsigned char *w_q4; /* row-aligned Q4_K bytes */
    const float *x;            /* blocks_per_row*256 f32 */
    float *y;                  /* out_dim f32 */
    int out_dim;
    int blocks_per_row;
} mgq_gemv_desc;

/* A decode step's matvecs as one launchable chain (the reference's per-layer
 * chain, rocm_gemma.rs:429-489). A launch runs the n matvecs with the
 * ordering of launching them one after another on a stream: matvec d sees
 * everything matvecs < d wrote (its x is typically an earlier y). A matvec's
 * y must not alias its own x or any weights. The chain keeps the
 * descriptors' pointers: buffers must outlive it.
 *
 * Three implementations:
 *   MGQ_CHAIN_PERSISTENT  one cooperative launch for the whole chain: a
 *       persistent kernel streams the next matvec's weights while it waits
 *       for the previous matvec's output (grid-wide completion counters
 *       behind agent-scope release/acquire fences). Row-aligned Q4_K with
 *       blocks_per_row <= 84. A launch is not
 *       capturable into a HIP graph, and launches of one chain must be
 *       ordered (one stream, or synchronized): the chain owns its counters.
 *       Measured on MI355X it is slower than the graph (one 15-wave
 *       work-group per CU streams weights at ~0.7x the standalone kernels'
 *       rate), so it is opt-in.
 *   MGQ_CHAIN_GRAPH       the n launch_matvec_q4k_ex launches recorded into
 *       a HIP graph (stream capture on a private stream).
 *   MGQ_CHAIN_EAGER       nothing recorded: every mgq_chain_launch enqueues
 *       the n launch_matvec_q4k_ex launches one after another on its
 *       stream, as the reference engine launches its kernels
 *       (rocm_gemma.rs:312-345); for callers that cannot keep a graph, and
 *       to measure that calling pattern.
 * MGQ_CHAIN_AUTO takes the graph (environment MGQ_CHAIN=persistent selects
 * the persistent kernel where it can run). MGQ_CHAIN_PERSISTENT returns
 * hipErrorNotSupported when it cannot run. */
#define MGQ_CHAIN_AUTO 0
#define MGQ_CHAIN_GRAPH 1
#define MGQ_CHAIN_PERSISTENT 2
#define MGQ_CHAIN_EAGER 3
hipError_t mgq_chain_create_ex(const mgq_gemv_desc *descs, int n, int mode, void **chain_out);
/* mgq_chain_create_ex with MGQ_CHAIN_AUTO. */
hipError_t mgq_chain_create(const mgq_gemv_desc *descs, int n, void **chain_out);
/* Launches the chain on `stream`; ordered after prior work on that stream. */
hipError_t mgq_chain_launch(void *chain, hipStream_t stream);
/* The chain's implementation (MGQ_CHAIN_GRAPH / _PERSISTENT / _EAGER) and,
 * for the persistent kernel, its fault word: nonzero when a grid-wide wait
 * gave up (bounded at seconds) in some launch, i.e. results are not to be
 * trusted. Reading it synchronizes with the device. Either pointer may be
 * null. */
hipError_t mgq_chain_info(void *chain, int *mode, unsigned *faults);
hipError_t mgq_chain_destroy(void *chain);

/* One kernel of a decode-step chain recorded by mgq_chain_create_ops: the
 * reference's per-layer sequence (rocm_gemma.rs:429-489, with the weight
 * type dispatch of RocmGemma::qmatvec, rocm_gemma.rs:291-309) for a real
 * GGUF mix of Q4_K, Q5_K and Q6_K tensors, including the fused glue matvecs.
 * Fields an op does not use are ignored (keep them zero/null).
 *
 *   MGQ_OP_MATVEC        y = W x; dtype Q4_K (layout MGQ_LAYOUT_ROWS or
 *                        MGQ_LAYOUT_FLAT, in_dim = K), Q5_K or Q6_K
 *                        (in_dim % 256 == 0); out_dim rows.
 *   MGQ_OP_MATVEC_NORM   y = W rms_norm(x, norm_w, eps); Q4_K, rows layout
 *                        (launch_matvec_q4k_rmsnorm_ex), or Q6_K where
 *                        launch_matvec_q6k_rmsnorm_ex runs (else
 *                        hipErrorNotSupported at creation).
 *   MGQ_OP_MATVEC_GLU    y = act(W xn) .* (W2 xn), xn = rms_norm(x, norm_w,
 *                        eps) when norm_w is not null, else x; Q4_K, rows
 *                        layout (launch_matvec_q4k_glu_ex).
 *   MGQ_OP_RMS_NORM      y = rms_norm(x, norm_w, eps) over `rows` rows of
 *                        in_dim (launch_rms_norm_ex).
 *   MGQ_OP_GLU           y = act(x) .* x2 over out_dim (launch_glu_ex).
 *   MGQ_OP_RESIDUAL_ADD  y += x over out_dim (launch_residual_add_ex).
 * The reference engine's default dp4a arm (rocm_gemma.rs:283,298-306;
 * rocm.rs:477-479,490-491):
 *   MGQ_OP_QUANTIZE_Q8_1 x (in_dim f32, in_dim % 32 == 0) -> Q8_1 xq, xd, xsum
 *                        (launch_quantize_q8_1_ex).
 *   MGQ_OP_MATVEC_DP4A   y = W . Q8_1(xq, xd, xsum); dtype Q4_K
 *                        (launch_matvec_q4k_dp4a_ex) or Q6_K
 *                        (launch_matvec_q6k_dp4a_ex), in_dim = K.
 *   MGQ_OP_QUANTIZE_MATVEC_DP4A  the two above in one launch for Q4_K
 *                        (launch_quantize_matvec_q4k_dp4a_ex: y from x, same
 *                        bits; xq/xd/xsum unused).
 * No counterpart in the reference's C ABI: its chain is Rust code that
 * launches these kernels one by one; this records them into one graph. */
#define MGQ_OP_MATVEC 0
#define MGQ_OP_MATVEC_NORM 1
#define MGQ_OP_MATVEC_GLU 2
#define MGQ_OP_RMS_NORM 3
#define MGQ_OP_GLU 4
#define MGQ_OP_RESIDUAL_ADD 5
#define MGQ_OP_QUANTIZE_Q8_1 6
#define MGQ_OP_MATVEC_DP4A 7
#define MGQ_OP_QUANTIZE_MATVEC_DP4A 8
/* GGML tensor types (gguf.rs:9-40) of the quantized weights */
#define MGQ_DTYPE_Q4_K 12
#define MGQ_DTYPE_Q5_K 13
#define MGQ_DTYPE_Q6_K 14
typedef struct mgq_op_desc {
    int op;                   /* MGQ_OP_* */
    int dtype;                /* MGQ_DTYPE_* (matvec ops) */
    int layout;               /* MGQ_LAYOUT_* (MGQ_OP_MATVEC on Q4_K) */
    int act;                  /* MGQ_ACT_* (GLU ops) */
    const unsigned char *w;   /* weights (the gate matrix for MGQ_OP_MATVEC_GLU) */
    const unsigned char *w2;  /* MGQ_OP_MATVEC_GLU: the up matrix */
    const float *x;           /* input */
    const float *x2;          /* MGQ_OP_GLU: the up vector */
    const float *norm_w;      /* RMSNorm weights */
    float *y;                 /* output (MGQ_OP_RESIDUAL_ADD: the accumulated h) */
    int out_dim;              /* matvec rows / elementwise length */
    int in_dim;               /* matvec K / RMSNorm row length */
    int rows;                 /* MGQ_OP_RMS_NORM: rows */
    float eps;                /* RMSNorm epsilon */
    signed char *xq;          /* Q8_1 ops: int8 activations [in_dim] */
    float *xd;                /* Q8_1 ops: scale per 32 activations [in_dim/32] */
    float *xsum;              /* Q8_1 ops: sum per 32 activations [in_dim/32] */
} mgq_op_desc;

/* A chain of mgq_op_desc kernels recorded into one HIP graph (the chain's
 * MGQ_CHAIN_GRAPH implementation; same launch/info/destroy calls and the
 * same ordering and lifetime rules as mgq_chain_create_ex). Every
 * descriptor is validated before any device call: hipErrorInvalidValue
 * names no device work; hipErrorNotSupported comes from an op whose fused
 * kernel cannot take the shape (e.g. MGQ_OP_MATVEC_NORM past its LDS
 * staging), and then no chain is created. */
hipError_t mgq_chain_create_ops(const mgq_op_desc *ops, int n, void **chain_out);

/* Prepares the current device: sets the GEMV kernels' LDS attributes, which
 * belong to a device (every launcher also does this on its first use on a
 * device), and looks up the device address of the fixed scratch array of
 * launch_matvec_q4k_batched_noalloc. Allocates nothing. Device memory the
 * library holds: that fixed array (used by that entry point only), and the
 * task table and completion counters that mgq_chain_create_ex allocates for
 * a persistent chain (MGQ_CHAIN_PERSISTENT), freed by mgq_chain_destroy.
 * Every other launcher allocates nothing and keeps no mutable device state,
 * so its launches on different streams may run concurrently. Safe to call
 * more than once. */
hipError_t mgq_prepare(void);

/* Library version string, e.g. "modgrad_q4k 0.1.0 gfx950". */
const char *mgq_version(void);

#ifdef __cplusplus
}
#endif
#endif /* MODGRAD_Q4K_H */
