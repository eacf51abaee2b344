/*
 * CPU ORACLE for the Q4_K matvec path -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's Q4_K format code, quantizer,
 * seeded RNG, f64 dequant-dot GEMV and CPU fused GEMV. It exists to check the
 * HIP kernels and to time the reference CPU path; the product library never
 * links it. Build flags (oracle/Makefile): -O2 -ffp-contract=off
 * -fno-fast-math, so every f32 multiply and subtract rounds on its own, as
 * the Rust reference does.
 *
 * Parity pins for each function live in tests/test_oracle_pins.py; see the
 * per-function notes below for what pins it.
 */
#include "q4k_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif
#if defined(__x86_64__)
#include <immintrin.h>
#endif

/* ---------------------------------------------------------------- f16 ---- */

static inline float bits_to_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* gguf.rs:281-292. Subnormals are exact (mant/1024 * 2^-14, both exact);
 * exponent 31 (Inf and NaN alike) decodes to NaN. */
float orq_f16_to_f32(uint16_t h) {
    uint32_t sign = (h >> 15) & 1u;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t mant = h & 0x3FFu;
    if (exp == 0) {
        if (mant == 0) return sign ? -0.0f : 0.0f;
        float m = (float)mant / 1024.0f * (1.0f / 16384.0f);
        return sign ? -m : m;
    }
    if (exp == 31) return bits_to_f32(0x7FC00000u);
    return bits_to_f32((sign << 31) | ((exp + 112u) << 23) | (mant << 13));
}

/* gguf.rs:297-328. NOTE: truncates the mantissa (mant >> 13) rather than
 * rounding to nearest; subnormal results are truncated too. */
uint16_t orq_f32_to_f16(float f) {
    uint32_t bits = f32_to_bits(f);
    uint16_t sign = (uint16_t)((bits >> 31) & 1u);
    int32_t exp = (int32_t)((bits >> 23) & 0xFFu);
    uint32_t mant = bits & 0x7FFFFFu;
    if (exp == 0xFF) {
        uint16_t m = (uint16_t)(mant >> 13);
        uint16_t payload = mant != 0 ? (m > 1 ? m : 1) : 0;
        return (uint16_t)((sign << 15) | (0x1Fu << 10) | payload);
    }
    int32_t unbiased = exp - 127 + 15;
    if (unbiased >= 0x1F) return (uint16_t)((sign << 15) | (0x1Fu << 10));
    if (unbiased <= 0) {
        if (unbiased < -10) return (uint16_t)(sign << 15);
        uint32_t with_lead = mant | 0x800000u;
        uint32_t shift = (uint32_t)(14 - unbiased);
        return (uint16_t)((sign << 15) | (uint16_t)(with_lead >> shift));
    }
    return (uint16_t)((sign << 15) | ((uint16_t)unbiased << 10) | (uint16_t)(mant >> 13));
}

/* ------------------------------------------------------ scales / mins ---- */

/* gguf.rs:334-342 (6-bit scale/min of sub-block j from the 12-byte header). */
void orq_get_scale_min_k4(int j, const uint8_t *s, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* gguf.rs:349-358 (inverse of the above for values < 64). */
void orq_pack_scales_mins(const uint8_t sc[8], const uint8_t m[8], uint8_t s[12]) {
    for (int i = 0; i < 4; ++i) {
        s[i] = (uint8_t)((sc[i] & 0x3F) | (((sc[i + 4] >> 4) & 0x3) << 6));
        s[i + 4] = (uint8_t)((m[i] & 0x3F) | (((m[i + 4] >> 4) & 0x3) << 6));
        s[i + 8] = (uint8_t)((sc[i + 4] & 0x0F) | ((m[i + 4] & 0x0F) << 4));
    }
}

/* ------------------------------------------------------------ dequant ---- */

static inline float finite_or_zero(float v) { return isfinite(v) ? v : 0.0f; }

/* gguf.rs:364-404, canonical order: for each 32-byte group j of qs, 32
 * low-nibble outputs (sub-block 2j/32) then 32 high-nibble outputs. Each
 * weight is fl(fl(d*sc)*q) - fl(dmin*m): two roundings, never fused. */
void orq_dequantize_row_q4_k(const uint8_t *data, float *out, size_t out_len,
                             size_t n_blocks) {
    for (size_t blk = 0; blk < n_blocks; ++blk) {
        const uint8_t *b = data + blk * ORQ_BLOCK_BYTES;
        float d = finite_or_zero(orq_f16_to_f32((uint16_t)(b[0] | (b[1] << 8))));
        float dmin = finite_or_zero(orq_f16_to_f32((uint16_t)(b[2] | (b[3] << 8))));
        const uint8_t *scales = b + 4;
        const uint8_t *qs = b + 16;
        size_t out_idx = blk * ORQ_BLOCK_ELEMS;
        int is = 0;
        for (int j = 0; j < 128; j += 32) {
            uint8_t sc, m;
            orq_get_scale_min_k4(is, scales, &sc, &m);
            float d1 = d * (float)sc, m1 = dmin * (float)m;
            for (int l = 0; l < 32; ++l, ++out_idx)
                if (out_idx < out_len) out[out_idx] = d1 * (float)(qs[j + l] & 0xF) - m1;
            ++is;
            orq_get_scale_min_k4(is, scales, &sc, &m);
            float d2 = d * (float)sc, m2 = dmin * (float)m;
            for (int l = 0; l < 32; ++l, ++out_idx)
                if (out_idx < out_len) out[out_idx] = d2 * (float)(qs[j + l] >> 4) - m2;
            ++is;
        }
    }
}

/* ----------------------------------------------------------- quantize ---- */

/* Rust `f32::round().clamp(0,hi) as u8`: round half away from zero, clamp,
 * saturating cast (NaN -> 0). */
static inline uint8_t round_clamp_u8(float v, float hi) {
    float r = roundf(v);
    if (isnan(r)) return 0;
    if (r < 0.0f) r = 0.0f;
    if (r > hi) r = hi;
    return (uint8_t)r;
}

/* gguf.rs:509-529 (q4k_sub_block_local_scale_min). */
static void local_scale_min(const float *x, float *local_d, float *local_dmin) {
    float x_min = x[0], x_max = x[0];
    for (int i = 1; i < 32; ++i) {
        if (x[i] < x_min) x_min = x[i];
        if (x[i] > x_max) x_max = x[i];
    }
    if (x_min > 0.0f) x_min = 0.0f;
    *local_d = (x_max - x_min) / 15.0f;
    *local_dmin = -x_min;
}

/* gguf.rs:534-566 (quantize_sub_block). */
static void quantize_sub_block(const float *x, uint8_t *sc, uint8_t *m, uint8_t *q,
                               float super_d, float super_dmin) {
    float local_d, local_dmin;
    local_scale_min(x, &local_d, &local_dmin);
    float sc_f = super_d > 0.0f ? local_d / super_d : 0.0f;
    float m_f = super_dmin > 0.0f ? local_dmin / super_dmin : 0.0f;
    uint8_t sc_q = round_clamp_u8(sc_f, 63.0f), m_q = round_clamp_u8(m_f, 63.0f);
    *sc = sc_q;
    *m = m_q;
    float d1 = super_d * (float)sc_q;
    float m1 = super_dmin * (float)m_q;
    for (int i = 0; i < 32; ++i)
        q[i] = d1 > 0.0f ? round_clamp_u8((x[i] + m1) / d1, 15.0f) : 0;
}

/* gguf.rs:581-663 with its sub-block table (gguf.rs:601) as a parameter:
 * sub-block `is` reads x[OFFS[is] .. +32]. */
size_t orq_quantize_row_q4_k_offsets(const float *x, size_t n, uint8_t *out, const int *OFFS) {
    if (n % ORQ_BLOCK_ELEMS != 0) return 0;
    size_t n_blocks = n / ORQ_BLOCK_ELEMS;
    for (size_t blk = 0; blk < n_blocks; ++blk) {
        const float *bx = x + blk * ORQ_BLOCK_ELEMS;
        float super_d = 0.0f, super_dmin = 0.0f;
        for (int is = 0; is < 8; ++is) {
            float ld, ldm;
            local_scale_min(bx + OFFS[is], &ld, &ldm);
            if (ld > super_d) super_d = ld;
            if (ldm > super_dmin) super_dmin = ldm;
        }
        float sd = orq_f16_to_f32(orq_f32_to_f16(super_d / 63.0f));
        float sdm = orq_f16_to_f32(orq_f32_to_f16(super_dmin / 63.0f));
        uint8_t sc[8], m[8], nib[8][32];
        for (int is = 0; is < 8; ++is)
            quantize_sub_block(bx + OFFS[is], &sc[is], &m[is], nib[is], sd, sdm);
        uint8_t *dst = out + blk * ORQ_BLOCK_BYTES;
        uint16_t dh = orq_f32_to_f16(sd), dmh = orq_f32_to_f16(sdm);
        dst[0] = (uint8_t)(dh & 0xFF); dst[1] = (uint8_t)(dh >> 8);
        dst[2] = (uint8_t)(dmh & 0xFF); dst[3] = (uint8_t)(dmh >> 8);
        orq_pack_scales_mins(sc, m, dst + 4);
        for (int j = 0; j < 128; ++j) {
            int lo = (j / 32) * 2;
            dst[16 + j] = (uint8_t)((nib[lo][j % 32] & 0xF) | ((nib[lo + 1][j % 32] & 0xF) << 4));
        }
    }
    return n_blocks * ORQ_BLOCK_BYTES;
}

/* gguf.rs:581-663 as the reference ships it: the all-low-then-all-high table
 * of gguf.rs:590-601, so its bytes decode, in the canonical order above, to
 * a 32-element-chunk permutation of x. */
size_t orq_quantize_row_q4_k(const float *x, size_t n, uint8_t *out) {
    static const int OFFS[8] = {0, 128, 32, 160, 64, 192, 96, 224};
    return orq_quantize_row_q4_k_offsets(x, n, out, OFFS);
}

/* ---------------------------------------------------------------- RNG ---- */

/* neuron.rs:1345-1367. Box-Muller in f32 with the C library's logf/cosf/sqrtf
 * (what Rust's f32::ln/cos/sqrt lower to on Linux). */
void orq_rng_init(orq_rng *r, uint64_t seed) { r->s = seed + 1u; }
uint64_t orq_rng_next_u64(orq_rng *r) {
    r->s = r->s * 6364136223846793005ull + 1442695040888963407ull;
    return r->s;
}
float orq_rng_next_f32(orq_rng *r) {
    return (float)(orq_rng_next_u64(r) >> 40) / 16777216.0f;
}
float orq_rng_next_normal(orq_rng *r) {
    float u1 = orq_rng_next_f32(r);
    if (u1 < 1e-10f) u1 = 1e-10f;
    float u2 = orq_rng_next_f32(r);
    const float two_pi = 2.0f * 3.14159265358979323846f;
    return sqrtf(-2.0f * logf(u1)) * cosf(two_pi * u2);
}
/* State after `steps` LCG steps from s (affine map composed by squaring), so
 * a long fill can be split across threads and still be the one sequential
 * stream SimpleRng produces. */
static uint64_t lcg_skip(uint64_t s, uint64_t steps) {
    uint64_t A = 1, C = 0, a = 6364136223846793005ull, c = 1442695040888963407ull;
    while (steps) {
        if (steps & 1) { A = a * A; C = a * C + c; }
        c = a * c + c;
        a = a * a;
        steps >>= 1;
    }
    return A * s + C;
}

void orq_fill_normal(uint64_t seed, float scale, float *out, size_t n) {
    const size_t chunk = 1u << 16;
    const long long nchunks = (long long)((n + chunk - 1) / chunk);
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (long long ci = 0; ci < nchunks; ++ci) {
        size_t i0 = (size_t)ci * chunk, i1 = i0 + chunk < n ? i0 + chunk : n;
        orq_rng r;
        orq_rng_init(&r, seed);
        r.s = lcg_skip(r.s, 2u * (uint64_t)i0); /* two draws per normal */
        for (size_t i = i0; i < i1; ++i) out[i] = orq_rng_next_normal(&r) * scale;
    }
}

/* --------------------------------------------------------------- GEMV ---- */

/* rocm_matvec_check.rs:38-47: dequantize the row, accumulate w*x in f64,
 * round once to f32. absdot[r] = sum |w||x| (f64). */
void orq_gemv_f64_abs(const uint8_t *w, const float *x, float *y, double *absdot,
                      int out_dim, int bpr) {
    size_t k = (size_t)bpr * ORQ_BLOCK_ELEMS;
    float *wr = (float *)malloc(k * sizeof(float));
    for (int r = 0; r < out_dim; ++r) {
        orq_dequantize_row_q4_k(w + (size_t)r * bpr * ORQ_BLOCK_BYTES, wr, k, (size_t)bpr);
        double acc = 0.0, aabs = 0.0;
        for (size_t i = 0; i < k; ++i) {
            acc += (double)wr[i] * (double)x[i];
            aabs += fabs((double)wr[i]) * fabs((double)x[i]);
        }
        y[r] = (float)acc;
        if (absdot) absdot[r] = aabs;
    }
    free(wr);
}
void orq_gemv_f64(const uint8_t *w, const float *x, float *y, int out_dim, int bpr) {
    orq_gemv_f64_abs(w, x, y, NULL, out_dim, bpr);
}

void orq_gemv_flat_f64_abs(const uint8_t *w, const float *x, float *y,
                           double *absdot, int out_dim, int k_elems) {
    float blk[ORQ_BLOCK_ELEMS];
    long cur = -1;
    for (int r = 0; r < out_dim; ++r) {
        double acc = 0.0, aabs = 0.0;
        for (int c = 0; c < k_elems; ++c) {
            size_t f = (size_t)r * (size_t)k_elems + (size_t)c;
            long b = (long)(f / ORQ_BLOCK_ELEMS);
            if (b != cur) {
                orq_dequantize_row_q4_k(w + (size_t)b * ORQ_BLOCK_BYTES, blk,
                                        ORQ_BLOCK_ELEMS, 1);
                cur = b;
            }
            double wv = blk[f % ORQ_BLOCK_ELEMS];
            acc += wv * (double)x[c];
            aabs += fabs(wv) * fabs((double)x[c]);
        }
        y[r] = (float)acc;
        if (absdot) absdot[r] = aabs;
    }
}

/* gguf.rs:419-447 (dequantize_row_q5_k). */
void orq_dequantize_row_q5_k(const uint8_t *data, float *out, size_t out_len, size_t n_blocks) {
    for (size_t blk = 0; blk < n_blocks; ++blk) {
        const uint8_t *b = data + blk * ORQ_Q5K_BYTES;
        float d = orq_f16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
        float dmin = orq_f16_to_f32((uint16_t)(b[2] | (b[3] << 8)));
        if (!isfinite(d)) d = 0.0f;
        if (!isfinite(dmin)) dmin = 0.0f;
        const uint8_t *scales = b + 4, *qh = b + 16, *ql = b + 48;
        size_t out_idx = blk * ORQ_BLOCK_ELEMS;
        for (int grp = 0; grp < 4; ++grp) {
            uint8_t sc1, m1, sc2, m2;
            orq_get_scale_min_k4(2 * grp, scales, &sc1, &m1);
            orq_get_scale_min_k4(2 * grp + 1, scales, &sc2, &m2);
            const float d1 = d * (float)sc1, dm1 = dmin * (float)m1;
            const float d2 = d * (float)sc2, dm2 = dmin * (float)m2;
            const uint8_t u1 = (uint8_t)(1u << (2 * grp)), u2 = (uint8_t)(2u << (2 * grp));
            for (int l = 0; l < 32; ++l) {
                const int hbit = (qh[l] & u1) ? 16 : 0;
                const float q = (float)((ql[32 * grp + l] & 0xF) + hbit);
                if (out_idx < out_len) out[out_idx] = d1 * q - dm1;
                ++out_idx;
            }
            for (int l = 0; l < 32; ++l) {
                const int hbit = (qh[l] & u2) ? 16 : 0;
                const float q = (float)((ql[32 * grp + l] >> 4) + hbit);
                if (out_idx < out_len) out[out_idx] = d2 * q - dm2;
                ++out_idx;
            }
        }
    }
}

/* gguf.rs:450-477 (dequantize_row_q6_k). */
void orq_dequantize_row_q6_k(const uint8_t *data, float *out, size_t out_len, size_t n_blocks) {
    for (size_t blk = 0; blk < n_blocks; ++blk) {
        const uint8_t *b = data + blk * ORQ_Q6K_BYTES;
        const uint8_t *ql = b, *qh = b + 128;
        const int8_t *sc = (const int8_t *)(b + 192);
        float d = orq_f16_to_f32((uint16_t)(b[208] | (b[209] << 8)));
        if (!isfinite(d)) d = 0.0f;
        const size_t base = blk * ORQ_BLOCK_ELEMS;
        for (int grp = 0; grp < 2; ++grp) {
            const int qlb = grp * 64, qhb = grp * 32, scb = grp * 8;
            const size_t yb = base + (size_t)grp * 128;
            for (int l = 0; l < 32; ++l) {
                const int is = l / 16;
                const int q1 = ((ql[qlb + l] & 0xF) | ((qh[qhb + l] & 3) << 4)) - 32;
                const int q2 = ((ql[qlb + l + 32] & 0xF) | (((qh[qhb + l] >> 2) & 3) << 4)) - 32;
                const int q3 = ((ql[qlb + l] >> 4) | (((qh[qhb + l] >> 4) & 3) << 4)) - 32;
                const int q4 = ((ql[qlb + l + 32] >> 4) | (((qh[qhb + l] >> 6) & 3) << 4)) - 32;
                if (yb + l + 96 < out_len) {
                    out[yb + l] = d * (float)sc[scb + is] * (float)q1;
                    out[yb + l + 32] = d * (float)sc[scb + is + 2] * (float)q2;
                    out[yb + l + 64] = d * (float)sc[scb + is + 4] * (float)q3;
                    out[yb + l + 96] = d * (float)sc[scb + is + 6] * (float)q4;
                }
            }
        }
    }
}

void orq_gemv_kquant_f64_abs(int block_bytes, const uint8_t *w, const float *x, float *y,
                             double *absdot, int out_dim, int bpr) {
    size_t k = (size_t)bpr * ORQ_BLOCK_ELEMS;
    float *wr = (float *)malloc(k * sizeof(float));
    for (int r = 0; r < out_dim; ++r) {
        const uint8_t *row = w + (size_t)r * bpr * block_bytes;
        if (block_bytes == ORQ_Q5K_BYTES) orq_dequantize_row_q5_k(row, wr, k, (size_t)bpr);
        else if (block_bytes == ORQ_Q6K_BYTES) orq_dequantize_row_q6_k(row, wr, k, (size_t)bpr);
        else orq_dequantize_row_q4_k(row, wr, k, (size_t)bpr);
        double acc = 0.0, aabs = 0.0;
        for (size_t i = 0; i < k; ++i) {
            acc += (double)wr[i] * (double)x[i];
            aabs += fabs((double)wr[i]) * fabs((double)x[i]);
        }
        y[r] = (float)acc;
        if (absdot) absdot[r] = aabs;
    }
    free(wr);
}

/* kernels/matvec_q6k_dp4a.hip (matvec_q6k_dp4a_kernel), in f64. */
void orq_gemv_q6k_dp4a_f64(const uint8_t *w, const int8_t *xq, const float *xd, int out_dim,
                           int bpr, double *y, double *absterm) {
    for (int r = 0; r < out_dim; ++r) {
        const uint8_t *wrow = w + (size_t)r * bpr * ORQ_Q6K_BYTES;
        double acc = 0.0, aabs = 0.0;
        for (int s = 0; s < bpr * 8; ++s) {
            const int blk = s >> 3, sub = s & 7, g = sub >> 2, quad = sub & 3;
            const uint8_t *b = wrow + (size_t)blk * ORQ_Q6K_BYTES;
            float d = orq_f16_to_f32((uint16_t)(b[208] | (b[209] << 8)));
            if (!isfinite(d)) d = 0.0f;
            const uint8_t *ql = b + g * 64, *qh = b + 128 + g * 32;
            const int8_t *sc = (const int8_t *)(b + 192);
            const int sc_lo = sc[g * 8 + quad * 2], sc_hi = sc[g * 8 + 1 + quad * 2];
            const int8_t *xv = xq + (size_t)s * 32;
            long ilo = 0, ihi = 0;
            for (int l = 0; l < 32; ++l) {
                const uint8_t qb = ql[l + ((quad & 1) ? 32 : 0)];
                const int nib = (quad >> 1) ? (qb >> 4) : (qb & 0xF);
                const int q6 = (nib | (((qh[l] >> (2 * quad)) & 3) << 4)) - 32;
                if (l < 16) ilo += (long)q6 * xv[l]; else ihi += (long)q6 * xv[l];
            }
            const double t = (double)sc_lo * (double)ilo + (double)sc_hi * (double)ihi;
            acc += (double)xd[s] * (double)d * t;
            aabs += fabs((double)xd[s] * (double)d) *
                    (fabs((double)sc_lo * (double)ilo) + fabs((double)sc_hi * (double)ihi));
        }
        y[r] = acc;
        if (absterm) absterm[r] = aabs;
    }
}

/* kernels/matvec_q4k_dp4a.hip:29-50 (quantize_q8_1_kernel). */
void orq_quantize_q8_1(const float *x, int n, int8_t *xq, float *xd, float *xsum) {
    const int nsub = n / 32;
    for (int s = 0; s < nsub; ++s) {
        const float *xs = x + (size_t)s * 32;
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(xs[i]));
        float d = amax / 127.0f;
        float id = (amax > 0.0f) ? 127.0f / amax : 0.0f;
        if (!isfinite(id)) { id = 0.0f; d = 0.0f; }
        int sum = 0;
        for (int i = 0; i < 32; ++i) {
            const float p = xs[i] * id;
            const float r = rintf(p);
            /* float -> int as the GPU converts: NaN -> 0, saturating */
            int q = isnan(r) ? 0 : (r >= 2147483647.0f ? 2147483647 : (r <= -2147483648.0f ? (-2147483647 - 1) : (int)r));
            q = q < -127 ? -127 : (q > 127 ? 127 : q);
            xq[(size_t)s * 32 + i] = (int8_t)q;
            sum += q;
        }
        xd[s] = d;
        xsum[s] = (float)sum;
    }
}

/* kernels/matvec_q4k_dp4a.hip:52-106 (matvec_q4k_dp4a_kernel), in f64. */
void orq_gemv_q4k_dp4a_f64(const uint8_t *w, const int8_t *xq, const float *xd,
                           const float *xsum, int out_dim, int bpr, double *y,
                           double *absterm) {
    for (int r = 0; r < out_dim; ++r) {
        const uint8_t *wrow = w + (size_t)r * bpr * ORQ_BLOCK_BYTES;
        double acc = 0.0, aabs = 0.0;
        for (int s = 0; s < bpr * 8; ++s) {
            const int blk = s >> 3, sub = s & 7;
            const uint8_t *b = wrow + (size_t)blk * ORQ_BLOCK_BYTES;
            float dw = orq_f16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
            float dmw = orq_f16_to_f32((uint16_t)(b[2] | (b[3] << 8)));
            if (!isfinite(dw)) dw = 0.0f;
            if (!isfinite(dmw)) dmw = 0.0f;
            uint8_t sc, m;
            orq_get_scale_min_k4(sub, b + 4, &sc, &m);
            const int g = sub >> 1, hi = sub & 1;
            const uint8_t *qs = b + 16 + g * 32;
            const int8_t *xv = xq + (size_t)s * 32;
            long isum = 0;
            for (int l = 0; l < 32; ++l) {
                const int nib = hi ? (qs[l] >> 4) : (qs[l] & 15);
                isum += (long)nib * (long)xv[l];
            }
            const double t1 = (double)dw * (double)sc * (double)isum;
            const double t2 = (double)dmw * (double)m * (double)xsum[s];
            acc += (double)xd[s] * (t1 - t2);
            aabs += fabs((double)xd[s]) * (fabs(t1) + fabs(t2));
        }
        y[r] = isfinite(acc) ? acc : 0.0;
        if (absterm) absterm[r] = aabs;
    }
}

void orq_gemv_batched_f64_abs(const uint8_t *w, const float *X, float *Y,
                              double *absdot, int out_dim, int bpr, int batch) {
    size_t k = (size_t)bpr * ORQ_BLOCK_ELEMS;
    float *wr = (float *)malloc(k * sizeof(float));
    for (int r = 0; r < out_dim; ++r) {
        orq_dequantize_row_q4_k(w + (size_t)r * bpr * ORQ_BLOCK_BYTES, wr, k, (size_t)bpr);
        for (int b = 0; b < batch; ++b) {
            const float *xb = X + (size_t)b * k;
            double acc = 0.0, aabs = 0.0;
            for (size_t i = 0; i < k; ++i) {
                acc += (double)wr[i] * (double)xb[i];
                aabs += fabs((double)wr[i]) * fabs((double)xb[i]);
            }
            Y[(size_t)b * out_dim + r] = (float)acc;
            if (absdot) absdot[(size_t)b * out_dim + r] = aabs;
        }
    }
    free(wr);
}

void orq_gemm_f16_f64(const uint8_t *w, const uint16_t *a_f16, float *c,
                      double *absdot, int out_dim, int bpr, int m_tokens,
                      const int *rows, int n_rows) {
    size_t k = (size_t)bpr * ORQ_BLOCK_ELEMS;
    float *wr = (float *)malloc(k * sizeof(float));
    int nr = rows ? n_rows : out_dim;
    for (int ii = 0; ii < nr; ++ii) {
        int r = rows ? rows[ii] : ii;
        orq_dequantize_row_q4_k(w + (size_t)r * bpr * ORQ_BLOCK_BYTES, wr, k, (size_t)bpr);
        for (int m = 0; m < m_tokens; ++m) {
            const uint16_t *am = a_f16 + (size_t)m * k;
            double acc = 0.0, aabs = 0.0;
            for (size_t i = 0; i < k; ++i) {
                double av = orq_f16_to_f32(am[i]);
                acc += (double)wr[i] * av;
                aabs += fabs((double)wr[i]) * fabs(av);
            }
            c[(size_t)m * nr + ii] = (float)acc;
            if (absdot) absdot[(size_t)m * nr + ii] = aabs;
        }
    }
    free(wr);
}

/* ------------------------------------------------ CPU timing baseline ---- */

/* llm.rs:695-735 (dot_q4k_row_scalar): one sequential f32 accumulator over
 * the row, canonical order, dequantized weight then multiply-add (unfused). */
static float dot_row_scalar(const uint8_t *row, const float *x, int nb) {
    float acc = 0.0f;
    for (int blk = 0; blk < nb; ++blk) {
        const uint8_t *b = row + (size_t)blk * ORQ_BLOCK_BYTES;
        float d = finite_or_zero(orq_f16_to_f32((uint16_t)(b[0] | (b[1] << 8))));
        float dmin = finite_or_zero(orq_f16_to_f32((uint16_t)(b[2] | (b[3] << 8))));
        const float *xb = x + (size_t)blk * ORQ_BLOCK_ELEMS;
        for (int g = 0; g < 4; ++g) {
            for (int half = 0; half < 2; ++half) {
                uint8_t sc, m;
                orq_get_scale_min_k4(2 * g + half, b + 4, &sc, &m);
                float d1 = d * (float)sc, m1 = dmin * (float)m;
                const float *xs = xb + g * 64 + half * 32;
                for (int l = 0; l < 32; ++l) {
                    uint8_t byte = b[16 + g * 32 + l];
                    float wv = d1 * (float)(half ? (byte >> 4) : (byte & 0xF)) - m1;
                    acc += wv * xs[l];
                }
            }
        }
    }
    return acc;
}

#if defined(__x86_64__)
/* llm.rs:748-806 (dot_q4k_row_avx512): per sub-block, 32 nibbles widened to
 * two 16-lane f32 vectors, weights by fused q*scale - offset, then fused
 * multiply-add into two 16-lane accumulators; horizontal sum at the end. */
__attribute__((target("avx512f,avx512bw,fma")))
static float dot_row_avx512(const uint8_t *row, const float *x, int nb) {
    __m512 acc0 = _mm512_setzero_ps(), acc1 = _mm512_setzero_ps();
    const __m256i low4 = _mm256_set1_epi8(0x0F);
    for (int blk = 0; blk < nb; ++blk) {
        const uint8_t *b = row + (size_t)blk * ORQ_BLOCK_BYTES;
        float d = finite_or_zero(orq_f16_to_f32((uint16_t)(b[0] | (b[1] << 8))));
        float dmin = finite_or_zero(orq_f16_to_f32((uint16_t)(b[2] | (b[3] << 8))));
        const float *xb = x + (size_t)blk * ORQ_BLOCK_ELEMS;
        for (int g = 0; g < 4; ++g) {
            __m256i bytes = _mm256_loadu_si256((const __m256i *)(b + 16 + 32 * g));
            __m256i nibs[2] = {_mm256_and_si256(bytes, low4),
                               _mm256_and_si256(_mm256_srli_epi16(bytes, 4), low4)};
            for (int half = 0; half < 2; ++half) {
                uint8_t sc, m;
                orq_get_scale_min_k4(2 * g + half, b + 4, &sc, &m);
                __m512 vs = _mm512_set1_ps(d * (float)sc);
                __m512 vo = _mm512_set1_ps(dmin * (float)m);
                __m512 q0 = _mm512_cvtepi32_ps(_mm512_cvtepu8_epi32(_mm256_castsi256_si128(nibs[half])));
                __m512 q1 = _mm512_cvtepi32_ps(_mm512_cvtepu8_epi32(_mm256_extracti128_si256(nibs[half], 1)));
                const float *xs = xb + 64 * g + 32 * half;
                acc0 = _mm512_fmadd_ps(_mm512_fmsub_ps(q0, vs, vo), _mm512_loadu_ps(xs), acc0);
                acc1 = _mm512_fmadd_ps(_mm512_fmsub_ps(q1, vs, vo), _mm512_loadu_ps(xs + 16), acc1);
            }
        }
    }
    return _mm512_reduce_add_ps(_mm512_add_ps(acc0, acc1));
}
#endif

int orq_cpu_has_avx512(void) {
#if defined(__x86_64__)
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
           __builtin_cpu_supports("fma");
#else
    return 0;
#endif
}

/* llm.rs:468-534: y[r] = dot(row r) for every row, rows in parallel (rayon
 * par_iter there, OpenMP static schedule here). */
int orq_cpu_matvec_q4k(const uint8_t *w, const float *x, float *y, int out_dim,
                       int bpr, int threads) {
    int avx = orq_cpu_has_avx512();
    size_t row_bytes = (size_t)bpr * ORQ_BLOCK_BYTES;
#ifdef _OPENMP
    int nt = threads > 0 ? threads : omp_get_num_procs();
#pragma omp parallel for schedule(static) num_threads(nt)
#endif
    for (int r = 0; r < out_dim; ++r) {
        const uint8_t *row = w + (size_t)r * row_bytes;
#if defined(__x86_64__)
        y[r] = avx ? dot_row_avx512(row, x, bpr) : dot_row_scalar(row, x, bpr);
#else
        y[r] = dot_row_scalar(row, x, bpr);
#endif
    }
    (void)threads;
    return avx;
}

/* The smooth test signal of the reference's own Q4_K tests
 * (gguf.rs:703-738 and tests/dequant_q4k.rs:70-78):
 * t = i/n (f32); v = sin(7.3 t)*0.5 + cos(17.1 t)*0.2, all in f32. */
void orq_fill_smooth(float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        float t = (float)i / (float)n;
        out[i] = sinf(t * 7.3f) * 0.5f + cosf(t * 17.1f) * 0.2f;
    }
}

/* ------------------------------------------------------------- glue ---- */

/* kernels/rms_norm.hip:28-75 (one 256-thread block per row). */
void orq_rms_norm(const float *x, const float *w, float *y, int rows, int hidden, float eps) {
    float part[256];
    for (int r = 0; r < rows; ++r) {
        const float *xr = x + (size_t)r * hidden;
        float *yr = y + (size_t)r * hidden;
        for (int t = 0; t < 256; ++t) {
            float s = 0.0f;
            for (int c = t; c < hidden; c += 256) s = fmaf(xr[c], xr[c], s);
            part[t] = s;
        }
        for (int off = 128; off > 0; off >>= 1)
            for (int t = 0; t < off; ++t) part[t] += part[t + off];
        const float mean_sq = part[0] / (float)hidden;
        const float rstd = 1.0f / sqrtf(mean_sq + eps);
        for (int c = 0; c < hidden; ++c) yr[c] = xr[c] * rstd * w[c];
    }
}

/* kernels/transformer_ops.hip:32-40 (act 0); act 1 = silu. */
void orq_glu(const float *gate, const float *up, float *out, int n, int act) {
    for (int i = 0; i < n; ++i) {
        const float v = gate[i];
        float g;
        if (act == 1) {
            g = v / (1.0f + expf(-v));
        } else {
            const float c = 0.7978845608f * fmaf(0.044715f * v * v, v, v);
            g = 0.5f * v * (1.0f + tanhf(c));
        }
        out[i] = g * up[i];
    }
}
