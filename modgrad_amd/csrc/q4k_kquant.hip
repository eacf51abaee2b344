// Q5_K and Q6_K matvecs (real GGUFs mix K-quants per layer; the lm_head is
// often Q6_K). Same C ABI shape as the Q4_K matvec:
// launch_matvec_q5k / launch_matvec_q6k (rocm.rs:467-486; kernels
// matvec_q5k.hip, matvec_q6k.hip) and launch_matvec_q6k_dp4a (rocm.rs:490-491,
// kernels/matvec_q6k_dp4a.hip) on the Q8_1 activations of
// launch_quantize_q8_1.
//
// Formats (canonical ggml order, gguf.rs:419-477):
//   Q5_K, 176 B / 256 values: d, dmin f16 | scales[12] (Q4_K packing) |
//     qh[32] | ql[128]; q = nibble + 16*(bit j of qh[p%32]) for sub-block j.
//   Q6_K, 210 B / 256 values: ql[128] | qh[64] | int8 scales[16] | d f16;
//     q = (nibble | 2 qh bits << 4) - 32, one scale per 16 values.
//
// Vector-ALU kernels: one wavefront per row, lane l owns positions l, l+64,
// l+128, l+192 of every block, so each byte array of a block is read by the
// wavefront as consecutive bytes (coalesced), and the activations as
// consecutive floats. Q6_K blocks are only 2-byte aligned (210 B), which is
// why these kernels read bytes rather than staging 16-byte pieces.
#include "q4k_device.hpp"
#include "q4k_launch.hpp"

namespace mgq {

constexpr int kQ5Bytes = 176, kQ6Bytes = 210;

__device__ __forceinline__ float half_at(const uint8_t *p) {
    return half_bits_finite((uint32_t)p[0] | ((uint32_t)p[1] << 8));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// f32 activations. y[r] = sum_p w[r][p] * x[p] with w = (d*sc_j)*q - dmin*m_j.
__global__ __launch_bounds__(256) void gemv_q5k_kernel(const uint8_t *__restrict__ w,
                                                       const float *__restrict__ x,
                                                       float *__restrict__ y, int n, int bpr) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n) return;  // uniform per wavefront
    const uint8_t *wr = w + (size_t)row * bpr * kQ5Bytes;
    const int l31 = lane & 31, odd = lane >> 5;  // position l + 64k: sub-block odd + 2k
    float acc = 0.0f;
    for (int b = 0; b < bpr; ++b) {
        const uint8_t *blk = wr + (size_t)b * kQ5Bytes;
        const float d = half_at(blk), dmin = half_at(blk + 2);
        const uint8_t *s = blk + 4;
        const uint32_t qh = blk[16 + l31];
        const float *xb = x + (size_t)b * kBlockElems + lane;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int j = odd + 2 * k;
            uint32_t sc, m;
            if (j < 4) {
                sc = s[j] & 63u;
                m = s[j + 4] & 63u;
            } else {
                sc = (s[j + 4] & 15u) | ((uint32_t)(s[j - 4] >> 6) << 4);
                m = (uint32_t)(s[j + 4] >> 4) | ((uint32_t)(s[j] >> 6) << 4);
            }
            const uint32_t byte = blk[48 + 32 * k + l31];
            const uint32_t q = (odd ? (byte >> 4) : (byte & 15u)) + (((qh >> j) & 1u) << 4);
            const float wv = (d * (float)sc) * (float)q - dmin * (float)m;
            acc += wv * xb[64 * k];
        }
    }
    acc = wave_sum(acc);
    if (lane == 0) y[row] = acc;
}

__global__ __launch_bounds__(256) void gemv_q6k_kernel(const uint8_t *__restrict__ w,
                                                       const float *__restrict__ x,
                                                       float *__restrict__ y, int n, int bpr) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n) return;
    const uint8_t *wr = w + (size_t)row * bpr * kQ6Bytes;
    const int l31 = lane & 31, hi32 = lane >> 5;
    float acc = 0.0f;
    for (int b = 0; b < bpr; ++b) {
        const uint8_t *blk = wr + (size_t)b * kQ6Bytes;
        const float d = half_at(blk + 208);
        const int8_t *sc = reinterpret_cast<const int8_t *>(blk + 192);
        const float *xb = x + (size_t)b * kBlockElems + lane;
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            // positions 128g + lane (quad = hi32, low nibble) and
            // 128g + 64 + lane (quad = 2 + hi32, high nibble) share ql[64g + lane]
            const uint32_t qb = blk[64 * g + lane];
            const uint32_t hb = blk[128 + 32 * g + l31];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int quad = hi32 + 2 * h;
                const int q = (int)(((h ? (qb >> 4) : (qb & 15u)) | (((hb >> (2 * quad)) & 3u) << 4))) - 32;
                const float s = (float)sc[8 * g + (l31 >> 4) + 2 * quad];
                acc += (d * s) * (float)q * xb[128 * g + 64 * h];
            }
        }
    }
    acc = wave_sum(acc);
    if (lane == 0) y[row] = acc;
}

// Q6_K on Q8_1 activations: y[r] = sum_s xd[s]*d*(sc_lo*isum_lo + sc_hi*isum_hi),
// isum over the 16-value halves of sub-block s (exact integer dots). Lane l
// owns the same positions as above; the 16 lanes of a half combine their
// integer products with xor shuffles, so the dots stay exact.
__global__ __launch_bounds__(256) void gemv_q6k_q8_kernel(const uint8_t *__restrict__ w,
                                                          const int8_t *__restrict__ xq,
                                                          const float *__restrict__ xd,
                                                          float *__restrict__ y, int n, int bpr) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n) return;
    const uint8_t *wr = w + (size_t)row * bpr * kQ6Bytes;
    const int l31 = lane & 31, hi32 = lane >> 5;
    float acc = 0.0f;
    for (int b = 0; b < bpr; ++b) {
        const uint8_t *blk = wr + (size_t)b * kQ6Bytes;
        const float d = half_at(blk + 208);
        const int8_t *sc = reinterpret_cast<const int8_t *>(blk + 192);
        const int8_t *xb = xq + (size_t)b * kBlockElems + lane;
        float part = 0.0f;
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            const uint32_t qb = blk[64 * g + lane];
            const uint32_t hb = blk[128 + 32 * g + l31];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int quad = hi32 + 2 * h;
                const int q = (int)(((h ? (qb >> 4) : (qb & 15u)) | (((hb >> (2 * quad)) & 3u) << 4))) - 32;
                int prod = q * (int)xb[128 * g + 64 * h];
                // integer sum over the 16 lanes of this half (lanes 16c..16c+15)
                prod += __shfl_xor(prod, 1, 64);
                prod += __shfl_xor(prod, 2, 64);
                prod += __shfl_xor(prod, 4, 64);
                prod += __shfl_xor(prod, 8, 64);
                // sub-block 4g + quad, half (l31 >> 4): add once per half
                const int s32 = 4 * g + quad;
                if ((lane & 15) == 0)
                    part += xd[(size_t)b * 8 + s32] * d *
                            ((float)sc[8 * g + (l31 >> 4) + 2 * quad] * (float)prod);
            }
        }
        acc += part;
    }
    acc = wave_sum(acc);
    if (lane == 0) y[row] = acc;
}

hipError_t gemv_q5k_launch(const uint8_t *w, const float *x, float *y, int n, int bpr,
                           hipStream_t stream) {
    gemv_q5k_kernel<<<(unsigned)((n + 3) / 4), 256, 0, stream>>>(w, x, y, n, bpr);
    return hipGetLastError();
}

hipError_t gemv_q6k_launch(const uint8_t *w, const float *x, float *y, int n, int bpr,
                           hipStream_t stream) {
    gemv_q6k_kernel<<<(unsigned)((n + 3) / 4), 256, 0, stream>>>(w, x, y, n, bpr);
    return hipGetLastError();
}

hipError_t gemv_q6k_q8_launch(const uint8_t *w, const int8_t *xq, const float *xd, float *y,
                              int n, int bpr, hipStream_t stream) {
    gemv_q6k_q8_kernel<<<(unsigned)((n + 3) / 4), 256, 0, stream>>>(w, xq, xd, y, n, bpr);
    return hipGetLastError();
}

}  // namespace mgq
