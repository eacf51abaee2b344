// Prefill dequant-GEMM: C[m][r] = sum_k dequant(W)[r][k] * A[m][k], A f16.
// No counterpart in the reference (its prefill is a per-token GEMV loop,
// modgrad-gemma/examples/gemma4_rocm.rs:26-34).
//
// Simple correct kernel: one thread per (token, row) pair, weights decoded on
// the fly in canonical order, f32 accumulation.
#include "q4k_device.hpp"
#include "q4k_launch.hpp"

namespace mgq {

__global__ __launch_bounds__(256) void gemm_f16_simple_kernel(const uint8_t *__restrict__ w,
                                                              const uint16_t *__restrict__ a,
                                                              float *__restrict__ c, int n,
                                                              int bpr, int m_tokens) {
    const int r = blockIdx.x * 256 + threadIdx.x;
    const int m = blockIdx.y;
    if (r >= n || m >= m_tokens) return;
    const int k = bpr * kBlockElems;
    const uint8_t *wr = w + (size_t)r * bpr * kBlockBytes;
    const uint16_t *am = a + (size_t)m * k;
    float acc = 0.0f;
    for (int b = 0; b < bpr; ++b) {
        const uint8_t *blk = wr + (size_t)b * kBlockBytes;
        const uint32_t h0 = ld_u32(blk), s0 = ld_u32(blk + 4), s1 = ld_u32(blk + 8),
                       s2 = ld_u32(blk + 12);
        const float d = half_bits_finite(h0), dmin = half_bits_finite(h0 >> 16);
        for (int sb = 0; sb < 8; ++sb) {
            uint32_t sc, mn;
            scale_min(sb, s0, s1, s2, sc, mn);
            const float d1 = d * (float)sc, m1 = dmin * (float)mn;
            for (int l = 0; l < 32; ++l) {
                const uint8_t byte = blk[16 + 32 * (sb >> 1) + l];
                const uint32_t q = (sb & 1) ? (byte >> 4) : (byte & 15u);
                const float wv = d1 * (float)q - m1;
                const float av = (float)__builtin_bit_cast(_Float16, am[b * 256 + 32 * sb + l]);
                acc += wv * av;
            }
        }
    }
    c[(size_t)m * n + r] = acc;
}

hipError_t gemm_f16_launch(const uint8_t *w, const uint16_t *a, float *c, int n, int bpr,
                           int m_tokens, hipStream_t stream) {
    if (m_tokens > 65535) return hipErrorInvalidValue;
    dim3 grid((unsigned)((n + 255) / 256), (unsigned)m_tokens);
    gemm_f16_simple_kernel<<<grid, 256, 0, stream>>>(w, a, c, n, bpr, m_tokens);
    return hipGetLastError();
}

}  // namespace mgq
