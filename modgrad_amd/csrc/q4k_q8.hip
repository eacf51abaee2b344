// Q8_1 activation path (the reference's "dp4a" Q4_K matvec, the default of
// its resident Gemma engine): kernels/matvec_q4k_dp4a.hip:29-116.
//
// quantize_q8_1_kernel: per 32-value sub-block, d = amax/127, id = 127/amax,
// q = clamp(rint(x*id), -127, 127), xsum = sum q -- bit-identical to the
// reference (same IEEE-rounded divisions, round-half-even, and the
// non-finite-scale guard). Eight lanes per sub-block, four values each.
//
// gemv_q8_generic_kernel: the vector-ALU fallback of the dp4a matvec (any
// 4-byte alignment, any K). One wavefront per row; lanes take sub-blocks;
// v_dot4_i32_i8 on 4 nibbles x 4 int8 activations. The fast path is the
// matrix-core GEMV kernel's Q8 mode (q4k_gemv.hip).
#include "q4k_device.hpp"
#include "q4k_launch.hpp"

namespace mgq {

__global__ __launch_bounds__(256) void quantize_q8_1_kernel(const float *__restrict__ x,
                                                            int8_t *__restrict__ xq,
                                                            float *__restrict__ xd,
                                                            float *__restrict__ xsum, int nsub,
                                                            bool aligned16) {
    const int t = blockIdx.x * 256 + threadIdx.x;
    const int s = t >> 3, part = t & 7;  // sub-block, 4-value part
    const bool live = s < nsub;
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (live) {
        const float *xp = x + (size_t)s * 32 + part * 4;
        if (aligned16) {
            const f32x4 a = ld_f32x4(xp);
            v[0] = a[0]; v[1] = a[1]; v[2] = a[2]; v[3] = a[3];
        } else {
            v[0] = xp[0]; v[1] = xp[1]; v[2] = xp[2]; v[3] = xp[3];
        }
    }
    float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 4, 64));
    float d = __fdiv_rn(amax, 127.0f);
    float id = (amax > 0.0f) ? __fdiv_rn(127.0f, amax) : 0.0f;
    if (!isfinite(id)) {
        id = 0.0f;
        d = 0.0f;
    }
    int sum = 0;
    uint32_t packed = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // rint: round half to even; the float -> int conversion maps NaN to 0
        int q = (int)__builtin_rintf(__fmul_rn(v[i], id));
        q = max(-127, min(127, q));
        sum += q;
        packed |= (uint32_t)(q & 0xFF) << (8 * i);
    }
    sum += __shfl_xor(sum, 1, 64);
    sum += __shfl_xor(sum, 2, 64);
    sum += __shfl_xor(sum, 4, 64);
    if (!live) return;
    st_u32(xq + (size_t)s * 32 + part * 4, packed);
    if (part == 0) {
        xd[s] = d;
        xsum[s] = (float)sum;
    }
}

hipError_t quantize_q8_1_launch(const float *x, int8_t *xq, float *xd, float *xsum, int n,
                                hipStream_t stream) {
    const int nsub = n / 32;
    const unsigned grid = (unsigned)((nsub * 8 + 255) / 256);
    quantize_q8_1_kernel<<<grid, 256, 0, stream>>>(x, xq, xd, xsum, nsub,
                                                   ((uintptr_t)x & 15u) == 0);
    return hipGetLastError();
}

// dp4a matvec, vector ALU: y[r] = sum_s xd[s]*(d*sc_s*isum_s - dmin*m_s*xsum[s]).
__global__ __launch_bounds__(256) void gemv_q8_generic_kernel(const uint8_t *__restrict__ w,
                                                              const int8_t *__restrict__ xq,
                                                              const float *__restrict__ xd,
                                                              const float *__restrict__ xsum,
                                                              float *__restrict__ y, int n, int bpr) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n) return;  // uniform per wavefront
    const uint8_t *wr = w + (size_t)row * bpr * kBlockBytes;
    float acc = 0.0f;
    for (int s = lane; s < bpr * 8; s += 64) {
        const int blk = s >> 3, sub = s & 7;
        const uint8_t *b = wr + (size_t)blk * kBlockBytes;
        const uint32_t h0 = ld_u32(b);
        const float d = half_bits_finite(h0), dmin = half_bits_finite(h0 >> 16);
        uint32_t sc, m;
        scale_min(sub, ld_u32(b + 4), ld_u32(b + 8), ld_u32(b + 12), sc, m);
        const uint8_t *qs = b + 16 + (sub >> 1) * 32;
        const int8_t *xv = xq + (size_t)s * 32;
        const int shift = (sub & 1) * 4;
        int isum = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t nib = (ld_u32(qs + 4 * j) >> shift) & 0x0F0F0F0Fu;
            isum = __builtin_amdgcn_sdot4((int)nib, (int)ld_u32(reinterpret_cast<const uint8_t *>(xv) + 4 * j), isum,
                                          false);
        }
        acc += xd[s] * (d * (float)sc * (float)isum - dmin * (float)m * xsum[s]);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if (lane == 0) y[row] = isfinite(acc) ? acc : 0.0f;  // the reference's clamp
}

hipError_t gemv_q8_generic_launch(const uint8_t *w, const int8_t *xq, const float *xd,
                                  const float *xsum, float *y, int n, int bpr, hipStream_t stream) {
    gemv_q8_generic_kernel<<<(unsigned)((n + 3) / 4), 256, 0, stream>>>(w, xq, xd, xsum, y, n, bpr);
    return hipGetLastError();
}

}  // namespace mgq
