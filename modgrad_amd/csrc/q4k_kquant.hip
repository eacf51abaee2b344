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
// Vector-ALU kernels, one wavefront per row. gemv_q5k_kernel and
// gemv_q6k_q8_kernel read bytes: lane l owns positions l, l+64, l+128, l+192
// of every block, so each byte array of a block is read by the wavefront as
// consecutive bytes and the activations as consecutive floats; they serve any
// alignment. gemv_q6k_staged_kernel streams Q6_K rows as whole 16-byte
// chunks through LDS (the fallback behind the matrix-core Q6_K kernels).
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

// Q6_K on Q8_1 activations: y[r] = sum_s xd[s]*d*(sc_lo*isum_lo + sc_hi*isum_hi),
// isum over the 16-value halves of sub-block s (exact integer dots). Lane l
// owns positions l, l+64, l+128, l+192 of every block; the 16 lanes of a half
// combine their integer products with xor shuffles, so the dots stay exact.
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

// Q6_K, staged: one wavefront per row; the row streams through a wave-private
// LDS window SEG blocks at a time. A segment's bytes are loaded as whole
// 16-byte chunks from the 16-byte boundary at or below its start (every load
// instruction moves 1 KiB of consecutive bytes), the next segment's chunks are
// in flight while the current one is decoded, and no work-group barrier is
// involved. Decode: half-wave h takes block 2i+h of the segment, lane l'
// (0..31) one ql dword (bytes 4l'..4l'+3) and the matching qh dword, i.e. 8
// weights at positions P..P+3 and P+64..P+67 (P = 128g + 4(l'%16), g = l'/16),
// with scales sc[P/16] and sc[P/16 + 4]. Blocks are only 2-byte aligned, so a
// dword is read as the aligned pair around it (ds_read2_b32) and shifted into
// place (v_alignbyte_b32). y[r] = sum d*(sc_lo*(sum q x - 32 sum x) + ...).
// Takes any w (windows start at the 16-byte boundary at or below the
// segment) and float-aligned x; the tensor's last row, whose final chunk
// would reach past the tensor when its end is not 16-byte aligned, is decoded
// with byte loads instead.
constexpr int kQ6Seg = 14;  // blocks per segment: 2940 B window per wavefront

__global__ __launch_bounds__(256) void gemv_q6k_staged_kernel(const uint8_t *__restrict__ w,
                                                              const float *__restrict__ x,
                                                              float *__restrict__ y, int n,
                                                              int bpr) {
    constexpr int SEG = kQ6Seg;
    constexpr int WIN = SEG * kQ6Bytes + 32;   // segment bytes + alignment slack
    constexpr int CPL = (WIN / 16 + 63) / 64;  // 16-byte chunks per lane (3)
    __shared__ __attribute__((aligned(16))) uint8_t win_all[4][WIN];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int row = blockIdx.x * 4 + wv;
    if (row >= n) return;  // uniform per wavefront; no work-group barrier below
    uint8_t *win = win_all[wv];
    const size_t RB = (size_t)bpr * kQ6Bytes;
    const uint8_t *rp = w + (size_t)row * RB;
    const bool tail_row = (row == n - 1) && ((((uintptr_t)w + (size_t)n * RB) & 15u) != 0);
    const int l2 = lane & 31, h = lane >> 5, g = l2 >> 4, q0 = (l2 & 15) >> 3;
    float acc = 0.0f;
    if (tail_row) {  // byte loads (the tensor may end mid-chunk)
        for (int b = 0; b < bpr; ++b) {
            const uint8_t *blk = rp + (size_t)b * kQ6Bytes;
            const float d = half_at(blk + 208);
            const int8_t *sc = reinterpret_cast<const int8_t *>(blk + 192);
            const float *xb = x + (size_t)b * kBlockElems + lane;
#pragma unroll
            for (int gg = 0; gg < 2; ++gg) {
                const uint32_t qb = blk[64 * gg + lane], hb = blk[128 + 32 * gg + l2];
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const int quad = h + 2 * hh;
                    const int q = (int)(((hh ? (qb >> 4) : (qb & 15u)) | (((hb >> (2 * quad)) & 3u) << 4))) - 32;
                    acc += (d * (float)sc[8 * gg + (l2 >> 4) + 2 * quad]) * (float)q * xb[128 * gg + 64 * hh];
                }
            }
        }
        acc = wave_sum(acc);
        if (lane == 0) y[row] = acc;
        return;
    }
    const int nseg = (bpr + SEG - 1) / SEG;
    u32x4 reg[CPL];
    auto seg_base = [&](int s) { return rp + (size_t)s * SEG * kQ6Bytes; };
    auto load = [&](int s) {  // chunks of [align16(start), align16up(end)); clamped duplicates
        const uint8_t *beg = seg_base(s);
        const uint8_t *a0 = reinterpret_cast<const uint8_t *>((uintptr_t)beg & ~(uintptr_t)15);
        const int nb = min(SEG, bpr - s * SEG);
        const int nch = (int)(((uintptr_t)(beg + nb * kQ6Bytes) - (uintptr_t)a0 + 15) >> 4);
#pragma unroll
        for (int k = 0; k < CPL; ++k)
            reg[k] = *reinterpret_cast<const u32x4 *>(a0 + 16 * min(lane + 64 * k, nch - 1));
    };
    auto store = [&](int s) {
        const uint8_t *beg = seg_base(s);
        const uint8_t *a0 = reinterpret_cast<const uint8_t *>((uintptr_t)beg & ~(uintptr_t)15);
        const int nb = min(SEG, bpr - s * SEG);
        const int nch = (int)(((uintptr_t)(beg + nb * kQ6Bytes) - (uintptr_t)a0 + 15) >> 4);
#pragma unroll
        for (int k = 0; k < CPL; ++k)
            *reinterpret_cast<u32x4 *>(win + 16 * min(lane + 64 * k, nch - 1)) = reg[k];
    };
    // 4 bytes at an even LDS offset: the aligned dword pair around it, shifted
    auto ld4 = [&](int off) -> uint32_t {
        const uint32_t *p = reinterpret_cast<const uint32_t *>(win + (off & ~3));
        return __builtin_amdgcn_alignbyte(p[1], p[0], (uint32_t)(off & 3));
    };
    load(0);
    store(0);
    for (int s = 0; s < nseg; ++s) {
        if (s + 1 < nseg) load(s + 1);
        __builtin_amdgcn_wave_barrier();
        const int off0 = (int)((uintptr_t)seg_base(s) & 15u);
        const int nb = min(SEG, bpr - s * SEG);
        for (int i = 0; 2 * i < nb; ++i) {
            const int bb = 2 * i + h;
            if (bb < nb) {
                const int bo = off0 + bb * kQ6Bytes;
                const uint32_t ql = ld4(bo + 4 * l2);
                const uint32_t qh = ld4(bo + 128 + 4 * (8 * g + (l2 & 7)));
                const int si = bo + 192 + 8 * g + ((l2 & 15) >> 2);
                const float sl = (float)(int8_t)win[si], sh = (float)(int8_t)win[si + 4];
                const float d = half_bits_finite((uint32_t)win[bo + 208] | ((uint32_t)win[bo + 209] << 8));
                const float *xb = x + (size_t)(s * SEG + bb) * kBlockElems + 128 * g + 4 * (l2 & 15);
                const f32x4 xl = ld_f32x4(xb);
                const f32x4 xh = ld_f32x4(xb + 64);
                const uint32_t lo = (ql & 0x0F0F0F0Fu) | (((qh >> (2 * q0)) & 0x03030303u) << 4);
                const uint32_t hi = ((ql >> 4) & 0x0F0F0F0Fu) | (((qh >> (2 * q0 + 4)) & 0x03030303u) << 4);
                float dl = 0.0f, dh = 0.0f;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    dl += (float)((lo >> (8 * t)) & 0xFFu) * xl[t];
                    dh += (float)((hi >> (8 * t)) & 0xFFu) * xh[t];
                }
                const float sxl = (xl[0] + xl[1]) + (xl[2] + xl[3]);
                const float sxh = (xh[0] + xh[1]) + (xh[2] + xh[3]);
                acc += d * (sl * (dl - 32.0f * sxl) + sh * (dh - 32.0f * sxh));
            }
        }
        if (s + 1 < nseg) {
            __builtin_amdgcn_wave_barrier();  // this wavefront's reads of the window come first
            store(s + 1);
        }
    }
    acc = wave_sum(acc);
    if (lane == 0) y[row] = acc;
}

hipError_t gemv_q5k_launch(const uint8_t *w, const float *x, float *y, int n, int bpr,
                           hipStream_t stream) {
    const hipError_t e = gemv_q5k_mfma_launch(w, x, y, n, bpr, stream);
    if (e != hipErrorNotSupported) return e;
    gemv_q5k_kernel<<<(unsigned)((n + 3) / 4), 256, 0, stream>>>(w, x, y, n, bpr);
    return hipGetLastError();
}

hipError_t gemv_q6k_launch(const uint8_t *w, const float *x, float *y, int n, int bpr,
                           hipStream_t stream) {
    const hipError_t e = gemv_q6k_mfma_launch(w, x, y, n, bpr, stream);
    if (e != hipErrorNotSupported) return e;
    // the staged kernel reads 16-byte windows aligned below each segment and
    // byte-decodes the tensor's last row when the tensor end is misaligned,
    // so it takes any w; x needs only float alignment
    gemv_q6k_staged_kernel<<<(unsigned)((n + 3) / 4), 256, 0, stream>>>(w, x, y, n, bpr);
    return hipGetLastError();
}

hipError_t gemv_q6k_q8_launch(const uint8_t *w, const int8_t *xq, const float *xd, float *y,
                              int n, int bpr, hipStream_t stream) {
    gemv_q6k_q8_kernel<<<(unsigned)((n + 3) / 4), 256, 0, stream>>>(w, xq, xd, y, n, bpr);
    return hipGetLastError();
}

}  // namespace mgq
