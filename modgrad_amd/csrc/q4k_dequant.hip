// Bit-exact Q4_K -> f32 dequantization (canonical order) for gfx950.
//
// Reference: the host dequantizer dequantize_row_q4_k
// (crates/modgrad-device/src/kfd/gguf.rs:364-404) is the spec; each weight is
// fl(fl(d*sc)*q) - fl(dmin*m). FP contraction is switched off in this file so
// the compiler cannot fuse the multiply into the subtract.
//
// Work split: one thread per (block, qs dword u). qs dword u of a block holds
// bytes 4u..4u+3 of qs, i.e. the low nibbles of positions 64G+4i..64G+4i+3 and
// the high nibbles of those positions + 32 (G = u/8, i = u%8). A thread writes
// those 8 floats as two 16-byte stores; a wave covers two whole blocks, so the
// 2 KiB it writes are contiguous. HBM-bound: 144 B read, 1024 B written per
// block.
#include "q4k_device.hpp"
#include "q4k_launch.hpp"

#pragma clang fp contract(off)

namespace mgq {

template <bool VEC_STORE>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t *__restrict__ q,
                                                      float *__restrict__ out,
                                                      int64_t n_units) {
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (gid >= n_units) return;
    const int64_t b = gid >> 5;
    const int u = (int)(gid & 31);
    const uint8_t *blk = q + b * kBlockBytes;
    const uint32_t h0 = ld_u32(blk), s0 = ld_u32(blk + 4), s1 = ld_u32(blk + 8),
                   s2 = ld_u32(blk + 12), qd = ld_u32(blk + 16 + 4 * u);
    const float d = half_bits_finite(h0), dmin = half_bits_finite(h0 >> 16);
    const int G = u >> 3, i = u & 7;
    uint32_t sc_lo, m_lo, sc_hi, m_hi;
    scale_min(2 * G, s0, s1, s2, sc_lo, m_lo);
    scale_min(2 * G + 1, s0, s1, s2, sc_hi, m_hi);
    const float d1 = d * (float)sc_lo, m1 = dmin * (float)m_lo;
    const float d2 = d * (float)sc_hi, m2 = dmin * (float)m_hi;
    float lo[4], hi[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        lo[t] = d1 * (float)((qd >> (8 * t)) & 15u) - m1;
        hi[t] = d2 * (float)((qd >> (8 * t + 4)) & 15u) - m2;
    }
    float *o = out + b * kBlockElems + 64 * G + 4 * i;
    if (VEC_STORE) {
        *reinterpret_cast<f32x4 *>(o) = f32x4{lo[0], lo[1], lo[2], lo[3]};
        *reinterpret_cast<f32x4 *>(o + 32) = f32x4{hi[0], hi[1], hi[2], hi[3]};
    } else {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            o[t] = lo[t];
            o[32 + t] = hi[t];
        }
    }
}

hipError_t dequant_launch(const uint8_t *q, int n_blocks, float *out, hipStream_t stream) {
    const int64_t units = (int64_t)n_blocks * 32;
    const int64_t grid = (units + 255) / 256;
    if (grid > 0x7FFFFFFF) return hipErrorInvalidValue;
    if (((uintptr_t)out & 15u) == 0)
        dequant_kernel<true><<<dim3((unsigned)grid), dim3(256), 0, stream>>>(q, out, units);
    else
        dequant_kernel<false><<<dim3((unsigned)grid), dim3(256), 0, stream>>>(q, out, units);
    return hipGetLastError();
}

}  // namespace mgq
