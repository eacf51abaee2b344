// Prefill dequant-GEMM on the gfx950 matrix cores:
//   C[m][r] = sum_k dequant(W)[r][k] * A[m][k],  A f16 [M][K], C f32 [M][N].
// No counterpart in the reference (its prefill is a per-token GEMV loop,
// crates/modgrad-gemma/examples/gemma4_rocm.rs:26-34); the dequantized value
// of each weight is the canonical one (gguf.rs:364-404) rounded once to f16.
//
// Work-group tile: 128 W rows x 128 tokens, K stepped by 64 (= one 32-byte qs
// group: sub-blocks 2G and 2G+1 of a super-block). Per K step every thread
// decodes 32 weights (16 qs bytes of one row) in f32, rounds them to f16 and
// stores them to LDS next to the 128x64 f16 activation tile; LDS is double
// buffered so the next step's global loads overlap this step's MFMAs.
// 4 wavefronts, each a 64x64 output tile = 4x4 v_mfma_f32_16x16x32_f16 tiles,
// W as the A operand (rows), activations as the B operand (tokens), so a
// lane's 4 accumulators are 4 consecutive W rows of one token: one 16-byte
// store into C's row-major [M][N].
#include "q4k_device.hpp"
#include "q4k_launch.hpp"

namespace mgq {

namespace gemm {
constexpr int BN = 128;        // W rows per work-group
constexpr int BM = 128;        // tokens per work-group
constexpr int BK = 64;         // k per step
constexpr int LDS_ROW = 72;    // halves per LDS row (64 + 8 pad, 144 B)
constexpr int TILE_HALVES = 128 * LDS_ROW;
}  // namespace gemm

__global__ __launch_bounds__(256) void gemm_q4k_f16_kernel(const uint8_t *__restrict__ w,
                                                           const uint16_t *__restrict__ a,
                                                           float *__restrict__ c, int n, int bpr,
                                                           int m_tokens) {
    using namespace gemm;
    __shared__ __attribute__((aligned(16))) _Float16 sW[2][TILE_HALVES];
    __shared__ __attribute__((aligned(16))) _Float16 sA[2][TILE_HALVES];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
    const int K = bpr * kBlockElems;
    const int steps = K / BK;  // 4 per super-block
    const size_t row_bytes = (size_t)bpr * kBlockBytes;

    // loader roles: W -> (row wr, 16-byte half wh); A -> 4 x 16 B of one token row
    const int wr = tid >> 1, wh = tid & 1;
    const uint8_t *wrow = w + (size_t)min(n0 + wr, n - 1) * row_bytes;
    const int ar = tid >> 1, ac = (tid & 1) * 32;  // token row, first half column
    const uint16_t *arow = a + (size_t)min(m0 + ar, m_tokens - 1) * K;

    u32x4 qreg, hreg;
    u32x4 areg[4];
    auto gload = [&](int s) {
        const int b = s >> 2, G = s & 3;
        const uint8_t *blk = wrow + (size_t)b * kBlockBytes;
        hreg = *reinterpret_cast<const u32x4 *>(blk);
        qreg = *reinterpret_cast<const u32x4 *>(blk + 16 + 32 * G + 16 * wh);
        const uint16_t *ap = arow + (size_t)s * BK + ac;
#pragma unroll
        for (int i = 0; i < 4; ++i) areg[i] = *reinterpret_cast<const u32x4 *>(ap + 8 * i);
    };
    auto lstore = [&](int s, int buf) {
        const int G = s & 3;
        const float d = half_bits_finite(hreg[0]), dmin = half_bits_finite(hreg[0] >> 16);
        uint32_t sc_lo, m_lo, sc_hi, m_hi;
        scale_min(2 * G, hreg[1], hreg[2], hreg[3], sc_lo, m_lo);
        scale_min(2 * G + 1, hreg[1], hreg[2], hreg[3], sc_hi, m_hi);
        const float d1 = d * (float)sc_lo, m1 = dmin * (float)m_lo;
        const float d2 = d * (float)sc_hi, m2 = dmin * (float)m_hi;
        half8 lo[2], hi[2];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint32_t byte = (qreg[j >> 2] >> (8 * (j & 3))) & 0xFFu;
            lo[j >> 3][j & 7] = (_Float16)(d1 * (float)(byte & 15u) - m1);
            hi[j >> 3][j & 7] = (_Float16)(d2 * (float)(byte >> 4) - m2);
        }
        _Float16 *dst = &sW[buf][wr * LDS_ROW + 16 * wh];
        *reinterpret_cast<half8 *>(dst) = lo[0];
        *reinterpret_cast<half8 *>(dst + 8) = lo[1];
        *reinterpret_cast<half8 *>(dst + 32) = hi[0];
        *reinterpret_cast<half8 *>(dst + 40) = hi[1];
        _Float16 *da = &sA[buf][ar * LDS_ROW + ac];
#pragma unroll
        for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4 *>(da + 8 * i) = areg[i];
    };

    // compute roles
    const int wn = (wave >> 1) * 64, wm = (wave & 1) * 64;  // wave's W-row / token offsets
    const int l16 = lane & 15, kq = (lane >> 4) * 8;
    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    gload(0);
    lstore(0, 0);
    __syncthreads();
    for (int s = 0; s < steps; ++s) {
        const int buf = s & 1;
        if (s + 1 < steps) gload(s + 1);
#pragma unroll
        for (int kk = 0; kk < BK; kk += 32) {
            half8 wa[4], tb[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                wa[i] = *reinterpret_cast<const half8 *>(&sW[buf][(wn + 16 * i + l16) * LDS_ROW + kk + kq]);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                tb[j] = *reinterpret_cast<const half8 *>(&sA[buf][(wm + 16 * j + l16) * LDS_ROW + kk + kq]);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa[i], tb[j], acc[i][j], 0, 0, 0);
        }
        if (s + 1 < steps) lstore(s + 1, buf ^ 1);
        __syncthreads();
    }

    // lane holds W rows wn+16i+4(l/16)+v (v=0..3) of token wm+16j+l%16
    const bool vec = (n % 4) == 0 && (((uintptr_t)c & 15u) == 0);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int m = m0 + wm + 16 * j + l16;
        if (m >= m_tokens) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = n0 + wn + 16 * i + 4 * (lane >> 4);
            float *dst = c + (size_t)m * n + r;
            if (vec && r + 3 < n) {
                *reinterpret_cast<f32x4 *>(dst) = acc[i][j];
            } else {
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    if (r + v < n) dst[v] = acc[i][j][v];
            }
        }
    }
}

hipError_t gemm_f16_launch(const uint8_t *w, const uint16_t *a, float *c, int n, int bpr,
                           int m_tokens, hipStream_t stream) {
    if (((uintptr_t)w & 15u) || ((uintptr_t)a & 15u)) return hipErrorInvalidValue;
    const unsigned gx = (unsigned)((n + gemm::BN - 1) / gemm::BN);
    const unsigned gy = (unsigned)((m_tokens + gemm::BM - 1) / gemm::BM);
    if (gy > 65535) return hipErrorInvalidValue;
    gemm_q4k_f16_kernel<<<dim3(gx, gy), 256, 0, stream>>>(w, a, c, n, bpr, m_tokens);
    return hipGetLastError();
}

}  // namespace mgq
