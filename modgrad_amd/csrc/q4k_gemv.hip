// Q4_K GEMV kernels for gfx950 (MI355X).
//
// Reference semantics: launch_matvec_q4k / matvec_q4k_kernel
// (crates/modgrad-device/kernels/matvec_q4k.hip:55-124) and the host oracle
// rocm_matvec_check.rs:38-47: y[r] = sum_k dequant(W)[r][k] * x[k], canonical
// element order (gguf.rs:364-404).
//
// Two kernels:
//
// 1. gemv_generic_kernel -- vector-ALU, one wavefront per row, flat-stream
//    addressing (element (r,c) at flat index r*k+c), so it serves both the
//    row-aligned GGUF layout and LinearResidentQuantized's flattened layout
//    (neuron.rs:931-951) where rows start mid-block.
//
// 2. gemv_mfma_kernel -- the fast path for the row-aligned layout. The
//    dequantize-multiply runs on the matrix cores (v_mfma_f32_16x16x32_f16):
//      * B operand = weights: lane (n = l%16, h = l/16) holds qs bytes of row n.
//        A nibble masked in place, (dword & 0x000F000F) or (dword & 0x00F000F0),
//        is already an f16 *subnormal* equal to q*2^-24 (or 16q*2^-24), so one
//        AND turns two nibbles into two exact f16 operands.
//      * A operand = activations, laid out per k-slot in LDS by a prologue: the
//        slot's x value goes to MFMA row m = its sub-block (xh part) and
//        m = 8 + sub-block (xl part), zero elsewhere. x is split as
//        x*2^e = xh + xl (two f16, ~22 bits) with a per-sub-block power of two
//        e, so the f32 accumulators receive sum q*x per (sub-block, row) to
//        within ~2^-22 relative -- f32-grade, far inside the 1e-4 bound.
//      * The 16x16 accumulator then holds, per W row, the 8 sub-block partial
//        sums (xh and xl halves); one permlane32 swap merges the halves of two
//        16-row tiles at once, and each lane applies d*sc and dmin*m*sum(x)
//        for 4 (row, sub-block) pairs.
//    Per 32 rows x 1 block a wave issues 5 16-byte loads per lane, 16 MFMAs and
//    about 130 VALU ops, i.e. ~1 VALU op per weight -- low enough to stay
//    HBM-bound on MI355X, where FP32 VALU rate / HBM rate leaves ~2.8 ops per
//    Q4_K weight at 100% of 8 TB/s.
#include "q4k_device.hpp"
#include "q4k_launch.hpp"

#include <algorithm>
#include <cstdlib>

namespace mgq {

// --------------------------------------------------------------- generic ---

template <bool ROW_ALIGNED>
__global__ __launch_bounds__(256) void gemv_generic_kernel(const uint8_t *__restrict__ w,
                                                           const float *__restrict__ x,
                                                           float *__restrict__ y, int n, int k) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n) return;  // uniform per wavefront
    const int64_t f0 = (int64_t)row * k;
    const int64_t b0 = f0 >> 8, b1 = (f0 + k - 1) >> 8;
    const int64_t n_units = (b1 - b0 + 1) * 32;
    float acc = 0.0f;
    for (int64_t j = lane; j < n_units; j += 64) {
        const int64_t b = b0 + (j >> 5);
        const int u = (int)(j & 31);
        const uint8_t *blk = w + b * kBlockBytes;
        const uint32_t h0 = ld_u32(blk), s0 = ld_u32(blk + 4), s1 = ld_u32(blk + 8),
                       s2 = ld_u32(blk + 12), qd = ld_u32(blk + 16 + 4 * u);
        const float d = half_bits_finite(h0), dmin = half_bits_finite(h0 >> 16);
        const int G = u >> 3, i = u & 7;
        uint32_t sc_lo, m_lo, sc_hi, m_hi;
        scale_min(2 * G, s0, s1, s2, sc_lo, m_lo);
        scale_min(2 * G + 1, s0, s1, s2, sc_hi, m_hi);
        const float d1 = d * (float)sc_lo, m1 = dmin * (float)m_lo;
        const float d2 = d * (float)sc_hi, m2 = dmin * (float)m_hi;
        const int64_t c0 = b * kBlockElems + 64 * G + 4 * i - f0;  // column of lo nibble 0
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const float wl = d1 * (float)((qd >> (8 * t)) & 15u) - m1;
            const float wh = d2 * (float)((qd >> (8 * t + 4)) & 15u) - m2;
            const int64_t cl = c0 + t, ch = c0 + t + 32;
            if (ROW_ALIGNED || (cl >= 0 && cl < k)) acc += wl * x[cl];
            if (ROW_ALIGNED || (ch >= 0 && ch < k)) acc += wh * x[ch];
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if (lane == 0) y[row] = acc;
}

hipError_t gemv_generic_launch(const uint8_t *w, const float *x, float *y, int n, int k,
                               hipStream_t stream) {
    const unsigned grid = (unsigned)((n + 3) / 4);
    if (k % kBlockElems == 0)
        gemv_generic_kernel<true><<<grid, 256, 0, stream>>>(w, x, y, n, k);
    else
        gemv_generic_kernel<false><<<grid, 256, 0, stream>>>(w, x, y, n, k);
    return hipGetLastError();
}

// ------------------------------------------------------------------ MFMA ---

// Byte offset inside qs[128] of the 8 bytes that MFMA slot-group (pair p,
// lane group h) reads: the lane's two 16-byte loads are qs[16h..] and
// qs[64+16h..]; pair p takes dwords 2p, 2p+1 of those 32 bytes.
__device__ __forceinline__ int pair_byte_offset(int p, int h) {
    return p < 2 ? 16 * h + 8 * p : 64 + 16 * h + 8 * (p - 2);
}

constexpr int kRowsPerGroup = 32;  // two 16-row MFMA tiles per wavefront

// LDS layout for one work-group (all bpr blocks of K):
//   atab [bpr][8 mfma c][4 lane-group h][xh|xl][8 halves]  bpr*1024 B
//   zero 16 B                                             at bpr*1024
//   meta [bpr][corr[8] | xsum[8]] f32                     bpr*64 B
//   aux  max(bpr*8*4, NW*64*4) B: x scale per sub-block, later the
//        cross-wave reduction buffer
__host__ __device__ constexpr size_t mfma_lds_bytes(int bpr, int nw) {
    return (size_t)bpr * 1024 + 16 + (size_t)bpr * 64 +
           ((size_t)bpr * 32 > (size_t)nw * 256 ? (size_t)bpr * 32 : (size_t)nw * 256);
}

constexpr int kMaxWaves = 8;

// One work-group = NW = blockDim.x/64 wavefronts (1..8) covering 32 rows; the
// wavefronts split the row's blocks and reduce through LDS at the end.
__global__ __launch_bounds__(kMaxWaves * 64) void gemv_mfma_kernel(const uint8_t *__restrict__ w,
                                                                   const float *__restrict__ x,
                                                                   float *__restrict__ y, int n,
                                                                   int bpr) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int NW = (int)(blockDim.x >> 6);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t zero_off = (uint32_t)bpr * 1024u;
    float *meta = reinterpret_cast<float *>(lds + zero_off + 16);
    float *aux = meta + bpr * 16;

    // ---- prologue: build the activation operand table in LDS -------------
    if (tid < 4) reinterpret_cast<uint32_t *>(lds + zero_off)[tid] = 0u;
    for (int i = tid; i < bpr * 8; i += NW * 64) {  // i = b*8 + sub-block
        const f32x4 *xs = reinterpret_cast<const f32x4 *>(x + (size_t)i * 32);
        float amax = 0.0f, sum = 0.0f;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const f32x4 v = xs[t];
            sum += (v[0] + v[1]) + (v[2] + v[3]);
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])),
                                     fmaxf(fabsf(v[2]), fabsf(v[3]))));
        }
        int e = 0;
        if (amax > 0.0f && amax <= 3.402823466e38f) {
            int ex;
            frexpf(amax, &ex);  // amax in [2^(ex-1), 2^ex)
            e = std::min(std::max(14 - ex, -90), 140);
        }
        reinterpret_cast<int *>(aux)[i] = e;  // 2^e may exceed f32: keep the exponent
        const int sb = i & 7;
        meta[(i >> 3) * 16 + sb] = ldexpf(1.0f, ((sb & 1) ? 20 : 24) - e);
        meta[(i >> 3) * 16 + 8 + sb] = sum;
    }
    __syncthreads();
    for (int i = tid; i < bpr * 32; i += NW * 64) {  // i = (b*8 + c)*4 + h
        const int b = i >> 5, c = (i >> 2) & 7, h = i & 3;
        const int o = pair_byte_offset(c >> 1, h), kind = c & 1;
        const int G = o >> 5;
        const int e = reinterpret_cast<const int *>(aux)[b * 8 + 2 * G + kind];
        const float *xp = x + (size_t)b * kBlockElems + 64 * G + (o & 31) + 32 * kind;
        const f32x4 v0 = *reinterpret_cast<const f32x4 *>(xp);
        const f32x4 v1 = *reinterpret_cast<const f32x4 *>(xp + 4);
        // slot s holds byte o + {0,2,1,3,4,6,5,7}[s] (see the B operand build)
        const float xv[8] = {v0[0], v0[2], v0[1], v0[3], v1[0], v1[2], v1[1], v1[3]};
        half8 hh, hl;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const float xs = ldexpf(xv[s], e);
            const _Float16 a = (_Float16)xs;
            hh[s] = a;
            hl[s] = (_Float16)(xs - (float)a);
        }
        *reinterpret_cast<half8 *>(lds + (size_t)i * 32) = hh;
        *reinterpret_cast<half8 *>(lds + (size_t)i * 32 + 16) = hl;
    }
    __syncthreads();

    // ---- per-lane constants ------------------------------------------------
    const int n16 = lane & 15, g = lane >> 4;       // B lane: W row n16, k-group g
    const int tdec = lane >> 5, jq = (lane >> 4) & 1;  // decode lane: tile, sub-block quad
    uint32_t abase[8], astride[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const int o = pair_byte_offset(c >> 1, g);
        const int sb = 2 * (o >> 5) + (c & 1);
        const bool hit = (n16 & 7) == sb;        // A lane m = n16
        abase[c] = hit ? (uint32_t)((c * 4 + g) * 32 + (n16 >> 3) * 16) : zero_off;
        astride[c] = hit ? 1024u : 0u;
    }
    const size_t row_bytes = (size_t)bpr * kBlockBytes;
    const int r0 = blockIdx.x * kRowsPerGroup;
    const int rA = std::min(r0 + n16, n - 1), rB = std::min(r0 + 16 + n16, n - 1);
    const int rD = std::min(r0 + 16 * tdec + n16, n - 1);
    const uint8_t *pA = w + (size_t)rA * row_bytes + 16 + 16 * g;
    const uint8_t *pB = w + (size_t)rB * row_bytes + 16 + 16 * g;
    const uint8_t *pD = w + (size_t)rD * row_bytes;
    const int kb0 = (bpr * wave) / NW, kb1 = (bpr * (wave + 1)) / NW;

    float yacc = 0.0f;
    u32x4 na0, na1, nb0, nb1, nh;
    if (kb0 < kb1) {
        na0 = *reinterpret_cast<const u32x4 *>(pA + (size_t)kb0 * kBlockBytes);
        na1 = *reinterpret_cast<const u32x4 *>(pA + (size_t)kb0 * kBlockBytes + 64);
        nb0 = *reinterpret_cast<const u32x4 *>(pB + (size_t)kb0 * kBlockBytes);
        nb1 = *reinterpret_cast<const u32x4 *>(pB + (size_t)kb0 * kBlockBytes + 64);
        nh = *reinterpret_cast<const u32x4 *>(pD + (size_t)kb0 * kBlockBytes);
    }
    for (int b = kb0; b < kb1; ++b) {
        const u32x4 qa0 = na0, qa1 = na1, qb0 = nb0, qb1 = nb1, hd = nh;
        if (b + 1 < kb1) {
            const size_t off = (size_t)(b + 1) * kBlockBytes;
            na0 = *reinterpret_cast<const u32x4 *>(pA + off);
            na1 = *reinterpret_cast<const u32x4 *>(pA + off + 64);
            nb0 = *reinterpret_cast<const u32x4 *>(pB + off);
            nb1 = *reinterpret_cast<const u32x4 *>(pB + off + 64);
            nh = *reinterpret_cast<const u32x4 *>(pD + off);
        }
        f32x4 accA = {0.f, 0.f, 0.f, 0.f}, accB = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const half8 a = *reinterpret_cast<const half8 *>(lds + abase[c] + (uint32_t)b * astride[c]);
            const int p = c >> 1;
            const uint32_t mask = (c & 1) ? 0x00F000F0u : 0x000F000Fu;
            const uint32_t wa0 = p < 2 ? qa0[2 * p] : qa1[2 * p - 4];
            const uint32_t wa1 = p < 2 ? qa0[2 * p + 1] : qa1[2 * p - 3];
            const uint32_t wb0 = p < 2 ? qb0[2 * p] : qb1[2 * p - 4];
            const uint32_t wb1 = p < 2 ? qb0[2 * p + 1] : qb1[2 * p - 3];
            const u32x4 ba = {wa0 & mask, (wa0 >> 8) & mask, wa1 & mask, (wa1 >> 8) & mask};
            const u32x4 bb = {wb0 & mask, (wb0 >> 8) & mask, wb1 & mask, (wb1 >> 8) & mask};
            accA = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(half8, ba), accA, 0, 0, 0);
            accB = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(half8, bb), accB, 0, 0, 0);
        }
        // Merge xh and xl halves: lanes 0..31 get tile A's (row, sub-block)
        // sums, lanes 32..63 tile B's. (Not __builtin_amdgcn_permlane32_swap:
        // this compiler miscombines its two results.)
        float s[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float mine = tdec ? accB[i] : accA[i];
            const float give = tdec ? accA[i] : accB[i];
            s[i] = mine + __shfl_xor(give, 32, 64);
        }
        const float d = half_bits_finite(hd[0]), dmin = half_bits_finite(hd[0] >> 16);
        const uint32_t scq = jq ? scales4(1, hd[1], hd[3]) : scales4(0, hd[1], hd[3]);
        const uint32_t mnq = jq ? mins4(1, hd[2], hd[3]) : mins4(0, hd[2], hd[3]);
        const f32x4 corr = *reinterpret_cast<const f32x4 *>(meta + b * 16 + 4 * jq);
        const f32x4 xsum = *reinterpret_cast<const f32x4 *>(meta + b * 16 + 8 + 4 * jq);
        float t1 = 0.0f, t2 = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            t1 += (float)((scq >> (8 * i)) & 0xFFu) * (s[i] * corr[i]);
            t2 += (float)((mnq >> (8 * i)) & 0xFFu) * xsum[i];
        }
        yacc += d * t1 - dmin * t2;
    }
    aux[wave * 64 + lane] = yacc;  // aux is free again (prologue done)
    __syncthreads();
    if (tid < kRowsPerGroup) {
        const int tl = (tid >> 4) * 32 + (tid & 15);  // lane holding row tid, quad 0
        float sum = 0.0f;
        for (int wv = 0; wv < NW; ++wv) sum += aux[wv * 64 + tl] + aux[wv * 64 + tl + 16];
        if (r0 + tid < n) y[r0 + tid] = sum;
    }
}

static int env_int(const char *name, int dflt) {
    const char *s = std::getenv(name);
    return (s && *s) ? std::atoi(s) : dflt;
}

hipError_t gemv_prepare() {
    // Allow up to the full 160 KiB of LDS, once per process (thread-safe
    // static init). Called before any stream capture records a launch.
    static const hipError_t attr = hipFuncSetAttribute(
        (const void *)gemv_mfma_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    return attr;
}

hipError_t gemv_mfma_launch(const uint8_t *w, const float *x, float *y, int n, int bpr,
                            hipStream_t stream) {
    if (((uintptr_t)w & 15u) || ((uintptr_t)x & 15u)) return hipErrorNotSupported;
    if (mfma_lds_bytes(bpr, kMaxWaves) > 160 * 1024) return hipErrorNotSupported;
    const hipError_t attr = gemv_prepare();
    if (attr != hipSuccess) return attr;
    static const int nw_env = env_int("MGQ_GEMV_WAVES", 0);  // tuning override
    int nw = nw_env > 0 ? std::min(nw_env, kMaxWaves) : (bpr >= 16 ? 8 : 4);
    const size_t lds = mfma_lds_bytes(bpr, nw);
    const unsigned grid = (unsigned)((n + kRowsPerGroup - 1) / kRowsPerGroup);
    gemv_mfma_kernel<<<grid, nw * 64, lds, stream>>>(w, x, y, n, bpr);
    return hipGetLastError();
}

static int env_force_generic() {
    static int v = -1;
    if (v < 0) {
        const char *s = std::getenv("MGQ_FORCE_GENERIC");
        v = (s && *s && *s != '0') ? 1 : 0;
    }
    return v;
}

hipError_t gemv_rows_launch(const uint8_t *w, const float *x, float *y, int n, int bpr,
                            hipStream_t stream) {
    if (!env_force_generic()) {
        hipError_t e = gemv_mfma_launch(w, x, y, n, bpr, stream);
        if (e != hipErrorNotSupported) return e;
    }
    return gemv_generic_launch(w, x, y, n, bpr * kBlockElems, stream);
}

// --------------------------------------------------------------- batched ---

// Vector-ALU batched GEMV: each weight is dequantized once and applied to up
// to BMAX activation rows. One wavefront per W row.
template <int BMAX>
__global__ __launch_bounds__(256) void gemv_batched_kernel(const uint8_t *__restrict__ w,
                                                           const float *__restrict__ X,
                                                           float *__restrict__ Y, int n, int bpr,
                                                           int batch) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n) return;
    const int k = bpr * kBlockElems;
    const uint8_t *wr = w + (size_t)row * bpr * kBlockBytes;
    float acc[BMAX];
#pragma unroll
    for (int bb = 0; bb < BMAX; ++bb) acc[bb] = 0.0f;
    for (int j = lane; j < bpr * 32; j += 64) {
        const int b = j >> 5, u = j & 31;
        const uint8_t *blk = wr + (size_t)b * kBlockBytes;
        const uint32_t h0 = ld_u32(blk), s0 = ld_u32(blk + 4), s1 = ld_u32(blk + 8),
                       s2 = ld_u32(blk + 12), qd = ld_u32(blk + 16 + 4 * u);
        const float d = half_bits_finite(h0), dmin = half_bits_finite(h0 >> 16);
        const int G = u >> 3, i = u & 7;
        uint32_t sc_lo, m_lo, sc_hi, m_hi;
        scale_min(2 * G, s0, s1, s2, sc_lo, m_lo);
        scale_min(2 * G + 1, s0, s1, s2, sc_hi, m_hi);
        const float d1 = d * (float)sc_lo, m1 = dmin * (float)m_lo;
        const float d2 = d * (float)sc_hi, m2 = dmin * (float)m_hi;
        const int c0 = b * kBlockElems + 64 * G + 4 * i;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const float wl = d1 * (float)((qd >> (8 * t)) & 15u) - m1;
            const float wh = d2 * (float)((qd >> (8 * t + 4)) & 15u) - m2;
#pragma unroll
            for (int bb = 0; bb < BMAX; ++bb) {
                if (bb < batch) {
                    const float *xb = X + (size_t)bb * k;
                    acc[bb] += wl * xb[c0 + t] + wh * xb[c0 + t + 32];
                }
            }
        }
    }
#pragma unroll
    for (int bb = 0; bb < BMAX; ++bb) {
        float a = acc[bb];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) a += __shfl_xor(a, off, 64);
        if (lane == 0 && bb < batch) Y[(size_t)bb * n + row] = a;
    }
}

hipError_t gemv_batched_launch(const uint8_t *w, const float *X, float *Y, int n, int bpr,
                               int batch, hipStream_t stream) {
    const unsigned grid = (unsigned)((n + 3) / 4);
    if (batch <= 1)
        gemv_batched_kernel<1><<<grid, 256, 0, stream>>>(w, X, Y, n, bpr, batch);
    else if (batch <= 2)
        gemv_batched_kernel<2><<<grid, 256, 0, stream>>>(w, X, Y, n, bpr, batch);
    else if (batch <= 4)
        gemv_batched_kernel<4><<<grid, 256, 0, stream>>>(w, X, Y, n, bpr, batch);
    else if (batch <= 8)
        gemv_batched_kernel<8><<<grid, 256, 0, stream>>>(w, X, Y, n, bpr, batch);
    else
        gemv_batched_kernel<16><<<grid, 256, 0, stream>>>(w, X, Y, n, bpr, batch);
    return hipGetLastError();
}

}  // namespace mgq
