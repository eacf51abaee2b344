// Q6_K matvec on the gfx950 matrix cores (launch_matvec_q6k, rocm.rs:482-485;
// canonical order of dequantize_row_q6_k, gguf.rs:441-477), for 16-byte
// aligned weights and float-aligned x. Two kernels share the decode: whole-row stages for
// K <= kQ6mMaxBpr * 256 (attention, lm_head) and K-chunked per-row stages for
// longer rows (ffn_down).
//
// Q6_K block, 210 B / 256 weights: ql[128] | qh[64] | int8 sc[16] | d f16.
// Position p = 128g' + 32quad + l (l < 32) is sub-block j = 4g' + quad:
// q = (nibble (quad >> 1) of ql[64g' + 32(quad & 1) + l]) | (2 bits (2quad) of
// qh[32g' + l]) << 4, and w = d * sc[2j + l/16] * (q - 32).
//
// Work-group = 16 rows x all K, persistent over row groups; 7 wavefronts
// (16 for the long-row kernels).
//   * Whole-row stage: a row group's 16 rows are one contiguous byte range
//     (16 x RB, RB = 210 bpr), copied flat into LDS as whole 16-byte chunks;
//     the next group's chunks wait in registers.
//   * Long rows (bpr > kQ6mMaxBpr), and the fused-RMSNorm launches of any
//     length (14 wavefronts), wave-private (gemv_q6k_wave_long_kernel, the
//     default): wavefront w stages block w, w + NW, ... of the 16 rows in
//     its own LDS slot (each row segment as the 16-byte chunks from the
//     16-byte boundary at or below its start; the segment's offset in that
//     chunk (s & 15) moves the lane's reads) and computes from it with no
//     barrier between units; the table covers the whole row.
//   * K-chunked stage (gemv_q6k_mfma_long_kernel, rows too long for the
//     wave-private kernel's LDS): a stage is 14 blocks of each of the 16
//     rows, staged by the whole work-group the same way. Row sums carry over
//     the chunks of a group.
//   * One v_mfma_f32_16x16x32_f16 per sub-block: B = weights (lane (n, g):
//     row n, positions 8g..8g+7 of the sub-block; the 6-bit q are f16
//     subnormals q*2^-24, exact, or 16q*2^-24 for the high-nibble sub-blocks,
//     whose halves are the nibble in place plus the qh bits as the high byte:
//     one byte permute per operand dword), A = the activation table built once per
//     work-group: x*2^e = xh + xl (f16) with one exponent per sub-block, in
//     A row m = 4(j % 4) + 2 half + part, so sub-blocks 0-3 and 4-7 of a block
//     land in two accumulators and lane (n, g) holds both halves (xh, xl) of
//     sub-blocks g and 4 + g of row n.
//   * A lane reads its 8 ql bytes (for two sub-blocks: low and high nibbles)
//     and its 8 qh bytes (for four) once per 128-position half; blocks are
//     only 2-byte aligned in LDS, so a 2-dword read is the 3 aligned dwords
//     around it shifted into place (v_alignbyte_b32).
//   * y_r = sum_j d * (corr_j * (sc_2j s_0 + sc_2j+1 s_1) - 32 (sc_2j X_0 +
//     sc_2j+1 X_1)), s_h the scaled sums of q*x over half h, X_h the sums of x.
// Bytes per unit: 210 per 256 weights of one row (plus x once per
// work-group): HBM-bound.
#include "q4k_device.hpp"
#include "q4k_launch.hpp"

#include <algorithm>
#include <cstdlib>

namespace mgq {

namespace q6m {
constexpr int R = 16, NW = 7, NT = NW * 64;
constexpr int BB = 210;                   // Q6_K block bytes
constexpr int MAX_BPR = 14;               // whole-row stages
constexpr int CPL = (R * MAX_BPR * BB / 16 + NT - 1) / NT;  // 16-byte chunks per lane (7)
constexpr int TAB = 1024;                 // per block: 1 KiB of A operands
constexpr int META = 24;                  // floats per block: corr[8] | X[16]
constexpr int SEG = 14;                   // blocks per K-chunk of a long row
// wavefronts of the K-chunked kernel: a long-row shape has few row groups
// (ffn_down: 224 for 256 CUs), so one work-group per CU carries the latency
// hiding (7 -> 16 waves: 25.5 -> 20.9 us on 3584x18944)
constexpr int LONG_NW = 16;
constexpr int SLOTC = (15 + SEG * BB + 15) / 16;            // 16-byte chunks per row slot (185)
}  // namespace q6m

constexpr int kQ6mMaxBpr = q6m::MAX_BPR;

struct Q6mLayout {
    uint32_t meta, stage, aux, ybuf, normp;
    size_t total;
};

// chunked = false: whole-row stages (bpr <= MAX_BPR); true: K-chunked slots;
// nw = wavefronts per work-group
__host__ __device__ inline Q6mLayout q6m_layout(int bpr, int rounds, bool chunked,
                                                int nw = q6m::NW) {
    using namespace q6m;
    Q6mLayout L;
    L.meta = (uint32_t)bpr * TAB;
    L.stage = L.meta + (uint32_t)bpr * META * 4;
    // + 16: the 3-dword window around the last bytes of row 15 may end past them
    L.aux = L.stage + (chunked ? (uint32_t)(R * SLOTC * 16) : (uint32_t)(R * bpr * BB)) + 16;
    L.ybuf = L.aux + (uint32_t)nw * R * 4;
    L.normp = L.ybuf + (uint32_t)R * rounds * 4;  // fused RMSNorm: one sum(x^2) per wavefront
    L.total = (size_t)L.normp + 16 * 4;
    return L;
}

// Activation-table item i = 8 floats (v0, v1) of x: block i/32, sub-block
// (i/4)%8, lane group i%4. Every lane calls it (the quad reductions are
// cross-lane); only lanes with `valid` store. x*2^e = xh + xl with e putting
// the sub-block's largest |x| in [2^13, 2^14); slot s of the 8 holds position
// {0,2,1,3,4,6,5,7}[s] (the B operand's order).
__device__ __forceinline__ void q6m_item(uint8_t *lds, float *meta, int i, bool valid, f32x4 v0,
                                         f32x4 v1) {
    using namespace q6m;
    float amax = fmaxf(fmaxf(fmaxf(fabsf(v0[0]), fabsf(v0[1])), fmaxf(fabsf(v0[2]), fabsf(v0[3]))),
                       fmaxf(fmaxf(fabsf(v1[0]), fabsf(v1[1])), fmaxf(fabsf(v1[2]), fabsf(v1[3]))));
    float sum = ((v0[0] + v0[1]) + (v0[2] + v0[3])) + ((v1[0] + v1[1]) + (v1[2] + v1[3]));
    amax = fmaxf(amax, quad_xor<1>(amax));
    amax = fmaxf(amax, quad_xor<2>(amax));
    sum += quad_xor<1>(sum);  // the 16 values of this half
    if (!valid) return;
    int e = 0;
    if (amax > 0.0f && amax <= 3.402823466e38f) {
        int ex;
        frexpf(amax, &ex);
        e = std::min(std::max(14 - ex, -103), 140);  // 2^(24 - e) stays finite
    }
    const int b = i >> 5, j = (i >> 2) & 7, kg = i & 3;
    // sub-blocks 2, 3, 6, 7 (high nibbles) arrive as 16q: their corr is / 16
    if (kg == 0) meta[b * META + j] = ldexpf(1.0f, ((j & 2) ? 20 : 24) - e);
    if ((kg & 1) == 0) meta[b * META + 8 + 2 * j + (kg >> 1)] = sum;
    const float xs[8] = {v0[0], v0[2], v0[1], v0[3], v1[0], v1[2], v1[1], v1[3]};
    u32x4 hh, hl;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float a0 = ldexpf(xs[2 * q], e), a1 = ldexpf(xs[2 * q + 1], e);
        const auto hp = __builtin_amdgcn_cvt_pkrtz(a0, a1);
        const auto lp = __builtin_amdgcn_cvt_pkrtz(a0 - (float)hp[0], a1 - (float)hp[1]);
        hh[q] = __builtin_bit_cast(uint32_t, hp);
        hl[q] = __builtin_bit_cast(uint32_t, lp);
    }
    uint8_t *ent = lds + (size_t)b * TAB + (size_t)((j * 4 + kg) * 2) * 16;
    *reinterpret_cast<u32x4 *>(ent) = hh;
    *reinterpret_cast<u32x4 *>(ent + 16) = hl;
}

// Lane (n16, g) supplies A row n16, k-slice g of every MFMA. Row n16 is
// nonzero only in the MFMAs of sub-blocks c with c % 4 = n16 / 4, and only in
// its half's k-slices (g / 2 = (n16 / 2) % 2): there it is table entry
// (c, g, part = n16 % 2), at byte 128 c + e of the block's table. hitq is
// that quad (-1: the lane's A data is zero in every MFMA).
struct Q6mLane {
    uint32_t e;
    int hitq;
};
__device__ __forceinline__ Q6mLane q6m_lane(int lane) {
    const int n16 = lane & 15, g = lane >> 4;
    Q6mLane L;
    L.e = (uint32_t)((g * 2 + (n16 & 1)) * 16);
    L.hitq = (((n16 >> 1) & 1) == (g >> 1)) ? (n16 >> 2) : -1;
    return L;
}

// One Q6_K block of row n16 staged at LDS byte rb (2-byte aligned), against
// table entry b: this lane's part of d * sum_j (corr_j (sc s_0 + sc s_1) -
// 32 (sc X_0 + sc X_1)) over its sub-blocks g and 4 + g. aop holds the A
// operands: zero (set once by the caller) except where the lane's row is
// nonzero, which only those lanes reload, block by block.
__device__ __forceinline__ float q6m_block(const uint8_t *lds, const uint8_t *stage, uint32_t rb,
                                           int b, Q6mLane ln, half8 (&aop)[8], const float *meta,
                                           int g) {
    using namespace q6m;
    // 8 bytes at an even LDS offset: the three aligned dwords around them
    const uint32_t sh = rb & 3u;
    const uint32_t *rw = reinterpret_cast<const uint32_t *>(stage + (rb & ~3u));
    auto ld8 = [&](uint32_t off, uint32_t &d0, uint32_t &d1) {  // off: a multiple of 4
        const uint32_t p0 = rw[off / 4], p1 = rw[off / 4 + 1], p2 = rw[off / 4 + 2];
        d0 = __builtin_amdgcn_alignbyte(p1, p0, sh);
        d1 = __builtin_amdgcn_alignbyte(p2, p1, sh);
    };
    const uint8_t *tb = lds + (uint32_t)b * TAB + ln.e;
#pragma unroll
    for (int c = 0; c < 8; ++c)
        if ((c & 3) == ln.hitq) aop[c] = *reinterpret_cast<const half8 *>(tb + 128 * c);
    f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int gh = 0; gh < 2; ++gh) {  // positions 128gh ..
        uint32_t qlA0, qlA1, qlB0, qlB1, qh0, qh1;
        ld8(64 * gh + 8 * g, qlA0, qlA1);       // quads 0, 2
        ld8(64 * gh + 32 + 8 * g, qlB0, qlB1);  // quads 1, 3
        ld8(128 + 32 * gh + 8 * g, qh0, qh1);
#pragma unroll
        for (int quad = 0; quad < 4; ++quad) {
            const int c = 4 * gh + quad;
            const uint32_t s0 = (quad & 1) ? qlB0 : qlA0, s1 = (quad & 1) ? qlB1 : qlA1;
            u32x4 bop;
            if (quad < 2) {
                // low nibbles: the 6-bit q bytes (nibble | qh bits << 4), then
                // bytes 0,2 and 1,3 into the low bytes of f16 halves: q*2^-24
                const int sh = 4 - 2 * quad;
                const uint32_t q0 = ((qh0 << sh) & 0x30303030u) | (s0 & 0x0F0F0F0Fu);
                const uint32_t q1 = ((qh1 << sh) & 0x30303030u) | (s1 & 0x0F0F0F0Fu);
                bop = u32x4{__builtin_amdgcn_perm(0u, q0, 0x0C020C00u), __builtin_amdgcn_perm(0u, q0, 0x0C030C01u),
                            __builtin_amdgcn_perm(0u, q1, 0x0C020C00u), __builtin_amdgcn_perm(0u, q1, 0x0C030C01u)};
            } else {
                // high nibbles in place (16*nibble) as a half's low byte and
                // the 2 qh bits as its high byte: 16*nibble + 256*qh = 16q,
                // i.e. 16q*2^-24 (the sub-block's corr carries the 1/16)
                const uint32_t m0 = s0 & 0xF0F0F0F0u, m1 = s1 & 0xF0F0F0F0u;
                const uint32_t h0 = (qh0 >> (2 * quad)) & 0x03030303u;
                const uint32_t h1 = (qh1 >> (2 * quad)) & 0x03030303u;
                bop = u32x4{__builtin_amdgcn_perm(h0, m0, 0x06020400u), __builtin_amdgcn_perm(h0, m0, 0x07030501u),
                            __builtin_amdgcn_perm(h1, m1, 0x06020400u), __builtin_amdgcn_perm(h1, m1, 0x07030501u)};
            }
            acc[gh] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop[c], __builtin_bit_cast(half8, bop),
                                                             acc[gh], 0, 0, 0);
        }
    }
    // this lane's sub-blocks g (acc[0]) and 4 + g (acc[1]) of row n16
    const float d = half_bits_finite((uint32_t)stage[rb + 208] | ((uint32_t)stage[rb + 209] << 8));
    const float *mb = meta + b * META;
    float y = 0.0f;
#pragma unroll
    for (int a = 0; a < 2; ++a) {
        const int j = 4 * a + g;
        const float sc0 = (float)(int8_t)stage[rb + 192 + 2 * j];
        const float sc1 = (float)(int8_t)stage[rb + 193 + 2 * j];
        const float s0 = acc[a][0] + acc[a][1], s1 = acc[a][2] + acc[a][3];
        y += d * (mb[j] * (sc0 * s0 + sc1 * s1) - 32.0f * (sc0 * mb[8 + 2 * j] + sc1 * mb[9 + 2 * j]));
    }
    return y;
}

// Row n16's sum over the 4 lane groups and the wavefronts -> ybuf[slot];
// ends with every wavefront done with the stage and aux.
template <int NW = q6m::NW>
__device__ __forceinline__ void q6m_row_sums(float yacc, float *aux, float *ybuf, int tid, int lane,
                                             int wave) {
    constexpr int R = q6m::R;
    yacc += __shfl_xor(yacc, 16, 64);
    yacc += __shfl_xor(yacc, 32, 64);
    if (lane < 16) aux[wave * R + lane] = yacc;
    __syncthreads();
    if (tid < R) {
        float s = 0.0f;
        for (int wv = 0; wv < NW; ++wv) s += aux[wv * R + tid];
        ybuf[tid] = s;
    }
}

// NORM: y = W * rms_norm(x, nw, eps) (the reference decode's launch_rms_norm
// + launch_matvec_q6k pair, rocm_gemma.rs:439-440), computed as
// rstd * (W * (x .* nw)): the table is built from x .* nw while sum(x^2) is
// reduced, and the rows are scaled once at the end.
template <bool NORM>
__global__ __launch_bounds__(q6m::NT) void gemv_q6k_mfma_kernel(const uint8_t *__restrict__ w,
                                                                const float *__restrict__ x,
                                                                float *__restrict__ y, int n,
                                                                int bpr, int rounds,
                                                                GemvSched sch,
                                                                const float *__restrict__ nw,
                                                                float eps) {
    using namespace q6m;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const Q6mLayout Lo = q6m_layout(bpr, rounds, false);
    float *meta = reinterpret_cast<float *>(lds + Lo.meta);
    float *aux = reinterpret_cast<float *>(lds + Lo.aux);
    float *ybuf = reinterpret_cast<float *>(lds + Lo.ybuf);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int RB = bpr * BB;            // row bytes; a group is RB 16-byte chunks
    const int groups = (n + R - 1) / R;
    const int my_groups = sched_count(sch, (int)blockIdx.x, (int)gridDim.x, groups);
    const u32x4 *wc = reinterpret_cast<const u32x4 *>(w);
    const long last_chunk = (long)n * RB / 16 - 1;

    // ---- stage loads: group q of this work-group, clamped (unconditional) ---
    u32x4 reg[CPL];
    auto gload = [&](int q) {
        q = min(q, my_groups - 1);
        const long base = (long)sched_group(sch, (int)blockIdx.x, (int)gridDim.x, q) * RB;
#pragma unroll
        for (int k = 0; k < CPL; ++k) {
            const int c = min(tid + k * NT, RB - 1);
            reg[k] = wc[min(base + c, last_chunk)];
        }
    };
    auto lstore = [&]() {
#pragma unroll
        for (int k = 0; k < CPL; ++k) {
            const int c = tid + k * NT;
            if (c < RB) *reinterpret_cast<u32x4 *>(lds + Lo.stage + 16 * c) = reg[k];
        }
    };

    // ---- prologue: the activation table (x loads first, then the weights) --
    // bpr <= 14 makes it at most one item per thread
    const int nitems = bpr * 32;
    const int ii = min(tid, nitems - 1);
    f32x4 v0 = ld_f32x4(x + (size_t)ii * 8);
    f32x4 v1 = ld_f32x4(x + (size_t)ii * 8 + 4);
    f32x4 n0, n1;
    if constexpr (NORM) {
        n0 = ld_f32x4(nw + (size_t)ii * 8);
        n1 = ld_f32x4(nw + (size_t)ii * 8 + 4);
    }
    gload(0);
    if constexpr (NORM) {
        // this item's sum of x^2 (a clamped duplicate past the end adds 0),
        // reduced per wavefront; the table holds x .* nw
        float ssq = tid < nitems ? ((v0[0] * v0[0] + v0[1] * v0[1]) + (v0[2] * v0[2] + v0[3] * v0[3])) +
                                       ((v1[0] * v1[0] + v1[1] * v1[1]) + (v1[2] * v1[2] + v1[3] * v1[3]))
                                 : 0.0f;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) ssq += __shfl_xor(ssq, off, 64);
        if (lane == 0) reinterpret_cast<float *>(lds + Lo.normp)[wave] = ssq;
        v0 *= n0;
        v1 *= n1;
    }
    q6m_item(lds, meta, tid, tid < nitems, v0, v1);
    lstore();
    gload(1);
    __syncthreads();

    const int n16 = lane & 15, g = lane >> 4;
    const Q6mLane ln = q6m_lane(lane);
    half8 aop[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) aop[c] = half8{};
    const uint8_t *stage = lds + Lo.stage;
    for (int q = 0; q < my_groups; ++q) {
        float yacc = 0.0f;
        for (int b = wave; b < bpr; b += NW)
            yacc += q6m_block(lds, stage, (uint32_t)(n16 * RB + b * BB), b, ln, aop, meta, g);
        q6m_row_sums(yacc, aux, ybuf + q * R, tid, lane, wave);
        lstore();       // group q + 1 (a clamped duplicate after the last)
        gload(q + 2);   // issued unconditionally, so every wait is exact
        __syncthreads();
    }
    float rstd = 1.0f;
    if constexpr (NORM) {
        // rms_norm's 1/sqrt(mean(x^2) + eps) (kernels/rms_norm.hip:63-68); the
        // partials were published by the barrier before the first group
        const float *np = reinterpret_cast<const float *>(lds + Lo.normp);
        float ss = 0.0f;
        for (int wv = 0; wv < NW; ++wv) ss += np[wv];
        rstd = rsqrtf(ss / (float)(bpr * kBlockElems) + eps);
    }
    for (int i = tid; i < my_groups * R; i += NT) {
        const int r = sched_group(sch, (int)blockIdx.x, (int)gridDim.x, i / R) * R + (i % R);
        if (r < n) y[r] = NORM ? ybuf[i] * rstd : ybuf[i];
    }
}

// Long rows: stage t = (group t / nck, K-chunk t % nck) of this work-group;
// chunk kc covers blocks [14 kc, min(14 kc + 14, bpr)) of the group's 16 rows.
template <int NW, int XI>
__global__ __launch_bounds__(NW * 64) void gemv_q6k_mfma_long_kernel(const uint8_t *__restrict__ w,
                                                                     const float *__restrict__ x,
                                                                     float *__restrict__ y, int n,
                                                                     int bpr, int rounds,
                                                                     GemvSched sch) {
    using q6m::R, q6m::BB, q6m::TAB, q6m::SEG, q6m::SLOTC;
    constexpr int NT = NW * 64, LCPL = (R * SLOTC + NT - 1) / NT;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const Q6mLayout Lo = q6m_layout(bpr, rounds, true, NW);
    float *meta = reinterpret_cast<float *>(lds + Lo.meta);
    float *aux = reinterpret_cast<float *>(lds + Lo.aux);
    float *ybuf = reinterpret_cast<float *>(lds + Lo.ybuf);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const long RB = (long)bpr * BB;
    const int groups = (n + R - 1) / R;
    const int my_groups = sched_count(sch, (int)blockIdx.x, (int)gridDim.x, groups);
    const int nck = (bpr + SEG - 1) / SEG;
    const int T = my_groups * nck;
    const u32x4 *wc = reinterpret_cast<const u32x4 *>(w);
    const long last_chunk = (long)n * RB / 16 - 1;

    // ---- stage loads: stage t, clamped (unconditional) ----------------------
    // slot chunk c = 16-byte chunk (c % SLOTC) of row c / SLOTC's segment,
    // taken from the 16-byte boundary at or below the segment's start
    u32x4 reg[LCPL];
    auto gload = [&](int t) {
        t = min(t, T - 1);
        const int q = t / nck, kc = t - q * nck;
        const int b0 = kc * SEG, cb = min(SEG, bpr - b0);
        const int row0 = sched_group(sch, (int)blockIdx.x, (int)gridDim.x, q) * R;
#pragma unroll
        for (int k = 0; k < LCPL; ++k) {
            const int c = min(tid + k * NT, R * SLOTC - 1);
            const int r = c / SLOTC, col = c - r * SLOTC;
            const long s = (long)min(row0 + r, n - 1) * RB + (long)b0 * BB;
            const int nch = (int)(((s & 15) + cb * BB + 15) >> 4);
            reg[k] = wc[min((s >> 4) + min(col, nch - 1), last_chunk)];
        }
    };
    auto lstore = [&]() {
#pragma unroll
        for (int k = 0; k < LCPL; ++k) {
            const int c = tid + k * NT;
            if (c < R * SLOTC) *reinterpret_cast<u32x4 *>(lds + Lo.stage + 16 * c) = reg[k];
        }
    };

    // ---- prologue: the whole row's activation table, XI items per thread ---
    const int nitems = bpr * 32;
    f32x4 xv[2 * XI];
#pragma unroll
    for (int k = 0; k < XI; ++k) {
        const int ii = min(tid + k * NT, nitems - 1);
        xv[2 * k] = ld_f32x4(x + (size_t)ii * 8);
        xv[2 * k + 1] = ld_f32x4(x + (size_t)ii * 8 + 4);
    }
    gload(0);
#pragma unroll
    for (int k = 0; k < XI; ++k)
        q6m_item(lds, meta, tid + k * NT, tid + k * NT < nitems, xv[2 * k], xv[2 * k + 1]);
    lstore();
    gload(1);
    __syncthreads();

    const int n16 = lane & 15, g = lane >> 4;
    const Q6mLane ln = q6m_lane(lane);
    half8 aop[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) aop[c] = half8{};
    const uint8_t *stage = lds + Lo.stage;
    float yacc = 0.0f;
    for (int t = 0; t < T; ++t) {
        const int q = t / nck, kc = t - q * nck;
        const int b0 = kc * SEG, cb = min(SEG, bpr - b0);
        const int row = min(sched_group(sch, (int)blockIdx.x, (int)gridDim.x, q) * R + n16, n - 1);
        const uint32_t rb0 =
            (uint32_t)(n16 * SLOTC * 16) + (uint32_t)(((long)row * RB + (long)b0 * BB) & 15);
        for (int bl = wave; bl < cb; bl += NW)
            yacc += q6m_block(lds, stage, rb0 + (uint32_t)(bl * BB), b0 + bl, ln, aop, meta, g);
        if (kc == nck - 1) {
            q6m_row_sums<NW>(yacc, aux, ybuf + q * R, tid, lane, wave);
            yacc = 0.0f;
        } else {
            __syncthreads();  // every wavefront is done with the stage
        }
        lstore();       // stage t + 1 (a clamped duplicate after the last)
        gload(t + 2);   // issued unconditionally, so every wait is exact
        __syncthreads();
    }
    for (int i = tid; i < my_groups * R; i += NT) {
        const int r = sched_group(sch, (int)blockIdx.x, (int)gridDim.x, i / R) * R + (i % R);
        if (r < n) y[r] = ybuf[i];
    }
}

// Long rows, wave-private: wavefront w takes blocks w, w + NW, ... of every
// row group of the work-group in turn (a unit = one block of the 16 rows); it
// copies the unit's 16 row segments (from the 16-byte boundary at or below
// each segment's start: 14 chunks hold the 210 bytes and the offset) into its
// own LDS slot (rows 15 chunks apart: the 16 rows' reads of one offset fall
// in 16 different bank groups) and computes from it while its next unit
// loads; no work-group barrier between units. Its row sums of every group go
// to its own LDS rows, and the work-group adds them over the wavefronts once,
// at the end.
namespace q6w {
constexpr int CH = 14;                        // 16-byte chunks per row segment
constexpr int PITCH = 15;                     // chunks per slot row
constexpr int UP = q6m::R * CH;               // chunks per unit (224)
constexpr int IPU = (UP + 63) / 64;           // wave loads per unit (4)
constexpr uint32_t SLOT = (uint32_t)q6m::R * PITCH * 16u;
}  // namespace q6w

__host__ __device__ inline Q6mLayout q6w_layout(int bpr, int rounds, int nw) {
    using namespace q6m;
    Q6mLayout L;
    L.meta = (uint32_t)bpr * TAB;
    L.stage = L.meta + (uint32_t)bpr * META * 4;
    L.aux = L.stage + (uint32_t)nw * q6w::SLOT;
    L.ybuf = L.aux + (uint32_t)rounds * nw * R * 4;  // (aux: rounds x nw x R row sums)
    L.normp = L.ybuf;                                 // fused RMSNorm: one sum(x^2) per wavefront
    L.total = (size_t)L.normp + (size_t)nw * 4;
    return L;
}

template <int NW, int XI, bool NORM = false>
__global__ __launch_bounds__(NW * 64) void gemv_q6k_wave_long_kernel(const uint8_t *__restrict__ w,
                                                                     const float *__restrict__ x,
                                                                     float *__restrict__ y, int n,
                                                                     int bpr, int rounds,
                                                                     GemvSched sch,
                                                                     const float *__restrict__ nw = nullptr,
                                                                     float eps = 0.0f) {
    using q6m::R, q6m::BB, q6m::TAB;
    using q6w::CH, q6w::PITCH, q6w::UP, q6w::IPU;
    constexpr int NT = NW * 64;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const Q6mLayout Lo = q6w_layout(bpr, rounds, NW);
    float *meta = reinterpret_cast<float *>(lds + Lo.meta);
    float *aux = reinterpret_cast<float *>(lds + Lo.aux);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    uint8_t *slot = lds + Lo.stage + (uint32_t)wave * q6w::SLOT;
    const long RB = (long)bpr * BB;
    const uint64_t last_off = ((uint64_t)n * RB / 16 - 1) * 16;  // the last whole chunk

    // chunk p of a unit: row p / CH, chunk p % CH of its segment (the 16-byte
    // chunks that hold the row's 210 bytes of the block)
    uint32_t prb[IPU], pc16[IPU], plds[IPU];
#pragma unroll
    for (int k = 0; k < IPU; ++k) {
        const int p = min(k * 64 + lane, UP - 1);
        const int row = p / CH, ch = p - row * CH;
        prb[k] = (uint32_t)row * (uint32_t)RB;
        pc16[k] = (uint32_t)(16 * ch);
        plds[k] = (uint32_t)((row * PITCH + ch) * 16);
    }
    u32x4 stg[IPU];
    // the unit (group row0, block b): the chunk-aligned start of its first row
    // segment as a uniform base, and per lane its row's chunk offset from it,
    // so a unit's loads go out a few VALU after the previous unit's slot
    // stores; chunks past the tensor's last whole chunk (rows past n, which
    // no result uses) read that chunk
    struct UnitAddr {
        const uint8_t *base;
        uint32_t mis, lim;
    };
    auto uaddr = [&](int row0, int b) -> UnitAddr {
        const uint64_t s = (uint64_t)row0 * RB + (uint64_t)b * BB, s16 = s & ~15ull;
        return UnitAddr{w + s16, (uint32_t)(s & 15), (uint32_t)min(last_off - s16, (uint64_t)0xFFFFFFF0u)};
    };
    auto gload_u = [&](const UnitAddr &a) {
#pragma unroll
        for (int k = 0; k < IPU; ++k) {
            const uint32_t o = ((a.mis + prb[k]) & ~15u) + pc16[k];
            stg[k] = ld_u32x4(a.base + min(o, a.lim));
        }
    };
    // this wavefront's blocks per group: w, w + NW, ...
    const int nb = wave < bpr ? (bpr - wave + NW - 1) / NW : 0;
    gload_u(uaddr((int)blockIdx.x * R, min(wave, bpr - 1)));  // group 0 of every schedule is blockIdx.x
    const int groups = (n + R - 1) / R;
    const int my_groups = sched_count(sch, (int)blockIdx.x, (int)gridDim.x, groups);
    const int U = my_groups * nb;

    // ---- prologue: the whole row's activation table, XI items per thread ---
    const int nitems = bpr * 32;
    f32x4 xv[2 * XI];
#pragma unroll
    for (int k = 0; k < XI; ++k) {
        const int ii = min(tid + k * NT, nitems - 1);
        xv[2 * k] = ld_f32x4(x + (size_t)ii * 8);
        xv[2 * k + 1] = ld_f32x4(x + (size_t)ii * 8 + 4);
    }
    float *normp = reinterpret_cast<float *>(lds + Lo.normp);
    if constexpr (NORM) {
        // sum(x^2) of this thread's items (clamped duplicates add 0), reduced
        // per wavefront; the table holds x .* nw (as gemv_q6k_mfma_kernel)
        float ssq = 0.0f;
#pragma unroll
        for (int k = 0; k < XI; ++k) {
            const f32x4 v0 = xv[2 * k], v1 = xv[2 * k + 1];
            const float s = ((v0[0] * v0[0] + v0[1] * v0[1]) + (v0[2] * v0[2] + v0[3] * v0[3])) +
                            ((v1[0] * v1[0] + v1[1] * v1[1]) + (v1[2] * v1[2] + v1[3] * v1[3]));
            ssq += tid + k * NT < nitems ? s : 0.0f;
            const int ii = min(tid + k * NT, nitems - 1);
            xv[2 * k] = v0 * ld_f32x4(nw + (size_t)ii * 8);
            xv[2 * k + 1] = v1 * ld_f32x4(nw + (size_t)ii * 8 + 4);
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) ssq += __shfl_xor(ssq, off, 64);
        if (lane == 0) normp[wave] = ssq;
    }
#pragma unroll
    for (int k = 0; k < XI; ++k)
        q6m_item(lds, meta, tid + k * NT, tid + k * NT < nitems, xv[2 * k], xv[2 * k + 1]);
    // a wavefront with no blocks contributes zero rows
    if (nb == 0)
        for (int i = lane; i < my_groups * R; i += 64) aux[((i / R) * NW + wave) * R + i % R] = 0.0f;
    __syncthreads();  // the table is complete; from here no wavefront waits for another

    const int n16 = lane & 15, g = lane >> 4;
    const Q6mLane ln = q6m_lane(lane);
    half8 aop[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) aop[c] = half8{};
    float yacc = 0.0f;
    int q = 0, k = 0;  // group index and block index (of nb) of unit u
    for (int u = 0; u < U; ++u) {
        // the next unit (past the last one: the last again, a cache hit), its
        // base worked out before the slot stores wait for this unit's data
        int q1 = q, k1 = k + 1;
        if (k1 == nb) {
            k1 = 0;
            q1 = q + 1;
        }
        if (q1 >= my_groups) {
            q1 = my_groups - 1;
            k1 = nb - 1;
        }
        const UnitAddr na = uaddr(sched_group(sch, (int)blockIdx.x, (int)gridDim.x, q1) * R, wave + k1 * NW);
#pragma unroll
        for (int i = 0; i < IPU; ++i) *reinterpret_cast<u32x4 *>(slot + plds[i]) = stg[i];
        __asm__ volatile("" ::: "memory");  // the unit's reads follow its stores (in-order LDS)
        gload_u(na);  // unconditional, so the load-counter waits stay exact
        const int b = wave + k * NW;
        const int row = min(sched_group(sch, (int)blockIdx.x, (int)gridDim.x, q) * R + n16, n - 1);
        const uint32_t rb = (uint32_t)(n16 * PITCH * 16) + (uint32_t)(((long)row * RB + (long)b * BB) & 15);
        yacc += q6m_block(lds, slot, rb, b, ln, aop, meta, g);
        if (++k == nb) {
            yacc += __shfl_xor(yacc, 16, 64);
            yacc += __shfl_xor(yacc, 32, 64);
            if (lane < 16) aux[(q * NW + wave) * R + lane] = yacc;
            yacc = 0.0f;
            k = 0;
            ++q;
        }
    }
    __syncthreads();
    float rstd = 1.0f;
    if constexpr (NORM) {
        // rms_norm's 1/sqrt(mean(x^2) + eps) (kernels/rms_norm.hip:63-68)
        float ss = 0.0f;
        for (int wv = 0; wv < NW; ++wv) ss += normp[wv];
        rstd = rsqrtf(ss / (float)(bpr * kBlockElems) + eps);
    }
    for (int i = tid; i < my_groups * R; i += NT) {
        const int qi = i / R, ri = i % R;
        const int r = sched_group(sch, (int)blockIdx.x, (int)gridDim.x, qi) * R + ri;
        if (r < n) {
            float s = 0.0f;
            for (int wv = 0; wv < NW; ++wv) s += aux[(qi * NW + wv) * R + ri];
            y[r] = NORM ? s * rstd : s;
        }
    }
}

namespace {

// LDS attribute and occupancy of `kern` for rows of up to `probe_bpr` blocks
// on the current device (both cached: only the first call per device asks
// the runtime).
template <typename K>
hipError_t q6m_setup(K kern, bool chunked, int nw, int probe_bpr, int *occ) {
    using namespace q6m;
    const hipError_t attr = allow_full_lds_by_addr((const void *)kern);
    if (attr != hipSuccess) return attr;
    *occ = occupancy_cached((const void *)kern, nw * 64, q6m_layout(probe_bpr, 32, chunked, nw).total, 1);
    return hipSuccess;
}

// Persistent launch of `kern` with the occupancy at `probe_bpr` blocks per row
// (persistent_plan: balanced, or age-skewed for pairs of work-groups per CU).
template <typename K, typename... Extra>
hipError_t q6m_launch(K kern, bool chunked, int nw, const uint8_t *w, const float *x, float *y,
                      int n, int bpr, int probe_bpr, hipStream_t stream, Extra... extra) {
    using namespace q6m;
    int occ = 1;
    const hipError_t attr = q6m_setup(kern, chunked, nw, probe_bpr, &occ);
    if (attr != hipSuccess) return attr;
    const PersistPlan p = persistent_plan((n + R - 1) / R, occ);
    const size_t lds = q6m_layout(bpr, (int)p.rounds, chunked, nw).total;
    if (lds > 160 * 1024) return hipErrorNotSupported;
    kern<<<(unsigned)p.grid, nw * 64, lds, stream>>>(w, x, y, n, bpr, (int)p.rounds, p.sch, extra...);
    return hipGetLastError();
}

// rows of the long (K-chunked) kernel with XI table items per thread: at most
template <int NW, int XI>
constexpr int q6m_long_probe() { return std::min(XI * NW * 64 / 32, 100); }

template <int NW, int XI>
hipError_t q6m_long_launch(const uint8_t *w, const float *x, float *y, int n, int bpr,
                           hipStream_t stream) {
    // occupancy at the largest row this instance serves
    return q6m_launch(gemv_q6k_mfma_long_kernel<NW, XI>, true, NW, w, x, y, n, bpr,
                      q6m_long_probe<NW, XI>(), stream);
}

template <int NW, int XI, bool NORM = false>
hipError_t q6w_long_setup(int *occ) {
    const void *kern = (const void *)gemv_q6k_wave_long_kernel<NW, XI, NORM>;
    const hipError_t attr = allow_full_lds_by_addr(kern);
    if (attr != hipSuccess) return attr;
    *occ = occupancy_cached(kern, NW * 64, q6w_layout(q6m_long_probe<NW, XI>(), 8, NW).total, 1);
    return hipSuccess;
}

template <int NW, int XI, bool NORM = false>
hipError_t q6w_long_launch(const uint8_t *w, const float *x, float *y, int n, int bpr,
                           hipStream_t stream, const float *nw = nullptr, float eps = 0.0f) {
    int occ = 1;
    const hipError_t attr = q6w_long_setup<NW, XI, NORM>(&occ);
    if (attr != hipSuccess) return attr;
    const PersistPlan p = persistent_plan((n + q6m::R - 1) / q6m::R, occ);
    const size_t lds = q6w_layout(bpr, (int)p.rounds, NW).total;
    if (lds > 160 * 1024) return hipErrorNotSupported;
    gemv_q6k_wave_long_kernel<NW, XI, NORM><<<(unsigned)p.grid, NW * 64, lds, stream>>>(
        w, x, y, n, bpr, (int)p.rounds, p.sch, nw, eps);
    return hipGetLastError();
}

template <int NW, int XI>
hipError_t q6m_long_setup() {
    int occ = 0;
    return q6m_setup(gemv_q6k_mfma_long_kernel<NW, XI>, true, NW, q6m_long_probe<NW, XI>(), &occ);
}

}  // namespace

// Sets every Q6_K matrix-core kernel's LDS attribute and caches its occupancy
// on the current device, so that no launcher makes those runtime calls later
// (e.g. inside a stream capture).
hipError_t q6k_prepare() {
    using namespace q6m;
    int occ = 0;
    hipError_t e = q6m_setup(gemv_q6k_mfma_kernel<false>, false, NW, MAX_BPR, &occ);
    if (e == hipSuccess) e = q6m_setup(gemv_q6k_mfma_kernel<true>, false, NW, MAX_BPR, &occ);
    if (e == hipSuccess) e = q6m_long_setup<LONG_NW, 1>();
    if (e == hipSuccess) e = q6m_long_setup<LONG_NW, 2>();
    if (e == hipSuccess) e = q6m_long_setup<LONG_NW, 4>();
    if (e == hipSuccess) e = q6m_long_setup<LONG_NW, 6>();
    if (e == hipSuccess) e = q6m_long_setup<LONG_NW, 8>();
    if (e == hipSuccess) e = q6w_long_setup<LONG_NW, 1>(&occ);
    if (e == hipSuccess) e = q6w_long_setup<LONG_NW, 2>(&occ);
    if (e == hipSuccess) e = q6w_long_setup<LONG_NW, 4>(&occ);
    if (e == hipSuccess) e = q6w_long_setup<LONG_NW, 6>(&occ);
    if (e == hipSuccess) e = q6w_long_setup<LONG_NW, 8>(&occ);
    if (e == hipSuccess) e = q6w_long_setup<14, 1, true>(&occ);
    return e;
}

hipError_t gemv_q6k_mfma_launch(const uint8_t *w, const float *x, float *y, int n, int bpr,
                                hipStream_t stream) {
    using namespace q6m;
    // whole 16-byte chunks from w up to the tensor end: w 16-byte aligned and
    // a tensor size that is a multiple of 16 (x needs only float alignment)
    if (((uintptr_t)w & 15u) || (((long)n * bpr * BB) % 16))
        return hipErrorNotSupported;
    // (the wave-private kernel over 14 wavefronts, one block each, measured
    // no faster on the plain lm_head: 86.0 -> 86.4-86.8 us; the whole-row
    // kernel stays for plain rows of up to 14 blocks)
    if (bpr <= MAX_BPR)
        return q6m_launch(gemv_q6k_mfma_kernel<false>, false, NW, w, x, y, n, bpr, MAX_BPR, stream,
                          (const float *)nullptr, 0.0f);
    constexpr int LNW = LONG_NW, LNT = LNW * 64;
    const int need = (bpr * 32 + LNT - 1) / LNT;  // table items per thread
    // wave-private long rows (no barrier between units; all 16 wavefronts
    // busy on 74 blocks where 14-block stages left 2 idle): Q4_K_M decode
    // step 1.414 -> 1.364 ms, alternating on one box; the staged kernel for
    // rows whose table and slots exceed LDS (bpr > ~80). MGQ_Q6K_WAVE=0
    // selects the staged kernel.
    static const int wave_env = [] {
        const char *v = std::getenv("MGQ_Q6K_WAVE");
        return (v && *v) ? std::atoi(v) : 1;
    }();
    if (wave_env) {
        hipError_t ew = hipErrorNotSupported;
        if (need <= 1) ew = q6w_long_launch<LNW, 1>(w, x, y, n, bpr, stream);
        else if (need <= 2) ew = q6w_long_launch<LNW, 2>(w, x, y, n, bpr, stream);
        else if (need <= 4) ew = q6w_long_launch<LNW, 4>(w, x, y, n, bpr, stream);
        else if (need <= 6) ew = q6w_long_launch<LNW, 6>(w, x, y, n, bpr, stream);
        else if (need <= 8) ew = q6w_long_launch<LNW, 8>(w, x, y, n, bpr, stream);
        if (ew != hipErrorNotSupported) return ew;
    }
    if (need <= 1) return q6m_long_launch<LNW, 1>(w, x, y, n, bpr, stream);
    if (need <= 2) return q6m_long_launch<LNW, 2>(w, x, y, n, bpr, stream);
    if (need <= 4) return q6m_long_launch<LNW, 4>(w, x, y, n, bpr, stream);
    if (need <= 6) return q6m_long_launch<LNW, 6>(w, x, y, n, bpr, stream);
    if (need <= 8) return q6m_long_launch<LNW, 8>(w, x, y, n, bpr, stream);
    return hipErrorNotSupported;
}

hipError_t gemv_q6k_mfma_norm_launch(const uint8_t *w, const float *x, const float *nw, float eps,
                                     float *y, int n, int bpr, hipStream_t stream) {
    using namespace q6m;
    // the whole-row kernel only: 16-byte aligned w, a tensor size that is a
    // multiple of 16, K <= MAX_BPR blocks (the shapes a norm feeds: q|k|v,
    // the output matrix)
    if (((uintptr_t)w & 15u) || (((long)n * bpr * BB) % 16) || bpr > MAX_BPR)
        return hipErrorNotSupported;
    // The wave-private kernel, one block per wavefront over 14 wavefronts
    // (no barrier between the copy and the compute): Q4_K_M decode step,
    // whose fused-norm Q6_K launches are attn_v (512 rows) and the output
    // matrix, 1.367 -> 1.356 ms alternating on one box. MGQ_Q6K_WHOLE_WAVE=0
    // keeps the whole-row kernel.
    static const int whole_env = [] {
        const char *v = std::getenv("MGQ_Q6K_WHOLE_WAVE");
        return (v && *v) ? std::atoi(v) : 1;
    }();
    if (whole_env) {
        const hipError_t ew = q6w_long_launch<14, 1, true>(w, x, y, n, bpr, stream, nw, eps);
        if (ew != hipErrorNotSupported) return ew;
    }
    return q6m_launch(gemv_q6k_mfma_kernel<true>, false, NW, w, x, y, n, bpr, MAX_BPR, stream, nw,
                      eps);
}

}  // namespace mgq
