// Batched Q4_K GEMV on the gfx950 matrix cores: Y[b][r] = dequant(W)[r] . X[b]
// for b < batch <= 16 (multi-sequence decode). No counterpart in the
// reference; the oracle is its f64 dequant-dot (rocm_matvec_check.rs:38-47)
// applied row by row.
//
// Three kernels:
//
// 1. batched_table_kernel turns X into matrix-core A operands, once per call,
//    in a caller-provided workspace. Batch b of a set of 8 occupies MFMA rows
//    m = 2*(b%8) + part, where x*2^e = xh + xl (part 0 = xh, 1 = xl, both f16)
//    with one power of two e per (batch, block). The k-slot order of every
//    16-byte entry matches the weight operand built from qs (below). A ninth
//    operand per (block, set) carries the 8 sub-block sums of x (same split)
//    for the dmin*m term.
//
// 2. gemv_batched_wave_kernel (the default) and 3. gemv_batched_mfma_kernel
//    (the stage kernel: shapes whose per-wavefront row sums do not fit LDS)
//    keep the batch on the MFMA M dimension, so one weight operand serves 8
//    batch rows per v_mfma_f32_16x16x32_f16. The wave kernel has every
//    wavefront stage its own units (R rows x 1-2 blocks) with no barrier
//    between them; the stage kernel streams 16 rows x 8 blocks per stage
//    through LDS as the GEMV's stage kernel does. Both:
//      * B operand = sc*q: the nibble masked in place is the f16 subnormal
//        q*2^-24 (low) or 16q*2^-24 (high); one packed f16 multiply by 16*sc
//        (low) or sc (high) makes it q*sc*2^-20 exactly (q*sc <= 945 fits the
//        f16 significand), so all 8 sub-blocks of a block accumulate into one
//        accumulator and only d is applied afterwards.
//      * min term: one more MFMA per block with the sub-block sums of x
//        (A) against m[0..7] of each row (B).
//      * Work runs K-slice-major (all of a work-group's row groups for one
//        slice of blocks, then the next), so a wavefront keeps the A
//        operands of its blocks of the slice in registers for the whole
//        slice.
//      * Shapes with few row groups and a long K split K in two: the table
//        kernel zeroes Y and each half adds its partials atomically (two
//        addends onto 0 round the same in either order).
#include "q4k_device.hpp"
#include "q4k_launch.hpp"

#include <algorithm>
#include <cstdlib>
#include <type_traits>
#include <utility>

namespace mgq {

// stage kernel: weight stages in flight for one / two batch sets (measurements
// at its launcher)
#ifndef MGQ_BPF1
#define MGQ_BPF1 2
#endif
#ifndef MGQ_BPF2
#define MGQ_BPF2 1
#endif

constexpr int kBatchOps = 9;  // A operands per (block, set): 8 k-slot groups + sub-block sums

// Workspace layout (bytes): atab [bpr][sets][9][64 lanes][16 B], then meta
// [bpr][sets][8 batches][corr, corr_min] f32.
struct BatchedWs {
    size_t meta, total;
};
__host__ __device__ inline BatchedWs batched_ws(int bpr, int sets) {
    BatchedWs L;
    L.meta = (size_t)bpr * sets * kBatchOps * 1024;
    L.total = L.meta + (size_t)bpr * sets * 8 * 8;
    return L;
}

size_t batched_workspace_bytes(int bpr, int batch) {
    return batched_ws(bpr, (batch + 7) / 8).total;
}

// Byte offset inside qs[128] of the 8 bytes that lane group g reads for
// pair p (the same map the GEMV uses): pairs 0,1 from qs[16g..16g+15],
// pairs 2,3 from qs[64+16g..64+16g+15].
__device__ __forceinline__ int bt_pair_offset(int p, int g) {
    return p < 2 ? 16 * g + 8 * p : 64 + 16 * g + 8 * (p - 2);
}

// exponent e with max|v|*2^e in [2^13, 2^14); 0 for 0 or non-finite
__device__ __forceinline__ int split_exponent(float amax) {
    int e = 0;
    if (amax > 0.0f && amax <= 3.402823466e38f) {
        int ex;
        frexpf(amax, &ex);
        e = std::min(std::max(14 - ex, -103), 120);  // 2^(20 - e) stays finite
    }
    return e;
}

// max over the 16 lanes of each DPP row (quad xor 1, quad xor 2, half-row
// mirror, row mirror: every lane ends with the row's max)
__device__ __forceinline__ float row_max16(float v) {
    v = fmaxf(v, quad_xor<1>(v));
    v = fmaxf(v, quad_xor<2>(v));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                                       0x141, 0xF, 0xF, false)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                                       0x140, 0xF, 0xF, false)));
    return v;
}

// grid (ceil(bpr / 2), sets), 256 threads = 2 blocks x 8 batches x 16
// threads: one 16-lane DPP row per batch; thread h of batch b' holds the
// 8-float chunks 2h and 2h+1 of block j (sub-block h / 2). Every A-operand
// entry of the 8 k-slot groups holds one aligned 8-float chunk of the block
// (its values in k-slot order 0,2,1,3,4,6,5,7): entry (c, g) takes chunk
// 16(c>>2) + 8(g>>1) + 4(c&1) + 2(g&1) + ((c>>1)&1) (bt_pair_offset), so the
// thread that loaded a chunk writes its two entries (xh and xl rows of its
// batch) from registers. The block max takes four DPP steps inside the row
// and the sub-block sum ((c0 + c1) + (c2 + c3) over its chunk sums) one; a
// layout of 32 lanes per batch needed five and two dependent lane shuffles
// (same table, ~0.1 us per call less).
__global__ __launch_bounds__(256) void batched_table_kernel(const float *__restrict__ X, int batch,
                                                            int bpr, int sets, bool x_aligned16,
                                                            uint8_t *__restrict__ ws,
                                                            float *__restrict__ yzero, int ytotal) {
    // Y = 0 ahead of a K-split main kernel (it adds its partials atomically)
    {
        const int nthr = (int)(gridDim.x * gridDim.y) * 256;
        for (int i = (int)(blockIdx.y * gridDim.x + blockIdx.x) * 256 + (int)threadIdx.x; i < ytotal;
             i += nthr)
            yzero[i] = 0.0f;
    }
    const int tid = threadIdx.x, s = blockIdx.y;
    const int j = (int)blockIdx.x * 2 + (tid >> 7);
    if (j >= bpr) return;  // both wavefronts of the missing block
    const int bl = (tid >> 4) & 7, h = tid & 15, b = s * 8 + bl;
    const size_t K = (size_t)bpr * kBlockElems;
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = 0.0f;
    if (b < batch) {
        const float *xp = X + (size_t)b * K + (size_t)j * kBlockElems + h * 16;
        if (x_aligned16) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const f32x4 a = ld_f32x4(xp + 4 * q);
                v[4 * q] = a[0]; v[4 * q + 1] = a[1]; v[4 * q + 2] = a[2]; v[4 * q + 3] = a[3];
            }
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = xp[i];
        }
    }
    float amax = 0.0f, c0 = 0.0f, c1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        amax = fmaxf(amax, fmaxf(fabsf(v[i]), fabsf(v[8 + i])));
        c0 += v[i];
        c1 += v[8 + i];
    }
    // sub-block sum ((c0 + c1) + (c2 + c3)) of its four chunks, in both lanes
    float sum = c0 + c1;
    sum += quad_xor<1>(sum);
    const int e = split_exponent(row_max16(amax));
    float *meta = reinterpret_cast<float *>(ws + batched_ws(bpr, sets).meta);
    const size_t js = (size_t)j * sets + s;
    if (h == 0) meta[(js * 8 + bl) * 2] = ldexpf(1.0f, 20 - e);

    uint8_t *atab = ws + js * kBatchOps * 1024;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int ch = 2 * h + t;
        const int c = (((ch >> 4) & 1) << 2) | ((ch & 1) << 1) | ((ch >> 2) & 1);
        const int g = (((ch >> 3) & 1) << 1) | ((ch >> 1) & 1);
        constexpr int perm[8] = {0, 2, 1, 3, 4, 6, 5, 7};
        half8 hi, lo;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float xv = ldexpf(v[8 * t + perm[q]], e);
            const _Float16 hh = (_Float16)xv;
            hi[q] = hh;
            lo[q] = (_Float16)(xv - (float)hh);
        }
        uint8_t *dst = atab + (size_t)c * 1024 + (size_t)(2 * bl + 16 * g) * 16;
        *reinterpret_cast<half8 *>(dst) = hi;
        *reinterpret_cast<half8 *>(dst + 16) = lo;
    }
    // sub-block-sum operand: lanes (m = 2b' + part, g = 0) hold the 8 sums of
    // batch b', lanes with g != 0 zero; thread h < 8 of batch b' writes lane
    // (2b' + (h & 1)) + 16 (h >> 1). Sum q is in lanes 2q, 2q+1 of the row.
    float sq[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) sq[q] = __shfl(sum, (tid & 48) + 2 * q, 64);
    if (h < 8) {
        const int part = h & 1, g = h >> 1;
        float smax = 0.0f;
#pragma unroll
        for (int q = 0; q < 8; ++q) smax = fmaxf(smax, fabsf(sq[q]));
        const int es = split_exponent(smax);
        half8 out;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float xv = ldexpf(sq[q], es);
            const _Float16 hh = (_Float16)xv;
            out[q] = g != 0 ? (_Float16)0.0f : (part ? (_Float16)(xv - (float)hh) : hh);
        }
        *reinterpret_cast<half8 *>(atab + (size_t)8 * 1024 + (size_t)(2 * bl + part + 16 * g) * 16) = out;
        if (g == 0 && part == 0) meta[(js * 8 + bl) * 2 + 1] = ldexpf(1.0f, -es);
    }
}

// Two f16 values from the bytes of src that sel picks for result bytes 0 and
// 2 (v_perm_b32 selectors 0..3; 4 picks 0x64): 1024 + byte via the
// exponent field, minus 1024 (both exact).
__device__ __forceinline__ uint32_t byte_to_h2(uint32_t src, uint32_t sel) {
    const uint32_t biased = __builtin_amdgcn_perm(0x64646464u, src, sel);
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 r = __builtin_bit_cast(h2, biased) - (h2){(_Float16)1024.0f, (_Float16)1024.0f};
    return __builtin_bit_cast(uint32_t, r);
}

// Work-group = 8 waves; stage = R (16; 32 also compiles) rows x 8 blocks (single LDS
// buffer), PF stages in flight; persistent over row groups. SETS = batch sets
// of 8.
template <int R, int SETS, int PF>
__global__ __launch_bounds__(512) void gemv_batched_mfma_kernel(const uint8_t *__restrict__ w,
                                                                const uint8_t *__restrict__ ws,
                                                                float *__restrict__ Y, int n,
                                                                int bpr, int batch, int rounds,
                                                                int kparts) {
    constexpr int C = 8, NW = 8, BP = 8 * SETS, TILES = R / 16;
    constexpr int RP = (9 * C) | 1;               // LDS pieces per staged row (odd: no bank conflicts)
    constexpr int STAGE_BYTES = R * RP * 16;
    constexpr int AUX_BYTES = NW * R * BP * 4;    // per buffer
    constexpr int PIECES = R * 9 * C;
    constexpr int IPW = ((PIECES + 63) / 64 + NW - 1) / NW;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    float *aux0 = reinterpret_cast<float *>(lds + STAGE_BYTES);
    float *ybuf = reinterpret_cast<float *>(lds + STAGE_BYTES + 2 * AUX_BYTES);

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const size_t row_bytes = (size_t)bpr * kBlockBytes;
    // K split (kparts = 1 or 2): work-group id = kp * G + bx; K part kp takes
    // slices [sl0, sl0 + slices) of all of them (kparts <= slices overall).
    // Shifts only: the first stage's loads go out before any division.
    const int G = (int)gridDim.x >> (kparts - 1);
    const int kp = (int)blockIdx.x >= G ? 1 : 0, bx = (int)blockIdx.x - kp * G;
    const int all_slices = (bpr + C - 1) / C;
    const int spk = (all_slices + kparts - 1) >> (kparts - 1);
    const int sl0 = kp * spk;
    const int slices = std::min(all_slices, sl0 + spk) - sl0;

    u32x4 stg[PF][IPW];
    uint32_t prow[IPW], pcol[IPW], plast[IPW], plds[IPW];
#pragma unroll
    for (int k = 0; k < IPW; ++k) {
        const int jp = std::min((wave + k * NW) * 64 + lane, PIECES - 1);
        const int row = jp / (9 * C), rem = jp - row * 9 * C;
        const int cb = rem / 9, pc = rem - cb * 9;
        plds[k] = (uint32_t)((row * RP + rem) * 16);
        prow[k] = (uint32_t)row;
        pcol[k] = (uint32_t)(cb * kBlockBytes + 16 * pc);
        plast[k] = (uint32_t)((bpr - 1) * kBlockBytes + 16 * pc);
    }
    // stage of the R rows from r0 at byte column tcol
    auto gload_at = [&](uint32_t r0, uint32_t tcol, u32x4(&dst)[IPW]) {
        const uint32_t rlast = (uint32_t)(n - 1), rb = (uint32_t)row_bytes;
#pragma unroll
        for (int k = 0; k < IPW; ++k) {
            const uint32_t rr = std::min(r0 + prow[k], rlast);
            const uint32_t col = std::min(tcol + pcol[k], plast[k]);
            dst[k] = ld_u32x4(w + (uint64_t)rr * rb + col);
        }
    };
    // stage 0 = (slice 0, group 0 = bx); every work-group has at least one
    // group in its K part
    gload_at((uint32_t)bx * R, (uint32_t)(sl0 * C * kBlockBytes), stg[0]);
    const int groups = (n + R - 1) / R;
    const int my_groups = (groups - bx + G - 1) / G;
    const int Q = my_groups * slices;  // stage q = (slice q / my_groups, group q % my_groups)
    auto gload = [&](int q, u32x4(&dst)[IPW]) {
        q = std::min(q, Q - 1);
        const int sl = q / my_groups, t = q - sl * my_groups;
        gload_at(((uint32_t)bx + (uint32_t)t * (uint32_t)G) * R,
                 (uint32_t)((sl0 + sl) * C * kBlockBytes), dst);
    };
    auto lstore = [&](const u32x4(&src)[IPW]) {
#pragma unroll
        for (int k = 0; k < IPW; ++k) *reinterpret_cast<u32x4 *>(lds + plds[k]) = src[k];
    };
    const int n16 = lane & 15, g = lane >> 4, hsel = g >> 1;
    // byte selectors for this lane's scales: sub-blocks 2h, 2h+1 of a
    // scales4 word (bytes 2h, 2h+1)
    const uint32_t sel0 = 0x04000400u | (uint32_t)(2 * hsel) | ((uint32_t)(2 * hsel) << 16);
    const uint32_t sel1 = sel0 + 0x00010001u;
    const BatchedWs Lw = batched_ws(bpr, SETS);

    // A operands of this wave's block of the current slice, and of the next
    // slice: the next slice's are loaded during the current slice's last
    // stage, ahead of that stage's weight refill, so waiting for them never
    // drains the weight stream.
    u32x4 areg[SETS][kBatchOps], anext[SETS][kBatchOps];
    f32x4 mreg[SETS], mnext[SETS];  // (corr, corr_min) of batches 2g, 2g+1 of each set
    auto load_a = [&](int sl, u32x4(&a)[SETS][kBatchOps], f32x4(&mr)[SETS]) {
        const int jb = std::min((sl0 + sl) * C + wave, bpr - 1);
#pragma unroll
        for (int s = 0; s < SETS; ++s) {
            const uint8_t *base = ws + ((size_t)jb * SETS + s) * kBatchOps * 1024 + lane * 16;
#pragma unroll
            for (int c = 0; c < kBatchOps; ++c) a[s][c] = *reinterpret_cast<const u32x4 *>(base + c * 1024);
            mr[s] = *reinterpret_cast<const f32x4 *>(ws + Lw.meta + (((size_t)jb * SETS + s) * 8 + 2 * g) * 8);
        }
    };
    load_a(0, anext, mnext);
#pragma unroll
    for (int f = 1; f < PF; ++f) gload(f, stg[f]);

    auto step = [&](const int q, auto fc, const bool more) {
        constexpr int F = decltype(fc)::value;
        const int sl = q / my_groups, t = q - sl * my_groups;
        if (t == 0) {
#pragma unroll
            for (int s = 0; s < SETS; ++s) {
                mreg[s] = mnext[s];
#pragma unroll
                for (int c = 0; c < kBatchOps; ++c) areg[s][c] = anext[s][c];
            }
        }
        const int jb = (sl0 + sl) * C + wave;  // this wave's block of the slice
        float *aux = aux0 + (q & 1) * (AUX_BYTES / 4);
        if (jb < bpr) {
#pragma unroll
            for (int T = 0; T < TILES; ++T) {
                const int row = T * 16 + n16;
                auto piece = [&](int pc) -> const u32x4 & {
                    return *reinterpret_cast<const u32x4 *>(lds + (row * RP + wave * 9 + pc) * 16);
                };
                const u32x4 hd = piece(0), qa0 = piece(1 + g), qa1 = piece(5 + g);
                const float d = half_bits_finite(hd[0]), dmin = half_bits_finite(hd[0] >> 16);
                // 16*sc (low nibbles) and sc (high nibbles) as f16 pairs, for
                // sub-block pairs G = h (k-slot pairs 0,1) and G = 2+h (2,3)
                const uint32_t sc_lo = scales4(0, hd[1], hd[3]), sc_hi = scales4(1, hd[1], hd[3]);
                typedef _Float16 h2 __attribute__((ext_vector_type(2)));
                const h2 sixteen = {(_Float16)16.0f, (_Float16)16.0f};
                uint32_t sf[2][2];
                sf[0][0] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, byte_to_h2(sc_lo, sel0)) * sixteen);
                sf[0][1] = byte_to_h2(sc_lo, sel1);
                sf[1][0] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, byte_to_h2(sc_hi, sel0)) * sixteen);
                sf[1][1] = byte_to_h2(sc_hi, sel1);
                // mins m0..m7 as f16 (k-slots of lane group 0; other groups
                // multiply zero A entries)
                const uint32_t mn_lo = mins4(0, hd[2], hd[3]), mn_hi = mins4(1, hd[2], hd[3]);
                const u32x4 bm = {byte_to_h2(mn_lo, 0x04010400u), byte_to_h2(mn_lo, 0x04030402u),
                                  byte_to_h2(mn_hi, 0x04010400u), byte_to_h2(mn_hi, 0x04030402u)};
                f32x4 acc[SETS], accm[SETS];
#pragma unroll
                for (int s = 0; s < SETS; ++s) {
                    acc[s] = (f32x4){0.f, 0.f, 0.f, 0.f};
                    accm[s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        __builtin_bit_cast(half8, areg[s][8]), __builtin_bit_cast(half8, bm),
                        (f32x4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                }
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    const int p = c >> 1, kind = c & 1;
                    const uint32_t mask = kind ? 0x00F000F0u : 0x000F000Fu;
                    const uint32_t w0 = p < 2 ? qa0[2 * p] : qa1[2 * p - 4];
                    const uint32_t w1 = p < 2 ? qa0[2 * p + 1] : qa1[2 * p - 3];
                    const h2 f = __builtin_bit_cast(h2, sf[p >> 1][kind]);
                    const u32x4 bq = {
                        __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, w0 & mask) * f),
                        __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, (w0 >> 8) & mask) * f),
                        __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, w1 & mask) * f),
                        __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, (w1 >> 8) & mask) * f)};
#pragma unroll
                    for (int s = 0; s < SETS; ++s)
                        acc[s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            __builtin_bit_cast(half8, areg[s][c]), __builtin_bit_cast(half8, bq), acc[s],
                            0, 0, 0);
                }
#pragma unroll
                for (int s = 0; s < SETS; ++s) {
                    const f32x4 mr = mreg[s];
                    const float y0 = d * ((acc[s][0] + acc[s][1]) * mr[0]) -
                                     dmin * ((accm[s][0] + accm[s][1]) * mr[1]);
                    const float y1 = d * ((acc[s][2] + acc[s][3]) * mr[2]) -
                                     dmin * ((accm[s][2] + accm[s][3]) * mr[3]);
                    // aux[wave][row][batch]
                    float *ap = aux + (wave * R + row) * BP + s * 8 + 2 * g;
                    ap[0] = y0;
                    ap[1] = y1;
                }
            }
        } else {
#pragma unroll
            for (int T = 0; T < TILES; ++T)
#pragma unroll
                for (int s = 0; s < SETS; ++s) {
                    float *ap = aux + (wave * R + T * 16 + n16) * BP + s * 8 + 2 * g;
                    ap[0] = 0.0f;
                    ap[1] = 0.0f;
                }
        }
        if (more) {
            if (t == my_groups - 1) load_a(sl + 1, anext, mnext);
            __syncthreads();  // every wave is done reading the stage buffer
            lstore(stg[(F + 1) % PF]);
            gload(q + 1 + PF, stg[(F + 1) % PF]);
        }
        __syncthreads();
        // cross-wave (block) reduction of this stage into the row buffer
        if (tid < R * BP) {
            float sum = 0.0f;
#pragma unroll
            for (int wv = 0; wv < NW; ++wv) sum += aux[wv * R * BP + tid];
            float *yb = ybuf + t * R * BP + tid;
            *yb = (sl == 0) ? sum : *yb + sum;
        }
    };
    static_assert(PF >= 1 && PF <= 8, "register sets are indexed by compile-time constants up to 8");
    // stage q0 + f with register set f (a compile-time index), for every
    // f < PF while q0 + f < lim
    auto steps = [&](const int q0, const int lim) __attribute__((always_inline)) {
#define MGQ_STEP(f)                                                                         \
        if constexpr (PF > (f))                                                             \
            if (q0 + (f) < lim) step(q0 + (f), std::integral_constant<int, (f) % PF>{}, q0 + (f) + 1 < Q);
        MGQ_STEP(0) MGQ_STEP(1) MGQ_STEP(2) MGQ_STEP(3)
        MGQ_STEP(4) MGQ_STEP(5) MGQ_STEP(6) MGQ_STEP(7)
#undef MGQ_STEP
    };
    lstore(stg[0]);
    int q0 = 0;
    if (Q > PF) {
        gload(PF, stg[0]);
        __syncthreads();
        // every stage of these rounds has a next one (q0 + PF < Q)
        for (; q0 + PF < Q; q0 += PF) steps(q0, q0 + PF);
    } else {
        __syncthreads();
    }
    steps(q0, Q);  // the last <= PF stages
    __syncthreads();
    // Y[b][r], rows fastest
    for (int i = tid; i < my_groups * R * BP; i += NW * 64) {
        const int t = i / (R * BP), rem = i - t * R * BP, b = rem / R, r = rem - b * R;
        const int row = (bx + t * G) * R + r;
        if (row < n && b < batch) {
            const float v = ybuf[(t * R + r) * BP + b];
            // two K parts: 0 + a + b rounds the same in either order
            if (kparts > 1)
                atomicAdd(&Y[(size_t)b * n + row], v);
            else
                Y[(size_t)b * n + row] = v;
        }
    }
}

// Wave-private batched kernel. A unit is R rows x CB blocks; wavefront w takes
// blocks CB*w .. CB*w + CB-1 of each K slice of NW*CB blocks, for each of the
// work-group's gpw row groups in turn (slice-major: the blocks' A operands
// stay in registers for gpw units). It loads the unit's pieces with 16-byte
// loads (runs of 9*CB pieces per row), stores them to its own LDS slot and
// computes from it, so no work-group barrier sits between units. Its sums of
// each (group, row, batch) accumulate over its slices in its own LDS rows; the
// work-group adds the wavefronts' rows in wavefront order once, after the
// stream. Every work-group takes exactly gpw groups (groups past the end
// re-read the last row and are not written), so every wavefront runs the
// same unit sequence. One unit is in flight per wavefront (its next unit's
// weights load while it computes; measured faster than two or three). A
// slice's A operands go into `areg` right after the previous slice's last
// unit is computed, behind the next unit's weights, which are already in
// flight: one register set.
template <int R, int SETS, int NW, int CB>
__global__ __launch_bounds__(NW * 64) void gemv_batched_wave_kernel(const uint8_t *__restrict__ w,
                                                                    const uint8_t *__restrict__ ws,
                                                                    float *__restrict__ Y, int n,
                                                                    int bpr, int batch, int gpw,
                                                                    int kparts, int gr) {
    static_assert(CB == 1 || CB == 2, "one or two blocks per unit");
    constexpr int PC = 9, BB = 144, TILES = R / 16, BP = 8 * SETS, RUN = PC * CB;
    constexpr int UP = R * RUN, IPU = (UP + 63) / 64;
    constexpr int SP = RUN | 1;  // LDS pieces per slot row (odd)
    constexpr uint32_t SLOT = (uint32_t)R * SP * 16u;
    constexpr int SW = NW * CB;  // blocks per K slice
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    uint8_t *slot = lds + (uint32_t)wave * SLOT;
    float *acc_all = reinterpret_cast<float *>(lds + NW * SLOT);
    const size_t row_bytes = (size_t)bpr * BB;

    // K split (kparts = 1 or 2): work-group id = kp * G + bx; K part kp takes
    // blocks [kb0, kb1), ceil(bpr / 2) of them for part 0
    const int G = (int)gridDim.x >> (kparts - 1);
    const int kp = (int)blockIdx.x >= G ? 1 : 0, bx = (int)blockIdx.x - kp * G;
    const int kspan = (bpr + kparts - 1) >> (kparts - 1);
    const int kb0 = kp * kspan, kb1 = std::min(bpr, kb0 + kspan);
    const int wb0 = kb0 + wave * CB;  // this wavefront's first block in slice 0

    // piece p of a unit: row p / RUN, piece p % RUN of the row's run; poff is
    // its byte offset from the unit's first piece (tile rows past the group
    // of gr <= R rows re-read its last row)
    uint32_t poff[IPU], plds[IPU];
#pragma unroll
    for (int k = 0; k < IPU; ++k) {
        const int p = std::min(k * 64 + lane, UP - 1);
        const int row = p / RUN, rem = p - row * RUN;
        poff[k] = (uint32_t)std::min(row, gr - 1) * (uint32_t)row_bytes + (uint32_t)(16 * rem);
        plds[k] = (uint32_t)((row * SP + rem) * 16);
    }
    // unit (slice sl, group index i): one uniform base and a 32-bit offset per
    // lane, so the next unit's loads go out one v_min after the slot stores.
    // A unit wholly past the row end re-reads the row's last blocks (cache
    // hits); blocks past the end of a unit that starts inside the row, and
    // rows past the matrix, read what follows (no result uses them), clamped
    // to the matrix's last piece.
    const uint64_t wlast = (uint64_t)n * row_bytes - 16;
    const uint32_t lastcol = (uint32_t)std::max(bpr - CB, 0) * BB;
    struct UnitAddr {
        const uint8_t *base;
        uint32_t lim;
    };
    // a group index past the last group (the work-group's last slots) re-reads
    // the last group; no result of it is stored
    const int groups = (n + gr - 1) / gr;
    auto uaddr = [&](int sl, int i) __attribute__((always_inline)) -> UnitAddr {
        const uint32_t c = (uint32_t)((wb0 + sl * SW) * BB);
        const uint32_t grp = (uint32_t)std::min(bx + i * G, groups - 1);
        const uint64_t b0 = (uint64_t)(grp * (uint32_t)gr) * row_bytes + (c < (uint32_t)row_bytes ? c : lastcol);
        return UnitAddr{w + b0, (uint32_t)std::min<uint64_t>(wlast - b0, 0xFFFFFFF0ull)};
    };
    u32x4 stg[IPU];
    auto gload_u = [&](const UnitAddr &a) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < IPU; ++k) stg[k] = ld_u32x4(a.base + std::min(poff[k], a.lim));
    };
    gload_u(uaddr(0, 0));  // the first unit before any schedule arithmetic
    const int slices = (kb1 - kb0 + SW - 1) / SW;
    const int U = slices * gpw;

    const BatchedWs Lw = batched_ws(bpr, SETS);
    const int n16 = lane & 15, g = lane >> 4, hsel = g >> 1;
    u32x4 areg[CB][SETS][kBatchOps];
    f32x4 mreg[CB][SETS];  // (corr, corr_min) of batches 2g, 2g+1 of each set
    auto load_a = [&](int sl) __attribute__((always_inline)) {
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
            const int jb = std::min(wb0 + sl * SW + cb, bpr - 1);
#pragma unroll
            for (int s = 0; s < SETS; ++s) {
                const uint8_t *base = ws + ((size_t)jb * SETS + s) * kBatchOps * 1024 + lane * 16;
#pragma unroll
                for (int c = 0; c < kBatchOps; ++c)
                    areg[cb][s][c] = *reinterpret_cast<const u32x4 *>(base + c * 1024);
                mreg[cb][s] = *reinterpret_cast<const f32x4 *>(ws + Lw.meta + (((size_t)jb * SETS + s) * 8 + 2 * g) * 8);
            }
        }
    };
    load_a(0);
    // load position (slice, group index) of the next unit to load
    int lsl = 0, li = 0;
    auto advance = [&](int &sl, int &i) __attribute__((always_inline)) {
        if (++i == gpw) {
            i = 0;
            ++sl;
        }
    };
    advance(lsl, li);
    const uint32_t sel0 = 0x04000400u | (uint32_t)(2 * hsel) | ((uint32_t)(2 * hsel) << 16);
    const uint32_t sel1 = sel0 + 0x00010001u;
    auto piece = [&](int row, int cb, int pc) -> const u32x4 & {
        return *reinterpret_cast<const u32x4 *>(slot + (row * SP + cb * PC + pc) * 16);
    };
    int csl = 0, ci = 0;  // compute position
    for (int u = 0; u < U; ++u) {
        // the next unit (past the last one: the last again, a cache hit), its
        // base worked out before the slot stores wait for this unit's data
        const bool new_slice = li == 0 && lsl < slices;
        const int next_sl = lsl;
        const UnitAddr na = lsl < slices ? uaddr(lsl, li) : uaddr(slices - 1, gpw - 1);
#pragma unroll
        for (int k = 0; k < IPU; ++k) *reinterpret_cast<u32x4 *>(slot + plds[k]) = stg[k];
        __asm__ volatile("" ::: "memory");  // the unit's reads follow its stores (in-order LDS)
        gload_u(na);
        advance(lsl, li);

        const int jb0 = wb0 + csl * SW;
        float yv[TILES][SETS][2];
#pragma unroll
        for (int T = 0; T < TILES; ++T)
#pragma unroll
            for (int s = 0; s < SETS; ++s) yv[T][s][0] = yv[T][s][1] = 0.0f;
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
            if (jb0 + cb >= kb1) break;
#pragma unroll
            for (int T = 0; T < TILES; ++T) {
                const int row = T * 16 + n16;
                const u32x4 hd = piece(row, cb, 0), qa0 = piece(row, cb, 1 + g), qa1 = piece(row, cb, 5 + g);
                const float d = half_bits_finite(hd[0]), dmin = half_bits_finite(hd[0] >> 16);
                const uint32_t sc_lo = scales4(0, hd[1], hd[3]), sc_hi = scales4(1, hd[1], hd[3]);
                typedef _Float16 h2 __attribute__((ext_vector_type(2)));
                const h2 sixteen = {(_Float16)16.0f, (_Float16)16.0f};
                uint32_t sf[2][2];
                sf[0][0] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, byte_to_h2(sc_lo, sel0)) * sixteen);
                sf[0][1] = byte_to_h2(sc_lo, sel1);
                sf[1][0] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, byte_to_h2(sc_hi, sel0)) * sixteen);
                sf[1][1] = byte_to_h2(sc_hi, sel1);
                const uint32_t mn_lo = mins4(0, hd[2], hd[3]), mn_hi = mins4(1, hd[2], hd[3]);
                const u32x4 bm = {byte_to_h2(mn_lo, 0x04010400u), byte_to_h2(mn_lo, 0x04030402u),
                                  byte_to_h2(mn_hi, 0x04010400u), byte_to_h2(mn_hi, 0x04030402u)};
                f32x4 acc[SETS], accm[SETS];
#pragma unroll
                for (int s = 0; s < SETS; ++s) {
                    acc[s] = (f32x4){0.f, 0.f, 0.f, 0.f};
                    accm[s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        __builtin_bit_cast(half8, areg[cb][s][8]), __builtin_bit_cast(half8, bm),
                        (f32x4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                }
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    const int p = c >> 1, kind = c & 1;
                    const uint32_t mask = kind ? 0x00F000F0u : 0x000F000Fu;
                    const uint32_t w0 = p < 2 ? qa0[2 * p] : qa1[2 * p - 4];
                    const uint32_t w1 = p < 2 ? qa0[2 * p + 1] : qa1[2 * p - 3];
                    const h2 f = __builtin_bit_cast(h2, sf[p >> 1][kind]);
                    const u32x4 bq = {
                        __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, w0 & mask) * f),
                        __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, (w0 >> 8) & mask) * f),
                        __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, w1 & mask) * f),
                        __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, (w1 >> 8) & mask) * f)};
#pragma unroll
                    for (int s = 0; s < SETS; ++s)
                        acc[s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            __builtin_bit_cast(half8, areg[cb][s][c]), __builtin_bit_cast(half8, bq), acc[s],
                            0, 0, 0);
                }
#pragma unroll
                for (int s = 0; s < SETS; ++s) {
                    const f32x4 mr = mreg[cb][s];
                    yv[T][s][0] += d * ((acc[s][0] + acc[s][1]) * mr[0]) -
                                   dmin * ((accm[s][0] + accm[s][1]) * mr[1]);
                    yv[T][s][1] += d * ((acc[s][2] + acc[s][3]) * mr[2]) -
                                   dmin * ((accm[s][2] + accm[s][3]) * mr[3]);
                }
            }
        }
        // the next unit starts a slice: its operands, now that these are read
        if (new_slice) load_a(next_sl);
        // this wavefront's rows: acc[wave][group index][row][batch]
        float *ap = acc_all + ((size_t)wave * gpw + ci) * R * BP;
#pragma unroll
        for (int T = 0; T < TILES; ++T)
#pragma unroll
            for (int s = 0; s < SETS; ++s) {
                float *p2 = ap + (T * 16 + n16) * BP + s * 8 + 2 * g;
                if (csl == 0) {
                    p2[0] = yv[T][s][0];
                    p2[1] = yv[T][s][1];
                } else if (jb0 < kb1) {
                    p2[0] += yv[T][s][0];
                    p2[1] += yv[T][s][1];
                }
            }
        advance(csl, ci);
    }
    __syncthreads();
    // Y[b][r], rows fastest; the wavefronts' sums added in wavefront order
    for (int i = tid; i < gpw * R * BP; i += NW * 64) {
        const int t = i / (R * BP), rem = i - t * R * BP, b = rem / R, r = rem - b * R;
        const int grp = bx + t * G, row = grp * gr + r;
        if (grp < groups && r < gr && row < n && b < batch) {
            float v = 0.0f;
            for (int wv = 0; wv < NW; ++wv) v += acc_all[(((size_t)wv * gpw + t) * R + r) * BP + b];
            // two K parts: 0 + a + b rounds the same in either order
            if (kparts > 1)
                atomicAdd(&Y[(size_t)b * n + row], v);
            else
                Y[(size_t)b * n + row] = v;
        }
    }
}

// Resident work-groups per CU from the occupancy query (at the LDS of one
// per CU), each taking gpw = ceil(groups / resident slots) row groups.
template <int R, int SETS, int NW, int CB>
static hipError_t batched_wave_launch(const uint8_t *w, const uint8_t *ws, float *Y, int n, int bpr,
                                      int batch, int kparts, hipStream_t stream) {
    constexpr int BP = 8 * SETS;
    constexpr size_t slots = (size_t)NW * R * ((9 * CB) | 1) * 16;
    auto kern = gemv_batched_wave_kernel<R, SETS, NW, CB>;
    const long cus = device_cus();
    const long gpw1 = ((long)(n + R - 1) / R * kparts + cus - 1) / cus;
    const int occ = occupancy_cached((const void *)kern, NW * 64, slots + (size_t)NW * gpw1 * R * BP * 4, 1);
    const long slots_total = cus * std::max(1, occ) / kparts;
    // fewer R-row groups than resident work-groups: groups of ceil(n / slots)
    // rows, one per work-group, so every CU works
    static const int gr_env = [] {
        const char *v = std::getenv("MGQ_BATCHED_GR");
        return (v && *v) ? std::atoi(v) : 1;
    }();
    int gr = R;
    if (gr_env && (n + R - 1) / R < slots_total) gr = (int)std::max<long>(1, (n + slots_total - 1) / slots_total);
    const long groups = (n + gr - 1) / gr;
    const long gpw = (groups + slots_total - 1) / slots_total;
    const long grid = (groups + gpw - 1) / gpw;
    const size_t lds = slots + (size_t)NW * gpw * R * BP * 4;
    if (lds > 160 * 1024) return hipErrorNotSupported;
    const hipError_t attr = allow_full_lds_by_addr((const void *)kern);
    if (attr != hipSuccess) return attr;
    kern<<<(unsigned)(grid * kparts), NW * 64, lds, stream>>>(w, ws, Y, n, bpr, batch, (int)gpw, kparts, gr);
    return hipGetLastError();
}

template <int R, int SETS, int PF>
static hipError_t batched_main_launch(const uint8_t *w, const uint8_t *ws, float *Y, int n, int bpr,
                                      int batch, int kparts, hipStream_t stream) {
    auto kern = gemv_batched_mfma_kernel<R, SETS, PF>;
    const hipError_t attr = allow_full_lds_by_addr((const void *)kern);
    if (attr != hipSuccess) return attr;
    constexpr int BP = 8 * SETS;
    constexpr size_t base = (size_t)R * ((9 * 8) | 1) * 16 + 2 * (size_t)8 * R * BP * 4;
    const long groups = (n + R - 1) / R;
    const int occ = occupancy_cached((const void *)kern, 512, base + 8 * R * BP * 4, 1);
    const long maxgrid = (long)device_cus() * occ;
    const long rounds = (groups + maxgrid - 1) / maxgrid;
    const long grid = (groups + rounds - 1) / rounds;
    const size_t lds = base + (size_t)rounds * R * BP * 4;
    if (lds > 160 * 1024) return hipErrorNotSupported;
    kern<<<(unsigned)(grid * kparts), 512, lds, stream>>>(w, ws, Y, n, bpr, batch, (int)rounds,
                                                          kparts);
    return hipGetLastError();
}

// the main kernels' LDS limit, set outside any stream capture (gemv_prepare)
hipError_t batched_prepare() {
    const void *kerns[] = {
        (const void *)gemv_batched_wave_kernel<16, 1, 7, 2>, (const void *)gemv_batched_wave_kernel<16, 2, 8, 1>,
        (const void *)gemv_batched_wave_kernel<32, 1, 7, 2>, (const void *)gemv_batched_wave_kernel<32, 2, 8, 1>,
        (const void *)gemv_batched_mfma_kernel<16, 1, MGQ_BPF1>, (const void *)gemv_batched_mfma_kernel<16, 2, MGQ_BPF2>,
        (const void *)gemv_batched_mfma_kernel<32, 1, MGQ_BPF1>, (const void *)gemv_batched_mfma_kernel<32, 2, MGQ_BPF2>};
    for (const void *k : kerns) {
        const hipError_t e = allow_full_lds_by_addr(k);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t gemv_batched_mfma_launch(const uint8_t *w, const float *X, float *Y, int n, int bpr,
                                    int batch, void *workspace, size_t workspace_bytes,
                                    hipStream_t stream) {
    const int sets = (batch + 7) / 8;
    if (workspace_bytes < batched_ws(bpr, sets).total) return hipErrorInvalidValue;
    if ((uintptr_t)workspace & 15u) return hipErrorNotSupported;
    uint8_t *ws = static_cast<uint8_t *>(workspace);
    // Few row groups and a long K (ffn_down): 32-row groups, K split in two,
    // so every CU is busy and each work-group reads the operand table for 32
    // rows instead of 16. Otherwise 16-row groups: at one 8-wave work-group
    // per CU, 32-row groups leave a coarser last round (gate 18944x3584: 3
    // rounds of 32 rows on 198 work-groups against 5 of 16 on 237; 14.6
    // against 16.6 us at B = 8, and slower at B = 4 and 16 too).
    const bool ksplit = (n + 15) / 16 <= device_cus() && (bpr + 7) / 8 >= 4;
    batched_table_kernel<<<dim3((unsigned)((bpr + 1) / 2), (unsigned)sets), 256, 0, stream>>>(
        X, batch, bpr, sets, ((uintptr_t)X & 15u) == 0, ws, Y, ksplit ? batch * n : 0);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // Main kernel: the wave-private kernel, with units of two blocks (a
    // 14-block slice over 7 wavefronts: gate's whole row) for one batch set
    // and of one block for two (the operands of two blocks and two sets do
    // not fit the registers). µs per call at B = 8 with the table pass,
    // against the stage kernel: gate 15.8-16.8 / 17.9-18.8, gate|up fused
    // 23.5-23.7 / 27.4-27.5, down 19.9-20.9 / 20.0-20.9. MGQ_BATCHED_WAVE=0
    // selects the stage kernel (a tuning switch).
    static const int wave_env = [] {
        const char *v = std::getenv("MGQ_BATCHED_WAVE");
        return (v && *v) ? std::atoi(v) : 1;
    }();
    if (wave_env) {
        hipError_t ew;
        if (ksplit)
            ew = sets == 1 ? batched_wave_launch<32, 1, 7, 2>(w, ws, Y, n, bpr, batch, 2, stream)
                           : batched_wave_launch<32, 2, 8, 1>(w, ws, Y, n, bpr, batch, 2, stream);
        else
            ew = sets == 1 ? batched_wave_launch<16, 1, 7, 2>(w, ws, Y, n, bpr, batch, 1, stream)
                           : batched_wave_launch<16, 2, 8, 1>(w, ws, Y, n, bpr, batch, 1, stream);
        if (ew != hipErrorNotSupported) return ew;
    }
    // The stage kernel: also for shapes whose per-wavefront row sums (gpw
    // groups) would not fit LDS beside the slots (more than ~143k rows at
    // B <= 8, ~70k at B <= 16).
    // Weight stages in flight (register sets). One batch set (B <= 8), µs
    // per call at B = 8, gate / down, table pass included: 2 stages
    // 18.8 / 20.8, 3: 19.7 / 21.7, 4: 19.7 / 22.8, 6: 21.2 / 24.2,
    // 8: 22.6 / 29.1 (VGPRs 167 -> 239 for the 16-row kernel). Two sets
    // (B <= 16) run at 256 VGPRs and stay at one stage (two: down 25.9 ->
    // 85 us).
    if (ksplit)
        return sets == 1 ? batched_main_launch<32, 1, MGQ_BPF1>(w, ws, Y, n, bpr, batch, 2, stream)
                         : batched_main_launch<32, 2, MGQ_BPF2>(w, ws, Y, n, bpr, batch, 2, stream);
    if (sets == 1) return batched_main_launch<16, 1, MGQ_BPF1>(w, ws, Y, n, bpr, batch, 1, stream);
    return batched_main_launch<16, 2, MGQ_BPF2>(w, ws, Y, n, bpr, batch, 1, stream);
}

}  // namespace mgq
