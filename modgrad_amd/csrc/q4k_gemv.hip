// Q4_K GEMV kernels for gfx950 (MI355X).
//
// Reference semantics: launch_matvec_q4k / matvec_q4k_kernel
// (crates/modgrad-device/kernels/matvec_q4k.hip:55-124) and the host oracle
// rocm_matvec_check.rs:38-47: y[r] = sum_k dequant(W)[r][k] * x[k], canonical
// element order (gguf.rs:364-404).
//
// Kernels:
//
// 1. gemv_generic_kernel -- vector-ALU, one wavefront per row, flat-stream
//    addressing (element (r,c) at flat index r*k+c), so it serves both the
//    row-aligned GGUF layout and LinearResidentQuantized's flattened layout
//    (neuron.rs:931-951) where rows start mid-block, and weights that are
//    only 4-byte aligned.
//
// 2. gemv_mfma_kernel -- the fast path for the row-aligned layout. The
//    dequantize-multiply runs on the matrix cores (v_mfma_f32_16x16x32_f16):
//      * B operand = weights: lane (n = l%16, g = l/16) holds qs bytes of row n.
//        A nibble masked in place, (dword & 0x000F000F) or (dword & 0x00F000F0),
//        is already an f16 *subnormal* equal to q*2^-24 (or 16q*2^-24), so one
//        AND turns two nibbles into two exact f16 operands.
//      * A operand = activations, from a table the work-group builds in LDS
//        once: the k-slot's x value sits in MFMA row m = 2*sub-block (xh part)
//        and m = 2*sub-block + 1 (xl part), zero elsewhere. x is split as
//        x*2^e = xh + xl (two f16, ~22 bits) with a per-sub-block power of two
//        e, so the f32 accumulators receive sum q*x per (sub-block, row) to
//        within ~2^-22 relative -- f32-grade, far inside the 1e-4 bound.
//      * Accumulator lane (n, g) holds rows 4g..4g+3 = both parts of
//        sub-blocks 2g and 2g+1 of W row n, so merging xh and xl is an in-lane
//        add, and each lane applies d*sc*2^-e and dmin*m*sum(x) for its two
//        (row, sub-block) pairs.
//      * Weights stream HBM -> registers -> LDS with fully coalesced 16-byte
//        loads (64 consecutive pieces per wave instruction), PF stages ahead
//        of the one being computed.
//    Per 32 rows x 1 block a wave issues 16 MFMAs and about 220 VALU ops.
//    Its kStageWave variant stages per wavefront (below) for the Q8 / dp4a,
//    fused RMSNorm / GLU and Q5_K modes; with kI8 the fused and Q5_K modes
//    multiply in the int8 form described under 3.
//
// 3. gemv_wave_kernel -- the same arithmetic (by default in its int8 form:
//    x as three signed 8-bit digits per value, the nibbles as int8 operands,
//    v_mfma_i32_16x16x64_i8) with every wavefront staging
//    its own unit through its own LDS slot, so stages need no work-group
//    barrier; used for plain f32 matvecs whose work-groups stream several
//    stages (gate|up, lm_head, down). With DIRECT (one unit per wavefront:
//    o, qkv's one group per CU and other single-stage launches) each lane
//    loads the pieces it multiplies straight into registers. A unit's loads
//    go out from a uniform base with one clamped 32-bit offset per lane,
//    the next unit's base worked out before the current unit's slot stores.
//
// 4. gemv_batched_kernel -- vector-ALU batched GEMV (up to 16 activation rows).
#include "q4k_device.hpp"
#include "q4k_launch.hpp"

#include <algorithm>
#include <cstdlib>
#include <type_traits>

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

// Flat-stream layout with k % 32 == 0 (k % 256 != 0): every sub-block lies
// inside one row, and U = 256 / gcd(k, 256) consecutive rows (a unit) are
// BPU = U*k/256 whole blocks. One wavefront per unit: lane (bi, j) = (lane/8,
// lane%8) takes 16-byte qs chunk j of block bi (+8 per pass), i.e. the 16 low
// nibbles of sub-block 2(j/2) and the 16 high nibbles of sub-block 2(j/2)+1,
// with 16-byte loads of the 16 matching x values each. Per sub-block half:
// d*sc * sum(q x) - dmin*m * sum(x), added to the accumulator of its row.
template <int U>
__global__ __launch_bounds__(256) void gemv_flat_kernel(const uint8_t *__restrict__ w,
                                                        const float *__restrict__ x,
                                                        float *__restrict__ y, int n, int k,
                                                        int bpu, int units, int64_t nblocks) {
    const int lane = threadIdx.x & 63;
    const int u = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (u >= units) return;  // uniform per wavefront
    const int64_t ub = (int64_t)u * bpu;
    const int nb = (int)std::min<int64_t>(bpu, nblocks - ub);
    const int bi = lane >> 3, j = lane & 7, G = j >> 1;
    float acc[U];
#pragma unroll
    for (int r = 0; r < U; ++r) acc[r] = 0.0f;
    for (int bl = bi; bl < nb; bl += 8) {
        const uint8_t *blk = w + (ub + bl) * kBlockBytes;
        const u32x4 hd = ld_u32x4(blk);
        const u32x4 qs = ld_u32x4(blk + 16 + 16 * j);
        const float d = half_bits_finite(hd[0]), dmin = half_bits_finite(hd[0] >> 16);
        uint32_t sc_lo, m_lo, sc_hi, m_hi;
        scale_min(2 * G, hd[1], hd[2], hd[3], sc_lo, m_lo);
        scale_min(2 * G + 1, hd[1], hd[2], hd[3], sc_hi, m_hi);
        const int f_lo = 256 * bl + 64 * G + 16 * (j & 1);  // unit-relative flat index
        const int r_lo = f_lo / k, r_hi = (f_lo + 32) / k;
        const float *xl = x + (f_lo - r_lo * k);
        const float *xh = x + (f_lo + 32 - r_hi * k);
        float dl = 0.0f, sl = 0.0f, dh = 0.0f, sh = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const f32x4 a = ld_f32x4(xl + 4 * c), b = ld_f32x4(xh + 4 * c);
            const uint32_t v = qs[c];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                dl += (float)((v >> (8 * t)) & 15u) * a[t];
                dh += (float)((v >> (8 * t + 4)) & 15u) * b[t];
                sl += a[t];
                sh += b[t];
            }
        }
        const float vl = (d * (float)sc_lo) * dl - (dmin * (float)m_lo) * sl;
        const float vh = (d * (float)sc_hi) * dh - (dmin * (float)m_hi) * sh;
#pragma unroll
        for (int r = 0; r < U; ++r) acc[r] += (r_lo == r ? vl : 0.0f) + (r_hi == r ? vh : 0.0f);
    }
#pragma unroll
    for (int r = 0; r < U; ++r) {
        float v = acc[r];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
        const int row = u * U + r;
        if (lane == 0 && row < n) y[row] = v;
    }
}

hipError_t gemv_flat_launch(const uint8_t *w, const float *x, float *y, int n, int k,
                            hipStream_t stream) {
    if (k % 32 != 0) return hipErrorNotSupported;
    int g = 256;
    while (k % g) g >>= 1;  // gcd(k, 256), >= 32 here
    const int U = 256 / g;
    if ((int64_t)U * k > 0x7FFFFFFFLL) return hipErrorNotSupported;  // unit-relative indices are int
    const int bpu = (int)((int64_t)U * k / kBlockElems);
    const int units = (n + U - 1) / U;
    const int64_t nblocks = (int64_t)n * k / kBlockElems;
    const unsigned grid = (unsigned)((units + 3) / 4);
    switch (U) {
    case 1: gemv_flat_kernel<1><<<grid, 256, 0, stream>>>(w, x, y, n, k, bpu, units, nblocks); break;
    case 2: gemv_flat_kernel<2><<<grid, 256, 0, stream>>>(w, x, y, n, k, bpu, units, nblocks); break;
    case 4: gemv_flat_kernel<4><<<grid, 256, 0, stream>>>(w, x, y, n, k, bpu, units, nblocks); break;
    default: gemv_flat_kernel<8><<<grid, 256, 0, stream>>>(w, x, y, n, k, bpu, units, nblocks); break;
    }
    return hipGetLastError();
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



// LDS layout of one work-group (rows R, all bpr blocks of K):
//   atab  [bpr][8 mfma c][4 lane-group h][xh|xl][8 halves] + 16 B of zeros,
//         bpr*1040 B (Q8: the int8 activations xq, bpr*256 B)
//   meta  [bpr][corr[8] | xsum[8]] f32 (Q8: [xd[8] | xsum[8]]) bpr*64 B
//   stage 2 (1 if bpr <= C) x SB bytes: weight bytes of R rows x C blocks,
//         row-major over (row, block, 16-byte piece), rows padded to an odd
//         number of pieces
//   aux   2 x NW*32*4 B: cross-wave reduction buffers (32 row sums per
//         wavefront), alternating by row group
//   ybuf  rounds x R row results (x2 with kFuseGlu: gate and up)
//   normp 16 f32 sum(x^2) partials (kFuseNorm only)
struct MfmaLayout {
    int bpr, R, C, NW, I;  // I = 1 KiB wave loads per stage
    uint32_t tab_stride, meta, stage, stage_bytes, aux, ybuf, normp;
    size_t total;
};

// Fused glue (f32 activations only). kFuseNorm: y = W * rms_norm(x, nw, eps),
// computed as rstd * (W * (x .* nw)) -- the prologue multiplies x by nw and
// accumulates sum(x^2), the row results are scaled once at the end.
// kFuseGlu: two weight matrices (gate w, up w2) of one shape; each row group
// streams through the same work-group twice (gate, then up) and the output is
// act(gate_row . x) * (up_row . x).
// kFuseQuant (Q8 mode only): the prologue quantizes f32 x to Q8_1 itself,
// bit-identically to quantize_q8_1_kernel (launch_quantize_q8_1 followed by
// the dp4a matvec, in one launch).
// kFmtQ5K (f32 mode, no other bit): the weights are Q5_K, 176-byte blocks
// of 11 16-byte pieces (header | qh[32] | qs[128]); the header and its scale
// packing are Q4_K's, and the fifth bit of every weight comes from qh.
// kStageWave (a staging variant, with any of the above): every wavefront
// loads and stores only its own unit's pieces (at their places in the stage
// buffer) and no work-group barrier sits between stages; the row sums of
// every pass go to per-wavefront LDS rows and are reduced once, after the
// stream, in the same order (results identical to the barrier-staged kernel
// of the same stage width). Needs one unit per wavefront and stage, one
// stage in flight and a single stage buffer.
// kI8 (with kStageWave, Q4_K f32 activations): the int8 matrix-core form of
// the wave-private kernel (i8_table_entry, i8_tile).
constexpr int kFuseNorm = 1, kFuseGlu = 2, kFuseQuant = 4, kFmtQ5K = 8, kStageWave = 16, kI8 = 32;
__host__ __device__ constexpr int block_pieces(int fuse) { return (fuse & kFmtQ5K) ? 11 : 9; }
struct GemvFuse {
    const uint8_t *w2;  // kFuseGlu: the up matrix
    const float *nw;    // kFuseNorm: RMSNorm weights [K]
    float eps;
    int act;            // kActGeluTanh or kActSilu
};

// rounds = row groups per work-group (persistent launch); their results stay
// in LDS (ybuf) until the stream ends, so no global store sits between the
// staged loads (a store would force the compiler to drain every load).
// Staged rows are padded to an odd number of 16-byte pieces, so the 16
// lanes that read one piece column of 16 different rows hit 16 different
// LDS bank groups.
__host__ __device__ constexpr int stage_row_pieces(int C, int bp = 9) { return (bp * C) | 1; }

__host__ __device__ inline MfmaLayout mfma_layout(int bpr, int R, int C, int NW, int rounds,
                                                  bool db, bool q8 = false, int fuse = 0) {
    MfmaLayout L;
    L.bpr = bpr; L.R = R; L.C = C; L.NW = NW;
    // wave loads per stage, padded so every wavefront issues the same count
    const int bp = block_pieces(fuse);
    L.I = ((R * bp * C + 63) / 64 + NW - 1) / NW * NW;
    // activation table: per block 1 KiB of f16 operands plus a 16-byte zero
    // slot (so a lane's A address is the block base plus a fixed offset), or
    // (Q8) the block's 256 int8 activations
    L.tab_stride = q8 ? 256u : 1040u;
    L.meta = (uint32_t)bpr * L.tab_stride;
    L.stage = L.meta + (uint32_t)bpr * 64u;
    L.stage_bytes = (uint32_t)(R * stage_row_pieces(C, bp) * 16);
    // two stage buffers when double-buffered and K needs more than one stage
    L.aux = L.stage + ((db && bpr > C) ? 2u : 1u) * L.stage_bytes;
    // kFuseGlu: gate and up results of every row group (2x rounds);
    // kFuseNorm: one sum(x^2) partial per wavefront
    const int vm = (fuse & kFuseGlu) ? 2 : 1;
    // kStageWave: 32 row sums per wavefront and pass (rounds x vm passes)
    L.ybuf = L.aux + ((fuse & kStageWave) ? (uint32_t)(rounds * vm) * NW * 128u : (uint32_t)NW * 256u);
    L.normp = L.ybuf + (uint32_t)(R * rounds * vm * 4);
    L.total = (size_t)L.normp + ((fuse & kFuseNorm) ? 64 : 0);
    return L;
}

// Work-group = R rows (R = 16 or 32) x all K, persistent over row groups
// blockIdx.x, blockIdx.x + gridDim.x, ... The weights stream through LDS C
// blocks at a time: every wave load instruction moves 64 consecutive 16-byte
// pieces of the rows' contiguous byte runs (fully coalesced) into registers,
// PF stages ahead of the stage being computed; each stage is then written to a
// double-buffered LDS stage and the MFMA operands are read from LDS. The stage
// sequence runs across row-group boundaries, so a persistent work-group keeps
// PF stages in flight from its first load to its last and builds the
// activation table only once.
// A wavefront's unit of work is two 16-row x 1-block MFMA tiles: rows
// [0,16) and [16,32) of one block when R = 32, or blocks 2u and 2u+1 of the
// 16 rows when R = 16. Per unit: 16 MFMAs, an xh/xl merge that leaves tile A
// in lanes 0..31 and tile B in lanes 32..63, and the scale/min decode of 4
// (row, sub-block) pairs per lane.
// DB: double-buffered LDS stage (one barrier per stage) or a single buffer
// (two barriers per stage, half the LDS, so more work-groups fit per CU).
typedef int i32x4 __attribute__((ext_vector_type(4)));

// The int8 form's activation table (one 1040-byte entry per block, as the
// f16 form's): item j (x values 8j .. 8j + 7) of sub-block sb of block b.
// x 2^e rounded to an integer X, |X| < 2^22, as three signed 8-bit digits:
// the bytes of Y = X + 128 (1 + 256 + 65536) with their top bits flipped
// (byte - 128), so X = sum (byte_i - 128) 256^i. Adding 1.5 2^23 rounds
// x 2^e to an integer in the mantissa's low bits. Digit dg of the item sits
// at ((sb 3 + dg) 2 + j / 2) 16 + (j % 2) 8: A row m = 4 (sub-block pair) +
// digit reads 16 bytes (two items) of one sub-block. meta[b 16 + sb] = 2^-e,
// meta[b 16 + 8 + sb] = the sub-block's sum.
__device__ __forceinline__ void i8_table_entry(uint8_t *lds, float *meta, int b, int sb, int j,
                                               const f32x4 &v0, const f32x4 &v1, float amax,
                                               float sum) {
    int e = 0;
    float corr = 1.0f;
    if (amax > 0.0f && amax <= 3.402823466e38f) {
        int ex;
        frexpf(amax, &ex);
        e = std::min(22 - ex, 140);  // ex <= 128: e >= -106
        corr = ldexpf(1.0f, -e);
    } else if (!(amax == 0.0f)) {
        corr = amax;  // Inf or NaN: the row sums come out non-finite
    }
    if (j == 0) {
        meta[b * 16 + sb] = corr;
        meta[b * 16 + 8 + sb] = sum;
    }
    const float xs[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
    uint32_t yv[8];
#pragma unroll
    for (int q = 0; q < 8; ++q)
        yv[q] = __builtin_bit_cast(uint32_t, ldexpf(xs[q], e) + 12582912.0f) - (0x4B400000u - 0x808080u);
#pragma unroll
    for (int dg = 0; dg < 3; ++dg) {
        // byte dg of values 4h .. 4h + 3 (v_perm: selector k picks byte k of
        // the second operand, 4 + k of the first; 0x0C a zero byte)
        const uint32_t sel = (uint32_t)dg | ((4u + dg) << 8) | 0x0C0C0000u;
        uint32_t dw[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t lo = __builtin_amdgcn_perm(yv[4 * h + 1], yv[4 * h], sel);
            const uint32_t hi = __builtin_amdgcn_perm(yv[4 * h + 3], yv[4 * h + 2], sel);
            dw[h] = __builtin_amdgcn_perm(hi, lo, 0x05040100u) ^ 0x80808080u;
        }
        *reinterpret_cast<u32x2 *>(lds + (size_t)b * 1040 + (size_t)(((sb * 3 + dg) * 2 + (j >> 1)) * 16 + (j & 1) * 8)) =
            u32x2{dw[0], dw[1]};
    }
}

// int8 form: MFMA c4 = low / high nibbles (c4 & 1) of qs pieces 1+g (c4 < 2)
// or 5+g: lane group g's 16 bytes are sub-block pair jp = 2 (c4 >> 1) +
// (g >> 1) at elements 16 (g & 1) ..; A row m = 4 jp + digit holds that
// pair's low (c4 even) or high sub-block's digits. The low-nibble MFMAs
// accumulate into one accumulator and the high-nibble ones into the other,
// so lane group G holds sub-blocks 2G and 2G + 1, as in the f16 form (same
// decode). Lanes whose row m takes no data read the block's zero slot.
__device__ __forceinline__ uint32_t i8_aoff(int c4, int n16, int g) {
    const int hi = c4 & 1, jp = 2 * (c4 >> 1) + (g >> 1), sbc = 2 * jp + hi;
    const bool hit = (n16 >> 2) == jp && (n16 & 3) < 3;
    return hit ? (uint32_t)(((sbc * 3 + (n16 & 3)) * 2 + (g & 1)) * 16) : 1024u;
}

// The scaled q*x sums s0, s1 (sub-blocks 2g, 2g + 1 of row n16) of one block
// (table entry tb) from its qs pieces q0 (1 + g) and q1 (5 + g): the three
// digit sums of each (|each| < 2^16) as a0 + 256 a1 exactly, then + 65536 a2.
// Q5K: the qs pieces are 3 + g and 7 + g, and bit j (sub-block j) of the
// qh byte of each qs byte (hq: qh piece 1 + (g & 1)) is the weight's fifth
// bit, q = nibble + 16 bit (a digit sum over 32 values stays below 2^17 in
// magnitude: exact in int32; its f32 combination rounds as an f32 sum does).
template <bool Q5K = false>
__device__ __forceinline__ void i8_tile(const uint8_t *tb, const uint32_t (&aoff8)[4], const u32x4 &q0,
                                        const u32x4 &q1, float &s0, float &s1,
                                        const u32x4 &hq = u32x4{0u, 0u, 0u, 0u}, int g = 0) {
    i32x4 alo = {0, 0, 0, 0}, ahi = {0, 0, 0, 0};
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) {
        const u32x4 src = c4 < 2 ? q0 : q1;
        u32x4 bq = (c4 & 1) ? ((src >> 4u) & 0x0F0F0F0Fu) : (src & 0x0F0F0F0Fu);
        if constexpr (Q5K) {
            const uint32_t j = (uint32_t)(2 * (2 * (c4 >> 1) + (g >> 1)) + (c4 & 1));
            bq |= ((hq >> j) & 0x01010101u) << 4u;
        }
        const i32x4 av = *reinterpret_cast<const i32x4 *>(tb + aoff8[c4]);
        if (c4 & 1) ahi = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, __builtin_bit_cast(i32x4, bq), ahi, 0, 0, 0);
        else alo = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, __builtin_bit_cast(i32x4, bq), alo, 0, 0, 0);
    }
    s0 = (float)alo[2] * 65536.0f + (float)((alo[1] << 8) + alo[0]);
    s1 = (float)ahi[2] * 65536.0f + (float)((ahi[1] << 8) + ahi[0]);
}

// Q8: the dp4a matvec of kernels/matvec_q4k_dp4a.hip:52-106 on the same
// weight stream: activations arrive as int8 xq with per-sub-block scale xd and
// sum xsum; each lane dots its 32 qs bytes (4 sub-block halves) with
// v_dot4_i32_i8 and applies xd*(d*sc*isum - dmin*m*xsum).
// FUSE (f32 activations only): kFuseNorm and/or kFuseGlu, see GemvFuse.
template <int R, int C, int NW, int PF, bool DB, int XIT, bool Q8, int FUSE>
__global__ __launch_bounds__(NW * 64) void gemv_mfma_kernel(const uint8_t *__restrict__ w,
                                                            const float *__restrict__ x,
                                                            const int8_t *__restrict__ xq,
                                                            const float *__restrict__ xdv,
                                                            const float *__restrict__ xsv,
                                                            float *__restrict__ y, int n,
                                                            int bpr, int rounds, GemvFuse fz,
                                                            GemvSched sch, int gr) {
    constexpr int FM = FUSE & ~(kStageWave | kI8);  // the mode bits
    static_assert(Q8 ? (FM == 0 || FM == kFuseQuant) : (FM & kFuseQuant) == 0,
                  "fused glue runs on f32 activations; quantization only in Q8 mode");
    static_assert(!(FM & kFmtQ5K) || FM == kFmtQ5K, "Q5_K weights: plain f32 matvec only");
    static_assert(R == 32 || C % 2 == 0, "R = 16: a unit is a pair of blocks, so C must be even");
    constexpr bool Q5 = (FUSE & kFmtQ5K) != 0;
    constexpr bool WV = (FUSE & kStageWave) != 0;
    static_assert(!WV || (PF == 1 && !DB), "kStageWave: one stage in flight, one stage buffer");
    constexpr bool I8 = (FUSE & kI8) != 0;
    static_assert(!I8 || (WV && !Q8), "kI8: Q4_K / Q5_K f32 activations on kStageWave only");
    constexpr int BP = block_pieces(FUSE);  // 16-byte pieces per block
    constexpr int BB = BP * 16;              // block bytes
    constexpr bool NORM = (FUSE & kFuseNorm) != 0;
    constexpr int VM = (FUSE & kFuseGlu) ? 2 : 1;  // passes per row group (gate, up)
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const MfmaLayout Lo = mfma_layout(bpr, R, C, NW, rounds, DB, Q8, FUSE);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar branches
    float *meta = reinterpret_cast<float *>(lds + Lo.meta);
    float *aux = reinterpret_cast<float *>(lds + Lo.aux);
    const size_t row_bytes = (size_t)bpr * BB;
    const int stages = (bpr + C - 1) / C;
    constexpr int PIECES = R * BP * C;            // 16-byte pieces per stage
    constexpr int UNITS = (R == 32) ? C : C / 2;  // tile pairs per stage
    static_assert(!WV || UNITS == NW, "kStageWave: one unit per wavefront and stage");
    constexpr int RUN = (R == 32) ? BP : 2 * BP;  // kStageWave: pieces of one row in a unit
    // wave loads per wavefront: a share of the stage, or (kStageWave) its unit
    constexpr int IPW = WV ? (R * RUN + 63) / 64 : ((PIECES + 63) / 64 + NW - 1) / NW;
    constexpr int I = IPW * NW;                   // wave loads per stage (padded)

    // ---- weight staging: global -> registers (PF sets) -> LDS ---------------
    // stg is only ever indexed with compile-time constants (the stage loop is
    // unrolled by PF), so the sets stay in registers with loads in flight.
    u32x4 stg[PF][IPW];
    // Loads are unconditional (a stage past the end re-reads the last one,
    // already cached) so the compiler's in-order vmcnt accounting stays
    // exact and only the set being stored is waited for. The piece -> (row,
    // byte column) split of each load is stage-invariant and precomputed.
    constexpr int RP = stage_row_pieces(C, BP);   // LDS pieces per staged row
    // kStageWave: the wavefront's unit starts at block cbu of each stage
    const int cbu = (R == 32) ? wave : 2 * wave;
    uint32_t poff[IPW], pcol[IPW], plast[IPW], plds[IPW];
#pragma unroll
    for (int k = 0; k < IPW; ++k) {
        int row, rem;
        if constexpr (WV) {
            // piece p of this wavefront's unit: row p / RUN, from its first block
            const int p = std::min(k * 64 + lane, R * RUN - 1);
            row = p / RUN;
            rem = cbu * BP + (p - row * RUN);
        } else {
            const int j = std::min((wave + k * NW) * 64 + lane, PIECES - 1);
            row = j / (BP * C);
            rem = j - row * BP * C;
        }
        const int cb = rem / BP, pc = rem - cb * BP;
        plds[k] = (uint32_t)((row * RP + rem) * 16);    // LDS byte offset in the stage
        // the tile rows past the group (gr <= R rows) re-read its last row
        poff[k] = (uint32_t)std::min(row, gr - 1) * (uint32_t)row_bytes;
        if constexpr (WV) poff[k] += (uint32_t)(16 * (rem - cbu * BP));  // within the unit
        pcol[k] = (uint32_t)(cb * BB + 16 * pc);          // byte column within the stage
        plast[k] = (uint32_t)((bpr - 1) * BB + 16 * pc);  // same piece of the last block
    }
    // Stage (pass vg, column tcol) of the rows from r0 in matrix wm: a
    // uniform base and one 32-bit offset per lane. Pieces past the row end
    // re-read the row's last block (kStageWave: a unit wholly past it, the
    // row's last blocks); rows past the matrix read its last piece.
    const uint64_t wlast = (uint64_t)n * row_bytes - 16;
    const uint32_t lastcol = (uint32_t)std::max(bpr - (R == 32 ? 1 : 2), 0) * BB;
    struct UnitAddr {
        const uint8_t *base;
        uint32_t lim, tcol;
    };
    auto uaddr = [&](uint32_t r0, uint32_t tcol, const uint8_t *wm) -> UnitAddr {
        uint64_t b0 = (uint64_t)std::min(r0, (uint32_t)(n - 1)) * row_bytes;
        if constexpr (WV) {
            const uint32_t c = tcol + (uint32_t)(cbu * BB);
            b0 += c < (uint32_t)row_bytes ? c : lastcol;
        }
        return UnitAddr{wm + b0, (uint32_t)std::min<uint64_t>(wlast - b0, 0xFFFFFFF0ull), tcol};
    };
    auto gload_u = [&](const UnitAddr &a, u32x4(&dst)[IPW]) {
#pragma unroll
        for (int k = 0; k < IPW; ++k) {
            const uint32_t o = WV ? poff[k] : poff[k] + std::min(a.tcol + pcol[k], plast[k]);
            dst[k] = ld_u32x4(a.base + std::min(o, a.lim));
        }
    };
    auto gload_at = [&](uint32_t r0, uint32_t tcol, const uint8_t *wm, u32x4(&dst)[IPW]) {
        gload_u(uaddr(r0, tcol, wm), dst);
    };
    // The first stage: row group 0 of every schedule is blockIdx.x (and a
    // work-group owns at least one), pass 0 reads w from column 0. It needs
    // no schedule arithmetic, so its loads go out before the divisions that
    // the schedule takes (plan(), right after them).
    auto gload_first = [&](u32x4(&dst)[IPW]) {
        gload_at((uint32_t)blockIdx.x * (uint32_t)gr, 0u, w, dst);
    };
    // The schedule, computed while the first loads are in flight (before the
    // activation table is built, so it never delays the next stage's loads).
    int groups = 0, my_groups = 0, Q = 0;  // row groups; this work-group's; its stages
    auto plan = [&]() {
        // a row group is gr <= R rows (the tile's rows past gr re-read row gr - 1)
        groups = (n + gr - 1) / gr;
        my_groups = sched_count(sch, (int)blockIdx.x, (int)gridDim.x, groups);
        Q = my_groups * VM * stages;
        __asm__ volatile("" : : "s"(Q), "s"(my_groups));  // materialized here
    };
    auto lstore = [&](int buf, const u32x4(&src)[IPW]) {
#pragma unroll
        for (int k = 0; k < IPW; ++k)
            *reinterpret_cast<u32x4 *>(lds + Lo.stage + buf * Lo.stage_bytes + plds[k]) = src[k];
    };
    // ---- prologue: the activation operand table, in LDS ---------------------
    // Item i = one 8-float chunk of x: block i/32, sub-block (i/4)%8, chunk
    // i%4, so the 4 chunks of a sub-block sit in 4 adjacent lanes. Every
    // lane loads its XIT chunks before any weight load is issued: the loads
    // complete in issue order, so waiting for x leaves the weight stream in
    // flight while the table is built.
  if constexpr (Q8 && (FUSE & kFuseQuant)) {
    // Q8 from f32 x: item i = 8 floats of sub-block (i/4)%8 of block i/32, the
    // sub-block's 4 items in 4 adjacent lanes (amax and the integer sum reduce
    // with two DPP quad permutes); the quantization steps are those of
    // quantize_q8_1_kernel, so xq/xd/xsum are bit-identical to it.
    const int nitems = bpr * 32;
    const int its = (nitems + NW * 64 - 1) / (NW * 64);  // <= XIT
    f32x4 xv0[XIT], xv1[XIT];
#pragma unroll
    for (int it = 0; it < XIT; ++it) {
        if (it >= its) break;
        const int i = std::min(tid + it * NW * 64, nitems - 1);
        xv0[it] = ld_f32x4(x + (size_t)i * 8);
        xv1[it] = ld_f32x4(x + (size_t)i * 8 + 4);
    }
    gload_first(stg[0]);
    plan();
#pragma unroll
    for (int it = 0; it < XIT; ++it) {
        if (it >= its) break;
        const int i = tid + it * NW * 64;
        const float v[8] = {xv0[it][0], xv0[it][1], xv0[it][2], xv0[it][3],
                            xv1[it][0], xv1[it][1], xv1[it][2], xv1[it][3]};
        float amax = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[e]));
        amax = fmaxf(amax, quad_xor<1>(amax));
        amax = fmaxf(amax, quad_xor<2>(amax));
        float d = __fdiv_rn(amax, 127.0f);
        float id = (amax > 0.0f) ? __fdiv_rn(127.0f, amax) : 0.0f;
        if (!isfinite(id)) {
            id = 0.0f;
            d = 0.0f;
        }
        int sum = 0;
        uint32_t p0 = 0, p1 = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            int q = (int)__builtin_rintf(__fmul_rn(v[e], id));  // NaN converts to 0
            q = std::max(-127, std::min(127, q));
            sum += q;
            if (e < 4) p0 |= (uint32_t)(q & 0xFF) << (8 * e);
            else p1 |= (uint32_t)(q & 0xFF) << (8 * (e - 4));
        }
        sum += __builtin_bit_cast(int, quad_xor<1>(__builtin_bit_cast(float, sum)));
        sum += __builtin_bit_cast(int, quad_xor<2>(__builtin_bit_cast(float, sum)));
        if (i >= nitems) continue;
        const int b = i >> 5, sb = (i >> 2) & 7, j = i & 3;
        *reinterpret_cast<u32x2 *>(lds + (size_t)b * 256 + sb * 32 + j * 8) = u32x2{p0, p1};
        if (j == 0) {
            meta[b * 16 + sb] = d;
            meta[b * 16 + 8 + sb] = (float)sum;
        }
    }
  } else if constexpr (Q8) {
    // Q8: copy xq (16 B items 0 .. 16*bpr), then xd and xsum (4 floats per
    // item) to LDS, loads again issued ahead of the weight stream
    const int nq = bpr * 16, nitems = bpr * 20;
    const int its = (nitems + NW * 64 - 1) / (NW * 64);  // <= XIT
    u32x4 cv[XIT];
#pragma unroll
    for (int it = 0; it < XIT; ++it) {
        if (it >= its) break;
        const int i = std::min(tid + it * NW * 64, nitems - 1);
        const uint8_t *src = i < nq ? reinterpret_cast<const uint8_t *>(xq) + (size_t)i * 16
                           : i < nq + 2 * bpr ? reinterpret_cast<const uint8_t *>(xdv + (size_t)(i - nq) * 4)
                                              : reinterpret_cast<const uint8_t *>(xsv + (size_t)(i - nq - 2 * bpr) * 4);
        cv[it] = ld_u32x4(src);
    }
    gload_first(stg[0]);
    plan();
#pragma unroll
    for (int it = 0; it < XIT; ++it) {
        const int i = tid + it * NW * 64;
        if (i >= nitems) break;
        uint32_t dst;
        if (i < nq) {
            dst = (uint32_t)i * 16u;
        } else {
            const int k = (i < nq + 2 * bpr) ? i - nq : i - nq - 2 * bpr;  // 4-float chunk
            dst = Lo.meta + (uint32_t)(((k >> 1) * 16 + (i < nq + 2 * bpr ? 0 : 8) + 4 * (k & 1)) * 4);
        }
        *reinterpret_cast<u32x4 *>(lds + dst) = cv[it];
    }
  } else {
    const int nitems = bpr * 32;
    const int its = (nitems + NW * 64 - 1) / (NW * 64);  // <= XIT
    f32x4 xv0[XIT], xv1[XIT], nv0[XIT], nv1[XIT];
#pragma unroll
    for (int it = 0; it < XIT; ++it) {
        if (it >= its) break;
        const int i = std::min(tid + it * NW * 64, nitems - 1);
        xv0[it] = ld_f32x4(x + (size_t)i * 8);
        xv1[it] = ld_f32x4(x + (size_t)i * 8 + 4);
        if constexpr (NORM) {
            nv0[it] = ld_f32x4(fz.nw + (size_t)i * 8);
            nv1[it] = ld_f32x4(fz.nw + (size_t)i * 8 + 4);
        }
    }
    float ssq = 0.0f;  // kFuseNorm: this lane's sum of x^2
    gload_first(stg[0]);
    plan();

    for (int b = tid; b < bpr; b += NW * 64)  // the blocks' zero slots
        *reinterpret_cast<u32x4 *>(lds + (size_t)b * Lo.tab_stride + 1024) = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int it = 0; it < XIT; ++it) {
        if (it >= its) break;
        const int i = tid + it * NW * 64;  // lanes of one sub-block share i/4
        f32x4 v0 = xv0[it], v1 = xv1[it];
        if constexpr (NORM) {
            if (i < nitems)  // items past the end are clamped duplicates
                ssq += ((v0[0] * v0[0] + v0[1] * v0[1]) + (v0[2] * v0[2] + v0[3] * v0[3])) +
                       ((v1[0] * v1[0] + v1[1] * v1[1]) + (v1[2] * v1[2] + v1[3] * v1[3]));
            v0 *= nv0[it];  // the table holds x .* nw; rstd scales the results
            v1 *= nv1[it];
        }
        float amax = fmaxf(fmaxf(fmaxf(fabsf(v0[0]), fabsf(v0[1])), fmaxf(fabsf(v0[2]), fabsf(v0[3]))),
                           fmaxf(fmaxf(fabsf(v1[0]), fabsf(v1[1])), fmaxf(fabsf(v1[2]), fabsf(v1[3]))));
        float sum = ((v0[0] + v0[1]) + (v0[2] + v0[3])) + ((v1[0] + v1[1]) + (v1[2] + v1[3]));
        amax = fmaxf(amax, quad_xor<1>(amax));
        amax = fmaxf(amax, quad_xor<2>(amax));
        sum += quad_xor<1>(sum);
        sum += quad_xor<2>(sum);
        if (i >= nitems) continue;
        if constexpr (I8) {
            i8_table_entry(lds, meta, i >> 5, (i >> 2) & 7, i & 3, v0, v1, amax, sum);
            continue;
        }
        int e = 0;  // x*2^e puts the sub-block's largest |x| in [2^13, 2^14)
        if (amax > 0.0f && amax <= 3.402823466e38f) {
            int ex;
            frexpf(amax, &ex);  // amax in [2^(ex-1), 2^ex)
            e = std::min(std::max(14 - ex, -103), 140);  // 2^(24 - e) stays finite
        }
        const int b = i >> 5, sb = (i >> 2) & 7, j = i & 3;
        if (j == 0) {
            // Q4_K high-nibble operands are 16q*2^-24 (masked in place); Q5_K's are q*2^-24
            meta[b * 16 + sb] = ldexpf(1.0f, ((sb & 1) && !Q5 ? 20 : 24) - e);
            meta[b * 16 + 8 + sb] = sum;
        }
        // table entry (c, h) of this chunk: byte offset pair_byte_offset(c/2, h)
        // = 32*(sb/2) + 8*j within the qs run, nibble parity c%2 = sb%2
        const int G = sb >> 1;
        const int c = 2 * (2 * (G >> 1) + (j & 1)) + (sb & 1), h = 2 * (G & 1) + (j >> 1);
        // slot q holds byte o + {0,2,1,3,4,6,5,7}[q] (see the B operand build).
        // xh = x*2^e rounded toward zero to f16, xl = the (exact) f32
        // remainder rounded toward zero: two packed conversions per pair.
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
        uint8_t *ent = lds + (size_t)b * Lo.tab_stride + (size_t)((c * 4 + h) * 32);
        *reinterpret_cast<u32x4 *>(ent) = hh;
        *reinterpret_cast<u32x4 *>(ent + 16) = hl;
    }
    if constexpr (NORM) {
        // one partial per wavefront; read after the stream's last barrier
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) ssq += __shfl_xor(ssq, off, 64);
        if (lane == 0) reinterpret_cast<float *>(lds + Lo.normp)[wave] = ssq;
    }
  }
    // Stage q's position: column t = q % stages and pass vg = q / stages (row
    // group vg / VM, matrix vg % VM). The stage loop keeps it in counters, so
    // no step divides by the (run-time) stage count.
    struct StagePos {
        int t, vg;
    };
    auto pos_of = [&](int q) { return StagePos{q % stages, q / stages}; };
    auto advance = [&](StagePos p, int k) {
        for (int i = 0; i < k; ++i)
            if (++p.t == stages) {
                p.t = 0;
                ++p.vg;
            }
        return p;
    };
    // the base of the stage at p
    auto paddr = [&](StagePos p) -> UnitAddr {
        const uint32_t r0 =
            (uint32_t)sched_group(sch, (int)blockIdx.x, (int)gridDim.x, p.vg / VM) * (uint32_t)gr;
        const uint8_t *wm = (VM == 2 && (p.vg & 1)) ? fz.w2 : w;
        return uaddr(r0, (uint32_t)(p.t * C * BB), wm);
    };
    // stage q (past the last one: the last again, a cache hit)
    auto gload = [&](int q, u32x4(&dst)[IPW]) { gload_u(paddr(pos_of(std::min(q, Q - 1))), dst); };
#pragma unroll
    for (int f = 1; f < PF; ++f) gload(f, stg[f]);
    // (the barrier before the first stage is computed also orders the table)
    lstore(0, stg[0]);

    // ---- per-lane constants -------------------------------------------------
    // B lane (n16, g): W row n16, k-slot group g. Accumulator lane: rows
    // m = 4g..4g+3 of the 16x16 result = (sub-block 2g, xh), (2g, xl),
    // (2g+1, xh), (2g+1, xl) of W row n16 -- both parts of a sub-block land in
    // the same lane, so merging xh and xl is an in-lane add.
    const int n16 = lane & 15, g = lane >> 4, jq = g >> 1, sh = 16 * (g & 1);
    // scales4/mins4 of quad jq without a divergent branch: the low bits come
    // from scale dword 0 (jq = 0) or 2 (jq = 1), the top two bits of quad 1
    // from dword 0 (scales) or 1 (mins)
    const uint32_t lmask = jq ? 0x0F0F0F0Fu : 0x3F3F3F3Fu, hmask = jq ? 0x30303030u : 0u;
    // A operand address of MFMA c for block b: b*1040 + aoff[c], where lanes
    // whose row m takes no data from c point at the block's zero slot
    uint32_t aoff[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const int o = pair_byte_offset(c >> 1, g);
        const int sb = 2 * (o >> 5) + (c & 1);
        const bool hit = (n16 >> 1) == sb;  // A lane m = n16 = 2*sb + part
        aoff[c] = hit ? (uint32_t)((c * 4 + g) * 32 + (n16 & 1) * 16) : 1024u;
    }
    uint32_t aoff8[4];  // I8: the int8 A operands (i8_aoff)
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) aoff8[c4] = i8_aoff(c4, n16, g);
    // y contribution of one tile: sub-blocks 2g, 2g+1 of W row n16 in block b,
    // from their q*x sums s0, s1 (scaled by corr) and the block header hd.
    auto decode = [&](const u32x4 &hd, int b, float s0, float s1) -> float {
        const float d = half_bits_finite(hd[0]), dmin = half_bits_finite(hd[0] >> 16);
        const uint32_t scs = jq ? hd[3] : hd[1], mns = jq ? (hd[3] >> 4) : hd[2];
        const uint32_t scq = ((scs & lmask) | ((hd[1] >> 2) & hmask)) >> sh;
        const uint32_t mnq = ((mns & lmask) | ((hd[2] >> 2) & hmask)) >> sh;
        const float *mb = meta + b * 16 + 2 * g;
        const float t1 = (float)(scq & 0xFFu) * (s0 * mb[0]) + (float)((scq >> 8) & 0xFFu) * (s1 * mb[1]);
        const float t2 = (float)(mnq & 0xFFu) * mb[8] + (float)((mnq >> 8) & 0xFFu) * mb[9];
        return d * t1 - dmin * t2;
    };
    // Q8: this lane's 32 qs bytes of W row n16 in block b are elements
    // 16*(g&1) .. +15 of sub-blocks s0 = 2*(g>>1) (low nibbles of q0), s0+1
    // (high), s0+4 (low nibbles of q1) and s0+5 (high); the other halves of
    // those sub-blocks sit in lane group g^1. The dmin*m*xsum term is added by
    // the lanes with g even only.
    auto decode_q8 = [&](const u32x4 &hd, int b, const u32x4 &q0, const u32x4 &q1) -> float {
        const int s0 = 2 * (g >> 1), half = g & 1;
        const uint8_t *xb = lds + (size_t)b * 256 + 16 * half;
        const u32x4 x0 = *reinterpret_cast<const u32x4 *>(xb + s0 * 32);
        const u32x4 x1 = *reinterpret_cast<const u32x4 *>(xb + (s0 + 1) * 32);
        const u32x4 x4 = *reinterpret_cast<const u32x4 *>(xb + (s0 + 4) * 32);
        const u32x4 x5 = *reinterpret_cast<const u32x4 *>(xb + (s0 + 5) * 32);
        int i0 = 0, i1 = 0, i4 = 0, i5 = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            i0 = __builtin_amdgcn_sdot4((int)(q0[j] & 0x0F0F0F0Fu), (int)x0[j], i0, false);
            i1 = __builtin_amdgcn_sdot4((int)((q0[j] >> 4) & 0x0F0F0F0Fu), (int)x1[j], i1, false);
            i4 = __builtin_amdgcn_sdot4((int)(q1[j] & 0x0F0F0F0Fu), (int)x4[j], i4, false);
            i5 = __builtin_amdgcn_sdot4((int)((q1[j] >> 4) & 0x0F0F0F0Fu), (int)x5[j], i5, false);
        }
        const float d = half_bits_finite(hd[0]), dmin = half_bits_finite(hd[0] >> 16);
        // sub-blocks s0, s0+1 are bytes s0, s0+1 of quad 0; s0+4, s0+5 of quad 1
        const uint32_t shq = 8 * s0;
        const uint32_t sc0 = scales4(0, hd[1], hd[3]) >> shq, sc1 = scales4(1, hd[1], hd[3]) >> shq;
        const uint32_t mn0 = mins4(0, hd[2], hd[3]) >> shq, mn1 = mins4(1, hd[2], hd[3]) >> shq;
        const float *mb = meta + b * 16;  // xd[8] | xsum[8]
        const float mk = half ? 0.0f : dmin;
        float r = mb[s0] * (d * (float)(sc0 & 0xFFu) * (float)i0 - mk * (float)(mn0 & 0xFFu) * mb[8 + s0]);
        r += mb[s0 + 1] * (d * (float)((sc0 >> 8) & 0xFFu) * (float)i1 -
                           mk * (float)((mn0 >> 8) & 0xFFu) * mb[9 + s0]);
        r += mb[s0 + 4] * (d * (float)(sc1 & 0xFFu) * (float)i4 - mk * (float)(mn1 & 0xFFu) * mb[12 + s0]);
        r += mb[s0 + 5] * (d * (float)((sc1 >> 8) & 0xFFu) * (float)i5 -
                           mk * (float)((mn1 >> 8) & 0xFFu) * mb[13 + s0]);
        return r;
    };

    // two LDS stage buffers only when double-buffered and K spans > 1 stage
    // (the layout allocates exactly that); otherwise one buffer, refilled
    // after a barrier, also across row groups of a persistent work-group
    const bool dbuf = DB && stages > 1;
    float yaccA = 0.0f, yaccB = 0.0f;  // R = 32: rows of tile A / tile B; R = 16: yaccA only
    // One stage: compute it, then (when `more`) move stage q+1 from its
    // register set into the other LDS buffer and refill that set with stage
    // q+1+PF. F = q % PF is a compile-time constant at every call site.
    // stage q at position pq; pn: the position of the refill, stage
    // min(q + 1 + PF, Q - 1)
    auto step = [&](const int q, const StagePos pq, const StagePos pn, auto fc, const bool more) {
        constexpr int F = decltype(fc)::value;
        const int t = pq.t;
        // the refill's base, worked out before the stage's loads are waited for
        const UnitAddr na = paddr(pn);
        const uint8_t *sbuf = lds + Lo.stage + (dbuf ? (q & 1) * Lo.stage_bytes : 0u);
        for (int u = wave; u < UNITS; u += NW) {
            // tile A = (rows rowA.., block cbA), tile B = (rows rowB.., block cbB)
            const int cbA = (R == 32) ? u : 2 * u, cbB = (R == 32) ? u : 2 * u + 1;
            const int rowA = 0, rowB = (R == 32) ? 16 : 0;
            const int bA = t * C + cbA, bB = t * C + cbB;
            if (bA >= bpr) break;
            const bool hasB = bB < bpr;
            const int bBc = hasB ? bB : bA;  // past the end: reuse tile A's operands
            auto piece = [&](int row, int cb, int pc) -> const u32x4 & {
                return *reinterpret_cast<const u32x4 *>(sbuf + (row * RP + cb * BP + pc) * 16);
            };
            // qs pieces 1+g, 5+g (Q5_K: 3+g, 7+g: qh takes pieces 1 and 2)
            constexpr int QS = Q5 ? 3 : 1;
            const u32x4 qa0 = piece(rowA + n16, cbA, QS + g), qa1 = piece(rowA + n16, cbA, QS + 4 + g);
            const u32x4 qb0 = piece(rowB + n16, cbB, QS + g), qb1 = piece(rowB + n16, cbB, QS + 4 + g);
            const u32x4 hdA = piece(rowA + n16, cbA, 0), hdB = piece(rowB + n16, cbB, 0);
          if constexpr (Q8) {
            const float cA = decode_q8(hdA, bA, qa0, qa1);
            const float cB = decode_q8(hdB, bBc, qb0, qb1);
            if (R == 32) {
                yaccA += cA;
                yaccB += cB;
            } else {
                yaccA += hasB ? cA + cB : cA;
            }
          } else if constexpr (I8) {
            float sa0, sa1, sb0, sb1;
            if constexpr (Q5) {
                const u32x4 hqa = piece(rowA + n16, cbA, 1 + (g & 1));
                const u32x4 hqb = piece(rowB + n16, cbB, 1 + (g & 1));
                i8_tile<true>(lds + (uint32_t)bA * 1040u, aoff8, qa0, qa1, sa0, sa1, hqa, g);
                i8_tile<true>(lds + (uint32_t)bBc * 1040u, aoff8, qb0, qb1, sb0, sb1, hqb, g);
            } else {
                i8_tile(lds + (uint32_t)bA * 1040u, aoff8, qa0, qa1, sa0, sa1);
                i8_tile(lds + (uint32_t)bBc * 1040u, aoff8, qb0, qb1, sb0, sb1);
            }
            const float cA = decode(hdA, bA, sa0, sa1);
            const float cB = decode(hdB, bBc, sb0, sb1);
            if (R == 32) {
                yaccA += cA;
                yaccB += cB;
            } else {
                yaccA += hasB ? cA + cB : cA;
            }
          } else {
            // Q5_K: the qh bytes of this lane's qs bytes t are qh[t % 32], the
            // same byte offsets within qh piece 1 + (g & 1)
            u32x4 hqa = {0u, 0u, 0u, 0u}, hqb = {0u, 0u, 0u, 0u};
            if constexpr (Q5) {
                hqa = piece(rowA + n16, cbA, 1 + (g & 1));
                hqb = piece(rowB + n16, cbB, 1 + (g & 1));
            }
            f32x4 accA = {0.f, 0.f, 0.f, 0.f}, accB = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const half8 aA = *reinterpret_cast<const half8 *>(lds + (uint32_t)bA * 1040u + aoff[c]);
                const half8 aB = (R == 32) ? aA
                    : *reinterpret_cast<const half8 *>(lds + (uint32_t)bBc * 1040u + aoff[c]);
                const int p = c >> 1;
                const uint32_t mask = (c & 1) ? 0x00F000F0u : 0x000F000Fu;
                const uint32_t wa0 = p < 2 ? qa0[2 * p] : qa1[2 * p - 4];
                const uint32_t wa1 = p < 2 ? qa0[2 * p + 1] : qa1[2 * p - 3];
                const uint32_t wb0 = p < 2 ? qb0[2 * p] : qb1[2 * p - 4];
                const uint32_t wb1 = p < 2 ? qb0[2 * p + 1] : qb1[2 * p - 3];
                u32x4 ba, bb;
                if constexpr (Q5) {
                    // 5-bit q bytes: the nibble plus bit j (this MFMA's
                    // sub-block) of the matching qh byte at bit 4, then two
                    // bytes per dword into f16 subnormals, as for Q4_K
                    const int d = p < 2 ? 2 * p : 2 * p - 4;
                    const int j = 2 * ((p < 2 ? 0 : 2) + (g >> 1)) + (c & 1);
                    auto q5 = [&](uint32_t wq, uint32_t hq) -> uint32_t {
                        const uint32_t nib = (c & 1) ? ((wq >> 4) & 0x0F0F0F0Fu) : (wq & 0x0F0F0F0Fu);
                        return nib | (((hq >> j) & 0x01010101u) << 4);
                    };
                    const uint32_t a0 = q5(wa0, hqa[d]), a1 = q5(wa1, hqa[d + 1]);
                    const uint32_t b0 = q5(wb0, hqb[d]), b1 = q5(wb1, hqb[d + 1]);
                    constexpr uint32_t m5 = 0x001F001Fu;
                    ba = u32x4{a0 & m5, (a0 >> 8) & m5, a1 & m5, (a1 >> 8) & m5};
                    bb = u32x4{b0 & m5, (b0 >> 8) & m5, b1 & m5, (b1 >> 8) & m5};
                } else {
                    ba = u32x4{wa0 & mask, (wa0 >> 8) & mask, wa1 & mask, (wa1 >> 8) & mask};
                    bb = u32x4{wb0 & mask, (wb0 >> 8) & mask, wb1 & mask, (wb1 >> 8) & mask};
                }
                accA = __builtin_amdgcn_mfma_f32_16x16x32_f16(aA, __builtin_bit_cast(half8, ba), accA, 0, 0, 0);
                accB = __builtin_amdgcn_mfma_f32_16x16x32_f16(aB, __builtin_bit_cast(half8, bb), accB, 0, 0, 0);
            }
            const float cA = decode(hdA, bA, accA[0] + accA[1], accA[2] + accA[3]);
            const float cB = decode(hdB, bBc, accB[0] + accB[1], accB[2] + accB[3]);
            if (R == 32) {
                yaccA += cA;
                yaccB += cB;
            } else {
                yaccA += hasB ? cA + cB : cA;
            }
          }
        }
        const bool group_end = (t == stages - 1);
        // The row group's aux buffer alternates with the group's parity. With
        // one stage per group the next group's sums are written before any
        // barrier of its step, while the first R threads may still be reading
        // this group's: the buffer they read is the other one, and reusing it
        // two groups later is ordered by the barrier between.
        float *auxg = aux + (WV ? pq.vg : (pq.vg & 1)) * (NW * 32);
        if (group_end) {
            // sum the 4 lanes (g = 0..3) of each row, then one value per row
            // and tile into aux (free after the prologue)
            yaccA += __shfl_xor(yaccA, 16, 64);
            yaccA += __shfl_xor(yaccA, 32, 64);
            yaccB += __shfl_xor(yaccB, 16, 64);
            yaccB += __shfl_xor(yaccB, 32, 64);
            if (lane < 16) {
                auxg[wave * 32 + lane] = yaccA;
                auxg[wave * 32 + 16 + lane] = yaccB;
            }
        }
        if constexpr (WV) {
            // own unit only: its reads above come before these stores (LDS
            // operations of one wavefront execute in order)
            if (more) {
                lstore(0, stg[(F + 1) % PF]);
                __asm__ volatile("" ::: "memory");
                gload_u(na, stg[(F + 1) % PF]);
            }
            if (group_end) {
                yaccA = 0.0f;
                yaccB = 0.0f;
            }
            return;
        }
        if (more) {
            if (!dbuf) __syncthreads();  // every wave is done reading the single buffer
            lstore(dbuf ? ((q + 1) & 1) : 0, stg[(F + 1) % PF]);
            gload_u(na, stg[(F + 1) % PF]);
        }
        __syncthreads();
        if (group_end) {
            // cross-wave reduction of this row group (its own aux buffer)
            if (tid < R) {
                float sum = 0.0f;
                for (int wv = 0; wv < NW; ++wv) sum += auxg[wv * 32 + tid];
                reinterpret_cast<float *>(lds + Lo.ybuf)[pq.vg * R + tid] = sum;
            }
            yaccA = 0.0f;
            yaccB = 0.0f;
        }
    };
    // Main loop: every step has a next stage, so the store/refill is
    // unconditional and the compiler waits only for the set being stored
    // (the loop is entered, and loops back, with the same load order).
    int q0 = 0;
    StagePos p0{0, 0};                                        // stage q0
    const StagePos qlast_pos = pos_of(std::max(Q - 1, 0));        // the last stage
    auto refill_pos = [&](int q, StagePos pq) {               // stage min(q + 1 + PF, Q - 1)
        return q + 1 + PF < Q ? advance(pq, 1 + PF) : qlast_pos;
    };
    if (Q > PF) {
        gload(PF, stg[0]);
        __syncthreads();
        for (; q0 + PF < Q; q0 += PF) {
            step(q0, p0, refill_pos(q0, p0), std::integral_constant<int, 0>{}, true);
            if constexpr (PF > 1) {
                const StagePos p1 = advance(p0, 1);
                step(q0 + 1, p1, refill_pos(q0 + 1, p1), std::integral_constant<int, 1 % PF>{}, true);
            }
            if constexpr (PF > 2) {
                const StagePos p2 = advance(p0, 2);
                step(q0 + 2, p2, refill_pos(q0 + 2, p2), std::integral_constant<int, 2 % PF>{}, true);
            }
            p0 = advance(p0, PF);
        }
    } else {
        __syncthreads();
    }
    // Tail: the last <= PF stages.
    if (q0 < Q) step(q0, p0, refill_pos(q0, p0), std::integral_constant<int, 0>{}, q0 + 1 < Q);
    if constexpr (PF > 1)
        if (q0 + 1 < Q) {
            const StagePos p1 = advance(p0, 1);
            step(q0 + 1, p1, refill_pos(q0 + 1, p1), std::integral_constant<int, 1 % PF>{}, q0 + 2 < Q);
        }
    if constexpr (PF > 2)
        if (q0 + 2 < Q) {
            const StagePos p2 = advance(p0, 2);
            step(q0 + 2, p2, refill_pos(q0 + 2, p2), std::integral_constant<int, 2 % PF>{}, q0 + 3 < Q);
        }
    __syncthreads();
    float rstd = 1.0f;
    if constexpr (NORM) {
        // rms_norm's 1/sqrt(mean(x^2) + eps) (kernels/rms_norm.hip:63-68)
        const float *np = reinterpret_cast<const float *>(lds + Lo.normp);
        float ss = 0.0f;
        for (int wv = 0; wv < NW; ++wv) ss += np[wv];
        rstd = rsqrtf(ss / (float)(bpr * kBlockElems) + fz.eps);
    }
    const float *yb = reinterpret_cast<const float *>(lds + Lo.ybuf);
    if constexpr (WV) {
        // pass vg's row ri: the wavefronts' sums in wavefront order (as the
        // per-stage reduction adds them)
        auto pass_sum = [&](int vg, int ri) -> float {
            float sum = 0.0f;
            for (int wv = 0; wv < NW; ++wv) sum += aux[(vg * NW + wv) * 32 + ri];
            return sum;
        };
        for (int i = tid; i < my_groups * R; i += NW * 64) {
            const int ri = i % R, gi = i / R;
            const int r = sched_group(sch, (int)blockIdx.x, (int)gridDim.x, gi) * gr + ri;
            if (ri < gr && r < n) {
                if constexpr (VM == 2) {
                    const float gv = pass_sum(2 * gi, ri) * rstd, uv = pass_sum(2 * gi + 1, ri) * rstd;
                    y[r] = glu_act(gv, fz.act) * uv;
                } else {
                    const float v0 = pass_sum(gi, ri);
                    const float v = NORM ? v0 * rstd : v0;
                    y[r] = (Q8 && !isfinite(v)) ? 0.0f : v;
                }
            }
        }
        return;
    }
    for (int i = tid; i < my_groups * R; i += NW * 64) {
        const int ri = i % R;
        const int r = sched_group(sch, (int)blockIdx.x, (int)gridDim.x, i / R) * gr + ri;
        if (ri < gr && r < n) {
            if constexpr (VM == 2) {
                // pass 2j = gate rows of group j, 2j+1 = up rows
                const int gi = (i / R) * 2 * R + (i % R);
                const float gv = yb[gi] * rstd, uv = yb[gi + R] * rstd;
                y[r] = glu_act(gv, fz.act) * uv;
            } else {
                const float v = NORM ? yb[i] * rstd : yb[i];
                y[r] = (Q8 && !isfinite(v)) ? 0.0f : v;  // Q8: the reference's clamp
            }
        }
    }
}

static int env_int(const char *name, int dflt) {
    const char *s = std::getenv(name);
    return (s && *s) ? std::atoi(s) : dflt;
}


// ---------------------------------------------------------- wave-private ---
// gemv_wave_kernel: the matrix-core GEMV with every wavefront streaming its
// own unit (f32 activations, Q4_K). The stage of a row group is UNITS = NW
// units (R = 16: blocks 2u, 2u+1 of the 16 rows; R = 32: block u of both
// 16-row tiles); wavefront u loads exactly the 288 16-byte pieces of unit u
// (18- or 9-piece runs of its rows, 16 bytes per lane), stores them to its own
// LDS slot and computes from it, so no work-group barrier sits between
// stages: a wavefront starts on its unit as soon as its own pieces land. Its
// row sums of each row group go to LDS (one slot per group and wavefront)
// and are reduced across wavefronts once, after the stream, in the same
// order as gemv_mfma_kernel (identical results in the f16 form).
// I8 (the int8 form): each 32-value sub-block of x is scaled by its own
// power of two to integers |X| <= 2^22 held as three signed 8-bit digits,
// the nibbles are the int8 B operand as they sit in the qs bytes (masked,
// not spread), and v_mfma_i32_16x16x64_i8 sums 64 products exactly: half
// the MFMAs, A-operand reads and nibble masks of the f16 form, whose x is
// split into two f16 halves (22 bits) times 16-bit B operands.

struct WaveLayout {
    uint32_t meta, slots, aux;
    size_t total;
};
template <int R, int NW>
__host__ __device__ constexpr uint32_t wave_slot_pitch() { return R == 32 ? 9u : 19u; }  // pieces per row
template <int R, int NW>
__host__ __device__ inline WaveLayout wave_layout(int bpr, int rounds) {
    WaveLayout L;
    L.meta = (uint32_t)bpr * 1040u;
    L.slots = L.meta + (uint32_t)bpr * 64u;
    L.aux = L.slots + (uint32_t)NW * R * wave_slot_pitch<R, NW>() * 16u;
    L.total = (size_t)L.aux + (size_t)rounds * NW * R * 4;
    return L;
}

// DIRECT (one unit per wavefront: a single stage, one group per work-group):
// every lane loads the three pieces it computes with (block header, quant
// pieces 1+g and 5+g of its row) straight into registers, with no LDS slot.
template <int R, int C, int NW, int XIT, bool DIRECT = false, bool I8 = false>
__global__ __launch_bounds__(NW * 64) void gemv_wave_kernel(const uint8_t *__restrict__ w,
                                                            const float *__restrict__ x,
                                                            float *__restrict__ y, int n, int bpr,
                                                            int rounds, GemvSched sch, int gr) {
    constexpr int UNITS = (R == 32) ? C : C / 2;
    static_assert(UNITS == NW, "one unit per wavefront and stage");
    static_assert(R == 32 || C % 2 == 0, "R = 16: a unit is a pair of blocks");
    constexpr int BP = 9, BB = 144;
    constexpr int RUN = (R == 32) ? BP : 2 * BP;         // pieces of one row in a unit
    constexpr int UP = R * RUN;                          // pieces per unit (288)
    constexpr int IPW = (UP + 63) / 64;                  // wave loads per unit
    constexpr uint32_t SP = wave_slot_pitch<R, NW>();    // LDS pieces per slot row
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const WaveLayout Lo = wave_layout<R, NW>(bpr, rounds);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    float *meta = reinterpret_cast<float *>(lds + Lo.meta);
    float *aux = reinterpret_cast<float *>(lds + Lo.aux);
    const size_t row_bytes = (size_t)bpr * BB;
    const int stages = (bpr + C - 1) / C;
    // this wavefront's unit: blocks cb0 (and cb0 + 1 when R = 16) of each stage
    const int cb0 = (R == 32) ? wave : 2 * wave;
    uint8_t *slot = lds + Lo.slots + (uint32_t)wave * (R * SP * 16u);

    // piece p of the unit: row p / RUN, piece p % RUN of the row's run (R = 16:
    // block cb0 + (p % RUN) / 9), clamped past the unit's 288; poff is its
    // byte offset from the unit's first piece in row 0 (tile rows past the
    // group re-read its last row)
    uint32_t poff[IPW], plds[IPW];
#pragma unroll
    for (int k = 0; k < IPW; ++k) {
        const int p = std::min(k * 64 + lane, UP - 1);
        const int row = p / RUN, rem = p - row * RUN;
        poff[k] = (uint32_t)std::min(row, gr - 1) * (uint32_t)row_bytes + (uint32_t)(16 * rem);
        plds[k] = (uint32_t)((row * SP + rem) * 16);
    }
    u32x4 stg[IPW];
    // unit pieces of stage column tcol of the rows from r0: one uniform base
    // and a 32-bit offset per lane, so the next unit's loads go out one
    // v_min after the current unit's slot stores. A unit wholly past the row
    // end re-reads the row's last blocks (cache hits); the second block of a
    // unit that starts at an odd row's last block, and rows past the matrix,
    // read what follows (no result uses them), clamped to the last piece.
    const uint64_t wlast = (uint64_t)n * row_bytes - 16;
    const uint32_t lastcol = (uint32_t)std::max(bpr - (R == 32 ? 1 : 2), 0) * BB;
    auto unit_b0 = [&](uint32_t r0, uint32_t tcol) {
        const uint32_t c = tcol + (uint32_t)(cb0 * BB);
        return (uint64_t)std::min(r0, (uint32_t)(n - 1)) * row_bytes + (c < (uint32_t)row_bytes ? c : lastcol);
    };
    auto unit_lim = [&](uint64_t b0) { return (uint32_t)std::min<uint64_t>(wlast - b0, 0xFFFFFFF0ull); };
    auto gload_b = [&](uint64_t b0, uint32_t lim) {
        const uint8_t *base = w + b0;
#pragma unroll
        for (int k = 0; k < IPW; ++k) stg[k] = ld_u32x4(base + std::min(poff[k], lim));
    };
    auto gload_at = [&](uint32_t r0, uint32_t tcol) {
        const uint64_t b0 = unit_b0(r0, tcol);
        gload_b(b0, unit_lim(b0));
    };
    auto lstore = [&]() {
#pragma unroll
        for (int k = 0; k < IPW; ++k) *reinterpret_cast<u32x4 *>(slot + plds[k]) = stg[k];
    };
    // DIRECT: header, pieces 1+g and 5+g of the unit's block(s) for this lane's
    // row(s): {A: hd, q0, q1, B: hd, q0, q1} (R = 16: blocks cb0, cb0 + 1 of
    // row n16; R = 32: block cb0 of rows n16 and 16 + n16)
    u32x4 dreg[6];
    auto gload_direct = [&](uint32_t r0) {
        const int dl = lane & 15, dg = lane >> 4;
        const uint32_t glast = (uint32_t)gr - 1u, rlast = (uint32_t)(n - 1);
        const uint32_t rA = std::min(r0 + std::min((uint32_t)dl, glast), rlast);
        const uint32_t rB = (R == 32) ? std::min(r0 + std::min((uint32_t)(16 + dl), glast), rlast) : rA;
        const uint32_t bA = (uint32_t)std::min(cb0, bpr - 1);
        const uint32_t bB = (R == 32) ? bA : (uint32_t)std::min(cb0 + 1, bpr - 1);
        const uint8_t *pA = w + ((uint64_t)rA * row_bytes + bA * BB);
        const uint8_t *pB = w + ((uint64_t)rB * row_bytes + bB * BB);
        dreg[0] = ld_u32x4(pA);
        dreg[1] = ld_u32x4(pA + 16 * (1 + dg));
        dreg[2] = ld_u32x4(pA + 16 * (5 + dg));
        dreg[3] = ld_u32x4(pB);
        dreg[4] = ld_u32x4(pB + 16 * (1 + dg));
        dreg[5] = ld_u32x4(pB + 16 * (5 + dg));
    };

    // ---- prologue: x loads, the first unit, then the activation table -------
    const int nitems = bpr * 32;
    const int its = (nitems + NW * 64 - 1) / (NW * 64);
    f32x4 xv0[XIT], xv1[XIT];
#pragma unroll
    for (int it = 0; it < XIT; ++it) {
        if (it >= its) break;
        const int i = std::min(tid + it * NW * 64, nitems - 1);
        xv0[it] = ld_f32x4(x + (size_t)i * 8);
        xv1[it] = ld_f32x4(x + (size_t)i * 8 + 4);
    }
    if constexpr (DIRECT)
        gload_direct((uint32_t)blockIdx.x * (uint32_t)gr);
    else
        gload_at((uint32_t)blockIdx.x * (uint32_t)gr, 0u);
    const int groups = (n + gr - 1) / gr;
    const int my_groups = sched_count(sch, (int)blockIdx.x, (int)gridDim.x, groups);
    const int Q = my_groups * stages;
    __asm__ volatile("" : : "s"(Q), "s"(my_groups));

    for (int b = tid; b < bpr; b += NW * 64)
        *reinterpret_cast<u32x4 *>(lds + (size_t)b * 1040 + 1024) = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int it = 0; it < XIT; ++it) {
        if (it >= its) break;
        const int i = tid + it * NW * 64;
        const f32x4 v0 = xv0[it], v1 = xv1[it];
        float amax = fmaxf(fmaxf(fmaxf(fabsf(v0[0]), fabsf(v0[1])), fmaxf(fabsf(v0[2]), fabsf(v0[3]))),
                           fmaxf(fmaxf(fabsf(v1[0]), fabsf(v1[1])), fmaxf(fabsf(v1[2]), fabsf(v1[3]))));
        float sum = ((v0[0] + v0[1]) + (v0[2] + v0[3])) + ((v1[0] + v1[1]) + (v1[2] + v1[3]));
        amax = fmaxf(amax, quad_xor<1>(amax));
        amax = fmaxf(amax, quad_xor<2>(amax));
        sum += quad_xor<1>(sum);
        sum += quad_xor<2>(sum);
        if (i >= nitems) continue;
        const int b = i >> 5, sb = (i >> 2) & 7, j = i & 3;
        if constexpr (I8) {
            i8_table_entry(lds, meta, b, sb, j, v0, v1, amax, sum);
            continue;
        }
        int e = 0;
        if (amax > 0.0f && amax <= 3.402823466e38f) {
            int ex;
            frexpf(amax, &ex);
            e = std::min(std::max(14 - ex, -103), 140);  // 2^(24 - e) stays finite
        }
        if (j == 0) {
            meta[b * 16 + sb] = ldexpf(1.0f, ((sb & 1) ? 20 : 24) - e);
            meta[b * 16 + 8 + sb] = sum;
        }
        const int G = sb >> 1;
        const int c = 2 * (2 * (G >> 1) + (j & 1)) + (sb & 1), h = 2 * (G & 1) + (j >> 1);
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
        uint8_t *ent = lds + (size_t)b * 1040 + (size_t)((c * 4 + h) * 32);
        *reinterpret_cast<u32x4 *>(ent) = hh;
        *reinterpret_cast<u32x4 *>(ent + 16) = hl;
    }
    __syncthreads();  // the table is complete; from here no wavefront waits for another

    // ---- per-lane constants (as in gemv_mfma_kernel) ------------------------
    const int n16 = lane & 15, g = lane >> 4, jq = g >> 1, sh = 16 * (g & 1);
    const uint32_t lmask = jq ? 0x0F0F0F0Fu : 0x3F3F3F3Fu, hmask = jq ? 0x30303030u : 0u;
    uint32_t aoff[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const int o = pair_byte_offset(c >> 1, g);
        const int sb = 2 * (o >> 5) + (c & 1);
        const bool hit = (n16 >> 1) == sb;
        aoff[c] = hit ? (uint32_t)((c * 4 + g) * 32 + (n16 & 1) * 16) : 1024u;
    }
    uint32_t aoff8[4];  // I8: the int8 A operands (i8_aoff)
#pragma unroll
    for (int c4 = 0; c4 < 4; ++c4) aoff8[c4] = i8_aoff(c4, n16, g);
    auto decode = [&](const u32x4 &hd, int b, float s0, float s1) -> float {
        const float d = half_bits_finite(hd[0]), dmin = half_bits_finite(hd[0] >> 16);
        const uint32_t scs = jq ? hd[3] : hd[1], mns = jq ? (hd[3] >> 4) : hd[2];
        const uint32_t scq = ((scs & lmask) | ((hd[1] >> 2) & hmask)) >> sh;
        const uint32_t mnq = ((mns & lmask) | ((hd[2] >> 2) & hmask)) >> sh;
        const float *mb = meta + b * 16 + 2 * g;
        const float t1 = (float)(scq & 0xFFu) * (s0 * mb[0]) + (float)((scq >> 8) & 0xFFu) * (s1 * mb[1]);
        const float t2 = (float)(mnq & 0xFFu) * mb[8] + (float)((mnq >> 8) & 0xFFu) * mb[9];
        return d * t1 - dmin * t2;
    };
    auto piece = [&](int row, int cbl, int pc) -> const u32x4 & {
        return *reinterpret_cast<const u32x4 *>(slot + (row * SP + cbl * BP + pc) * 16);
    };

    float yaccA = 0.0f, yaccB = 0.0f;
    int t = 0, ug = 0;  // this unit's stage, and its group's index in the work-group's schedule
    for (int q = 0; q < Q; ++q) {
        // the next unit (past the last one: the last again, a cache hit)
        int t1 = t + 1, g1 = ug;
        if (t1 == stages) {
            t1 = 0;
            ++g1;
        }
        if (q + 1 >= Q) {
            t1 = t;
            g1 = ug;
        }
        // its base, worked out before this unit's slot stores wait for its data
        const uint64_t nb0 =
            unit_b0((uint32_t)sched_group(sch, (int)blockIdx.x, (int)gridDim.x, g1) * (uint32_t)gr,
                    (uint32_t)(t1 * C * BB));
        const uint32_t nlim = unit_lim(nb0);
        if constexpr (!DIRECT) {
            __asm__ volatile("" : : "s"(nlim), "s"((uint32_t)nb0), "s"((uint32_t)(nb0 >> 32)));
            lstore();
            __asm__ volatile("" ::: "memory");  // the unit's reads follow its stores (in-order LDS)
            gload_b(nb0, nlim);  // unconditional, so the load-counter waits stay exact
        }
        const int bA = t * C + cb0, bB = (R == 32) ? bA : bA + 1;
        if (bA < bpr) {
            const bool hasB = bB < bpr;
            const int bBc = hasB ? bB : bA;
            const int rowB = (R == 32) ? 16 : 0, cbB = (R == 32) ? 0 : 1;
            const u32x4 qa0 = DIRECT ? dreg[1] : piece(n16, 0, 1 + g);
            const u32x4 qa1 = DIRECT ? dreg[2] : piece(n16, 0, 5 + g);
            const u32x4 qb0 = DIRECT ? dreg[4] : piece(rowB + n16, cbB, 1 + g);
            const u32x4 qb1 = DIRECT ? dreg[5] : piece(rowB + n16, cbB, 5 + g);
            const u32x4 hdA = DIRECT ? dreg[0] : piece(n16, 0, 0);
            const u32x4 hdB = DIRECT ? dreg[3] : piece(rowB + n16, cbB, 0);
          if constexpr (I8) {
            auto tile8 = [&](const u32x4 &hd, int b, const u32x4 &q0, const u32x4 &q1) -> float {
                float s0, s1;
                i8_tile(lds + (uint32_t)b * 1040u, aoff8, q0, q1, s0, s1);
                return decode(hd, b, s0, s1);
            };
            const float cA = tile8(hdA, bA, qa0, qa1);
            const float cB = tile8(hdB, bBc, qb0, qb1);
            if (R == 32) {
                yaccA += cA;
                yaccB += cB;
            } else {
                yaccA += hasB ? cA + cB : cA;
            }
          } else {
            f32x4 accA = {0.f, 0.f, 0.f, 0.f}, accB = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const half8 aA = *reinterpret_cast<const half8 *>(lds + (uint32_t)bA * 1040u + aoff[c]);
                const half8 aB = (R == 32) ? aA
                    : *reinterpret_cast<const half8 *>(lds + (uint32_t)bBc * 1040u + aoff[c]);
                const int p = c >> 1;
                const uint32_t mask = (c & 1) ? 0x00F000F0u : 0x000F000Fu;
                const uint32_t wa0 = p < 2 ? qa0[2 * p] : qa1[2 * p - 4];
                const uint32_t wa1 = p < 2 ? qa0[2 * p + 1] : qa1[2 * p - 3];
                const uint32_t wb0 = p < 2 ? qb0[2 * p] : qb1[2 * p - 4];
                const uint32_t wb1 = p < 2 ? qb0[2 * p + 1] : qb1[2 * p - 3];
                const u32x4 ba = u32x4{wa0 & mask, (wa0 >> 8) & mask, wa1 & mask, (wa1 >> 8) & mask};
                const u32x4 bb = u32x4{wb0 & mask, (wb0 >> 8) & mask, wb1 & mask, (wb1 >> 8) & mask};
                accA = __builtin_amdgcn_mfma_f32_16x16x32_f16(aA, __builtin_bit_cast(half8, ba), accA, 0, 0, 0);
                accB = __builtin_amdgcn_mfma_f32_16x16x32_f16(aB, __builtin_bit_cast(half8, bb), accB, 0, 0, 0);
            }
            const float cA = decode(hdA, bA, accA[0] + accA[1], accA[2] + accA[3]);
            const float cB = decode(hdB, bBc, accB[0] + accB[1], accB[2] + accB[3]);
            if (R == 32) {
                yaccA += cA;
                yaccB += cB;
            } else {
                yaccA += hasB ? cA + cB : cA;
            }
          }
        }
        if (t == stages - 1) {
            // this wavefront's sums of the group's rows, to its own slot
            yaccA += __shfl_xor(yaccA, 16, 64);
            yaccA += __shfl_xor(yaccA, 32, 64);
            yaccB += __shfl_xor(yaccB, 16, 64);
            yaccB += __shfl_xor(yaccB, 32, 64);
            float *ag = aux + ((size_t)ug * NW + wave) * R;
            if (lane < 16) {
                ag[lane] = yaccA;
                if (R == 32) ag[16 + lane] = yaccB;
            }
            yaccA = 0.0f;
            yaccB = 0.0f;
        }
        t = t1;
        ug = g1;
    }
    __syncthreads();
    for (int i = tid; i < my_groups * R; i += NW * 64) {
        const int gi = i / R, ri = i % R;
        const int r = sched_group(sch, (int)blockIdx.x, (int)gridDim.x, gi) * gr + ri;
        if (ri < gr && r < n) {
            const float *ag = aux + (size_t)gi * NW * R + ri;
            float sum = 0.0f;
            for (int wv = 0; wv < NW; ++wv) sum += ag[wv * R];
            y[r] = sum;
        }
    }
}

template <int R, int C, int NW, int XIT, bool DIRECT = false, bool I8 = false>
static hipError_t launch_wave_xit(const uint8_t *w, const float *x, float *y, int n, int bpr,
                                  hipStream_t stream, bool persistent, int gr) {
    auto kern = gemv_wave_kernel<R, C, NW, XIT, DIRECT, I8>;
    // DIRECT: one unit per wavefront (a single stage, one group per work-group)
    if (DIRECT && (persistent || bpr > C)) return hipErrorNotSupported;
    const hipError_t attr = allow_full_lds_by_addr((const void *)kern);
    if (attr != hipSuccess) return attr;
    if (gr <= 0 || gr > R) gr = R;
    const long groups = (n + gr - 1) / gr;
    long grid = groups, rounds = 1;
    GemvSched sch{(int)groups, 0};
    if (persistent) {
        const size_t base = wave_layout<R, NW>(bpr, 8).total;
        const int occ = occupancy_cached((const void *)kern, NW * 64, base,
                                         (int)std::min<size_t>(4, (160 * 1024) / base));
        const PersistPlan p = persistent_plan(groups, occ);
        grid = p.grid;
        rounds = p.rounds;
        sch = p.sch;
    }
    const WaveLayout Lo = wave_layout<R, NW>(bpr, (int)rounds);
    if (Lo.total > 160 * 1024) return hipErrorNotSupported;
    kern<<<(unsigned)grid, NW * 64, Lo.total, stream>>>(w, x, y, n, bpr, (int)rounds, sch, gr);
    return hipGetLastError();
}

// the kernels' LDS limit, set outside any stream capture
template <int R, int C, int NW>
static hipError_t wave_prepare() {
    hipError_t e = allow_full_lds_by_addr((const void *)gemv_wave_kernel<R, C, NW, 1>);
    if (e == hipSuccess) e = allow_full_lds_by_addr((const void *)gemv_wave_kernel<R, C, NW, 2>);
    if (e == hipSuccess) e = allow_full_lds_by_addr((const void *)gemv_wave_kernel<R, C, NW, 4>);
    if (e == hipSuccess) e = allow_full_lds_by_addr((const void *)gemv_wave_kernel<R, C, NW, 8>);
    if (e == hipSuccess) e = allow_full_lds_by_addr((const void *)gemv_wave_kernel<R, C, NW, 1, false, true>);
    if (e == hipSuccess) e = allow_full_lds_by_addr((const void *)gemv_wave_kernel<R, C, NW, 2, false, true>);
    if (e == hipSuccess) e = allow_full_lds_by_addr((const void *)gemv_wave_kernel<R, C, NW, 4, false, true>);
    if (e == hipSuccess) e = allow_full_lds_by_addr((const void *)gemv_wave_kernel<R, C, NW, 8, false, true>);
    return e;
}

// one unit per wavefront with direct register loads (single-stage rows)
template <int R, int C, int NW>
static hipError_t launch_wave_direct(const uint8_t *w, const float *x, float *y, int n, int bpr,
                                     hipStream_t stream, int gr, bool i8) {
    if (bpr * 32 > NW * 64) return hipErrorNotSupported;
    if (i8) return launch_wave_xit<R, C, NW, 1, true, true>(w, x, y, n, bpr, stream, false, gr);
    return launch_wave_xit<R, C, NW, 1, true>(w, x, y, n, bpr, stream, false, gr);
}

template <int R, int C, int NW>
static hipError_t launch_wave(const uint8_t *w, const float *x, float *y, int n, int bpr,
                              hipStream_t stream, bool persistent, bool i8, int gr = 0) {
    const int need = (bpr * 32 + NW * 64 - 1) / (NW * 64);
    if (i8) {
        if (need <= 1) return launch_wave_xit<R, C, NW, 1, false, true>(w, x, y, n, bpr, stream, persistent, gr);
        if (need <= 2) return launch_wave_xit<R, C, NW, 2, false, true>(w, x, y, n, bpr, stream, persistent, gr);
        if (need <= 4) return launch_wave_xit<R, C, NW, 4, false, true>(w, x, y, n, bpr, stream, persistent, gr);
        if (need <= 8) return launch_wave_xit<R, C, NW, 8, false, true>(w, x, y, n, bpr, stream, persistent, gr);
        return hipErrorNotSupported;
    }
    if (need <= 1) return launch_wave_xit<R, C, NW, 1>(w, x, y, n, bpr, stream, persistent, gr);
    if (need <= 2) return launch_wave_xit<R, C, NW, 2>(w, x, y, n, bpr, stream, persistent, gr);
    if (need <= 4) return launch_wave_xit<R, C, NW, 4>(w, x, y, n, bpr, stream, persistent, gr);
    if (need <= 8) return launch_wave_xit<R, C, NW, 8>(w, x, y, n, bpr, stream, persistent, gr);
    return hipErrorNotSupported;
}

// Activation operands of one launch: f32 x, or (Q8) int8 xq with its
// per-sub-block scale xd and sum xsum.
struct GemvAct {
    const float *x;
    const int8_t *xq;
    const float *xd, *xsum;
};

// Allows the kernel the whole 160 KiB of gfx950 LDS (once per process).
template <int R, int C, int NW, int PF, bool DB, int XIT, bool Q8, int FUSE>
static hipError_t lds_attr() {
    static std::atomic<int> lds_state[64];
    return allow_full_lds((const void *)gemv_mfma_kernel<R, C, NW, PF, DB, XIT, Q8, FUSE>,
                          lds_state);
}

template <int R, int C, int NW, int PF, bool DB, bool Q8, int FUSE = 0>
static hipError_t lds_attr_all() {
    hipError_t e = lds_attr<R, C, NW, PF, DB, 1, Q8, FUSE>();
    if (e == hipSuccess) e = lds_attr<R, C, NW, PF, DB, 2, Q8, FUSE>();
    if (e == hipSuccess) e = lds_attr<R, C, NW, PF, DB, 4, Q8, FUSE>();
    if (e == hipSuccess) e = lds_attr<R, C, NW, PF, DB, 8, Q8, FUSE>();
    return e;
}

template <int R, int C, int NW, int PF, bool DB, int XIT, bool Q8, int FUSE>
static hipError_t launch_xit(const uint8_t *w, const GemvAct &a, const GemvFuse &fz, float *y,
                             int n, int bpr, hipStream_t stream, bool persistent, int gr) {
    auto kern = gemv_mfma_kernel<R, C, NW, PF, DB, XIT, Q8, FUSE>;
    const hipError_t attr = lds_attr<R, C, NW, PF, DB, XIT, Q8, FUSE>();
    if (attr != hipSuccess) return attr;
    if (gr <= 0 || gr > R) gr = R;
    const long groups = (n + gr - 1) / gr;
    long grid = groups, rounds = 1;
    GemvSched sch{(int)groups, 0};
    if (persistent) {
        static const int occ_env = env_int("MGQ_GEMV_OCC", 0);
        const size_t base = mfma_layout(bpr, R, C, NW, 8, DB, Q8, FUSE).total;
        // resident work-groups per CU (registers and LDS)
        int occ = occupancy_cached((const void *)kern, NW * 64, base,
                                   (int)std::min<size_t>(4, (160 * 1024) / base));
        if (occ_env > 0) occ = occ_env;
        const PersistPlan p = persistent_plan(groups, occ);
        grid = p.grid;
        rounds = p.rounds;
        sch = p.sch;
    }
    const MfmaLayout Lo = mfma_layout(bpr, R, C, NW, (int)rounds, DB, Q8, FUSE);
    if (Lo.total > 160 * 1024) return hipErrorNotSupported;
    kern<<<(unsigned)grid, NW * 64, Lo.total, stream>>>(w, a.x, a.xq, a.xd, a.xsum, y, n, bpr,
                                                        (int)rounds, fz, sch, gr);
    return hipGetLastError();
}

// The activation loads per lane (XIT) are a compile-time count so they stay
// in registers: 1, 2, 4 or 8 (f32: 8-float chunks, bpr*32 of them; Q8:
// 16-byte items, bpr*20 of them).
template <int R, int C, int NW, int PF, bool DB, bool Q8, int FUSE>
static hipError_t launch_cfg(const uint8_t *w, const GemvAct &a, const GemvFuse &fz, float *y,
                             int n, int bpr, hipStream_t stream, bool persistent, int gr = 0) {
    const int items = (Q8 && !(FUSE & kFuseQuant)) ? bpr * 20 : bpr * 32;
    const int need = (items + NW * 64 - 1) / (NW * 64);
#define MGQ_XIT(X) launch_xit<R, C, NW, PF, DB, X, Q8, FUSE>(w, a, fz, y, n, bpr, stream, persistent, gr)
    if (need <= 1) return MGQ_XIT(1);
    if (need <= 2) return MGQ_XIT(2);
    if (need <= 4) return MGQ_XIT(4);
    if (need <= 8) return MGQ_XIT(8);
#undef MGQ_XIT
    return hipErrorNotSupported;
}

// Launch configurations (rows per work-group, blocks per stage, wavefronts,
// stages in flight, LDS double buffer, persistent). 1, 3, 4 and 5 are
// tuning alternatives kept for the sweep (MGQ_GEMV_CFG).
// (The fused variants instantiate only the dispatched configurations 0-3.)
template <bool Q8, int FUSE>
static hipError_t launch_any(int cfg, const uint8_t *w, const GemvAct &a, const GemvFuse &fz,
                             float *y, int n, int bpr, hipStream_t stream, int gr = 0) {
    switch (cfg) {
        // one group of gr (17..32) rows per CU: two 16-row tiles, 14 waves
        case 8: return launch_cfg<32, 14, 14, 1, false, Q8, FUSE>(w, a, fz, y, n, bpr, stream, false, gr);
        case 0: return launch_cfg<32, 8, 8, 1, false, Q8, FUSE>(w, a, fz, y, n, bpr, stream, true);
        case 1: return launch_cfg<16, 14, 7, 1, true, Q8, FUSE>(w, a, fz, y, n, bpr, stream, false);
        case 2: return launch_cfg<16, 16, 8, 1, true, Q8, FUSE>(w, a, fz, y, n, bpr, stream, false);
        case 3: return launch_cfg<16, 14, 7, 1, true, Q8, FUSE>(w, a, fz, y, n, bpr, stream, true);
        case 6: return launch_cfg<16, 14, 7, 1, false, Q8, FUSE>(w, a, fz, y, n, bpr, stream, true);
        default:
            if constexpr (FUSE == 0) {
                if (cfg == 4)
                    return launch_cfg<16, 14, 7, 2, true, Q8, 0>(w, a, fz, y, n, bpr, stream, true);
                if (cfg == 5)
                    return launch_cfg<32, 14, 7, 1, true, Q8, 0>(w, a, fz, y, n, bpr, stream, true);
            }
            return hipErrorInvalidValue;
    }
}

// the kStageWave configurations of one mode
template <bool Q8, int FUSE>
static hipError_t prepare_swave() {
    hipError_t e = lds_attr_all<16, 14, 7, 1, false, Q8, FUSE | kStageWave>();
    if (e == hipSuccess) e = lds_attr_all<16, 16, 8, 1, false, Q8, FUSE | kStageWave>();
    return e;
}

template <int FUSE>
static hipError_t prepare_fuse() {
    hipError_t e = lds_attr_all<32, 8, 8, 1, false, false, FUSE>();
    if (e == hipSuccess) e = lds_attr_all<32, 14, 14, 1, false, false, FUSE>();
    if (e == hipSuccess) e = lds_attr_all<16, 14, 7, 1, false, false, FUSE>();
    if (e == hipSuccess) e = lds_attr_all<16, 14, 7, 1, true, false, FUSE>();
    if (e == hipSuccess) e = lds_attr_all<16, 16, 8, 1, true, false, FUSE>();
    return e;
}

hipError_t gemv_prepare() {
    hipError_t e = prepare_fuse<0>();
    if (e == hipSuccess) e = lds_attr_all<32, 8, 8, 1, false, true>();
    if (e == hipSuccess) e = lds_attr_all<16, 14, 7, 1, true, true>();
    if (e == hipSuccess) e = lds_attr_all<16, 16, 8, 1, true, true>();
    if (e == hipSuccess) e = lds_attr_all<16, 14, 7, 1, false, true>();
    if (e == hipSuccess) e = lds_attr_all<32, 14, 14, 1, false, true>();
    if (e == hipSuccess) e = lds_attr_all<32, 14, 14, 1, false, true, kFuseQuant>();
    if (e == hipSuccess) e = lds_attr_all<32, 8, 8, 1, false, true, kFuseQuant>();
    if (e == hipSuccess) e = lds_attr_all<16, 14, 7, 1, true, true, kFuseQuant>();
    if (e == hipSuccess) e = lds_attr_all<16, 16, 8, 1, true, true, kFuseQuant>();
    if (e == hipSuccess) e = lds_attr_all<16, 14, 7, 1, false, true, kFuseQuant>();
    if (e == hipSuccess) e = prepare_fuse<kFmtQ5K>();
    if (e == hipSuccess) e = prepare_fuse<kFuseNorm>();
    if (e == hipSuccess) e = prepare_fuse<kFuseGlu>();
    if (e == hipSuccess) e = prepare_fuse<kFuseNorm | kFuseGlu>();
    if (e == hipSuccess) e = q6k_prepare();
    if (e == hipSuccess) e = wave_prepare<16, 14, 7>();
    if (e == hipSuccess) e = wave_prepare<16, 20, 10>();
    if (e == hipSuccess) e = allow_full_lds_by_addr((const void *)gemv_wave_kernel<16, 14, 7, 1, true>);
    if (e == hipSuccess) e = allow_full_lds_by_addr((const void *)gemv_wave_kernel<16, 14, 7, 1, true, true>);
    if (e == hipSuccess) e = allow_full_lds_by_addr((const void *)gemv_wave_kernel<32, 14, 14, 1, true, true>);
    if (e == hipSuccess) e = allow_full_lds_by_addr((const void *)gemv_wave_kernel<32, 14, 14, 1, true>);
    if (e == hipSuccess) e = prepare_swave<true, 0>();
    if (e == hipSuccess) e = prepare_swave<true, kFuseQuant>();
    if (e == hipSuccess) e = prepare_swave<false, kFmtQ5K>();
    if (e == hipSuccess) e = prepare_swave<false, kFuseNorm>();
    if (e == hipSuccess) e = prepare_swave<false, kFuseGlu>();
    if (e == hipSuccess) e = prepare_swave<false, kFuseNorm | kFuseGlu>();
    if (e == hipSuccess) e = prepare_swave<false, kFuseNorm | kI8>();
    if (e == hipSuccess) e = prepare_swave<false, kFmtQ5K | kI8>();
    if (e == hipSuccess) e = lds_attr_all<32, 14, 14, 1, false, false, kFuseNorm | kStageWave | kI8>();
    if (e == hipSuccess) e = prepare_swave<false, kFuseGlu | kI8>();
    if (e == hipSuccess) e = prepare_swave<false, kFuseNorm | kFuseGlu | kI8>();
    if (e == hipSuccess) e = batched_prepare();
    return e;
}

// work_rows: rows of work (2n for the gate/up pair) for the persistence choice
template <bool Q8, int FUSE = 0>
static hipError_t mfma_dispatch(const uint8_t *w, const GemvAct &a, float *y, int n, int bpr,
                                hipStream_t stream, const GemvFuse &fz = GemvFuse{},
                                int work_rows = 0) {
    static const int force = env_int("MGQ_GEMV_CFG", -1);  // tuning override
    int cfg, gr = 0;
    if (force >= 0) {
        cfg = force;
    } else {
        // K <= 3584: whole rows per stage (each 16-row stage is one contiguous
        // run of HBM), single-buffered so three work-groups share a CU,
        // persistent. Longer K: 16 blocks per stage, or persistent 32-row
        // groups of 8 blocks when the groups outnumber the CUs.
        const long g16 = ((work_rows > 0 ? work_rows : n) + 15) / 16, cus = device_cus();
        const bool many = g16 > cus;
        if (bpr <= 14) cfg = 6;
        else cfg = many ? 0 : 2;
        // Between one and 1.5 16-row groups per CU (qkv 4608 x 3584: 288),
        // the CUs that get a second group set the time (256 groups: 5.45 us,
        // 257: 6.21, 288: 6.73): one group of ceil(N / #CUs) rows per CU
        // instead (288: 6.30, 384: 6.78 against 6.82). From ~416 groups on
        // the second groups are spread evenly enough that it loses.
        if (bpr <= 14 && work_rows == 0 && g16 > cus && 2 * g16 <= 3 * cus) {
            gr = (int)((n + cus - 1) / cus);
            cfg = 8;
        }
    }
    hipError_t e = hipErrorNotSupported;
    if constexpr (!Q8 && FUSE == 0) {
        // Plain f32 matvecs whose work-groups stream more than one stage:
        // the wave-private kernel (no barrier between stages). Decode step,
        // alternating on one box: 1182-1183 -> 1140-1141 us (gate|up -0.8,
        // down -0.55 us per launch), and 20-block stages over 10 wavefronts
        // for the long rows: 1146 -> 1137-1138 us (down 12.3 -> 12.0 us;
        // 16 / 26 / 28 / 32 blocks: 12.3 / 12.0 / 12.45 / 12.75 us).
        // One-stage 16-row launches (o: one group per work-group) load each
        // lane's pieces straight into registers (DIRECT): o 4.47 -> 4.30 us
        // per launch in chains, decode step 1.138-1.140 -> 1.132-1.133 ms;
        // with LDS slots they measured 0.1 us slower than the staged kernel.
        // qkv's groups of ceil(N / #CUs) rows in 32-row tiles (cfg 8) load
        // directly too: 5.76 -> 5.61-5.66 us per launch, decode step 1114 ->
        // 1108 us (once the wave kernel's per-unit divisions were gone; before,
        // 5.59 -> 5.63). MGQ_GEMV_WAVE=0 turns the wave-private kernel off,
        // MGQ_GEMV_DIRECT=0 the direct loads for o, MGQ_GEMV_QKV_DIRECT=0 for
        // qkv.
        // The int8 matrix-core form (I8) on every wave launch, against the
        // f16 form, alternating on one box: decode step 1119 -> 1077 us
        // (qkv 5.81 -> 5.46, o 4.33 -> 4.20, gate|up 17.6 -> 15.8, down
        // 11.93 -> 11.77 us per launch in chains). MGQ_GEMV_I8=0 turns it off.
        static const int wave_env = env_int("MGQ_GEMV_WAVE", 1);
        static const int direct_env = env_int("MGQ_GEMV_DIRECT", 1);
        static const int qkv_direct_env = env_int("MGQ_GEMV_QKV_DIRECT", 1);
        static const bool i8 = env_int("MGQ_GEMV_I8", 1) != 0;
        const bool multi = (long)(n + 15) / 16 > 2 * device_cus();
        if (wave_env && force < 0) {
            if (cfg == 6 && multi) e = launch_wave<16, 14, 7>(w, a.x, y, n, bpr, stream, true, i8);
            else if (cfg == 2) e = launch_wave<16, 20, 10>(w, a.x, y, n, bpr, stream, false, i8);
            else if (cfg == 6 && direct_env)
                e = launch_wave_direct<16, 14, 7>(w, a.x, y, n, bpr, stream, 0, i8);
            else if (cfg == 8 && qkv_direct_env)
                e = launch_wave_direct<32, 14, 14>(w, a.x, y, n, bpr, stream, gr, i8);
        }
    }
    if constexpr (Q8 || FUSE != 0) {
        // The other modes (Q8 / dp4a, fused RMSNorm and GLU, Q5_K): the same
        // per-wavefront staging inside the staged kernel (kStageWave), at the
        // staged kernel's stage widths (14 blocks over 7 wavefronts, or 16
        // over 8 for long rows). Steps, alternating on one box:
        // decode7b_dp4a 1.206 -> 1.149-1.151 ms, decode7b_q4km 1.457 ->
        // 1.414-1.415 ms (20-block stages over 10 wavefronts: the same).
        // MGQ_GEMV_SWAVE=0 turns it off.
        static const int swave_env = env_int("MGQ_GEMV_SWAVE", 1);
        const bool multi = (long)(n + 15) / 16 > 2 * device_cus();
        if constexpr (!Q8) {
            // the fused Q4_K and the Q5_K modes in the int8 form (MGQ_GEMV_I8=0: f16)
            static const bool i8f = env_int("MGQ_GEMV_I8", 1) != 0;
            if (swave_env && i8f && force < 0 && e == hipErrorNotSupported) {
                if (cfg == 6 && multi)
                    e = launch_cfg<16, 14, 7, 1, false, Q8, FUSE | kStageWave | kI8>(w, a, fz, y, n, bpr, stream, true);
                else if (cfg == 2)
                    e = launch_cfg<16, 16, 8, 1, false, Q8, FUSE | kStageWave | kI8>(w, a, fz, y, n, bpr, stream, false);
                else if constexpr (FUSE == kFuseNorm) {
                    // qkv with its RMSNorm: one group of gr rows per CU, 32-row tiles
                    if (cfg == 8)
                        e = launch_cfg<32, 14, 14, 1, false, Q8, FUSE | kStageWave | kI8>(w, a, fz, y, n, bpr,
                                                                                          stream, false, gr);
                }
            }
        }
        if (swave_env && force < 0 && e == hipErrorNotSupported) {
            if (cfg == 6 && multi)
                e = launch_cfg<16, 14, 7, 1, false, Q8, FUSE | kStageWave>(w, a, fz, y, n, bpr, stream, true);
            else if (cfg == 2)
                e = launch_cfg<16, 16, 8, 1, false, Q8, FUSE | kStageWave>(w, a, fz, y, n, bpr, stream, false);
        }
    }
    if (e == hipErrorNotSupported) e = launch_any<Q8, FUSE>(cfg, w, a, fz, y, n, bpr, stream, gr);
    // LDS too small for the double-buffered stages (Q5_K's 176-byte blocks on
    // down): single-buffered 16-row stages (26.2 -> 17.9 us on Q5_K
    // 3584x18944), then persistent 32-row groups
    if (e == hipErrorNotSupported && cfg != 6 && cfg != 0)
        e = launch_any<Q8, FUSE>(6, w, a, fz, y, n, bpr, stream);
    if (e == hipErrorNotSupported && cfg != 0) e = launch_any<Q8, FUSE>(0, w, a, fz, y, n, bpr, stream);
    return e;
}

hipError_t gemv_fused_launch(const uint8_t *w_gate, const uint8_t *w_up, const float *x,
                             const float *norm_w, float eps, int act, float *y, int n, int bpr,
                             hipStream_t stream) {
    const GemvAct a{x, nullptr, nullptr, nullptr};
    const GemvFuse fz{w_up, norm_w, eps, act};
    if (w_up == nullptr) {
        if (norm_w == nullptr) return mfma_dispatch<false, 0>(w_gate, a, y, n, bpr, stream, fz);
        return mfma_dispatch<false, kFuseNorm>(w_gate, a, y, n, bpr, stream, fz);
    }
    if (norm_w == nullptr)
        return mfma_dispatch<false, kFuseGlu>(w_gate, a, y, n, bpr, stream, fz, 2 * n);
    return mfma_dispatch<false, kFuseNorm | kFuseGlu>(w_gate, a, y, n, bpr, stream, fz, 2 * n);
}

hipError_t gemv_mfma_launch(const uint8_t *w, const float *x, float *y, int n, int bpr,
                            hipStream_t stream) {
    return mfma_dispatch<false>(w, GemvAct{x, nullptr, nullptr, nullptr}, y, n, bpr, stream);
}

hipError_t gemv_q5k_mfma_launch(const uint8_t *w, const float *x, float *y, int n, int bpr,
                                hipStream_t stream) {
    return mfma_dispatch<false, kFmtQ5K>(w, GemvAct{x, nullptr, nullptr, nullptr}, y, n, bpr, stream);
}

hipError_t gemv_q8x_launch(const uint8_t *w, const float *x, float *y, int n, int bpr,
                           hipStream_t stream) {
    return mfma_dispatch<true, kFuseQuant>(w, GemvAct{x, nullptr, nullptr, nullptr}, y, n, bpr,
                                           stream);
}

hipError_t gemv_q8_launch(const uint8_t *w, const int8_t *xq, const float *xd, const float *xsum,
                          float *y, int n, int bpr, hipStream_t stream) {
    const hipError_t e = mfma_dispatch<true>(w, GemvAct{nullptr, xq, xd, xsum}, y, n, bpr, stream);
    if (e != hipErrorNotSupported) return e;
    return gemv_q8_generic_launch(w, xq, xd, xsum, y, n, bpr, stream);
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
