// Prefill dequant-GEMM on the gfx950 matrix cores:
//   C[m][r] = sum_k dequant(W)[r][k] * A[m][k],  A f16 [M][K], C f32 [M][N].
// No counterpart in the reference (its prefill is a per-token GEMV loop,
// crates/modgrad-gemma/examples/gemma4_rocm.rs:26-34); each weight is the
// canonical dequantized value (gguf.rs:364-404) times a per-row power of two
// 2^e that keeps every |weight| of the row below 2^15, so f16 neither
// overflows nor goes subnormal (gemm_q4k_f16_kernel: row_range_exp over all
// of the row's blocks; gemm_q4k_f16_lds_kernel: a running exponent, see
// there), with d*sc*2^e and dmin*m*2^e rounded to f16 and the weight
// computed and rounded in f16; C is scaled back by 2^-e exactly.
// (gemm_q4k_f16_lds_kernel applies one more fixed power of two, 2^-20, to
// the weights and takes it back in C.)
//
// Two kernels: gemm_q4k_f16_lds_kernel (below), which dequantizes each W
// element once per work-group into an f16 LDS tile, where its 160 x 256
// tiles fill their rounds (config 5: M = 512, N = 18944; M = 1024);
// otherwise gemm_q4k_f16_kernel, whose 128-token tiles keep every CU busy.
//
// gemm_q4k_f16_kernel -- work-group tile: BN W rows x 128 tokens (BN = 128 or 160, whichever gives
// the busiest CU fewer rows to compute), 4 wavefronts of BN/2 x 64 outputs (BN/32 x 4
// v_mfma_f32_16x16x32_f16, W rows as the A operand, tokens as the B operand,
// so a lane's 4 accumulators are 4 consecutive W rows of one token: one
// 16-byte store into C's [M][N]).
//
// Memory path. Global loads are whole cache lines: the W tile of a
// super-block (BN rows x 144 B) is copied raw into LDS as 9*BN contiguous
// 16-byte pieces (a wavefront's 64 pieces cover ~7 rows), once per 8 MFMA
// k-steps; the activation tile of a 64-wide K step is 128 tokens x 128 B,
// 8 lanes per token. Loads for the next super-block / K step are in flight
// while the current one is computed.
//
// Dequantization happens where the MFMA operand is built, straight from the
// raw bytes in LDS: a lane's 8 qs bytes B0..B7 give the operand of the low
// nibbles (sub-block 2G) and of the high nibbles (2G+1). (w & 0x000F000F) |
// 0x64006400 puts the low nibbles of bytes 0 and 2 into the mantissas of two
// f16 1024.0s (exact), (w >> 8) does the same for bytes 1 and 3, and a mask of
// 0x00F000F0 yields 1024 + 16*q for the high nibbles (scaled back by using
// d*sc/16). v_pk_add_f16(-1024) and v_pk_fma_f16(d*sc, -dmin*m) finish two
// weights per instruction. The operand's k order is therefore
// 0,2,1,3,4,6,5,7 within each group of 8; the activation tile is stored in
// the same order (two v_perm_b32 per 8 values), so every product pairs a
// weight with its own activation. Per-row (d*sc, -dmin*m) pairs of the 8
// sub-blocks are decoded once per super-block by the lane that loaded the
// row's header piece.
#include "q4k_device.hpp"
#include "q4k_launch.hpp"

#include <atomic>
#include <cstdlib>

namespace mgq {

namespace gemm {
constexpr int BM = 128;        // tokens per work-group
constexpr int BK = 64;         // k per step (one 32-byte qs group: 2 sub-blocks)
// halves per activation LDS row: 64 + 16 pad (160 B). At this pitch the 16
// lanes of a b128 operand read hit distinct banks (measured: 4 cycles per
// read against 8 at a 72-half pitch, and ~60 when rows are not 16-byte
// aligned).
constexpr int AROW = 80;
constexpr int SROW = 10;       // dwords per scale row (8 + 2 pad: conflict-free b64 reads)
constexpr int NXCD = 8;        // XCDs the hardware deals work-groups across, round robin
}  // namespace gemm

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

// (v & mask) | magic in one instruction. gfx9 VOP3 encodings take no literal
// constants, so the compiler would otherwise emit a v_and/v_or pair.
__device__ __forceinline__ uint32_t and_or(uint32_t v, uint32_t mask, uint32_t magic) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "s"(mask), "v"(magic));
    return r;
}

// Two f16 weights (bytes 0 and 2 of v, nibble selected by mask) as a pair:
// (q * d1 + nm1) with q recovered exactly from the 1024.0 mantissa.
__device__ __forceinline__ uint32_t dq2(uint32_t v, uint32_t mask, uint32_t magic, h2_t d1,
                                        h2_t nm1) {
    const h2_t k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
    const h2_t q = __builtin_bit_cast(h2_t, and_or(v, mask, magic)) - k1024;
    return __builtin_bit_cast(uint32_t, q * d1 + nm1);
}

// Two f16 weights (bytes 0 and 2 of v, nibble selected by mask) as a pair:
// the masked nibble is the f16 subnormal q * 2^-24 (or 16q * 2^-24), exact,
// and one fused multiply-add with d1 = D (the multiplier times 2^24) gives
// q * d1 * 2^-24 + nm1 rounded once.
__device__ __forceinline__ uint32_t dqs2(uint32_t v, uint32_t mask, h2_t d1, h2_t nm1) {
    const h2_t q = __builtin_bit_cast(h2_t, v & mask);
    return __builtin_bit_cast(uint32_t, q * d1 + nm1);
}

// MFMA A operand of 8 weights from qs bytes B0..B7 (dwords w0, w1; s0, s1 =
// w0 >> 8, w1 >> 8), k order 0,2,1,3,4,6,5,7; sp = (d1, nm1) of the
// sub-block as an f16 pair. magic holds 0x64006400.
__device__ __forceinline__ half8 dq8(uint32_t w0, uint32_t w1, uint32_t s0, uint32_t s1,
                                     uint32_t mask, uint32_t magic, uint32_t sp) {
    const h2_t s = __builtin_bit_cast(h2_t, sp);
    const h2_t d1 = {s[0], s[0]}, nm1 = {s[1], s[1]};
    u32x4 r;
    r[0] = dq2(w0, mask, magic, d1, nm1);
    r[1] = dq2(s0, mask, magic, d1, nm1);
    r[2] = dq2(w1, mask, magic, d1, nm1);
    r[3] = dq2(s1, mask, magic, d1, nm1);
    return __builtin_bit_cast(half8, r);
}

// 8 consecutive f16 activations x0..x7 -> order x0,x2,x1,x3,x4,x6,x5,x7.
__device__ __forceinline__ u32x4 act_order(u32x4 v) {
    u32x4 r;
    r[0] = __builtin_amdgcn_perm(v[1], v[0], 0x05040100u);
    r[1] = __builtin_amdgcn_perm(v[1], v[0], 0x07060302u);
    r[2] = __builtin_amdgcn_perm(v[3], v[2], 0x05040100u);
    r[3] = __builtin_amdgcn_perm(v[3], v[2], 0x07060302u);
    return r;
}

// Power-of-two range scale of one W row: e such that every dequantized
// |weight| of the row times 2^e is below 2^15 (|q*d*sc - dmin*m| <=
// 945*|d| + 63*|dmin|), so the f16 weights neither overflow nor fall into
// f16 subnormals when d is small. The caller's threads split the blocks:
// this one reads blocks j0, j0 + step, ..., eight header loads in flight.
__device__ __forceinline__ float row_range_bound(const uint8_t *row, int j0, int step, int bpr) {
    float bound = 0.0f;
    for (int j = j0; j < bpr; j += 8 * step) {
        uint32_t hv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
            hv[i] = ld_u32(row + (size_t)min(j + step * i, bpr - 1) * kBlockBytes);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float d = half_bits_finite(hv[i]), dm = half_bits_finite(hv[i] >> 16);
            bound = fmaxf(bound, fabsf(d) * 945.0f + fabsf(dm) * 63.0f);
        }
    }
    return bound;
}

__device__ __forceinline__ int range_exp(float bound) {
    int e = 0;
    if (bound > 0.0f && bound <= 3.402823466e38f) {
        int ex;
        frexpf(bound, &ex);  // bound in [2^(ex-1), 2^ex)
        e = min(max(15 - ex, -120), 120);
    }
    return e;
}

__device__ __forceinline__ int row_range_exp(const uint8_t *row, int j0, int step, int bpr) {
    return range_exp(row_range_bound(row, j0, step, bpr));
}

// BN = W rows per work-group (128 or 160): two wavefronts along N of BN/2
// rows = TI 16-row MFMA tiles each.
template <int BN>
__global__ __launch_bounds__(256, 2) void gemm_q4k_f16_kernel(const uint8_t *__restrict__ w,
                                                           const uint16_t *__restrict__ a,
                                                           float *__restrict__ c, int n, int bpr,
                                                           int m_tokens, int tiles_n, int tiles_m) {
    using namespace gemm;
    constexpr int TI = BN / 32;                            // 16-row tiles per wavefront
    constexpr int RAW_PIECES = BN * kBlockBytes / 16;      // 16-byte pieces per super-block
    constexpr int NPL = (RAW_PIECES + 255) / 256;          // raw loads per thread
    __shared__ __attribute__((aligned(16))) uint8_t sRaw[BN * kBlockBytes];
    __shared__ __attribute__((aligned(16))) uint32_t sScl[BN * SROW];
    __shared__ __attribute__((aligned(16))) _Float16 sA[2][BM * AROW];      // 36864 B
    __shared__ __attribute__((aligned(16))) float sInv[BN];                  // 2^-e per row

    // work-group -> tile: the hardware sends work-group i to XCD i % 8; give
    // XCD x a contiguous range of tiles (token tiles of a W tile adjacent)
    const int ntiles = tiles_n * tiles_m;
    const int per_xcd = (ntiles + NXCD - 1) / NXCD;
    const int tile = (int)(blockIdx.x % NXCD) * per_xcd + (int)(blockIdx.x / NXCD);
    if (tile >= ntiles) return;  // uniform; only when ntiles % 8 != 0
    const int n0 = (tile / tiles_m) * BN, m0 = (tile % tiles_m) * BM;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int K = bpr * kBlockElems;
    const int T = bpr * 4;  // K steps
    const size_t row_bytes = (size_t)bpr * kBlockBytes;

    // raw W loader: piece p = tid + 256*k (k < NPL - 1, and the last k for
    // tid < RAW_PIECES - 256 (NPL - 1)) is bytes 16*(p%9) .. +15 of row p/9's
    // super-block
    const uint8_t *rsrc[NPL];
#pragma unroll
    for (int k = 0; k < NPL; ++k) {
        const int p = min(tid + 256 * k, RAW_PIECES - 1);
        rsrc[k] = w + (size_t)min(n0 + p / 9, n - 1) * row_bytes + 16 * (p % 9);
    }
    const bool haslast = tid < RAW_PIECES - 256 * (NPL - 1);
    // the lane holding a row's header piece decodes that row's scales
    int hk = -1, hrow = 0;
#pragma unroll
    for (int k = 0; k < NPL; ++k) {
        const int p = tid + 256 * k;
        if (p < RAW_PIECES && p % 9 == 0) {
            hk = k;
            hrow = p / 9;
        }
    }
    // ... and the row's power-of-two range scale (row_range_scale), from all
    // of its block headers; C is scaled back by the inverse in the epilogue
    float srow = 1.0f;
    if (hk >= 0) {
        const int e = row_range_exp(w + (size_t)min(n0 + hrow, n - 1) * row_bytes, 0, 1, bpr);
        srow = ldexpf(1.0f, e);
        sInv[hrow] = ldexpf(1.0f, -e);
    }
    u32x4 R[NPL];
    auto rload = [&](int b) __attribute__((always_inline)) {  // piece 4 is loaded by every lane (clamped address): no branch
#pragma unroll
        for (int k = 0; k < NPL; ++k)
            R[k] = ld_u32x4(rsrc[k] + (size_t)b * kBlockBytes);
    };
    auto rstore = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < NPL - 1; ++k) *reinterpret_cast<u32x4 *>(&sRaw[16 * (tid + 256 * k)]) = R[k];
        if (haslast) *reinterpret_cast<u32x4 *>(&sRaw[16 * (tid + 256 * (NPL - 1))]) = R[NPL - 1];
        if (hk >= 0) {
            // this lane stored the row's header piece just above; reading it
            // back from LDS avoids indexing R with the runtime hk
            const u32x4 h = *reinterpret_cast<const u32x4 *>(&sRaw[16 * 9 * hrow]);
            const float d = half_bits_finite(h[0]), dmin = half_bits_finite(h[0] >> 16);
            uint32_t pr[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                uint32_t sc, m;
                scale_min(j, h[1], h[2], h[3], sc, m);
                // high nibbles arrive as 16*q
                const _Float16 d1 = (_Float16)(d * (float)sc * srow * ((j & 1) ? 0.0625f : 1.0f));
                const _Float16 nm1 = (_Float16)(-(dmin * (float)m * srow));
                pr[j] = __builtin_bit_cast(uint32_t, (h2_t){d1, nm1});
            }
            u32x2 *dst = reinterpret_cast<u32x2 *>(&sScl[hrow * SROW]);
#pragma unroll
            for (int j = 0; j < 4; ++j) dst[j] = (u32x2){pr[2 * j], pr[2 * j + 1]};
        }
    };

    // activation loader: 8 lanes per token (128 B), tokens tid/8 + 32*k
    const int ap = tid & 7;
    const uint16_t *asrc[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
        asrc[k] = a + (size_t)min(m0 + (tid >> 3) + 32 * k, m_tokens - 1) * K + 8 * ap;
    u32x4 Areg[2][4];  // two register sets: step t+2's loads fly while t+1's are stored
    auto aload = [&](int t, int set) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < 4; ++k)
            Areg[set][k] = ld_u32x4(asrc[k] + (size_t)t * BK);
    };
    auto astore = [&](int set, int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < 4; ++k)
            *reinterpret_cast<u32x4 *>(&sA[buf][((tid >> 3) + 32 * k) * AROW + 8 * ap]) =
                act_order(Areg[set][k]);
    };

    // compute roles
    const int wn = (wave >> 1) * (BN / 2), wm = (wave & 1) * 64;  // wave's W-row / token offsets
    const int l16 = lane & 15, q = lane >> 4;
    f32x4 acc[TI][4];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) acc[i][jj] = f32x4{0.f, 0.f, 0.f, 0.f};

    // magic 0x64006400 in a VGPR (the VOP3 constant bus takes one SGPR: the mask)
    const uint32_t magic = __builtin_amdgcn_readfirstlane(0x64006400u) + (uint32_t)(tid >> 16);
    auto compute = [&](int G, int buf) __attribute__((always_inline)) {
        half8 wlo[TI], whi[TI];
#pragma unroll
        for (int i = 0; i < TI; ++i) {
            const int row = wn + 16 * i + l16;
            const u32x2 wq = *reinterpret_cast<const u32x2 *>(&sRaw[row * kBlockBytes + 16 + 32 * G + 8 * q]);
            const u32x2 sp = *reinterpret_cast<const u32x2 *>(&sScl[row * SROW + 2 * G]);
            const uint32_t s0 = wq[0] >> 8, s1 = wq[1] >> 8;
            wlo[i] = dq8(wq[0], wq[1], s0, s1, 0x000F000Fu, magic, sp[0]);
            whi[i] = dq8(wq[0], wq[1], s0, s1, 0x00F000F0u, magic, sp[1]);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            half8 tb[4];
#pragma unroll
            for (int jj = 0; jj < 4; ++jj)
                tb[jj] = *reinterpret_cast<const half8 *>(
                    &sA[buf][(wm + 16 * jj + l16) * AROW + 32 * h + 8 * q]);
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int jj = 0; jj < 4; ++jj)
                    acc[i][jj] = __builtin_amdgcn_mfma_f32_16x16x32_f16(h ? whi[i] : wlo[i], tb[jj],
                                                                        acc[i][jj], 0, 0, 0);
        }
    };

    // K step t = 4b + G computes activation buffer t&1 against super-block b
    // in sRaw; it stores step t+1's activations (register set (t+1)&1) into
    // the other buffer and refills that set with step t+3. After a
    // super-block's last step and a barrier, the next super-block's raw
    // bytes (loaded during this one) replace it. Every load is issued
    // unconditionally (indices clamped to the last step / super-block), so
    // the hardware load counter waits only for the data each store needs.
    rload(0);
    aload(0, 0);
    aload(min(1, T - 1), 1);
    rstore();
    astore(0, 0);
    rload(min(1, bpr - 1));
    aload(min(2, T - 1), 0);
    __syncthreads();
    for (int b = 0; b < bpr; ++b) {
#pragma unroll
        for (int G = 0; G < 4; ++G) {
            const int t = 4 * b + G;
            compute(G, G & 1);
            astore((G + 1) & 1, (G + 1) & 1);  // after the last step: an unused buffer
            aload(min(t + 3, T - 1), (G + 1) & 1);
            if (G == 3) {
                __syncthreads();  // every wavefront is done with super-block b
                rstore();         // after the last super-block: rewrites unused data
                rload(min(b + 2, bpr - 1));
            }
            __syncthreads();
        }
    }

    // lane holds W rows wn+16i+4q+v (v=0..3) of token wm+16jj+l16
    const bool vec = (n % 4) == 0 && (((uintptr_t)c & 15u) == 0);
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
        const int m = m0 + wm + 16 * jj + l16;
        if (m >= m_tokens) continue;
#pragma unroll
        for (int i = 0; i < TI; ++i) {
            const int r = n0 + wn + 16 * i + 4 * q;
            const f32x4 v4 = acc[i][jj] * *reinterpret_cast<const f32x4 *>(&sInv[wn + 16 * i + 4 * q]);
            float *dst = c + (size_t)m * n + r;
            if (vec && r + 3 < n) {
                *reinterpret_cast<f32x4 *>(dst) = v4;
            } else {
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    if (r + v < n) dst[v] = v4[v];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Large-M prefill GEMM: the work-group dequantizes its W slice ONCE per K
// step into an f16 LDS tile and runs a plain f16 matrix-core GEMM on it.
//
// Work-group tile: 160 W rows x 256 tokens, 8 wavefronts as 2 (W rows) x 4
// (tokens), each 80 rows x 64 tokens = 5 x 4 v_mfma_f32_16x16x32_f16 tiles
// (W rows the A operand, tokens the B operand, so a lane's 4 accumulators
// are 4 consecutive W rows of one token: one 16-byte store into C [M][N]).
// One work-group per CU (134 KiB of LDS); at M = 512 and N = 18944 the 238
// tiles are one round on the 256 CUs.
//
// K step = 64 (one 32-byte qs group: sub-blocks 2G and 2G+1 of a
// super-block). Per step the work-group loads 160 x 2 16-byte qs pieces and
// 256 tokens x 128 B of activations into registers (weights two steps
// before their store, activations one); they are written to a double-
// buffered LDS stage (activations as they are, weights dequantized to f16
// in natural k order). The 320 pieces are exactly five wavefronts of one
// piece per lane, so the first five wavefronts dequantize and no LDS store
// repeats another (a store instruction costs the same whatever its active
// lanes); all eight copy activations and compute. The barrier of each step
// sits between its two k halves (see the pipeline below), and
// sched_group_barrier interleaves each half's MFMAs with its LDS operand
// reads, stores and loads.
//
// Range. Each W row carries a running power-of-two exponent e. Any e at or
// below tight = range_exp(running max of 945|d| + 63|dmin| over the row's
// blocks so far) keeps every |weight| * 2^e below 2^15. A row starts at
// tight - kRangeHeadroom of its first nonzero block and keeps e while the
// later blocks' tight stays at or above it; a block that overruns it (more
// than 2^kRangeHeadroom above the first block's bound) lowers e to its
// tight - kRangeHeadroom. The nibble is masked in place as the f16
// subnormal q * 2^-24 (or 16q * 2^-24 for the high nibble), exact, and one
// v_pk_fma_f16 with the sub-block pair (d*sc*2^(e+4), -dmin*m*2^(e-20))
// gives (q*d*sc - dmin*m) * 2^(e-20), rounded once; |d*sc| * 2^(e+4) <
// 2^15 * 63*16/945 stays below the f16 maximum, and weights above
// 2^-(9 - kRangeHeadroom) of the largest seen so far stay normal f16. When
// a block changes some row's e (a flag in LDS says so), the work-group's
// sums so far are multiplied by 2^(e_new - e_old) per row (exact, a power
// of two) between the two blocks' MFMAs; C is multiplied by 2^(20-e) of
// the last block at the end. No pass over the row's headers precedes the
// first MFMA.
constexpr int kRangeHeadroom = 4;
struct G2Cfg {
    static constexpr int WN = 2, WM = 4, TI = 5, TJ = 4;
    static constexpr int BN = WN * 16 * TI;       // 160 W rows per work-group
    static constexpr int BM = WM * 16 * TJ;       // 256 tokens per work-group
    static constexpr int NT = 64 * WN * WM;       // 512 threads
    static constexpr int KS = 64;                 // k per step
    static constexpr int PITCH = 80;              // halves per LDS row (64 + pad)
    static constexpr int WP = BN * 2;             // 16-byte qs pieces per step
    static constexpr int WWAVES = WP / 64;        // wavefronts that dequantize W (5)
    static constexpr int APT = BM * 8 / NT;       // activation pieces per thread per step
    static constexpr uint32_t SW = BN * PITCH * 2, SA = BM * PITCH * 2;
    static constexpr uint32_t LDS = 2 * SW + 2 * SA + 2 * BN * 4 + 16;
    static_assert(PITCH % 8 == 0, "16-byte aligned LDS rows (b128 accesses)");
    static_assert(WP % 64 == 0 && WWAVES <= NT / 64, "whole wavefronts of W pieces");
    static_assert(BM * 8 % NT == 0, "whole activation pieces per thread");
};

__global__ __launch_bounds__(G2Cfg::NT, 1) void gemm_q4k_f16_lds_kernel(
    const uint8_t *__restrict__ w, const uint16_t *__restrict__ a, float *__restrict__ c, int n,
    int bpr, int m_tokens, int tiles_n, int tiles_m) {
    using Cfg = G2Cfg;
    constexpr int WN = Cfg::WN, TI = Cfg::TI, TJ = Cfg::TJ, BN = Cfg::BN, BM = Cfg::BM;
    constexpr int KS = Cfg::KS, PITCH = Cfg::PITCH, APT = Cfg::APT;
    constexpr uint32_t SW = Cfg::SW, SA = Cfg::SA;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    _Float16 *sW = reinterpret_cast<_Float16 *>(lds);
    _Float16 *sA = reinterpret_cast<_Float16 *>(lds + 2 * SW);
    float *sE = reinterpret_cast<float *>(lds + 2 * SW + 2 * SA);  // per row: 2^(20-e), C's scale
    float *sF = sE + BN;  // per row: 2^(e_new - e_old) of the block being opened
    int *sFlag = reinterpret_cast<int *>(sF + BN);  // [1]: some row's e changed; [0]: dummy

    // work-group -> tile: work-group i runs on XCD i % 8; XCD x takes a
    // contiguous range of tiles, so the token tiles of one W tile share an L2
    const int ntiles = tiles_n * tiles_m;
    const int per_xcd = (ntiles + gemm::NXCD - 1) / gemm::NXCD;
    const int tile = (int)(blockIdx.x % gemm::NXCD) * per_xcd + (int)(blockIdx.x / gemm::NXCD);
    if (tile >= ntiles) return;  // uniform
    const int n0 = (tile / tiles_m) * BN, m0 = (tile % tiles_m) * BM;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int K = bpr * kBlockElems;
    const int T = bpr * 4;  // K steps
    const size_t row_bytes = (size_t)bpr * kBlockBytes;

    // W dequantization: the first WWAVES wavefronts, one qs piece per lane
    // (an LDS store instruction costs the same whatever its active lanes, so
    // whole wavefronts take the 320 pieces of a step). Piece p: W row
    // wr = p % BN (clamped past n), bytes 16*wh.. (wh = p / BN) of each
    // step's 32-byte qs group; the 8 lanes of an LDS store group write 8
    // consecutive rows (distinct banks at an 80-half pitch)
    const bool isW = __builtin_amdgcn_readfirstlane(wave) < Cfg::WWAVES;
    const int p = (isW ? wave : 0) * 64 + lane;
    const int wr = p % BN, wh = p / BN;
    // Global loads are raw buffer loads: a 32-bit per-lane byte offset plus
    // a per-step scalar offset (the launcher keeps W and A below 2^32 bytes),
    // so no per-load address arithmetic. Offsets: the lane's row header and
    // its qs piece.
    const __amdgpu_buffer_rsrc_t wbuf = __builtin_amdgcn_make_buffer_rsrc(
        (void *)w, 0, (int)(uint32_t)((uint64_t)n * row_bytes), kRawBufWord3);
    const __amdgpu_buffer_rsrc_t abuf = __builtin_amdgcn_make_buffer_rsrc(
        (void *)a, 0, (int)(uint32_t)((uint64_t)m_tokens * K * 2), kRawBufWord3);
    const uint32_t hoff = (uint32_t)((size_t)min(n0 + wr, n - 1) * row_bytes);

    // ---- step loaders (registers) ------------------------------------------
    // activation piece k of this thread: token tid/8 + 64k of the tile, 16
    // bytes at 8*(tid%8) of the step's 64 values. The per-lane offset stays
    // below 2^32 (the launcher checks (m_tokens + BM) * K * 2), and token
    // rows past m_tokens fall past num_records, so they read as zeros; the
    // per-step scalar offset stays inside a token row.
    const uint32_t aoff0 = (uint32_t)(((size_t)(m0 + (tid >> 3)) * K + 8 * (tid & 7)) * 2);
    const uint32_t astride = (uint32_t)(Cfg::NT / 8) * (uint32_t)K * 2;
    const uint32_t alds0 = (uint32_t)(((tid >> 3) * PITCH + 8 * (tid & 7)) * 2);
    u32x4 Ar[APT], Wq[2], Hd;
    auto loadA_to = [&](u32x4(&dst)[APT], int t) __attribute__((always_inline)) {
        const int so = min(t, T - 1) * KS * 2;
#pragma unroll
        for (int k = 0; k < APT; ++k)
            dst[k] = __builtin_amdgcn_raw_buffer_load_b128(abuf, aoff0 + k * astride, so, 0);
    };
    auto loadA = [&](int t) __attribute__((always_inline)) { loadA_to(Ar, t); };
    auto loadW = [&](int t, int set) __attribute__((always_inline)) {
        t = min(t, T - 1);
        Wq[set] = __builtin_amdgcn_raw_buffer_load_b128(wbuf, hoff + 16 * wh, (t >> 2) * kBlockBytes + 32 * (t & 3) + 16, 0);
    };
    // header of the super-block that step t opens (once per 4 steps)
    auto loadH = [&](int t) __attribute__((always_inline)) {
        Hd = __builtin_amdgcn_raw_buffer_load_b128(wbuf, hoff, (min(t, T - 1) >> 2) * kBlockBytes, 0);
    };

    // step t -> LDS buffer: activations copied, weights dequantized
    auto storeA = [&](int buf) __attribute__((always_inline)) {
        uint8_t *dA = lds + 2 * SW + buf * SA + alds0;
#pragma unroll
        for (int k = 0; k < APT; ++k)
            *reinterpret_cast<u32x4 *>(dA + k * (Cfg::NT / 8) * PITCH * 2) = Ar[k];
    };
    // the block's 8 sub-block pairs (d*sc*2^(e+4), -dmin*m*2^(e-20)) as f16,
    // decoded once per super-block from its header (sub-block index
    // constant: no branches); d*sc and dmin*m are exact in f32 and the
    // factors are powers of two, so each is rounded to f16 once. The row's
    // exponent follows the running bound; every piece lane of the row
    // publishes the same rescale of the sums so far and C's scale (no
    // branch), and a lane whose row changed e sets the flag (the others
    // write the dummy slot).
    float bnd = 0.0f;  // max of 945|d| + 63|dmin| over the row's blocks so far
    int erow = 0;
    uint32_t scl[8];
    auto decode = [&]() __attribute__((always_inline)) {
        const float dh = half_bits_finite(Hd[0]), mh = half_bits_finite(Hd[0] >> 16);
        const bool fresh = bnd == 0.0f;  // no nonzero block before this one
        bnd = fmaxf(bnd, fabsf(dh) * 945.0f + fabsf(mh) * 63.0f);
        const int tight = range_exp(bnd);
        const int e = (fresh || tight < erow) ? tight - kRangeHeadroom : erow;
        float *se = sE + wr;  // sF[wr] = se[BN]: one address for both
        se[BN] = ldexpf(1.0f, e - erow);
        se[0] = ldexpf(1.0f, 20 - e);
        sFlag[e != erow ? 1 : 0] = 1;
        erow = e;
        const float d = dh * ldexpf(1.0f, e + 4);
        const float nm = -(mh * ldexpf(1.0f, e - 20));
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint32_t sc, mn;
            scale_min(j, Hd[1], Hd[2], Hd[3], sc, mn);
            const _Float16 d1 = (_Float16)(d * (float)sc * ((j & 1) ? 0.0625f : 1.0f));  // high nibbles arrive as 16*q
            const _Float16 n1 = (_Float16)(nm * (float)mn);
            scl[j] = __builtin_bit_cast(uint32_t, (h2_t){d1, n1});
        }
    };
    auto storeW = [&](auto gc, int set, int buf) __attribute__((always_inline)) {
        constexpr int G = decltype(gc)::value;  // qs group of the step: sub-blocks 2G, 2G+1
        const h2_t sl = __builtin_bit_cast(h2_t, scl[2 * G]);
        const h2_t sh = __builtin_bit_cast(h2_t, scl[2 * G + 1]);
        const h2_t dl2 = {sl[0], sl[0]}, nl2 = {sl[1], sl[1]}, dh2 = {sh[0], sh[0]}, nh2 = {sh[1], sh[1]};
        u32x4 lo[2], hi[2];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t v = Wq[set][u];
            const uint32_t p0 = __builtin_amdgcn_perm(v, v, 0x0C010C00u);  // bytes 0, 1 -> 0, 2
            const uint32_t p1 = __builtin_amdgcn_perm(v, v, 0x0C030C02u);  // bytes 2, 3 -> 0, 2
            lo[u >> 1][2 * (u & 1)] = dqs2(p0, 0x000F000Fu, dl2, nl2);
            lo[u >> 1][2 * (u & 1) + 1] = dqs2(p1, 0x000F000Fu, dl2, nl2);
            hi[u >> 1][2 * (u & 1)] = dqs2(p0, 0x00F000F0u, dh2, nh2);
            hi[u >> 1][2 * (u & 1) + 1] = dqs2(p1, 0x00F000F0u, dh2, nh2);
        }
        // low nibbles: k = 16*wh + 0..15 of the step; high nibbles: 32 + that
        uint8_t *dW = lds + buf * SW + (size_t)(wr * PITCH + 16 * wh) * 2;
        *reinterpret_cast<u32x4 *>(dW) = lo[0];
        *reinterpret_cast<u32x4 *>(dW + 16) = lo[1];
        *reinterpret_cast<u32x4 *>(dW + 64) = hi[0];
        *reinterpret_cast<u32x4 *>(dW + 80) = hi[1];
    };

    // ---- compute roles -----------------------------------------------------
    const int wn = (wave % WN) * (16 * TI), wm = (wave / WN) * (16 * TJ);
    const int l16 = lane & 15, q = lane >> 4;
    f32x4 acc[TI][TJ];
    // Operand registers: the token operands of both k halves (32 of the
    // step's 64 k each), and one set of W operands: wa[i] is reread for the
    // next half right after the four MFMAs that use it, so a half's MFMAs run
    // while the next half's operands arrive without holding two W sets.
    half8 wa[TI], tb[2][TJ];
    auto readA = [&](int buf, auto hc) __attribute__((always_inline)) {
        constexpr int h = decltype(hc)::value;
        const _Float16 *A_ = sA + buf * (BM * PITCH);
#pragma unroll
        for (int j = 0; j < TJ; ++j)
            tb[h][j] = *reinterpret_cast<const half8 *>(&A_[(wm + 16 * j + l16) * PITCH + 32 * h + 8 * q]);
    };
    auto readW = [&](int buf, auto hc, int i) __attribute__((always_inline)) {
        constexpr int h = decltype(hc)::value;
        const _Float16 *W_ = sW + buf * (BN * PITCH);
        wa[i] = *reinterpret_cast<const half8 *>(&W_[(wn + 16 * i + l16) * PITCH + 32 * h + 8 * q]);
    };
    // MFMAs of half hc; the token operands of half rc from buffer rbuf first,
    // then the W operands of that half, each after its last use here
    auto halfStep = [&](auto hc, int rbuf, auto rc) __attribute__((always_inline)) {
        constexpr int h = decltype(hc)::value;
        readA(rbuf, rc);
#pragma unroll
        for (int i = 0; i < TI; ++i) {
#pragma unroll
            for (int j = 0; j < TJ; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa[i], tb[h][j], acc[i][j], 0, 0, 0);
            readW(rbuf, rc, i);
        }
    };
    using H0 = std::integral_constant<int, 0>;
    using H1 = std::integral_constant<int, 1>;

    // ---- pipeline ----------------------------------------------------------
    // Weights are loaded two steps before their dequantized store (two
    // register sets), activations one step before theirs. The header of the
    // block that step t+4 opens is loaded at t = 0 mod 4 and decoded at
    // t = 2 mod 4, just before that block's first store. Loads past the last
    // step re-read it (clamped), so every load is unconditional and the load
    // counter waits only for the data it needs.
    // prologue: steps 0 and 1 of both operands in flight at once (the
    // accumulators are not live yet)
    u32x4 A1[APT];
    loadA(0);
    loadA_to(A1, 1);
    if (isW) {
        loadH(0);
        loadW(0, 0);
        loadW(1, 1);
        decode();
        storeW(std::integral_constant<int, 0>{}, 0, 0);
        loadW(2, 0);
        storeW(std::integral_constant<int, 1>{}, 1, 1);
        loadW(3, 1);
    }
    storeA(0);
#pragma unroll
    for (int k = 0; k < APT; ++k) Ar[k] = A1[k];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    readA(0, H0{});
#pragma unroll
    for (int i = 0; i < TI; ++i) readW(0, H0{}, i);
    // One barrier per step, between its two k halves; step t's operands sit
    // in LDS buffer t & 1. Before the barrier: the first half's MFMAs
    // (operands read after the previous barrier), the second half's operand
    // reads from the same buffer, step t+1's activation stores into the
    // other buffer and the loads that refill those registers (one step
    // before their use). After it: the second half's MFMAs, the first-half
    // operand reads of step t+1, and step t+2's dequantized weights into
    // buffer t & 1, whose last reads came before the barrier (with the
    // weight loads for step t+4). Every read of a buffer comes before the
    // barrier that precedes its next store, so LDS latency hides under the
    // MFMAs, and the LDS stores and dequant work split across both halves.
    auto stage = [&](int t, auto ph) __attribute__((always_inline)) {
        constexpr int PH = decltype(ph)::value;  // t & 3
        constexpr int P = PH & 1;                 // buffer of step t (and t+2)
        constexpr int NS = P ^ 1;                 // buffer of step t+1
        constexpr int NM = TI * TJ;               // MFMAs per half
        halfStep(H0{}, P, H1{});
        storeA(NS);
        loadA(t + 2);
#pragma unroll
        for (int i = 0; i < NM; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x0008, 1, 0);                       // MFMA
            if (i < TJ) __builtin_amdgcn_sched_group_barrier(0x0100, 1, 0);             // DS read (tokens)
            if (i % TJ == TJ - 1) __builtin_amdgcn_sched_group_barrier(0x0100, 1, 0);   // DS read (W)
            if (i >= 10 && i % 2 == 0 && i < 18) __builtin_amdgcn_sched_group_barrier(0x0200, 1, 0);  // DS write
            if (i >= 11 && i % 2 == 1) __builtin_amdgcn_sched_group_barrier(0x0020, 1, 0);  // VMEM read
            __builtin_amdgcn_sched_group_barrier(0x0002, 1, 0);                       // VALU
        }
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        halfStep(H1{}, NS, H0{});
        // the block ends with this half: the next block's decode (one step
        // ago, before the barrier) flagged whether some row's e changed
        int changed = 0;
        if constexpr (PH == 3) changed = sFlag[1];
#pragma unroll
        for (int i = 0; i < NM; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x0008, 1, 0);                 // MFMA
            if (i < TJ + (PH == 3 ? 1 : 0)) __builtin_amdgcn_sched_group_barrier(0x0100, 1, 0);  // DS read (tokens)
            if (i % TJ == TJ - 1) __builtin_amdgcn_sched_group_barrier(0x0100, 1, 0);  // DS read (W)
        }
        __builtin_amdgcn_sched_barrier(0);
        if (isW) {
            // step t+2's weights open the next block at t = 2 mod 4: its
            // scales replace this block's, whose last step (t+1) was stored
            // one step ago
            if constexpr (PH == 2) decode();
            storeW(std::integral_constant<int, (PH + 2) & 3>{}, P, P);
            loadW(t + 4, P);
            if constexpr (PH == 0) loadH(t + 4);
        }
        if constexpr (PH == 1) sFlag[1] = 0;  // read at step 3 mod 4, set at 2 mod 4
        if constexpr (PH == 3) {
            if (__builtin_amdgcn_readfirstlane(changed)) {  // rare: rescale the sums so far
#pragma unroll
                for (int i = 0; i < TI; ++i) {
                    const f32x4 fr = *reinterpret_cast<const f32x4 *>(&sF[wn + 16 * i + 4 * q]);
#pragma unroll
                    for (int j = 0; j < TJ; ++j) acc[i][j] *= fr;
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    for (int t = 0; t < T; t += 4) {  // T = 4 * bpr
        stage(t, std::integral_constant<int, 0>{});
        stage(t + 1, std::integral_constant<int, 1>{});
        stage(t + 2, std::integral_constant<int, 2>{});
        stage(t + 3, std::integral_constant<int, 3>{});
    }

    // ---- epilogue: lane holds W rows wn+16i+4q+v of token wm+16j+l16 --------
    const bool vec = (n % 4) == 0 && (((uintptr_t)c & 15u) == 0);
#pragma unroll
    for (int i = 0; i < TI; ++i) {
        const int rl = wn + 16 * i + 4 * q;
        const f32x4 sc = *reinterpret_cast<const f32x4 *>(&sE[rl]);
        const int r = n0 + rl;
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const int m = m0 + wm + 16 * j + l16;
            if (m >= m_tokens) continue;
            const f32x4 v = acc[i][j] * sc;
            float *dst = c + (size_t)m * n + r;
            if (vec && r + 3 < n) {
                *reinterpret_cast<f32x4 *>(dst) = v;
            } else {
#pragma unroll
                for (int x = 0; x < 4; ++x)
                    if (r + x < n) dst[x] = v[x];
            }
        }
    }
}

static std::atomic<int> g_gemm_lds_state[64];

hipError_t gemm_prepare() {
    return allow_full_lds((const void *)gemm_q4k_f16_lds_kernel, g_gemm_lds_state);
}

static hipError_t gemm_lds_launch(const uint8_t *w, const uint16_t *a, float *c, int n, int bpr,
                                  int m_tokens, hipStream_t stream) {
    const hipError_t attr = gemm_prepare();
    if (attr != hipSuccess) return attr;
    const int tn = (n + G2Cfg::BN - 1) / G2Cfg::BN, tm = (m_tokens + G2Cfg::BM - 1) / G2Cfg::BM;
    const long ntiles = (long)tn * tm;
    const long grid = (ntiles + gemm::NXCD - 1) / gemm::NXCD * gemm::NXCD;
    if (grid > 0x7FFFFFFFL) return hipErrorInvalidValue;
    gemm_q4k_f16_lds_kernel<<<(unsigned)grid, G2Cfg::NT, G2Cfg::LDS, stream>>>(
        w, a, c, n, bpr, m_tokens, tn, tm);
    return hipGetLastError();
}

template <int BN>
static hipError_t gemm_launch_bn(const uint8_t *w, const uint16_t *a, float *c, int n, int bpr,
                                 int m_tokens, hipStream_t stream) {
    const int tn = (n + BN - 1) / BN, tm = (m_tokens + gemm::BM - 1) / gemm::BM;
    const long ntiles = (long)tn * tm;
    const long grid = (ntiles + gemm::NXCD - 1) / gemm::NXCD * gemm::NXCD;
    if (grid > 0x7FFFFFFFL) return hipErrorInvalidValue;
    gemm_q4k_f16_kernel<BN><<<(unsigned)grid, 256, 0, stream>>>(w, a, c, n, bpr, m_tokens, tn, tm);
    return hipGetLastError();
}

hipError_t gemm_f16_launch(const uint8_t *w, const uint16_t *a, float *c, int n, int bpr,
                           int m_tokens, hipStream_t stream) {
    if ((uintptr_t)a & 1u) return hipErrorInvalidValue;
    static const int big_env = [] {
        const char *v = std::getenv("MGQ_GEMM_LDS");
        return (v && *v) ? std::atoi(v) : -1;
    }();
    // The LDS-dequant kernel computes whole 256-token tiles, one work-group
    // per CU. Measured on 18944 x 3584 (us, warm; LDS kernel against the
    // 128-token kernel below): M = 256 76 / 61, 384 82 / 80, 512 83 / 94,
    // 640 150 / 120, 768 154 / 137, 1024 159 / 176. It wins when its token
    // tiles are at least 90 % full and its tiles fill their rounds: one round
    // more than half full, or several rounds at least 85 % full.
    const long tn2 = (n + G2Cfg::BN - 1) / G2Cfg::BN, tm2 = (m_tokens + G2Cfg::BM - 1) / G2Cfg::BM;
    const long cus2 = device_cus(), tiles2 = tn2 * tm2;
    const long rounds2 = (tiles2 + cus2 - 1) / cus2;
    const bool lds_fits = 10L * m_tokens >= 9L * G2Cfg::BM * tm2 &&
                          (rounds2 == 1 ? 2 * tiles2 > cus2 : 20 * tiles2 >= 17 * rounds2 * cus2);
    // the LDS kernel addresses A (including a tile's token rows past
    // m_tokens) and W with 32-bit byte offsets
    const bool a32 = ((uint64_t)m_tokens + G2Cfg::BM) * (uint64_t)bpr * kBlockElems * 2 <= 0xFFFFFFFFull &&
                     (uint64_t)n * (uint64_t)bpr * kBlockBytes <= 0xFFFFFFFFull;
    // its buffer_load_b128 reads assume 16-byte aligned W and A; the
    // 128/160-token kernel below reads both through alignment-1 global loads
    const bool aligned16 = (((uintptr_t)w | (uintptr_t)a) & 15u) == 0;
    if (a32 && aligned16 && (big_env == 1 || (big_env < 0 && lds_fits)))
        return gemm_lds_launch(w, a, c, n, bpr, m_tokens, stream);
    // Tile height by the rows the busiest CU computes: ceil(tiles / #CUs) x
    // BN, the lower one, ties to 160 (a second resident tile on a CU adds
    // only part of a tile's throughput). Measured on 18944 x 3584 (us, 128 vs
    // 160 rows): M = 256 80 / 65, 512 129 / 110, 640 136 / 145, 768 161 /
    // 146, 1024 193 / 180. MGQ_GEMM_BN=128 or 160 forces one.
    static const int bn_env = [] {
        const char *v = std::getenv("MGQ_GEMM_BN");
        return (v && *v) ? std::atoi(v) : 0;
    }();
    const long tm = (m_tokens + gemm::BM - 1) / gemm::BM, cus = device_cus();
    const long c128 = ((n + 127) / 128 * tm + cus - 1) / cus * 128;
    const long c160 = ((n + 159) / 160 * tm + cus - 1) / cus * 160;
    const bool wide = bn_env ? bn_env == 160 : c160 <= c128;
    return wide ? gemm_launch_bn<160>(w, a, c, n, bpr, m_tokens, stream)
                : gemm_launch_bn<128>(w, a, c, n, bpr, m_tokens, stream);
}

}  // namespace mgq
