// Persistent decode-step chain: the matvecs of a decode step (the
// reference's per-layer chain, rocm_gemma.rs:429-489, here a list of
// row-aligned Q4_K matvec descriptors) run in ONE cooperative launch instead
// of one kernel per matvec.
//
// Why: between dependent kernels the GPU idles for the launch gap (~1.6 us
// in a graph on MI355X) plus the next kernel's first weight arrival and the
// previous one's tail, 4-5 us per matvec, ~0.5 ms of a 7B decode step. The
// weights never depend on the activations, so a persistent work-group can
// keep streaming the next matvec's weights while the step waits for the
// previous matvec's output.
//
// Semantics: descriptor d may read anything descriptors < d wrote (its x is
// typically an earlier y). Before a work-group builds descriptor d's
// activation table it waits until every work-group has finished every
// descriptor < d, exactly the ordering of launching them one after another
// on a stream. A descriptor's y must not alias its own x or any weights.
//
// Completion signalling by the HSA memory model: y values are written with
// agent-scope atomic stores, then the work-group's control wave issues an
// agent-scope release fence (its stores complete and reach the device
// coherence point) and adds 1 to its shard of the finished descriptor's
// counter (relaxed, so the fence heads the release sequence); a waiter that
// has read every shard at its target issues an agent-scope acquire fence
// before its work-group reads any y. Descriptor d has 16
// device-scope counters, work-group b adds to counter b % 16, so no counter
// takes more than 16 adds per launch. A work-group with no rows in a
// descriptor signals it as soon as it moves past it. Every work-group
// signals descriptors in order, so descriptor d's 16 counters being full
// means every work-group is done with d and everything before it; waiters
// poll those 16 counters with agent-scope loads. Counters only grow (64-bit;
// the launch index is folded into the targets) and are never reset.
// Sharding measured on MI355X (before the fences): ~1.5 us per grid-wide
// wait, against 3.5-8 us for one shared counter or one flag per work-group.
//
// Work-group layout (one per CU): 14 compute waves + 1 control wave. The
// compute waves run the matrix-core GEMV of gemv_mfma_kernel (16-row groups,
// stages of 14 blocks x 16 rows through a double-buffered LDS stage, the
// activations as matrix-core operands in an LDS table), one 16-row x 1-block
// tile per wave and stage; their weight loads run PF stages ahead across
// descriptor boundaries. The control wave does no weight loads, so its
// waits for y stores and counters never drain the compute waves' streams.
#include "../../include/modgrad_q4k.h"
#include "q4k_device.hpp"
#include "q4k_launch.hpp"

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <new>
#include <vector>

namespace mgq {

namespace pc {
constexpr int R = 16;                  // rows per group (one MFMA N tile)
constexpr int C = 14;                  // blocks per stage
constexpr int BP = 9;                  // 16-byte pieces per Q4_K block
constexpr int BB = 144;                // bytes per block
constexpr int RP = (BP * C) | 1;       // LDS pieces per staged row (odd: conflict-free)
constexpr int SB = R * RP * 16;        // LDS bytes per stage buffer
constexpr int PIECES = R * BP * C;     // 16-byte pieces per stage
constexpr int NW = 14;                 // compute waves: one 16-row x 1-block tile each
constexpr int NT = (NW + 1) * 64;      // + the control wave
constexpr int IPW = ((PIECES + 63) / 64 + NW - 1) / NW;  // loads per lane per stage
constexpr int NCTR = 16;               // completion counters per descriptor
constexpr int CTR_STRIDE = 16;         // u64 slots between counters (128 B)
constexpr int XIT = 3;                 // activation items (8 floats) per compute thread
constexpr int MAX_BPR = XIT * NW * 64 / 32;  // 84 blocks: K <= 21504
constexpr int TAB = 1040;              // LDS table bytes per block (1 KiB + zero slot)
}  // namespace pc

// One matvec of the chain, as the kernel reads it.
struct ChainTask {
    const uint8_t *w;
    const float *x;
    float *y;
    int n, bpr;
    int groups;  // ceil(n / 16)
    int offset;  // group g is handled by work-group (g + offset) % gridDim.x
    int stages;  // ceil(bpr / 14)
    int pad;
};

struct ChainLds {
    uint32_t meta, stage, aux, ybuf, total;
};

__host__ __device__ inline ChainLds chain_lds(int tab_blocks, int ymax) {
    ChainLds L;
    L.meta = (uint32_t)tab_blocks * pc::TAB;
    L.stage = (L.meta + (uint32_t)tab_blocks * 64u + 15u) & ~15u;
    L.aux = L.stage + 2u * pc::SB;
    L.ybuf = L.aux + 2u * pc::NW * 64u;
    L.total = L.ybuf + (uint32_t)ymax * pc::R * 4u;
    return L;
}

// groups of task t that work-group b handles, and the first of them
__device__ __forceinline__ int my_first(const ChainTask &t, int b, int G) {
    int f = (b - t.offset) % G;
    return f < 0 ? f + G : f;
}
__device__ __forceinline__ int my_count(const ChainTask &t, int f, int G) {
    return t.groups > f ? (t.groups - f - 1) / G + 1 : 0;
}

// The task table holds plain (generic) pointers; accesses through them are
// made global-address-space explicitly, so the compiler emits global_*
// instructions instead of flat_* ones (a flat load also counts against the
// LDS wait counter, which would make every LDS wait drain the weight stream).
typedef __attribute__((address_space(1))) uint8_t g_u8;
typedef __attribute__((address_space(1))) uint32_t g_u32;
typedef __attribute__((address_space(1))) float g_f32;
typedef __attribute__((address_space(1))) u32x4_a1 g_u32x4_a1;

// Activation reads: 16-byte buffer loads with the device-scope coherence bit
// (sc1) over a resource covering exactly the vector, so reads past its end
// return zeros without touching memory.
constexpr int kBufSc1 = 16;  // cache-policy bit sc1 of buffer instructions
__device__ __forceinline__ u32x4 ld_w16(const uint8_t *p) { return *(const g_u32x4_a1 *)p; }
__device__ __forceinline__ void st_sc1(float *p, float v) {
    __hip_atomic_store((g_f32 *)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int PF>
__global__ __launch_bounds__(pc::NT) void chain_kernel(const ChainTask *__restrict__ tasks,
                                                       int ntasks, int tab_blocks, int ymax,
                                                       uint64_t *__restrict__ ctr, uint64_t launch,
                                                       unsigned *__restrict__ err,
                                                       int spin_limit) {
    using namespace pc;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const ChainLds Lo = chain_lds(tab_blocks, ymax);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = gridDim.x, b = blockIdx.x;
    float *meta = reinterpret_cast<float *>(lds + Lo.meta);
    float *aux = reinterpret_cast<float *>(lds + Lo.aux);
    float *ybuf = reinterpret_cast<float *>(lds + Lo.ybuf);

    // task d's parameters through a wave-uniform index (scalar loads)
    auto task = [&](int d) -> const ChainTask & {
        return tasks[__builtin_amdgcn_readfirstlane(d)];
    };
    // ---- this work-group's stage sequence ----------------------------------
    // A cursor walks (task d, group j of mine, stage s) over the tasks where
    // this work-group has groups; all fields are wave-uniform. Every wave
    // walks the same sequence and meets the same barriers.
    struct Cur {
        int d, j, s, cnt, f;
    };
    auto skip_empty = [&](Cur &c) {
        while (c.d < ntasks) {
            const ChainTask &t = task(c.d);
            c.f = my_first(t, b, G);
            c.cnt = my_count(t, c.f, G);
            if (c.cnt > 0) break;
            ++c.d;
        }
    };
    auto advance = [&](Cur &c) {
        if (c.d >= ntasks) return;
        if (++c.s == task(c.d).stages) {
            c.s = 0;
            if (++c.j == c.cnt) {
                c.j = 0;
                ++c.d;
                skip_empty(c);
            }
        }
    };
    Cur cc{0, 0, 0, 0, 0};
    skip_empty(cc);

    if (wave == NW) {
        // ================= control wave: publish, signal, wait ==============
        int signaled = 0;  // tasks this work-group has signaled
        // Store this work-group's rows of task `done` (if >= 0) with
        // agent-scope stores, wait for them, then signal every task below
        // `upto` not signaled yet; if `wait`, poll until all work-groups have
        // signaled task upto - 1 (and so every task before it).
        auto signal_wait = [&](int done, int upto, bool wait) {
            if (done >= 0) {
                const ChainTask &t = task(done);
                const int f = my_first(t, b, G), cnt = my_count(t, f, G);
                for (int i = lane; i < cnt * R; i += 64) {
                    const int row = (f + (i / R) * G) * R + (i % R);
                    if (row < t.n) st_sc1(t.y + row, ybuf[i]);
                }
            }
            // release at agent scope: every y store of this wave (and anything
            // else this work-group wrote before) is visible device-wide before
            // any counter add below is
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
            // one lane per task to signal, in parallel (a work-group skips
            // ahead over tasks where it has no rows)
            for (int t = signaled + lane; t < upto; t += 64)
                __hip_atomic_fetch_add(ctr + ((size_t)t * NCTR + b % NCTR) * CTR_STRIDE, (uint64_t)1,
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            signaled = upto;
            if (!wait) return;
            // counter c of a task collects the work-groups b with b % 16 == c,
            // once per launch
            const uint64_t members = (uint64_t)((G - lane + NCTR - 1) / NCTR);
            const uint64_t target = (launch + 1) * members;
            const uint64_t *tc = ctr + (size_t)(upto - 1) * NCTR * CTR_STRIDE;
            // Bounded: after spin_limit polls the wait gives up and sets the
            // error word; a wait that finds the word set gives up at once, so
            // a broken launch ends after one time-out instead of one per task.
            int spins = 0;
            while (true) {
                bool ok = true, bad = false;
                if (lane < NCTR)
                    ok = __hip_atomic_load(tc + (size_t)lane * CTR_STRIDE, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT) >= target;
                else if (lane == NCTR)
                    bad = __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u;
                if (__all(ok)) {
                    // acquire at agent scope: the counters read above were
                    // made by adds that followed their work-group's release,
                    // so every y they cover is visible to this work-group's
                    // reads after the barrier that follows this wait
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
                    break;
                }
                if (__any(bad)) break;
                if (++spins > spin_limit) {
                    if (lane == 0) atomicOr(err, 1u);
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
        };
        if (cc.d >= ntasks) {  // no groups for this work-group
            signal_wait(-1, ntasks, false);
            return;
        }
        int prev_d = -1;
        while (cc.d < ntasks) {
            if (cc.d != prev_d) {
                __syncthreads();                      // A: ybuf holds task prev_d
                signal_wait(prev_d, cc.d, cc.d > 0);
                __syncthreads();                      // B: tasks < cc.d complete
                __syncthreads();                      // C: the table is built
                prev_d = cc.d;
            }
            __syncthreads();                          // D: the stage is done
            advance(cc);
        }
        __syncthreads();                              // E: ybuf holds the last task
        signal_wait(prev_d, ntasks, false);
        return;
    }

    // ======================= compute waves (NW of them) ======================
    if (cc.d >= ntasks) return;
    constexpr int NTC = NW * 64;  // compute threads
    // ---- weight staging: global -> registers (PF sets) -> LDS -------------
    // Piece k of this lane: row prow, block-in-stage pcb, piece-in-block ppc
    // (stage-invariant). Loads past the end of the sequence re-read a valid
    // address (the last task's first bytes), so every load is unconditional.
    u32x4 stg[PF][IPW];
    uint32_t prow[IPW], pcb[IPW], ppc[IPW], plds[IPW];
#pragma unroll
    for (int k = 0; k < IPW; ++k) {
        const int j = std::min((wave + k * NW) * 64 + lane, PIECES - 1);
        const int row = j / (BP * C), rem = j - row * BP * C;
        const int cb = rem / BP, pp = rem - cb * BP;
        prow[k] = (uint32_t)row;
        pcb[k] = (uint32_t)cb;
        ppc[k] = (uint32_t)pp;
        plds[k] = (uint32_t)((row * RP + rem) * 16);
    }
    auto gload = [&](const Cur &c, u32x4(&dst)[IPW]) __attribute__((always_inline)) {
        const bool past = c.d >= ntasks;
        const ChainTask &t = task(past ? ntasks - 1 : c.d);
        const uint32_t g = past ? 0u : (uint32_t)(c.f + c.j * G);
        const uint32_t s = past ? 0u : (uint32_t)c.s;
        const uint32_t rlast = (uint32_t)(t.n - 1), blast = (uint32_t)(t.bpr - 1);
        const uint64_t rb = (uint64_t)t.bpr * BB;
#pragma unroll
        for (int k = 0; k < IPW; ++k) {
            const uint32_t rr = std::min(g * R + prow[k], rlast);
            const uint32_t bl = std::min(s * C + pcb[k], blast);
            dst[k] = ld_w16(t.w + rr * rb + bl * BB + ppc[k] * 16u);
        }
    };
    auto lstore = [&](int buf, const u32x4(&src)[IPW]) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < IPW; ++k)
            *reinterpret_cast<u32x4 *>(lds + Lo.stage + buf * SB + plds[k]) = src[k];
    };

    // ---- per-lane MFMA constants (as gemv_mfma_kernel, R = 16) --------------
    const int n16 = lane & 15, g = lane >> 4, jq = g >> 1, sh = 16 * (g & 1);
    const uint32_t lmask = jq ? 0x0F0F0F0Fu : 0x3F3F3F3Fu, hmask = jq ? 0x30303030u : 0u;
    uint32_t aoff[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const int p = c >> 1;
        const int o = p < 2 ? 16 * g + 8 * p : 64 + 16 * g + 8 * (p - 2);
        const int sb = 2 * (o >> 5) + (c & 1);
        aoff[c] = ((n16 >> 1) == sb) ? (uint32_t)((c * 4 + g) * 32 + (n16 & 1) * 16) : 1024u;
    }
    auto decode = [&](const u32x4 &hd, int bl, float s0, float s1) -> float {
        const float d = half_bits_finite(hd[0]), dmin = half_bits_finite(hd[0] >> 16);
        const uint32_t scs = jq ? hd[3] : hd[1], mns = jq ? (hd[3] >> 4) : hd[2];
        const uint32_t scq = ((scs & lmask) | ((hd[1] >> 2) & hmask)) >> sh;
        const uint32_t mnq = ((mns & lmask) | ((hd[2] >> 2) & hmask)) >> sh;
        const float *mb = meta + bl * 16 + 2 * g;
        const float t1 = (float)(scq & 0xFFu) * (s0 * mb[0]) + (float)((scq >> 8) & 0xFFu) * (s1 * mb[1]);
        const float t2 = (float)(mnq & 0xFFu) * mb[8] + (float)((mnq >> 8) & 0xFFu) * mb[9];
        return d * t1 - dmin * t2;
    };

    // ---- the activation table of task d (the compute waves) ----------------
    // Item i = 8 floats of x: block i/32, sub-block (i/4)%8, chunk i%4, so a
    // sub-block's 4 chunks sit in 4 adjacent lanes. x is read with
    // agent-scope loads: it may be a y that other work-groups just wrote.
    // Every thread loads XIT items (items past the end read as zeros, outside
    // the buffer resource) and consumes all of them: a load whose value is
    // never used would leave its register pending into the stage loop, where
    // the compiler would then wait for it and every weight load before it.
    auto build_table = [&](int d) __attribute__((always_inline)) {
        const ChainTask &t = task(d);
        const int bpr = t.bpr, nitems = bpr * 32;
        const __amdgpu_buffer_rsrc_t xr =
            __builtin_amdgcn_make_buffer_rsrc((void *)t.x, 0, nitems * 32, kRawBufWord3);
        // eight dword loads per item, which the compiler merges into two
        // 16-byte loads (the 128-bit builtin's vector result does not survive
        // element extraction on this compiler)
        uint32_t xv[XIT][8];
#pragma unroll
        for (int it = 0; it < XIT; ++it) {
            const int i = tid + it * NTC;
#pragma unroll
            for (int e = 0; e < 8; ++e)
                xv[it][e] = __builtin_amdgcn_raw_buffer_load_b32(xr, i * 32 + 4 * e, 0, kBufSc1);
        }
        for (int bl = tid; bl < bpr; bl += NTC)  // the blocks' zero slots
            *reinterpret_cast<u32x4 *>(lds + (size_t)bl * TAB + 1024) = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int it = 0; it < XIT; ++it) {
            const int i = tid + it * NTC;
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = __builtin_bit_cast(float, xv[it][e]);
            float amax = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[e]));
            float sum = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
            amax = fmaxf(amax, quad_xor<1>(amax));
            amax = fmaxf(amax, quad_xor<2>(amax));
            sum += quad_xor<1>(sum);
            sum += quad_xor<2>(sum);
            if (i >= nitems) continue;
            int e = 0;  // x*2^e puts the sub-block's largest |x| in [2^13, 2^14)
            if (amax > 0.0f && amax <= 3.402823466e38f) {
                int ex;
                frexpf(amax, &ex);
                e = std::min(std::max(14 - ex, -103), 140);  // 2^(24 - e) stays finite
            }
            const int bl = i >> 5, sb = (i >> 2) & 7, jj = i & 3;
            if (jj == 0) {
                // high-nibble operands are 16q*2^-24 (masked in place)
                meta[bl * 16 + sb] = ldexpf(1.0f, ((sb & 1) ? 20 : 24) - e);
                meta[bl * 16 + 8 + sb] = sum;
            }
            const int G2 = sb >> 1;
            const int c = 2 * (2 * (G2 >> 1) + (jj & 1)) + (sb & 1), h = 2 * (G2 & 1) + (jj >> 1);
            const float xs[8] = {v[0], v[2], v[1], v[3], v[4], v[6], v[5], v[7]};
            u32x4 hh, hl;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float a0 = ldexpf(xs[2 * q], e), a1 = ldexpf(xs[2 * q + 1], e);
                const auto hp = __builtin_amdgcn_cvt_pkrtz(a0, a1);
                const auto lp = __builtin_amdgcn_cvt_pkrtz(a0 - (float)hp[0], a1 - (float)hp[1]);
                hh[q] = __builtin_bit_cast(uint32_t, hp);
                hl[q] = __builtin_bit_cast(uint32_t, lp);
            }
            uint8_t *ent = lds + (size_t)bl * TAB + (size_t)((c * 4 + h) * 32);
            *reinterpret_cast<u32x4 *>(ent) = hh;
            *reinterpret_cast<u32x4 *>(ent + 16) = hl;
        }
    };

    // prologue: PF stages in flight, the first stored to LDS buffer 0
    Cur lc = cc;
#pragma unroll
    for (int f = 0; f < PF; ++f) {
        gload(lc, stg[f]);
        advance(lc);
    }
    lstore(0, stg[0]);
    gload(lc, stg[0]);
    advance(lc);
    int prev_d = -1;  // task of the previous stage
    float yacc = 0.0f;
    int q = 0;
    // One stage: at a task's first stage, wait (barriers A, B) while the
    // control wave finishes the previous task, then build this task's table
    // (C); compute the stage from LDS buffer q & 1, store stage q + 1 from
    // its register set into the other buffer, refill that set with stage
    // q + 1 + PF (D).
    auto step = [&](auto fc) __attribute__((always_inline)) {
        constexpr int F = decltype(fc)::value;  // == q % PF
        if (cc.d != prev_d) {
            __syncthreads();  // A
            __syncthreads();  // B
            build_table(cc.d);
            __syncthreads();  // C
            prev_d = cc.d;
        }
        const ChainTask &t = task(cc.d);
        const int bpr = t.bpr;
        const uint8_t *sbuf = lds + Lo.stage + (q & 1) * SB;
        const bool group_end = cc.s == t.stages - 1;
        const int bA = cc.s * C + wave;
        if (bA < bpr) {
            auto piece = [&](int pp) -> const u32x4 & {
                return *reinterpret_cast<const u32x4 *>(sbuf + (n16 * RP + wave * BP + pp) * 16);
            };
            const u32x4 qa0 = piece(1 + g), qa1 = piece(5 + g), hdA = piece(0);
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const half8 aA = *reinterpret_cast<const half8 *>(lds + (uint32_t)bA * TAB + aoff[c]);
                const int p = c >> 1;
                const uint32_t mask = (c & 1) ? 0x00F000F0u : 0x000F000Fu;
                const uint32_t wa0 = p < 2 ? qa0[2 * p] : qa1[2 * p - 4];
                const uint32_t wa1 = p < 2 ? qa0[2 * p + 1] : qa1[2 * p - 3];
                const u32x4 ba = u32x4{wa0 & mask, (wa0 >> 8) & mask, wa1 & mask, (wa1 >> 8) & mask};
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(aA, __builtin_bit_cast(half8, ba), acc, 0, 0, 0);
            }
            yacc += decode(hdA, bA, acc[0] + acc[1], acc[2] + acc[3]);
        }
        // a group's aux buffer alternates with the group's parity: the next
        // group writes the other one before any barrier of its own
        float *auxg = aux + (cc.j & 1) * (NW * 16);
        if (group_end) {
            yacc += __shfl_xor(yacc, 16, 64);
            yacc += __shfl_xor(yacc, 32, 64);
            if (lane < 16) auxg[wave * 16 + lane] = yacc;
        }
        lstore((q + 1) & 1, stg[(F + 1) % PF]);
        gload(lc, stg[(F + 1) % PF]);
        advance(lc);
        __syncthreads();  // D
        if (group_end) {
            if (tid < R) {
                float sum = 0.0f;
                for (int wv = 0; wv < NW; ++wv) sum += auxg[wv * 16 + tid];
                ybuf[cc.j * R + tid] = sum;
            }
            yacc = 0.0f;
        }
        advance(cc);
        ++q;
    };
    // Main loop, a counted loop unrolled by PF so that every register set is
    // indexed with a compile-time constant (and the compiler's load-wait
    // accounting stays exact: each stage waits only for its own set).
    int Q = 0;  // this work-group's stages
    for (int d = 0; d < ntasks; ++d) {
        const ChainTask &t = task(d);
        Q += my_count(t, my_first(t, b, G), G) * t.stages;
    }
    int q0 = 0;
    for (; q0 + PF <= Q; q0 += PF) {
        step(std::integral_constant<int, 0>{});
        if constexpr (PF > 1) step(std::integral_constant<int, 1 % PF>{});
        if constexpr (PF > 2) step(std::integral_constant<int, 2 % PF>{});
    }
    if (q0 < Q) step(std::integral_constant<int, 0>{});
    if constexpr (PF > 2)
        if (q0 + 1 < Q) step(std::integral_constant<int, 1>{});
    __syncthreads();  // E: the last group's results are in ybuf
}

// ------------------------------------------------------------------ host --

struct PersistentChain {
    void *mem = nullptr;  // tasks | counters | error word (one allocation)
    ChainTask *tasks = nullptr;
    uint64_t *ctr = nullptr;
    unsigned *err = nullptr;
    int ntasks = 0, grid = 0, tab_blocks = 0, ymax = 0;
    uint32_t lds = 0;
    uint64_t launches = 0;
};

constexpr int kChainPF = 2;

static hipError_t chain_attr() {
    static std::atomic<int> state[64];
    return allow_full_lds((const void *)chain_kernel<kChainPF>, state);
}

// 0 if the descriptors fit the persistent chain (row-aligned Q4_K, K <= 84
// blocks, LDS within 160 KiB, cooperative launch on this device), else the
// reason as a hipError_t.
hipError_t chain_persistent_create(const mgq_gemv_desc *descs, int n, PersistentChain **out) {
    *out = nullptr;
    int dev = 0, coop = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess || !coop)
        return hipErrorNotSupported;
    int max_bpr = 1;
    for (int i = 0; i < n; ++i) {
        if (descs[i].blocks_per_row > pc::MAX_BPR) return hipErrorNotSupported;
        max_bpr = std::max(max_bpr, descs[i].blocks_per_row);
    }
    e = chain_attr();
    if (e != hipSuccess) return e;
    const int G = device_cus();
    std::vector<ChainTask> tasks((size_t)n);
    long offset = 0;
    int ymax = 1;
    for (int i = 0; i < n; ++i) {
        const mgq_gemv_desc &d = descs[i];
        ChainTask &t = tasks[(size_t)i];
        t.w = d.w_q4;
        t.x = d.x;
        t.y = d.y;
        t.n = d.out_dim;
        t.bpr = d.blocks_per_row;
        t.groups = (d.out_dim + pc::R - 1) / pc::R;
        t.offset = (int)(offset % G);
        t.stages = (d.blocks_per_row + pc::C - 1) / pc::C;
        t.pad = 0;
        offset += t.groups;
        ymax = std::max(ymax, (t.groups + G - 1) / G);
    }
    const ChainLds L = chain_lds(max_bpr, ymax);
    if (L.total > 160 * 1024) return hipErrorNotSupported;
    int occ = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, (const void *)chain_kernel<kChainPF>,
                                                     pc::NT, L.total) != hipSuccess || occ < 1)
        return hipErrorNotSupported;
    auto *pcn = new (std::nothrow) PersistentChain;
    if (!pcn) return hipErrorOutOfMemory;
    const size_t tb = ((size_t)n * sizeof(ChainTask) + 255) & ~(size_t)255;
    const size_t cb = (size_t)n * pc::NCTR * pc::CTR_STRIDE * sizeof(uint64_t);
    e = hipMalloc(&pcn->mem, tb + cb + 256);
    if (e == hipSuccess) e = hipMemcpy(pcn->mem, tasks.data(), (size_t)n * sizeof(ChainTask),
                                       hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemset(static_cast<uint8_t *>(pcn->mem) + tb, 0, cb + 256);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        if (pcn->mem) (void)hipFree(pcn->mem);
        delete pcn;
        return e;
    }
    pcn->tasks = static_cast<ChainTask *>(pcn->mem);
    pcn->ctr = reinterpret_cast<uint64_t *>(static_cast<uint8_t *>(pcn->mem) + tb);
    pcn->err = reinterpret_cast<unsigned *>(static_cast<uint8_t *>(pcn->mem) + tb + cb);
    pcn->ntasks = n;
    pcn->grid = G;
    pcn->tab_blocks = max_bpr;
    pcn->ymax = ymax;
    pcn->lds = L.total;
    *out = pcn;
    return hipSuccess;
}

// spin limit of the grid-wide waits: ~1 us per poll, so about a second
// before a wait gives up (and flags the chain's error word)
constexpr int kChainSpinLimit = 1 << 20;

hipError_t chain_persistent_launch(PersistentChain *p, hipStream_t stream) {
    const ChainTask *tasks = p->tasks;
    int ntasks = p->ntasks, tab = p->tab_blocks, ymax = p->ymax, spin = kChainSpinLimit;
    uint64_t *ctr = p->ctr;
    uint64_t launch = p->launches;
    unsigned *err = p->err;
    void *args[] = {&tasks, &ntasks, &tab, &ymax, &ctr, &launch, &err, &spin};
    const hipError_t e = hipLaunchCooperativeKernel((const void *)chain_kernel<kChainPF>,
                                                    dim3((unsigned)p->grid), dim3(pc::NT), args,
                                                    p->lds, stream);
    if (e == hipSuccess) ++p->launches;
    return e;
}

hipError_t chain_persistent_faults(PersistentChain *p, unsigned *faults) {
    return hipMemcpy(faults, p->err, sizeof(unsigned), hipMemcpyDeviceToHost);
}

hipError_t chain_persistent_destroy(PersistentChain *p) {
    const hipError_t e = p->mem ? hipFree(p->mem) : hipSuccess;
    delete p;
    return e;
}

}  // namespace mgq
