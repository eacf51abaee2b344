// Internal (C++) launchers behind the C ABI. Arguments are validated by the
// ABI layer (q4k_abi.hip) before any of these is called.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/modgrad_q4k.h"

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <map>
#include <mutex>
#include <tuple>

namespace mgq {

// Compute units of the current device, cached per device (the persistent
// launches size their grids from it on every call).
inline int device_cus() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
            v = 256;
        cus[dev] = v;
    }
    return cus[dev];
}

// Resident work-groups per CU of `kern` at `threads` threads and `lds` bytes
// of dynamic LDS on the current device, from the runtime's occupancy query,
// or `dflt` when the query fails. Cached per (kernel, device, threads, lds):
// the runtime is asked once per shape class, not on every launch (the
// reference's engine launches every matvec eagerly, 113+ per token).
inline int occupancy_cached(const void *kern, int threads, size_t lds, int dflt) {
    static std::mutex mu;
    static std::map<std::tuple<const void *, int, int, size_t>, int> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return dflt;
    const auto key = std::make_tuple(kern, dev, threads, lds);
    {
        std::lock_guard<std::mutex> g(mu);
        const auto it = cache.find(key);
        if (it != cache.end()) return it->second;
    }
    int occ = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kern, threads, lds) != hipSuccess || occ <= 0)
        occ = dflt;
    std::lock_guard<std::mutex> g(mu);
    cache.emplace(key, occ);
    return occ;
}

// Allows `kern` the whole 160 KiB of gfx950 LDS. The attribute belongs to the
// current device, so it is set once per (kernel, device); `state` is the
// call site's per-device record (0 = not yet set, else hipError_t + 1).
inline hipError_t allow_full_lds(const void *kern, std::atomic<int> (&state)[64]) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    int s = state[dev].load(std::memory_order_acquire);
    if (s == 0) {
        s = (int)hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) + 1;
        state[dev].store(s, std::memory_order_release);
    }
    return (hipError_t)(s - 1);
}

// allow_full_lds for kernels told apart by address only (instances of one
// signature): the per-device state is kept per kernel in a map.
inline hipError_t allow_full_lds_by_addr(const void *kern) {
    static std::mutex mu;
    static std::map<std::pair<const void *, int>, hipError_t> done;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> g(mu);
    const auto key = std::make_pair(kern, dev);
    const auto it = done.find(key);
    if (it != done.end()) return it->second;
    const hipError_t e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    done.emplace(key, e);
    return e;
}

// Row-group schedule of a persistent launch (G = gridDim.x work-groups). In
// rounds j < shared every work-group b takes group b + j*G; the groups past
// shared*G go to the `lead` lowest-numbered work-groups only, strided by lead.
// {lead = G, shared = 0} is the plain strided schedule. With two work-groups
// per CU the hardware dispatches the lower-numbered one of each pair first and
// issues its waves first, so it streams faster; giving those `lead` = #CUs
// work-groups the extra rounds lets both members of a pair finish together.
struct GemvSched {
    int lead, shared;
};

__host__ __device__ __forceinline__ int sched_group(const GemvSched &s, int b, int G, int j) {
    return j < s.shared ? b + j * G : s.shared * G + (j - s.shared) * s.lead + b;
}

// groups work-group b takes out of `groups`
__host__ __device__ inline int sched_count(const GemvSched &s, int b, int G, int groups) {
    if (b >= groups) return 0;
    const int own = std::min(s.shared, (groups - b - 1) / G + 1);
    const int rest = groups - s.shared * G;
    return own + ((b < s.lead && rest > b) ? (rest - b - 1) / s.lead + 1 : 0);
}

// Share of the row groups, in percent of the average, that the
// second-dispatched work-group of each CU pair takes in a persistent launch
// (MGQ_GEMV_SKEW overrides; 0 keeps the plain strided schedule).
constexpr int kGemvSkew = 70;

inline int gemv_skew() {
    static const int v = [] {
        const char *s = std::getenv("MGQ_GEMV_SKEW");
        return std::max(0, std::min(100, (s && *s) ? std::atoi(s) : kGemvSkew));
    }();
    return v;
}

// Grid, per-work-group rounds (the LDS result buffer is sized for them) and
// schedule of a persistent launch of `groups` row groups at `occ` resident
// work-groups per CU. Balanced by default: every work-group gets `rounds`
// groups or one fewer. With two per CU and at least two full rounds of
// pairs, the grid is exactly 2 x #CUs and the younger member of each pair
// (ids >= #CUs) takes gemv_skew() percent of the average share.
struct PersistPlan {
    long grid, rounds;
    GemvSched sch;
};

inline PersistPlan persistent_plan(long groups, int occ) {
    const long cus = device_cus();
    const long maxgrid = cus * std::max(1, occ);
    PersistPlan p;
    p.rounds = (groups + maxgrid - 1) / maxgrid;
    p.grid = (groups + p.rounds - 1) / p.rounds;
    p.sch = GemvSched{(int)p.grid, 0};
    const int skew = gemv_skew();
    if (skew > 0 && occ == 2 && groups >= 2 * maxgrid) {
        // at least one round each: the kernels assume every work-group owns a group
        const long shared = std::max(1L, groups * skew / (100 * maxgrid));
        const long rest = groups - shared * maxgrid;
        p.grid = maxgrid;
        p.sch = GemvSched{(int)cus, (int)shared};
        p.rounds = shared + (rest + cus - 1) / cus;
    }
    return p;
}

// Bit-exact canonical dequant of n_blocks super-blocks; q must be 4-B aligned.
hipError_t dequant_launch(const uint8_t *q, int n_blocks, float *out, hipStream_t stream);

// Generic GEMV over the flat-stream layout (element (r,c) at flat r*k+c);
// any k with n*k % 256 == 0; w 4-B aligned. Also serves the row-aligned
// layout (k % 256 == 0) when the fast kernel does not apply.
hipError_t gemv_generic_launch(const uint8_t *w, const float *x, float *y, int n, int k,
                               hipStream_t stream);
// Flat-stream layout with k % 32 == 0 (whole sub-blocks per row), w and x
// 16-byte aligned; hipErrorNotSupported otherwise (then: generic).
hipError_t gemv_flat_launch(const uint8_t *w, const float *x, float *y, int n, int k,
                            hipStream_t stream);

// Matrix-core GEMV for the row-aligned layout. Returns hipErrorNotSupported
// when the shape or alignment does not fit it (caller then uses generic).
hipError_t gemv_mfma_launch(const uint8_t *w, const float *x, float *y, int n, int bpr,
                            hipStream_t stream);

// One-time kernel attribute setup (dynamic LDS limit) of the GEMV kernels,
// the Q6_K and batched kernels included; safe to call often.
hipError_t gemv_prepare();
// The Q6_K matrix-core kernels' LDS attributes and occupancy (q4k_q6k_mfma.hip).
hipError_t q6k_prepare();
// The batched matvec kernels' LDS attributes (q4k_batched.hip).
hipError_t batched_prepare();

// Looks up the current device's address of the no-allocation entry point's
// fixed scratch array (once per device).
hipError_t noalloc_prepare();

// Row-aligned GEMV: picks the matrix-core kernel when it applies.
hipError_t gemv_rows_launch(const uint8_t *w, const float *x, float *y, int n, int bpr,
                            hipStream_t stream);

// Vector-ALU batched GEMV (any 4-byte alignment, no workspace).
hipError_t gemv_batched_launch(const uint8_t *w, const float *X, float *Y, int n, int bpr,
                               int batch, hipStream_t stream);

// Matrix-core batched GEMV: an operand-table pass into `workspace`, then the
// main kernel. hipErrorNotSupported when w or the workspace is not 16-byte
// aligned (the caller then uses the vector-ALU kernel).
size_t batched_workspace_bytes(int bpr, int batch);
hipError_t gemv_batched_mfma_launch(const uint8_t *w, const float *X, float *Y, int n, int bpr,
                                    int batch, void *workspace, size_t workspace_bytes,
                                    hipStream_t stream);

// Q8_1 activation quantizer (bit-identical to the reference's) and the dp4a
// matvec on the quantized activations: the matrix-core kernel's Q8 mode when
// every pointer is 16-byte aligned and the shape fits LDS, else the
// vector-ALU kernel.
hipError_t quantize_q8_1_launch(const float *x, int8_t *xq, float *xd, float *xsum, int n,
                                hipStream_t stream);
hipError_t gemv_q8_launch(const uint8_t *w, const int8_t *xq, const float *xd, const float *xsum,
                          float *y, int n, int bpr, hipStream_t stream);
// launch_quantize_q8_1 + the dp4a matvec in one launch (the matrix-core
// kernel's Q8 mode quantizing f32 x in its prologue); w and x 16-byte aligned
// (hipErrorNotSupported otherwise).
hipError_t gemv_q8x_launch(const uint8_t *w, const float *x, float *y, int n, int bpr,
                           hipStream_t stream);
hipError_t gemv_q8_generic_launch(const uint8_t *w, const int8_t *xq, const float *xd,
                                  const float *xsum, float *y, int n, int bpr, hipStream_t stream);

// Matrix-core Q5_K matvec (the Q4_K kernel's Q5_K format mode); w and x
// 16-byte aligned, else hipErrorNotSupported (as when LDS does not fit).
hipError_t gemv_q5k_mfma_launch(const uint8_t *w, const float *x, float *y, int n, int bpr,
                                hipStream_t stream);

// Matrix-core Q6_K matvec (whole-row stages for K <= 3584, K-chunked stages
// beyond, up to ~100 blocks per row); hipErrorNotSupported for longer K,
// misaligned w or x, or a tensor that does not end on a 16-byte boundary.
hipError_t gemv_q6k_mfma_launch(const uint8_t *w, const float *x, float *y, int n, int bpr,
                                hipStream_t stream);
// Fused RMSNorm -> Q6_K matvec on the matrix cores (whole-row stages only:
// K <= 14 blocks); hipErrorNotSupported outside them or for misaligned w.
hipError_t gemv_q6k_mfma_norm_launch(const uint8_t *w, const float *x, const float *nw, float eps,
                                     float *y, int n, int bpr, hipStream_t stream);

// Q5_K / Q6_K matvecs (f32 activations) and Q6_K on Q8_1 activations.
hipError_t gemv_q5k_launch(const uint8_t *w, const float *x, float *y, int n, int bpr,
                           hipStream_t stream);
hipError_t gemv_q6k_launch(const uint8_t *w, const float *x, float *y, int n, int bpr,
                           hipStream_t stream);
hipError_t gemv_q6k_q8_launch(const uint8_t *w, const int8_t *xq, const float *xd, float *y,
                              int n, int bpr, hipStream_t stream);

// Fused glue matvec: w_up == nullptr -> y = W * rms_norm(x) (norm_w not
// null) or W * x; w_up != nullptr -> y = act(W_gate*xn) .* (W_up*xn). All
// pointers 16-byte aligned (hipErrorNotSupported otherwise, as when the LDS
// staging does not fit).
hipError_t gemv_fused_launch(const uint8_t *w_gate, const uint8_t *w_up, const float *x,
                             const float *norm_w, float eps, int act, float *y, int n, int bpr,
                             hipStream_t stream);

// Standalone glue: RMSNorm over rows of `hidden`, and act(gate) * up.
hipError_t rms_norm_launch(const float *x, const float *w, float *y, int rows, int hidden,
                           float eps, hipStream_t stream);
hipError_t glu_launch(const float *gate, const float *up, float *out, int n, int act,
                      hipStream_t stream);
// h += x and h *= s, elementwise over n.
hipError_t residual_add_launch(float *h, const float *x, int n, hipStream_t stream);
hipError_t scale_launch(float *h, float s, int n, hipStream_t stream);

// Persistent decode-step chain (q4k_chain.hip): one cooperative launch runs
// a list of row-aligned Q4_K matvecs in order.
struct PersistentChain;
hipError_t chain_persistent_create(const mgq_gemv_desc *descs, int n, PersistentChain **out);
hipError_t chain_persistent_launch(PersistentChain *p, hipStream_t stream);
hipError_t chain_persistent_faults(PersistentChain *p, unsigned *faults);
hipError_t chain_persistent_destroy(PersistentChain *p);

hipError_t gemm_f16_launch(const uint8_t *w, const uint16_t *a, float *c, int n, int bpr,
                           int m_tokens, hipStream_t stream);
// One-time LDS attribute of the large-M GEMM kernel (safe to call often).
hipError_t gemm_prepare();

}  // namespace mgq
