// Batched Q4_K matvec that allocates nothing: launch_matvec_q4k_batched with
// its operand-table workspace taken from a fixed device array of this
// library instead of the caller. For callers that cannot allocate device
// memory (code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc).
//
// The array is a file-scope __device__ symbol: every GPU the library runs on
// holds its own copy, at its own address, until the process ends. Its name
// in host code is only a host-side stand-in, so the device address is looked
// up once per device (hipGetSymbolAddress, with that device current) and
// only that address is ever passed to kernels. Calls on one GPU share the
// array and keep the last call's contents; the table pass rewrites every
// byte a call reads (and zeroes Y itself where the main kernel accumulates),
// so nothing needs clearing between calls, but calls that overlap on one GPU
// (different streams, no ordering between them) race on the array.
#include "../../include/modgrad_q4k.h"
#include "q4k_launch.hpp"

#include <atomic>

constexpr size_t kScratchBytes = MGQ_NOALLOC_SCRATCH_BYTES;

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

// Device address of `scratch` per device ordinal (0 = not looked up yet).
std::atomic<uintptr_t> scratch_addr[64];

// The current device's address of `scratch`, looked up on first use.
hipError_t scratch_ptr(uint8_t **out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    uintptr_t p = scratch_addr[dev].load(std::memory_order_acquire);
    if (p == 0) {
        void *addr = nullptr;
        e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (addr == nullptr) return hipErrorInvalidSymbol;
        p = reinterpret_cast<uintptr_t>(addr);
        scratch_addr[dev].store(p, std::memory_order_release);
    }
    *out = reinterpret_cast<uint8_t *>(p);
    return hipSuccess;
}

}  // namespace

namespace mgq {
// Looks up the current device's scratch address (library init).
hipError_t noalloc_prepare() {
    uint8_t *p = nullptr;
    return scratch_ptr(&p);
}
}  // namespace mgq

extern "C" {

hipError_t launch_matvec_q4k_batched_noalloc(const unsigned char *w_q4, const float *X, float *Y,
                                             int out_dim, int blocks_per_row, int batch,
                                             hipStream_t stream) {
    if (out_dim <= 0 || blocks_per_row <= 0 || batch <= 0 || batch > 16) return hipErrorInvalidValue;
    if (!w_q4 || !X || !Y || ((uintptr_t)X & 3u) || ((uintptr_t)Y & 3u)) return hipErrorInvalidValue;
    if ((int64_t)blocks_per_row * 256 > 0x7FFFFFFFLL) return hipErrorInvalidValue;
    if (batch == 1)  // one activation row is a plain matvec: no table, no scratch
        return mgq::gemv_rows_launch(w_q4, X, Y, out_dim, blocks_per_row, stream);
    const size_t need = mgq::batched_workspace_bytes(blocks_per_row, batch);
    if (need > kScratchBytes) return hipErrorInvalidValue;  // beyond the fixed scratch
    uint8_t *ws = nullptr;
    const hipError_t e = scratch_ptr(&ws);
    if (e != hipSuccess) return e;
    const hipError_t m = mgq::gemv_batched_mfma_launch(w_q4, X, Y, out_dim, blocks_per_row, batch,
                                                       ws, kScratchBytes, stream);
    if (m != hipErrorNotSupported) return m;
    return mgq::gemv_batched_launch(w_q4, X, Y, out_dim, blocks_per_row, batch, stream);
}

}  // extern "C"
