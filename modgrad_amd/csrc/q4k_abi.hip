// C ABI of libmodgrad_q4k (declarations and contracts: include/modgrad_q4k.h).
//
// Reference-compatible launchers keep the reference's conventions
// (matvec_q4k.hip:110-124, dequant_q4k.hip:147-157): null stream, no
// synchronization, hipErrorInvalidValue on non-positive sizes, otherwise the
// launch status from hipGetLastError(). Quantized weight bytes (and int8
// activations) may start at any byte, as the reference's byte-reading
// kernels allow; float pointers need float (4-byte) alignment, f16 ones 2.
#include "../../include/modgrad_q4k.h"
#include "q4k_launch.hpp"

#include <cstdlib>
#include <cstring>
#include <new>
#include <vector>

namespace {

constexpr int64_t kMaxI32 = 0x7FFFFFFF;

bool misaligned4(const void *p) { return ((uintptr_t)p & 3u) != 0; }

}  // namespace

extern "C" {

hipError_t launch_dequant_q4k_ex(const unsigned char *q4k, int n_blocks, float *fp32_out,
                                 hipStream_t stream) {
    if (n_blocks <= 0 || !q4k || !fp32_out) return hipErrorInvalidValue;
    if (misaligned4(fp32_out)) return hipErrorInvalidValue;
    if ((int64_t)n_blocks * 32 > kMaxI32 * 256LL) return hipErrorInvalidValue;
    return mgq::dequant_launch(q4k, n_blocks, fp32_out, stream);
}

hipError_t launch_dequant_q4k(const unsigned char *q4k, int n_blocks, float *fp32_out) {
    return launch_dequant_q4k_ex(q4k, n_blocks, fp32_out, nullptr);
}

hipError_t launch_matvec_q4k_ex(const unsigned char *w_q4, const float *x, float *y,
                                int out_dim, int k_elems, int layout, hipStream_t stream) {
    if (out_dim <= 0 || k_elems <= 0 || !w_q4 || !x || !y) return hipErrorInvalidValue;
    if (misaligned4(x) || misaligned4(y)) return hipErrorInvalidValue;
    if (layout == MGQ_LAYOUT_ROWS) {
        if (k_elems % 256 != 0) return hipErrorInvalidValue;
        return mgq::gemv_rows_launch(w_q4, x, y, out_dim, k_elems / 256, stream);
    }
    if (layout == MGQ_LAYOUT_FLAT) {
        if (((int64_t)out_dim * k_elems) % 256 != 0) return hipErrorInvalidValue;
        if (k_elems % 256 == 0)
            return mgq::gemv_rows_launch(w_q4, x, y, out_dim, k_elems / 256, stream);
        const hipError_t e = mgq::gemv_flat_launch(w_q4, x, y, out_dim, k_elems, stream);
        if (e != hipErrorNotSupported) return e;
        return mgq::gemv_generic_launch(w_q4, x, y, out_dim, k_elems, stream);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_matvec_q4k(const unsigned char *w_q4, const float *x, float *y, int out_dim,
                             int blocks_per_row) {
    if (out_dim <= 0 || blocks_per_row <= 0) return hipErrorInvalidValue;
    if ((int64_t)blocks_per_row * 256 > kMaxI32) return hipErrorInvalidValue;
    return launch_matvec_q4k_ex(w_q4, x, y, out_dim, blocks_per_row * 256, MGQ_LAYOUT_ROWS,
                                nullptr);
}

size_t mgq_batched_workspace_bytes(int blocks_per_row, int batch) {
    if (blocks_per_row <= 0 || batch <= 0 || batch > 16) return 0;
    return mgq::batched_workspace_bytes(blocks_per_row, batch);
}

hipError_t launch_matvec_q4k_batched(const unsigned char *w_q4, const float *X, float *Y,
                                     int out_dim, int blocks_per_row, int batch,
                                     void *workspace, size_t workspace_bytes,
                                     hipStream_t stream) {
    if (out_dim <= 0 || blocks_per_row <= 0 || batch <= 0 || batch > 16) return hipErrorInvalidValue;
    if (!w_q4 || !X || !Y || misaligned4(X) || misaligned4(Y))
        return hipErrorInvalidValue;
    if ((int64_t)blocks_per_row * 256 > kMaxI32) return hipErrorInvalidValue;
    if (!workspace || workspace_bytes < mgq::batched_workspace_bytes(blocks_per_row, batch))
        return hipErrorInvalidValue;
    if (batch == 1)  // one activation row is a plain matvec: no operand-table pass
        return mgq::gemv_rows_launch(w_q4, X, Y, out_dim, blocks_per_row, stream);
    const hipError_t e = mgq::gemv_batched_mfma_launch(w_q4, X, Y, out_dim, blocks_per_row, batch,
                                                       workspace, workspace_bytes, stream);
    if (e != hipErrorNotSupported) return e;
    return mgq::gemv_batched_launch(w_q4, X, Y, out_dim, blocks_per_row, batch, stream);
}

hipError_t launch_quantize_q8_1_ex(const float *x, signed char *xq, float *xd, float *xsum, int n,
                                   hipStream_t stream) {
    if (n < 32) return hipErrorInvalidValue;
    if (!x || !xq || !xd || !xsum || misaligned4(x) || misaligned4(xd) || misaligned4(xsum))
        return hipErrorInvalidValue;
    return mgq::quantize_q8_1_launch(x, reinterpret_cast<int8_t *>(xq), xd, xsum, n, stream);
}

hipError_t launch_quantize_q8_1(const float *x, signed char *xq, float *xd, float *xsum, int n) {
    return launch_quantize_q8_1_ex(x, xq, xd, xsum, n, nullptr);
}

hipError_t launch_matvec_q4k_dp4a_ex(const unsigned char *w, const signed char *xq,
                                     const float *xd, const float *xsum, float *y, int out_dim,
                                     int bpr, hipStream_t stream) {
    if (out_dim <= 0 || bpr <= 0) return hipErrorInvalidValue;
    if (!w || !xq || !xd || !xsum || !y || misaligned4(xd) || misaligned4(xsum) || misaligned4(y))
        return hipErrorInvalidValue;
    if ((int64_t)bpr * 256 > kMaxI32) return hipErrorInvalidValue;
    return mgq::gemv_q8_launch(w, reinterpret_cast<const int8_t *>(xq), xd, xsum, y, out_dim, bpr,
                               stream);
}

hipError_t launch_matvec_q4k_dp4a(const unsigned char *w, const signed char *xq, const float *xd,
                                  const float *xsum, float *y, int out_dim, int bpr) {
    return launch_matvec_q4k_dp4a_ex(w, xq, xd, xsum, y, out_dim, bpr, nullptr);
}

static hipError_t check_kquant(const unsigned char *w, const float *x, const float *y,
                               int out_dim, int bpr) {
    if (out_dim <= 0 || bpr <= 0) return hipErrorInvalidValue;
    if (!w || !x || !y || misaligned4(x) || misaligned4(y)) return hipErrorInvalidValue;
    if ((int64_t)bpr * 256 > kMaxI32) return hipErrorInvalidValue;
    return hipSuccess;
}

hipError_t launch_quantize_matvec_q4k_dp4a_ex(const unsigned char *w, const float *x, float *y,
                                              int out_dim, int bpr, hipStream_t stream) {
    if (out_dim <= 0 || bpr <= 0 || !w || !x || !y) return hipErrorInvalidValue;
    if ((int64_t)bpr * 256 > kMaxI32) return hipErrorInvalidValue;
    if (misaligned4(x) || misaligned4(y)) return hipErrorInvalidValue;
    return mgq::gemv_q8x_launch(w, x, y, out_dim, bpr, stream);
}

hipError_t launch_matvec_q5k_ex(const unsigned char *w_q5, const float *x, float *y, int out_dim,
                                int blocks_per_row, hipStream_t stream) {
    const hipError_t e = check_kquant(w_q5, x, y, out_dim, blocks_per_row);
    return e != hipSuccess ? e : mgq::gemv_q5k_launch(w_q5, x, y, out_dim, blocks_per_row, stream);
}

hipError_t launch_matvec_q5k(const unsigned char *w_q5, const float *x, float *y, int out_dim,
                             int blocks_per_row) {
    return launch_matvec_q5k_ex(w_q5, x, y, out_dim, blocks_per_row, nullptr);
}

hipError_t launch_matvec_q6k_ex(const unsigned char *w_q6, const float *x, float *y, int out_dim,
                                int blocks_per_row, hipStream_t stream) {
    const hipError_t e = check_kquant(w_q6, x, y, out_dim, blocks_per_row);
    return e != hipSuccess ? e : mgq::gemv_q6k_launch(w_q6, x, y, out_dim, blocks_per_row, stream);
}

hipError_t launch_matvec_q6k(const unsigned char *w_q6, const float *x, float *y, int out_dim,
                             int blocks_per_row) {
    return launch_matvec_q6k_ex(w_q6, x, y, out_dim, blocks_per_row, nullptr);
}

hipError_t launch_matvec_q6k_dp4a_ex(const unsigned char *w, const signed char *xq,
                                     const float *xd, const float *xsum, float *y, int out_dim,
                                     int bpr, hipStream_t stream) {
    (void)xsum;  // part of the reference signature; the Q6_K formula has no min term
    if (out_dim <= 0 || bpr <= 0) return hipErrorInvalidValue;
    if (!w || !xq || !xd || !y || misaligned4(xd) || misaligned4(y)) return hipErrorInvalidValue;
    if ((int64_t)bpr * 256 > kMaxI32) return hipErrorInvalidValue;
    return mgq::gemv_q6k_q8_launch(w, reinterpret_cast<const int8_t *>(xq), xd, y, out_dim, bpr,
                                   stream);
}

hipError_t launch_matvec_q6k_dp4a(const unsigned char *w, const signed char *xq, const float *xd,
                                  const float *xsum, float *y, int out_dim, int bpr) {
    return launch_matvec_q6k_dp4a_ex(w, xq, xd, xsum, y, out_dim, bpr, nullptr);
}

hipError_t launch_gemm_q4k_f16(const unsigned char *w_q4, const uint16_t *a_f16, float *c,
                               int out_dim, int blocks_per_row, int m_tokens,
                               hipStream_t stream) {
    if (out_dim <= 0 || blocks_per_row <= 0 || m_tokens <= 0) return hipErrorInvalidValue;
    if (!w_q4 || !a_f16 || !c || ((uintptr_t)a_f16 & 1u) || misaligned4(c))
        return hipErrorInvalidValue;
    if ((int64_t)blocks_per_row * 256 > kMaxI32) return hipErrorInvalidValue;
    return mgq::gemm_f16_launch(w_q4, a_f16, c, out_dim, blocks_per_row, m_tokens, stream);
}

// ------------------------------------------------------ decode-step chain --

struct mgq_chain {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    mgq::PersistentChain *pers = nullptr;
    std::vector<mgq_gemv_desc> eager;  // MGQ_CHAIN_EAGER: launched one by one
};

}  // extern "C"

// Records launches 0..n-1 (enqueue(i, stream)) into a HIP graph through
// stream capture on a private stream, and instantiates it.
template <class F>
static hipError_t chain_record(int n, void **chain_out, F enqueue) {
    hipStream_t s = nullptr;
    hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (e != hipSuccess) return e;
    auto *ch = new (std::nothrow) mgq_chain;
    if (!ch) {
        hipStreamDestroy(s);
        return hipErrorOutOfMemory;
    }
    e = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
    hipError_t launch_err = hipSuccess;
    if (e == hipSuccess) {
        for (int i = 0; i < n && launch_err == hipSuccess; ++i) launch_err = enqueue(i, s);
        hipGraph_t g = nullptr;
        e = hipStreamEndCapture(s, &g);
        ch->graph = g;
        if (e == hipSuccess) e = launch_err;
        if (e == hipSuccess) e = hipGraphInstantiate(&ch->exec, ch->graph, nullptr, nullptr, 0);
    }
    hipStreamDestroy(s);
    if (e != hipSuccess) {
        if (ch->exec) hipGraphExecDestroy(ch->exec);
        if (ch->graph) hipGraphDestroy(ch->graph);
        delete ch;
        return e;
    }
    *chain_out = ch;
    return hipSuccess;
}

extern "C" {

static bool env_chain_persistent() {
    const char *s = std::getenv("MGQ_CHAIN");
    return s && std::strcmp(s, "persistent") == 0;
}

hipError_t mgq_chain_create_ex(const mgq_gemv_desc *descs, int n, int mode, void **chain_out) {
    if (!chain_out || !descs || n <= 0) return hipErrorInvalidValue;
    if (mode != MGQ_CHAIN_AUTO && mode != MGQ_CHAIN_GRAPH && mode != MGQ_CHAIN_PERSISTENT &&
        mode != MGQ_CHAIN_EAGER)
        return hipErrorInvalidValue;
    *chain_out = nullptr;
    for (int i = 0; i < n; ++i) {
        const mgq_gemv_desc &d = descs[i];
        if (d.out_dim <= 0 || d.blocks_per_row <= 0 || !d.w_q4 || !d.x || !d.y)
            return hipErrorInvalidValue;
        if (misaligned4(d.x) || misaligned4(d.y)) return hipErrorInvalidValue;
        if ((int64_t)d.blocks_per_row * 256 > kMaxI32) return hipErrorInvalidValue;
    }
    hipError_t e = mgq::gemv_prepare();  // not allowed to happen mid-capture
    if (e != hipSuccess) return e;
    if (mode == MGQ_CHAIN_EAGER) {
        auto *ch = new (std::nothrow) mgq_chain;
        if (!ch) return hipErrorOutOfMemory;
        try {
            ch->eager.assign(descs, descs + n);
        } catch (...) {
            delete ch;
            return hipErrorOutOfMemory;
        }
        *chain_out = ch;
        return hipSuccess;
    }
    if (mode == MGQ_CHAIN_PERSISTENT || (mode == MGQ_CHAIN_AUTO && env_chain_persistent())) {
        mgq::PersistentChain *p = nullptr;
        e = mgq::chain_persistent_create(descs, n, &p);
        if (e == hipSuccess) {
            auto *ch = new (std::nothrow) mgq_chain;
            if (!ch) {
                mgq::chain_persistent_destroy(p);
                return hipErrorOutOfMemory;
            }
            ch->pers = p;
            *chain_out = ch;
            return hipSuccess;
        }
        if (mode == MGQ_CHAIN_PERSISTENT) return e;
    }
    return chain_record(n, chain_out, [descs](int i, hipStream_t s) {
        const mgq_gemv_desc &d = descs[i];
        return launch_matvec_q4k_ex(d.w_q4, d.x, d.y, d.out_dim, d.blocks_per_row * 256,
                                    MGQ_LAYOUT_ROWS, s);
    });
}

// ---------------------------------------------------------- op chains --

static bool bad_f32(const float *p) { return !p || misaligned4(p); }

// The fused RMSNorm -> Q6_K matvec runs on the whole-row matrix-core kernel
// only: 16-byte aligned w, a tensor of whole 16-byte chunks, K <= 14 blocks.
static bool q6k_norm_fits(const unsigned char *w, int out_dim, int bpr) {
    return ((uintptr_t)w & 15u) == 0 && ((int64_t)out_dim * bpr * 210) % 16 == 0 && bpr <= 14;
}

// Host-side checks of one op descriptor (the launchers check again).
static hipError_t op_check(const mgq_op_desc &o) {
    switch (o.op) {
    case MGQ_OP_MATVEC:
        if (!o.w || bad_f32(o.x) || bad_f32(o.y) || o.out_dim <= 0 || o.in_dim <= 0)
            return hipErrorInvalidValue;
        if (o.dtype == MGQ_DTYPE_Q4_K) {
            if (o.layout != MGQ_LAYOUT_ROWS && o.layout != MGQ_LAYOUT_FLAT) return hipErrorInvalidValue;
            if (o.layout == MGQ_LAYOUT_ROWS && o.in_dim % 256) return hipErrorInvalidValue;
            if (o.layout == MGQ_LAYOUT_FLAT && ((int64_t)o.out_dim * o.in_dim) % 256)
                return hipErrorInvalidValue;
            return hipSuccess;
        }
        if (o.dtype != MGQ_DTYPE_Q5_K && o.dtype != MGQ_DTYPE_Q6_K) return hipErrorInvalidValue;
        return o.in_dim % 256 ? hipErrorInvalidValue : hipSuccess;
    case MGQ_OP_MATVEC_NORM:
        if (o.dtype == MGQ_DTYPE_Q6_K) {
            if (!o.w || bad_f32(o.x) || bad_f32(o.y) || bad_f32(o.norm_w) || o.out_dim <= 0 ||
                o.in_dim <= 0 || o.in_dim % 256)
                return hipErrorInvalidValue;
            return q6k_norm_fits(o.w, o.out_dim, o.in_dim / 256) ? hipSuccess : hipErrorNotSupported;
        }
        [[fallthrough]];
    case MGQ_OP_MATVEC_GLU: {
        if (o.dtype != MGQ_DTYPE_Q4_K || !o.w || bad_f32(o.x) || bad_f32(o.y)) return hipErrorInvalidValue;
        if (o.out_dim <= 0 || o.in_dim <= 0 || o.in_dim % 256) return hipErrorInvalidValue;
        if (o.op == MGQ_OP_MATVEC_NORM) return bad_f32(o.norm_w) ? hipErrorInvalidValue : hipSuccess;
        if (!o.w2 || (o.norm_w && misaligned4(o.norm_w))) return hipErrorInvalidValue;
        return (o.act == MGQ_ACT_GELU_TANH || o.act == MGQ_ACT_SILU) ? hipSuccess : hipErrorInvalidValue;
    }
    case MGQ_OP_RMS_NORM:
        if (bad_f32(o.x) || bad_f32(o.y) || bad_f32(o.norm_w) || o.rows <= 0 || o.in_dim <= 0)
            return hipErrorInvalidValue;
        return (int64_t)o.rows * o.in_dim > kMaxI32 * 4LL ? hipErrorInvalidValue : hipSuccess;
    case MGQ_OP_GLU:
        if (bad_f32(o.x) || bad_f32(o.x2) || bad_f32(o.y) || o.out_dim <= 0) return hipErrorInvalidValue;
        return (o.act == MGQ_ACT_GELU_TANH || o.act == MGQ_ACT_SILU) ? hipSuccess : hipErrorInvalidValue;
    case MGQ_OP_RESIDUAL_ADD:
        return (bad_f32(o.x) || bad_f32(o.y) || o.out_dim <= 0) ? hipErrorInvalidValue : hipSuccess;
    case MGQ_OP_QUANTIZE_Q8_1:
        if (bad_f32(o.x) || !o.xq || bad_f32(o.xd) || bad_f32(o.xsum) || o.in_dim < 32 || o.in_dim % 32)
            return hipErrorInvalidValue;
        return hipSuccess;
    case MGQ_OP_MATVEC_DP4A:
        if (!o.w || !o.xq || bad_f32(o.xd) || bad_f32(o.y) || o.out_dim <= 0 || o.in_dim <= 0 ||
            o.in_dim % 256)
            return hipErrorInvalidValue;
        if (o.dtype == MGQ_DTYPE_Q4_K) return bad_f32(o.xsum) ? hipErrorInvalidValue : hipSuccess;
        return o.dtype == MGQ_DTYPE_Q6_K ? hipSuccess : hipErrorInvalidValue;
    case MGQ_OP_QUANTIZE_MATVEC_DP4A:
        if (o.dtype != MGQ_DTYPE_Q4_K || !o.w || bad_f32(o.x) || bad_f32(o.y) || o.out_dim <= 0 ||
            o.in_dim <= 0 || o.in_dim % 256)
            return hipErrorInvalidValue;
        return hipSuccess;
    default:
        return hipErrorInvalidValue;
    }
}

static hipError_t op_launch(const mgq_op_desc &o, hipStream_t s) {
    switch (o.op) {
    case MGQ_OP_MATVEC:
        if (o.dtype == MGQ_DTYPE_Q4_K)
            return launch_matvec_q4k_ex(o.w, o.x, o.y, o.out_dim, o.in_dim, o.layout, s);
        if (o.dtype == MGQ_DTYPE_Q5_K)
            return launch_matvec_q5k_ex(o.w, o.x, o.y, o.out_dim, o.in_dim / 256, s);
        return launch_matvec_q6k_ex(o.w, o.x, o.y, o.out_dim, o.in_dim / 256, s);
    case MGQ_OP_MATVEC_NORM:
        if (o.dtype == MGQ_DTYPE_Q6_K)
            return launch_matvec_q6k_rmsnorm_ex(o.w, o.x, o.norm_w, o.eps, o.y, o.out_dim,
                                                o.in_dim / 256, s);
        return launch_matvec_q4k_rmsnorm_ex(o.w, o.x, o.norm_w, o.eps, o.y, o.out_dim,
                                            o.in_dim / 256, s);
    case MGQ_OP_MATVEC_GLU:
        return launch_matvec_q4k_glu_ex(o.w, o.w2, o.x, o.norm_w, o.eps, o.act, o.y, o.out_dim,
                                        o.in_dim / 256, s);
    case MGQ_OP_RMS_NORM:
        return launch_rms_norm_ex(o.x, o.norm_w, o.y, o.rows, o.in_dim, o.eps, s);
    case MGQ_OP_GLU:
        return launch_glu_ex(o.x, o.x2, o.y, o.out_dim, o.act, s);
    case MGQ_OP_QUANTIZE_Q8_1:
        return launch_quantize_q8_1_ex(o.x, o.xq, o.xd, o.xsum, o.in_dim, s);
    case MGQ_OP_MATVEC_DP4A:
        if (o.dtype == MGQ_DTYPE_Q4_K)
            return launch_matvec_q4k_dp4a_ex(o.w, o.xq, o.xd, o.xsum, o.y, o.out_dim, o.in_dim / 256, s);
        return launch_matvec_q6k_dp4a_ex(o.w, o.xq, o.xd, o.xsum, o.y, o.out_dim, o.in_dim / 256, s);
    case MGQ_OP_QUANTIZE_MATVEC_DP4A:
        return launch_quantize_matvec_q4k_dp4a_ex(o.w, o.x, o.y, o.out_dim, o.in_dim / 256, s);
    default:
        return launch_residual_add_ex(o.y, o.x, o.out_dim, s);
    }
}

hipError_t mgq_chain_create_ops(const mgq_op_desc *ops, int n, void **chain_out) {
    if (!chain_out || !ops || n <= 0) return hipErrorInvalidValue;
    *chain_out = nullptr;
    for (int i = 0; i < n; ++i) {
        const hipError_t e = op_check(ops[i]);
        if (e != hipSuccess) return e;
    }
    hipError_t e = mgq::gemv_prepare();  // not allowed to happen mid-capture
    if (e != hipSuccess) return e;
    return chain_record(n, chain_out, [ops](int i, hipStream_t s) { return op_launch(ops[i], s); });
}

hipError_t mgq_chain_create(const mgq_gemv_desc *descs, int n, void **chain_out) {
    return mgq_chain_create_ex(descs, n, MGQ_CHAIN_AUTO, chain_out);
}

hipError_t mgq_chain_launch(void *chain, hipStream_t stream) {
    if (!chain) return hipErrorInvalidValue;
    auto *ch = static_cast<mgq_chain *>(chain);
    if (ch->pers) return mgq::chain_persistent_launch(ch->pers, stream);
    if (!ch->exec) {  // eager: the reference's one-launch-per-matvec pattern
        for (const mgq_gemv_desc &d : ch->eager) {
            const hipError_t e = launch_matvec_q4k_ex(d.w_q4, d.x, d.y, d.out_dim,
                                                      d.blocks_per_row * 256, MGQ_LAYOUT_ROWS, stream);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    return hipGraphLaunch(ch->exec, stream);
}

hipError_t mgq_chain_info(void *chain, int *mode, unsigned *faults) {
    if (!chain) return hipErrorInvalidValue;
    auto *ch = static_cast<mgq_chain *>(chain);
    if (mode) *mode = ch->pers ? MGQ_CHAIN_PERSISTENT : ch->exec ? MGQ_CHAIN_GRAPH : MGQ_CHAIN_EAGER;
    if (faults) {
        *faults = 0;
        if (ch->pers) return mgq::chain_persistent_faults(ch->pers, faults);
    }
    return hipSuccess;
}

hipError_t mgq_chain_destroy(void *chain) {
    if (!chain) return hipErrorInvalidValue;
    auto *ch = static_cast<mgq_chain *>(chain);
    if (ch->pers) {
        const hipError_t e = mgq::chain_persistent_destroy(ch->pers);
        delete ch;
        return e;
    }
    hipError_t e1 = ch->exec ? hipGraphExecDestroy(ch->exec) : hipSuccess;
    hipError_t e2 = ch->graph ? hipGraphDestroy(ch->graph) : hipSuccess;
    delete ch;
    return e1 != hipSuccess ? e1 : e2;
}

hipError_t launch_rms_norm_ex(const float *x, const float *weight, float *y, int n, int hidden,
                              float eps, hipStream_t stream) {
    if (n <= 0 || hidden <= 0 || !x || !weight || !y) return hipErrorInvalidValue;
    if ((int64_t)n * hidden > kMaxI32 * 4LL) return hipErrorInvalidValue;
    return mgq::rms_norm_launch(x, weight, y, n, hidden, eps, stream);
}

hipError_t launch_rms_norm(const float *x, const float *weight, float *y, int n, int hidden,
                           float eps) {
    return launch_rms_norm_ex(x, weight, y, n, hidden, eps, nullptr);
}

hipError_t launch_glu_ex(const float *gate, const float *up, float *out, int n, int act,
                         hipStream_t stream) {
    if (n <= 0 || !gate || !up || !out) return hipErrorInvalidValue;
    if (act != MGQ_ACT_GELU_TANH && act != MGQ_ACT_SILU) return hipErrorInvalidValue;
    return mgq::glu_launch(gate, up, out, n, act, stream);
}

hipError_t launch_geglu(const float *gate, const float *up, float *out, int n) {
    return launch_glu_ex(gate, up, out, n, MGQ_ACT_GELU_TANH, nullptr);
}

hipError_t launch_residual_add_ex(float *h, const float *x, int n, hipStream_t stream) {
    if (n <= 0 || !h || !x) return hipErrorInvalidValue;
    return mgq::residual_add_launch(h, x, n, stream);
}

hipError_t launch_residual_add(float *h, const float *x, int n) {
    return launch_residual_add_ex(h, x, n, nullptr);
}

hipError_t launch_scale_ex(float *h, float s, int n, hipStream_t stream) {
    if (n <= 0 || !h) return hipErrorInvalidValue;
    return mgq::scale_launch(h, s, n, stream);
}

hipError_t launch_scale(float *h, float s, int n) { return launch_scale_ex(h, s, n, nullptr); }

hipError_t launch_matvec_q4k_rmsnorm_ex(const unsigned char *w_q4, const float *x,
                                        const float *norm_w, float eps, float *y, int out_dim,
                                        int blocks_per_row, hipStream_t stream) {
    if (out_dim <= 0 || blocks_per_row <= 0 || !w_q4 || !x || !norm_w || !y)
        return hipErrorInvalidValue;
    if ((int64_t)blocks_per_row * 256 > kMaxI32) return hipErrorInvalidValue;
    if (misaligned4(x) || misaligned4(norm_w) || misaligned4(y))
        return hipErrorInvalidValue;
    return mgq::gemv_fused_launch(w_q4, nullptr, x, norm_w, eps, MGQ_ACT_GELU_TANH, y, out_dim,
                                  blocks_per_row, stream);
}

hipError_t launch_matvec_q6k_rmsnorm_ex(const unsigned char *w_q6, const float *x,
                                        const float *norm_w, float eps, float *y, int out_dim,
                                        int blocks_per_row, hipStream_t stream) {
    const hipError_t e = check_kquant(w_q6, x, y, out_dim, blocks_per_row);
    if (e != hipSuccess) return e;
    if (!norm_w || misaligned4(norm_w)) return hipErrorInvalidValue;
    return mgq::gemv_q6k_mfma_norm_launch(w_q6, x, norm_w, eps, y, out_dim, blocks_per_row, stream);
}

hipError_t launch_matvec_q4k_glu_ex(const unsigned char *w_gate, const unsigned char *w_up,
                                    const float *x, const float *norm_w, float eps, int act,
                                    float *y, int out_dim, int blocks_per_row,
                                    hipStream_t stream) {
    if (out_dim <= 0 || blocks_per_row <= 0 || !w_gate || !w_up || !x || !y)
        return hipErrorInvalidValue;
    if (act != MGQ_ACT_GELU_TANH && act != MGQ_ACT_SILU) return hipErrorInvalidValue;
    if ((int64_t)blocks_per_row * 256 > kMaxI32) return hipErrorInvalidValue;
    if (misaligned4(x) || (norm_w && misaligned4(norm_w)) || misaligned4(y))
        return hipErrorInvalidValue;
    return mgq::gemv_fused_launch(w_gate, w_up, x, norm_w, eps, act, y, out_dim, blocks_per_row,
                                  stream);
}

hipError_t mgq_prepare(void) {
    hipError_t e = mgq::gemv_prepare();
    if (e == hipSuccess) e = mgq::gemm_prepare();
    return e != hipSuccess ? e : mgq::noalloc_prepare();
}

const char *mgq_version(void) { return "modgrad_q4k 0.1.0 gfx950"; }

}  // extern "C"
