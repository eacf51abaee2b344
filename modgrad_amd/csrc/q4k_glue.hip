// Decode glue around the matvecs (kernels/rms_norm.hip, kernels/
// transformer_ops.hip:32-46): RMSNorm and the gated-linear-unit product.
// Standalone versions under the reference's names; the matvec also runs them
// fused (q4k_gemv.hip: RMSNorm in the activation staging, the GLU on the
// gate/up results).
#include "q4k_device.hpp"
#include "q4k_launch.hpp"

namespace mgq {

// y[r][c] = (x[r][c] * rstd) * w[c], rstd = 1/sqrt(mean(x[r]^2) + eps), one
// 256-thread work-group per row. The sum of squares follows the reference's
// order (thread t sums c = t, t+256, ...; then a pairwise tree t += t+128,
// t+64, ..., 1), so it matches the reference bit for bit; the tree's last six
// levels run inside one wavefront (DPP row shifts via shfl_down).
// Elements per thread whose loads are all issued before the first is used
// (hidden <= 4096 is one such chunk: one memory latency per pass instead of
// one per element).
constexpr int kNormPT = 16;

__global__ __launch_bounds__(256) void rms_norm_kernel(const float *__restrict__ x,
                                                       const float *__restrict__ w,
                                                       float *__restrict__ y, int hidden,
                                                       float eps) {
    __shared__ float part[256];
    const int tid = threadIdx.x;
    const float *xr = x + (size_t)blockIdx.x * hidden;
    float *yr = y + (size_t)blockIdx.x * hidden;
    // sum of squares in the order c = tid, tid + 256, ... (one fmaf each;
    // elements past the end load as 0 and leave the sum unchanged)
    float xv[kNormPT], wv[kNormPT];
    float s = 0.0f;
    const bool one = hidden <= 256 * kNormPT;  // uniform: x stays in registers
    for (int c0 = 0; c0 < hidden; c0 += 256 * kNormPT) {
#pragma unroll
        for (int i = 0; i < kNormPT; ++i) {
            const int c = c0 + tid + 256 * i;
            xv[i] = c < hidden ? xr[c] : 0.0f;
        }
        if (one) {
#pragma unroll
            for (int i = 0; i < kNormPT; ++i) {
                const int c = tid + 256 * i;
                wv[i] = c < hidden ? w[c] : 0.0f;  // in flight during the reduction
            }
        }
#pragma unroll
        for (int i = 0; i < kNormPT; ++i) s = fmaf(xv[i], xv[i], s);
    }
    part[tid] = s;
    __syncthreads();
    if (tid < 128) part[tid] += part[tid + 128];
    __syncthreads();
    if (tid < 64) {
        float v = part[tid] + part[tid + 64];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) v += __shfl_down(v, off, 64);
        if (tid == 0) part[0] = v;
    }
    __syncthreads();
    const float rstd = rsqrtf(part[0] / (float)hidden + eps);
    if (one) {
#pragma unroll
        for (int i = 0; i < kNormPT; ++i) {
            const int c = tid + 256 * i;
            if (c < hidden) yr[c] = xv[i] * rstd * wv[i];
        }
        return;
    }
    for (int c0 = 0; c0 < hidden; c0 += 256 * kNormPT) {
#pragma unroll
        for (int i = 0; i < kNormPT; ++i) {
            const int c = c0 + tid + 256 * i;
            xv[i] = c < hidden ? xr[c] : 0.0f;
            wv[i] = c < hidden ? w[c] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < kNormPT; ++i) {
            const int c = c0 + tid + 256 * i;
            if (c < hidden) yr[c] = xv[i] * rstd * wv[i];
        }
    }
}

hipError_t rms_norm_launch(const float *x, const float *w, float *y, int rows, int hidden,
                           float eps, hipStream_t stream) {
    rms_norm_kernel<<<(unsigned)rows, 256, 0, stream>>>(x, w, y, hidden, eps);
    return hipGetLastError();
}

// out[i] = act(gate[i]) * up[i]
__global__ __launch_bounds__(256) void glu_kernel(const float *__restrict__ gate,
                                                  const float *__restrict__ up,
                                                  float *__restrict__ out, int n, int act) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = glu_act(gate[i], act) * up[i];
}

hipError_t glu_launch(const float *gate, const float *up, float *out, int n, int act,
                      hipStream_t stream) {
    glu_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(gate, up, out, n, act);
    return hipGetLastError();
}

// h[i] += x[i] (kernels/transformer_ops.hip:10-19): the residual add after the
// attention and FFN projections, and the bias add of a resident linear layer.
__global__ __launch_bounds__(256) void residual_add_kernel(float *__restrict__ h,
                                                           const float *__restrict__ x, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) h[i] += x[i];
}

hipError_t residual_add_launch(float *h, const float *x, int n, hipStream_t stream) {
    residual_add_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(h, x, n);
    return hipGetLastError();
}

// h[i] *= s (kernels/transformer_ops.hip:21-30).
__global__ __launch_bounds__(256) void scale_kernel(float *__restrict__ h, float s, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) h[i] *= s;
}

hipError_t scale_launch(float *h, float s, int n, hipStream_t stream) {
    scale_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(h, s, n);
    return hipGetLastError();
}

}  // namespace mgq
