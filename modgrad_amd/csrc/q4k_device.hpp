// Device-side helpers shared by the Q4_K kernels (gfx950 / CDNA4).
//
// Q4_K super-block, 144 bytes = 9 x 16 B: dword 0 = {d:f16, dmin:f16},
// dwords 1..3 = scales[12], dwords 4..35 = qs[128]. Canonical (ggml) order:
// qs byte t holds the low nibble of position 64*(t/32) + t%32 (sub-block
// 2*(t/32)) and the high nibble of that position + 32 (sub-block 2*(t/32)+1).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mgq {

constexpr int kBlockBytes = 144;
constexpr int kBlockElems = 256;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// IEEE half bits -> f32, with exponent 31 (Inf and NaN) mapped to 0, the
// reference's treatment of d/dmin (gguf.rs:371-372, matvec_q4k.hip:78-79).
// The hardware conversion is exact for every finite half (f16 denormals are
// enabled in the default FP mode), so this equals the reference's
// bit-level f16_to_f32 (gguf.rs:281-292) on every finite input.
__device__ __forceinline__ float half_bits_finite(uint32_t h) {
    _Float16 hv = __builtin_bit_cast(_Float16, (uint16_t)(h & 0xFFFFu));
    float f = (float)hv;
    return ((h & 0x7C00u) == 0x7C00u) ? 0.0f : f;
}

// 6-bit scale and min of sub-block j from the header's scale dwords
// s0 = bytes 4..7, s1 = bytes 8..11, s2 = bytes 12..15 (gguf.rs:334-342).
__device__ __forceinline__ void scale_min(int j, uint32_t s0, uint32_t s1, uint32_t s2,
                                          uint32_t &sc, uint32_t &m) {
    if (j < 4) {
        sc = (s0 >> (8 * j)) & 63u;
        m = (s1 >> (8 * j)) & 63u;
    } else {
        const int jj = 8 * (j - 4);
        const uint32_t c = (s2 >> jj) & 0xFFu;
        sc = (c & 15u) | (((s0 >> jj) >> 6 & 3u) << 4);
        m = (c >> 4) | (((s1 >> jj) >> 6 & 3u) << 4);
    }
}

// All four scales (or mins) of sub-blocks 4j..4j+3 as bytes of one dword,
// from the header's scale dwords (byte-parallel form of scale_min).
__device__ __forceinline__ uint32_t scales4(int j, uint32_t s0, uint32_t s2) {
    return j == 0 ? (s0 & 0x3F3F3F3Fu)
                  : ((s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u));
}
__device__ __forceinline__ uint32_t mins4(int j, uint32_t s1, uint32_t s2) {
    return j == 0 ? (s1 & 0x3F3F3F3Fu)
                  : (((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u));
}

// Loads of caller data at any byte alignment. The reference reads weight
// bytes one at a time and accepts any address (matvec_q4k.hip:66-96), and its
// engine packs tensors back to back in one arena (rocm_gemma.rs:214-215), so
// a tensor can start at any byte. The types below carry alignment 1 (floats:
// 4); for gfx950 under the HSA ABI, which runs with unaligned access enabled,
// the compiler still emits single global_load_dword / _dwordx4 instructions,
// so an aligned pointer costs nothing extra and a misaligned one stays
// correct.
typedef uint32_t u32_a1 __attribute__((aligned(1)));
typedef uint32_t u32x4_a1 __attribute__((ext_vector_type(4), aligned(1)));
typedef uint32_t u32x2_a1 __attribute__((ext_vector_type(2), aligned(1)));
typedef float f32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

__device__ __forceinline__ uint32_t ld_u32(const uint8_t *p) {
    return *reinterpret_cast<const u32_a1 *>(p);
}
// Word 3 of a raw buffer resource (stride 0, 32-bit data format): offsets
// are in bytes, and a read at or past num_records returns zeros.
constexpr int kRawBufWord3 = 0x00020000;

__device__ __forceinline__ u32x4 ld_u32x4(const void *p) {
    return *reinterpret_cast<const u32x4_a1 *>(p);
}
__device__ __forceinline__ f32x4 ld_f32x4(const float *p) {
    return *reinterpret_cast<const f32x4_a4 *>(p);
}
__device__ __forceinline__ void st_u32(void *p, uint32_t v) { *reinterpret_cast<u32_a1 *>(p) = v; }

// v from lane (lane ^ MASK) within each group of 4 lanes (DPP quad_perm).
template <int MASK>
__device__ __forceinline__ float quad_xor(float v) {
    static_assert(MASK == 1 || MASK == 2, "quad lane xor");
    constexpr int ctrl = MASK == 1 ? 0xB1 : 0x4E;  // quad_perm [1,0,3,2] / [2,3,0,1]
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), ctrl,
                                                                 0xF, 0xF, false));
}

// GLU activations: kActGeluTanh is gelu_tanh in the order
// kernels/transformer_ops.hip:36-38 evaluates it; kActSilu is v*sigmoid(v).
constexpr int kActGeluTanh = 0, kActSilu = 1;
__device__ __forceinline__ float glu_act(float v, int act) {
    if (act == kActSilu) return v / (1.0f + expf(-v));
    const float c = 0.7978845608f * (v + 0.044715f * v * v * v);
    return 0.5f * v * (1.0f + tanhf(c));
}

}  // namespace mgq
