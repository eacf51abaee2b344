"""ctypes binding of the CPU oracle (oracle/q4k_oracle.c).

TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import this module as the checker. The product package
(modgrad_amd) never imports it.

Seeded input generation follows one fixed convention:
  W[n][k] = 0.02 * SimpleRng(seed_w).next_normal(), row-major, then quantized
  by the reference quantizer over the flattened tensor (neuron.rs:931-951);
  x[k] = SimpleRng(seed_x).next_normal().
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle_q4k.so")

BLOCK_BYTES = 144
BLOCK_ELEMS = 256

_lib = None


def build() -> str:
    """Compile the oracle with its Makefile (gcc, -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    L = ctypes.CDLL(LIB_PATH)
    P = ctypes.c_void_p
    i, z, f, u64 = ctypes.c_int, ctypes.c_size_t, ctypes.c_float, ctypes.c_uint64
    sig = {
        "orq_f16_to_f32": (f, [ctypes.c_uint16]),
        "orq_f32_to_f16": (ctypes.c_uint16, [f]),
        "orq_get_scale_min_k4": (None, [i, P, P, P]),
        "orq_pack_scales_mins": (None, [P, P, P]),
        "orq_dequantize_row_q4_k": (None, [P, P, z, z]),
        "orq_quantize_row_q4_k": (z, [P, z, P]),
        "orq_quantize_row_q4_k_offsets": (z, [P, z, P, P]),
        "orq_rng_init": (None, [P, u64]),
        "orq_rng_next_u64": (u64, [P]),
        "orq_rng_next_f32": (f, [P]),
        "orq_rng_next_normal": (f, [P]),
        "orq_fill_normal": (None, [u64, f, P, z]),
        "orq_gemv_f64": (None, [P, P, P, i, i]),
        "orq_gemv_f64_abs": (None, [P, P, P, P, i, i]),
        "orq_gemv_flat_f64_abs": (None, [P, P, P, P, i, i]),
        "orq_gemv_batched_f64_abs": (None, [P, P, P, P, i, i, i]),
        "orq_gemm_f16_f64": (None, [P, P, P, P, i, i, i, P, i]),
        "orq_cpu_matvec_q4k": (i, [P, P, P, i, i, i]),
        "orq_cpu_has_avx512": (i, []),
        "orq_fill_smooth": (None, [P, z]),
        "orq_quantize_q8_1": (None, [P, i, P, P, P]),
        "orq_dequantize_row_q5_k": (None, [P, P, z, z]),
        "orq_dequantize_row_q6_k": (None, [P, P, z, z]),
        "orq_gemv_kquant_f64_abs": (None, [i, P, P, P, P, i, i]),
        "orq_gemv_q6k_dp4a_f64": (None, [P, P, P, i, i, P, P]),
        "orq_gemv_q4k_dp4a_f64": (None, [P, P, P, P, i, i, P, P]),
        "orq_rms_norm": (None, [P, P, P, i, i, f]),
        "orq_glu": (None, [P, P, P, i, i]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


# ------------------------------------------------------------------ scalars --
def f16_to_f32(h: int) -> float:
    return lib().orq_f16_to_f32(h)


def f32_to_f16(v: float) -> int:
    return lib().orq_f32_to_f16(v)


def get_scale_min_k4(j: int, scales: bytes):
    s = np.frombuffer(bytes(scales), dtype=np.uint8).copy()
    sc = ctypes.c_uint8()
    m = ctypes.c_uint8()
    lib().orq_get_scale_min_k4(j, _p(s), ctypes.byref(sc), ctypes.byref(m))
    return sc.value, m.value


def pack_scales_mins(sc, m) -> bytes:
    a = np.asarray(sc, dtype=np.uint8).copy()
    b = np.asarray(m, dtype=np.uint8).copy()
    out = np.zeros(12, dtype=np.uint8)
    lib().orq_pack_scales_mins(_p(a), _p(b), _p(out))
    return out.tobytes()


# ------------------------------------------------------------------ arrays ---
def dequantize(data: np.ndarray, n_blocks: int | None = None, out_len: int | None = None) -> np.ndarray:
    data = np.ascontiguousarray(data, dtype=np.uint8)
    nb = data.size // BLOCK_BYTES if n_blocks is None else n_blocks
    n = nb * BLOCK_ELEMS if out_len is None else out_len
    out = np.zeros(n, dtype=np.float32)
    lib().orq_dequantize_row_q4_k(_p(data), _p(out), n, nb)
    return out


def quantize(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    if x.size % BLOCK_ELEMS:
        raise ValueError(f"quantize: len {x.size} not a multiple of {BLOCK_ELEMS}")
    out = np.zeros(x.size // BLOCK_ELEMS * BLOCK_BYTES, dtype=np.uint8)
    n = lib().orq_quantize_row_q4_k(_p(x), x.size, _p(out))
    assert n == out.size
    return out


def quantize_with_offsets(x: np.ndarray, offsets) -> np.ndarray:
    """quantize() with the sub-block table of gguf.rs:601 replaced by
    `offsets` (offsets[is] = first element of sub-block is)."""
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    if x.size % BLOCK_ELEMS:
        raise ValueError(f"quantize: len {x.size} not a multiple of {BLOCK_ELEMS}")
    offs = np.ascontiguousarray(offsets, dtype=np.int32)
    assert offs.size == 8
    out = np.zeros(x.size // BLOCK_ELEMS * BLOCK_BYTES, dtype=np.uint8)
    n = lib().orq_quantize_row_q4_k_offsets(_p(x), x.size, _p(out), _p(offs))
    assert n == out.size
    return out


class SimpleRng:
    """neuron.rs:1345-1367 through the oracle (one C state per instance)."""

    def __init__(self, seed: int):
        self._st = np.zeros(1, dtype=np.uint64)
        lib().orq_rng_init(_p(self._st), seed & 0xFFFFFFFFFFFFFFFF)

    def next_u64(self) -> int:
        return lib().orq_rng_next_u64(_p(self._st))

    def next_f32(self) -> float:
        return lib().orq_rng_next_f32(_p(self._st))

    def next_normal(self) -> float:
        return lib().orq_rng_next_normal(_p(self._st))


def smooth(n: int) -> np.ndarray:
    """The reference tests' signal sin(7.3 t)/2 + cos(17.1 t)/5, t = i/n."""
    out = np.empty(n, dtype=np.float32)
    lib().orq_fill_smooth(_p(out), n)
    return out


def normal(seed: int, n: int, scale: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().orq_fill_normal(seed & 0xFFFFFFFFFFFFFFFF, scale, _p(out), n)
    return out


# ------------------------------------------------------------------ GEMV -----
def gemv(w: np.ndarray, x: np.ndarray, out_dim: int, bpr: int):
    """(y f32, absdot f64) for the row-aligned layout."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert w.size >= out_dim * bpr * BLOCK_BYTES and x.size >= bpr * BLOCK_ELEMS
    y = np.empty(out_dim, dtype=np.float32)
    a = np.empty(out_dim, dtype=np.float64)
    lib().orq_gemv_f64_abs(_p(w), _p(x), _p(y), _p(a), out_dim, bpr)
    return y, a


def gemv_flat(w: np.ndarray, x: np.ndarray, out_dim: int, k_elems: int):
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert w.size * BLOCK_ELEMS >= out_dim * k_elems * BLOCK_BYTES and x.size >= k_elems
    y = np.empty(out_dim, dtype=np.float32)
    a = np.empty(out_dim, dtype=np.float64)
    lib().orq_gemv_flat_f64_abs(_p(w), _p(x), _p(y), _p(a), out_dim, k_elems)
    return y, a


def gemv_batched(w: np.ndarray, X: np.ndarray, out_dim: int, bpr: int):
    w = np.ascontiguousarray(w, dtype=np.uint8)
    X = np.ascontiguousarray(X, dtype=np.float32)
    batch = X.shape[0]
    assert X.shape[1] == bpr * BLOCK_ELEMS
    Y = np.empty((batch, out_dim), dtype=np.float32)
    A = np.empty((batch, out_dim), dtype=np.float64)
    lib().orq_gemv_batched_f64_abs(_p(w), _p(X), _p(Y), _p(A), out_dim, bpr, batch)
    return Y, A


Q5K_BYTES, Q6K_BYTES = 176, 210


def dequantize_q5k(data: np.ndarray) -> np.ndarray:
    data = np.ascontiguousarray(data, dtype=np.uint8)
    nb = data.size // Q5K_BYTES
    out = np.empty(nb * BLOCK_ELEMS, dtype=np.float32)
    lib().orq_dequantize_row_q5_k(_p(data), _p(out), out.size, nb)
    return out


def dequantize_q6k(data: np.ndarray) -> np.ndarray:
    data = np.ascontiguousarray(data, dtype=np.uint8)
    nb = data.size // Q6K_BYTES
    out = np.empty(nb * BLOCK_ELEMS, dtype=np.float32)
    lib().orq_dequantize_row_q6_k(_p(data), _p(out), out.size, nb)
    return out


def gemv_kquant(block_bytes: int, w: np.ndarray, x: np.ndarray, out_dim: int, bpr: int):
    """(y f32, absdot f64): f64 dequant-dot of a Q4_K/Q5_K/Q6_K row-aligned matrix."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert w.size >= out_dim * bpr * block_bytes and x.size >= bpr * BLOCK_ELEMS
    y = np.empty(out_dim, dtype=np.float32)
    a = np.empty(out_dim, dtype=np.float64)
    lib().orq_gemv_kquant_f64_abs(block_bytes, _p(w), _p(x), _p(y), _p(a), out_dim, bpr)
    return y, a


def gemv_q6k_dp4a(w: np.ndarray, xq: np.ndarray, xd: np.ndarray, out_dim: int, bpr: int):
    w = np.ascontiguousarray(w, dtype=np.uint8)
    xq = np.ascontiguousarray(xq, dtype=np.int8)
    xd = np.ascontiguousarray(xd, dtype=np.float32)
    y = np.empty(out_dim, dtype=np.float64)
    a = np.empty(out_dim, dtype=np.float64)
    lib().orq_gemv_q6k_dp4a_f64(_p(w), _p(xq), _p(xd), out_dim, bpr, _p(y), _p(a))
    return y, a


def quantize_q8_1(x: np.ndarray):
    """(xq int8[n/32*32], xd f32[n/32], xsum f32[n/32]) -- matvec_q4k_dp4a.hip:29-50."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    nsub = x.size // 32
    xq = np.zeros(nsub * 32, dtype=np.int8)
    xd = np.zeros(nsub, dtype=np.float32)
    xs = np.zeros(nsub, dtype=np.float32)
    lib().orq_quantize_q8_1(_p(x), x.size, _p(xq), _p(xd), _p(xs))
    return xq, xd, xs


def gemv_dp4a(w: np.ndarray, xq: np.ndarray, xd: np.ndarray, xsum: np.ndarray, out_dim: int,
              bpr: int):
    """(y f64, absterm f64) -- the dp4a matvec of matvec_q4k_dp4a.hip:52-106 in f64."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    xq = np.ascontiguousarray(xq, dtype=np.int8)
    xd = np.ascontiguousarray(xd, dtype=np.float32)
    xsum = np.ascontiguousarray(xsum, dtype=np.float32)
    assert xq.size >= bpr * BLOCK_ELEMS and xd.size >= bpr * 8
    y = np.empty(out_dim, dtype=np.float64)
    a = np.empty(out_dim, dtype=np.float64)
    lib().orq_gemv_q4k_dp4a_f64(_p(w), _p(xq), _p(xd), _p(xsum), out_dim, bpr, _p(y), _p(a))
    return y, a


def gemm_f16(w: np.ndarray, a_f16: np.ndarray, out_dim: int, bpr: int, rows=None):
    """C[m][i] for rows[i] (all rows if None); a_f16 is uint16 half bits [M][K]."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    a = np.ascontiguousarray(a_f16, dtype=np.uint16)
    m_tokens = a.shape[0]
    assert a.shape[1] == bpr * BLOCK_ELEMS
    if rows is None:
        nr, rp = out_dim, None
    else:
        rows = np.ascontiguousarray(rows, dtype=np.int32)
        nr, rp = rows.size, _p(rows)
    C = np.empty((m_tokens, nr), dtype=np.float32)
    A = np.empty((m_tokens, nr), dtype=np.float64)
    lib().orq_gemm_f16_f64(_p(w), _p(a), _p(C), _p(A), out_dim, bpr, m_tokens, rp, nr)
    return C, A


def cpu_matvec(w: np.ndarray, x: np.ndarray, y: np.ndarray, out_dim: int, bpr: int,
               threads: int = 0) -> int:
    """Reference CPU GEMV restatement (timing baseline). Returns 1 if AVX-512."""
    return lib().orq_cpu_matvec_q4k(_p(w), _p(x), _p(y), out_dim, bpr, threads)


def cpu_has_avx512() -> bool:
    return bool(lib().orq_cpu_has_avx512())


# ------------------------------------------------------------ workloads ------
def seeded_weight(seed: int, out_dim: int, k: int, scale: float = 0.02) -> np.ndarray:
    """Q4_K bytes of W[out_dim][k] = scale*N(0,1) from SimpleRng(seed)."""
    return quantize(normal(seed, out_dim * k, scale))


def layer_seed(layer: int, tensor: int) -> int:
    """seed_W for tensor t of layer l (q=0,k=1,v=2,o=3,gate=4,up=5,down=6;
    lm_head is layer 28, t=7); seed_x = seed_W ^ 0xA5A5."""
    return 0x514B00 + 16 * layer + tensor


def rms_norm(x: np.ndarray, w: np.ndarray, rows: int, hidden: int, eps: float) -> np.ndarray:
    """f32 [rows][hidden] -- kernels/rms_norm.hip:28-75 in the reference's order."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    y = np.empty(rows * hidden, dtype=np.float32)
    lib().orq_rms_norm(_p(x), _p(w), _p(y), rows, hidden, eps)
    return y


def glu(gate: np.ndarray, up: np.ndarray, act: int = 0) -> np.ndarray:
    """act(gate) * up -- act 0: gelu_tanh (transformer_ops.hip:32-40), 1: silu."""
    gate = np.ascontiguousarray(gate, dtype=np.float32)
    up = np.ascontiguousarray(up, dtype=np.float32)
    out = np.empty(gate.size, dtype=np.float32)
    lib().orq_glu(_p(gate), _p(up), _p(out), gate.size, act)
    return out
