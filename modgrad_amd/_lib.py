"""ctypes binding of libmodgrad_q4k.so (the C ABI in include/modgrad_q4k.h).

There is no fallback: if the library is missing or does not export every
declared symbol, loading raises. Build it with `python -m modgrad_amd.build`.
"""
from __future__ import annotations

import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmodgrad_q4k.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "modgrad_q4k.h")

hipSuccess = 0
hipErrorInvalidValue = 1
hipErrorNotSupported = 801

P = ctypes.c_void_p
I = ctypes.c_int
S = ctypes.c_size_t
F = ctypes.c_float

SIGNATURES = {
    "launch_dequant_q4k": (I, [P, I, P]),
    "launch_matvec_q4k": (I, [P, P, P, I, I]),
    "launch_matvec_q4k_ex": (I, [P, P, P, I, I, I, P]),
    "launch_quantize_q8_1": (I, [P, P, P, P, I]),
    "launch_matvec_q5k": (I, [P, P, P, I, I]),
    "launch_matvec_q6k": (I, [P, P, P, I, I]),
    "launch_matvec_q6k_dp4a": (I, [P, P, P, P, P, I, I]),
    "launch_matvec_q5k_ex": (I, [P, P, P, I, I, P]),
    "launch_matvec_q6k_ex": (I, [P, P, P, I, I, P]),
    "launch_matvec_q6k_dp4a_ex": (I, [P, P, P, P, P, I, I, P]),
    "launch_matvec_q4k_dp4a": (I, [P, P, P, P, P, I, I]),
    "launch_quantize_q8_1_ex": (I, [P, P, P, P, I, P]),
    "launch_matvec_q4k_dp4a_ex": (I, [P, P, P, P, P, I, I, P]),
    "launch_dequant_q4k_ex": (I, [P, I, P, P]),
    "mgq_batched_workspace_bytes": (S, [I, I]),
    "launch_matvec_q4k_batched": (I, [P, P, P, I, I, I, P, S, P]),
    "launch_matvec_q4k_batched_noalloc": (I, [P, P, P, I, I, I, P]),
    "launch_gemm_q4k_f16": (I, [P, P, P, I, I, I, P]),
    "launch_quantize_matvec_q4k_dp4a_ex": (I, [P, P, P, I, I, P]),
    "launch_rms_norm": (I, [P, P, P, I, I, F]),
    "launch_rms_norm_ex": (I, [P, P, P, I, I, F, P]),
    "launch_geglu": (I, [P, P, P, I]),
    "launch_glu_ex": (I, [P, P, P, I, I, P]),
    "launch_residual_add": (I, [P, P, I]),
    "launch_residual_add_ex": (I, [P, P, I, P]),
    "launch_scale": (I, [P, F, I]),
    "launch_scale_ex": (I, [P, F, I, P]),
    "launch_matvec_q4k_rmsnorm_ex": (I, [P, P, P, F, P, I, I, P]),
    "launch_matvec_q6k_rmsnorm_ex": (I, [P, P, P, F, P, I, I, P]),
    "launch_matvec_q4k_glu_ex": (I, [P, P, P, P, F, I, P, I, I, P]),
    "mgq_chain_create": (I, [P, I, P]),
    "mgq_chain_create_ex": (I, [P, I, I, P]),
    "mgq_chain_create_ops": (I, [P, I, P]),
    "mgq_chain_info": (I, [P, P, P]),
    "mgq_chain_launch": (I, [P, P]),
    "mgq_chain_destroy": (I, [P]),
    "mgq_prepare": (I, []),
    "mgq_version": (ctypes.c_char_p, []),
}

ACT_GELU_TANH = 0
ACT_SILU = 1
LAYOUT_ROWS = 0
LAYOUT_FLAT = 1
CHAIN_AUTO = 0
CHAIN_GRAPH = 1
CHAIN_PERSISTENT = 2
CHAIN_EAGER = 3
OP_MATVEC = 0
OP_MATVEC_NORM = 1
OP_MATVEC_GLU = 2
OP_RMS_NORM = 3
OP_GLU = 4
OP_RESIDUAL_ADD = 5
OP_QUANTIZE_Q8_1 = 6
OP_MATVEC_DP4A = 7
OP_QUANTIZE_MATVEC_DP4A = 8
DTYPE_Q4_K = 12
DTYPE_Q5_K = 13
DTYPE_Q6_K = 14


class GemvDesc(ctypes.Structure):
    """mgq_gemv_desc."""
    _fields_ = [("w_q4", P), ("x", P), ("y", P), ("out_dim", I), ("blocks_per_row", I)]


class OpDesc(ctypes.Structure):
    """mgq_op_desc (one kernel of an op chain)."""
    _fields_ = [("op", I), ("dtype", I), ("layout", I), ("act", I), ("w", P), ("w2", P),
                ("x", P), ("x2", P), ("norm_w", P), ("y", P), ("out_dim", I), ("in_dim", I),
                ("rows", I), ("eps", F), ("xq", P), ("xd", P), ("xsum", P)]


class HipError(RuntimeError):
    def __init__(self, fn: str, code: int):
        super().__init__(f"{fn} returned hipError {code}")
        self.code = code


_lib = None


def declared_symbols() -> list[str]:
    """Function names declared in include/modgrad_q4k.h."""
    text = open(HEADER).read()
    return re.findall(r"^\s*(?:hipError_t|const char \*)\s*\*?\s*(\w+)\s*\(", text, re.M)


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m modgrad_amd.build` "
            "(there is no CPU fallback)")
    L = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(L, name)  # AttributeError if the symbol is not exported
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def check(fn: str, code: int) -> None:
    if code != hipSuccess:
        raise HipError(fn, code)
