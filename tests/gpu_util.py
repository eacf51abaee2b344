"""Helpers for GPU tests: device buffers from numpy and the tolerance check."""
import ctypes

import numpy as np


def dev(a: np.ndarray):
    """Copy a numpy array to a CUDA tensor (bytes kept, dtype kept)."""
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a)).to("cuda")
    return t


def ptr(t) -> int:
    return t.data_ptr()


def host(t) -> np.ndarray:
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def empty_f32(n: int):
    import torch
    return torch.full((n,), float("nan"), dtype=torch.float32, device="cuda")


def filled_u8(n: int, value: int):
    """Device byte buffer of n bytes, every byte = value (stale-workspace stand-in)."""
    import torch
    return torch.full((max(n, 1),), value, dtype=torch.uint8, device="cuda")


def assert_gemv_close(y: np.ndarray, y_ref: np.ndarray, absdot: np.ndarray, tol: float = 1e-4):
    """BASELINE gate: per row |y - y_ref| <= tol * sum_k |w_rk||x_k|."""
    err = np.abs(y.astype(np.float64) - y_ref.astype(np.float64))
    bound = tol * absdot
    bad = np.nonzero(~(err <= bound))[0]
    assert bad.size == 0, (
        f"{bad.size} rows out of tolerance; first {bad[:5].tolist()}: "
        f"err={err[bad[:5]].tolist()} bound={bound[bad[:5]].tolist()}")
    return float(np.max(err / np.maximum(absdot, 1e-300))) if absdot.size else 0.0


def random_q4k_bytes(rng: np.random.Generator, n_blocks: int, finite_scales: bool = True,
                     d_scale: float = 1e-3) -> np.ndarray:
    """Random Q4_K blocks; with finite_scales, d/dmin are f16 of |N(0, d_scale)|."""
    b = rng.integers(0, 256, size=(n_blocks, 144), dtype=np.uint8)
    if finite_scales:
        d = np.abs(rng.normal(0, d_scale, size=(n_blocks, 2))).astype(np.float16)
        b[:, 0:4] = d.view(np.uint8).reshape(n_blocks, 4)
    return b.ravel()


c_void_p = ctypes.c_void_p


def random_kquant_bytes(rng: np.random.Generator, n_blocks: int, block_bytes: int,
                        d_scale: float = 1e-3) -> np.ndarray:
    """Random Q5_K (176 B) or Q6_K (210 B) blocks with finite f16 d (and dmin)."""
    b = rng.integers(0, 256, size=(n_blocks, block_bytes), dtype=np.uint8)
    if block_bytes == 176:
        d = np.abs(rng.normal(0, d_scale, size=(n_blocks, 2))).astype(np.float16)
        b[:, 0:4] = d.view(np.uint8).reshape(n_blocks, 4)
    else:
        d = np.abs(rng.normal(0, d_scale, size=(n_blocks, 1))).astype(np.float16)
        b[:, 208:210] = d.view(np.uint8).reshape(n_blocks, 2)
    return b.ravel()
