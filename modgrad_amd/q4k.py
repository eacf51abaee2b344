"""Host-side mirror of the reference's Q4_K device interface, over the C ABI.

Names, argument meaning and error behaviour follow the reference's Rust host
(crates/modgrad-device/src/backend/rocm.rs, ops.rs and
crates/modgrad-compute/src/neuron.rs), so tests read like the reference's:

  BackendError        backend/mod.rs:107-123
  HipBuffer           rocm.rs:603-935  (RAII device buffer; here a torch
                                        uint8 CUDA tensor holds the memory)
  HipBuffer.matvec_q4k / matvec_q4k_into   rocm.rs:681-738
  HipBuffer.matvec_q5k / matvec_q5k_into   rocm.rs:743-776
  kern.*                                   rocm.rs:943-996
  ops.dequant_q4k_resident                 ops.rs:531-539
  GpuVec, ResidencyError                   compute/src/backend.rs:35-278
  HipBatch                                 rocm.rs:1089-1211
  LinearResidentQuantized                  neuron.rs:897-1108

PyTorch is only the device-memory allocator here; every computation goes
through libmodgrad_q4k.so (modgrad_amd._lib), with no CPU fallback.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib

Q4K_BLOCK_BYTES = 144
Q4K_BLOCK_ELEMS = 256


class BackendError(RuntimeError):
    """backend/mod.rs:107-123 (Runtime / Unsupported / OutOfMemory)."""

    def __init__(self, kind: str, msg: str):
        super().__init__(f"{kind}: {msg}")
        self.kind = kind


def _torch():
    import torch
    if not torch.cuda.is_available():
        raise BackendError("Unsupported", "no HIP device visible")
    return torch


def _chk(code: int, what: str) -> None:
    if code != 0:
        raise BackendError("Runtime", f"{what}: hip error {code}")


def _stream_ptr(stream) -> ctypes.c_void_p:
    if stream is None:
        return ctypes.c_void_p(0)
    return ctypes.c_void_p(stream.cuda_stream)


class HipBuffer:
    """A device allocation of `nbytes` bytes (rocm.rs:620-635)."""

    def __init__(self, nbytes: int):
        torch = _torch()
        if nbytes < 0:
            raise BackendError("Runtime", f"hipMalloc({nbytes}): negative size")
        # round up to 16 B so 128-bit loads of the tail stay in the allocation
        try:
            self._t = torch.empty(max(16, (nbytes + 15) // 16 * 16), dtype=torch.uint8,
                                  device="cuda")
        except torch.cuda.OutOfMemoryError as e:
            raise BackendError("OutOfMemory", f"hipMalloc({nbytes})") from e
        self._bytes = nbytes

    @classmethod
    def new(cls, nbytes: int) -> "HipBuffer":
        return cls(nbytes)

    def device_ptr(self) -> int:
        return self._t.data_ptr()

    def bytes(self) -> int:
        return self._bytes

    def len_f32(self) -> int:
        return self._bytes // 4

    def tensor(self):
        return self._t[: self._bytes]

    def u8_at(self, offset: int) -> int:
        """Device pointer `offset` bytes in (rocm.rs:913-934)."""
        if offset > self._bytes:
            raise BackendError("Runtime", f"u8_at: offset {offset} > buf {self._bytes}")
        return self.device_ptr() + offset

    def f32_at(self, index: int) -> int:
        return self.u8_at(4 * index)

    def f32_ptr(self) -> int:
        return self.device_ptr()

    def u8_ptr(self) -> int:
        return self.device_ptr()

    def copy_from_host_bytes(self, src) -> None:
        torch = _torch()
        a = np.frombuffer(bytes(src), dtype=np.uint8) if not isinstance(src, np.ndarray) else src
        a = np.ascontiguousarray(a, dtype=np.uint8).ravel()
        if a.size > self._bytes:
            raise BackendError("Runtime", f"copy_from_host_bytes: src {a.size} > buf {self._bytes}")
        self._t[: a.size].copy_(torch.from_numpy(a))

    def copy_from_host_bytes_at(self, off: int, src) -> None:
        """Stage host bytes at a byte offset, for packing many tensors into
        one allocation (rocm.rs:917-934)."""
        torch = _torch()
        a = np.frombuffer(bytes(src), dtype=np.uint8) if not isinstance(src, np.ndarray) else src
        a = np.ascontiguousarray(a, dtype=np.uint8).ravel()
        if off < 0 or off + a.size > self._bytes:
            raise BackendError("Runtime", f"copy_from_host_bytes_at: off {off} + {a.size} > "
                                          f"buf {self._bytes}")
        self._t[off: off + a.size].copy_(torch.from_numpy(a))

    def copy_from_host(self, src) -> None:
        a = np.ascontiguousarray(src, dtype=np.float32).ravel()
        if a.nbytes > self._bytes:
            raise BackendError("Runtime", f"upload_f32: src is {a.nbytes} bytes, device buffer "
                                          f"is {self._bytes} bytes")
        self.copy_from_host_bytes(a.view(np.uint8))

    def copy_to_host(self, n_f32: int | None = None) -> np.ndarray:
        """The first `n_f32` floats (all of them by default); asking for more
        than the buffer holds is an error (rocm.rs:779-781, 873-895)."""
        n = self.len_f32() if n_f32 is None else n_f32
        if n < 0 or 4 * n > self._bytes:
            raise BackendError("Runtime", f"download_f32: dst is {4 * n} bytes, device buffer "
                                          f"is {self._bytes} bytes")
        _torch().cuda.synchronize()
        return self._t[: 4 * n].cpu().numpy().view(np.float32).copy()

    def copy_range_from(self, src: "HipBuffer", src_offset_f32: int, dst_offset_f32: int,
                        len_f32: int) -> None:
        """Device-to-device copy of `len_f32` floats from `src` at
        `src_offset_f32` into this buffer at `dst_offset_f32`, both ranges
        bounds-checked (rocm.rs:791-837)."""
        if min(src_offset_f32, dst_offset_f32, len_f32) < 0:
            raise BackendError("Runtime", "copy_range_from: negative offset or length")
        nb, so, do = 4 * len_f32, 4 * src_offset_f32, 4 * dst_offset_f32
        if so + nb > src._bytes:
            raise BackendError("Runtime", f"copy_range_from: src range [{so},{so + nb}) bytes "
                                          f"exceeds src buffer ({src._bytes} bytes)")
        if do + nb > self._bytes:
            raise BackendError("Runtime", f"copy_range_from: dst range [{do},{do + nb}) bytes "
                                          f"exceeds dst buffer ({self._bytes} bytes)")
        self._t[do: do + nb].copy_(src._t[so: so + nb])

    def matvec_q4k(self, x, out_dim: int, blocks_per_row: int) -> np.ndarray:
        """y = dequant(self) @ x with host x in and host y out (rocm.rs:681-709)."""
        in_dim = blocks_per_row * Q4K_BLOCK_ELEMS
        x_dev = HipBuffer(in_dim * 4)
        x_dev.copy_from_host(np.asarray(x, np.float32)[:in_dim])
        y_dev = HipBuffer(out_dim * 4)
        self.matvec_q4k_into(x_dev, y_dev, out_dim, blocks_per_row)
        return y_dev.copy_to_host(out_dim)

    def matvec_q4k_into(self, x_dev: "HipBuffer", y_dev: "HipBuffer", out_dim: int,
                        blocks_per_row: int) -> None:
        """Launch + device sync, resident x/y (rocm.rs:711-738)."""
        kern.matvec_q4k(self.device_ptr(), x_dev.device_ptr(), y_dev.device_ptr(), out_dim,
                        blocks_per_row)
        kern.hip_sync()

    def matvec_q5k(self, x, out_dim: int, blocks_per_row: int) -> np.ndarray:
        """Q5_K twin of matvec_q4k (rocm.rs:743-761)."""
        in_dim = blocks_per_row * Q4K_BLOCK_ELEMS
        x_dev = HipBuffer(in_dim * 4)
        x_dev.copy_from_host(np.asarray(x, np.float32)[:in_dim])
        y_dev = HipBuffer(out_dim * 4)
        self.matvec_q5k_into(x_dev, y_dev, out_dim, blocks_per_row)
        return y_dev.copy_to_host(out_dim)

    def matvec_q5k_into(self, x_dev: "HipBuffer", y_dev: "HipBuffer", out_dim: int,
                        blocks_per_row: int) -> None:
        """Q5_K twin of matvec_q4k_into (rocm.rs:765-776)."""
        kern.matvec_q5k(self.device_ptr(), x_dev.device_ptr(), y_dev.device_ptr(), out_dim,
                        blocks_per_row)
        kern.hip_sync()


class kern:
    """Launch-only wrappers, null stream, no sync (rocm.rs:942-979)."""

    @staticmethod
    def hip_sync() -> None:
        _torch().cuda.synchronize()

    @staticmethod
    def vram_free_total() -> tuple[int, int]:
        """(free, total) device memory in bytes (rocm.rs:956-961)."""
        return tuple(int(v) for v in _torch().cuda.mem_get_info())

    @staticmethod
    def residual_add(h: int, x: int, n: int, stream=None) -> None:
        """rocm.rs:984-986: h += x over n floats."""
        _chk(_lib.load().launch_residual_add_ex(h, x, n, _stream_ptr(stream)), "residual_add")

    @staticmethod
    def scale(h: int, s: float, n: int, stream=None) -> None:
        """rocm.rs:987-989: h *= s over n floats."""
        _chk(_lib.load().launch_scale_ex(h, s, n, _stream_ptr(stream)), "scale")

    @staticmethod
    def matvec_q4k(w: int, x: int, y: int, out_dim: int, bpr: int) -> None:
        _chk(_lib.load().launch_matvec_q4k(w, x, y, out_dim, bpr), "matvec_q4k")

    @staticmethod
    def matvec_q5k(w: int, x: int, y: int, out_dim: int, bpr: int, stream=None) -> None:
        """rocm.rs:964-966."""
        _chk(_lib.load().launch_matvec_q5k_ex(w, x, y, out_dim, bpr, _stream_ptr(stream)),
             "matvec_q5k")

    @staticmethod
    def matvec_q6k(w: int, x: int, y: int, out_dim: int, bpr: int, stream=None) -> None:
        """rocm.rs:967-969."""
        _chk(_lib.load().launch_matvec_q6k_ex(w, x, y, out_dim, bpr, _stream_ptr(stream)),
             "matvec_q6k")

    @staticmethod
    def matvec_q6k_dp4a(w: int, xq: int, xd: int, xsum: int, y: int, out_dim: int, bpr: int,
                        stream=None) -> None:
        """rocm.rs:977-980."""
        _chk(_lib.load().launch_matvec_q6k_dp4a_ex(w, xq, xd, xsum, y, out_dim, bpr,
                                                   _stream_ptr(stream)), "matvec_q6k_dp4a")

    @staticmethod
    def quantize_q8_1(x: int, xq: int, xd: int, xsum: int, n: int, stream=None) -> None:
        """rocm.rs:970-972: int8 activations + per-32 scale and sum."""
        _chk(_lib.load().launch_quantize_q8_1_ex(x, xq, xd, xsum, n, _stream_ptr(stream)),
             "quantize_q8_1")

    @staticmethod
    def matvec_q4k_dp4a(w: int, xq: int, xd: int, xsum: int, y: int, out_dim: int, bpr: int,
                        stream=None) -> None:
        """rocm.rs:973-976: the dp4a matvec on quantize_q8_1's output."""
        _chk(_lib.load().launch_matvec_q4k_dp4a_ex(w, xq, xd, xsum, y, out_dim, bpr,
                                                   _stream_ptr(stream)), "matvec_q4k_dp4a")

    @staticmethod
    def rms_norm(x: int, w: int, y: int, n: int, hidden: int, eps: float, stream=None) -> None:
        """rocm.rs:981-983: y = x * rstd * w over n rows of `hidden`."""
        _chk(_lib.load().launch_rms_norm_ex(x, w, y, n, hidden, eps, _stream_ptr(stream)),
             "rms_norm")

    @staticmethod
    def geglu(gate: int, up: int, out: int, n: int, stream=None) -> None:
        """rocm.rs:990-992: out = gelu_tanh(gate) * up."""
        _chk(_lib.load().launch_glu_ex(gate, up, out, n, _lib.ACT_GELU_TANH, _stream_ptr(stream)),
             "geglu")

    # additive entry points -------------------------------------------------
    @staticmethod
    def quantize_matvec_q4k_dp4a(w: int, x: int, y: int, out_dim: int, bpr: int,
                                 stream=None) -> None:
        """quantize_q8_1 + matvec_q4k_dp4a in one launch (bit-identical y)."""
        _chk(_lib.load().launch_quantize_matvec_q4k_dp4a_ex(w, x, y, out_dim, bpr,
                                                            _stream_ptr(stream)),
             "quantize_matvec_q4k_dp4a")

    @staticmethod
    def glu(gate: int, up: int, out: int, n: int, act: int = _lib.ACT_GELU_TANH,
            stream=None) -> None:
        """out = act(gate) * up, act = ACT_GELU_TANH or ACT_SILU."""
        _chk(_lib.load().launch_glu_ex(gate, up, out, n, act, _stream_ptr(stream)), "glu")

    @staticmethod
    def matvec_q4k_rmsnorm(w: int, x: int, norm_w: int, eps: float, y: int, out_dim: int,
                           bpr: int, stream=None) -> None:
        """y = W * rms_norm(x, norm_w, eps) in one launch (the reference's
        rms_norm + matvec_q4k pair, rocm_gemma.rs:439-440)."""
        _chk(_lib.load().launch_matvec_q4k_rmsnorm_ex(w, x, norm_w, eps, y, out_dim, bpr,
                                                      _stream_ptr(stream)), "matvec_q4k_rmsnorm")

    @staticmethod
    def matvec_q6k_rmsnorm(w: int, x: int, norm_w: int, eps: float, y: int, out_dim: int,
                           bpr: int, stream=None) -> None:
        """y = W * rms_norm(x, norm_w, eps) for Q6_K W in one launch (the
        reference's rms_norm + matvec_q6k pair); BackendError("Unsupported")
        outside q6k_norm_fits."""
        _chk(_lib.load().launch_matvec_q6k_rmsnorm_ex(w, x, norm_w, eps, y, out_dim, bpr,
                                                      _stream_ptr(stream)), "matvec_q6k_rmsnorm")

    @staticmethod
    def matvec_q4k_glu(w_gate: int, w_up: int, x: int, y: int, out_dim: int, bpr: int,
                       norm_w: int | None = None, eps: float = 0.0,
                       act: int = _lib.ACT_GELU_TANH, stream=None) -> None:
        """y = act(W_gate xn) * (W_up xn), xn = rms_norm(x) when norm_w is
        given: the reference FFN's rms_norm + gate + up + geglu
        (rocm_gemma.rs:477-481) in one launch."""
        _chk(_lib.load().launch_matvec_q4k_glu_ex(w_gate, w_up, x, norm_w, eps, act, y, out_dim,
                                                  bpr, _stream_ptr(stream)), "matvec_q4k_glu")

    @staticmethod
    def matvec_q4k_ex(w: int, x: int, y: int, out_dim: int, k_elems: int,
                      layout: int = _lib.LAYOUT_ROWS, stream=None) -> None:
        _chk(_lib.load().launch_matvec_q4k_ex(w, x, y, out_dim, k_elems, layout,
                                              _stream_ptr(stream)), "matvec_q4k_ex")

    @staticmethod
    def batched_workspace_bytes(bpr: int, batch: int) -> int:
        return int(_lib.load().mgq_batched_workspace_bytes(bpr, batch))

    @staticmethod
    def matvec_q4k_batched(w: int, X: int, Y: int, out_dim: int, bpr: int, batch: int,
                           stream=None, workspace=None) -> None:
        """Y[b] = dequant(W) X[b] for b < batch. `workspace` is a device
        tensor of at least batched_workspace_bytes(bpr, batch) bytes; without
        one, a fresh one comes from torch's caching allocator, tied to the
        launch stream."""
        torch = _torch()
        nbytes = kern.batched_workspace_bytes(bpr, batch)
        if workspace is None:
            workspace = torch.empty(max(nbytes, 1), dtype=torch.uint8, device="cuda")
            if isinstance(stream, torch.cuda.Stream):
                workspace.record_stream(stream)
        if workspace.numel() * workspace.element_size() < nbytes:
            raise BackendError("Runtime", "matvec_q4k_batched: workspace too small")
        _chk(_lib.load().launch_matvec_q4k_batched(
            w, X, Y, out_dim, bpr, batch, workspace.data_ptr(),
            workspace.numel() * workspace.element_size(), _stream_ptr(stream)),
            "matvec_q4k_batched")

    @staticmethod
    def gemm_q4k_f16(w: int, a: int, c: int, out_dim: int, bpr: int, m_tokens: int,
                     stream=None) -> None:
        _chk(_lib.load().launch_gemm_q4k_f16(w, a, c, out_dim, bpr, m_tokens,
                                             _stream_ptr(stream)), "gemm_q4k_f16")

    @staticmethod
    def dequant_q4k(q: int, n_blocks: int, out: int, stream=None) -> None:
        _chk(_lib.load().launch_dequant_q4k_ex(q, n_blocks, out, _stream_ptr(stream)),
             "dequant_q4k")


class ops:
    """ops.rs façade for the Q4_K op."""

    @staticmethod
    def dequant_q4k_resident(q4k_dev: int, fp32_dev: int, n_blocks: int) -> None:
        """ops.rs:531-539 -> Op::DequantQ4KResident (rocm.rs:2988-3005)."""
        if n_blocks <= 0:
            raise BackendError("Runtime", "dequant_q4k_resident: n_blocks must be > 0")
        _chk(_lib.load().launch_dequant_q4k(q4k_dev, n_blocks, fp32_dev), "launch_dequant_q4k")


def op_matvec(dtype: int, w: int, x: int, y: int, out_dim: int, in_dim: int,
              layout: int = _lib.LAYOUT_ROWS) -> "_lib.OpDesc":
    """y = W x for a Q4_K/Q5_K/Q6_K weight (mgq_op_desc MGQ_OP_MATVEC)."""
    return _lib.OpDesc(op=_lib.OP_MATVEC, dtype=dtype, layout=layout, w=w, x=x, y=y,
                       out_dim=out_dim, in_dim=in_dim)


def op_matvec_norm(w: int, x: int, norm_w: int, eps: float, y: int, out_dim: int,
                   in_dim: int, dtype: int = _lib.DTYPE_Q4_K) -> "_lib.OpDesc":
    """y = W rms_norm(x) in one fused kernel: Q4_K, or Q6_K where
    q6k_norm_fits(w, out_dim, in_dim // 256)."""
    return _lib.OpDesc(op=_lib.OP_MATVEC_NORM, dtype=dtype, w=w, x=x, norm_w=norm_w,
                       eps=eps, y=y, out_dim=out_dim, in_dim=in_dim)


def q6k_norm_fits(w: int, out_dim: int, bpr: int) -> bool:
    """Whether the fused RMSNorm -> Q6_K matvec takes this tensor: 16-byte
    aligned, whole 16-byte chunks (210-byte blocks), K <= 14 blocks."""
    return w % 16 == 0 and (out_dim * bpr * 210) % 16 == 0 and bpr <= 14


def op_matvec_glu(w_gate: int, w_up: int, x: int, y: int, out_dim: int, in_dim: int,
                  norm_w: int | None = None, eps: float = 0.0,
                  act: int = _lib.ACT_GELU_TANH) -> "_lib.OpDesc":
    """y = act(W_gate xn) * (W_up xn), xn = rms_norm(x) if norm_w (Q4_K)."""
    return _lib.OpDesc(op=_lib.OP_MATVEC_GLU, dtype=_lib.DTYPE_Q4_K, act=act, w=w_gate, w2=w_up,
                       x=x, norm_w=norm_w, eps=eps, y=y, out_dim=out_dim, in_dim=in_dim)


def op_rms_norm(x: int, norm_w: int, y: int, rows: int, hidden: int,
                eps: float) -> "_lib.OpDesc":
    return _lib.OpDesc(op=_lib.OP_RMS_NORM, x=x, norm_w=norm_w, y=y, rows=rows, in_dim=hidden,
                       eps=eps)


def op_glu(gate: int, up: int, y: int, n: int, act: int = _lib.ACT_GELU_TANH) -> "_lib.OpDesc":
    return _lib.OpDesc(op=_lib.OP_GLU, act=act, x=gate, x2=up, y=y, out_dim=n)


def op_residual_add(h: int, x: int, n: int) -> "_lib.OpDesc":
    """h += x."""
    return _lib.OpDesc(op=_lib.OP_RESIDUAL_ADD, x=x, y=h, out_dim=n)


def op_quantize_q8_1(x: int, xq: int, xd: int, xsum: int, n: int) -> "_lib.OpDesc":
    """x (n f32) -> Q8_1 xq, xd, xsum (launch_quantize_q8_1, rocm.rs:477)."""
    return _lib.OpDesc(op=_lib.OP_QUANTIZE_Q8_1, x=x, xq=xq, xd=xd, xsum=xsum, in_dim=n)


def op_matvec_dp4a(dtype: int, w: int, xq: int, xd: int, xsum: int, y: int, out_dim: int,
                   in_dim: int) -> "_lib.OpDesc":
    """y = W . Q8_1(xq, xd, xsum) for Q4_K or Q6_K weights
    (launch_matvec_q4k_dp4a / launch_matvec_q6k_dp4a, rocm.rs:478-491)."""
    return _lib.OpDesc(op=_lib.OP_MATVEC_DP4A, dtype=dtype, w=w, xq=xq, xd=xd, xsum=xsum, y=y,
                       out_dim=out_dim, in_dim=in_dim)


def op_quantize_matvec_dp4a(w: int, x: int, y: int, out_dim: int, in_dim: int) -> "_lib.OpDesc":
    """op_quantize_q8_1 then op_matvec_dp4a (Q4_K) in one launch, same bits."""
    return _lib.OpDesc(op=_lib.OP_QUANTIZE_MATVEC_DP4A, dtype=_lib.DTYPE_Q4_K, w=w, x=x, y=y,
                       out_dim=out_dim, in_dim=in_dim)


class Chain:
    """A decode step's row-aligned matvecs as one launchable chain
    (mgq_chain_create_ex): a persistent kernel (mode CHAIN_PERSISTENT), a
    HIP graph (CHAIN_GRAPH) or the launches enqueued one by one at every
    launch (CHAIN_EAGER); CHAIN_AUTO takes the graph unless the
    environment variable MGQ_CHAIN=persistent is set. Each launch runs the
    matvecs in order, each seeing the earlier ones' outputs."""

    def __init__(self, descs, mode: int = _lib.CHAIN_AUTO):
        if descs is None:  # from_ops
            return
        arr = (_lib.GemvDesc * len(descs))()
        for i, (w, x, y, out_dim, bpr) in enumerate(descs):
            arr[i] = _lib.GemvDesc(w, x, y, out_dim, bpr)
        h = ctypes.c_void_p()
        _chk(_lib.load().mgq_chain_create_ex(arr, len(descs), mode, ctypes.byref(h)),
             "mgq_chain_create_ex")
        self._h = h
        self.n = len(descs)

    @classmethod
    def from_ops(cls, ops) -> "Chain":
        """A chain of mgq_op_desc kernels (mixed Q4_K/Q5_K/Q6_K matvecs, fused
        RMSNorm/GLU matvecs and the glue kernels) recorded into one HIP graph
        (mgq_chain_create_ops)."""
        ops = list(ops)
        arr = (_lib.OpDesc * len(ops))(*ops)
        h = ctypes.c_void_p()
        _chk(_lib.load().mgq_chain_create_ops(arr, len(ops), ctypes.byref(h)),
             "mgq_chain_create_ops")
        self = cls(None)
        self._h = h
        self.n = len(ops)
        return self

    def launch(self, stream=None) -> None:
        _chk(_lib.load().mgq_chain_launch(self._h, _stream_ptr(stream)), "mgq_chain_launch")

    def mode(self) -> int:
        m = ctypes.c_int(-1)
        _chk(_lib.load().mgq_chain_info(self._h, ctypes.byref(m), None), "mgq_chain_info")
        return m.value

    def faults(self) -> int:
        """Nonzero when a grid-wide wait of the persistent kernel gave up in
        some launch (synchronizes with the device)."""
        f = ctypes.c_uint(0)
        _chk(_lib.load().mgq_chain_info(self._h, None, ctypes.byref(f)), "mgq_chain_info")
        return f.value

    def close(self) -> None:
        if self._h:
            _chk(_lib.load().mgq_chain_destroy(self._h), "mgq_chain_destroy")
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class HipBatch:
    """Dispatch counter that drains the device every `sync_every` queued
    kernels (rocm.rs:1089-1211), so long runs of resident dispatches cannot
    pile up unsynchronized. Resident ops call note_dispatch() after queueing
    a kernel; flush() drains now; a batch with pending work drains when it is
    dropped."""

    DEFAULT_SYNC_EVERY = 256

    def __init__(self, sync_every: int = DEFAULT_SYNC_EVERY):
        if sync_every < 1:
            raise ValueError("HipBatch::with_sync_every: n must be >= 1")
        self.sync_every = sync_every
        self.pending = 0

    @classmethod
    def new(cls) -> "HipBatch":
        return cls()

    @classmethod
    def with_sync_every(cls, n: int) -> "HipBatch":
        return cls(n)

    def note_dispatch(self) -> None:
        n = self.pending + 1
        if n >= self.sync_every:
            self.pending = 0  # reset even when the drain fails
            self._sync("HipBatch sync (every %d)" % self.sync_every)
        else:
            self.pending = n

    def flush(self) -> None:
        self.pending = 0
        self._sync("HipBatch::flush")

    @staticmethod
    def _sync(what: str) -> None:
        try:
            _torch().cuda.synchronize()
        except BackendError:
            raise
        except RuntimeError as e:
            raise BackendError("Runtime", f"{what}: {e}") from e

    def __del__(self):
        if getattr(self, "pending", 0) > 0:
            try:
                _torch().cuda.synchronize()
            except Exception:
                pass


class ResidencyError(Exception):
    """Error of a device-resident dispatch (compute/src/backend.rs:244-278):
    either a wrapped BackendError (`backend`) or a GpuVec of the wrong
    residency variant handed to a Hip-only entry point (`expected`, `got`)."""

    def __init__(self, backend: BackendError | None = None, expected: str | None = None,
                 got: str | None = None):
        self.backend, self.expected, self.got = backend, expected, got
        if backend is not None:
            super().__init__(str(backend))
        else:
            super().__init__(f"wrong GpuVec variant: expected {expected}, got {got}")

    @classmethod
    def wrong_variant(cls, expected: str, got: str) -> "ResidencyError":
        return cls(expected=expected, got=got)


class GpuVec:
    """An f32 vector on the host heap or resident on the device
    (compute/src/backend.rs:35-205).

    Variants are "Heap" (a numpy array) and "Hip" (a HipBuffer). The
    reference's third variant, "Vram", is its gfx1102 KFD arena mapped
    through the PCIe BAR; this build has no such arena, so try_vram takes
    the reference's own fallback and returns a Heap vector.
    """

    def __init__(self, heap: np.ndarray | None = None, hip: HipBuffer | None = None):
        if (heap is None) == (hip is None):
            raise ValueError("GpuVec holds exactly one of a heap array or a HipBuffer")
        self._heap = None if heap is None else np.ascontiguousarray(heap, np.float32).ravel()
        self._hip = hip

    @classmethod
    def heap(cls, n: int) -> "GpuVec":
        return cls(heap=np.zeros(n, np.float32))

    @classmethod
    def from_host(cls, v) -> "GpuVec":
        """From<Vec<f32>>: a Heap vector."""
        return cls(heap=np.array(v, np.float32, copy=True).ravel())

    @classmethod
    def try_vram(cls, n: int) -> "GpuVec":
        return cls.heap(n)

    @classmethod
    def try_hip(cls, n: int) -> "GpuVec":
        """A device-resident vector of n floats; allocation failure raises
        ResidencyError wrapping the BackendError."""
        try:
            return cls(hip=HipBuffer.new(4 * n))
        except BackendError as e:
            raise ResidencyError(backend=e) from e

    def variant_name(self) -> str:
        return "Heap" if self._hip is None else "Hip"

    def hip_buffer(self) -> HipBuffer:
        """The HipBuffer of a Hip vector; WrongVariant otherwise."""
        if self._hip is None:
            raise ResidencyError.wrong_variant("Hip", self.variant_name())
        return self._hip

    def __len__(self) -> int:
        return self._heap.size if self._hip is None else self._hip.len_f32()

    def len(self) -> int:
        return len(self)

    def is_host_visible(self) -> bool:
        return self._hip is None

    def copy_from(self, src) -> None:
        """Copy a host slice into the front of this vector (an explicit
        host-to-device copy for Hip)."""
        a = np.ascontiguousarray(src, np.float32).ravel()
        if self._hip is None:
            if a.size > self._heap.size:
                raise ValueError(f"copy_from: src {a.size} > len {self._heap.size}")
            self._heap[: a.size] = a
        else:
            self._hip.copy_from_host(a)

    def as_slice(self) -> np.ndarray:
        """The host array of a Heap vector. A Hip vector is not host-visible
        and raises, as the reference panics (backend.rs:139-151)."""
        if self._hip is not None:
            raise ResidencyError.wrong_variant("Heap or Vram", "Hip")
        return self._heap

    def copy_to_host(self) -> np.ndarray:
        """A host copy of the contents (a device-to-host copy for Hip)."""
        return self._heap.copy() if self._hip is None else self._hip.copy_to_host()

    def clone(self) -> "GpuVec":
        """Always a Heap vector; a Hip vector is downloaded first
        (backend.rs:45-61)."""
        return GpuVec(heap=self.copy_to_host())


# Where the reference quantizer takes sub-block `is` of each 256-element block
# from: elements start[is] .. start[is] + 31 (gguf.rs:590-601, its "legacy"
# order), while every decoder -- the reference's own host dequantize_row_q4_k
# (gguf.rs:364-404), its CPU matvec (llm.rs:684-806) and this library -- puts
# sub-block is at elements 32*is .. 32*is + 31 (canonical ggml order).
LEGACY_SUBBLOCK_START = (0, 128, 32, 160, 64, 192, 96, 224)
_LEGACY_POS = np.concatenate([np.arange(s, s + 32) for s in LEGACY_SUBBLOCK_START])


def legacy_quantizer_input(weight) -> np.ndarray:
    """The flattened weight reordered so that a legacy-order quantizer emits
    canonical Q4_K bytes: within each 256-element block, x'[start[is] + l] =
    w[32*is + l]. The quantizer reads sub-block is from x'[start[is] ..] =
    w[32*is ..] and packs it where the canonical decoder looks for sub-block
    is, so the bytes decode to (a quantization of) w itself, in place."""
    w = np.ascontiguousarray(weight, dtype=np.float32).reshape(-1, Q4K_BLOCK_ELEMS)
    out = np.empty_like(w)
    out[:, _LEGACY_POS] = w
    return out.ravel()


def _hip_of(v, what: str) -> HipBuffer:
    if isinstance(v, HipBuffer):
        return v
    if isinstance(v, GpuVec):
        return v.hip_buffer()
    raise ResidencyError.wrong_variant("Hip", f"{type(v).__name__} ({what})")


class LinearResidentQuantized:
    """Q4_K-quantised resident linear layer (neuron.rs:897-1108).

    Host keeps the Q4_K bytes of the flattened [out x in] weight plus an f32
    bias. Unlike the reference, forward() runs the fused Q4_K GEMV directly on
    the resident Q4_K bytes (0.5625 B/weight) instead of dequantising to an f32
    weight and calling hipblasSgemv (4 B/weight); ensure_resident() still
    materialises the f32 weight via the dequant kernel so dequant-based
    callers and the evict/re-dequant determinism check keep working.
    """

    Q4K_BLOCK_ELEMS = Q4K_BLOCK_ELEMS

    def __init__(self, q4k_bytes: np.ndarray, bias: np.ndarray, in_dim: int, out_dim: int):
        self.host_weight_q4k = np.ascontiguousarray(q4k_bytes, dtype=np.uint8)
        self.host_bias = np.ascontiguousarray(bias, dtype=np.float32)
        self._in, self._out = in_dim, out_dim
        self.weight_q4k_dev = None
        self.weight_dev = None
        self.bias_dev = None

    @classmethod
    def from_q4k(cls, q4k_bytes, bias, in_dim: int, out_dim: int) -> "LinearResidentQuantized":
        """Wrap already-quantized bytes (the reference's from_linear quantizes on
        the host with quantize_row_q4_k, gguf.rs:581-663, neuron.rs:931-951)."""
        if (in_dim * out_dim) % Q4K_BLOCK_ELEMS:
            raise ResidencyError.wrong_variant("weight len multiple of 256",
                                               "weight len not aligned to Q4_K block")
        if np.asarray(q4k_bytes).size != in_dim * out_dim // 256 * Q4K_BLOCK_BYTES:
            raise ResidencyError.wrong_variant("q4k bytes of (in_dim*out_dim/256)*144",
                                               "q4k byte count does not match dims")
        if np.asarray(bias).size != out_dim:
            raise ResidencyError.wrong_variant("bias of out_dim floats",
                                               f"bias of {np.asarray(bias).size}")
        return cls(q4k_bytes, bias, in_dim, out_dim)

    @classmethod
    def from_linear(cls, weight, bias, in_dim: int, out_dim: int, quantize_row_q4_k,
                    legacy_order: bool = True) -> "LinearResidentQuantized":
        """neuron.rs:931-951: quantize the flattened [out_dim x in_dim] f32
        weight on the host and keep the f32 bias. `quantize_row_q4_k` is the
        host's own quantizer (the reference's gguf.rs:581-663 stays on the
        Rust side; it maps n*256 floats to n*144 bytes). That quantizer packs
        sub-blocks in its legacy order; with legacy_order the weight is first
        reordered by legacy_quantizer_input, so the bytes are canonical and
        forward() computes W x + b of this very W. (legacy_order=False is for
        a quantizer that is canonical already.) A weight whose length is not
        a multiple of 256 is WrongVariant, as in the reference."""
        w = np.ascontiguousarray(weight, dtype=np.float32).ravel()
        if w.size != in_dim * out_dim:
            raise ResidencyError.wrong_variant("weight of out_dim*in_dim floats",
                                               f"weight of {w.size}")
        if w.size % Q4K_BLOCK_ELEMS:
            raise ResidencyError.wrong_variant("weight len multiple of 256",
                                               "weight len not aligned to Q4_K block")
        q = np.asarray(quantize_row_q4_k(legacy_quantizer_input(w) if legacy_order else w),
                       dtype=np.uint8)
        return cls.from_q4k(q, bias, in_dim, out_dim)

    def in_dim(self) -> int:
        return self._in

    def out_dim(self) -> int:
        return self._out

    def is_resident(self) -> bool:
        return (self.weight_dev is not None and self.bias_dev is not None
                and self.weight_q4k_dev is not None)

    def host_size_bytes(self) -> int:
        return self.host_weight_q4k.size + self.host_bias.size * 4

    def dequant_size_bytes(self) -> int:
        return self.host_weight_q4k.size + self._in * self._out * 4 + self.host_bias.size * 4

    def ensure_resident(self, batch: HipBatch | None = None) -> None:
        """Upload, dequantize and stage the bias unless resident
        (neuron.rs:1018-1038); the dequant kernel counts against `batch`."""
        if self.is_resident():
            return
        q = HipBuffer(self.host_weight_q4k.size)
        q.copy_from_host_bytes(self.host_weight_q4k)
        wf = HipBuffer(self._in * self._out * 4)
        ops.dequant_q4k_resident(q.device_ptr(), wf.device_ptr(),
                                 self.host_weight_q4k.size // Q4K_BLOCK_BYTES)
        if batch is not None:
            batch.note_dispatch()
        b = HipBuffer(self.host_bias.size * 4)
        b.copy_from_host(self.host_bias)
        self.weight_q4k_dev, self.weight_dev, self.bias_dev = q, wf, b

    def evict(self) -> None:
        self.weight_q4k_dev = self.weight_dev = self.bias_dev = None

    def forward(self, x_dev, out_dev, auto_evict: bool = False, stream=None,
                batch: HipBatch | None = None) -> None:
        """out = W x + b, W the canonical dequant of the resident Q4_K bytes
        (neuron.rs:1059-1108). x_dev and out_dev are HipBuffers or Hip
        GpuVecs; a Heap GpuVec raises ResidencyError WrongVariant, as in the
        reference. The bias is added after the product, one rounding, as
        hipblasSgemv's beta = 1 on a bias-filled y does (rocm.rs:2000-2056).
        With a HipBatch, every kernel queued here counts against it."""
        x_buf, out_buf = _hip_of(x_dev, "x"), _hip_of(out_dev, "out")
        self.ensure_resident(batch)
        kern.matvec_q4k_ex(self.weight_q4k_dev.device_ptr(), x_buf.device_ptr(),
                           out_buf.device_ptr(), self._out, self._in, _lib.LAYOUT_FLAT, stream)
        if batch is not None:
            batch.note_dispatch()
        kern.residual_add(out_buf.device_ptr(), self.bias_dev.device_ptr(), self._out, stream)
        if batch is not None:
            batch.note_dispatch()
        if auto_evict:
            self.evict()
