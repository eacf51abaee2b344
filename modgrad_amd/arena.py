"""Consolidated weight arena: every weight of a model in ONE device
allocation, with a byte offset per tensor, and matvecs dispatched by each
tensor's own quantization type.

Reference: RocmGemma::load packs all quantized layer weights into one
HipBuffer with per-tensor offsets (crates/modgrad-gemma/src/rocm_gemma.rs:
210-224, "less VRAM fragmentation than hundreds of hipMallocs"), and
RocmGemma::qmatvec picks the kernel from the tensor's actual dtype
(rocm_gemma.rs:303-330: Q5_K -> matvec_q5k, Q6_K -> matvec_q6k, Q4_K -> the
dp4a pair or the f32 matvec).

Differences, both for the matrix-core path:
  * each tensor's offset is rounded up to `align` (256 B by default); the
    reference packs tensors back to back, which leaves a tensor that follows
    an odd number of 210-byte Q6_K blocks only 2-byte aligned, and the
    matrix-core matvec needs 16-byte aligned weights;
  * f32 tensors (norm weights) may live in the same allocation.
torch supplies the device memory (one `torch.empty`) and streams; the
matvecs are the library's C ABI (modgrad_amd.q4k.kern).
"""
from __future__ import annotations

import warnings

import numpy as np

from . import _lib
from .gguf import GgmlType, GgufFile, data_size
from .q4k import (BackendError, _stream_ptr, kern, op_matvec, op_matvec_glu, op_matvec_norm,
                  q6k_norm_fits)

ALIGN = 256


def plan_offsets(sizes: list[int], align: int = ALIGN) -> tuple[list[int], int]:
    """Offsets of consecutive tensors of the given byte sizes, each rounded
    up to `align`, and the total allocation size."""
    if align <= 0 or align & (align - 1):
        raise ValueError("align must be a power of two")
    offs, pos = [], 0
    for s in sizes:
        pos = (pos + align - 1) // align * align
        offs.append(pos)
        pos += int(s)
    return offs, pos


class WeightArena:
    """Device-resident weights: name -> (dims, dtype, byte offset)."""

    def __init__(self, entries: list[tuple[str, list[int], GgmlType]], align: int = ALIGN):
        import torch
        self.align = align
        self.names = [e[0] for e in entries]
        self.dims = {n: list(d) for n, d, _ in entries}
        self.dtype = {n: GgmlType(t) for n, _, t in entries}
        sizes = [data_size(GgmlType(t), max(int(np.prod(d)), 1)) for _, d, t in entries]
        offs, total = plan_offsets(sizes, align)
        self.offset = dict(zip(self.names, offs))
        self.nbytes = dict(zip(self.names, sizes))
        self.total_bytes = total
        self.buf = torch.empty(max(total, 1), dtype=torch.uint8, device="cuda")
        self._base = self.buf.data_ptr()

    # -- construction --------------------------------------------------------
    @classmethod
    def from_gguf(cls, g: GgufFile, names: list[str] | None = None,
                  align: int = ALIGN) -> "WeightArena":
        """All (or the named) tensors of an opened GGUF file, uploaded in file
        order from the memory map."""
        names = list(g.tensor_list) if names is None else list(names)
        for n in names:
            t = g.tensors.get(n)
            if t is None:
                raise BackendError("Runtime", f"missing {n}")
            if t.dtype == GgmlType.UNKNOWN:
                raise BackendError("Unsupported", f"{n}: GGML type {t.dtype_id}")
        a = cls([(n, g.tensors[n].dims, g.tensors[n].dtype) for n in names], align)
        for n in names:
            a.upload(n, g.tensor_bytes(n))
        return a

    @classmethod
    def from_arrays(cls, items: list[tuple[str, list[int], GgmlType, object]],
                    align: int = ALIGN) -> "WeightArena":
        """Tensors given as (name, dims, dtype, bytes-like)."""
        a = cls([(n, d, t) for n, d, t, _ in items], align)
        for n, _, _, data in items:
            a.upload(n, data)
        return a

    def upload(self, name: str, data) -> None:
        import torch
        src = np.frombuffer(data, dtype=np.uint8)
        if src.size != self.nbytes[name]:
            raise BackendError("Runtime", f"{name}: {src.size} bytes, expected {self.nbytes[name]}")
        o = self.offset[name]
        with warnings.catch_warnings():
            warnings.simplefilter("ignore")  # read-only views of the file map
            self.buf[o: o + src.size].copy_(torch.from_numpy(src))

    # -- access --------------------------------------------------------------
    def ptr(self, name: str) -> int:
        """Device address of a tensor (the reference's qbase.u8_at(qoff))."""
        return self._base + self.offset[name]

    def shape(self, name: str) -> tuple[int, int]:
        """(out_dim N, in_dim K) of a 2-D weight: dims[1], dims[0]."""
        d = self.dims[name]
        if len(d) != 2:
            raise BackendError("Runtime", f"{name}: not a matrix (dims {d})")
        return d[1], d[0]

    def tensor(self, name: str):
        """The tensor's bytes as a uint8 view of the arena."""
        o = self.offset[name]
        return self.buf[o: o + self.nbytes[name]]

    # -- matvecs -------------------------------------------------------------
    def qmatvec(self, name: str, x: int, y: int, stream=None, q8=None) -> None:
        """y = W x for W = `name`, by its quantization type (rocm_gemma.rs:
        303-330). q8 = (xq, xd, xsum) device buffers selects the dp4a path
        for Q4_K, as the reference engine does by default."""
        n, k = self.shape(name)
        if k % 256:
            raise BackendError("Runtime", f"{name}: in_dim {k} is not a multiple of 256")
        w, bpr, t = self.ptr(name), k // 256, self.dtype[name]
        if t == GgmlType.Q5_K:
            kern.matvec_q5k(w, x, y, n, bpr, stream)
        elif t == GgmlType.Q6_K:
            kern.matvec_q6k(w, x, y, n, bpr, stream)
        elif t == GgmlType.Q4_K:
            if q8 is not None:
                xq, xd, xsum = q8
                kern.quantize_q8_1(x, xq, xd, xsum, k, stream)
                kern.matvec_q4k_dp4a(w, xq, xd, xsum, y, n, bpr, stream)
            else:
                kern.matvec_q4k_ex(w, x, y, n, k, _lib.LAYOUT_ROWS, stream)
        else:
            raise BackendError("Unsupported", f"{name}: no matvec for {t.name}")

    def norm_fusable(self, name: str) -> bool:
        """Whether y = W rms_norm(x) runs as one launch for this tensor: Q4_K
        always, Q6_K where the fused kernel takes it (q4k.q6k_norm_fits)."""
        n, k = self.shape(name)
        t = self.dtype[name]
        if t == GgmlType.Q4_K:
            return True
        return t == GgmlType.Q6_K and k % 256 == 0 and q6k_norm_fits(self.ptr(name), n, k // 256)

    def qmatvec_rmsnorm(self, name: str, x: int, norm: str, eps: float, y: int,
                        stream=None) -> None:
        """y = W rms_norm(x, norm, eps) in one launch (Q4_K weights, or Q6_K
        where norm_fusable)."""
        n, k = self.shape(name)
        self._need(norm, GgmlType.F32)
        if self.dtype[name] == GgmlType.Q6_K and self.norm_fusable(name):
            kern.matvec_q6k_rmsnorm(self.ptr(name), x, self.ptr(norm), eps, y, n, k // 256, stream)
            return
        self._need(name, GgmlType.Q4_K)
        kern.matvec_q4k_rmsnorm(self.ptr(name), x, self.ptr(norm), eps, y, n, k // 256, stream)

    def qmatvec_glu(self, gate: str, up: str, x: int, y: int, norm: str | None = None,
                    eps: float = 0.0, act: int = _lib.ACT_GELU_TANH, stream=None) -> None:
        """y = act(W_gate xn) * (W_up xn), xn = rms_norm(x) if `norm` (Q4_K)."""
        n, k = self.shape(gate)
        if self.shape(up) != (n, k):
            raise BackendError("Runtime", f"{gate} and {up} differ in shape")
        self._need(gate, GgmlType.Q4_K)
        self._need(up, GgmlType.Q4_K)
        nw = None
        if norm is not None:
            self._need(norm, GgmlType.F32)
            nw = self.ptr(norm)
        kern.matvec_q4k_glu(self.ptr(gate), self.ptr(up), x, y, n, k // 256, nw, eps, act, stream)

    # -- the same calls as mgq_op_desc descriptors, for a recorded chain
    #    (q4k.Chain.from_ops): RocmGemma's per-layer chain through the C ABI
    def op_qmatvec(self, name: str, x: int, y: int) -> "_lib.OpDesc":
        """Descriptor of y = W x, the kernel picked by W's dtype."""
        n, k = self.shape(name)
        t = self.dtype[name]
        if t not in (GgmlType.Q4_K, GgmlType.Q5_K, GgmlType.Q6_K):
            raise BackendError("Unsupported", f"{name}: no matvec for {t.name}")
        if k % 256:
            raise BackendError("Runtime", f"{name}: in_dim {k} is not a multiple of 256")
        return op_matvec(int(t), self.ptr(name), x, y, n, k)

    def op_qmatvec_rmsnorm(self, name: str, x: int, norm: str, eps: float,
                           y: int) -> "_lib.OpDesc":
        n, k = self.shape(name)
        self._need(norm, GgmlType.F32)
        if self.dtype[name] == GgmlType.Q6_K and self.norm_fusable(name):
            return op_matvec_norm(self.ptr(name), x, self.ptr(norm), eps, y, n, k, _lib.DTYPE_Q6_K)
        self._need(name, GgmlType.Q4_K)
        return op_matvec_norm(self.ptr(name), x, self.ptr(norm), eps, y, n, k)

    def op_qmatvec_glu(self, gate: str, up: str, x: int, y: int, norm: str | None = None,
                       eps: float = 0.0, act: int = _lib.ACT_GELU_TANH) -> "_lib.OpDesc":
        n, k = self.shape(gate)
        if self.shape(up) != (n, k):
            raise BackendError("Runtime", f"{gate} and {up} differ in shape")
        self._need(gate, GgmlType.Q4_K)
        self._need(up, GgmlType.Q4_K)
        nw = None
        if norm is not None:
            self._need(norm, GgmlType.F32)
            nw = self.ptr(norm)
        return op_matvec_glu(self.ptr(gate), self.ptr(up), x, y, n, k, nw, eps, act)

    def _need(self, name: str, t: GgmlType) -> None:
        if self.dtype[name] != t:
            raise BackendError("Unsupported", f"{name}: {self.dtype[name].name}, needs {t.name}")
