"""C-ABI checks that need no GPU: the library loads, exports every symbol the
header declares, and rejects invalid arguments before touching the device
(the reference's hipErrorInvalidValue contract, matvec_q4k.hip:118,
dequant_q4k.hip:152)."""
import ctypes
import subprocess

import pytest

from modgrad_amd import _lib

NOT_SUPPORTED = 801  # hipErrorNotSupported
INVALID = _lib.hipErrorInvalidValue
FAKE = 0x10000  # never dereferenced: every call below fails validation first


@pytest.fixture(scope="module")
def L():
    return _lib.load()


def test_exports_every_declared_symbol(L):
    declared = _lib.declared_symbols()
    assert {"launch_matvec_q4k", "launch_dequant_q4k"} <= set(declared)
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = [s for s in declared if s not in exported]
    assert not missing, missing
    for s in declared:
        getattr(L, s)


def test_version(L):
    assert L.mgq_version().startswith(b"modgrad_q4k")


def test_matvec_rejects_nonpositive_dims(L):
    assert L.launch_matvec_q4k(FAKE, FAKE, FAKE, 0, 14) == INVALID
    assert L.launch_matvec_q4k(FAKE, FAKE, FAKE, 16, 0) == INVALID
    assert L.launch_matvec_q4k(FAKE, FAKE, FAKE, -1, 14) == INVALID
    assert L.launch_matvec_q4k(FAKE, FAKE, FAKE, 16, 1 << 24) == INVALID  # K overflows int


def test_dp4a_path_rejects_bad_args(L):
    # launch_quantize_q8_1: fewer than one 32-value sub-block, null, a float
    # pointer off float alignment (the int8 xq may start at any byte)
    assert L.launch_quantize_q8_1(FAKE, FAKE, FAKE, FAKE, 31) == INVALID
    assert L.launch_quantize_q8_1(FAKE, FAKE, FAKE, FAKE, 0) == INVALID
    assert L.launch_quantize_q8_1(None, FAKE, FAKE, FAKE, 64) == INVALID
    assert L.launch_quantize_q8_1(FAKE + 2, FAKE, FAKE, FAKE, 64) == INVALID
    assert L.launch_quantize_q8_1(FAKE, FAKE + 1, FAKE + 1, FAKE, 64) == INVALID
    # launch_matvec_q4k_dp4a: reference checks (matvec_q4k_dp4a.hip:111) + pointers
    assert L.launch_matvec_q4k_dp4a(FAKE, FAKE, FAKE, FAKE, FAKE, 0, 14) == INVALID
    assert L.launch_matvec_q4k_dp4a(FAKE, FAKE, FAKE, FAKE, FAKE, 16, 0) == INVALID
    assert L.launch_matvec_q4k_dp4a(FAKE, None, FAKE, FAKE, FAKE, 16, 1) == INVALID
    assert L.launch_matvec_q4k_dp4a(FAKE, FAKE, FAKE, FAKE + 2, FAKE, 16, 1) == INVALID


def test_q5k_q6k_reject_bad_args(L):
    for fn in (L.launch_matvec_q5k, L.launch_matvec_q6k):
        assert fn(FAKE, FAKE, FAKE, 0, 14) == INVALID
        assert fn(FAKE, FAKE, FAKE, 16, 0) == INVALID
        assert fn(None, FAKE, FAKE, 16, 1) == INVALID
        assert fn(FAKE, FAKE + 2, FAKE, 16, 1) == INVALID
    assert L.launch_matvec_q6k_dp4a(FAKE, FAKE, FAKE, FAKE, FAKE, 0, 1) == INVALID
    assert L.launch_matvec_q6k_dp4a(FAKE, None, FAKE, FAKE, FAKE, 8, 1) == INVALID


def test_matvec_rejects_null_and_misaligned_floats(L):
    # weight bytes may start at any byte (the GPU tests run +1/+2/+4 offsets);
    # x and y are float pointers and need float alignment
    assert L.launch_matvec_q4k(None, FAKE, FAKE, 16, 1) == INVALID
    assert L.launch_matvec_q4k(FAKE, None, FAKE, 16, 1) == INVALID
    assert L.launch_matvec_q4k(FAKE + 1, FAKE + 1, FAKE, 16, 1) == INVALID
    assert L.launch_matvec_q4k(FAKE + 3, FAKE, FAKE + 2, 16, 1) == INVALID


def test_matvec_ex_layout_rules(L):
    # row layout needs k % 256 == 0; flat layout needs n*k % 256 == 0
    assert L.launch_matvec_q4k_ex(FAKE, FAKE, FAKE, 16, 300, _lib.LAYOUT_ROWS, None) == INVALID
    assert L.launch_matvec_q4k_ex(FAKE, FAKE, FAKE, 3, 100, _lib.LAYOUT_FLAT, None) == INVALID
    assert L.launch_matvec_q4k_ex(FAKE, FAKE, FAKE, 16, 256, 7, None) == INVALID


def test_dequant_rejects_bad_args(L):
    assert L.launch_dequant_q4k(FAKE, 0, FAKE) == INVALID
    assert L.launch_dequant_q4k(FAKE, -3, FAKE) == INVALID
    assert L.launch_dequant_q4k(None, 1, FAKE) == INVALID
    assert L.launch_dequant_q4k(FAKE, 1, FAKE + 2) == INVALID


def test_batched_workspace_size(L):
    # 9 operand tables of 1 KiB plus 8 (corr, corr_min) pairs per (block, set of 8)
    for bpr, batch in [(1, 1), (14, 8), (14, 9), (74, 16)]:
        sets = (batch + 7) // 8
        assert L.mgq_batched_workspace_bytes(bpr, batch) == bpr * sets * (9 * 1024 + 64)
    assert L.mgq_batched_workspace_bytes(0, 4) == 0
    assert L.mgq_batched_workspace_bytes(4, 17) == 0


def test_batched_and_gemm_reject_bad_args(L):
    ws = L.mgq_batched_workspace_bytes(1, 16)
    assert L.launch_matvec_q4k_batched(FAKE, FAKE, FAKE, 16, 1, 0, FAKE, ws, None) == INVALID
    assert L.launch_matvec_q4k_batched(FAKE, FAKE, FAKE, 16, 1, 17, FAKE, ws, None) == INVALID
    # missing or undersized workspace
    assert L.launch_matvec_q4k_batched(FAKE, FAKE, FAKE, 16, 1, 4, None, ws, None) == INVALID
    assert L.launch_matvec_q4k_batched(FAKE, FAKE, FAKE, 16, 1, 16, FAKE, ws - 1, None) == INVALID
    assert L.launch_gemm_q4k_f16(FAKE, FAKE, FAKE, 16, 1, 0, None) == INVALID
    assert L.launch_gemm_q4k_f16(FAKE, FAKE, FAKE, 0, 1, 4, None) == INVALID


def test_chain_rejects_bad_descs(L):
    h = ctypes.c_void_p()
    assert L.mgq_chain_create(None, 1, ctypes.byref(h)) == INVALID
    arr = (_lib.GemvDesc * 1)(_lib.GemvDesc(FAKE, FAKE, FAKE, 0, 14))
    assert L.mgq_chain_create(arr, 1, ctypes.byref(h)) == INVALID
    assert L.mgq_chain_create(arr, 0, ctypes.byref(h)) == INVALID
    assert L.mgq_chain_launch(None, None) == INVALID
    assert L.mgq_chain_destroy(None) == INVALID


def test_host_api_rejects_misshaped_weights():
    # neuron.rs:933-938: a weight that is not a whole number of Q4_K blocks is
    # ResidencyError::WrongVariant
    import numpy as np
    from modgrad_amd.q4k import LinearResidentQuantized, ResidencyError
    with pytest.raises(ResidencyError) as e:
        LinearResidentQuantized.from_q4k(np.zeros(144, np.uint8), np.zeros(3), 100, 3)
    assert e.value.backend is None and e.value.got == "weight len not aligned to Q4_K block"
    with pytest.raises(ResidencyError):
        LinearResidentQuantized.from_q4k(np.zeros(100, np.uint8), np.zeros(4), 64, 4)
    with pytest.raises(ResidencyError):
        LinearResidentQuantized.from_q4k(np.zeros(144, np.uint8), np.zeros(3), 64, 4)


def test_gpuvec_heap_variant():
    # backend.rs:35-205: the Heap variant is host-visible, clones to Heap, and
    # a Hip-only entry point rejects it with WrongVariant
    import numpy as np
    from modgrad_amd.q4k import GpuVec, LinearResidentQuantized, ResidencyError
    v = GpuVec.heap(8)
    assert v.variant_name() == "Heap" and len(v) == 8 and v.is_host_visible()
    v.copy_from([1.0, 2.0, 3.0])
    assert v.as_slice()[:4].tolist() == [1.0, 2.0, 3.0, 0.0]
    c = v.clone()
    c.as_slice()[0] = 9.0
    assert v.as_slice()[0] == 1.0 and c.variant_name() == "Heap"
    assert GpuVec.try_vram(4).variant_name() == "Heap"  # no KFD BAR arena here
    assert GpuVec.from_host([5.0, 6.0]).copy_to_host().tolist() == [5.0, 6.0]
    with pytest.raises(ResidencyError) as e:
        v.hip_buffer()
    assert (e.value.expected, e.value.got) == ("Hip", "Heap")
    assert str(e.value) == "wrong GpuVec variant: expected Hip, got Heap"
    lin = LinearResidentQuantized.from_q4k(np.zeros(144, np.uint8), np.zeros(1, np.float32),
                                           256, 1)
    with pytest.raises(ResidencyError):
        lin.forward(GpuVec.heap(256), GpuVec.heap(1))
    assert not lin.is_resident()  # the variant check comes before any allocation


def test_hipbatch_counts_dispatches():
    # rocm.rs:1089-1211: a cadence below 1 is rejected; below the cadence a
    # dispatch only counts (the drain itself needs a device)
    from modgrad_amd.q4k import HipBatch
    with pytest.raises(ValueError):
        HipBatch.with_sync_every(0)
    b = HipBatch.new()
    assert b.sync_every == HipBatch.DEFAULT_SYNC_EVERY == 256
    for i in range(255):
        b.note_dispatch()
    assert b.pending == 255
    b.pending = 0  # nothing queued on a device here: let it drop quietly


def test_host_size_savings():
    # neuron.rs:2002-2028: a 1024->256 layer's Q4_K host footprint < 16% of f32
    import numpy as np
    from modgrad_amd.q4k import LinearResidentQuantized
    lin = LinearResidentQuantized.from_q4k(np.zeros(1024 * 256 // 256 * 144, np.uint8),
                                           np.zeros(256, np.float32), 1024, 256)
    ratio = lin.host_size_bytes() / (1024 * 256 * 4 + 256 * 4)
    assert ratio < 0.16 and abs(ratio - 0.1415) < 0.001


def test_glue_rejects_bad_args(L):
    # launch_rms_norm: the reference's n/hidden checks (rms_norm.hip:87-89) + pointers
    assert L.launch_rms_norm(FAKE, FAKE, FAKE, 0, 3584, 1e-6) == INVALID
    assert L.launch_rms_norm(FAKE, FAKE, FAKE, 1, 0, 1e-6) == INVALID
    assert L.launch_rms_norm(None, FAKE, FAKE, 1, 3584, 1e-6) == INVALID
    assert L.launch_geglu(FAKE, FAKE, FAKE, 0) == INVALID
    assert L.launch_geglu(FAKE, None, FAKE, 16) == INVALID
    assert L.launch_glu_ex(FAKE, FAKE, FAKE, 16, 2, None) == INVALID  # unknown activation
    assert L.launch_residual_add(FAKE, FAKE, 0) == INVALID
    assert L.launch_residual_add(None, FAKE, 16) == INVALID
    assert L.launch_residual_add_ex(FAKE, None, 16, None) == INVALID
    assert L.launch_scale(FAKE, 2.0, -1) == INVALID
    assert L.launch_scale_ex(None, 2.0, 16, None) == INVALID


def test_fused_matvecs_reject_bad_args(L):
    rms = L.launch_matvec_q4k_rmsnorm_ex
    assert rms(FAKE, FAKE, FAKE, 1e-6, FAKE, 0, 14, None) == INVALID
    assert rms(FAKE, FAKE, FAKE, 1e-6, FAKE, 16, 0, None) == INVALID
    assert rms(FAKE, FAKE, None, 1e-6, FAKE, 16, 14, None) == INVALID   # norm weights required
    assert rms(FAKE + 1, FAKE + 2, FAKE, 1e-6, FAKE, 16, 14, None) == INVALID  # x off float alignment
    assert rms(FAKE + 1, FAKE, FAKE + 2, 1e-6, FAKE, 16, 14, None) == INVALID  # norm_w likewise
    glu = L.launch_matvec_q4k_glu_ex
    assert glu(FAKE, None, FAKE, None, 0.0, 0, FAKE, 16, 14, None) == INVALID  # up matrix required
    assert glu(FAKE, FAKE, FAKE, None, 0.0, 7, FAKE, 16, 14, None) == INVALID  # unknown activation
    assert glu(FAKE, FAKE + 1, FAKE + 2, None, 0.0, 0, FAKE, 16, 14, None) == INVALID
    assert glu(FAKE, FAKE, FAKE, FAKE + 2, 0.0, 0, FAKE, 16, 14, None) == INVALID
    assert glu(FAKE, FAKE, FAKE, None, 0.0, 1, FAKE, -1, 14, None) == INVALID


def test_fused_quantize_dp4a_rejects_bad_args(L):
    fn = L.launch_quantize_matvec_q4k_dp4a_ex
    assert fn(FAKE, FAKE, FAKE, 0, 14, None) == INVALID
    assert fn(FAKE, FAKE, FAKE, 16, 0, None) == INVALID
    assert fn(FAKE, None, FAKE, 16, 14, None) == INVALID
    assert fn(FAKE + 1, FAKE + 2, FAKE, 16, 14, None) == INVALID   # x off float alignment
    assert fn(FAKE + 1, FAKE, FAKE + 2, 16, 14, None) == INVALID   # y likewise


def test_op_chain_rejects_bad_descriptors_before_any_device_call(L):
    """mgq_chain_create_ops validates every descriptor on the host first, so
    these return hipErrorInvalidValue without touching a device."""
    import ctypes
    h = ctypes.c_void_p()
    good = dict(op=_lib.OP_MATVEC, dtype=_lib.DTYPE_Q4_K, layout=_lib.LAYOUT_ROWS, w=FAKE, x=FAKE,
                y=FAKE, out_dim=16, in_dim=256)
    bad = [dict(op=99), dict(dtype=15), dict(w=None), dict(x=FAKE + 2), dict(in_dim=300),
           dict(out_dim=0), dict(layout=7), dict(dtype=_lib.DTYPE_Q6_K, in_dim=512 + 32),
           dict(op=_lib.OP_MATVEC_NORM),                      # no norm weights
           dict(op=_lib.OP_MATVEC_GLU, w2=FAKE, act=5),       # bad activation
           dict(op=_lib.OP_MATVEC_GLU, dtype=_lib.DTYPE_Q6_K, w2=FAKE),
           dict(op=_lib.OP_RMS_NORM, norm_w=FAKE, rows=0),
           dict(op=_lib.OP_GLU, x2=None),
           dict(op=_lib.OP_RESIDUAL_ADD, out_dim=-1),
           # the dp4a arm: Q8_1 buffers required, K a multiple of 32 / 256,
           # Q4_K or Q6_K weights (Q4_K only when fused with the quantizer)
           dict(op=_lib.OP_QUANTIZE_Q8_1, xq=None, xd=FAKE, xsum=FAKE),
           dict(op=_lib.OP_QUANTIZE_Q8_1, xq=FAKE, xd=FAKE + 2, xsum=FAKE),
           dict(op=_lib.OP_QUANTIZE_Q8_1, xq=FAKE, xd=FAKE, xsum=FAKE, in_dim=48),
           dict(op=_lib.OP_MATVEC_DP4A, xq=FAKE, xd=FAKE, xsum=None),
           dict(op=_lib.OP_MATVEC_DP4A, xq=FAKE, xd=FAKE, xsum=FAKE, dtype=_lib.DTYPE_Q5_K),
           dict(op=_lib.OP_MATVEC_DP4A, xq=FAKE, xd=FAKE, xsum=FAKE, in_dim=288),
           dict(op=_lib.OP_MATVEC_DP4A, xq=None, xd=FAKE, xsum=FAKE, dtype=_lib.DTYPE_Q6_K),
           dict(op=_lib.OP_QUANTIZE_MATVEC_DP4A, dtype=_lib.DTYPE_Q6_K),
           dict(op=_lib.OP_QUANTIZE_MATVEC_DP4A, x=None)]
    for change in bad:
        d = dict(good)
        d.update(change)
        arr = (_lib.OpDesc * 2)(_lib.OpDesc(**good), _lib.OpDesc(**d))
        assert L.mgq_chain_create_ops(arr, 2, ctypes.byref(h)) == INVALID, change
        assert h.value is None
    # the fused RMSNorm Q6_K matvec: no norm weights is invalid; a tensor its
    # whole-row kernel cannot take (K > 14 blocks, w not 16-byte aligned, a
    # size that is not whole 16-byte chunks) is hipErrorNotSupported, still
    # before any device call
    q6n = dict(op=_lib.OP_MATVEC_NORM, dtype=_lib.DTYPE_Q6_K, norm_w=FAKE)
    for change, code in [(dict(norm_w=None), INVALID), (dict(in_dim=300), INVALID),
                         (dict(in_dim=15 * 256), NOT_SUPPORTED), (dict(w=FAKE + 2), NOT_SUPPORTED),
                         (dict(out_dim=3), NOT_SUPPORTED)]:
        d = dict(good)
        d.update(q6n)
        d.update(change)
        arr = (_lib.OpDesc * 2)(_lib.OpDesc(**good), _lib.OpDesc(**d))
        assert L.mgq_chain_create_ops(arr, 2, ctypes.byref(h)) == code, change
        assert h.value is None
    arr = (_lib.OpDesc * 1)(_lib.OpDesc(**good))
    assert L.mgq_chain_create_ops(arr, 0, ctypes.byref(h)) == INVALID
    assert L.mgq_chain_create_ops(None, 1, ctypes.byref(h)) == INVALID
    assert L.mgq_chain_create_ops(arr, 1, None) == INVALID
