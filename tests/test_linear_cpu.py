"""CPU tests of LinearResidentQuantized.from_linear and the quantizer-order
reordering it applies (no GPU: quantization and sizes are host-side).

The reference quantizer (gguf.rs:581-663) packs sub-block `is` from elements
LEGACY_SUBBLOCK_START[is].. of each block, while its own host dequantizer
(gguf.rs:364-404), its CPU matvec and this library decode sub-block is at
elements 32*is.. (canonical order). from_linear reorders the weight before the
quantizer so that the bytes decode to the weight itself. The oracle restates
that quantizer (legacy order) and the canonical dequantizer.
"""
import numpy as np
import pytest

from modgrad_amd.q4k import (LEGACY_SUBBLOCK_START, LinearResidentQuantized, ResidencyError,
                             legacy_quantizer_input)


def rms_rel(got, want) -> float:
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.sqrt(np.sum((got - want) ** 2) / max(np.sum(want ** 2), 1e-300)))


def linear_new_weight(orc, in_dim: int, out_dim: int) -> np.ndarray:
    """Linear::new (neuron.rs:66-74): SimpleRng(in ^ out).next_normal() *
    sqrt(2 / in_dim) in f32, row-major [out][in]."""
    scale = float(np.sqrt(np.float32(2.0) / np.float32(in_dim)))
    return orc.normal(in_dim ^ out_dim, in_dim * out_dim, scale)


def test_reordering_is_the_inverse_of_the_quantizer_order():
    # element 32*is + l of a block lands at LEGACY_SUBBLOCK_START[is] + l
    w = np.arange(512, dtype=np.float32)
    x = legacy_quantizer_input(w).reshape(2, 256)
    for blk in range(2):
        for s, start in enumerate(LEGACY_SUBBLOCK_START):
            assert np.array_equal(x[blk, start:start + 32], w[256 * blk + 32 * s: 256 * blk + 32 * s + 32])
    assert sorted(LEGACY_SUBBLOCK_START) == list(range(0, 256, 32))


def test_constant_sub_blocks_decode_in_place(orc):
    # sub-block is of each block holds the constant c = is + 1 + 10*block. A
    # constant sub-block decodes to d*sc*15 with its 6-bit scale rounded
    # against the block's largest one: within max|w|/126 of c. The canonical
    # decode must return c at elements 32*is.. of the same block.
    nb = 3
    w = np.repeat(np.arange(nb * 8, dtype=np.float32) % 8 + 1, 32)
    w += np.repeat(10.0 * np.arange(nb, dtype=np.float32), 256)
    tol = np.repeat(np.abs(w).reshape(nb, 256).max(axis=1) / 120.0, 256)
    got = orc.dequantize(orc.quantize(legacy_quantizer_input(w)))
    assert np.all(np.abs(got - w) <= tol)
    # without the reordering the same quantizer's bytes decode elsewhere
    plain = orc.dequantize(orc.quantize(w))
    assert not np.all(np.abs(plain - w) <= 0.1 * np.abs(w))


def test_round_trip_gates_pass_only_with_the_reordering(orc):
    # the reference's own round-trip gate (gguf.rs:703-738: 4 blocks of its
    # smooth signal, RMS_rel < 5 %) and the weight-level analogue of its
    # `basic` gate (neuron.rs:1885-1936: the Linear::new(1024, 256) weight,
    # < 10 %): both met through the reordering (1.4 % and 7.8 %), both
    # missed by the raw legacy bytes (43 % and 122 %)
    x = orc.smooth(4 * 256)
    assert rms_rel(orc.dequantize(orc.quantize(legacy_quantizer_input(x))), x) < 0.05
    assert rms_rel(orc.dequantize(orc.quantize(x)), x) > 0.3
    w = linear_new_weight(orc, 1024, 256)
    assert rms_rel(orc.dequantize(orc.quantize(legacy_quantizer_input(w))), w) < 0.10
    assert rms_rel(orc.dequantize(orc.quantize(w)), w) > 1.0


def test_from_linear_sizes_and_host_size_savings(orc):
    # neuron.rs:2002-2028 (host_size_savings): 1024x1024 Q4_K bytes are
    # 144/1024 = 14.06 % of the f32 weight, below the 16 % and 25 % gates
    w = linear_new_weight(orc, 1024, 1024)
    lin = LinearResidentQuantized.from_linear(w, np.zeros(1024, np.float32), 1024, 1024,
                                              orc.quantize)
    assert not lin.is_resident()  # from_linear allocates no device memory
    q_bytes, fp32 = lin.host_size_bytes(), w.size * 4
    assert lin.host_weight_q4k.size == 1024 * 1024 // 256 * 144
    assert q_bytes < fp32 // 4 and q_bytes / fp32 < 0.16
    assert abs(lin.host_weight_q4k.size / fp32 - 144 / 1024) < 1e-12


def test_from_linear_rejects_a_weight_of_partial_blocks(orc):
    # neuron.rs:933-938: WrongVariant when the weight is not whole blocks
    with pytest.raises(ResidencyError) as e:
        LinearResidentQuantized.from_linear(np.zeros(100 * 3, np.float32), np.zeros(3), 100, 3,
                                            orc.quantize)
    assert e.value.got == "weight len not aligned to Q4_K block"
    with pytest.raises(ResidencyError):
        LinearResidentQuantized.from_linear(np.zeros(512, np.float32), np.zeros(4), 256, 4,
                                            orc.quantize)


def test_canonical_table_patch_gives_the_reordered_bytes(orc):
    # the one-line alternative at gguf.rs:601 (sub-block table {0, 32, .., 224})
    # emits exactly the bytes that from_linear's reordering gets out of the
    # shipped quantizer: each sub-block's scale, min and nibbles depend only
    # on its own 32 values and the block-wide maxima
    w = linear_new_weight(orc, 1024, 64)
    patched = orc.quantize_with_offsets(w, [0, 32, 64, 96, 128, 160, 192, 224])
    assert np.array_equal(patched, orc.quantize(legacy_quantizer_input(w)))
    # and the shipped table through the same entry is the shipped quantizer
    assert np.array_equal(orc.quantize_with_offsets(w, LEGACY_SUBBLOCK_START), orc.quantize(w))
