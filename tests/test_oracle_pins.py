"""Pins for the CPU oracle (oracle/q4k_oracle.c): closed forms, invariants and
an independent numpy restatement, chosen so that a plausible transcription
mistake (dropped term, wrong shift, swapped operand, wrong sub-block order)
fails at least one of them. CPU only."""
import math
import struct

import numpy as np
import pytest

from tests import q4k_spec_numpy as spec

OFFS = [0, 128, 32, 160, 64, 192, 96, 224]  # gguf.rs:590-601


def f32(v):
    return np.float32(v)


def trunc_f16_bits(x: np.float32) -> int:
    """Truncation toward zero computed a different way than the oracle:
    numpy's round-to-nearest-even, then one ulp toward zero if it overshot."""
    h = np.array([x], np.float32).astype(np.float16)
    hb = int(h.view(np.uint16)[0])
    if np.isinf(h[0]) and abs(x) < 65536.0:
        return (hb & 0x8000) | 0x7BFF
    if abs(np.float32(h[0])) > abs(x) and (hb & 0x7FFF) != 0:
        hb -= 1
    return hb


# ------------------------------------------------------------ f16 helpers ---
def test_f16_to_f32_exhaustive(orc):
    L = orc.lib()
    for h in range(65536):
        got = L.orq_f16_to_f32(h)
        ref = np.array([h], np.uint16).view(np.float16).astype(np.float32)[0]
        if (h >> 10) & 0x1F == 31:
            assert math.isnan(got), hex(h)  # gguf.rs:291: Inf and NaN -> NaN
        else:
            assert struct.pack("<f", got) == struct.pack("<f", ref), hex(h)


def test_f32_to_f16_truncates(orc):
    L = orc.lib()
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, size=200_000, dtype=np.uint64).astype(np.uint32)
    vals = bits.view(np.float32)
    vals = vals[np.isfinite(vals) & (np.abs(vals) < 65504.0)]
    dense = np.linspace(-70000, 70000, 20001, dtype=np.float32)
    tiny = (np.arange(-2000, 2000, dtype=np.float32) * np.float32(2.0**-30))
    for x in np.concatenate([vals[:50_000], dense, tiny]):
        h = L.orq_f32_to_f16(float(x))
        if abs(x) >= 65536.0:
            assert h & 0x7FFF == 0x7C00
            continue
        assert h == trunc_f16_bits(x), (x, hex(h))
        back = np.array([h], np.uint16).view(np.float16).astype(np.float32)[0]
        assert abs(back) <= abs(x)
        nxt = np.array([(h & 0x7FFF) + 1], np.uint16).view(np.float16).astype(np.float32)[0]
        assert abs(x) < nxt or h & 0x7FFF == 0x7BFF


def test_f32_to_f16_specials(orc):
    L = orc.lib()
    assert L.orq_f32_to_f16(65504.0) == 0x7BFF
    assert L.orq_f32_to_f16(65535.0) == 0x7BFF          # truncation, not Inf
    assert L.orq_f32_to_f16(65536.0) == 0x7C00
    assert L.orq_f32_to_f16(-1e30) == 0xFC00
    assert L.orq_f32_to_f16(float("inf")) == 0x7C00
    assert L.orq_f32_to_f16(float("nan")) & 0x7C00 == 0x7C00
    assert L.orq_f32_to_f16(float("nan")) & 0x3FF != 0
    assert L.orq_f32_to_f16(2.0**-25) == 0x0000          # below half-ulp of subnormal
    assert L.orq_f32_to_f16(2.0**-24) == 0x0001
    assert L.orq_f32_to_f16(-(2.0**-24) * 3.9) == 0x8003
    assert L.orq_f32_to_f16(1.0) == 0x3C00
    assert L.orq_f32_to_f16(1.0 + 2.0**-11) == 0x3C00    # RNE would give 0x3C00 too
    assert L.orq_f32_to_f16(1.0 + 3 * 2.0**-11) == 0x3C01  # RNE would give 0x3C02
    assert L.orq_f32_to_f16(1.0 + 3 * 2.0**-12) == 0x3C00  # RNE would give 0x3C01


# ------------------------------------------------------------ scales -------
def test_scale_pack_unpack_exhaustive(orc):
    rng = np.random.default_rng(2)
    for j in range(8):
        for sc in range(64):
            for m in range(64):
                scs = rng.integers(0, 64, 8)
                ms = rng.integers(0, 64, 8)
                scs[j], ms[j] = sc, m
                packed = orc.pack_scales_mins(scs, ms)
                got = [orc.get_scale_min_k4(i, packed) for i in range(8)]
                assert got == list(zip(scs.tolist(), ms.tolist()))


def test_scale_unpack_matches_spec(orc):
    rng = np.random.default_rng(3)
    s = rng.integers(0, 256, size=(500, 12), dtype=np.uint8)
    sc, m = spec.unpack_scales(s)
    for b in range(500):
        for j in range(8):
            assert orc.get_scale_min_k4(j, s[b].tobytes()) == (sc[b, j], m[b, j])


# ------------------------------------------------------------ dequant ------
def _block(d_bits, dmin_bits, sc, m, qs):
    head = struct.pack("<HH", d_bits, dmin_bits)
    from oracle.oracle import pack_scales_mins
    return np.frombuffer(head + pack_scales_mins(sc, m) + bytes(qs), np.uint8).copy()


def test_dequant_positions_closed_form(orc):
    # d = 1, dmin = 0, every scale 1: output p is its own nibble.
    qs = [(j % 16) | ((15 - j % 16) << 4) for j in range(128)]
    out = orc.dequantize(_block(0x3C00, 0, [1] * 8, [0] * 8, qs))
    p = np.arange(256)
    want = np.where((p // 32) % 2 == 0, p % 16, 15 - p % 16).astype(np.float32)
    assert np.array_equal(out, want)


def test_dequant_subblock_to_position(orc):
    # q = 0, d = 0, dmin = 1, m[is] = is+1: out[p] = -(p//32 + 1).
    out = orc.dequantize(_block(0x0000, 0x3C00, [5] * 8, list(range(1, 9)), [0] * 128))
    assert np.array_equal(out, -(np.arange(256) // 32 + 1).astype(np.float32))


def test_dequant_nonfinite_scale_is_zero(orc):
    qs = list(range(128))
    for bad in (0x7C00, 0xFC00, 0x7E00):
        out = orc.dequantize(_block(bad, 0x3800, [7] * 8, [3] * 8, qs))
        assert np.array_equal(out, np.full(256, -0.5 * 3, np.float32))
        out = orc.dequantize(_block(0x3800, bad, [7] * 8, [3] * 8, qs))
        assert np.all(out >= 0)


def test_dequant_matches_numpy_spec_random_bytes(orc):
    rng = np.random.default_rng(4)
    data = rng.integers(0, 256, size=144 * 400, dtype=np.uint8)
    # force some non-finite, subnormal and zero scales
    blocks = data.reshape(400, 144)
    blocks[0, 0:2] = [0x00, 0x7C]
    blocks[1, 2:4] = [0x01, 0x7E]
    blocks[2, 0:2] = [0x03, 0x00]
    blocks[3, 0:4] = 0
    got = orc.dequantize(data)
    want = spec.dequantize(data)
    assert got.view(np.uint32).tolist() == want.view(np.uint32).tolist()


def test_dequant_is_pure_function_of_bytes(orc):
    # gguf.rs:745-760
    x = np.sin(np.arange(512, dtype=np.float32) * np.float32(0.013)).astype(np.float32)
    q = orc.quantize(x)
    assert np.array_equal(orc.dequantize(q).view(np.uint32), orc.dequantize(q).view(np.uint32))


def test_dequant_respects_out_len(orc):
    q = orc.quantize(orc.normal(5, 512, 0.02))
    full = orc.dequantize(q)
    part = orc.dequantize(q, n_blocks=2, out_len=300)
    assert np.array_equal(part, full[:300])


# ------------------------------------------------------------ quantizer ----
def _legacy_decode(q: np.ndarray) -> np.ndarray:
    """Decode with the quantizer's own (legacy) sub-block order."""
    blocks = q.reshape(-1, 144)
    out = np.zeros((blocks.shape[0], 256), np.float32)
    d = spec.half_bits_to_f32(blocks[:, 0:2].copy().view(np.uint16)[:, 0])
    dm = spec.half_bits_to_f32(blocks[:, 2:4].copy().view(np.uint16)[:, 0])
    sc, m = spec.unpack_scales(blocks[:, 4:16])
    for b in range(blocks.shape[0]):
        for i in range(8):
            byt = blocks[b, 16 + 32 * (i // 2): 16 + 32 * (i // 2) + 32]
            nib = (byt & 15) if i % 2 == 0 else (byt >> 4)
            out[b, OFFS[i]:OFFS[i] + 32] = (d[b] * f32(sc[b, i])) * nib.astype(np.float32) - dm[b] * f32(m[b, i])
    return out.ravel()


def test_quantize_constant_closed_form(orc):
    q = orc.quantize(np.ones(256, np.float32))
    sd = trunc_f16_bits(np.float32(np.float32(1.0) / np.float32(15.0)) / np.float32(63.0))
    want = struct.pack("<HH", sd, 0) + bytes([0xFF] * 4 + [0x00] * 4 + [0x0F] * 4) + bytes([0xFF] * 128)
    assert q.tobytes() == want


def test_quantize_ties_round_half_away_from_zero(orc):
    # gguf.rs:549-559 rounds scales and nibbles with f32::round, which takes
    # an exact half away from zero; rint (half to even) differs at every even
    # k + 0.5. Sub-block 0 (legacy positions 0..31) has max 945/1024, so its
    # local d is 63*2^-10, the super-block d is 2^-10 (f16 0x1400), its scale
    # 63 and d1 = 63*2^-10; x = t*d1 then quantizes from exactly t. Sub-block
    # 1 (positions 128..159) has local d = 41*2^-11, i.e. scale exactly 20.5.
    d1 = 63.0 / 1024.0
    ties = [0.5, 1.5, 2.5, 4.5, 6.5, 14.5]
    x = np.zeros(256, np.float32)
    x[0] = np.float32(945.0 / 1024.0)
    for i, t in enumerate(ties):
        x[1 + i] = np.float32(t * d1)
        assert float(x[1 + i]) / d1 == t  # exact in f32
    x[128] = np.float32(615.0 / 2048.0)
    q = orc.quantize(x)
    assert q[0:4].tobytes() == struct.pack("<HH", 0x1400, 0)
    nib = q[16:48] & 15
    assert nib[0] == 15
    assert list(nib[1:1 + len(ties)]) == [1, 2, 3, 5, 7, 15]  # half to even: 0, 2, 2, 4, 6, 14
    assert orc.get_scale_min_k4(0, q[4:16].tobytes()) == (63, 0)
    assert orc.get_scale_min_k4(1, q[4:16].tobytes()) == (21, 0)  # half to even: 20


def test_quantize_uses_legacy_subblock_order(orc):
    # Sub-block is (legacy positions OFFS[is]..+32) holds the constant 0.1*(is+1):
    # its scale must then grow with is like 63*(is+1)/8. A quantizer using the
    # canonical order would see [0.1,0.3,0.5,0.7,0.2,0.4,0.6,0.8] instead.
    x = np.zeros(256, np.float32)
    for i in range(8):
        x[OFFS[i]:OFFS[i] + 32] = np.float32(0.1 * (i + 1))
    q = orc.quantize(x)
    scs = [orc.get_scale_min_k4(i, q[4:16].tobytes())[0] for i in range(8)]
    want = [round(63 * (i + 1) / 8) for i in range(8)]
    assert all(abs(a - b) <= 1 for a, b in zip(scs, want)), scs
    assert np.max(np.abs(_legacy_decode(q) - x)) < 0.01


@pytest.mark.parametrize("seed", [11, 12, 13])
def test_quantize_error_bound_legacy_order(orc, seed):
    x = orc.normal(seed, 256 * 64, 0.02)
    x[:256] = np.abs(x[:256])                    # all-positive block: x_min clamps to 0
    x[256:512] = 0.0                             # all-zero block
    q = orc.quantize(x)
    blocks = q.reshape(-1, 144)
    sd = spec.half_bits_to_f32(blocks[:, 0:2].copy().view(np.uint16)[:, 0])
    sdm = spec.half_bits_to_f32(blocks[:, 2:4].copy().view(np.uint16)[:, 0])
    # d, dmin are the truncated f16 of (max local)/63
    for b in range(blocks.shape[0]):
        xb = x[256 * b: 256 * b + 256]
        loc = []
        for o in OFFS:
            s = xb[o:o + 32]
            mn = min(s.min(), np.float32(0.0))
            loc.append((np.float32(np.float32(s.max() - mn) / np.float32(15.0)), -mn))
        super_d = super_dm = np.float32(0.0)   # +0 start, strict '>' as gguf.rs:609-613
        for a, c in loc:
            super_d = a if a > super_d else super_d
            super_dm = c if c > super_dm else super_dm
        assert blocks[b, 0:2].view(np.uint16)[0] == trunc_f16_bits(np.float32(super_d / np.float32(63.0)))
        assert blocks[b, 2:4].view(np.uint16)[0] == trunc_f16_bits(np.float32(super_dm / np.float32(63.0)))
    v = _legacy_decode(q).reshape(-1, 256)
    xr = x.reshape(-1, 256)
    sc, m = spec.unpack_scales(blocks[:, 4:16])
    for b in range(blocks.shape[0]):
        for i in range(8):
            d1 = sd[b] * sc[b, i]
            bound = max(d1 / 2, sdm[b] / 2 + 7.5 * sd[b]) * 1.0001 + 1e-7
            e = np.abs(xr[b, OFFS[i]:OFFS[i] + 32] - v[b, OFFS[i]:OFFS[i] + 32])
            assert e.max() <= bound, (b, i, e.max(), bound)


def test_reference_round_trip_test_fails_in_canonical_order(orc):
    # gguf.rs:703-738 gates rms_rel < 0.05 for quantize -> dequantize_row_q4_k.
    # The quantizer writes legacy order and the dequant reads canonical order,
    # so that round trip is a chunk permutation and the gate fails; the same
    # bytes decoded in the quantizer's own order pass it.
    x = orc.smooth(4 * 256)
    q = orc.quantize(x)
    canon = orc.dequantize(q)
    leg = _legacy_decode(q)
    rms = lambda y: math.sqrt(float(np.sum((x - y) ** 2)) / float(np.sum(x * x)))
    assert rms(canon) > 0.05
    assert rms(leg) < 0.05


# ------------------------------------------------------------ SimpleRng ----
def test_rng_integer_core(orc):
    r = orc.SimpleRng(0xCAFEBABE)
    s = (0xCAFEBABE + 1) & (2**64 - 1)
    for _ in range(1000):
        s = (s * 6364136223846793005 + 1442695040888963407) & (2**64 - 1)
        assert r.next_u64() == s
    r = orc.SimpleRng(7)
    s = 8
    for _ in range(1000):
        s = (s * 6364136223846793005 + 1442695040888963407) & (2**64 - 1)
        assert r.next_f32() == np.float32((s >> 40) / 2.0**24)


def test_rng_normal_box_muller(orc):
    r = orc.SimpleRng(0xC0FFEEFE)
    s = (0xC0FFEEFE + 1) & (2**64 - 1)
    for _ in range(2000):
        s = (s * 6364136223846793005 + 1442695040888963407) & (2**64 - 1)
        u1 = max(float(np.float32((s >> 40) / 2.0**24)), float(np.float32(1e-10)))
        s = (s * 6364136223846793005 + 1442695040888963407) & (2**64 - 1)
        u2 = float(np.float32((s >> 40) / 2.0**24))
        ref = math.sqrt(-2.0 * math.log(u1)) * math.cos(2.0 * math.pi * u2)
        got = r.next_normal()
        assert abs(got - ref) <= 4e-6 * max(1.0, abs(ref)), (got, ref)
    v = orc.normal(123, 200_000)
    assert abs(float(v.mean())) < 0.01 and abs(float(v.std()) - 1.0) < 0.01


def test_rng_parallel_fill_is_the_sequential_stream(orc):
    # orq_fill_normal splits the stream across threads with an LCG skip-ahead.
    n = 3 * (1 << 16) + 123
    bulk = orc.normal(0x51B00, n, 0.02)
    r = orc.SimpleRng(0x51B00)
    seq = np.array([r.next_normal() for _ in range(n)], np.float32) * np.float32(0.02)
    assert np.array_equal(bulk, seq.astype(np.float32))


# ------------------------------------------------------------ GEMV ---------
def test_gemv_unit_vector_returns_column(orc):
    n, bpr = 24, 3
    w = orc.seeded_weight(21, n, bpr * 256)
    wd = spec.dequantize(w).reshape(n, bpr * 256)
    for k in (0, 1, 31, 32, 255, 256, 700, 767):
        x = np.zeros(bpr * 256, np.float32)
        x[k] = 1.0
        y, _ = orc.gemv(w, x, n, bpr)
        assert np.array_equal(y, wd[:, k])


def test_gemv_ones_gives_row_sums_and_matches_numpy(orc):
    n, bpr = 40, 4
    w = orc.seeded_weight(22, n, bpr * 256)
    wd = spec.dequantize(w).reshape(n, bpr * 256).astype(np.float64)
    y, a = orc.gemv(w, np.ones(bpr * 256, np.float32), n, bpr)
    assert np.array_equal(y, wd.sum(axis=1).astype(np.float32))
    x = orc.normal(23, bpr * 256)
    y, a = orc.gemv(w, x, n, bpr)
    ref = wd @ x.astype(np.float64)
    assert np.allclose(y, ref.astype(np.float32), rtol=0, atol=1e-6 * np.abs(wd) @ np.abs(x))
    assert np.allclose(a, np.abs(wd) @ np.abs(x.astype(np.float64)), rtol=1e-12)


def test_gemv_flat_matches_row_aligned_and_numpy(orc):
    n, k = 16, 512
    w = orc.seeded_weight(24, n, k)
    x = orc.normal(25, k)
    y1, a1 = orc.gemv(w, x, n, k // 256)
    y2, a2 = orc.gemv_flat(w, x, n, k)
    assert np.array_equal(y1, y2) and np.allclose(a1, a2, rtol=1e-12)
    n, k = 8, 96             # 768 elements = 3 blocks, rows straddle blocks
    w = orc.seeded_weight(26, n, k)
    x = orc.normal(27, k)
    y, a = orc.gemv_flat(w, x, n, k)
    wd = spec.dequantize(w).reshape(n, k).astype(np.float64)
    assert np.allclose(y, (wd @ x).astype(np.float32), rtol=0, atol=1e-6 * (np.abs(wd) @ np.abs(x)))


def test_gemv_batched_is_rowwise_gemv(orc):
    n, bpr, B = 10, 2, 5
    w = orc.seeded_weight(28, n, bpr * 256)
    X = orc.normal(29, B * bpr * 256).reshape(B, -1)
    Y, A = orc.gemv_batched(w, X, n, bpr)
    for b in range(B):
        y, a = orc.gemv(w, X[b], n, bpr)
        assert np.array_equal(Y[b], y) and np.array_equal(A[b], a)


def test_gemm_f16_matches_numpy(orc):
    n, bpr, M = 12, 2, 6
    w = orc.seeded_weight(30, n, bpr * 256)
    a = orc.normal(31, M * bpr * 256).astype(np.float16).reshape(M, -1)
    C, _ = orc.gemm_f16(w, a.view(np.uint16), n, bpr)
    wd = spec.dequantize(w).reshape(n, -1).astype(np.float64)
    ref = a.astype(np.float64) @ wd.T
    assert np.allclose(C, ref.astype(np.float32), rtol=1e-6, atol=1e-6)
    rows = np.array([3, 0, 11])
    Cs, _ = orc.gemm_f16(w, a.view(np.uint16), n, bpr, rows=rows)
    assert np.array_equal(Cs, C[:, rows])


def test_cpu_baseline_matches_oracle(orc):
    n, bpr = 300, 14
    w = orc.seeded_weight(32, n, bpr * 256)
    x = orc.normal(33, bpr * 256)
    y_ref, a = orc.gemv(w, x, n, bpr)
    for threads in (1, 0):
        y = np.empty(n, np.float32)
        orc.cpu_matvec(w, x, y, n, bpr, threads)
        assert np.all(np.abs(y - y_ref) <= 1e-5 * a)


# --------------------------------------------------- dp4a / Q8_1 activations --
def test_quantize_q8_1_matches_numpy_and_special_blocks(orc):
    rng = np.random.default_rng(81)
    x = (rng.standard_normal(32 * 64) * rng.choice([1e-3, 1.0, 50.0], size=32 * 64)).astype(np.float32)
    x[0:32] = 0.0                                  # all-zero block
    x[32:64] = np.float32(1e-40)                   # denormal max: 127/amax overflows -> zeroed
    x[64:96] = np.float32(3.0e38) * np.sign(rng.standard_normal(32)).astype(np.float32)
    x[96:128] = np.float32(2.5)                    # constant block: every q = 127
    x[128:160] = (np.arange(32, dtype=np.float32) - 16) * np.float32(0.5)  # exact halves after scaling
    xq, xd, xs = orc.quantize_q8_1(x)
    rq, rd, rs = spec.quantize_q8_1(x)
    assert np.array_equal(xq, rq)
    assert np.array_equal(xd.view(np.uint32), rd.view(np.uint32))
    assert np.array_equal(xs, rs)
    assert np.all(xq[0:64] == 0) and xd[0] == 0 and xd[1] == 0
    assert np.all(xq[96:128] == 127) and xs[3] == 32 * 127
    assert np.all(np.abs(xq.astype(int)) <= 127)


def test_quantize_q8_1_rounds_half_to_even(orc):
    # amax = 127 -> id = 1 exactly, so q = rint(x): 0.5 -> 0, 1.5 -> 2, 2.5 -> 2
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1:6] = [0.5, 1.5, 2.5, -0.5, -2.5]
    xq, xd, xs = orc.quantize_q8_1(x)
    assert xq[1:6].tolist() == [0, 2, 2, 0, -2]
    assert xd[0] == np.float32(1.0) and xs[0] == 127 + 2 + 2 - 2


def test_dp4a_gemv_extracts_nibbles_in_canonical_order(orc):
    # one block, d = 1, dmin = 0, every scale 1: y = xd * q[p] for xq = e_p
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([0x3C00], np.uint16).view(np.uint8)
    sc = np.ones(8, np.uint8)
    blk[4:16] = np.frombuffer(orc.pack_scales_mins(sc, np.zeros(8, np.uint8)), np.uint8)
    blk[16:144] = np.random.default_rng(3).integers(0, 256, 128, dtype=np.uint8)
    q = spec.nibbles(blk)[0]
    xd = np.ones(8, np.float32)
    xs = np.zeros(8, np.float32)
    for p in (0, 1, 31, 32, 63, 64, 100, 191, 255):
        xq = np.zeros(256, np.int8)
        xq[p] = 1
        y, _ = orc.gemv_dp4a(blk, xq, xd, xs, 1, 1)
        assert y[0] == q[p], p


def test_dp4a_gemv_matches_numpy_formula(orc):
    rng = np.random.default_rng(82)
    n, bpr = 7, 3
    from tests.gpu_util import random_q4k_bytes
    w = random_q4k_bytes(rng, n * bpr)
    x = rng.standard_normal(bpr * 256).astype(np.float32)
    xq, xd, xs = orc.quantize_q8_1(x)
    y, a = orc.gemv_dp4a(w, xq, xd, xs, n, bpr)
    blocks = w.reshape(n, bpr, 144)
    q = spec.nibbles(w).reshape(n, bpr, 8, 32)
    d = spec.half_bits_to_f32(blocks[:, :, 0:2].copy().view(np.uint16)[..., 0]).astype(np.float64)
    dm = spec.half_bits_to_f32(blocks[:, :, 2:4].copy().view(np.uint16)[..., 0]).astype(np.float64)
    sc, m = spec.unpack_scales(blocks.reshape(-1, 144)[:, 4:16])
    sc = sc.reshape(n, bpr, 8).astype(np.float64)
    m = m.reshape(n, bpr, 8).astype(np.float64)
    isum = (q * xq.reshape(bpr, 8, 32)[None].astype(np.int64)).sum(axis=3)
    t = xd.reshape(bpr, 8)[None].astype(np.float64) * (
        d[..., None] * sc * isum - dm[..., None] * m * xs.reshape(bpr, 8)[None].astype(np.float64))
    assert np.allclose(y, t.sum(axis=(1, 2)), rtol=1e-12, atol=0)
    assert np.all(a >= np.abs(y))


@pytest.mark.parametrize("bias", [0.0, 100.0])
def test_dp4a_close_to_f32_gemv_reference_check(orc, bias):
    # the reference's own acceptance check (examples/rocm_dp4a_check.rs:31-63):
    # x = sin(0.21 i) * 30 + bias, RMS_rel(dp4a - f32 dequant-dot) < 0.02
    n, bpr = 64, 14
    w = orc.seeded_weight(orc.layer_seed(0, 4), n, bpr * 256)
    x = (np.sin(np.arange(bpr * 256, dtype=np.float32) * np.float32(0.21)) * np.float32(30.0)
         + np.float32(bias)).astype(np.float32)
    xq, xd, xs = orc.quantize_q8_1(x)
    y8, _ = orc.gemv_dp4a(w, xq, xd, xs, n, bpr)
    y32, _ = orc.gemv(w, x, n, bpr)
    rms_rel = np.sqrt(np.sum((y8 - y32) ** 2) / np.sum(y32.astype(np.float64) ** 2))
    assert rms_rel < 0.02
    assert rms_rel > 1e-6  # int8 activations really are lossy


# ------------------------------------------------------------- Q5_K, Q6_K --
def test_q5k_dequant_matches_numpy_spec(orc):
    rng = np.random.default_rng(55)
    data = rng.integers(0, 256, size=(40, 176), dtype=np.uint8)
    data[:, 0:4] = np.abs(rng.normal(0, 1e-2, (40, 2))).astype(np.float16).view(np.uint8).reshape(40, 4)
    data[3, 0:2] = np.array([0x7C00], np.uint16).view(np.uint8)  # d = Inf -> 0
    got = orc.dequantize_q5k(data.ravel())
    ref = spec.dequantize_q5k(data)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_q5k_high_bit_closed_form(orc):
    # d = 1, dmin = 0, all scales 1: out[p] = nibble + 16*(bit j of qh[p%32])
    blk = np.zeros(176, np.uint8)
    blk[0:2] = np.array([0x3C00], np.uint16).view(np.uint8)
    blk[4:16] = np.frombuffer(orc.pack_scales_mins(np.ones(8, np.uint8), np.zeros(8, np.uint8)), np.uint8)
    blk[48:176] = (np.arange(128) % 16) | ((15 - np.arange(128) % 16) << 4)
    blk[16 + 5] = 0b10100101  # position 5 of sub-blocks 0, 2, 5, 7 gets +16
    out = orc.dequantize_q5k(blk)
    for p in range(256):
        j, byte_i = p // 32, 32 * (p // 64) + p % 32
        nib = (byte_i % 16) if j % 2 == 0 else 15 - byte_i % 16
        hb = 16 if (p % 32 == 5 and j in (0, 2, 5, 7)) else 0
        assert out[p] == nib + hb, p


def test_q6k_dequant_matches_numpy_spec_and_signed_scales(orc):
    rng = np.random.default_rng(66)
    data = rng.integers(0, 256, size=(40, 210), dtype=np.uint8)
    data[:, 208:210] = np.abs(rng.normal(0, 1e-2, (40, 1))).astype(np.float16).view(np.uint8).reshape(40, 2)
    got = orc.dequantize_q6k(data.ravel())
    ref = spec.dequantize_q6k(data)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    # closed form: d = 1, scales[i] = i - 8, q = -32 everywhere except where set
    blk = np.zeros(210, np.uint8)
    blk[208:210] = np.array([0x3C00], np.uint16).view(np.uint8)
    blk[192:208] = (np.arange(16) - 8).astype(np.int8).view(np.uint8)
    out = orc.dequantize_q6k(blk)
    _, si = spec.q6k_values(blk)
    assert np.array_equal(out, (si - 8).astype(np.float32) * -32.0)


@pytest.mark.parametrize("fmt", [176, 210])
def test_kquant_gemv_unit_vectors_return_columns(orc, fmt):
    rng = np.random.default_rng(fmt)
    n, bpr = 9, 2
    w = rng.integers(0, 256, size=n * bpr * fmt, dtype=np.uint8).reshape(n * bpr, fmt)
    dpos = 0 if fmt == 176 else 208
    w[:, dpos:dpos + 2] = np.abs(rng.normal(0, 1e-2, (n * bpr, 1))).astype(np.float16).view(np.uint8)
    w = w.ravel()
    deq = (orc.dequantize_q5k(w) if fmt == 176 else orc.dequantize_q6k(w)).reshape(n, -1)
    for k in (0, 31, 32, 100, 255, 256, 511):
        x = np.zeros(bpr * 256, np.float32)
        x[k] = 1.0
        y, _ = orc.gemv_kquant(fmt, w, x, n, bpr)
        assert np.array_equal(y, deq[:, k])


def test_q6k_dp4a_matches_numpy_and_reference_check(orc):
    rng = np.random.default_rng(67)
    n, bpr = 32, 14
    w = rng.integers(0, 256, size=(n * bpr, 210), dtype=np.uint8)
    w[:, 208:210] = np.abs(rng.normal(0, 1e-3, (n * bpr, 1))).astype(np.float16).view(np.uint8)
    w = w.ravel()
    x = (np.sin(np.arange(bpr * 256, dtype=np.float32) * np.float32(0.21)) * np.float32(30.0))
    xq, xd, _ = orc.quantize_q8_1(x)
    y, a = orc.gemv_q6k_dp4a(w, xq, xd, n, bpr)
    q, si = spec.q6k_values(w)
    blocks = w.reshape(n * bpr, 210)
    s = blocks[:, 192:208].view(np.int8).astype(np.int64)
    d = spec.half_bits_to_f32(blocks[:, 208:210].copy().view(np.uint16)[:, 0]).astype(np.float64)
    xqb = xq.reshape(bpr, 256).astype(np.int64)
    yr = np.zeros(n)
    for r in range(n):
        for b in range(bpr):
            bi = r * bpr + b
            prod = q[bi] * xqb[b]                       # per position
            per16 = prod.reshape(16, 16).sum(axis=1)    # 16-value halves
            sc16 = s[bi][si.reshape(16, 16)[:, 0]]
            xd16 = np.repeat(xd.reshape(bpr, 8)[b].astype(np.float64), 2)
            yr[r] += np.sum(xd16 * d[bi] * sc16 * per16)
    assert np.allclose(y, yr, rtol=1e-12, atol=1e-300)
    y32, _ = orc.gemv_kquant(210, w, x, n, bpr)
    rms = np.sqrt(np.sum((y - y32) ** 2) / np.sum(y32.astype(np.float64) ** 2))
    assert 1e-6 < rms < 0.02


# ------------------------------------------------------------------ glue --
# orq_rms_norm restates kernels/rms_norm.hip:28-75 and orq_glu
# kernels/transformer_ops.hip:32-40 (+ silu). Pinned against f64 closed forms;
# the f32 reduction order itself only shows at the ulp level (bounded below).

@pytest.mark.parametrize("hidden", [1, 100, 256, 3584, 5000])
def test_rms_norm_matches_f64_formula(orc, hidden):
    rng = np.random.default_rng(hidden)
    rows = 3
    x = rng.standard_normal(rows * hidden).astype(np.float32) * 3.0
    w = rng.standard_normal(hidden).astype(np.float32)
    eps = 1e-6
    y = orc.rms_norm(x, w, rows, hidden, eps).reshape(rows, hidden)
    x64 = x.astype(np.float64).reshape(rows, hidden)
    ref = x64 / np.sqrt(np.mean(x64 * x64, axis=1, keepdims=True) + eps) * w.astype(np.float64)
    # f32 sums of non-negative terms: a few dozen ulps at most
    assert np.all(np.abs(y - ref) <= 4e-6 * np.abs(ref) + 1e-30)


def test_rms_norm_eps_is_added_to_the_mean(orc):
    # c^2 == eps: y = c / sqrt(c^2 + eps); eps added to the sum (or outside
    # the sqrt) would give a different value
    hidden, c, eps = 512, np.float32(1e-3), 1e-6
    x = np.full(hidden, c, np.float32)
    y = orc.rms_norm(x, np.ones(hidden, np.float32), 1, hidden, eps)
    assert np.allclose(y, 1e-3 / math.sqrt(2e-6), rtol=2e-6)
    assert np.all(orc.rms_norm(np.zeros(hidden, np.float32), np.ones(hidden, np.float32), 1,
                               hidden, eps) == 0.0)


def test_rms_norm_rows_are_independent(orc):
    rng = np.random.default_rng(7)
    rows, hidden = 4, 300
    x = rng.standard_normal(rows * hidden).astype(np.float32)
    w = rng.standard_normal(hidden).astype(np.float32)
    y = orc.rms_norm(x, w, rows, hidden, 1e-5)
    for r in range(rows):
        one = orc.rms_norm(x[r * hidden:(r + 1) * hidden], w, 1, hidden, 1e-5)
        assert np.array_equal(y[r * hidden:(r + 1) * hidden], one)


@pytest.mark.parametrize("act", [0, 1])
def test_glu_matches_f64_formula(orc, act):
    rng = np.random.default_rng(11 + act)
    g = np.concatenate([rng.standard_normal(4000) * 4, [0.0, 1.0, -1.0, 30.0, -30.0]]).astype(np.float32)
    u = rng.standard_normal(g.size).astype(np.float32)
    out = orc.glu(g, u, act)
    v = g.astype(np.float64)
    if act == 0:
        a = 0.5 * v * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (v + 0.044715 * v ** 3)))
    else:
        a = v / (1.0 + np.exp(-v))
    ref = a * u.astype(np.float64)
    assert np.all(np.abs(out - ref) <= 2e-6 * np.abs(v * u) + 1e-30)


@pytest.mark.parametrize("act", [0, 1])
def test_glu_identities(orc, act):
    # act(v) - act(-v) == v for both activations; up scales the product
    v = np.linspace(-8, 8, 1601).astype(np.float32)
    one = np.ones_like(v)
    d = orc.glu(v, one, act).astype(np.float64) - orc.glu(-v, one, act).astype(np.float64)
    assert np.all(np.abs(d - v) <= 2e-6 * np.abs(v) + 1e-7)
    u = np.random.default_rng(3).standard_normal(v.size).astype(np.float32)
    assert np.array_equal(orc.glu(v, 2 * u, act), 2 * orc.glu(v, u, act))
    known = {0: (1.0, 0.8411919906082768), 1: (2.0, 1.7615941559557649)}[act]
    assert abs(float(orc.glu(np.float32([known[0]]), np.float32([1.0]), act)[0]) - known[1]) < 1e-6
