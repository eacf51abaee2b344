"""Independent numpy restatement of the Q4_K block format, written from the
format description (not from the C oracle), used to cross-check the oracle.

Block (144 B, little-endian): +0 d:f16, +2 dmin:f16, +4 scales[12], +16 qs[128].
Sub-block j in 0..8 has a 6-bit scale sc[j] and min m[j]:
  j < 4:  sc = s[j] & 63,                         m = s[j+4] & 63
  j >= 4: sc = (s[j+4] & 15) | ((s[j-4] >> 6) << 4), m = (s[j+4] >> 4) | ((s[j] >> 6) << 4)
Output position p in 0..256 (ggml order): sub-block p // 32; byte
qs[32*(p // 64) + p % 32]; low nibble when (p // 32) is even, else high.
w[p] = f32(f32(d*sc) * q) - f32(dmin*m); d or dmin with exponent 31 -> 0.
"""
import numpy as np


def unpack_scales(s: np.ndarray):
    """s: uint8 [nb, 12] -> (sc, m) uint8 [nb, 8]."""
    s = s.astype(np.uint16)
    sc = np.empty((s.shape[0], 8), np.uint16)
    m = np.empty((s.shape[0], 8), np.uint16)
    sc[:, :4] = s[:, 0:4] & 63
    m[:, :4] = s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)
    m[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    return sc.astype(np.uint8), m.astype(np.uint8)


def half_bits_to_f32(h: np.ndarray) -> np.ndarray:
    f = h.astype(np.uint16).view(np.float16).astype(np.float32)
    return np.where(np.isfinite(f), f, np.float32(0.0)).astype(np.float32)


def dequantize(data: np.ndarray) -> np.ndarray:
    blocks = np.asarray(data, np.uint8).reshape(-1, 144)
    nb = blocks.shape[0]
    d = half_bits_to_f32(blocks[:, 0:2].copy().view(np.uint16)[:, 0])
    dmin = half_bits_to_f32(blocks[:, 2:4].copy().view(np.uint16)[:, 0])
    sc, m = unpack_scales(blocks[:, 4:16])
    qs = blocks[:, 16:144]
    p = np.arange(256)
    sub = p // 32
    byte = qs[:, 32 * (p // 64) + p % 32]
    q = np.where(sub % 2 == 0, byte & 15, byte >> 4).astype(np.float32)
    d1 = (d[:, None] * sc.astype(np.float32))[:, sub]          # f32 product
    m1 = (dmin[:, None] * m.astype(np.float32))[:, sub]
    out = (d1 * q).astype(np.float32) - m1                      # two roundings
    return out.astype(np.float32).reshape(nb * 256)


def nibbles(data: np.ndarray) -> np.ndarray:
    """Canonical-order quants q[p] in 0..15 per block: int64 [nb, 256]."""
    blocks = np.asarray(data, np.uint8).reshape(-1, 144)
    qs = blocks[:, 16:144]
    p = np.arange(256)
    byte = qs[:, 32 * (p // 64) + p % 32].astype(np.int64)
    return np.where((p // 32) % 2 == 0, byte & 15, byte >> 4)


def quantize_q8_1(x: np.ndarray):
    """Q8_1 activation quantizer in numpy float32 arithmetic (written from the
    description: per 32 values, d = amax/127, id = 127/amax (0 when amax is
    0 or 127/amax is not finite, which also zeroes d), q = clamp(rint(x*id)))."""
    x = np.asarray(x, np.float32).reshape(-1, 32)
    amax = np.max(np.abs(x), axis=1)
    with np.errstate(divide="ignore", over="ignore", invalid="ignore"):
        d = (amax / np.float32(127.0)).astype(np.float32)
        idv = np.where(amax > 0, np.float32(127.0) / np.where(amax > 0, amax, 1), 0).astype(np.float32)
        bad = ~np.isfinite(idv)
        idv[bad] = 0
        d[bad] = 0
        prod = (x * idv[:, None]).astype(np.float32)
        r = np.rint(prod)
    r = np.where(np.isnan(r), 0, r)
    q = np.clip(r, -127, 127).astype(np.int8)
    return q.ravel(), d, q.astype(np.int64).sum(axis=1).astype(np.float32)


def dequantize_q5k(data: np.ndarray) -> np.ndarray:
    """Q5_K, 176 B: +0 d f16, +2 dmin f16, +4 scales[12] (Q4_K packing),
    +16 qh[32], +48 ql[128]. Position p: sub-block j = p // 32, low nibble of
    ql[32*(p // 64) + p % 32] for even j (high for odd), plus 16 when bit j of
    qh[p % 32] is set; w = f32(f32(d*sc_j) * q) - f32(dmin*m_j)."""
    blocks = np.asarray(data, np.uint8).reshape(-1, 176)
    nb = blocks.shape[0]
    d = half_bits_to_f32(blocks[:, 0:2].copy().view(np.uint16)[:, 0])
    dmin = half_bits_to_f32(blocks[:, 2:4].copy().view(np.uint16)[:, 0])
    sc, m = unpack_scales(blocks[:, 4:16])
    qh, ql = blocks[:, 16:48], blocks[:, 48:176]
    p = np.arange(256)
    j = p // 32
    byte = ql[:, 32 * (p // 64) + p % 32].astype(np.int64)
    nib = np.where(j % 2 == 0, byte & 15, byte >> 4)
    hb = (qh[:, p % 32].astype(np.int64) >> j) & 1
    q = (nib + 16 * hb).astype(np.float32)
    d1 = (d[:, None] * sc.astype(np.float32))[:, j]
    m1 = (dmin[:, None] * m.astype(np.float32))[:, j]
    return ((d1 * q).astype(np.float32) - m1).astype(np.float32).reshape(nb * 256)


def q6k_values(data: np.ndarray):
    """(q in -32..31, scale index) per canonical position of each Q6_K block."""
    blocks = np.asarray(data, np.uint8).reshape(-1, 210)
    ql, qh = blocks[:, 0:128].astype(np.int64), blocks[:, 128:192].astype(np.int64)
    p = np.arange(256)
    g, r = p // 128, p % 128
    quad, l = r // 32, r % 32
    byte = ql[:, 64 * g + l + 32 * (quad % 2)]
    nib = np.where(quad < 2, byte & 15, byte >> 4)
    hb = (qh[:, 32 * g + l] >> (2 * quad)) & 3
    return (nib | (hb << 4)) - 32, 8 * g + l // 16 + 2 * quad


def dequantize_q6k(data: np.ndarray) -> np.ndarray:
    """Q6_K, 210 B: +0 ql[128], +128 qh[64], +192 int8 scales[16], +208 d f16.
    Position p = 128g + 32quad + l: low (quad < 2) or high nibble of
    ql[64g + l + 32*(quad % 2)], bits 2quad..2quad+1 of qh[32g + l] on top,
    minus 32; scale scales[8g + l // 16 + 2quad]; w = f32(f32(d*s) * q)."""
    blocks = np.asarray(data, np.uint8).reshape(-1, 210)
    nb = blocks.shape[0]
    q, si = q6k_values(blocks)
    s = blocks[:, 192:208].view(np.int8).astype(np.float32)[:, si]
    d = half_bits_to_f32(blocks[:, 208:210].copy().view(np.uint16)[:, 0])
    return ((d[:, None] * s).astype(np.float32) * q.astype(np.float32)).astype(np.float32).reshape(nb * 256)
