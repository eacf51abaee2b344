"""GPU parity over a seeded random sweep of shapes, byte offsets and batch sizes.

The other parity tests pick shapes that select each launch configuration on
purpose; this sweep draws them at random (a fixed seed, so the same cases run
every time) to reach the combinations nobody picked: ragged row groups and
stages, the persistent schedules at odd group counts, weights at every byte
offset, activations 4 bytes past 16-byte alignment, and batch sizes between
the powers of two; and the same for the Q5_K / Q6_K matvecs and the
RMSNorm / GLU-fused Q4_K matvecs, and the Q8_1 quantizer + dp4a matvec.
Gates are the BASELINE ones (per row |y - y_f64| <=
1e-4 * sum_k |w_rk||x_k|; the f16 GEMM at the tolerance of its own tests).
"""
import numpy as np
import pytest

from modgrad_amd import _lib
from tests.gpu_util import (assert_gemv_close, dev, empty_f32, filled_u8, host, ptr,
                            random_q4k_bytes)

pytestmark = pytest.mark.gpu


def note(msg: str) -> None:
    print(f"[case] {msg}", flush=True)


def _cases():
    rng = np.random.default_rng(0x5EED2026)
    mv, bt, gm, fl = [], [], [], []
    while len(mv) < 48:  # matvec: n log-uniform in [1, 60000] or uniform in
        # [4000, 60000] (the persistent and one-group-per-CU launches), bpr in [1, 80]
        n = int(np.exp(rng.uniform(0, np.log(60000)))) if len(mv) % 2 else int(rng.integers(4000, 60001))
        bpr = int(rng.integers(1, 81)) if len(mv) % 3 else int(rng.integers(1, 15))
        if n * bpr <= 300_000:
            mv.append((n, bpr, int(rng.integers(0, 16)), int(rng.integers(0, 2)) * 4))
    while len(bt) < 20:  # batched: B in [1, 16]
        n = int(np.exp(rng.uniform(0, np.log(20000))))
        bpr = int(rng.integers(1, 81))
        if n * bpr <= 150_000:
            bt.append((n, bpr, int(rng.integers(1, 17)), int(rng.integers(0, 16))))
    while len(gm) < 12:  # f16 GEMM: m in [1, 640]
        n = int(np.exp(rng.uniform(np.log(16), np.log(20000))))
        bpr = int(rng.integers(1, 21))
        m = int(rng.integers(1, 641))
        if m * n * bpr * 256 <= 4e8:
            gm.append((n, bpr, m))
    while len(fl) < 10:  # flattened layout: any k, n a multiple of 256 / gcd(k, 256)
        k = int(rng.integers(1, 80)) * 32 + (0 if len(fl) % 2 else int(rng.integers(1, 32)))
        unit = 256 // int(np.gcd(k, 256))
        n = unit * int(rng.integers(1, max(2, 3000 // unit)))
        if n * k <= 20_000_000:
            fl.append((n, k))
    lds = []  # prefill-sized GEMMs: the 160 x 256 tile kernel, rows sampled
    while len(lds) < 4:
        lds.append((int(rng.integers(17000, 20001)), int(rng.integers(2, 15)),
                    int(rng.integers(480, 513))))
    return mv, bt, gm, fl, lds


MATVEC, BATCHED, GEMM, FLAT, GEMM_LDS = _cases()


@pytest.fixture(scope="module")
def L():
    return _lib.load()


@pytest.mark.parametrize("n,bpr,woff,xoff", MATVEC)
def test_random_matvec(L, orc, n, bpr, woff, xoff):
    import torch
    note(f"sweep matvec n={n} bpr={bpr} w+{woff} x+{xoff}")
    rng = np.random.default_rng(n * 131 + bpr)
    w = random_q4k_bytes(rng, n * bpr)
    x = rng.standard_normal(bpr * 256).astype(np.float32)
    wt = torch.zeros(w.size + 16, dtype=torch.uint8, device="cuda")
    wt[woff:woff + w.size].copy_(torch.from_numpy(w))
    xt = torch.zeros(x.size + 4, dtype=torch.float32, device="cuda")
    xt[xoff // 4:xoff // 4 + x.size].copy_(torch.from_numpy(x))
    yt = empty_f32(n)
    _lib.check("launch_matvec_q4k", L.launch_matvec_q4k(ptr(wt) + woff, ptr(xt) + xoff, ptr(yt), n, bpr))
    y_ref, a = orc.gemv(w, x, n, bpr)
    assert_gemv_close(host(yt), y_ref, a)


@pytest.mark.parametrize("n,bpr,batch,woff", BATCHED)
def test_random_batched(L, orc, n, bpr, batch, woff):
    note(f"sweep batched n={n} bpr={bpr} B={batch} w+{woff}")
    rng = np.random.default_rng(n * 7 + bpr * 3 + batch)
    w = random_q4k_bytes(rng, n * bpr)
    X = rng.standard_normal((batch, bpr * 256)).astype(np.float32)
    wt = dev(np.concatenate([np.zeros(woff, np.uint8), w]))
    Xt, Yt = dev(X), empty_f32(batch * n)
    nws = L.mgq_batched_workspace_bytes(bpr, batch)
    ws = filled_u8(nws, 0x5A)  # stale bytes from an earlier user
    _lib.check("batched", L.launch_matvec_q4k_batched(ptr(wt) + woff, ptr(Xt), ptr(Yt), n, bpr,
                                                      batch, ptr(ws), nws, None))
    Y = host(Yt).reshape(batch, n)
    Y_ref, A = orc.gemv_batched(w, X, n, bpr)
    for b in range(batch):
        assert_gemv_close(Y[b], Y_ref[b], A[b])


@pytest.mark.parametrize("n,bpr,m", GEMM)
def test_random_gemm_f16(L, orc, n, bpr, m):
    note(f"sweep gemm n={n} bpr={bpr} m={m}")
    rng = np.random.default_rng(n + 17 * bpr + 1009 * m)
    w = random_q4k_bytes(rng, n * bpr)
    a = rng.standard_normal((m, bpr * 256)).astype(np.float16)
    wt, at, ct = dev(w), dev(a.view(np.uint16)), empty_f32(m * n)
    _lib.check("gemm", L.launch_gemm_q4k_f16(ptr(wt), ptr(at), ptr(ct), n, bpr, m, None))
    C = host(ct).reshape(m, n)
    C_ref, A = orc.gemm_f16(w, a.view(np.uint16), n, bpr)
    k = bpr * 256
    assert np.all(np.abs(C - C_ref) <= 1e-2 * A / np.sqrt(k))
    assert np.linalg.norm(C - C_ref) <= 1e-3 * np.linalg.norm(C_ref)


@pytest.mark.parametrize("n,bpr,m", GEMM_LDS)
def test_random_gemm_f16_prefill_sized(L, orc, n, bpr, m):
    note(f"sweep gemm (prefill-sized) n={n} bpr={bpr} m={m}")
    rng = np.random.default_rng(n + 31 * bpr + 7 * m)
    w = random_q4k_bytes(rng, n * bpr)
    a = rng.standard_normal((m, bpr * 256)).astype(np.float16)
    wt, at, ct = dev(w), dev(a.view(np.uint16)), empty_f32(m * n)
    _lib.check("gemm", L.launch_gemm_q4k_f16(ptr(wt), ptr(at), ptr(ct), n, bpr, m, None))
    rows = np.sort(rng.choice(n, size=256, replace=False))
    C = host(ct).reshape(m, n)[:, rows]
    C_ref, A = orc.gemm_f16(w, a.view(np.uint16), n, bpr, rows=rows)
    k = bpr * 256
    assert np.all(np.abs(C - C_ref) <= 1e-2 * A / np.sqrt(k))
    assert np.linalg.norm(C - C_ref) <= 1e-3 * np.linalg.norm(C_ref)


@pytest.mark.parametrize("n,k", FLAT)
def test_random_flat_layout(L, orc, n, k):
    note(f"sweep flat n={n} k={k}")
    rng = np.random.default_rng(n * 3 + k)
    w = random_q4k_bytes(rng, n * k // 256)
    x = rng.standard_normal(k).astype(np.float32)
    wt, xt, yt = dev(w), dev(x), empty_f32(n)
    _lib.check("launch_matvec_q4k_ex",
               L.launch_matvec_q4k_ex(ptr(wt), ptr(xt), ptr(yt), n, k, _lib.LAYOUT_FLAT, None))
    y_ref, a = orc.gemv_flat(w, x, n, k)
    assert_gemv_close(host(yt), y_ref, a)


def _more_cases():
    rng = np.random.default_rng(0x5EED2027)
    kq, glu = [], []
    while len(kq) < 24:  # Q5_K / Q6_K: both kernel families, K up to 100 blocks
        fmt = 176 if len(kq) % 2 else 210
        n = int(np.exp(rng.uniform(0, np.log(30000)))) if len(kq) % 3 else int(rng.integers(4000, 30001))
        bpr = int(rng.integers(1, 101)) if len(kq) % 4 else int(rng.integers(1, 15))
        if n * bpr <= 200_000:
            kq.append((fmt, n, bpr))
    while len(glu) < 12:  # fused RMSNorm and/or GLU on the Q4_K matvec
        n = int(np.exp(rng.uniform(0, np.log(20000))))
        bpr = int(rng.integers(1, 30))
        if n * bpr <= 150_000:
            g, nm = int(rng.integers(0, 2)), int(rng.integers(0, 2))
            glu.append((n, bpr, g, nm if g else 1, int(rng.integers(0, 2))))
    return kq, glu


KQUANT, GLU = _more_cases()


@pytest.mark.parametrize("fmt,n,bpr", KQUANT)
def test_random_kquant_matvec(L, orc, fmt, n, bpr):
    from tests.gpu_util import random_kquant_bytes
    note(f"sweep {'q5k' if fmt == 176 else 'q6k'} n={n} bpr={bpr}")
    rng = np.random.default_rng(fmt * 7919 + n * 3 + bpr)
    w = random_kquant_bytes(rng, n * bpr, fmt)
    x = rng.standard_normal(bpr * 256).astype(np.float32)
    wt, xt, yt = dev(w), dev(x), empty_f32(n)
    fn = L.launch_matvec_q5k if fmt == 176 else L.launch_matvec_q6k
    _lib.check("kquant", fn(ptr(wt), ptr(xt), ptr(yt), n, bpr))
    y_ref, a = orc.gemv_kquant(fmt, w, x, n, bpr)
    assert_gemv_close(host(yt), y_ref, a)


@pytest.mark.parametrize("n,bpr,glu,norm,act", GLU)
def test_random_fused_matvec(L, orc, n, bpr, glu, norm, act):
    """RMSNorm-fused matvec, or the gate/up matvec with its GLU (with or
    without the norm), against norm -> matvec(s) -> activation in the oracle."""
    note(f"sweep fused n={n} bpr={bpr} glu={glu} norm={norm} act={act}")
    rng = np.random.default_rng(n * 5 + bpr * 11 + 2 * glu + norm)
    k = bpr * 256
    wg = random_q4k_bytes(rng, n * bpr)
    wu = random_q4k_bytes(rng, n * bpr)
    x = (1.3 * rng.standard_normal(k)).astype(np.float32)
    nw = (0.5 * rng.standard_normal(k) + 1.0).astype(np.float32)
    eps = 1e-5
    wgt, wut, xt, nt, yt = dev(wg), dev(wu), dev(x), dev(nw), empty_f32(n)
    xn = orc.rms_norm(x, nw, 1, k, eps) if norm else x
    if not glu:
        _lib.check("norm matvec", L.launch_matvec_q4k_rmsnorm_ex(ptr(wgt), ptr(xt), ptr(nt), eps,
                                                                 ptr(yt), n, bpr, None))
        y_ref, A = orc.gemv(wg, xn, n, bpr)
        assert_gemv_close(host(yt), y_ref, A)
        return
    _lib.check("glu matvec", L.launch_matvec_q4k_glu_ex(ptr(wgt), ptr(wut), ptr(xt),
                                                        ptr(nt) if norm else None, eps, act,
                                                        ptr(yt), n, bpr, None))
    y = host(yt).astype(np.float64)
    g, Ag = orc.gemv(wg, xn, n, bpr)
    u, Au = orc.gemv(wu, xn, n, bpr)
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    if act == 0:
        a = 0.5 * g64 * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (g64 + 0.044715 * g64 ** 3)))
    else:
        a = g64 / (1.0 + np.exp(-g64))
    ref = a * u64
    # the glue tests' bound: the activation's slope (at most 1.13) carries the
    # gate's matvec error, |a| the up matvec's
    bound = 1e-4 * (1.13 * Ag * np.abs(u64) + np.abs(a) * Au) + 1e-5 * np.abs(ref) + 1e-30
    err = np.abs(y - ref)
    bad = np.nonzero(~(err <= bound))[0]
    assert bad.size == 0, (bad[:5].tolist(), err[bad[:5]].tolist(), bound[bad[:5]].tolist())


def _dp4a_cases():
    rng = np.random.default_rng(0x5EED2028)
    out = []
    while len(out) < 16:  # Q8_1 activations, weights at any byte offset
        n = int(np.exp(rng.uniform(0, np.log(40000)))) if len(out) % 2 else int(rng.integers(4000, 40001))
        bpr = int(rng.integers(1, 81)) if len(out) % 3 else int(rng.integers(1, 15))
        if n * bpr <= 250_000:
            out.append((n, bpr, int(rng.integers(0, 16))))
    return out


DP4A = _dp4a_cases()


@pytest.mark.parametrize("n,bpr,woff", DP4A)
def test_random_dp4a_matvec(L, orc, n, bpr, woff):
    """quantize_q8_1 bit-exact, then the dp4a matvec against the oracle's f64
    evaluation of the same formula (the dp4a tests' bound)."""
    note(f"sweep dp4a n={n} bpr={bpr} w+{woff}")
    rng = np.random.default_rng(n * 13 + bpr * 5 + woff)
    w = random_q4k_bytes(rng, n * bpr)
    x = rng.standard_normal(bpr * 256).astype(np.float32)
    nsub = x.size // 32
    xt = dev(x)
    xq, xd, xs = filled_u8(nsub * 32 + 64, 0x5A), empty_f32(nsub + 4), empty_f32(nsub + 4)
    _lib.check("quantize_q8_1", L.launch_quantize_q8_1(ptr(xt), ptr(xq), ptr(xd), ptr(xs), x.size))
    q, d, s = host(xq)[:nsub * 32].view(np.int8), host(xd)[:nsub], host(xs)[:nsub]
    rq, rd, rs = orc.quantize_q8_1(x)
    assert np.array_equal(q, rq) and np.array_equal(d.view(np.uint32), rd.view(np.uint32))
    assert np.array_equal(s, rs)
    wt, yt = dev(np.concatenate([np.zeros(woff, np.uint8), w])), empty_f32(n)
    _lib.check("dp4a", L.launch_matvec_q4k_dp4a(ptr(wt) + woff, ptr(xq), ptr(xd), ptr(xs), ptr(yt),
                                                n, bpr))
    y_ref, absterm = orc.gemv_dp4a(w, q, d, s, n, bpr)
    err = np.abs(host(yt).astype(np.float64) - y_ref)
    bad = np.nonzero(~(err <= 1e-5 * absterm + 1e-30))[0]
    assert bad.size == 0, (bad[:5].tolist(), err[bad[:5]].tolist(), absterm[bad[:5]].tolist())
