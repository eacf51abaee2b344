"""GPU tests of the decode-step chain (mgq_chain_create_ex), its three
implementations, through the C ABI against the oracle.

- The persistent kernel and the graph of launch_matvec_q4k launches both meet
  the per-row bound of the f64 oracle (their partial sums are reduced in
  different orders, so their bits may differ in the last places).
- Real dependencies: each matvec's x is the previous matvec's y, so a
  work-group that read x before the grid-wide wait would read stale values;
  every y is checked against the oracle applied to the GPU's own previous y.
- Repeated launches (the completion counters only grow) keep giving the same
  bits, and the chain's fault word stays 0.
"""
import sys

import numpy as np
import pytest

from modgrad_amd import _lib
from tests.gpu_util import assert_gemv_close, dev, empty_f32, host, ptr, random_q4k_bytes

pytestmark = pytest.mark.gpu


def note(msg: str) -> None:
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def L():
    return _lib.load()


def make_chain(descs, mode):
    from modgrad_amd.q4k import Chain
    return Chain(descs, mode)


def independent(orc, shapes, seed):
    """(buffers, descs, refs) for matvecs with their own seeded x."""
    bufs, descs, refs = [], [], []
    for i, (n, bpr) in enumerate(shapes):
        rng = np.random.default_rng(seed + 7 * i)
        w = random_q4k_bytes(rng, n * bpr)
        x = rng.standard_normal(bpr * 256).astype(np.float32)
        wt, xt, yt = dev(w), dev(x), empty_f32(n)
        bufs.append((wt, xt, yt))
        descs.append((ptr(wt), ptr(xt), ptr(yt), n, bpr))
        refs.append(orc.gemv(w, x, n, bpr))
    return bufs, descs, refs


SHAPES = [[(256, 14), (64, 74), (512, 14)],
          [(4608, 14), (3584, 14), (37888, 14), (3584, 74)],
          [(1, 1), (17, 3), (300, 20), (16, 80), (5000, 14), (33, 15)]]


@pytest.mark.parametrize("k", range(len(SHAPES)))
def test_persistent_and_graph_chains_match_oracle(L, orc, k):
    shapes = SHAPES[k]
    note(f"chain persistent vs graph {shapes}")
    bufs, descs, refs = independent(orc, shapes, 100 + k)
    pers = make_chain(descs, _lib.CHAIN_PERSISTENT)
    assert pers.mode() == _lib.CHAIN_PERSISTENT
    graph = make_chain(descs, _lib.CHAIN_GRAPH)
    assert graph.mode() == _lib.CHAIN_GRAPH
    for rep in range(3):
        for _, _, yt in bufs:
            yt.fill_(float("nan"))
        pers.launch()
        got = [host(yt).copy() for _, _, yt in bufs]
        for (y_ref, a), y in zip(refs, got):
            assert_gemv_close(y, y_ref, a)
        if rep == 0:
            first = got
        else:
            for y0, y in zip(first, got):
                assert np.array_equal(y0.view(np.uint32), y.view(np.uint32))
    assert pers.faults() == 0
    for _, _, yt in bufs:
        yt.fill_(float("nan"))
    graph.launch()
    for (y_ref, a), (_, _, yt) in zip(refs, bufs):
        assert_gemv_close(host(yt), y_ref, a)
    pers.close()
    graph.close()


@pytest.mark.parametrize("mode", [_lib.CHAIN_PERSISTENT, _lib.CHAIN_GRAPH, _lib.CHAIN_EAGER])
def test_chain_with_real_dependencies(L, orc, mode):
    # x_{d+1} = y_d: dims 3584 -> 512 -> 256 -> 4608 -> 3584 -> 18944 -> 3584
    dims = [3584, 512, 256, 4608, 3584, 18944, 3584]
    note(f"chain y_d -> x_(d+1), mode {mode}, dims {dims}")
    rng = np.random.default_rng(77)
    x0 = rng.standard_normal(dims[0]).astype(np.float32)
    vecs = [dev(x0)] + [empty_f32(n) for n in dims[1:]]
    ws, descs = [], []
    for d in range(len(dims) - 1):
        k, n = dims[d], dims[d + 1]
        w = orc.seeded_weight(500 + d, n, k, scale=0.05)
        ws.append((w, dev(w)))
        descs.append((ptr(ws[-1][1]), ptr(vecs[d]), ptr(vecs[d + 1]), n, k // 256))
    ch = make_chain(descs, mode)
    assert ch.mode() == mode
    for rep in range(2):
        for v in vecs[1:]:
            v.fill_(float("nan"))
        ch.launch()
        outs = [host(v).copy() for v in vecs]
        for d in range(len(dims) - 1):
            k, n = dims[d], dims[d + 1]
            y_ref, a = orc.gemv(ws[d][0], outs[d], n, k // 256)
            assert_gemv_close(outs[d + 1], y_ref, a)
    if mode == _lib.CHAIN_PERSISTENT:
        assert ch.faults() == 0
    ch.close()


@pytest.mark.parametrize("k", range(len(SHAPES)))
def test_eager_chain_equals_graph_chain(L, orc, k):
    # MGQ_CHAIN_EAGER enqueues the same launch_matvec_q4k_ex launches the
    # graph records, so both give the same bits, on the null stream too
    shapes = SHAPES[k]
    note(f"chain eager vs graph {shapes}")
    bufs, descs, refs = independent(orc, shapes, 300 + k)
    eager = make_chain(descs, _lib.CHAIN_EAGER)
    assert eager.mode() == _lib.CHAIN_EAGER
    graph = make_chain(descs, _lib.CHAIN_GRAPH)
    got = []
    for ch in (graph, eager, eager):
        for _, _, yt in bufs:
            yt.fill_(float("nan"))
        ch.launch()
        got.append([host(yt).copy() for _, _, yt in bufs])
    for (y_ref, a), y in zip(refs, got[1]):
        assert_gemv_close(y, y_ref, a)
    for run in got[1:]:
        for y0, y in zip(got[0], run):
            assert np.array_equal(y0.view(np.uint32), y.view(np.uint32))
    eager.close()
    graph.close()


def test_persistent_chain_rejects_long_rows(L, orc):
    # K beyond the persistent kernel's activation staging: PERSISTENT reports
    # hipErrorNotSupported; AUTO is the graph
    note("chain persistent with bpr 90: not supported; auto -> graph")
    from modgrad_amd.q4k import BackendError
    bufs, descs, refs = independent(orc, [(40, 90), (64, 14)], 9)
    with pytest.raises(BackendError):
        make_chain(descs, _lib.CHAIN_PERSISTENT)
    ch = make_chain(descs, _lib.CHAIN_AUTO)
    assert ch.mode() == _lib.CHAIN_GRAPH
    ch.launch()
    for (y_ref, a), (_, _, yt) in zip(refs, bufs):
        assert_gemv_close(host(yt), y_ref, a)
    ch.close()


# ------------------------------------------------ op chains (mixed dtypes) --
def _glu_ref(g: np.ndarray, u: np.ndarray, act: int) -> np.ndarray:
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    if act == 0:
        a = 0.5 * g64 * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (g64 + 0.044715 * g64 ** 3)))
    else:
        a = g64 / (1.0 + np.exp(-g64))
    return a, a * u64


def test_op_chain_mixed_dtypes_and_glue(L, orc):
    """mgq_chain_create_ops on one recorded graph of the reference's layer
    sequence (rocm_gemma.rs:429-489) over a GGUF-like mix: RMSNorm, Q6_K and
    Q5_K matvecs on its output, the fused RMSNorm Q4_K matvec, the fused
    gate/up GLU matvec on that, a Q4_K down matvec on the GLU output, the
    standalone GLU, a residual add and a flat-layout Q4_K matvec reading the
    residual sum, and the fused RMSNorm Q6_K matvec. Every output is checked
    against the oracle applied to the inputs the GPU actually produced, on
    three replays."""
    from modgrad_amd import q4k
    from tests.gpu_util import random_kquant_bytes
    note("op chain: Q4_K/Q5_K/Q6_K matvecs, fused norm/GLU matvecs, glue")
    rng = np.random.default_rng(0xC4A1)
    H, I, KV, eps = 512, 768, 256, 1e-5
    h0 = (rng.standard_normal(H) * 1.5).astype(np.float32)
    nw1 = (rng.standard_normal(H) * 0.3 + 1.0).astype(np.float32)
    nw2 = (rng.standard_normal(H) * 0.3 + 1.0).astype(np.float32)
    w6 = random_kquant_bytes(rng, KV * H // 256, 210)
    w5 = random_kquant_bytes(rng, KV * H // 256, 176)
    w4 = orc.seeded_weight(11, H, H)
    wg = orc.seeded_weight(12, I, H)
    wu = orc.seeded_weight(13, I, H)
    wd = orc.seeded_weight(14, H, I)
    wf = random_q4k_bytes(rng, 8 * 96 // 256)  # flat 8 x 96
    dv = {k: dev(v) for k, v in dict(h0=h0, nw1=nw1, nw2=nw2, w6=w6, w5=w5, w4=w4, wg=wg,
                                          wu=wu, wd=wd, wf=wf).items()}
    out = {k: empty_f32(n) for k, n in dict(xn=H, q=KV, v=KV, y3=H, g=I, d=H, z=KV,
                                            yf=8, q6n=KV).items()}
    P = lambda k: ptr(dv[k]) if k in dv else ptr(out[k])
    Q4, Q5, Q6 = _lib.DTYPE_Q4_K, _lib.DTYPE_Q5_K, _lib.DTYPE_Q6_K
    ops = [
        q4k.op_rms_norm(P("h0"), P("nw1"), P("xn"), 1, H, eps),
        q4k.op_matvec(Q6, P("w6"), P("xn"), P("q"), KV, H),
        q4k.op_matvec(Q5, P("w5"), P("xn"), P("v"), KV, H),
        q4k.op_matvec_norm(P("w4"), P("h0"), P("nw1"), eps, P("y3"), H, H),
        q4k.op_matvec_glu(P("wg"), P("wu"), P("y3"), P("g"), I, H, P("nw2"), eps, _lib.ACT_SILU),
        q4k.op_matvec(Q4, P("wd"), P("g"), P("d"), H, I),
        q4k.op_glu(P("q"), P("v"), P("z"), KV, _lib.ACT_GELU_TANH),
        q4k.op_residual_add(P("d"), P("y3"), H),
        q4k.op_matvec(Q4, P("wf"), P("d"), P("yf"), 8, 96, _lib.LAYOUT_FLAT),
        q4k.op_matvec_norm(P("w6"), P("h0"), P("nw1"), eps, P("q6n"), KV, H, Q6),
    ]
    ch = q4k.Chain.from_ops(ops)
    assert ch.mode() == _lib.CHAIN_GRAPH
    first = None
    for rep in range(3):
        for t in out.values():
            t.fill_(float("nan"))
        ch.launch()
        r = {k: host(t) for k, t in out.items()}
        xn_ref = orc.rms_norm(h0, nw1, 1, H, eps)
        assert np.all(np.abs(r["xn"].astype(np.float64) - xn_ref) <= 4e-6 * np.abs(xn_ref) + 1e-30)
        y, A = orc.gemv_kquant(210, w6, r["xn"], KV, H // 256)
        assert_gemv_close(r["q"], y, A)
        y, A = orc.gemv_kquant(176, w5, r["xn"], KV, H // 256)
        assert_gemv_close(r["v"], y, A)
        y, A = orc.gemv(w4, xn_ref, H, H // 256)
        assert_gemv_close(r["y3"], y, A)
        xn2 = orc.rms_norm(r["y3"], nw2, 1, H, eps)
        gg, Ag = orc.gemv(wg, xn2, I, H // 256)
        uu, Au = orc.gemv(wu, xn2, I, H // 256)
        a, ref = _glu_ref(gg, uu, _lib.ACT_SILU)
        bound = 1e-4 * (1.13 * Ag * np.abs(uu) + np.abs(a) * Au) + 1e-5 * np.abs(ref) + 1e-30
        assert np.all(np.abs(r["g"].astype(np.float64) - ref) <= bound)
        # d = Wd g, then d += y3 (one f32 add per element)
        dd, Ad = orc.gemv(wd, r["g"], H, I // 256)
        res = r["d"].astype(np.float64) - r["y3"]
        assert np.all(np.abs(res - dd) <= 1e-4 * Ad + 2 ** -23 * np.abs(r["d"]) + 1e-30)
        zref = orc.glu(r["q"], r["v"], 0)
        assert np.all(np.abs(r["z"].astype(np.float64) - zref) <= 2e-6 * np.abs(r["q"] * r["v"]) + 1e-30)
        y, A = orc.gemv_flat(wf, r["d"][:96], 8, 96)
        assert_gemv_close(r["yf"], y, A)
        y, A = orc.gemv_kquant(210, w6, xn_ref, KV, H // 256)
        assert_gemv_close(r["q6n"], y, A)
        if first is None:
            first = r
        else:
            for k in r:
                assert np.array_equal(r[k].view(np.uint32), first[k].view(np.uint32)), k
    ch.close()


def _dp4a_close(y, y_ref, absterm):
    # the dp4a formula in f64 (the oracle) against the kernel's f32 sums
    err = np.abs(y.astype(np.float64) - y_ref)
    assert np.all(err <= 1e-5 * absterm + 1e-30), float(np.max(err / np.maximum(absterm, 1e-300)))


def test_op_chain_dp4a_arm(L, orc):
    """The reference engine's default Q8_1/dp4a arm (rocm_gemma.rs:283,
    298-306; rocm.rs:477-479, 490-491) recorded by mgq_chain_create_ops:
    RMSNorm, quantize_q8_1, the Q4_K and Q6_K dp4a matvecs on its Q8_1
    activations, the fused quantize + Q4_K dp4a matvec, a GLU, a second
    quantize and dp4a matvec on the GLU output, and a residual add. Every
    output is checked against the oracle on the GPU's own inputs (Q8_1 bit for
    bit, matvecs against the f64 dp4a formula), the Q4_K result also against
    the reference's RMS-relative < 0.02 gate on f32 activations, on three
    replays with identical bits."""
    from modgrad_amd import q4k
    from tests.gpu_util import random_kquant_bytes
    import torch
    note("op chain: the dp4a arm (quantize_q8_1, Q4_K/Q6_K dp4a, fused quantize+dp4a)")
    rng = np.random.default_rng(0xD4A)
    H, KV, eps = 1024, 512, 1e-5
    h0 = (rng.standard_normal(H) * 1.5).astype(np.float32)
    nw = (rng.standard_normal(H) * 0.3 + 1.0).astype(np.float32)
    wq = orc.seeded_weight(31, KV, H)
    wv = random_kquant_bytes(rng, KV * H // 256, 210)
    wo = orc.seeded_weight(32, H, H)
    wd = orc.seeded_weight(33, H, KV)
    dv = {k: dev(v) for k, v in dict(h0=h0, nw=nw, wq=wq, wv=wv, wo=wo, wd=wd).items()}
    out = {k: empty_f32(n) for k, n in dict(xn=H, q=KV, v=KV, o=H, z=KV, d=H).items()}
    q8 = {k: (torch.empty(n, dtype=torch.int8, device="cuda"), empty_f32(n // 32), empty_f32(n // 32))
          for k, n in dict(a=H, b=KV).items()}
    P = lambda k: ptr(dv[k]) if k in dv else ptr(out[k])
    Q = lambda k: tuple(ptr(t) for t in q8[k])
    Q4, Q6 = _lib.DTYPE_Q4_K, _lib.DTYPE_Q6_K
    ops = [
        q4k.op_rms_norm(P("h0"), P("nw"), P("xn"), 1, H, eps),
        q4k.op_quantize_q8_1(P("xn"), *Q("a"), H),
        q4k.op_matvec_dp4a(Q4, P("wq"), *Q("a"), P("q"), KV, H),
        q4k.op_matvec_dp4a(Q6, P("wv"), *Q("a"), P("v"), KV, H),
        q4k.op_quantize_matvec_dp4a(P("wo"), P("xn"), P("o"), H, H),
        q4k.op_glu(P("q"), P("v"), P("z"), KV, _lib.ACT_SILU),
        q4k.op_quantize_q8_1(P("z"), *Q("b"), KV),
        q4k.op_matvec_dp4a(Q4, P("wd"), *Q("b"), P("d"), H, KV),
        q4k.op_residual_add(P("d"), P("o"), H),
    ]
    ch = q4k.Chain.from_ops(ops)
    assert ch.mode() == _lib.CHAIN_GRAPH
    first = None
    for rep in range(3):
        for t in out.values():
            t.fill_(float("nan"))
        ch.launch()
        r = {k: host(t) for k, t in out.items()}
        r8 = {k: tuple(host(t) for t in v) for k, v in q8.items()}
        qa, da, sa = orc.quantize_q8_1(r["xn"])
        assert np.array_equal(r8["a"][0], qa) and np.array_equal(r8["a"][1].view(np.uint32), da.view(np.uint32))
        assert np.array_equal(r8["a"][2].view(np.uint32), sa.view(np.uint32))
        y, A = orc.gemv_dp4a(wq, qa, da, sa, KV, H // 256)
        _dp4a_close(r["q"], y, A)
        yf, _ = orc.gemv(wq, r["xn"], KV, H // 256)
        rms = np.sqrt(np.sum((r["q"].astype(np.float64) - yf) ** 2) / np.sum(yf.astype(np.float64) ** 2))
        assert rms < 0.02  # the reference's dp4a acceptance gate (rocm_dp4a_check.rs:63)
        y, A = orc.gemv_q6k_dp4a(wv, qa, da, KV, H // 256)
        _dp4a_close(r["v"], y, A)
        y, A = orc.gemv_dp4a(wo, qa, da, sa, H, H // 256)
        o_ref = y
        qb, db, sb = orc.quantize_q8_1(r["z"])
        assert np.array_equal(r8["b"][0], qb) and np.array_equal(r8["b"][1].view(np.uint32), db.view(np.uint32))
        y, A = orc.gemv_dp4a(wd, qb, db, sb, H, KV // 256)
        # d = Wd . Q8(z), then d += o (one f32 add per element)
        res = r["d"].astype(np.float64) - r["o"]
        assert np.all(np.abs(res - y) <= 1e-5 * A + 2 ** -23 * np.abs(r["d"]) + 1e-30)
        # o came from the fused quantize+dp4a launch: the dp4a formula on Q8(xn)
        o_gpu = r["o"].astype(np.float64)
        _, Ao = orc.gemv_dp4a(wo, qa, da, sa, H, H // 256)
        assert np.all(np.abs(o_gpu - o_ref) <= 1e-5 * Ao + 1e-30)
        if first is None:
            first = r
        else:
            for k in r:
                assert np.array_equal(r[k].view(np.uint32), first[k].view(np.uint32)), k
    ch.close()
