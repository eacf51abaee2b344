"""GPU tests of the decode-step chain (mgq_chain_create_ex), both
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


@pytest.mark.parametrize("mode", [_lib.CHAIN_PERSISTENT, _lib.CHAIN_GRAPH])
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
