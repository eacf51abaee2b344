"""launch_matvec_q4k_batched_noalloc: the batched matvec with its operand
table in the library's fixed device scratch array instead of a caller
workspace. Checked bit for bit against launch_matvec_q4k_batched (same
kernels, deterministic) on two calls in a row, the second with a smaller
input, so the second call runs over the first call's leftover scratch."""
import sys

import numpy as np
import pytest

from modgrad_amd import _lib
from tests.gpu_util import dev, empty_f32, filled_u8, host, ptr

FAKE = 0x10000  # never dereferenced: the call fails validation first


def note(msg: str) -> None:
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def test_noalloc_rejects_shapes_beyond_the_scratch():
    # the fixed array holds 4 MiB: workspace bytes of bpr 452 at batch 8 or
    # bpr 226 at batch 16 do not fit (before any device call)
    L = _lib.load()
    cap = 4 << 20
    assert L.mgq_batched_workspace_bytes(451, 8) <= cap < L.mgq_batched_workspace_bytes(452, 8)
    assert L.mgq_batched_workspace_bytes(225, 16) <= cap < L.mgq_batched_workspace_bytes(226, 16)
    fn = L.launch_matvec_q4k_batched_noalloc
    assert fn(FAKE, FAKE, FAKE, 16, 452, 8, None) == _lib.hipErrorInvalidValue
    assert fn(FAKE, FAKE, FAKE, 16, 226, 16, None) == _lib.hipErrorInvalidValue
    assert fn(FAKE, FAKE, FAKE, 16, 14, 17, None) == _lib.hipErrorInvalidValue
    assert fn(FAKE, FAKE, FAKE, 0, 14, 8, None) == _lib.hipErrorInvalidValue
    assert fn(FAKE, FAKE + 2, FAKE, 16, 14, 8, None) == _lib.hipErrorInvalidValue


@pytest.mark.gpu
def test_noalloc_under_graph_capture(orc):
    # The process's first noalloc call (no mgq_prepare before it; this test
    # runs before the ones that call it) is made inside a torch.cuda.graph
    # capture, so the scratch lookup happens mid-capture. The graph then
    # holds the fixed scratch address: three replays with new X contents,
    # each followed by eager work of the program (the workspace entry point
    # on the same X), must give the workspace entry point's bits.
    import torch
    L = _lib.load()
    n, bpr, batch = 1000, 14, 8
    w = orc.seeded_weight(41, n, bpr * 256)
    wt = dev(w)
    Xt = torch.zeros(batch * bpr * 256, dtype=torch.float32, device="cuda")
    Y_g, Y_ws = empty_f32(batch * n), empty_f32(batch * n)
    nws = L.mgq_batched_workspace_bytes(bpr, batch)
    ws = filled_u8(nws, 0x55)
    note(f"noalloc captured in a graph: n={n} bpr={bpr} B={batch}")
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    with torch.cuda.graph(g, stream=side):
        rc = L.launch_matvec_q4k_batched_noalloc(ptr(wt), ptr(Xt), ptr(Y_g), n, bpr, batch,
                                                 torch.cuda.current_stream().cuda_stream)
    _lib.check("batched_noalloc (captured)", rc)
    for rep in range(3):
        X = orc.normal(4100 + rep, batch * bpr * 256)
        Xt.copy_(torch.from_numpy(X))
        Y_g.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        _lib.check("batched", L.launch_matvec_q4k_batched(ptr(wt), ptr(Xt), ptr(Y_ws), n, bpr,
                                                          batch, ptr(ws), nws, None))
        a, b = host(Y_ws), host(Y_g)
        assert np.all(np.isfinite(a))
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"replay {rep}"


def run_pair(L, orc, n, bpr, batch, seed):
    w = orc.seeded_weight(seed, n, bpr * 256)
    X = orc.normal(seed + 1, batch * bpr * 256).reshape(batch, -1)
    wt, Xt = dev(w), dev(X)
    nws = L.mgq_batched_workspace_bytes(bpr, batch)
    ws = filled_u8(nws, 0x77)
    Y_ws, Y_na = empty_f32(batch * n), empty_f32(batch * n)
    _lib.check("batched", L.launch_matvec_q4k_batched(ptr(wt), ptr(Xt), ptr(Y_ws), n, bpr, batch,
                                                      ptr(ws), nws, None))
    _lib.check("batched_noalloc", L.launch_matvec_q4k_batched_noalloc(ptr(wt), ptr(Xt), ptr(Y_na),
                                                                      n, bpr, batch, None))
    a, b = host(Y_ws), host(Y_na)
    assert np.all(np.isfinite(a))
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("first,second", [((3584, 74, 16), (1000, 14, 5)),
                                          ((18944, 14, 8), (300, 9, 2))])
def test_noalloc_matches_the_workspace_entry_point(orc, first, second):
    # first: the K-split path (down 3584x18944, two batch sets) or 16-row
    # groups (gate 18944x3584); second: a smaller shape over the leftovers
    L = _lib.load()
    _lib.check("mgq_prepare", L.mgq_prepare())
    for i, (n, bpr, batch) in enumerate((first, second)):
        note(f"noalloc call {i + 1}: n={n} bpr={bpr} B={batch}")
        run_pair(L, orc, n, bpr, batch, 900 + 17 * i + bpr)


@pytest.mark.gpu
def test_noalloc_single_row_is_the_matvec(orc):
    # batch 1 is the plain matvec (no table, no scratch)
    note("noalloc B=1")
    L = _lib.load()
    n, bpr = 500, 14
    w = orc.seeded_weight(77, n, bpr * 256)
    x = orc.normal(78, bpr * 256)
    wt, xt, y1, y2 = dev(w), dev(x), empty_f32(n), empty_f32(n)
    _lib.check("noalloc", L.launch_matvec_q4k_batched_noalloc(ptr(wt), ptr(xt), ptr(y1), n, bpr, 1, None))
    _lib.check("matvec", L.launch_matvec_q4k(ptr(wt), ptr(xt), ptr(y2), n, bpr))
    assert np.array_equal(host(y1).view(np.uint32), host(y2).view(np.uint32))
