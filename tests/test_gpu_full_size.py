"""GPU parity at the BASELINE configurations' full sizes, through the C ABI.

- config 4: launch_matvec_q4k_batched on gate 18944x3584 and down 3584x18944
  at B = 1, 2, 4, 8, 16 (128 sampled rows of every batch row);
- config 5: launch_gemm_q4k_f16 on 18944x3584 x 512 tokens (64 sampled rows:
  per-element and Frobenius bounds);
- the f32 GEMV on the fused qkv 4608x3584 (every row);
- config 3: the 113-launch decode step (28 x qkv, o, gate|up, down + lm_head,
  3.98 GB of Q4_K) replayed twice through one mgq_chain; sampled rows of each
  distinct shape in the first, a middle and the last layer, and of lm_head.

Sampled rows are checked with the oracle's f64 dequant-dot (the reference's
method, examples/rocm_matvec_check.rs:38-54) at the BASELINE bound
|y - y_f64| <= 1e-4 * sum|w||x| per row; weights are the seeded reference
quantizer's bytes (configs 4, 5 and qkv) or seeded random blocks with finite
model-like d/dmin (the decode step, as bench.py builds it).
"""
import sys

import numpy as np
import pytest

from modgrad_amd import _lib
from tests.gpu_util import assert_gemv_close, dev, empty_f32, filled_u8, host, ptr

pytestmark = pytest.mark.gpu

HIDDEN, INTER, VOCAB = 3584, 18944, 152064
QKV = 28 * 128 + 2 * 4 * 128


def note(msg: str) -> None:
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def L():
    return _lib.load()


def sample(n: int, count: int, seed: int) -> np.ndarray:
    return np.sort(np.random.default_rng(seed).choice(n, size=min(count, n), replace=False))


def rows_of(w_host: np.ndarray, idx: np.ndarray, bpr: int) -> np.ndarray:
    return w_host.reshape(-1, bpr * 144)[idx].ravel()


# ------------------------------------------------------------- config 4 -----
_W4 = {}


def config4_weight(orc, name: str):
    """Seeded layer-0 gate / down weights (quantized once per module)."""
    if name not in _W4:
        n, k, t = (INTER, HIDDEN, 4) if name == "gate" else (HIDDEN, INTER, 6)
        seed = orc.layer_seed(0, t)
        w = orc.seeded_weight(seed, n, k)
        _W4[name] = (w, dev(w), n, k, seed)
    return _W4[name]


@pytest.mark.parametrize("batch", [1, 2, 4, 8, 16])
@pytest.mark.parametrize("name", ["gate", "down"])
def test_config4_batched_full_size(L, orc, name, batch):
    w, wt, n, k, seed = config4_weight(orc, name)
    bpr = k // 256
    note(f"config 4 batched {name} {n}x{k} B={batch}")
    X = orc.normal(seed ^ 0xA5A5 ^ batch, batch * k).reshape(batch, k)
    Xt, Yt = dev(X), empty_f32(batch * n)
    nws = L.mgq_batched_workspace_bytes(bpr, batch)
    ws = filled_u8(nws, 0xC3)
    _lib.check("batched", L.launch_matvec_q4k_batched(ptr(wt), ptr(Xt), ptr(Yt), n, bpr, batch,
                                                      ptr(ws), nws, None))
    Y = host(Yt).reshape(batch, n)
    idx = sample(n, 128, n + batch)
    Y_ref, A = orc.gemv_batched(rows_of(w, idx, bpr), X, idx.size, bpr)
    for b in range(batch):
        assert_gemv_close(Y[b, idx], Y_ref[b], A[b])
    assert np.all(np.isfinite(Y))


# ------------------------------------------------------------- config 5 -----
def test_config5_prefill_gemm_full_size(L, orc):
    n, k, m = INTER, HIDDEN, 512
    bpr = k // 256
    note(f"config 5 prefill gemm {n}x{k} x {m} tokens")
    w, wt, _, _, _ = config4_weight(orc, "gate")
    a = orc.normal(0xF16, m * k).astype(np.float16).reshape(m, k)
    at, ct = dev(a.view(np.uint16)), empty_f32(m * n)
    _lib.check("gemm", L.launch_gemm_q4k_f16(ptr(wt), ptr(at), ptr(ct), n, bpr, m, None))
    C = host(ct).reshape(m, n)
    assert np.all(np.isfinite(C))
    idx = sample(n, 64, 5)
    C_ref, A = orc.gemm_f16(w, a.view(np.uint16), n, bpr, rows=idx)
    Cg = C[:, idx].astype(np.float64)
    C_ref = C_ref.astype(np.float64)
    assert np.all(np.abs(Cg - C_ref) <= 1e-2 * A / np.sqrt(k))
    assert np.linalg.norm(Cg - C_ref) <= 1e-3 * np.linalg.norm(C_ref)


# ------------------------------------------------------------ f32 qkv -------
def test_qkv_f32_matvec_full_size(L, orc):
    note(f"f32 matvec fused qkv {QKV}x{HIDDEN}")
    seed = orc.layer_seed(2, 0)
    w = orc.seeded_weight(seed, QKV, HIDDEN)
    x = orc.normal(seed ^ 0xA5A5, HIDDEN)
    wt, xt, yt = dev(w), dev(x), empty_f32(QKV)
    _lib.check("matvec", L.launch_matvec_q4k(ptr(wt), ptr(xt), ptr(yt), QKV, HIDDEN // 256))
    y_ref, a = orc.gemv(w, x, QKV, HIDDEN // 256)
    assert_gemv_close(host(yt), y_ref, a)


# ------------------------------------------------------ config 3: the step --
def decode_shapes():
    out = []
    for l in range(28):
        out += [(l, "qkv", QKV, HIDDEN), (l, "o", HIDDEN, HIDDEN),
                (l, "gate_up", 2 * INTER, HIDDEN), (l, "down", HIDDEN, INTER)]
    out.append((28, "lm_head", VOCAB, HIDDEN))
    return out


def test_config3_decode_step_chain_full_size(L, orc):
    import torch
    from modgrad_amd.q4k import Chain
    shapes = decode_shapes()
    note(f"config 3 decode step: {len(shapes)} launches through one chain")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0x7B)
    launches = []
    for l, name, n, k in shapes:
        nblk = n * (k // 256)
        w = torch.randint(0, 256, (nblk, 144), dtype=torch.uint8, device="cuda", generator=gen)
        dd = (torch.rand((nblk, 2), device="cuda", generator=gen) * 2e-3 + 1e-4).to(torch.float16)
        w[:, 0:4] = dd.view(torch.uint8).view(nblk, 4)
        x = torch.randn(k, device="cuda", generator=gen)
        y = torch.full((n,), float("nan"), device="cuda")
        launches.append((l, name, w.view(-1), x, y, n, k))
    torch.cuda.synchronize()
    assert len(launches) == 113
    ch = Chain([(w.data_ptr(), x.data_ptr(), y.data_ptr(), n, k // 256)
                for _, _, w, x, y, n, k in launches])
    ch.launch()
    torch.cuda.synchronize()
    first = [y.clone() for *_, y, _, _ in launches]
    for *_, y, _, _ in launches:
        y.fill_(float("nan"))
    ch.launch()  # a replay: same bits
    torch.cuda.synchronize()
    ch.close()
    for (l, name, w, x, y, n, k), y0 in zip(launches, first):
        assert torch.equal(y.view(torch.int32), y0.view(torch.int32)), f"L{l}.{name} replay differs"
    worst = 0.0
    for l, name, w, x, y, n, k in launches:
        if l not in (0, 13, 27, 28):
            continue
        bpr = k // 256
        idx = sample(n, 96, 31 * l + n)
        wr = w.view(n, bpr * 144)[torch.from_numpy(idx).cuda()].cpu().numpy().ravel()
        y_ref, a = orc.gemv(wr, x.cpu().numpy(), idx.size, bpr)
        worst = max(worst, assert_gemv_close(y.cpu().numpy()[idx], y_ref, a))
    print(f"decode step: worst sampled err/absdot {worst:.3e}")
