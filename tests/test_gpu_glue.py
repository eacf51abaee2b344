"""GPU parity of the decode glue and its fusion into the matvec, through the C
ABI, against the CPU oracle (orq_rms_norm, orq_glu, orq_gemv_f64_abs).

Bounds:
  rms_norm  |y - y_ref| <= 4e-6 |y_ref|   (same reduction order; the GPU
            rsqrtf may differ from 1/sqrtf by about an ulp)
  glu       |out - ref| <= 2e-6 |gate * up| (tanhf/expf of the device
            library vs the host's)
  fused     the matvec bound, 1e-4 * sum|w||xn| per row, xn the oracle's
            normalized vector (Q4_K and Q6_K); for the GLU the bound propagates through
            act (|act'| <= 1.13 for gelu_tanh, <= 1.1 for silu).
"""
import sys

import numpy as np
import pytest

from modgrad_amd import _lib
from tests.gpu_util import assert_gemv_close, dev, empty_f32, host, ptr

pytestmark = pytest.mark.gpu


def note(msg: str) -> None:
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def L():
    return _lib.load()


@pytest.mark.parametrize("rows,hidden", [(1, 3584), (28, 256), (4, 100), (1, 1), (3, 5000)])
def test_rms_norm_matches_oracle(L, orc, rows, hidden):
    note(f"rms_norm rows={rows} hidden={hidden}")
    rng = np.random.default_rng(rows * 7 + hidden)
    x = (rng.standard_normal(rows * hidden) * 2.5).astype(np.float32)
    w = rng.standard_normal(hidden).astype(np.float32)
    xt, wt, yt = dev(x), dev(w), empty_f32(rows * hidden)
    _lib.check("launch_rms_norm", L.launch_rms_norm(ptr(xt), ptr(wt), ptr(yt), rows, hidden, 1e-6))
    y = host(yt)
    ref = orc.rms_norm(x, w, rows, hidden, 1e-6)
    assert np.all(np.abs(y.astype(np.float64) - ref) <= 4e-6 * np.abs(ref) + 1e-30)


@pytest.mark.parametrize("n,act", [(18944, 0), (1, 0), (1000, 1), (4097, 1)])
def test_glu_matches_oracle(L, orc, n, act):
    note(f"glu n={n} act={act}")
    rng = np.random.default_rng(n + act)
    g = (rng.standard_normal(n) * 3).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    gt, ut, ot = dev(g), dev(u), empty_f32(n)
    if act == 0:
        _lib.check("launch_geglu", L.launch_geglu(ptr(gt), ptr(ut), ptr(ot), n))
    else:
        _lib.check("launch_glu_ex", L.launch_glu_ex(ptr(gt), ptr(ut), ptr(ot), n, act, None))
    out = host(ot)
    ref = orc.glu(g, u, act)
    assert np.all(np.abs(out.astype(np.float64) - ref) <= 2e-6 * np.abs(g * u) + 1e-30)


@pytest.mark.parametrize("n", [3584, 1, 257, 18944])
def test_residual_add_and_scale_are_exact(L, n):
    # transformer_ops.hip:10-30: h += x and h *= s are single IEEE f32
    # operations per element, so the result is the correctly rounded one that
    # numpy's float32 arithmetic gives, bit for bit, specials included
    note(f"residual_add / scale n={n}")
    rng = np.random.default_rng(n)
    h = (rng.standard_normal(n) * 10).astype(np.float32)
    x = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    if n >= 4:
        h[:4] = [np.inf, -0.0, 3.0e38, np.nan]
        x[:4] = [1.0, 0.0, 3.0e38, 1.0]
    ht, xt = dev(h), dev(x)
    _lib.check("launch_residual_add", L.launch_residual_add(ptr(ht), ptr(xt), n))
    with np.errstate(over="ignore", invalid="ignore"):
        ref = h + x
    got = host(ht)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    s = np.float32(0.7071068)
    _lib.check("launch_scale_ex", L.launch_scale_ex(ptr(ht), float(s), n, None))
    with np.errstate(invalid="ignore"):
        ref_s = ref * s
    assert np.array_equal(host(ht).view(np.uint32), ref_s.view(np.uint32))


def _weights(orc, seed, n, bpr):
    return orc.seeded_weight(seed, n, bpr * 256)


# (n, bpr): persistent whole-row (cfg 3), small-N (cfg 1), long K small-N
# (cfg 2), long K persistent (cfg 0), ragged row groups
FUSED_SHAPES = [(4608, 14), (3584, 14), (300, 3), (64, 74), (5000, 74), (33, 1), (4609, 14)]


@pytest.mark.parametrize("n,bpr", FUSED_SHAPES)
def test_matvec_rmsnorm_matches_norm_then_matvec(L, orc, n, bpr):
    note(f"matvec_q4k_rmsnorm n={n} bpr={bpr}")
    k = bpr * 256
    w = _weights(orc, 500 + n, n, bpr)
    x = orc.normal(600 + n, k, 1.7)
    nw = orc.normal(700 + n, k, 0.5) + np.float32(1.0)
    eps = 1e-6
    wt, xt, nt, yt = dev(w), dev(x), dev(nw), empty_f32(n)
    _lib.check("rmsnorm matvec", L.launch_matvec_q4k_rmsnorm_ex(ptr(wt), ptr(xt), ptr(nt), eps,
                                                                ptr(yt), n, bpr, None))
    y = host(yt)
    xn = orc.rms_norm(x, nw, 1, k, eps)
    y_ref, A = orc.gemv(w, xn, n, bpr)
    assert_gemv_close(y, y_ref, A)


@pytest.mark.parametrize("n,bpr", FUSED_SHAPES)
@pytest.mark.parametrize("act,norm", [(0, True), (1, True), (0, False)])
def test_matvec_glu_matches_unfused_chain(L, orc, n, bpr, act, norm):
    note(f"matvec_q4k_glu n={n} bpr={bpr} act={act} norm={norm}")
    k = bpr * 256
    wg = _weights(orc, 800 + n, n, bpr)
    wu = _weights(orc, 900 + n, n, bpr)
    x = orc.normal(1000 + n, k, 1.3)
    nw = orc.normal(1100 + n, k, 0.5) + np.float32(1.0)
    eps = 1e-5
    wgt, wut, xt, nt, yt = dev(wg), dev(wu), dev(x), dev(nw), empty_f32(n)
    _lib.check("glu matvec", L.launch_matvec_q4k_glu_ex(ptr(wgt), ptr(wut), ptr(xt),
                                                        ptr(nt) if norm else None, eps, act,
                                                        ptr(yt), n, bpr, None))
    y = host(yt).astype(np.float64)
    xn = orc.rms_norm(x, nw, 1, k, eps) if norm else x
    g, Ag = orc.gemv(wg, xn, n, bpr)
    u, Au = orc.gemv(wu, xn, n, bpr)
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    if act == 0:
        a = 0.5 * g64 * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (g64 + 0.044715 * g64 ** 3)))
    else:
        a = g64 / (1.0 + np.exp(-g64))
    ref = a * u64
    bound = 1e-4 * (1.13 * Ag * np.abs(u64) + np.abs(a) * Au) + 1e-5 * np.abs(ref) + 1e-30
    err = np.abs(y - ref)
    bad = np.nonzero(~(err <= bound))[0]
    assert bad.size == 0, (bad[:5].tolist(), err[bad[:5]].tolist(), bound[bad[:5]].tolist())


# Q6_K tensors a norm feeds: attn_v 512x3584, a 1000-row K = 2048 shape, one
# block, ragged row groups (4104 rows); n * bpr a multiple of 8 (whole
# 16-byte chunks), as the fused kernel requires
Q6_NORM_SHAPES = [(512, 14), (1000, 8), (48, 1), (4104, 14)]


@pytest.mark.parametrize("n,bpr", Q6_NORM_SHAPES)
def test_matvec_q6k_rmsnorm_matches_norm_then_matvec(L, orc, n, bpr):
    from tests.gpu_util import random_kquant_bytes
    note(f"matvec_q6k_rmsnorm n={n} bpr={bpr}")
    k = bpr * 256
    w = random_kquant_bytes(np.random.default_rng(0x66 + n + bpr), n * bpr, 210)
    x = orc.normal(1200 + n, k, 1.7)
    nw = orc.normal(1300 + n, k, 0.5) + np.float32(1.0)
    eps = 1e-6
    wt, xt, nt, yt = dev(w), dev(x), dev(nw), empty_f32(n)
    _lib.check("q6k rmsnorm matvec", L.launch_matvec_q6k_rmsnorm_ex(ptr(wt), ptr(xt), ptr(nt), eps,
                                                                    ptr(yt), n, bpr, None))
    y = host(yt)
    xn = orc.rms_norm(x, nw, 1, k, eps)
    y_ref, A = orc.gemv_kquant(210, w, xn, n, bpr)
    assert_gemv_close(y, y_ref, A)


def test_matvec_q6k_rmsnorm_output_matrix(L, orc):
    """The Q4_K_M output matrix, 152064 x 3584 Q6_K, at full size (rows
    sampled, including the last ones)."""
    import torch
    note("matvec_q6k_rmsnorm 152064x3584")
    n, bpr = 152064, 14
    k = bpr * 256
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0x6F)
    wt = torch.randint(0, 256, (n * bpr, 210), dtype=torch.uint8, device="cuda", generator=gen)
    dd = (torch.rand((n * bpr,), device="cuda", generator=gen) * 2e-3 + 1e-4).to(torch.float16)
    wt[:, 208:210] = dd.view(torch.uint8).view(-1, 2)
    x = orc.normal(1400, k, 1.1)
    nw = orc.normal(1500, k, 0.4) + np.float32(1.0)
    xt, nt, yt = dev(x), dev(nw), empty_f32(n)
    _lib.check("q6k rmsnorm lm_head", L.launch_matvec_q6k_rmsnorm_ex(wt.data_ptr(), ptr(xt), ptr(nt),
                                                                     1e-6, ptr(yt), n, bpr, None))
    idx = np.unique(np.concatenate([np.random.default_rng(3).choice(n, 200, replace=False),
                                    np.arange(n - 24, n)]))
    wr = wt.view(n, bpr * 210)[torch.from_numpy(idx).cuda()].cpu().numpy().ravel()
    xn = orc.rms_norm(x, nw, 1, k, 1e-6)
    y_ref, A = orc.gemv_kquant(210, wr, xn, idx.size, bpr)
    assert_gemv_close(host(yt)[idx], y_ref, A)


def test_matvec_q6k_rmsnorm_rejects_what_its_kernel_cannot_take(L, orc):
    """hipErrorNotSupported (no launch) for a weight that is not 16-byte
    aligned, K > 14 blocks, or a tensor that is not whole 16-byte chunks;
    hipErrorInvalidValue without norm weights."""
    from tests.gpu_util import random_kquant_bytes
    note("matvec_q6k_rmsnorm argument checks")
    n, bpr = 64, 16
    w = random_kquant_bytes(np.random.default_rng(5), n * bpr + 1, 210)
    x = orc.normal(1, bpr * 256)
    wt, xt, nt, yt = dev(w), dev(x), dev(np.ones(bpr * 256, np.float32)), empty_f32(n)
    f = L.launch_matvec_q6k_rmsnorm_ex
    assert f(ptr(wt) + 2, ptr(xt), ptr(nt), 1e-6, ptr(yt), n, 8, None) == 801
    assert f(ptr(wt), ptr(xt), ptr(nt), 1e-6, ptr(yt), n, 15, None) == 801
    assert f(ptr(wt), ptr(xt), ptr(nt), 1e-6, ptr(yt), 3, 1, None) == 801
    assert f(ptr(wt), ptr(xt), None, 1e-6, ptr(yt), n, 8, None) == _lib.hipErrorInvalidValue


def test_fused_matvecs_are_deterministic(L, orc):
    note("fused matvecs repeat bit-exactly")
    n, bpr = 2000, 14
    wg, wu = _weights(orc, 1, n, bpr), _weights(orc, 2, n, bpr)
    x = orc.normal(3, bpr * 256)
    nw = np.ones(bpr * 256, np.float32)
    wgt, wut, xt, nt = dev(wg), dev(wu), dev(x), dev(nw)
    outs = []
    for _ in range(3):
        yt = empty_f32(n)
        _lib.check("glu", L.launch_matvec_q4k_glu_ex(ptr(wgt), ptr(wut), ptr(xt), ptr(nt), 1e-6, 0,
                                                     ptr(yt), n, bpr, None))
        outs.append(host(yt))
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[1], outs[2])
