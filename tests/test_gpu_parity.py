"""GPU parity: libmodgrad_q4k through its C ABI vs the CPU oracle.

Gates (BASELINE): dequant bit-exact; GEMV per row
|y - y_f64| <= 1e-4 * sum_k |w_rk||x_k|. Inputs follow the seeded convention
(oracle.oracle docstring); each case prints its name before touching the GPU.
"""
import ctypes
import sys

import numpy as np
import pytest

from modgrad_amd import _lib
from tests.gpu_util import (assert_gemv_close, dev, empty_f32, filled_u8, host, ptr,
                            random_q4k_bytes)

pytestmark = pytest.mark.gpu


def note(msg: str) -> None:
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def L():
    return _lib.load()


def run_gemv(L, w: np.ndarray, x: np.ndarray, n: int, bpr: int, w_offset: int = 0) -> np.ndarray:
    import torch
    wt = torch.zeros(w.size + 64, dtype=torch.uint8, device="cuda")
    wt[w_offset: w_offset + w.size].copy_(torch.from_numpy(w))
    xt = dev(x)
    yt = empty_f32(n)
    _lib.check("launch_matvec_q4k", L.launch_matvec_q4k(ptr(wt) + w_offset, ptr(xt), ptr(yt), n, bpr))
    return host(yt)


# ------------------------------------------------------------------ dequant --
@pytest.mark.parametrize("n_blocks", [1, 8])
def test_dequant_matches_host_reference_signal(L, orc, n_blocks):
    # tests/dequant_q4k.rs:48-129 (there max|diff| < 1e-5; here bit-exact)
    note(f"dequant smooth n_blocks={n_blocks}")
    q = orc.quantize(orc.smooth(n_blocks * 256))
    qt, out = dev(q), empty_f32(n_blocks * 256)
    _lib.check("launch_dequant_q4k", L.launch_dequant_q4k(ptr(qt), n_blocks, ptr(out)))
    got = host(out)
    assert got.view(np.uint32).tolist() == orc.dequantize(q).view(np.uint32).tolist()


def test_dequant_every_half_scale_value(L, orc):
    # d takes all 65536 half bit patterns (subnormals, Inf, NaN included)
    note("dequant exhaustive d/dmin")
    rng = np.random.default_rng(100)
    b = rng.integers(0, 256, size=(65536, 144), dtype=np.uint8)
    h = np.arange(65536, dtype=np.uint16)
    b[:, 0:2] = h.view(np.uint8).reshape(-1, 2)
    b[:, 2:4] = ((h.astype(np.uint32) * 7919) & 0xFFFF).astype(np.uint16).view(np.uint8).reshape(-1, 2)
    q = b.ravel()
    qt, out = dev(q), empty_f32(65536 * 256)
    _lib.check("launch_dequant_q4k", L.launch_dequant_q4k(ptr(qt), 65536, ptr(out)))
    got = host(out)
    want = orc.dequantize(q)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_dequant_seeded_layer_tensor_and_unaligned_output(L, orc):
    note("dequant seeded 512x3584, out offset 4 B")
    import torch
    q = orc.seeded_weight(orc.layer_seed(0, 1), 512, 3584)
    nb = q.size // 144
    qt = dev(q)
    out = torch.zeros(nb * 256 + 4, dtype=torch.float32, device="cuda")
    _lib.check("launch_dequant_q4k", L.launch_dequant_q4k(ptr(qt), nb, ptr(out) + 4))
    got = host(out)
    assert np.all(got[0] == 0) and np.all(got[1 + nb * 256:] == 0)  # nothing outside
    assert np.array_equal(got[1:1 + nb * 256].view(np.uint32), orc.dequantize(q).view(np.uint32))


# --------------------------------------------------------------------- GEMV --
SMALL = [(1, 1), (15, 1), (16, 2), (17, 3), (31, 13), (33, 14), (64, 74), (100, 5), (47, 148)]


@pytest.mark.parametrize("n,bpr", SMALL)
def test_matvec_small_shapes_seeded(L, orc, n, bpr):
    note(f"matvec seeded n={n} bpr={bpr}")
    w = orc.seeded_weight(1000 + n * 7 + bpr, n, bpr * 256)
    x = orc.normal(2000 + n + bpr, bpr * 256)
    y = run_gemv(L, w, x, n, bpr)
    y_ref, a = orc.gemv(w, x, n, bpr)
    assert_gemv_close(y, y_ref, a)


def test_matvec_random_bytes_wide_dynamic_range(L, orc):
    note("matvec random bytes, x over 1e-20..1e20")
    rng = np.random.default_rng(7)
    n, bpr = 96, 14
    w = random_q4k_bytes(rng, n * bpr, finite_scales=False)
    w.reshape(-1, 144)[::5, 0:2] = 0x00  # some zero d
    mag = 10.0 ** rng.uniform(-20, 20, size=bpr * 256)
    x = (mag * rng.choice([-1.0, 1.0], size=mag.size)).astype(np.float32)
    y = run_gemv(L, w, x, n, bpr)
    y_ref, a = orc.gemv(w, x, n, bpr)
    ok = np.isfinite(y_ref)
    assert np.array_equal(np.isfinite(y), ok)
    assert_gemv_close(y[ok], y_ref[ok], a[ok])


@pytest.mark.parametrize("n,bpr", [(24576 + 17, 2), (30000, 14), (16, 40), (17, 29),
                                   (4100, 17), (4200, 74), (5000, 112), (300, 100),
                                   (20005, 13), (16009, 7), (3590, 75), (4609, 14), (2047, 20)])
def test_matvec_random_bytes_all_configs(L, orc, n, bpr):
    # shapes that select each launch configuration (many / few row groups,
    # single- and multi-stage K, ragged last stage and row group) and each
    # count of activation chunks per lane (1, 2, 4, 8), including the
    # single-buffered fallback when the double-buffered stages do not fit;
    # odd blocks per row on the persistent and the long-row wave kernels
    # (a unit half past the row end, units wholly past it) with a partial
    # last row group, and one-group-per-CU rows with a ragged last group
    note(f"matvec random bytes n={n} bpr={bpr}")
    rng = np.random.default_rng(n + bpr)
    w = random_q4k_bytes(rng, n * bpr)
    x = rng.standard_normal(bpr * 256).astype(np.float32)
    y = run_gemv(L, w, x, n, bpr)
    y_ref, a = orc.gemv(w, x, n, bpr)
    assert_gemv_close(y, y_ref, a)


def test_matvec_unit_vectors_extract_columns(L, orc):
    note("matvec x = e_k")
    n, bpr = 48, 3
    w = orc.seeded_weight(31, n, bpr * 256)
    wd = orc.dequantize(w).reshape(n, -1)
    for k in (0, 5, 32, 63, 64, 255, 256, 511, 767):
        x = np.zeros(bpr * 256, np.float32)
        x[k] = 1.0
        y = run_gemv(L, w, x, n, bpr)
        # d*sc*q - dmin*m may cancel; the kernel rounds its two terms in a
        # different order than the oracle, so compare at that terms' scale.
        assert np.all(np.abs(y - wd[:, k]) <= 1e-6 * np.abs(wd).max())


def test_matvec_all_zero_rows_give_zero(L, orc):
    note("matvec zero weights")
    n, bpr = 40, 4
    w = np.zeros(n * bpr * 144, np.uint8)
    x = orc.normal(5, bpr * 256)
    y = run_gemv(L, w, x, n, bpr)
    assert np.all(y == 0.0)


@pytest.mark.parametrize("name,n,k,t", [("q", 3584, 3584, 0), ("k", 512, 3584, 1),
                                        ("gate", 18944, 3584, 4), ("down", 3584, 18944, 6),
                                        ("gate_up", 37888, 3584, 5)])
def test_matvec_baseline_layer_shapes(L, orc, name, n, k, t):
    note(f"matvec layer-0 {name} {n}x{k}")
    seed = orc.layer_seed(0, t)
    w = orc.seeded_weight(seed, n, k)
    x = orc.normal(seed ^ 0xA5A5, k)
    y = run_gemv(L, w, x, n, k // 256)
    y_ref, a = orc.gemv(w, x, n, k // 256)
    worst = assert_gemv_close(y, y_ref, a)
    print(f"{name}: worst err/absdot = {worst:.3e}")


@pytest.mark.parametrize("fmt", [144, 210])
def test_matvec_lm_head_full_size(L, orc, fmt):
    # BASELINE lm_head 152064x3584: the longest persistent schedule (19 rounds
    # of row groups per work-group, the older member of each CU pair taking
    # the extra rounds); every row against the f64 oracle
    from tests.gpu_util import random_kquant_bytes
    n, bpr = 152064, 14
    note(f"{'q4k' if fmt == 144 else 'q6k'} lm_head {n}x{bpr * 256}")
    rng = np.random.default_rng(0x1A4EAD + fmt)
    w = (random_q4k_bytes(rng, n * bpr) if fmt == 144
         else random_kquant_bytes(rng, n * bpr, 210))
    x = rng.standard_normal(bpr * 256).astype(np.float32)
    wt, xt, yt = dev(w), dev(x), empty_f32(n)
    fn = L.launch_matvec_q4k if fmt == 144 else L.launch_matvec_q6k
    _lib.check("lm_head", fn(ptr(wt), ptr(xt), ptr(yt), n, bpr))
    y_ref, a = orc.gemv_kquant(fmt, w, x, n, bpr)
    assert_gemv_close(host(yt), y_ref, a)


@pytest.mark.parametrize("n,bpr", [(3584, 14), (3584, 74), (40, 148)])
def test_matvec_is_deterministic(L, orc, n, bpr):
    # shapes that split K across work-groups: the last arriver sums the
    # partials in slice order, so repeated launches agree bit for bit
    note(f"matvec determinism {n}x{bpr * 256}")
    w = orc.seeded_weight(7000 + bpr, n, bpr * 256)
    x = orc.normal(7100 + bpr, bpr * 256)
    import torch
    wt, xt = dev(w), dev(x)
    outs = []
    for _ in range(3):
        yt = empty_f32(n)
        _lib.check("launch_matvec_q4k", L.launch_matvec_q4k(ptr(wt), ptr(xt), ptr(yt), n, bpr))
        outs.append(host(yt))
    assert all(np.array_equal(outs[0].view(np.uint32), o.view(np.uint32)) for o in outs[1:])
    y_ref, a = orc.gemv(w, x, n, bpr)
    assert_gemv_close(outs[0], y_ref, a)
    del torch


# (n, k): rows of U = 256/gcd(k, 256) rows per unit (U = 2, 8, 4, 2, 8 with a
# 153-block unit), k % 32 != 0 (vector-ALU kernel), k % 256 == 0 (row layout)
@pytest.mark.parametrize("n,k", [(4864, 896), (8, 96), (16, 320), (64, 1152), (40, 4896),
                                 (128, 258), (3, 256 * 3)])
def test_matvec_flat_layout(L, orc, n, k):
    note(f"matvec flat {n}x{k}")
    w = orc.seeded_weight(0xC0F1 + k, n, k)
    x = orc.normal(0xC0F1 ^ 0xA5A5, k)
    wt, xt, yt = dev(w), dev(x), empty_f32(n)
    _lib.check("launch_matvec_q4k_ex",
               L.launch_matvec_q4k_ex(ptr(wt), ptr(xt), ptr(yt), n, k, _lib.LAYOUT_FLAT, None))
    y = host(yt)
    y_ref, a = orc.gemv_flat(w, x, n, k)
    assert_gemv_close(y, y_ref, a)


def test_matvec_flat_layout_random_bytes_and_misaligned_x(L, orc):
    # random blocks (non-finite d / dmin included) on the whole-unit kernel,
    # with x 16-byte aligned and 4 bytes past that, same result
    note("matvec flat 4864x896 random bytes; x offset 4 B")
    import torch
    n, k = 4864, 896
    rng = np.random.default_rng(0xF1A7)
    w = random_q4k_bytes(rng, n * k // 256, finite_scales=False)
    x = rng.standard_normal(k).astype(np.float32)
    wt, yt = dev(w), empty_f32(n)
    xt = torch.zeros(k + 4, dtype=torch.float32, device="cuda")
    xt[1:k + 1].copy_(torch.from_numpy(x))
    y_ref, a = orc.gemv_flat(w, x, n, k)
    ok = np.isfinite(y_ref)
    xa = dev(x)  # 16-byte aligned copy
    for off in (4, 0):
        xp = ptr(xt) + off if off else ptr(xa)
        _lib.check("launch_matvec_q4k_ex",
                   L.launch_matvec_q4k_ex(ptr(wt), xp, ptr(yt), n, k, _lib.LAYOUT_FLAT, None))
        y = host(yt)
        assert np.array_equal(np.isfinite(y), ok)
        assert_gemv_close(y[ok], y_ref[ok], a[ok])


# ------------------------------------------------------------------ batched --
def run_batched(L, w, X, n, bpr, batch, w_offset=0):
    wt = dev(np.concatenate([np.zeros(w_offset, np.uint8), w]))
    Xt, Yt = dev(X), empty_f32(batch * n)
    nws = L.mgq_batched_workspace_bytes(bpr, batch)
    ws = filled_u8(nws, 0xAB)  # stale bytes from an earlier user
    _lib.check("batched", L.launch_matvec_q4k_batched(ptr(wt) + w_offset, ptr(Xt), ptr(Yt), n, bpr,
                                                      batch, ptr(ws), nws, None))
    return host(Yt).reshape(batch, n)


@pytest.mark.parametrize("batch", [1, 2, 3, 4, 8, 9, 16])
def test_matvec_batched(L, orc, batch):
    note(f"batched B={batch}")
    n, bpr = 1000, 14
    w = orc.seeded_weight(51, n, bpr * 256)
    X = orc.normal(52 + batch, batch * bpr * 256).reshape(batch, -1)
    Y = run_batched(L, w, X, n, bpr, batch)
    Y_ref, A = orc.gemv_batched(w, X, n, bpr)
    for b in range(batch):
        assert_gemv_close(Y[b], Y_ref[b], A[b])


@pytest.mark.parametrize("n,bpr,batch", [(17, 1, 5), (33, 3, 16), (700, 74, 4), (300, 9, 12),
                                         (9000, 16, 2)])
def test_matvec_batched_shapes_random_bytes(L, orc, n, bpr, batch):
    # ragged row groups, partial K slices (idle waves), several K slices,
    # two batch sets, many row groups per work-group
    note(f"batched random bytes n={n} bpr={bpr} B={batch}")
    rng = np.random.default_rng(n * 31 + bpr + batch)
    w = random_q4k_bytes(rng, n * bpr)
    X = rng.standard_normal((batch, bpr * 256)).astype(np.float32)
    X[:, ::7] *= 1e-3  # mixed magnitudes within a block
    Y = run_batched(L, w, X, n, bpr, batch)
    Y_ref, A = orc.gemv_batched(w, X, n, bpr)
    for b in range(batch):
        assert_gemv_close(Y[b], Y_ref[b], A[b])


def test_matvec_batched_matches_gemv_and_is_deterministic(L, orc):
    note("batched vs gemv, determinism")
    n, bpr, batch = 512, 14, 16
    w = orc.seeded_weight(61, n, bpr * 256)
    X = orc.normal(62, batch * bpr * 256).reshape(batch, -1)
    Y1 = run_batched(L, w, X, n, bpr, batch)
    Y2 = run_batched(L, w, X, n, bpr, batch)
    assert np.array_equal(Y1, Y2)
    for b in (0, 7, 8, 15):
        y = run_gemv(L, w, X[b], n, bpr)
        y_ref, a = orc.gemv(w, X[b], n, bpr)
        assert_gemv_close(Y1[b], y_ref, a)
        assert_gemv_close(y, y_ref, a)


@pytest.mark.parametrize("n,bpr,batch", [(45, 33, 8), (300, 74, 16), (3584, 74, 5)])
def test_matvec_batched_k_split(L, orc, n, bpr, batch):
    # few row groups and K >= 4 slices of 8 blocks: 32-row groups, K split in
    # two, partials added onto a zeroed Y. Odd slice count (33 blocks: 3 + 2
    # slices, the last one block), a ragged row group, two batch sets, the
    # ffn_down shape; two K parts add in either order to the same bits
    note(f"batched K split n={n} bpr={bpr} B={batch}")
    w = orc.seeded_weight(71 + n, n, bpr * 256)
    X = orc.normal(72 + bpr, batch * bpr * 256).reshape(batch, -1)
    Y1 = run_batched(L, w, X, n, bpr, batch)
    Y2 = run_batched(L, w, X, n, bpr, batch)
    assert np.array_equal(Y1.view(np.uint32), Y2.view(np.uint32))
    Y_ref, A = orc.gemv_batched(w, X, n, bpr)
    for b in range(batch):
        assert_gemv_close(Y1[b], Y_ref[b], A[b])


@pytest.mark.parametrize("n,bpr,batch", [(150000, 1, 8), (80000, 1, 16)])
def test_matvec_batched_many_rows_stage_kernel(L, orc, n, bpr, batch):
    # so many row groups per work-group that the wave kernel's per-wavefront
    # row sums would not fit LDS: the stage kernel runs these
    note(f"batched stage kernel n={n} bpr={bpr} B={batch}")
    w = orc.seeded_weight(81 + batch, n, bpr * 256)
    X = orc.normal(82 + batch, batch * bpr * 256).reshape(batch, -1)
    Y = run_batched(L, w, X, n, bpr, batch)
    Y_ref, A = orc.gemv_batched(w, X, n, bpr)
    for b in range(batch):
        assert_gemv_close(Y[b], Y_ref[b], A[b])


def test_matvec_batched_single_row_is_the_matvec(L, orc):
    # batch 1 runs the matvec itself (no operand-table pass): bit-identical
    note("batched B=1 == gemv")
    n, bpr = 3000, 14
    w = orc.seeded_weight(63, n, bpr * 256)
    x = orc.normal(64, bpr * 256)
    Y = run_batched(L, w, x.reshape(1, -1), n, bpr, 1)
    assert np.array_equal(Y[0], run_gemv(L, w, x, n, bpr))


# Just past one 16-row group per CU the launcher runs one group of
# ceil(N / #CUs) rows per CU (two 16-row tiles, rows past the group re-read
# its last row): ragged groups, several K lengths, random bytes.
@pytest.mark.parametrize("n,bpr", [(4112, 14), (4600, 7), (6000, 1), (5000, 14)])
def test_matvec_one_group_per_cu_shapes(L, orc, n, bpr):
    note(f"matvec one group per CU n={n} bpr={bpr}")
    rng = np.random.default_rng(n * 31 + bpr)
    w = random_q4k_bytes(rng, n * bpr)
    x = rng.standard_normal(bpr * 256).astype(np.float32)
    y = run_gemv(L, w, x, n, bpr)
    y_ref, a = orc.gemv(w, x, n, bpr)
    assert_gemv_close(y, y_ref, a)


# Each 32-value sub-block of x at its own power of two, from float32's
# denormals to 2^110, on the shapes of each wave launch (qkv's one group per
# CU, o, the persistent gate|up, the long-row down, a ragged persistent one):
# the matrix-core forms scale each sub-block of x by a power of two of their
# own before splitting it into digits, and that scale must cover every
# exponent (a sub-block at 2^110 dominates each row's bound and pins it).
# Much larger activations can overflow float32 in a sub-block's partial
# products sc * sum(q x) and m * sum(x), which the kernels round before they
# multiply by d and dmin, as the sum of 32 values near 2^127 itself can.
@pytest.mark.parametrize("n,bpr", [(4608, 14), (3584, 14), (37888, 14), (3584, 74), (20005, 13)])
def test_matvec_per_subblock_magnitudes(L, orc, n, bpr):
    note(f"matvec per-sub-block magnitudes n={n} bpr={bpr}")
    rng = np.random.default_rng(n * 13 + bpr)
    k = bpr * 256
    w = random_q4k_bytes(rng, n * bpr, d_scale=1e-5)
    ex = rng.integers(-140, 100, size=k // 32)
    ex[0], ex[1], ex[2] = 110, -149, 0
    x = (rng.standard_normal((k // 32, 32)) * np.exp2(ex.astype(np.float64))[:, None])
    x = x.astype(np.float32).ravel()
    y = run_gemv(L, w, x, n, bpr)
    y_ref, a = orc.gemv(w, x, n, bpr)
    assert np.all(np.isfinite(y_ref))
    assert_gemv_close(y, y_ref, a)
    # the same vector without the 2^110 sub-block: the next largest (up to
    # 2^99) then sets the bound
    x[0:32] = 0.0
    y = run_gemv(L, w, x, n, bpr)
    y_ref, a = orc.gemv(w, x, n, bpr)
    assert_gemv_close(y, y_ref, a)


def test_matvec_f16_wave_forms_under_switch():
    # MGQ_GEMV_I8=0 (read once per process) puts every wave launch, the
    # fused RMSNorm / GLU matvecs and the Q5_K matvec on the f16 matrix-core
    # form: the matvec, Q5_K / Q6_K and fused cases again, in one child
    # process with the switch set
    import os
    import subprocess
    note("matvec f16 wave forms (child process, MGQ_GEMV_I8=0)")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    cases = ("matvec_random_bytes_all_configs or per_subblock or baseline_layer_shapes or "
             "one_group_per_cu or lm_head_full_size or matvec_small_shapes or "
             "matvec_rmsnorm_matches_norm_then_matvec or matvec_glu_matches_unfused_chain or "
             "kquant_matvec_matches_oracle")
    glue = os.path.join(os.path.dirname(os.path.abspath(__file__)), "test_gpu_glue.py")
    r = subprocess.run([sys.executable, "-m", "pytest", os.path.abspath(__file__), glue, "-m", "gpu",
                        "-x", "-q", "-p", "no:cacheprovider", "-k", cases],
                       env=dict(os.environ, MGQ_GEMV_I8="0"), cwd=root, capture_output=True,
                       text=True, timeout=110)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-2000:]
    assert " passed" in r.stdout and "deselected" in r.stdout


# --------------------------------------------------------------------- GEMM --
# (70000, 1, 16): 547 tiles of 128 rows but 438 of 160 for 512 resident
# slots, so the 160-row tile runs; the others, ragged tiles of either height
@pytest.mark.parametrize("n,bpr,m", [(64, 2, 8), (100, 14, 33), (256, 1, 1), (300, 5, 130),
                                     (1030, 3, 257), (130, 9, 384), (70000, 1, 16)])
def test_gemm_f16_small(L, orc, n, bpr, m):
    note(f"gemm n={n} bpr={bpr} m={m}")
    w = orc.seeded_weight(61, n, bpr * 256)
    a = orc.normal(0xF16, m * bpr * 256).astype(np.float16).reshape(m, -1)
    wt, at, ct = dev(w), dev(a.view(np.uint16)), empty_f32(m * n)
    _lib.check("gemm", L.launch_gemm_q4k_f16(ptr(wt), ptr(at), ptr(ct), n, bpr, m, None))
    C = host(ct).reshape(m, n)
    C_ref, A = orc.gemm_f16(w, a.view(np.uint16), n, bpr)
    k = bpr * 256
    assert np.all(np.abs(C - C_ref) <= 1e-2 * A / np.sqrt(k))
    assert np.linalg.norm(C - C_ref) <= 1e-3 * np.linalg.norm(C_ref)


# Random-byte blocks across the f16 range of d/dmin: tiny (f16 subnormal d,
# weights ~1e-4), huge (weights up to ~6e7, past f16's 65504), ten decades
# mixed inside one row, eight decades rising along every row (each block
# larger than the one before), and raw random header bytes (Inf/NaN d read
# as 0).
def _range_weight(rng, n, bpr, kind):
    nb = n * bpr
    if kind == "random":
        return random_q4k_bytes(rng, nb, finite_scales=False)
    b = rng.integers(0, 256, size=(nb, 144), dtype=np.uint8)
    if kind == "tiny":
        d = rng.uniform(1e-8, 3e-6, size=(nb, 2))
    elif kind == "huge":
        d = rng.uniform(1e2, 6e4, size=(nb, 2))
    elif kind == "rising":
        j = np.tile(np.arange(bpr), n)[:, None] + rng.uniform(0, 1, size=(nb, 2))
        d = 10.0 ** (-7 + 8 * j / bpr)
    else:  # mixed
        d = 10.0 ** rng.uniform(-7, 1, size=(nb, 2))
    b[:, 0:4] = d.astype(np.float16).view(np.uint8).reshape(nb, 4)
    return b.ravel()


def _gemm_check(L, orc, w, a, n, bpr, m, rows=None):
    wt, at, ct = dev(w), dev(a.view(np.uint16)), empty_f32(m * n)
    _lib.check("gemm", L.launch_gemm_q4k_f16(ptr(wt), ptr(at), ptr(ct), n, bpr, m, None))
    C = host(ct).reshape(m, n).astype(np.float64)
    assert np.all(np.isfinite(C))
    C_ref, A = orc.gemm_f16(w, a.view(np.uint16), n, bpr, rows=rows)
    if rows is not None:
        C = C[:, rows]
    k = bpr * 256
    assert np.all(np.abs(C - C_ref) <= 1e-2 * A / np.sqrt(k))
    assert np.linalg.norm(C - C_ref) <= 1e-3 * np.linalg.norm(C_ref)


# (200, 40): the 128-token kernel; (32000, 256): 200 tiles of 160 x 256, the
# LDS-dequant kernel, one block per row; (20000, 512): the LDS-dequant kernel
# with 14 blocks per row, where a row's scale follows its blocks (rows
# sampled on the large shapes)
@pytest.mark.parametrize("n,m", [(200, 40), (32000, 256), (20000, 512)])
@pytest.mark.parametrize("kind", ["tiny", "huge", "mixed", "rising", "random"])
def test_gemm_f16_dynamic_range(L, orc, kind, n, m):
    bpr = {200: 4, 32000: 1, 20000: 14}[n]
    note(f"gemm range {kind} n={n} bpr={bpr} m={m}")
    rng = np.random.default_rng(0x6E11 + m)
    w = _range_weight(rng, n, bpr, kind)
    a = rng.normal(0, 1, size=(m, bpr * 256)).astype(np.float16)
    rows = None if n < 1000 else np.sort(rng.choice(n, size=192, replace=False)).astype(np.int32)
    _gemm_check(L, orc, w, a, n, bpr, m, rows)


# The 128-token kernel at its 160-row tile height with several super-blocks
# (the raw-W LDS refill across super-blocks) and several token tiles:
# (70000, 3, 16) and the config-5 weight at M = 256 (rows sampled)
@pytest.mark.parametrize("n,bpr,m", [(70000, 3, 16), (18944, 14, 256)])
def test_gemm_160_row_tiles_multi_block(L, orc, n, bpr, m):
    note(f"gemm 160-row tiles n={n} bpr={bpr} m={m}")
    rng = np.random.default_rng(n + bpr + m)
    w = orc.seeded_weight(0x160 + bpr, n, bpr * 256)
    a = orc.normal(0xF18 + m, m * bpr * 256).astype(np.float16).reshape(m, -1)
    rows = np.unique(np.concatenate([rng.choice(n, size=160, replace=False),
                                     np.arange(n - 32, n)])).astype(np.int32)
    _gemm_check(L, orc, w, a, n, bpr, m, rows)


# Shapes the LDS-dequant kernel takes (one round of 160 x 256 tiles more than
# half full, or several rounds at least 85 % full): full token tiles, ragged
# tokens, ragged rows, several super-blocks; two rounds (476 tiles) with full
# and with ragged token tiles
@pytest.mark.parametrize("n,bpr,m", [(32000, 1, 256), (30000, 3, 250), (20000, 14, 512),
                                     (18944, 2, 1024), (18944, 2, 1000)])
def test_gemm_lds_kernel_shapes(L, orc, n, bpr, m):
    note(f"gemm lds kernel n={n} bpr={bpr} m={m}")
    rng = np.random.default_rng(n + m)
    w = orc.seeded_weight(n + bpr, n, bpr * 256)
    a = orc.normal(0xF17 + m, m * bpr * 256).astype(np.float16).reshape(m, -1)
    rows = np.sort(np.concatenate([rng.choice(n - 160, size=120, replace=False),
                                   np.arange(n - 40, n)])).astype(np.int32)
    _gemm_check(L, orc, w, a, n, bpr, m, np.unique(rows))


# -------------------------------------------------------------------- chain --
def test_chain_replays_the_recorded_matvecs(L, orc):
    note("chain of 3 matvecs")
    from modgrad_amd.q4k import Chain
    shapes = [(256, 14), (64, 74), (512, 14)]
    bufs, descs, refs = [], [], []
    for i, (n, bpr) in enumerate(shapes):
        w = orc.seeded_weight(70 + i, n, bpr * 256)
        x = orc.normal(80 + i, bpr * 256)
        wt, xt, yt = dev(w), dev(x), empty_f32(n)
        bufs += [wt, xt, yt]
        descs.append((ptr(wt), ptr(xt), ptr(yt), n, bpr))
        refs.append(orc.gemv(w, x, n, bpr))
    ch = Chain(descs)
    for rep in range(3):
        for t in bufs[2::3]:
            t.fill_(float("nan"))
        ch.launch()
        for (y_ref, a), yt in zip(refs, bufs[2::3]):
            assert_gemv_close(host(yt), y_ref, a)
    ch.close()


# ---------------------------------------------- LinearResidentQuantized ------
def test_linear_resident_quantized_forward_and_evict(L, orc):
    # neuron.rs:1944-1994 (evict_then_redequant: bit-identical re-dequant)
    note("LinearResidentQuantized 896->4864 flat")
    from modgrad_amd.q4k import HipBuffer, LinearResidentQuantized
    in_dim, out_dim = 896, 4864
    w = orc.seeded_weight(0xCAFEBABE, out_dim, in_dim)
    bias = orc.normal(0xC0FFEEFE, out_dim, 0.1)
    lin = LinearResidentQuantized.from_q4k(w, bias, in_dim, out_dim)
    x = orc.normal(3, in_dim)
    xb, yb = HipBuffer(in_dim * 4), HipBuffer(out_dim * 4)
    xb.copy_from_host(x)
    lin.forward(xb, yb)
    y = yb.copy_to_host(out_dim)
    y_ref, a = orc.gemv_flat(w, x, out_dim, in_dim)
    assert_gemv_close(y - bias, y_ref, a + 1e-30)
    first = lin.weight_dev.copy_to_host()
    assert np.array_equal(first.view(np.uint32), orc.dequantize(w).view(np.uint32))
    lin.evict()
    assert not lin.is_resident()
    lin.ensure_resident()
    assert np.array_equal(lin.weight_dev.copy_to_host().view(np.uint32), first.view(np.uint32))


def test_linear_forward_takes_hip_gpuvecs(L, orc):
    # neuron.rs:1059-1108 with GpuVec::Hip operands: out = fl(W x + b), the bias
    # added after the product in one rounding, as hipblasSgemv's beta = 1 on a
    # bias-filled y (rocm.rs:2000-2056)
    note("LinearResidentQuantized.forward on Hip GpuVecs 1024->512")
    from modgrad_amd import _lib as lib
    from modgrad_amd.q4k import GpuVec, HipBuffer, LinearResidentQuantized, kern
    in_dim, out_dim = 1024, 512
    w = orc.seeded_weight(0xB1A5, out_dim, in_dim)
    bias = orc.normal(0xB1A6, out_dim, 0.3)
    lin = LinearResidentQuantized.from_q4k(w, bias, in_dim, out_dim)
    xv, yv = GpuVec.try_hip(in_dim), GpuVec.try_hip(out_dim)
    assert xv.variant_name() == "Hip" and not xv.is_host_visible() and len(yv) == out_dim
    x = orc.normal(0xB1A7, in_dim)
    xv.copy_from(x)
    lin.forward(xv, yv)
    y = yv.copy_to_host()
    plain = HipBuffer(out_dim * 4)
    kern.matvec_q4k_ex(lin.weight_q4k_dev.device_ptr(), xv.hip_buffer().device_ptr(),
                       plain.device_ptr(), out_dim, in_dim, lib.LAYOUT_FLAT)
    y0 = plain.copy_to_host()
    assert np.array_equal(y.view(np.uint32), (y0 + bias).view(np.uint32))
    y_ref, a = orc.gemv_flat(w, x, out_dim, in_dim)
    assert_gemv_close(y0, y_ref, a + 1e-30)
    assert yv.clone().variant_name() == "Heap"
    with pytest.raises(Exception):
        yv.as_slice()  # Hip memory is not host-visible (backend.rs:139-151)
    # with a HipBatch (neuron.rs:1059-1108): every queued kernel counts and the
    # batch drains at its cadence; the result is unchanged
    from modgrad_amd.q4k import HipBatch
    batch = HipBatch.with_sync_every(3)
    lin.evict()
    lin.ensure_resident(batch)       # dequant: 1
    assert batch.pending == 1
    lin.forward(xv, yv, batch=batch)  # matvec + bias add: 3 -> drained
    assert batch.pending == 0
    assert np.array_equal(yv.copy_to_host().view(np.uint32), y.view(np.uint32))
    batch.flush()


def test_hipbuffer_range_copies_and_q5k(L, orc):
    # rocm.rs:791-837 copy_range_from, rocm.rs:917-934 copy_from_host_bytes_at,
    # rocm.rs:743-776 matvec_q5k / matvec_q5k_into
    note("HipBuffer copy_range_from / copy_from_host_bytes_at / matvec_q5k")
    from modgrad_amd.q4k import BackendError, HipBuffer, kern
    a = HipBuffer(64 * 4)
    a.copy_from_host(np.arange(64, dtype=np.float32))
    b = HipBuffer(32 * 4)
    b.copy_from_host(np.full(32, -1.0, np.float32))
    b.copy_range_from(a, 10, 4, 20)
    got = b.copy_to_host()
    assert got[:4].tolist() == [-1.0] * 4 and got[24:].tolist() == [-1.0] * 8
    assert got[4:24].tolist() == list(range(10, 30))
    with pytest.raises(BackendError):
        b.copy_range_from(a, 50, 0, 20)   # past the end of src
    with pytest.raises(BackendError):
        b.copy_range_from(a, 0, 20, 20)   # past the end of dst
    with pytest.raises(BackendError):
        b.copy_to_host(33)
    arena = HipBuffer(256)
    arena.copy_from_host_bytes_at(100, np.arange(50, dtype=np.uint8))
    assert np.array_equal(arena.tensor()[100:150].cpu().numpy(), np.arange(50, dtype=np.uint8))
    with pytest.raises(BackendError):
        arena.copy_from_host_bytes_at(250, np.zeros(7, np.uint8))
    free, total = kern.vram_free_total()
    assert 0 < free <= total
    from tests.gpu_util import random_kquant_bytes
    n, bpr = 96, 3
    w5 = random_kquant_bytes(np.random.default_rng(0x55), n * bpr, 176)
    wb = HipBuffer(w5.size)
    wb.copy_from_host_bytes(w5)
    x = orc.normal(0x56, bpr * 256)
    y = wb.matvec_q5k(x, n, bpr)
    y_ref, aa = orc.gemv_kquant(176, w5, x, n, bpr)
    assert_gemv_close(y, y_ref, aa)


def test_hipbuffer_matvec_q4k_host_roundtrip(L, orc):
    # rocm.rs:681-709 path (host x in, host y out)
    note("HipBuffer.matvec_q4k")
    from modgrad_amd.q4k import HipBuffer
    n, bpr = 300, 15
    w = orc.seeded_weight(90, n, bpr * 256)
    wb = HipBuffer(w.size)
    wb.copy_from_host_bytes(w)
    x = (np.sin(np.arange(bpr * 256, dtype=np.float32) * np.float32(0.37)) * np.float32(180.0)
         + (np.arange(bpr * 256) * 7 % 13).astype(np.float32)).astype(np.float32)
    y = wb.matvec_q4k(x, n, bpr)
    y_ref, a = orc.gemv(w, x, n, bpr)
    assert_gemv_close(y, y_ref, a)
    assert np.max(np.abs(y - y_ref)) < 0.02  # rocm_matvec_check.rs:49-54 gate


# ------------------------------------------------------- dp4a / Q8_1 path --
def run_q8(L, x: np.ndarray, off: int = 0):
    """launch_quantize_q8_1 on x (device copy at byte offset `off`)."""
    n = x.size
    xt = dev(np.concatenate([np.zeros(off // 4, np.float32), x]))
    nsub = n // 32
    xq, xd, xs = filled_u8(nsub * 32 + 64, 0x5A), empty_f32(nsub + 4), empty_f32(nsub + 4)
    _lib.check("quantize_q8_1", L.launch_quantize_q8_1(ptr(xt) + off, ptr(xq), ptr(xd), ptr(xs), n))
    return (xq, xd, xs), (host(xq)[:nsub * 32].view(np.int8), host(xd)[:nsub], host(xs)[:nsub])


def test_quantize_q8_1_bit_exact(L, orc):
    note("quantize_q8_1 bit-exact")
    rng = np.random.default_rng(91)
    x = (rng.standard_normal(32 * 600) * rng.choice([1e-6, 1e-2, 1.0, 300.0], size=32 * 600))
    x = x.astype(np.float32)
    x[0:32] = 0.0
    x[32:64] = np.float32(1e-40)          # 127/amax overflows: zero sub-block
    x[64:96] = np.float32(3.0e38)
    x[96:128] = (np.arange(32, dtype=np.float32) - 16) * np.float32(0.5)
    x[128:160] = np.float32(7.0)
    x[160] = np.float32(127.0)
    x[161:166] = [0.5, 1.5, 2.5, -0.5, -2.5]  # halves: round to even
    for off in (0, 4):                    # 16-byte aligned and 4-byte aligned input
        _, (q, d, s) = run_q8(L, x, off)
        rq, rd, rs = orc.quantize_q8_1(x)
        assert np.array_equal(q, rq)
        assert np.array_equal(d.view(np.uint32), rd.view(np.uint32))
        assert np.array_equal(s, rs)


def assert_dp4a_close(y, y_ref, absterm, tol=1e-5):
    """Same formula in f32 (kernel) and f64 (oracle): only rounding differs."""
    err = np.abs(y.astype(np.float64) - y_ref)
    bad = np.nonzero(~(err <= tol * absterm + 1e-30))[0]
    assert bad.size == 0, (bad[:5].tolist(), err[bad[:5]].tolist(), absterm[bad[:5]].tolist())


@pytest.mark.parametrize("n,bpr", [(1, 1), (17, 3), (64, 14), (3584, 14), (700, 74), (4100, 17),
                                   (30000, 14), (300, 100), (4608, 14), (6000, 5),
                                   (20005, 13), (701, 75)])
def test_dp4a_matvec_matches_oracle(L, orc, n, bpr):
    # shapes that take each launch configuration of the matrix-core kernel's
    # Q8 mode (few/many row groups, one/several stages, fallback to
    # single-buffered stages)
    note(f"dp4a n={n} bpr={bpr}")
    rng = np.random.default_rng(n * 7 + bpr)
    w = random_q4k_bytes(rng, n * bpr)
    x = rng.standard_normal(bpr * 256).astype(np.float32)
    (xq, xd, xs), (q, d, s) = run_q8(L, x)
    wt, yt = dev(w), empty_f32(n)
    _lib.check("dp4a", L.launch_matvec_q4k_dp4a(ptr(wt), ptr(xq), ptr(xd), ptr(xs), ptr(yt), n, bpr))
    y_ref, absterm = orc.gemv_dp4a(w, q, d, s, n, bpr)
    assert_dp4a_close(host(yt), y_ref, absterm)


def test_dp4a_vector_alu_fallback_matches_oracle(L, orc):
    # K = 102400: the Q8 activation staging exceeds the matrix-core kernel's
    # per-lane item count, so the vector-ALU dp4a kernel runs; xq at a 4-byte
    # offset
    note("dp4a vector-ALU kernel (bpr 400, xq offset 4)")
    n, bpr = 8, 400
    rng = np.random.default_rng(93)
    w = random_q4k_bytes(rng, n * bpr)
    x = rng.standard_normal(bpr * 256).astype(np.float32)
    q, d, s = orc.quantize_q8_1(x)
    xq = dev(np.concatenate([np.zeros(4, np.int8), q]))
    xdt, xst, wt, yt = dev(d), dev(s), dev(w), empty_f32(n)
    _lib.check("dp4a", L.launch_matvec_q4k_dp4a(ptr(wt), ptr(xq) + 4, ptr(xdt), ptr(xst), ptr(yt), n, bpr))
    y_ref, absterm = orc.gemv_dp4a(w, q, d, s, n, bpr)
    assert_dp4a_close(host(yt), y_ref, absterm)


@pytest.mark.parametrize("bias", [0.0, 100.0])
def test_dp4a_reference_acceptance_check(L, orc, bias):
    # examples/rocm_dp4a_check.rs:31-63: x = sin(0.21 i)*30 + bias,
    # RMS_rel(dp4a GPU - f64 dequant-dot) < 0.02, on a seeded 7B shape
    note(f"dp4a acceptance bias={bias}")
    n, bpr = 3584, 14
    w = orc.seeded_weight(orc.layer_seed(0, 0), n, bpr * 256)
    x = (np.sin(np.arange(bpr * 256, dtype=np.float32) * np.float32(0.21)) * np.float32(30.0)
         + np.float32(bias)).astype(np.float32)
    (xq, xd, xs), _ = run_q8(L, x)
    wt, yt = dev(w), empty_f32(n)
    _lib.check("dp4a", L.launch_matvec_q4k_dp4a(ptr(wt), ptr(xq), ptr(xd), ptr(xs), ptr(yt), n, bpr))
    y_ref, _ = orc.gemv(w, x, n, bpr)
    y = host(yt).astype(np.float64)
    rms_rel = np.sqrt(np.sum((y - y_ref) ** 2) / np.sum(y_ref.astype(np.float64) ** 2))
    assert rms_rel < 0.02


@pytest.mark.parametrize("n,bpr", [(1, 1), (64, 2), (300, 3), (3584, 14), (4608, 14),
                                   (600, 74), (5000, 74)])
def test_fused_quantize_dp4a_is_the_two_launch_sequence(L, orc, n, bpr):
    # launch_quantize_matvec_q4k_dp4a_ex == launch_quantize_q8_1 followed by
    # launch_matvec_q4k_dp4a, bit for bit, including the quantizer's special
    # sub-blocks (zero, denormal max, huge, NaN / Inf, exact halves)
    note(f"fused quantize+dp4a n={n} bpr={bpr}")
    k = bpr * 256
    rng = np.random.default_rng(n * 7 + bpr)
    w = random_q4k_bytes(rng, n * bpr)
    x = (rng.standard_normal(k) * rng.choice([1e-6, 1e-2, 1.0, 300.0], size=k)).astype(np.float32)
    x[0:32] = 0.0
    if k >= 256:
        x[32:64] = np.float32(1e-40)
        x[64:96] = np.float32(3.0e38)
        x[96:128] = (np.arange(32, dtype=np.float32) - 16) * np.float32(0.5)
        x[130] = np.float32("nan")
        x[200] = np.float32("inf")
    wt, xt = dev(w), dev(x)
    (xq, xd, xs), _ = run_q8(L, x)
    y_two = empty_f32(n)
    _lib.check("dp4a", L.launch_matvec_q4k_dp4a(ptr(wt), ptr(xq), ptr(xd), ptr(xs), ptr(y_two), n, bpr))
    y_one = empty_f32(n)
    _lib.check("fused", L.launch_quantize_matvec_q4k_dp4a_ex(ptr(wt), ptr(xt), ptr(y_one), n, bpr, None))
    a, b = host(y_two), host(y_one)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_dp4a_nonfinite_rows_are_zero(L, orc):
    # an Inf activation gives xd = Inf and a non-finite row sum: written as 0
    note("dp4a non-finite clamp")
    n, bpr = 40, 2
    w = orc.seeded_weight(94, n, bpr * 256)
    x = orc.normal(95, bpr * 256)
    x[3] = np.inf
    (xq, xd, xs), (q, d, s) = run_q8(L, x)
    wt, yt = dev(w), empty_f32(n)
    _lib.check("dp4a", L.launch_matvec_q4k_dp4a(ptr(wt), ptr(xq), ptr(xd), ptr(xs), ptr(yt), n, bpr))
    y_ref, absterm = orc.gemv_dp4a(w, q, d, s, n, bpr)
    y = host(yt)
    assert np.all(np.isfinite(y))
    assert np.array_equal(y == 0, y_ref == 0)


# ------------------------------------------------------------ Q5_K / Q6_K --
@pytest.mark.parametrize("fmt", [176, 210])
@pytest.mark.parametrize("n,bpr", [(1, 1), (5, 3), (64, 14), (3584, 14), (300, 74), (4099, 2),
                                   (7, 15), (33, 29), (20000, 14), (9001, 3), (8, 1), (40, 1),
                                   (24, 3), (136, 7), (1000, 14), (4096, 2),
                                   # Q6_K K-chunked stages: chunk remainders, odd bpr (2-byte
                                   # aligned rows), a partial last group, 2 rounds, 8 items/thread
                                   (16, 15), (48, 29), (520, 43), (9600, 16), (3584, 74),
                                   (232, 101),
                                   # one row group per CU (Q5_K: 17..24-row groups)
                                   (4608, 14), (6000, 7)])
def test_kquant_matvec_matches_oracle(L, orc, fmt, n, bpr):
    from tests.gpu_util import random_kquant_bytes
    note(f"{'q5k' if fmt == 176 else 'q6k'} n={n} bpr={bpr}")
    rng = np.random.default_rng(fmt * 1000 + n + bpr)
    w = random_kquant_bytes(rng, n * bpr, fmt)
    x = rng.standard_normal(bpr * 256).astype(np.float32)
    wt, xt, yt = dev(w), dev(x), empty_f32(n)
    fn = L.launch_matvec_q5k if fmt == 176 else L.launch_matvec_q6k
    _lib.check("kquant", fn(ptr(wt), ptr(xt), ptr(yt), n, bpr))
    y_ref, a = orc.gemv_kquant(fmt, w, x, n, bpr)
    assert_gemv_close(host(yt), y_ref, a)


def test_q5k_matvec_long_rows_use_the_vector_alu_kernel(L, orc):
    # K = 37888 exceeds the matrix-core kernel's activation staging: the
    # byte-reading vector-ALU Q5_K kernel runs (weights at a 4-byte offset)
    from tests.gpu_util import random_kquant_bytes
    note("q5k vector-ALU kernel (bpr 148, w offset 4)")
    n, bpr = 10, 148
    w = random_kquant_bytes(np.random.default_rng(8), n * bpr, 176)
    x = np.random.default_rng(9).standard_normal(bpr * 256).astype(np.float32)
    import torch
    wt = torch.zeros(w.size + 64, dtype=torch.uint8, device="cuda")
    wt[4:4 + w.size].copy_(torch.from_numpy(w))
    xt, yt = dev(x), empty_f32(n)
    _lib.check("q5k", L.launch_matvec_q5k(ptr(wt) + 4, ptr(xt), ptr(yt), n, bpr))
    y_ref, a = orc.gemv_kquant(176, w, x, n, bpr)
    assert_gemv_close(host(yt), y_ref, a)


def test_kquant_matvec_odd_weight_offset(L, orc):
    # the reference arena places tensors at arbitrary offsets: Q6_K weights
    # starting 2 bytes past an allocation boundary
    from tests.gpu_util import random_kquant_bytes
    note("q6k weights at an odd offset")
    n, bpr = 33, 5
    w = random_kquant_bytes(np.random.default_rng(7), n * bpr, 210)
    x = orc.normal(8, bpr * 256)
    wt = dev(np.concatenate([np.zeros(2, np.uint8), w]))
    xt, yt = dev(x), empty_f32(n)
    _lib.check("q6k", L.launch_matvec_q6k(ptr(wt) + 2, ptr(xt), ptr(yt), n, bpr))
    y_ref, a = orc.gemv_kquant(210, w, x, n, bpr)
    assert_gemv_close(host(yt), y_ref, a)


@pytest.mark.parametrize("n,bpr", [(1, 1), (40, 14), (3584, 14), (129, 74)])
def test_q6k_dp4a_matches_oracle(L, orc, n, bpr):
    from tests.gpu_util import random_kquant_bytes
    note(f"q6k dp4a n={n} bpr={bpr}")
    rng = np.random.default_rng(n + 17 * bpr)
    w = random_kquant_bytes(rng, n * bpr, 210)
    x = rng.standard_normal(bpr * 256).astype(np.float32)
    (xq, xd, xs), (q, d, s) = run_q8(L, x)
    wt, yt = dev(w), empty_f32(n)
    _lib.check("q6k dp4a", L.launch_matvec_q6k_dp4a(ptr(wt), ptr(xq), ptr(xd), ptr(xs), ptr(yt), n, bpr))
    y_ref, absterm = orc.gemv_q6k_dp4a(w, q, d, n, bpr)
    assert_dp4a_close(host(yt), y_ref, absterm)
