"""GGUF file -> one-allocation weight arena -> matvecs dispatched by each
tensor's quantization type (rocm_gemma.rs:210-224, 303-330), on the GPU,
against the CPU oracle. The model file is written by modgrad_amd.gguf's
writer: a Q4_K_M-style mix (Q4_K projections, Q6_K attn_v / ffn_down /
output, a Q5_K tensor, F32 norms)."""
import sys

import numpy as np
import pytest

from modgrad_amd import gguf
from modgrad_amd.gguf import GgmlType
from tests.gpu_util import assert_gemv_close, dev, empty_f32, host, random_kquant_bytes

pytestmark = pytest.mark.gpu

D, FF, VOCAB = 512, 768, 1000


def note(msg: str) -> None:
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def model(tmp_path_factory, orc):
    rng = np.random.default_rng(42)
    t = []

    def q4(name, n, k, seed):
        t.append((name, [k, n], int(GgmlType.Q4_K), orc.seeded_weight(seed, n, k).tobytes()))

    def kq(name, n, k, fmt):
        nb = 176 if fmt == GgmlType.Q5_K else 210
        t.append((name, [k, n], int(fmt), random_kquant_bytes(rng, n * (k // 256), nb).tobytes()))

    def f32(name, n):
        t.append((name, [n], int(GgmlType.F32), (rng.random(n, dtype=np.float32) + 0.5).tobytes()))

    f32("blk.0.attn_norm.weight", D)
    q4("blk.0.attn_q.weight", D, D, 1)
    kq("blk.0.attn_v.weight", 128, D, GgmlType.Q6_K)      # 256 Q6_K blocks: 2-B multiple
    q4("blk.0.attn_k.weight", 128, D, 2)
    f32("blk.0.ffn_norm.weight", D)
    q4("blk.0.ffn_gate.weight", FF, D, 3)
    q4("blk.0.ffn_up.weight", FF, D, 4)
    kq("blk.0.ffn_down.weight", D, FF, GgmlType.Q6_K)
    kq("blk.1.ffn_down.weight", D, FF, GgmlType.Q5_K)
    kq("output.weight", VOCAB, D, GgmlType.Q6_K)
    meta = [("general.architecture", gguf.STRING, "llama"),
            ("llama.embedding_length", gguf.U32, D),
            ("llama.feed_forward_length", gguf.U32, FF),
            ("llama.attention.layer_norm_rms_epsilon", gguf.F32, 1e-5)]
    path = str(tmp_path_factory.mktemp("gguf") / "mix.gguf")
    gguf.write_gguf(path, meta, t)
    g = gguf.GgufFile.open(path)
    from modgrad_amd.arena import WeightArena
    arena = WeightArena.from_gguf(g)
    yield g, arena, {name: np.frombuffer(data, np.uint8) for name, _, _, data in t}
    g.close()


def test_arena_holds_the_file_bytes_aligned(model):
    note("arena bytes and alignment")
    g, arena, raw = model
    for name in g.tensor_list:
        assert arena.ptr(name) % 256 == 0
        assert np.array_equal(host(arena.tensor(name)), raw[name])


@pytest.mark.parametrize("name", ["blk.0.attn_q.weight", "blk.0.attn_v.weight",
                                  "blk.0.attn_k.weight", "blk.0.ffn_down.weight",
                                  "blk.1.ffn_down.weight", "output.weight"])
def test_qmatvec_dispatches_by_dtype(model, orc, name):
    g, arena, raw = model
    n, k = arena.shape(name)
    t = arena.dtype[name]
    note(f"qmatvec {name} {t.name} {n}x{k}")
    x = orc.normal(len(name), k)
    xt, yt = dev(x), empty_f32(n)
    arena.qmatvec(name, xt.data_ptr(), yt.data_ptr())
    y = host(yt)
    if t == GgmlType.Q4_K:
        y_ref, a = orc.gemv(raw[name], x, n, k // 256)
    else:
        y_ref, a = orc.gemv_kquant(176 if t == GgmlType.Q5_K else 210, raw[name], x, n, k // 256)
    assert_gemv_close(y, y_ref, a)


def test_qmatvec_dp4a_arm(model, orc):
    note("qmatvec Q4_K through quantize_q8_1 + dp4a")
    import torch
    g, arena, raw = model
    name = "blk.0.ffn_gate.weight"
    n, k = arena.shape(name)
    x = orc.normal(77, k)
    xt, yt = dev(x), empty_f32(n)
    q8 = (torch.empty(k, dtype=torch.int8, device="cuda"), torch.empty(k // 32, device="cuda"),
          torch.empty(k // 32, device="cuda"))
    arena.qmatvec(name, xt.data_ptr(), yt.data_ptr(), q8=tuple(b.data_ptr() for b in q8))
    y = host(yt).astype(np.float64)
    xq, xd, xs = orc.quantize_q8_1(x)
    y_ref, a = orc.gemv_dp4a(raw[name], xq, xd, xs, n, k // 256)
    assert np.all(np.abs(y - y_ref) <= 1e-5 * a + 1e-30)


def test_fused_glue_from_the_arena(model, orc):
    note("arena rmsnorm+matvec and gate/up glu")
    g, arena, raw = model
    eps = g.meta_f32("llama.attention.layer_norm_rms_epsilon")
    x = orc.normal(5, D)
    xt = dev(x)
    nw = np.frombuffer(raw["blk.0.attn_norm.weight"], np.float32)
    yt = empty_f32(D)
    arena.qmatvec_rmsnorm("blk.0.attn_q.weight", xt.data_ptr(), "blk.0.attn_norm.weight", eps,
                          yt.data_ptr())
    xn = orc.rms_norm(x, nw, 1, D, eps)
    y_ref, a = orc.gemv(raw["blk.0.attn_q.weight"], xn, D, D // 256)
    assert_gemv_close(host(yt), y_ref, a)
    ot = empty_f32(FF)
    arena.qmatvec_glu("blk.0.ffn_gate.weight", "blk.0.ffn_up.weight", xt.data_ptr(),
                      ot.data_ptr(), norm="blk.0.ffn_norm.weight", eps=eps)
    nf = np.frombuffer(raw["blk.0.ffn_norm.weight"], np.float32)
    xn = orc.rms_norm(x, nf, 1, D, eps)
    gg, ag = orc.gemv(raw["blk.0.ffn_gate.weight"], xn, FF, D // 256)
    uu, au = orc.gemv(raw["blk.0.ffn_up.weight"], xn, FF, D // 256)
    g64, u64 = gg.astype(np.float64), uu.astype(np.float64)
    act = 0.5 * g64 * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (g64 + 0.044715 * g64 ** 3)))
    bound = 1e-4 * (1.13 * ag * np.abs(u64) + np.abs(act) * au) + 1e-5 * np.abs(act * u64)
    assert np.all(np.abs(host(ot) - act * u64) <= bound)


def test_unsupported_types_are_refused(model):
    g, arena, raw = model
    from modgrad_amd.q4k import BackendError
    with pytest.raises(BackendError):
        arena.qmatvec("blk.0.attn_norm.weight", 0, 0)          # F32: not a matrix
    with pytest.raises(BackendError):
        arena.qmatvec_rmsnorm("blk.0.attn_v.weight", 0, "blk.0.attn_norm.weight", 1e-5, 0)
