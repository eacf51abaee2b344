"""GGUF container (modgrad_amd.gguf) and arena planning, CPU only.

The parser follows crates/modgrad-device/src/kfd/gguf.rs:153-244, 665-694.
The reference holds no GGUF fixture, so the parser is pinned by bytes this
test assembles field by field from the GGUF v3 layout (independently of
modgrad_amd.gguf.write_gguf), by its error cases, and by a writer round trip.
"""
import io
import struct

import numpy as np
import pytest

from modgrad_amd import gguf
from modgrad_amd.arena import plan_offsets
from modgrad_amd.gguf import GgmlType, GgufError, GgufFile


def s(txt: str) -> bytes:
    b = txt.encode()
    return struct.pack("<Q", len(b)) + b


def hand_built() -> bytes:
    """GGUF v3: 4 KV pairs and 2 tensors, data section at the next 32 B."""
    out = b"GGUF" + struct.pack("<IQQ", 3, 2, 4)
    out += s("general.architecture") + struct.pack("<I", 8) + s("llama")
    out += s("llama.block_count") + struct.pack("<II", 4, 28)
    out += s("llama.attention.layer_norm_rms_epsilon") + struct.pack("<If", 6, 1e-6)
    out += s("flags") + struct.pack("<IIQ", 9, 7, 3) + bytes([1, 0, 1])
    out += s("blk.0.attn_q.weight") + struct.pack("<I", 2) + struct.pack("<QQ", 512, 64)
    out += struct.pack("<IQ", 12, 0)                       # Q4_K at data + 0
    out += s("blk.0.attn_norm.weight") + struct.pack("<I", 1) + struct.pack("<Q", 512)
    out += struct.pack("<IQ", 0, 64 * 2 * 144)            # F32 after it
    hdr = len(out)
    pad = (hdr + 31) // 32 * 32 - hdr
    return out + b"\0" * pad + bytes(range(256)) * 80


def test_parses_hand_built_file():
    raw = hand_built()
    g = GgufFile.parse(io.BytesIO(raw))
    assert g.version == 3
    assert g.architecture() == "llama"
    assert g.meta_u32("llama.block_count") == 28
    assert g.meta_f32("llama.attention.layer_norm_rms_epsilon") == np.float32(1e-6)
    assert g.meta("flags").as_bool_array() == [True, False, True]
    assert g.tensor_list == ["blk.0.attn_q.weight", "blk.0.attn_norm.weight"]
    q = g.tensors["blk.0.attn_q.weight"]
    assert q.dims == [512, 64] and q.dtype == GgmlType.Q4_K and q.offset == 0
    assert q.n_elements() == 512 * 64 and q.data_bytes() == 64 * 2 * 144
    nw = g.tensors["blk.0.attn_norm.weight"]
    assert nw.dtype == GgmlType.F32 and nw.data_bytes() == 2048
    assert g.data_offset % 32 == 0 and 0 <= g.data_offset - (len(raw) - 256 * 80) < 32
    assert g.tensor_file_offset("blk.0.attn_norm.weight") == g.data_offset + 64 * 2 * 144
    assert g.tensor_file_offset("missing") is None and g.meta_u32("missing") is None


@pytest.mark.parametrize("mutate,msg", [
    (lambda b: b"GGUX" + b[4:], "not a GGUF file"),
    (lambda b: b[:4] + struct.pack("<I", 1) + b[8:], "unsupported GGUF version 1"),
    (lambda b: b[:4] + struct.pack("<I", 4) + b[8:], "unsupported GGUF version 4"),
    (lambda b: b[:60], "failed to fill whole buffer"),
])
def test_rejects_malformed_headers(mutate, msg):
    with pytest.raises(GgufError, match=msg):
        GgufFile.parse(io.BytesIO(mutate(hand_built())))


def test_rejects_unknown_value_type_and_long_strings():
    bad = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + s("k") + struct.pack("<I", 13)
    with pytest.raises(GgufError, match="unknown GGUF value type 13"):
        GgufFile.parse(io.BytesIO(bad))
    long = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1_000_001)
    with pytest.raises(GgufError, match="string too long"):
        GgufFile.parse(io.BytesIO(long))


def test_version_2_and_unknown_tensor_type():
    b = bytearray(hand_built())
    b[4:8] = struct.pack("<I", 2)
    i = bytes(b).index(s("blk.0.attn_norm.weight")) + len(s("blk.0.attn_norm.weight")) + 12
    b[i:i + 4] = struct.pack("<I", 99)  # type id of the second tensor
    g = GgufFile.parse(io.BytesIO(bytes(b)))
    t = g.tensors["blk.0.attn_norm.weight"]
    assert g.version == 2 and t.dtype == GgmlType.UNKNOWN and t.dtype_id == 99
    assert t.data_bytes() == 0  # (0, 1) block size, as the reference's Unknown


def test_meta_value_casts():
    M = gguf.MetaValue
    assert M(gguf.I32, -1).as_u32() == 0xFFFFFFFF
    assert M(gguf.U64, 5).as_u32() == 5 and M(gguf.F32, 1.0).as_u32() is None
    assert M(gguf.F64, 0.1).as_f32() == np.float32(0.1)
    assert M(gguf.STRING, "x").as_str() == "x" and M(gguf.U8, 1).as_str() is None


@pytest.mark.parametrize("t,n,nbytes", [
    (GgmlType.Q4_K, 256, 144), (GgmlType.Q4_K, 257, 288), (GgmlType.Q5_K, 512, 352),
    (GgmlType.Q6_K, 256 * 3, 630), (GgmlType.Q8_0, 64, 68), (GgmlType.F32, 10, 40),
    (GgmlType.F16, 10, 20), (GgmlType.Q2_K, 256, 84), (GgmlType.Q8_K, 256, 292)])
def test_data_sizes(t, n, nbytes):
    assert gguf.data_size(t, n) == nbytes


def test_writer_round_trip(tmp_path):
    rng = np.random.default_rng(0)
    tens = [("a.weight", [512, 3], 12, rng.integers(0, 256, 3 * 2 * 144, dtype=np.uint8).tobytes()),
            ("b.weight", [256, 5], 14, rng.integers(0, 256, 5 * 210, dtype=np.uint8).tobytes()),
            ("c.weight", [7], 0, np.arange(7, dtype=np.float32).tobytes())]
    meta = [("general.architecture", gguf.STRING, "qwen2"),
            ("qwen2.context_length", gguf.U64, 32768),
            ("neg", gguf.I64, -3), ("pi", gguf.F64, 3.25), ("b", gguf.BOOL, True),
            ("toks", gguf.ARRAY, (gguf.STRING, ["<s>", "é", ""])),
            ("ids", gguf.ARRAY, (gguf.I16, [-1, 2, 3]))]
    for align in (32, 64):
        p = str(tmp_path / f"m{align}.gguf")
        gguf.write_gguf(p, meta, tens, alignment=align)
        g = GgufFile.open(p)
        try:
            assert g.data_offset % align == 0
            assert g.architecture() == "qwen2" and g.meta_u32("qwen2.context_length") == 32768
            assert g.meta("neg").value == -3 and g.meta("pi").as_f32() == 3.25
            assert g.meta("toks").as_list() == ["<s>", "é", ""]
            assert g.meta("ids").as_list() == [-1, 2, 3]
            for name, dims, tid, data in tens:
                t = g.tensors[name]
                assert t.dims == dims and int(t.dtype) == tid and t.offset % align == 0
                assert bytes(g.tensor_bytes(name)) == data
        finally:
            g.close()


def test_arena_offsets_are_aligned_and_disjoint():
    sizes = [144 * 14 * 4608, 210 * 3, 4 * 3584, 1, 176 * 74 * 7]
    offs, total = plan_offsets(sizes, 256)
    assert all(o % 256 == 0 for o in offs)
    for (o, n), o2 in zip(zip(offs, sizes), offs[1:] + [total]):
        assert o + n <= o2
    assert total == offs[-1] + sizes[-1]
    with pytest.raises(ValueError):
        plan_offsets(sizes, 48)
