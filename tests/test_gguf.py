"""GGUF reading (src/gguf.rs:95-172) and the expert-slot layout (src/expert_cache.rs:66-90)."""
import os
import struct

import numpy as np
import pytest

from rustingstrata_amd import ggml, gguf
from tests.helpers import random_blocks


def w_str(b, s):
    b += struct.pack("<Q", len(s)) + s.encode()


def synthetic_bytes():
    """The file of tests/gguf.rs:10-31: two keys and one 4 x 2 F32 tensor."""
    b = bytearray(b"GGUF")
    b += struct.pack("<IQQ", 3, 1, 2)
    w_str(b, "general.architecture")
    b += struct.pack("<I", 8)
    w_str(b, "qwen35moe")
    w_str(b, "qwen35moe.block_count")
    b += struct.pack("<II", 4, 41)
    w_str(b, "t")
    b += struct.pack("<IQQIQ", 2, 4, 2, 0, 0)
    b += bytes(-len(b) % 32)
    b += np.arange(1, 9, dtype=np.float32).tobytes()
    return bytes(b)


def test_parses_synthetic_file(tmp_path):
    """tests/gguf.rs:9-45: metadata, dims, bytes; 4 bytes cut off the data is a clean error naming the tensor."""
    p = tmp_path / "syn.gguf"
    p.write_bytes(synthetic_bytes())
    g = gguf.Gguf(str(p))
    assert g.get("general.architecture") == "qwen35moe"
    assert g.get("qwen35moe.block_count") == 41
    t = g.tensors["t"]
    assert t.dims == [4, 2]
    raw = g.bytes(t)
    assert len(raw) == 32 and raw[28:32].view(np.float32)[0] == 8.0
    cut = tmp_path / "syn.cut.gguf"
    cut.write_bytes(synthetic_bytes()[:-4])
    with pytest.raises(gguf.GgufError, match=r"GGUF truncated \(tensor t "):
        gguf.Gguf(str(cut))
    with pytest.raises(gguf.GgufError, match="missing GGUF key nope"):
        g.get("nope")


def test_rejects_bad_headers(tmp_path):
    b = bytearray(synthetic_bytes())
    p = tmp_path / "v.gguf"
    b[4:8] = struct.pack("<I", 4)
    p.write_bytes(bytes(b))
    with pytest.raises(gguf.GgufError, match="unsupported GGUF version 4"):
        gguf.Gguf(str(p))
    p.write_bytes(b"GGUX" + bytes(b[4:]))
    with pytest.raises(gguf.GgufError, match="not a GGUF file"):
        gguf.Gguf(str(p))
    b[4:8] = struct.pack("<I", 3)
    p.write_bytes(bytes(b[:30]))
    with pytest.raises(gguf.GgufError, match="GGUF truncated"):
        gguf.Gguf(str(p))


def test_round_trip_all_value_types(tmp_path):
    meta = [("a.u8", gguf.U8, 200), ("a.i8", gguf.I8, -5), ("a.u16", gguf.U16, 60000), ("a.i16", gguf.I16, -30000),
            ("a.u32", gguf.U32, 4000000000), ("a.i32", gguf.I32, -2000000000), ("a.f32", gguf.F32, 0.5),
            ("a.bool", gguf.BOOL, True), ("a.str", gguf.STR, "héllo"), ("a.u64", gguf.U64, 2 ** 63 + 5),
            ("a.i64", gguf.I64, -(2 ** 62)), ("a.f64", gguf.F64, 0.1), ("general.alignment", gguf.U32, 64),
            ("a.arr", gguf.ARR, (gguf.STR, ["x", "yz"])), ("a.nested", gguf.ARR, (gguf.ARR, [(gguf.I32, [1, 2]), (gguf.I32, [])]))]
    w1 = random_blocks(ggml.Q4_K, 3, 512, seed=1)
    w2 = random_blocks(ggml.Q8_0, 5, 64, seed=2)
    p = tmp_path / "rt.gguf"
    gguf.write_gguf(str(p), meta, [("w1", [512, 3], ggml.Q4_K, w1.tobytes()), ("w2", [64, 5], ggml.Q8_0, w2.tobytes())],
                    alignment=64)
    g = gguf.Gguf(str(p))
    for k, t, v in meta:
        got = g.get(k)
        if t == gguf.ARR:
            if v[0] == gguf.ARR:
                assert got == [x[1] for x in v[1]]
            else:
                assert got == v[1]
        elif t == gguf.F32:
            assert got == np.float32(v)
        else:
            assert got == v
    assert np.array_equal(g.bytes("w1"), w1.reshape(-1)) and np.array_equal(g.bytes("w2"), w2.reshape(-1))
    assert g._maps[0][2] % 64 == 0 and g.tensors["w2"].offset % 64 == 0
    g.close()


def moe_layer_file(path, E=4, H=512, F=256, seed=10):
    gate = random_blocks(ggml.Q5_K, E * F, H, seed=seed)
    up = random_blocks(ggml.Q5_K, E * F, H, seed=seed + 1)
    down = random_blocks(ggml.Q6_K, E * H, F, seed=seed + 2)
    gguf.write_gguf(path, [("general.architecture", gguf.STR, "qwen3moe")],
                    [("blk.0.ffn_gate_exps.weight", [H, F, E], ggml.Q5_K, gate.tobytes()),
                     ("blk.0.ffn_up_exps.weight", [H, F, E], ggml.Q5_K, up.tobytes()),
                     ("blk.0.ffn_down_exps.weight", [F, H, E], ggml.Q6_K, down.tobytes())])
    return gate, up, down


def test_slot_layout(tmp_path):
    """Gate, up, down of an expert back to back in its slot, each on a 16-byte boundary (src/expert_cache.rs:80-84)."""
    p = str(tmp_path / "moe.gguf")
    moe_layer_file(p)
    g = gguf.Gguf(p)
    mats, slot, ne = gguf.slot_layout(g, 0)
    gb = ggml.row_bytes(ggml.Q5_K, 512) * 256
    db = ggml.row_bytes(ggml.Q6_K, 256) * 512
    assert ne == 4
    assert [(m.ty, m.rows, m.cols, m.off, m.bytes) for m in mats] == [
        (ggml.Q5_K, 256, 512, 0, gb), (ggml.Q5_K, 256, 512, gb, gb), (ggml.Q6_K, 512, 256, 2 * gb, db)]
    assert slot == -(-(2 * gb + db) // 16) * 16
    with pytest.raises(gguf.GgufError, match="missing tensor blk.1.ffn_gate_exps.weight"):
        gguf.slot_layout(g, 1)


def test_split_model_reads_each_shard(tmp_path):
    """A split model (src/gguf.rs: open_one(path, i, ...)): a tensor of shard i reads shard i's bytes, at the same
    offset as a tensor of shard 0, and a name in two shards is an error."""
    a = np.arange(64, dtype=np.uint8)
    b = np.arange(64, dtype=np.uint8)[::-1].copy()
    c = np.full(64, 7, dtype=np.uint8)
    meta = [("split.count", gguf.U16, 3)]
    for i, (name, raw) in enumerate([("t0", a), ("t1", b), ("t2", c)]):
        gguf.write_gguf(str(tmp_path / f"m-{i + 1:05d}-of-00003.gguf"), meta, [(name, [16], 0, raw.tobytes())])
    g = gguf.Gguf(str(tmp_path / "m-00001-of-00003.gguf"))
    assert [g.tensors[n].file for n in ("t0", "t1", "t2")] == [0, 1, 2]
    assert np.array_equal(g.bytes("t0"), a) and np.array_equal(g.bytes("t1"), b) and np.array_equal(g.bytes("t2"), c)
    g.close()
    gguf.write_gguf(str(tmp_path / "m-00002-of-00003.gguf"), meta, [("t0", [16], 0, b.tobytes())])
    with pytest.raises(gguf.GgufError, match="tensor t0 in two shards"):
        gguf.Gguf(str(tmp_path / "m-00001-of-00003.gguf"))
