"""The GGUF reader (include/c0ven_gguf.h) on files written from the format by tests/gguf_writer.py, without a GPU:
metadata of every value type, the tensor table (shapes, types, offsets at general.alignment, the mapped bytes), split
files, header-only architecture reads, page release, and the errors of malformed files. The reference's own test reads
the real model (core/tests/gguf_test.cpp:12-56), which is not on this machine; its census
(docs/model/tensors-IQ3_S.tsv) gives the names and shapes the MoE loader expects."""
import os
import struct

import numpy as np
import pytest

from tests import gguf_writer as gw
from tests.harness import moe

rng = np.random.default_rng(9)

KV = [("general.architecture", gw.STRING, "qwen4exp"), ("qwen4exp.block_count", gw.U32, 48),
      ("qwen4exp.embedding_length", gw.U64, 2560), ("a.i8", gw.I8, -5), ("a.u16", gw.U16, 65535),
      ("a.i16", gw.I16, -32768), ("a.i32", gw.I32, -7), ("a.i64", gw.I64, 23703573157769), ("a.f32", gw.F32, 0.5),
      ("a.f64", gw.F64, 1e-300), ("a.bool", gw.BOOL, 1), ("a.u8", gw.U8, 200),
      ("a.ints", gw.ARRAY, (gw.I32, [1, -2, 3])), ("a.u64s", gw.ARRAY, (gw.U64, [2**40, 5])),
      ("a.floats", gw.ARRAY, (gw.F32, [0.25, -1.5])), ("a.strs", gw.ARRAY, (gw.STRING, ["x", "yz"]))]


def tensors():
    q4 = rng.integers(0, 256, size=2 * 144, dtype=np.uint8)     # 2 x 256 Q4_K values
    bf = rng.integers(0, 65536, size=3 * 5, dtype=np.uint16)     # 5 x 3 BF16
    f32 = rng.standard_normal(7).astype(np.float32)
    return [("blk.0.w", moe.QT_Q4_K, (256, 2), q4), ("z.bf", 30, (5, 3), bf.view(np.uint8)),
            ("a.f", 0, (7,), f32.view(np.uint8))]


@pytest.mark.parametrize("alignment", [None, 64])
def test_metadata_and_tensors(tmp_path, alignment):
    path = str(tmp_path / "m.gguf")
    ts = tensors()
    gw.write(path, KV, ts, alignment)
    g = moe.GgufFile(path)
    assert g.n_files == 1
    assert g.get_string("general.architecture") == "qwen4exp" and moe.gguf_architecture(path) == "qwen4exp"
    assert g.get_int("qwen4exp.block_count") == 48 and g.get_int("qwen4exp.embedding_length") == 2560
    assert [g.get_int(k) for k in ("a.i8", "a.u16", "a.i16", "a.i32", "a.i64", "a.u8", "a.bool")] == \
        [-5, 65535, -32768, -7, 23703573157769, 200, 1]
    assert g.get_float("a.f32") == 0.5 and g.get_float("a.f64") == 1e-300 and g.get_float("a.i32") == -7.0
    assert g.get_ints("a.ints") == [1, -2, 3] and g.get_ints("a.u64s") == [2**40, 5]
    assert g.has("a.floats") and g.has("a.strs") and not g.has("nope")
    for bad in (lambda: g.get_int("a.f32"), lambda: g.get_string("a.i8"), lambda: g.get_ints("a.floats"),
                lambda: g.get_int("nope"), lambda: g.tensor("nope")):
        with pytest.raises(moe.MoeError):
            bad()
    infos = g.tensors()
    assert [t["name"] for t in infos] == sorted(t[0] for t in ts)  # name order
    align = alignment or 32
    size = os.path.getsize(path)
    for name, t, shape, data in ts:
        info = g.tensor(name)
        assert info["type"] == t and info["shape"] == shape and info["shard"] == 0
        assert info["bytes"] == data.size and info["offset"] % align == 0 and info["offset"] + info["bytes"] <= size
        assert np.array_equal(g.tensor_bytes(name), data)
        with open(path, "rb") as f:
            f.seek(info["offset"])
            assert f.read(data.size) == data.tobytes()
    g.release("blk.0.w")  # the pages go back; the bytes stay readable
    assert np.array_equal(g.tensor_bytes("blk.0.w"), ts[0][3])
    g.close()


def test_split_files(tmp_path):
    """<stem>-0000i-of-0000N.gguf: every shard is opened from the first's name; the split.* keys of the other shards
    are dropped, the first shard's kept (GgufModel::open_shard)."""
    stem = str(tmp_path / "model")
    ts = tensors()
    gw.write(stem + "-00001-of-00002.gguf", KV + [("split.no", gw.U16, 0)], ts[:2])
    gw.write(stem + "-00002-of-00002.gguf", [("split.no", gw.U16, 1), ("b.extra", gw.U32, 9)], ts[2:], alignment=128)
    for name in ("-00001-of-00002.gguf", "-00002-of-00002.gguf"):
        g = moe.GgufFile(stem + name)
        assert g.n_files == 2
        assert g.get_int("split.no") == 0 and g.get_int("b.extra") == 9
        assert g.tensor("a.f")["shard"] == 1 and g.tensor("blk.0.w")["shard"] == 0
        for tname, _, _, data in ts:
            assert np.array_equal(g.tensor_bytes(tname), data)
        g.close()
    os.remove(stem + "-00002-of-00002.gguf")
    with pytest.raises(moe.MoeError):
        moe.GgufFile(stem + "-00001-of-00002.gguf")


def test_malformed_files(tmp_path):
    path = str(tmp_path / "bad.gguf")
    gw.write(path, KV, tensors())
    good = open(path, "rb").read()
    cases = {
        "magic": b"GGUX" + good[4:],
        "version": good[:4] + (2).to_bytes(4, "little") + good[8:],
        "truncated header": good[:60],
        "truncated data": good[:-200],
    }
    for what, data in cases.items():
        with open(path, "wb") as f:
            f.write(data)
        with pytest.raises(moe.MoeError):
            moe.GgufFile(path)
    gw.write(path, KV, tensors() + [tensors()[0]])  # a name twice
    with pytest.raises(moe.MoeError):
        moe.GgufFile(path)
    gw.write(path, KV, [("x", moe.QT_Q4_K, (100,), np.zeros(144, np.uint8))])  # not whole blocks
    with pytest.raises(moe.MoeError):
        moe.GgufFile(path)
    with pytest.raises(moe.MoeError):
        moe.GgufFile(str(tmp_path / "missing.gguf"))
    gw.write(path, [("x", gw.U32, 1)], [])
    with pytest.raises(moe.MoeError):
        moe.gguf_architecture(path)


def test_type_bytes():
    tb = moe.lib.gguf_type_bytes
    assert tb(moe.QT_Q4_K, 2560) == 10 * 144 and tb(moe.QT_IQ4_NL, 640) == 20 * 18 and tb(moe.QT_Q2_0, 640) == 180
    assert tb(moe.QT_IQ3_XXS, 2560 * 640) == 6400 * 98 and tb(moe.QT_IQ2_S, 256) == 82 and tb(30, 5) == 10
    assert tb(0, 3) == 12 and tb(moe.QT_Q4_K, 100) == 0 and tb(99, 256) == 0


def test_hostile_offsets_and_shapes(tmp_path):
    """Tensor records whose offset or element count would wrap 64-bit arithmetic are refused, not mapped."""
    path = str(tmp_path / "h.gguf")
    q4 = np.zeros(144, np.uint8)
    gw.write(path, KV, [("x", moe.QT_Q4_K, (256,), q4)])
    raw = bytearray(open(path, "rb").read())
    at = raw.find(b"x" + struct.pack("<I", 1)) + 1 + 4 + 8 + 4  # name, dims, shape[0], type: the offset
    for off in (2**64 - 32, 2**63, len(raw) * 2 // 32 * 32):
        bad = bytearray(raw)
        bad[at:at + 8] = struct.pack("<Q", off)
        open(path, "wb").write(bytes(bad))
        with pytest.raises(moe.MoeError):
            moe.GgufFile(path)
    gw.write(path, KV, [("x", moe.QT_Q4_K, (256, 2**62, 8), q4)])  # 2^73 elements
    with pytest.raises(moe.MoeError):
        moe.GgufFile(path)


def test_split_shard_alignment_is_its_own(tmp_path):
    """Each file of a set places its data section at its own general.alignment, whatever the first file says."""
    stem = str(tmp_path / "s")
    ts = tensors()
    gw.write(stem + "-00001-of-00002.gguf", KV, ts[:1], alignment=256)
    gw.write(stem + "-00002-of-00002.gguf", [], ts[1:])  # default 32
    g = moe.GgufFile(stem + "-00001-of-00002.gguf")
    for tname, _, _, data in ts:
        assert np.array_equal(g.tensor_bytes(tname), data)
    g.close()
