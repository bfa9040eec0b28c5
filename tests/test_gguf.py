"""The library's GGUF reader (kf_gguf_*) against files written by an independent writer from the format description
(tests/gguf_writer.py): metadata of every value kind, tensor infos and byte views, alignment, versions, split shards,
and the reference's error cases (crates/kf-gguf/src/lib.rs)."""
import os
import struct

import numpy as np
import pytest

import kungfu_amd as kf
from kungfu_amd.gguf import GGUF
import gguf_writer as gw


def _blob(n, seed):
    return np.random.default_rng(seed).integers(0, 256, n, dtype=np.uint8).tobytes()


KVS = [
    ("general.architecture", "str", "llama"),
    ("a.u8", "u8", 250), ("a.i8", "i8", -7), ("a.u16", "u16", 65000), ("a.i16", "i16", -30000),
    ("a.u32", "u32", 4_000_000_000), ("a.i32", "i32", -2_000_000_000), ("a.f32", "f32", 1.5),
    ("a.bool", "bool", 1), ("a.u64", "u64", 2**63 + 5), ("a.i64", "i64", -(2**62)), ("a.f64", "f64", 2.0**-40),
    ("tok.scores", "arr", (6, [0.5, -1.25, 3.0])), ("tok.tokens", "arr", (8, ["<s>", "héllo", ""])),
    ("tok.ids", "arr", (4, [1, 2, 3, 4])), ("nested", "arr", (9, [(4, [1, 2]), (4, [3])])),
]


def _tensors():
    return [
        ("blk.0.ffn_gate.weight", [512, 3], kf.TYPE_Q4_K, _blob(3 * 2 * 144, 1)),
        ("token_embd.norm", [7], 0, _blob(28, 2)),
        ("output.weight", [256, 2], kf.TYPE_Q6_K, _blob(2 * 210, 3)),
        ("blk.0.attn_q.weight", [64, 4], kf.TYPE_Q8_0, _blob(4 * 2 * 34, 4)),
    ]


def test_metadata_tensors_and_bytes_round_trip(tmp_path):
    path = tmp_path / "m.gguf"
    ts = _tensors()
    data_start, offsets = gw.write(path, KVS, ts)
    with GGUF(path) as g:
        assert g.n_shards == 1
        m = g.meta
        assert m["general.architecture"] == "llama"
        assert (m["a.u8"], m["a.i8"], m["a.u16"], m["a.i16"]) == (250, -7, 65000, -30000)
        assert (m["a.u32"], m["a.i32"], m["a.u64"], m["a.i64"]) == (4_000_000_000, -2_000_000_000, 2**63 + 5, -(2**62))
        assert m["a.f32"] == 1.5 and m["a.f64"] == 2.0**-40 and m["a.bool"] is True
        assert m["tok.scores"] == [0.5, -1.25, 3.0] and m["tok.tokens"] == ["<s>", "héllo", ""] and m["tok.ids"] == [1, 2, 3, 4]
        assert list(m) == sorted(m)  # key order, as the reference's BTreeMap
        assert [t.name for t in g.tensors] == [t[0] for t in ts]
        for (name, dims, ty, blob), off in zip(ts, offsets):
            t = g.tensor(name)
            assert (t.dims, t.ggml_type, t.shard, t.offset, t.nbytes) == (tuple(dims), ty, 0, off, len(blob))
            assert g.data(name).tobytes() == blob
        assert g.tensor("missing") is None
    raw = open(path, "rb").read()
    assert data_start % 32 == 0 and raw[data_start + offsets[2] : data_start + offsets[2] + 420] == ts[2][3]


def test_alignment_key_and_version_2(tmp_path):
    path = tmp_path / "a.gguf"
    kvs = [("general.alignment", "u32", 64), ("x", "str", "y")]
    ts = _tensors()[:2]
    data_start, offsets = gw.write(path, kvs, ts, version=2, alignment=64)
    assert data_start % 64 == 0 and offsets[1] % 64 == 0
    with GGUF(path) as g:
        assert g.meta["general.alignment"] == 64
        for name, _, _, blob in ts:
            assert g.data(name).tobytes() == blob


def test_split_shards_open_as_one(tmp_path):
    ts = _tensors()
    gw.write(tmp_path / "model-00001-of-00002.gguf", KVS[:3], ts[:2])
    gw.write(tmp_path / "model-00002-of-00002.gguf", [("split.only", "u32", 9)], ts[2:])
    for first in ("model-00001-of-00002.gguf", "model-00002-of-00002.gguf"):
        with GGUF(tmp_path / first) as g:
            assert g.n_shards == 2
            assert "split.only" not in g.meta and g.meta["general.architecture"] == "llama"  # the first shard's header
            assert [t.shard for t in g.tensors] == [0, 0, 1, 1]
            for name, _, _, blob in ts:
                assert g.data(name).tobytes() == blob
    os.remove(tmp_path / "model-00002-of-00002.gguf")
    with pytest.raises(kf.KfError, match="open .*00002-of-00002"):
        GGUF(tmp_path / "model-00001-of-00002.gguf")


def test_reader_errors(tmp_path):
    good = tmp_path / "g.gguf"
    gw.write(good, KVS, _tensors())
    raw = open(good, "rb").read()
    bad = tmp_path / "b.gguf"
    cases = [
        (b"GGUX" + raw[4:], "not a GGUF file"),
        (raw[:4] + struct.pack("<I", 4) + raw[8:], "unsupported GGUF version 4"),
        (raw[:60], "truncated header"),
    ]
    for blob, needle in cases:
        open(bad, "wb").write(blob)
        with pytest.raises(kf.KfError, match=needle):
            GGUF(bad)
    gw.write(bad, [("k", "u32", 1)], [])
    raw = bytearray(open(bad, "rb").read())
    raw[24 + 9 : 24 + 13] = struct.pack("<I", 13)  # the key's value type
    open(bad, "wb").write(raw)
    with pytest.raises(kf.KfError, match="unknown metadata value type 13"):
        GGUF(bad)
    # a tensor whose data runs past the end: the header opens, its bytes do not (Gguf::bytes)
    data_start, _ = gw.write(bad, [], [("t", [256, 1], kf.TYPE_Q4_K, _blob(144, 5))])
    os.truncate(bad, data_start + 100)
    with GGUF(bad) as g:
        with pytest.raises(kf.KfError, match="past end"):
            g.data("t")
    # an unknown ggml type has no size (TensorInfo::nbytes fails) and no data
    gw.write(bad, [], [("u", [32, 1], 5, _blob(32, 6)), ("v", [100, 2], kf.TYPE_Q4_K, _blob(8, 7))])
    with GGUF(bad) as g:
        assert g.tensor("u").nbytes == -1 and g.tensor("v").nbytes == -1  # type 5 is unknown; 100 is not 256-divisible
        with pytest.raises(kf.KfError, match="does not fit"):
            g.data("u")
    with pytest.raises(kf.KfError, match="open"):
        GGUF(tmp_path / "none.gguf")


def test_typed_reads_follow_the_reference_conversions(tmp_path):
    import ctypes

    path = tmp_path / "t.gguf"
    gw.write(path, KVS, [])
    with GGUF(path) as g:
        L, h = kf.lib(), g._h
        i = L.kf_gguf_find_kv(h, b"a.i8")
        u, s, f = ctypes.c_uint64(), ctypes.c_int64(), ctypes.c_double()
        assert L.kf_gguf_kv_u64(h, i, 0, ctypes.byref(u)) == kf.KF_E_INVALID  # a negative signed value is no u64
        assert L.kf_gguf_kv_i64(h, i, 0, ctypes.byref(s)) == 0 and s.value == -7
        assert L.kf_gguf_kv_f64(h, i, 0, ctypes.byref(f)) == 0 and f.value == -7.0  # integers read as floats
        b = L.kf_gguf_find_kv(h, b"a.bool")
        assert L.kf_gguf_kv_u64(h, b, 0, ctypes.byref(u)) == 0 and u.value == 1
        fl = L.kf_gguf_find_kv(h, b"a.f32")
        assert L.kf_gguf_kv_i64(h, fl, 0, ctypes.byref(s)) == kf.KF_E_INVALID  # floats are not integers
        arr = L.kf_gguf_find_kv(h, b"tok.ids")
        assert L.kf_gguf_kv_u64(h, arr, 3, ctypes.byref(u)) == 0 and u.value == 4
        assert L.kf_gguf_kv_u64(h, arr, 4, ctypes.byref(u)) == kf.KF_E_INVALID and "array index 4" in kf.last_error()
        assert L.kf_gguf_find_kv(h, b"nope") == kf.KF_E_INVALID
