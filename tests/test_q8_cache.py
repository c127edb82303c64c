"""The LFM3Q8C1 weight cache (lib/src/q8_cache.dart): layout, round trips,
misses, and the failure cases of test/failure_recovery_test.dart:27-74 and
test/vision_backbone_cache_test.dart:88-106. CPU only."""

import json
import os
import struct

import numpy as np
import pytest

from dianoia_amd.errors import FormatException, StateError
from dianoia_amd.formats import QuantMatrix
from dianoia_amd.q8_cache import (ALIGN, HEADER_REGION, MAGIC, MappedFile, Q8Cache,
                                  byte_lengths, fnv1a64)


def q8(rng, rows, cols):
    qs = rng.integers(-127, 128, (rows, cols), dtype=np.int8)
    sc = rng.random(rows * cols // 32, dtype=np.float32)
    return QuantMatrix.q8(qs, sc)


def q4(rng, rows, cols):
    qs = rng.integers(0, 256, (rows, cols // 2), dtype=np.uint8)
    sc = rng.integers(0, 0x7C00, rows * cols // 32, dtype=np.uint16)
    return QuantMatrix.q4(qs, sc)


@pytest.fixture()
def written(tmp_path):
    rng = np.random.default_rng(3)
    mats = {"layers.0.q": q8(rng, 48, 64), "layers.0.ffn": q4(rng, 40, 96),
            "lm_head": q8(rng, 7, 32)}
    path = str(tmp_path / "lfm3-q8.cache")
    Q8Cache.write(path, "k1", mats)
    return path, mats


def test_fnv1a64_published_vectors():
    # The FNV-1a 64-bit test vectors of the algorithm's authors.
    assert fnv1a64(b"") == 0xCBF29CE484222325
    assert fnv1a64(b"a") == 0xAF63DC4C8601EC8C
    assert fnv1a64(b"foobar") == 0x85944171F73967E8
    # Streaming: hashing in pieces equals hashing the concatenation.
    assert fnv1a64(b"bar", fnv1a64(b"foo")) == fnv1a64(b"foobar")


def test_layout(written):
    path, mats = written
    raw = open(path, "rb").read()
    assert raw[:8] == MAGIC
    (hlen,) = struct.unpack("<Q", raw[8:16])
    header = json.loads(raw[16:16 + hlen])
    assert header["version"] == 1 and header["key"] == "k1"
    assert list(header["tensors"]) == list(mats)       # writer order kept
    assert raw[16 + hlen:HEADER_REGION] == bytes(HEADER_REGION - 16 - hlen)
    offset = HEADER_REGION
    for name, m in mats.items():
        e = header["tensors"][name]
        assert e["format"] == m.format and e["rows"] == m.rows and e["cols"] == m.cols
        qs_len, sc_len = byte_lengths(m.format, m.rows, m.cols)
        # Values then scales, each at the next 64-byte boundary.
        assert e["qs"] == (offset + ALIGN - 1) // ALIGN * ALIGN
        assert e["scales"] == (e["qs"] + qs_len + ALIGN - 1) // ALIGN * ALIGN
        offset = e["scales"] + sc_len
        assert raw[e["qs"]:e["qs"] + qs_len] == m.qs_bytes.tobytes()
        assert raw[e["scales"]:e["scales"] + sc_len] == m.scale_bytes.tobytes()
    assert len(raw) == offset
    assert not os.path.exists(path + ".partial")


def test_round_trip(written):
    path, mats = written
    cache = Q8Cache.open(path, "k1")
    assert cache is not None
    try:
        assert set(cache.shapes) == {(n, m.rows, m.cols) for n, m in mats.items()}
        for name, m in mats.items():
            got = cache.matrix(name, m.rows, m.cols)
            assert got.format == m.format
            assert np.array_equal(got.qs_bytes, m.qs_bytes)
            assert np.array_equal(got.scale_bytes, m.scale_bytes)
            o = cache.offsets(name, m.rows, m.cols)
            assert o["end"] == o["scales"] + byte_lengths(m.format, m.rows, m.cols)[1]
        assert cache.matrix("lm_head", 7, 64) is None      # another shape
        assert cache.matrix("absent", 7, 32) is None
    finally:
        cache.close()
    assert not MappedFile.is_mapped(path)


def test_shared_mapping_is_counted(written):
    path, _ = written
    a = Q8Cache.open(path, "k1")
    b = Q8Cache.open(path, "k1")
    assert a.file is b.file
    a.close()
    assert MappedFile.is_mapped(path)
    b.close()
    assert not MappedFile.is_mapped(path)


def test_misses(tmp_path, written):
    path, _ = written
    assert Q8Cache.open(str(tmp_path / "none"), "k1") is None
    short = tmp_path / "short"
    short.write_bytes(MAGIC)
    assert Q8Cache.open(str(short), "k1") is None
    other = tmp_path / "other"
    other.write_bytes(b"GGUF" + bytes(60))
    assert Q8Cache.open(str(other), "k1") is None
    assert not MappedFile.is_mapped(str(other))
    assert Q8Cache.open(path, "another key") is None
    assert not MappedFile.is_mapped(path)
    raw = bytearray(open(path, "rb").read())
    (hlen,) = struct.unpack("<Q", raw[8:16])
    text = raw[16:16 + hlen].decode().replace('"version":1', '"version":2')
    versioned = tmp_path / "v2"
    versioned.write_bytes(bytes(raw[:16]) + text.encode() + bytes(raw[16 + hlen:]))
    assert Q8Cache.open(str(versioned), "k1") is None


def test_truncated_cache_throws_and_releases(written):
    path, _ = written
    raw = open(path, "rb").read()
    open(path, "wb").write(raw[:-1])
    with pytest.raises(FormatException):
        Q8Cache.open(path, "k1")
    assert not MappedFile.is_mapped(path)


def test_header_length_past_the_end_throws(written):
    path, _ = written
    raw = bytearray(open(path, "rb").read())
    raw[8:16] = struct.pack("<Q", len(raw))
    open(path, "wb").write(raw)
    with pytest.raises(FormatException):
        Q8Cache.open(path, "k1")
    assert not MappedFile.is_mapped(path)


def test_matrix_offset_outside_the_file_throws(written):
    path, mats = written
    cache = Q8Cache.open(path, "k1")
    name, rows, cols = list(cache.shapes)[0]
    qs = cache.offsets(name, rows, cols)["qs"]
    cache.close()
    raw = bytearray(open(path, "rb").read())
    text = raw[16:16 + 4096].decode("latin-1")
    at = text.index(f'"qs":{qs}')
    raw[16 + at + len('"qs":')] = ord("9")   # one digit more moves it far past the end
    open(path, "wb").write(raw)
    with pytest.raises(FormatException):
        Q8Cache.open(path, "k1")
    assert not MappedFile.is_mapped(path)


@pytest.mark.parametrize("change", [
    {"format": "q6"}, {"cols": 48}, {"rows": 0}, {"scales": 2}, {"qs": -64},
    {"rows": True}, {"cols": 64.0}, {"qs": "1048576"},
])
def test_entries_that_do_not_fit(tmp_path, written, change):
    path, _ = written
    raw = bytearray(open(path, "rb").read())
    (hlen,) = struct.unpack("<Q", raw[8:16])
    header = json.loads(raw[16:16 + hlen])
    header["tensors"]["lm_head"].update(change)
    text = json.dumps(header, separators=(",", ":")).encode()
    assert 16 + len(text) <= HEADER_REGION
    damaged = tmp_path / "damaged"
    damaged.write_bytes(bytes(raw[:8]) + struct.pack("<Q", len(text)) + text
                        + bytes(raw[16 + len(text):]))
    with pytest.raises(FormatException):
        Q8Cache.open(str(damaged), "k1")
    assert not MappedFile.is_mapped(str(damaged))


def test_header_not_an_object_throws(tmp_path):
    path = tmp_path / "list"
    text = b"[1,2]"
    path.write_bytes(MAGIC + struct.pack("<Q", len(text)) + text + bytes(64))
    with pytest.raises(FormatException):
        Q8Cache.open(str(path), "k1")


def test_write_each_rejects_a_mismatched_matrix_and_hands_it_back(tmp_path):
    rng = np.random.default_rng(1)
    released = []
    with pytest.raises(StateError):
        Q8Cache.write_each(str(tmp_path / "cache"), "key", [("matrix", "q4", 2, 32)],
                           lambda name: q8(rng, 2, 32), done=released.append)
    assert len(released) == 1
    assert not os.path.exists(tmp_path / "cache")   # only the .partial file was written


def test_write_each_streams_in_order(tmp_path):
    rng = np.random.default_rng(2)
    made = []

    def matrix(name):
        made.append(name)
        return q4(rng, 4, 64) if name.endswith("4") else q8(rng, 4, 64)

    shapes = [("b4", "q4", 4, 64), ("a8", "q8", 4, 64)]
    done = []
    Q8Cache.write_each(str(tmp_path / "c"), "key", shapes, matrix,
                       done=lambda m: done.append(m.format))
    assert made == ["b4", "a8"] and done == ["q4", "q8"]
    cache = Q8Cache.open(str(tmp_path / "c"), "key")
    assert cache.offsets("b4", 4, 64)["qs"] < cache.offsets("a8", 4, 64)["qs"]
    cache.close()


def test_header_that_does_not_fit_its_region(tmp_path):
    rng = np.random.default_rng(0)
    m = q8(rng, 1, 32)
    names = {f"t{'x' * 200}{i}": m for i in range(6000)}   # > 1 MiB of JSON
    with pytest.raises(StateError):
        Q8Cache.write(str(tmp_path / "big"), "k", names)


def test_key_for(tmp_path):
    d = tmp_path / "model"
    d.mkdir()
    header = json.dumps({"w": {"dtype": "BF16", "shape": [2, 2],
                               "data_offsets": [0, 8]}}).encode()
    st = struct.pack("<Q", len(header)) + header + bytes(8)
    (d / "model.safetensors").write_bytes(st)
    (d / "config.json").write_bytes(b'{"hidden_size": 4}')
    key = Q8Cache.key_for(str(d))
    assert len(key) == 16 and int(key, 16) >= 0 and key == key.lower()
    # The fingerprint is FNV-1a over, in order: the 8 length bytes, the
    # header, the file size in decimal, config.json and the format text.
    want = fnv1a64(struct.pack("<Q", len(header)) + header + str(len(st)).encode()
                   + b'{"hidden_size": 4}' + b"LFM3Q8C1 v1 q8 block 32")
    assert key == f"{want:016x}"
    assert Q8Cache.key_for(str(d), weights="q4") != key
    (d / "config.json").write_bytes(b'{"hidden_size": 8}')
    assert Q8Cache.key_for(str(d)) != key
