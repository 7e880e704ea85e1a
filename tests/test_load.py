"""The safetensors reader of libbq (host code; no GPU): tensor metadata and
bytes from files written by the safetensors library, and the header
validation rules of safetensors/parser.mojo:215-320 on malformed files."""
import ctypes as C
import json
import struct

import numpy as np
import pytest


@pytest.fixture(scope="module")
def bq():
    import bq
    return bq


def write_st(path, header: dict, payload: bytes, raw_header: bytes | None = None):
    h = raw_header if raw_header is not None else json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        f.write(payload)


def test_reads_library_files(bq, tmp_path):
    from safetensors.numpy import save_file
    rng = np.random.default_rng(0)
    t = {
        "layer.w": rng.integers(-127, 128, (32, 128), dtype=np.int8),
        "layer.w.scale": rng.random(32).astype(np.float32),
        "experts.w": rng.integers(-127, 128, (2, 16, 64), dtype=np.int8),
        "vec": np.arange(7, dtype=np.int64),
        "empty": np.zeros((0, 4), np.float32),
    }
    p = tmp_path / "m.safetensors"
    save_file(t, str(p), metadata={"format": "pt", "note": "quote \" and \\u00e9"})
    f = bq.SafetensorsFile(str(p))
    assert len(f) == len(t)
    for name, a in t.items():
        dt, shape, nbytes, addr = f.info(name)
        assert shape == a.shape and nbytes == a.nbytes
        assert dt == {np.int8: "I8", np.float32: "F32", np.int64: "I64"}[a.dtype.type]
        if nbytes:
            assert C.string_at(addr, nbytes) == a.tobytes()
    with pytest.raises(bq.BqError, match="missing tensor"):
        f.info("nope")
    f.close()


def good_header():
    return {"__metadata__": {"k": "v"},
            "a": {"dtype": "I8", "shape": [2, 4], "data_offsets": [0, 8]},
            "b": {"dtype": "F32", "shape": [2], "data_offsets": [8, 16]}}


@pytest.mark.parametrize("case,msg", [
    ("short", "too small"),
    ("hlen", "exceeds file"),
    ("huge", "too large"),
    ("trailing", "trailing content"),
    ("overlap", "overlapping"),
    ("size", "byte size does not match"),
    ("dtype", "unsupported dtype"),
    ("dup", "duplicate tensor"),
    ("unindexed", "not fully indexed"),
    ("fields", "missing required fields"),
    ("past", "exceed the payload"),
    ("syntax", "parse error"),
])
def test_rejects_malformed(bq, tmp_path, case, msg):
    p = tmp_path / f"{case}.safetensors"
    h = good_header()
    payload = bytes(16)
    if case == "short":
        p.write_bytes(b"\x01\x02")
    elif case == "hlen":
        p.write_bytes(struct.pack("<Q", 1000) + b"{}")
    elif case == "huge":
        p.write_bytes(struct.pack("<Q", 200 << 20) + b"{}")
    elif case == "trailing":
        write_st(p, None, payload, json.dumps(h).encode() + b" x")
    elif case == "overlap":
        h["b"]["data_offsets"] = [4, 12]
        h["b"]["dtype"] = "I8"
        h["b"]["shape"] = [8]
        write_st(p, h, payload)
    elif case == "size":
        h["a"]["shape"] = [3, 4]
        write_st(p, h, payload)
    elif case == "dtype":
        h["a"]["dtype"] = "Q4"
        write_st(p, h, payload)
    elif case == "dup":
        raw = b'{"a": {"dtype": "I8", "shape": [8], "data_offsets": [0, 8]},' \
              b' "a": {"dtype": "I8", "shape": [8], "data_offsets": [8, 16]}}'
        write_st(p, None, payload, raw)
    elif case == "unindexed":
        write_st(p, h, payload + bytes(4))
    elif case == "fields":
        del h["b"]["shape"]
        write_st(p, h, payload)
    elif case == "past":
        h["b"]["data_offsets"] = [8, 24]
        h["b"]["shape"] = [4]
        write_st(p, h, payload)
    elif case == "syntax":
        write_st(p, None, payload, b'{"a": {"dtype": "I8" "shape": [8]}}')
    with pytest.raises(bq.BqError) as ei:
        bq.SafetensorsFile(str(p))
    assert ei.value.code == 1 and msg in str(ei.value)


def test_well_formed_hand_written(bq, tmp_path):
    p = tmp_path / "ok.safetensors"
    write_st(p, good_header(), bytes(range(8)) + np.array([1.5, -2.0], np.float32).tobytes())
    f = bq.SafetensorsFile(str(p))
    assert f.info("a")[:3] == ("I8", (2, 4), 8)
    dt, shape, nb, addr = f.info("b")
    assert np.frombuffer(C.string_at(addr, nb), np.float32).tolist() == [1.5, -2.0]
