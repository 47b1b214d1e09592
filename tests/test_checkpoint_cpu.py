"""The library's safetensors reader (mtpx_st_* / mtpx_checkpoint_*) on the CPU: files written by the
`safetensors` package (an independent writer) read back name by name with their dtypes, shapes,
bytes and metadata; every malformed header the reference's reader refuses
(Sources/MLXFastCore/Safetensors.swift:75-176: too small, empty or oversized header length, a header
past the file, non-JSON, a JSON value that is not an object, a tensor without a string dtype, reversed
or out-of-file data offsets) is refused with its message; non-object entries and a non-string
metadata map are skipped; a checkpoint over several files (or a directory) is one name space and
refuses a name in two files.  No GPU call is made."""
import json
import os
import struct

import numpy as np
import pytest

import mtpx
from mtpx import MtpxError

st_np = pytest.importorskip("safetensors.numpy")


def _raw(path, header: bytes, data: bytes = b"", length=None):
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(header) if length is None else length))
        f.write(header)
        f.write(data)


def test_reads_back_what_the_safetensors_package_wrote(tmp_path):
    r = np.random.default_rng(3)
    t = {
        "b.weight": r.integers(0, 2 ** 32, (5, 4), dtype=np.uint32),
        "a.scales": r.standard_normal((5, 2)).astype(np.float16),
        "c.multipliers": r.integers(-2 ** 62, 2 ** 62, 3, dtype=np.int64),
        "z.empty": np.zeros((0, 7), np.float32),
        "d.scalar": np.array(3.5, np.float64),
    }
    p = tmp_path / "m.safetensors"
    st_np.save_file(t, str(p), metadata={"format": "mlx", "note": "tensors é中"})
    f = mtpx.SafetensorsFile(str(p))
    got = f.tensors()
    assert [g[0] for g in got] == sorted(t)
    dt = {np.uint32: "U32", np.float16: "F16", np.int64: "I64", np.float32: "F32", np.float64: "F64"}
    for name, dtype, shape, nbytes in got:
        a = t[name]
        assert dtype == dt[a.dtype.type] and shape == a.shape and nbytes == a.nbytes
        assert f.read(name) == a.tobytes()
    assert f.metadata("format") == "mlx" and f.metadata("note") == "tensors é中"
    assert f.metadata("absent") is None
    with pytest.raises(MtpxError, match="no tensor"):
        f.read("missing")
    f.close()


def test_bf16_tensor_bytes(tmp_path):
    """bf16 written as raw uint16 patterns under dtype BF16 (the checkpoints' scales and biases)."""
    bits = np.array([0x3F80, 0xC000, 0x7FC0, 0x0001], np.uint16)
    hdr = json.dumps({"s": {"dtype": "BF16", "shape": [4], "data_offsets": [0, 8]}}).encode()
    p = tmp_path / "b.safetensors"
    _raw(p, hdr, bits.tobytes())
    f = mtpx.SafetensorsFile(str(p))
    assert f.tensors() == [("s", "BF16", (4,), 8)]
    assert np.frombuffer(f.read("s"), np.uint16).tolist() == bits.tolist()


@pytest.mark.parametrize("case,message", [
    ("tiny", "too small"),
    ("zero", "header is empty"),
    ("huge", "exceeds 100000000 bytes"),
    ("past", "truncated safetensors header"),
    ("json", "invalid safetensors header JSON"),
    ("trailing", "invalid safetensors header JSON"),
    ("array", "must be a JSON object"),
    ("nodtype", "invalid tensor header for t"),
    ("reversed", "invalid data_offsets for t"),
    ("negative", "invalid data_offsets for t"),
    ("beyond", "exceed safetensors file size"),
    ("badshape", "invalid shape for t"),
    ("dupkey", "appears twice"),
])
def test_malformed_headers_are_refused(tmp_path, case, message):
    p = tmp_path / f"{case}.safetensors"
    ok = {"t": {"dtype": "U8", "shape": [2], "data_offsets": [0, 2]}}
    if case == "tiny":
        p.write_bytes(b"\x01\x00\x00")
    elif case == "zero":
        _raw(p, b"", b"xx", length=0)
    elif case == "huge":
        _raw(p, b"{}", b"", length=100_000_001)
    elif case == "past":
        _raw(p, b"{}", b"", length=50)
    elif case == "json":
        _raw(p, b'{"t": {"dtype": "U8",', b"ab")
    elif case == "trailing":
        _raw(p, json.dumps(ok).encode() + b" x", b"ab")
    elif case == "array":
        _raw(p, b"[1, 2]", b"ab")
    elif case == "nodtype":
        _raw(p, json.dumps({"t": {"dtype": 3, "shape": [2], "data_offsets": [0, 2]}}).encode(), b"ab")
    elif case == "reversed":
        _raw(p, json.dumps({"t": {"dtype": "U8", "shape": [2], "data_offsets": [2, 0]}}).encode(), b"ab")
    elif case == "negative":
        _raw(p, json.dumps({"t": {"dtype": "U8", "shape": [2], "data_offsets": [-1, 1]}}).encode(), b"ab")
    elif case == "beyond":
        _raw(p, json.dumps({"t": {"dtype": "U8", "shape": [4], "data_offsets": [0, 4]}}).encode(), b"ab")
    elif case == "badshape":
        _raw(p, json.dumps({"t": {"dtype": "U8", "shape": [2.5], "data_offsets": [0, 2]}}).encode(), b"ab")
    elif case == "dupkey":
        h = b'{"t": {"dtype": "U8", "shape": [2], "data_offsets": [0, 2]}, ' \
            b'"t": {"dtype": "U8", "shape": [2], "data_offsets": [0, 2]}}'
        _raw(p, h, b"ab")
    with pytest.raises(MtpxError, match=message):
        mtpx.SafetensorsFile(str(p))


def test_skipped_entries_and_escapes(tmp_path):
    """Entries whose value is not an object are skipped (as the reference's reader skips them), so is a
    metadata map with a non-string value; escaped names decode; whitespace is free."""
    hdr = ('{ "__metadata__": {"a": 1},  "note": "not a tensor", "n\\u00e9\\"q": '
           '{"dtype": "U8", "shape": [1, 2], "data_offsets": [1, 3]} }').encode()
    p = tmp_path / "s.safetensors"
    _raw(p, hdr, b"\x09\x07\x05")
    f = mtpx.SafetensorsFile(str(p))
    assert f.tensors() == [('né"q', "U8", (1, 2), 2)]
    assert f.read('né"q') == b"\x07\x05"
    assert f.metadata("a") is None


def test_checkpoint_name_space(tmp_path):
    d = tmp_path / "ckpt"
    d.mkdir()
    st_np.save_file({"x.a": np.ones(3, np.float32)}, str(d / "model-00001-of-00002.safetensors"))
    st_np.save_file({"x.b": np.ones(2, np.int64), "x.c": np.zeros(1, np.uint8)},
                    str(d / "model-00002-of-00002.safetensors"))
    (d / "model.safetensors.index.json").write_text("{}")  # not a shard: ignored by the directory scan
    ck = mtpx.Checkpoint(str(d))
    assert ck.count() == 3
    ck.close()
    ck = mtpx.Checkpoint([str(d / "model-00002-of-00002.safetensors")])
    assert ck.count() == 2
    ck.close()
    st_np.save_file({"x.a": np.ones(3, np.float32)}, str(tmp_path / "again.safetensors"))
    with pytest.raises(MtpxError, match="in two files"):
        mtpx.Checkpoint([str(d), str(tmp_path / "again.safetensors")])
    with pytest.raises(MtpxError, match="cannot open"):
        mtpx.Checkpoint([str(tmp_path / "absent.safetensors")])
    empty = tmp_path / "none"
    empty.mkdir()
    with pytest.raises(MtpxError, match="no safetensors files"):
        mtpx.Checkpoint(str(empty))
    assert os.path.exists(d / "model.safetensors.index.json")
