"""safetensors host loading (HostTensor::from_safetensors, tensor/memory.rs:190-223) at the C ABI.

The header query runs on the host and is checked here against files written by the `safetensors`
package itself; the device load is a GPU test. The reference checks only the shape (against the
element mapping's pair-flattened sizes) and the byte length; the bytes are the device image.
"""
import json
import struct

import numpy as np
import pytest

import furiosa_hip as fh

safetensors_numpy = pytest.importorskip("safetensors.numpy")


def write_raw(path, tensors):
    """A safetensors file from (name, dtype string, shape, raw bytes), laid out by the format spec."""
    header, off, blobs = {}, 0, []
    for name, dt, shape, raw in tensors:
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        off += len(raw)
        blobs.append(raw)
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    path.write_bytes(struct.pack("<Q", len(h)) + h + b"".join(blobs))


def test_info_matches_the_safetensors_package(tmp_path):
    p = tmp_path / "t.safetensors"
    tensors = {"w": np.arange(12, dtype=np.float32).reshape(3, 4), "b": np.arange(-5, 5, dtype=np.int8),
               "i": np.arange(6, dtype=np.int32).reshape(1, 2, 3)}
    safetensors_numpy.save_file(tensors, str(p), metadata={"format": "np"})
    raw = p.read_bytes()
    for name, arr in tensors.items():
        dt, shape, (b, e) = fh.safetensors_info(p, name)
        assert dt == {np.float32: fh.F32, np.int8: fh.I8, np.int32: fh.I32}[arr.dtype.type]
        assert shape == list(arr.shape)
        assert raw[b:e] == arr.tobytes()
    with pytest.raises(fh.FoError, match="no tensor"):
        fh.safetensors_info(p, "missing")
    with pytest.raises(fh.FoError, match="no tensor"):
        fh.safetensors_info(p, "__metadata__")


def test_info_of_bf16_and_fp8_entries(tmp_path):
    p = tmp_path / "t.safetensors"
    w = np.arange(8, dtype=np.uint16)
    write_raw(p, [("w", "BF16", (2, 4), w.tobytes()), ("f", "F8_E4M3", (4,), bytes([0x38, 0x30, 0, 0x7e])),
                  ("h", "F16", (2,), b"\0\0\0\0")])
    assert fh.safetensors_info(p, "w")[:2] == (fh.BF16, [2, 4])
    assert fh.safetensors_info(p, "f")[:2] == (fh.F8E4M3, [4])
    assert fh.safetensors_info(p, "h")[0] == -1  # no code for f16 here


def test_corrupt_files_are_errors(tmp_path):
    p = tmp_path / "bad.safetensors"
    p.write_bytes(struct.pack("<Q", 1000) + b"{}")
    with pytest.raises(fh.FoError, match="truncated header"):
        fh.safetensors_info(p, "w")
    write_raw(p, [("w", "F32", (4,), b"\0" * 16)])
    data = p.read_bytes()
    p.write_bytes(data[:-4])
    with pytest.raises(fh.FoError, match="past the end"):
        fh.safetensors_info(p, "w")
    with pytest.raises(fh.FoError, match="cannot open"):
        fh.safetensors_info(tmp_path / "none.safetensors", "w")


def test_hostile_headers_are_errors_not_crashes(tmp_path):
    # A header nested far deeper than any real one is refused (no unbounded recursion).
    p = tmp_path / "deep.safetensors"
    h = b'{"w": ' + b"[" * 100000 + b"]" * 100000 + b"}"
    h += b" " * (-len(h) % 8)
    p.write_bytes(struct.pack("<Q", len(h)) + h)
    with pytest.raises(fh.FoError, match="nesting too deep"):
        fh.safetensors_info(p, "w")
    # An offset that is a double far outside int64 is refused, not cast.
    h = b'{"w": {"dtype": "F32", "shape": [1], "data_offsets": [0, 1e300]}}'
    h += b" " * (-len(h) % 8)
    p.write_bytes(struct.pack("<Q", len(h)) + h + b"\0" * 4)
    with pytest.raises(fh.FoError):
        fh.safetensors_info(p, "w")


def test_escaped_tensor_names_decode(tmp_path):
    # JSON \u escapes (including a surrogate pair) decode to the UTF-8 name a caller passes.
    p = tmp_path / "esc.safetensors"
    h = b'{"w\\u00e9\\ud83d\\ude00": {"dtype": "I8", "shape": [2], "data_offsets": [0, 2]}}'
    h += b" " * (-len(h) % 8)
    p.write_bytes(struct.pack("<Q", len(h)) + h + b"\x05\x06")
    dt, shape, _ = fh.safetensors_info(p, "wé\U0001F600")
    assert dt == fh.I8 and shape == [2]
