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
