"""The C ABI library loads, exports every symbol include/furiosa_hip.h declares, and fails cleanly
(status + message, no crash) where it needs a device this container does not have. CPU only."""
import ctypes
import re
from pathlib import Path

import pytest

import furiosa_hip as fh

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    text = (ROOT / "include" / "furiosa_hip.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z0-9_]+\s*\*?\s*(fo_[a-z0-9_]+)\(", text, re.M)))


def test_every_declared_symbol_is_exported():
    lib = ctypes.CDLL(str(fh.LIB_PATH))
    names = declared_symbols()
    assert len(names) >= 25
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_the_header():
    assert set(declared_symbols()) == set(fh.EXPORTED)


def test_errors_are_reported_not_raised_in_c():
    with pytest.raises(fh.FoError) as e:
        fh.m("A / ", A=4)
    assert e.value.status == -1 and "expected a number" in str(e.value)
    with pytest.raises(fh.FoError):
        fh.sequence("{not json", fh.m("A", A=2))


def test_null_runtime_is_invalid():
    lib = ctypes.CDLL(str(fh.LIB_PATH))
    lib.fo_runtime_synchronize.argtypes = [ctypes.c_void_p]
    assert lib.fo_runtime_synchronize(None) == -1
    lib.fo_buffer_free.argtypes = [ctypes.c_void_p]
    lib.fo_buffer_free(None)  # no-op
    lib.fo_runtime_free.argtypes = [ctypes.c_void_p]
    lib.fo_runtime_free(None)  # no-op


def test_zero_counts_in_mappings_are_rejected():
    # a zero stride / size / modulo would divide by zero in the resolver: refused at parse time
    zero_stride = '{"Stride":{"stride":0,"inner":{"Symbol":{"symbol":"A","size":4}}}}'
    with pytest.raises(fh.FoError, match="must be positive"):
        fh.sequence(zero_stride, fh.m("A", A=4))
    with pytest.raises(fh.FoError, match="must be positive"):
        fh.sequence('{"Symbol":{"symbol":"A","size":0}}', fh.m("A", A=4))
    with pytest.raises(fh.FoError, match="must be positive"):
        fh.m("A / 0", A=4)
    with pytest.raises(fh.FoError, match="must be positive"):
        fh.m("A % 0", A=4)


def test_oversized_mappings_are_rejected():
    # counts and wire sizes above 2^48 would overflow the resolver's int64 weights and strides
    # (found by the sanitizer harness): refused where the mapping enters
    huge = '{"Symbol":{"symbol":"A","size":%d}}' % (2 ** 49)
    with pytest.raises(fh.FoError, match="exceeds 2"):
        fh.sequence(huge, fh.m("A", A=4))
    pair = ('{"Pair":{"left":{"Symbol":{"symbol":"A","size":%d}},"right":{"Symbol":{"symbol":"B","size":%d}}}}'
            % (2 ** 30, 2 ** 30))
    with pytest.raises(fh.FoError, match="exceeds 2"):
        fh.sequence(pair, fh.m("A", A=4))
    with pytest.raises(fh.FoError, match="2\\^48"):
        fh.m("A, B", A=2 ** 30, B=2 ** 30)
    assert fh.sequence(fh.m("A, B", A=2 ** 24, B=2 ** 24), fh.m("A, B", A=2 ** 24, B=2 ** 24))  # 2^48 itself is fine
