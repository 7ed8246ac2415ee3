"""GPU parity of the 4-bit stream types (i4, f4e2m1) through the C ABI, bit exact.

A 4-bit stream packs two elements per byte, element 2k in the low nibble of byte k. The casts
i4 <-> i32 and the f4e2m1 -> f8e4m3 / f8e5m2 table lookups run as maps over element pairs; an i4
contraction unpacks both operands to i8 (exact) and runs the i8 paths (MFMA or the generic fold),
an i4 result narrowing each i32 cell to its low nibble. Integer results are exact in any order,
so every comparison here is bit for bit.
"""
import numpy as np
import pytest

import furiosa_hip as fh
from oracle import emulator as emu
from oracle import mapping_ref as mr
from test_gpu_storage import CHAIN_AXES, CHAINS
from test_mapping_resolver import PAIRS

pytestmark = pytest.mark.gpu

I32, I4, F4E2M1, F8E4M3, F8E5M2 = fh.I32, fh.I4, fh.F4E2M1, fh.F8E4M3, fh.F8E5M2


def gpu_map(rt, x, src_t, dst_t, n, code):
    s = rt.upload(x)
    d = rt.alloc(n // 2 if dst_t in (I4, F4E2M1) else n * np.dtype(fh.NP_DTYPE[dst_t]).itemsize)
    rt.map(d, dst_t, s, src_t, n, fh.op(code))
    return d.read(fh.NP_DTYPE[dst_t])


@pytest.mark.parametrize("t", [F8E4M3, F8E5M2], ids=["e4m3", "e5m2"])
def test_f4e2m1_table_lookup_every_pair(rt, t):
    x = np.arange(256, dtype=np.uint8)  # every pair of codes
    want = emu.map_(x, F4E2M1, t, fh.OP["TABLE_LOOKUP"])
    assert np.array_equal(gpu_map(rt, x, F4E2M1, t, 512, "TABLE_LOOKUP"), want)


def test_i4_casts(rt):
    rng = np.random.default_rng(70)
    w = rng.integers(-2 ** 31, 2 ** 31 - 1, 100_000, dtype=np.int64).astype(np.int32)
    want = emu.map_(w, I32, I4, fh.OP["CAST"])
    assert np.array_equal(gpu_map(rt, w, I32, I4, len(w), "CAST"), want)
    b = rng.integers(0, 256, 50_001, dtype=np.uint8)
    want = emu.map_(b, I4, I32, fh.OP["CAST"])
    assert np.array_equal(gpu_map(rt, b, I4, I32, 2 * len(b), "CAST"), want)
    assert np.array_equal(gpu_map(rt, b, I4, I4, 2 * len(b), "CAST"), b)


def test_4bit_errors(rt):
    x, y = rt.upload(np.zeros(64, np.uint8)), rt.alloc(1024)
    with pytest.raises(fh.FoError, match="even"):
        rt.map(y, I32, x, I4, 7, fh.op("CAST"))
    for dst_t, src_t, code in [(fh.I8, I4, "CAST"), (fh.F32, F4E2M1, "CAST"), (fh.BF16, F4E2M1, "TABLE_LOOKUP"),
                               (I32, I4, "ADD_FXP")]:
        with pytest.raises(fh.FoError):
            rt.map(y, dst_t, x, src_t, 8, fh.op(code))
    with pytest.raises(fh.FoError, match="reads past"):  # 129 nibbles from a 128-nibble buffer
        rt.transpose(y, x, I4, fh.m("A", A=129), fh.m("A", A=129))


# ---- 4-bit relayouts: Backend::transpose over a packed stream (storage/buf.rs:56-80, 257-313) ------
# Each case runs on the unpacked elements in the oracle and is packed back; a destination whose
# element count is odd has a pad nibble, and every nibble the relayout does not write (dead cells,
# cells outside a window, the pad) must keep the random value the destination started with.

def i4_stream(rng, n):
    """n random i4 elements, packed (an odd count gets a random pad nibble)."""
    return rng.integers(0, 256, (n + 1) // 2, dtype=np.uint8)


def i4_want(init, src, n_dst, n_src, fn):
    cells = emu.unpack_i4(init)
    cells[:n_dst] = fn(cells[:n_dst].copy(), emu.unpack_i4(src)[:n_src])
    return emu.pack_nibbles(cells)


@pytest.mark.parametrize("case", PAIRS, ids=[f"{c[1]} -> {c[2]}" for c in PAIRS])
def test_i4_transpose_pairs(rt, case):
    sizes, a, b = case
    rng = np.random.default_rng(74)
    so, do = mr.parse(a, sizes), mr.parse(b, sizes)
    ns, nd = mr.size(so), mr.size(do)
    src, init = i4_stream(rng, ns), i4_stream(rng, nd)
    want = i4_want(init, src, nd, ns, lambda d, s_: emu.transpose(d, s_, so, do))
    d = rt.upload(init)
    rt.transpose(d, rt.upload(src), I4, fh.m(a, **sizes), fh.m(b, **sizes), allow_broadcast=True)
    assert np.array_equal(d.read(np.uint8), want)


@pytest.mark.parametrize("case", range(len(CHAINS)), ids=[" -> ".join(c[0]) for c in CHAINS])
def test_i4_transpose_chain(rt, case):
    views, bc = CHAINS[case]
    rng = np.random.default_rng(75 + case)
    parsed = [mr.parse(v, CHAIN_AXES) for v in views]
    ns, nd = mr.size(parsed[0]), mr.size(parsed[-1])
    src, init = i4_stream(rng, ns), i4_stream(rng, nd)
    want = i4_want(init, src, nd, ns, lambda d, s_: emu.transpose_chain(d, s_, parsed))
    d = rt.upload(init)
    rt.transpose_chain(d, rt.upload(src), I4, [fh.m(v, **CHAIN_AXES) for v in views], bc)
    assert np.array_equal(d.read(np.uint8), want)


def test_i4_transpose_odd_windows(rt):
    """Windows that start on an odd element: the first and last bytes are shared with cells the
    relayout must not touch."""
    s = dict(A=3, B=7)
    rng = np.random.default_rng(76)
    full, row = mr.parse("A, B", s), mr.parse("B", s)
    # a row into the middle of a [3, 7] storage: elements 7 .. 13 (bytes 3 .. 6, both ends shared)
    src, init = i4_stream(rng, 7), i4_stream(rng, 21)
    want = i4_want(init, src, 21, 7, lambda d, s_: emu.transpose(d, s_, row, row, dst_map=full, dst_offset={"A": 1}))
    d = rt.upload(init)
    rt.transpose(d, rt.upload(src), I4, fh.m("B", **s), fh.m("B", **s), dst_map=fh.m("A, B", **s),
                 dst_offset={"A": 1})
    assert np.array_equal(d.read(np.uint8), want)
    # the middle row of a [3, 7] storage (elements 7 .. 13, starting in a byte's high nibble) into
    # a 7-cell stream with a pad nibble
    src, init = i4_stream(rng, 21), i4_stream(rng, 7)
    want = i4_want(init, src, 7, 21, lambda d, s_: emu.transpose(d, s_, row, row, src_map=full, src_offset={"A": 1}))
    d = rt.upload(init)
    rt.transpose(d, rt.upload(src), I4, fh.m("B", **s), fh.m("B", **s), src_map=fh.m("A, B", **s),
                 src_offset={"A": 1})
    assert np.array_equal(d.read(np.uint8), want)


def run_gemm(rt, out_t, Mm, Nn, Kk, seed):
    rng = np.random.default_rng(seed)
    a = emu.pack_nibbles(rng.integers(-8, 8, Mm * Kk))
    b = emu.pack_nibbles(rng.integers(-8, 8, Nn * Kk))
    s = dict(M=Mm, N=Nn, K=Kk)
    out = rt.alloc(Mm * Nn * 4 if out_t == I32 else Mm * Nn // 2)
    rt.contraction(out, rt.upload(a), rt.upload(b), I4, out_t, fh.m("M / 8, M % 8, K", **s), fh.m("N, K", **s),
                   fh.m("M / 8, M % 8, N, K", **s), fh.m("M / 8, M % 8, N", **s))
    got = out.read(np.int32 if out_t == I32 else np.uint8)
    return a, b, (got if out_t == I32 else emu.unpack_i4(got)).reshape(Mm, Nn)


@pytest.mark.parametrize("out_t", [I32, I4], ids=["i32", "i4"])
def test_i4_gemm_whole(rt, out_t):
    Mm, Nn, Kk = 256, 320, 512
    a, b, got = run_gemm(rt, out_t, Mm, Nn, Kk, 71)
    want = emu.gemm_rows(a, b, Mm, Nn, Kk, 0, Mm, out_t=I32, in_t=I4).reshape(Mm, Nn)
    if out_t == I4:
        want = ((want.astype(np.int64) + 8) % 16) - 8
    assert np.array_equal(got, want)


def test_i4_gemm_large_ragged(rt):
    Mm, Nn, Kk = 2056, 4000, 208
    a, b, got = run_gemm(rt, I32, Mm, Nn, Kk, 72)
    for r0 in (0, 255, 1031, Mm - 3):
        want = emu.gemm_rows(a, b, Mm, Nn, Kk, r0, r0 + 3, out_t=I32, in_t=I4).reshape(3, Nn)
        assert np.array_equal(got[r0:r0 + 3], want)


def test_zero_point_sub(rt):
    rng = np.random.default_rng(73)
    b = rng.integers(0, 256, 4096, dtype=np.uint8)
    for zp in (-8, 3, 7):
        want = emu.map_(b, I4, I32, fh.OP["ZERO_POINT_SUB"], 0, zp & 0xFFFFFFFF)
        d = rt.alloc(8192 * 4)
        rt.map(d, I32, rt.upload(b), I4, 8192, fh.op("ZERO_POINT_SUB", 0, zp))
        assert np.array_equal(d.read(np.int32), want)
    a = rng.integers(-128, 128, 5000).astype(np.int8)
    for zp in (-128, 0, 127):
        want = emu.map_(a, fh.I8, I32, fh.OP["ZERO_POINT_SUB"], 0, zp & 0xFFFFFFFF)
        d = rt.alloc(5000 * 4)
        rt.map(d, I32, rt.upload(a), fh.I8, 5000, fh.op("ZERO_POINT_SUB", 0, zp))
        assert np.array_equal(d.read(np.int32), want)
    x, y = rt.upload(np.zeros(64, np.uint8)), rt.alloc(1024)
    with pytest.raises(fh.FoError, match="quantized range"):
        rt.map(y, I32, x, I4, 8, fh.op("ZERO_POINT_SUB", 0, 8))
    with pytest.raises(fh.FoError, match="quantized range"):
        rt.map(y, I32, x, fh.I8, 8, fh.op("ZERO_POINT_SUB", 0, -129))
