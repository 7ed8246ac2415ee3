"""GPU parity of the 8-bit float types (f8e4m3, f8e5m2) through the C ABI.

Casts and table lookups are bit exact against the oracle over every code and over a set of f32
inputs that holds every rounding tie. The contraction's generic path folds in the emulator's
order and is bit exact too (here, and over the padded / permuted / broadcast mappings of
test_gpu_storage.py's contraction cases). The MFMA path (v_mfma_f32_32x32x64_f8f6f4) multiplies exactly but
sums each 64-wide k block at reduced internal precision (measured: about 2e-5 of sum |a b| on
average per instruction, 1.6e-4 at most), so it is held to a bound per output cell:
|got - ref| <= 2^-11 * sum_k |a_k b_k| for an f32 result, and for an 8-bit result the code must lie
between the narrows of ref -+ that bound (the narrow is monotone), i.e. one code step at most
where the exact sum sits near a rounding boundary.
"""
import numpy as np
import pytest

import furiosa_hip as fh
from oracle import emulator as emu
from oracle import mapping_ref as mr
from test_gpu_storage import gpu_map

pytestmark = pytest.mark.gpu

F32, BF16, F8E4M3, F8E5M2 = fh.F32, fh.BF16, fh.F8E4M3, fh.F8E5M2
FORMATS = [F8E4M3, F8E5M2]
IDS = ["e4m3", "e5m2"]
ALL_CODES = np.arange(256, dtype=np.uint8)


def encode_inputs(rng, t):
    """f32 inputs covering every class and every tie: random bit patterns, the midpoints between
    consecutive codes and their f32 neighbours, saturation and the e5m2 subnormal cap band."""
    f = emu.f8_to_f32(ALL_CODES, t).astype(np.float64)
    fin = np.sort(np.unique(f[np.isfinite(f)]))
    mids = ((fin[1:] + fin[:-1]) / 2).astype(np.float32)
    up = np.nextafter(mids, np.float32(np.inf))
    dn = np.nextafter(mids, np.float32(-np.inf))
    rnd = rng.integers(0, 2 ** 32, 200_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    near = (rng.standard_normal(100_000) * np.exp2(rng.integers(-20, 18, 100_000))).astype(np.float32)
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 448.0, 464.0, 480.0, 57344.0, 61440.0, 65536.0,
                        3.5 * 2.0 ** -16, 3.99 * 2.0 ** -16, 1e-45, -1e-45, 1e-39], np.float32)
    return np.concatenate([mids, -mids, up, dn, -up, -dn, rnd, near, special]).astype(np.float32)


@pytest.mark.parametrize("t", FORMATS, ids=IDS)
def test_f8_decode_every_code(rt, t):
    want = emu.map_(ALL_CODES, t, F32, fh.OP["CAST"])
    got = gpu_map(rt, ALL_CODES, t, F32, fh.op("CAST"))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("t", FORMATS, ids=IDS)
def test_f8_table_lookup_every_code(rt, t):
    want = emu.map_(ALL_CODES, t, BF16, fh.OP["TABLE_LOOKUP"])
    got = gpu_map(rt, ALL_CODES, t, BF16, fh.op("TABLE_LOOKUP"))
    assert np.array_equal(got, want)


@pytest.mark.parametrize("t", FORMATS, ids=IDS)
def test_f8_encode_every_tie(rt, t):
    x = encode_inputs(np.random.default_rng(60), t)
    want = emu.map_(x, F32, t, fh.OP["CAST"])
    got = gpu_map(rt, x, F32, t, fh.op("CAST"))
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, f"{bad.size} differ, first x={x[bad[0]]!r} got {got[bad[0]]:#x} want {want[bad[0]]:#x}"


@pytest.mark.parametrize("t", FORMATS, ids=IDS)
def test_f8_identity_cast_keeps_bits(rt, t):
    got = gpu_map(rt, ALL_CODES, t, t, fh.op("CAST"))
    assert np.array_equal(got, ALL_CODES)


def test_f8_non_reference_casts_are_errors(rt):
    x = rt.upload(np.zeros(16, np.uint8))
    y = rt.alloc(64)
    for dst_t, src_t, code in [(F8E4M3, BF16, "CAST"), (BF16, F8E4M3, "CAST"), (F8E4M3, F8E5M2, "CAST"),
                               (F32, F8E4M3, "EXP"), (F32, BF16, "TABLE_LOOKUP")]:
        with pytest.raises(fh.FoError):
            rt.map(y, dst_t, x, src_t, 8, fh.op(code))
    with pytest.raises(fh.FoError):
        rt.zip_with(y, F8E4M3, x, x, F8E4M3, 8, fh.op("ADD_F"))


def f8_operands(rng, t, n, scale=1.0):
    return emu.f32_to_f8((rng.standard_normal(n) * scale).astype(np.float32), t)


def run_gemm(rt, t, out_t, Mm, Nn, Kk, seed):
    rng = np.random.default_rng(seed)
    a, b = f8_operands(rng, t, Mm * Kk), f8_operands(rng, t, Nn * Kk)
    s = dict(M=Mm, N=Nn, K=Kk)
    ob = 4 if out_t == F32 else 1
    out = rt.alloc(Mm * Nn * ob)
    rt.contraction(out, rt.upload(a), rt.upload(b), t, out_t, fh.m("M / 8, M % 8, K", **s), fh.m("N, K", **s),
                   fh.m("M / 8, M % 8, N, K", **s), fh.m("M / 8, M % 8, N", **s))
    return a, b, out.read(np.float32 if out_t == F32 else np.uint8).reshape(Mm, Nn)


def abs_products(a, b, t, Kk, rows):
    av = np.abs(emu.f8_to_f32(a, t).astype(np.float64)).reshape(-1, Kk)[rows]
    bv = np.abs(emu.f8_to_f32(b, t).astype(np.float64)).reshape(-1, Kk)
    return av @ bv.T


def check_mfma_rows(a, b, got, t, out_t, Mm, Nn, Kk, rows):
    bound = 2.0 ** -11 * abs_products(a, b, t, Kk, rows)
    ref = np.stack([emu.gemm_rows(a, b, Mm, Nn, Kk, r, r + 1, out_t=F32, in_t=t) for r in rows]).astype(np.float64)
    if out_t == F32:
        err = np.abs(got[rows].astype(np.float64) - ref)
        assert np.all(err <= bound), f"worst excess {(err - bound).max()}"
    else:
        lo = emu.f8_to_f32(emu.f32_to_f8((ref - bound).astype(np.float32).ravel(), t), t).reshape(ref.shape)
        hi = emu.f8_to_f32(emu.f32_to_f8((ref + bound).astype(np.float32).ravel(), t), t).reshape(ref.shape)
        gv = emu.f8_to_f32(got[rows].ravel(), t).reshape(ref.shape)
        assert np.all((gv >= lo) & (gv <= hi)), f"{np.sum(~((gv >= lo) & (gv <= hi)))} codes outside the bracket"
        exact = emu.f32_to_f8(ref.astype(np.float32).ravel(), t).reshape(ref.shape)
        assert np.mean(got[rows] == exact) > 0.99  # off-by-one codes only at rounding boundaries


@pytest.mark.parametrize("t", FORMATS, ids=IDS)
@pytest.mark.parametrize("out", ["f32", "f8"])
def test_f8_gemm_mfma_whole(rt, t, out):
    Mm, Nn, Kk = 256, 320, 512
    out_t = F32 if out == "f32" else t
    a, b, got = run_gemm(rt, t, out_t, Mm, Nn, Kk, 61)
    check_mfma_rows(a, b, got, t, out_t, Mm, Nn, Kk, np.arange(Mm))


@pytest.mark.parametrize("t", FORMATS, ids=IDS)
def test_f8_gemm_mfma_large_ragged(rt, t):
    # 256x256 tiles with partial last tiles in M and N, and a K that ends inside a stage.
    Mm, Nn, Kk = 2056, 4000, 208
    for out_t in (F32, t):
        a, b, got = run_gemm(rt, t, out_t, Mm, Nn, Kk, 62)
        check_mfma_rows(a, b, got, t, out_t, Mm, Nn, Kk, np.array([0, 1, 255, 256, 1031, 2048, Mm - 1]))


@pytest.mark.parametrize("t", FORMATS, ids=IDS)
@pytest.mark.parametrize("out", ["f32", "f8"])
def test_f8_contraction_generic_bit_exact(rt, t, out):
    # K = 100 is not a multiple of 16 bytes: the thread-per-cell fold in the emulator's order.
    Mm, Nn, Kk = 48, 40, 100
    out_t = F32 if out == "f32" else t
    rng = np.random.default_rng(63)
    a, b = f8_operands(rng, t, Mm * Kk), f8_operands(rng, t, Nn * Kk)
    s = dict(M=Mm, N=Nn, K=Kk)
    maps = (fh.m("M / 8, M % 8, K", **s), fh.m("N, K", **s), fh.m("M / 8, M % 8, N, K", **s),
            fh.m("M / 8, M % 8, N", **s))
    want = emu.contraction(a, b, t, out_t, *(mr.parse(x, s) for x in
                                               ("M / 8, M % 8, K", "N, K", "M / 8, M % 8, N, K", "M / 8, M % 8, N")))
    out_buf = rt.alloc(Mm * Nn * (4 if out_t == F32 else 1))
    rt.contraction(out_buf, rt.upload(a), rt.upload(b), t, out_t, *maps)
    got = out_buf.read(np.float32 if out_t == F32 else np.uint8)
    assert np.array_equal(got.view(np.uint8), want.view(np.uint8))
