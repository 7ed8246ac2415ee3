"""Replays of the Backend call streams that reference kernels issue, through the C ABI.

An unchanged `#[device]` kernel reaches this backend only as a sequence of seam calls: every DMA
and stage change is a `Tensor::transpose` into a fresh zeroed storage (`to_dm` / `to_hbm`,
tensor/memory.rs:365-422; fetch, collect, commit), and a contraction is `contract_outer`'s two
`map(widen)` calls followed by `contract_lane`'s `contraction_prewidened` onto
[Chip, Cluster, Slice, Lane, Time, Packet] (engine/contraction/outer/mod.rs:145-163,
engine/contraction/lane.rs:60-79), a `transpose(false)` and the cast. The mappings below are the
ones those stages build from each kernel's type parameters.

  * base-template/src/kernel/gemm_kernel.rs:11-50 (I = J = 512, K = 64; Slice m![I / 32, J / 32],
    Lane m![J % 8], Cluster m![1 # 2]): the contraction has 1024 batch cells (I / 32, J / 32 and the
    DM copies along J / 8 % 4), rows I % 32, columns J % 8 and a padded cluster axis -- the
    wheel-decoded MFMA kernel runs it on the bf16 sources of the widened operands.
  * furiosa-opt-examples/src/mnist/mod.rs:8-34 (fc1, X = 800, H = 256): 256 batch cells of one
    800-long dot product each (M = N = 1), which the generic fold runs, bit-exact, on the bf16
    sources.
  * furiosa-opt-examples/src/contract_element_types.rs:24-232, one single-flit contraction per
    engine input type (i8, f8e4m3, the i8 zero-point subtraction, i4, f8e5m2, bf16; A = R = 8,
    Cluster m![1 # 2], Slice m![1 # 256], Lane m![R]): every stage, the 4-bit ones included, as the
    seam sees it, checked against the integer matmul the reference's answer key computes by hand
    (tests/contract_element_types_answer_tests.rs:19-54) and against the oracle.
"""
import numpy as np
import pytest

import furiosa_hip as fh
from oracle import emulator as emu
from oracle import mapping_ref as mr
from test_gpu_storage import close

pytestmark = pytest.mark.gpu

BF16, F32 = fh.BF16, fh.F32


def mapping_size(js):
    """Mapping::size (furiosa-mapping-types/src/lib.rs:208-219) of a MappingSerde JSON string."""
    import json

    def size(node):
        (tag, b), = node.items()
        if tag == "Symbol":
            return b["size"]
        if tag == "Stride":
            return size(b["inner"]) // b["stride"]
        if tag == "Pair":
            return size(b["left"]) * size(b["right"])
        return b[{"Modulo": "modulo", "Resize": "resize", "Padding": "padding", "Broadcast": "size"}[tag]]
    return size(json.loads(js))


def relayout(rt, src, sizes, views, allow_broadcast=None, dtype=BF16):
    """A chain of Tensor::transpose calls (each into a fresh zeroed storage of the next view)."""
    ms = [fh.m(v, **sizes) for v in views]
    out = rt.upload(np.zeros(mapping_size(ms[-1]), fh.NP_DTYPE[dtype]))
    rt.transpose_chain(out, src, dtype, ms, allow_broadcast)
    return out


def widen(rt, src, n):
    """contract_outer's `map(|v| v.cast())` to the f32 accumulator."""
    out = rt.alloc(n * 4)
    rt.map(out, F32, src, BF16, n, fh.op("CAST"))
    return out


GEMM = dict(I=512, J=512, K=64)
CHIP_CLUSTER = "1, 1 # 2"


def gemm_kernel_stream(rt, a, b):
    s = GEMM
    # to_dm: the operands spread over 256 slices (A copied along J / 32, B along I / 32)
    a_dm = relayout(rt, a, s, ["I, K", f"{CHIP_CLUSTER}, I / 32, J / 32, I % 32, K"], [True])
    b_dm = relayout(rt, b, s, ["J, K", f"{CHIP_CLUSTER}, I / 32, J / 32, J % 32, K"], [True])
    # sub: fetch -> collect -> to_trf of B: TRF [Chip, Cluster, Slice, Lane = J % 8, J / 8 % 4, K]
    trf = relayout(rt, b_dm, s, [f"{CHIP_CLUSTER}, I / 32, J / 32, J % 32, K",
                                 f"{CHIP_CLUSTER}, I / 32, J / 32, J % 8, J / 8 % 4, K",
                                 f"{CHIP_CLUSTER}, I / 32, J / 32, J % 8, J / 8 % 4, K / 16, K % 16",
                                 f"{CHIP_CLUSTER}, I / 32, J / 32, J % 8, J / 8 % 4, K"])
    # main: fetch (J / 8 % 4 broadcast into time) -> collect of A
    lhs_view = f"{CHIP_CLUSTER}, I / 32, J / 32, I % 32, J / 8 % 4, K / 16, K % 16"
    lhs = relayout(rt, a_dm, s, [f"{CHIP_CLUSTER}, I / 32, J / 32, I % 32, K",
                                 f"{CHIP_CLUSTER}, I / 32, J / 32, I % 32, J / 8 % 4, K", lhs_view], [True, False])
    rhs_view = f"{CHIP_CLUSTER}, I / 32, J / 32, J % 8, J / 8 % 4, K"
    n_l, n_r = mapping_size(fh.m(lhs_view, **s)), mapping_size(fh.m(rhs_view, **s))
    lw, rw = widen(rt, lhs, n_l), widen(rt, trf, n_r)
    pre = f"{CHIP_CLUSTER}, I / 32, J / 32, J % 8, I % 32, J / 8 % 4, K / 32, K % 32"
    out_view = f"{CHIP_CLUSTER}, I / 32, J / 32, J % 8, I % 32, J / 8 % 4"
    acc = rt.upload(np.full(mapping_size(fh.m(out_view, **s)), 7.0, np.float32))  # dead cells must become 0
    rt.contraction(acc, lw, rw, F32, F32, *(fh.m(t, **s) for t in (lhs_view, rhs_view, pre, out_view)))
    raw = acc.read(np.float32)
    # transpose(false) to [Chip, Cluster, Slice, OutTime, OutPacket], the cast, commit, to_hbm
    ct_view = f"{CHIP_CLUSTER}, I / 32, J / 32, I % 32, J / 8 % 4, J % 8"
    acc_t = relayout(rt, acc, s, [out_view, ct_view], dtype=F32)
    n_ct = mapping_size(fh.m(ct_view, **s))
    cast = rt.alloc(n_ct * 2)
    rt.map(cast, BF16, acc_t, F32, n_ct, fh.op("CAST"))
    c = relayout(rt, cast, s, [ct_view, f"{CHIP_CLUSTER}, I / 32, J / 32, I % 32, J % 32", "I, J"])
    return raw, c.read(np.uint16)


def test_gemm_kernel_seam_stream(rt):
    s = GEMM
    rng = np.random.default_rng(40)
    a = emu.f32_to_bf16(rng.standard_normal(512 * 64).astype(np.float32))
    b = emu.f32_to_bf16(rng.standard_normal(512 * 64).astype(np.float32))
    acc, c = gemm_kernel_stream(rt, rt.upload(a), rt.upload(b))
    # The emulator's sequential f32 fold (gemm_rows: lhs [I, K], rhs [J, K]) with one bf16 narrow.
    want = emu.bf16_to_f32(emu.gemm_rows(a, b, 512, 512, 64, 0, 512)).reshape(512, 512)
    close(emu.bf16_to_f32(c).reshape(512, 512), want)
    want_f32 = emu.gemm_rows(a, b, 512, 512, 64, 0, 512, out_t=F32).reshape(512, 512)
    # the f32 contraction result in its own layout [cluster(2, 1 live), I/32, J/32, J%8, I%32, J/8%4]
    got = acc.reshape(2, 16, 16, 8, 32, 4)[0]
    got = got.transpose(0, 3, 1, 4, 2).reshape(512, 512)  # rows I/32 I%32, cols J/32 J/8%4 J%8
    close(got, want_f32, rel=1e-5)
    assert np.all(acc.reshape(2, -1)[1] == 0)  # the padded cluster half was zeroed


def test_mnist_fc1_seam_stream(rt):
    s = dict(X=800, H=256)
    rng = np.random.default_rng(41)
    x = emu.f32_to_bf16(rng.uniform(0, 1, 800).astype(np.float32))
    w1 = emu.f32_to_bf16((0.05 * rng.standard_normal(256 * 800)).astype(np.float32))
    w_dm = relayout(rt, rt.upload(w1), s, ["H, X", f"{CHIP_CLUSTER}, H, X"], [True])
    x_dm = relayout(rt, rt.upload(x), s, ["X", f"{CHIP_CLUSTER}, H, X"], [True])
    trf = relayout(rt, x_dm, s, [f"{CHIP_CLUSTER}, H, X", f"{CHIP_CLUSTER}, H, X / 16, X % 16",
                                 f"{CHIP_CLUSTER}, H, X"])
    lhs_view = f"{CHIP_CLUSTER}, H, X / 16, X % 16"
    lhs = relayout(rt, w_dm, s, [f"{CHIP_CLUSTER}, H, X", lhs_view])
    n = mapping_size(fh.m(lhs_view, **s))
    lw, rw = widen(rt, lhs, n), widen(rt, trf, n)
    out_view = f"{CHIP_CLUSTER}, H"
    acc = rt.upload(np.full(512, 3.0, np.float32))  # dead cells must become 0
    rt.contraction(acc, lw, rw, F32, F32, fh.m(lhs_view, **s), fh.m(f"{CHIP_CLUSTER}, H, X", **s),
                   fh.m(f"{CHIP_CLUSTER}, H, X / 32, X % 32", **s), fh.m(out_view, **s))
    cast = rt.alloc(512 * 2)
    rt.map(cast, BF16, acc, F32, 512, fh.op("CAST"))
    h = cast.read(np.uint16)
    want = emu.gemm_rows(x, w1, 1, 256, 800, 0, 1)  # h = bf16(sum_k f32 x f32 w1), the sequential fold
    assert np.array_equal(h[:256], want)             # bit-exact
    assert np.all(h[256:] == 0)                       # dead cluster half


def test_widen_record_dropped_when_the_source_is_rewritten(rt):
    """After map(widen) the f32 copy is the operand; rewriting its bf16 source afterwards must not
    change what the contraction reads."""
    s = dict(M=64, N=64, K=64)
    rng = np.random.default_rng(42)
    a = emu.f32_to_bf16(rng.standard_normal(64 * 64).astype(np.float32))
    b = emu.f32_to_bf16(rng.standard_normal(64 * 64).astype(np.float32))
    da, db = rt.upload(a), rt.upload(b)
    la, lb = widen(rt, da, 64 * 64), widen(rt, db, 64 * 64)
    da.write(np.zeros_like(a))  # the source changes after the widen
    maps = [fh.m(t, **s) for t in ("M, K", "N, K", "M, N, K", "M, N")]
    out = rt.alloc(64 * 64 * 4)
    rt.contraction(out, la, lb, F32, F32, *maps)
    want = emu.gemm_rows(a, b, 64, 64, 64, 0, 64, out_t=F32)
    assert np.array_equal(out.read(np.float32), want)  # the generic fold over the f32 copies: exact


def test_widened_contraction_matches_the_f32_fold(rt):
    """contraction_prewidened over two widened bf16 operands whose k axis is not contiguous in lhs
    (lhs stored K-major), so no GEMM or GEMV kernel takes it: the generic fold reads the narrow
    sources (kept alive here, so the widens stay pending) and is bit-exact with the f32 fold."""
    s = dict(M=4, N=96, K=160)
    rng = np.random.default_rng(43)
    a = emu.f32_to_bf16(rng.standard_normal(4 * 160).astype(np.float32))
    b = emu.f32_to_bf16(rng.standard_normal(96 * 160).astype(np.float32))
    sa, sb = rt.upload(np.ascontiguousarray(a.reshape(4, 160).T).ravel()), rt.upload(b)
    la, lb = widen(rt, sa, 4 * 160), widen(rt, sb, 96 * 160)
    out = rt.alloc(4 * 96 * 4)
    rt.contraction(out, la, lb, F32, F32, *(fh.m(t, **s) for t in ("K, M", "N, K", "M, N, K", "M, N")))
    assert np.array_equal(out.read(np.float32), emu.gemm_rows(a, b, 4, 96, 160, 0, 4, out_t=F32))


# ---- contract_element_types.rs: one single-flit contract_outer per engine input type -----------
# (kernel, element type, packet axis K, accumulator). K is one 32-byte flit of the type.
ELEMENT_KERNELS = [
    ("i8_contract", fh.I8, 32, fh.I32),                    # contract_element_types.rs:24-57
    ("f8e4m3_contract", fh.F8E4M3, 32, F32),               # :59-90
    ("zero_point_sub_contract", fh.I8, 32, fh.I32),        # :92-128, zero point 3
    ("i4_contract", fh.I4, 64, fh.I32),                    # :130-163
    ("f8e5m2_contract", fh.F8E5M2, 32, F32),               # :165-196
    ("bf16_contract", BF16, 16, F32),                      # :198-232
]
ELEM_CC = "1, 1 # 2, 1 # 256"  # [Chip, Cluster, Slice] = m![1], m![1 # 2], m![1 # 256]
ZERO_POINT = 3


def nbytes_of(t, n):
    return (n + 1) // 2 if t == fh.I4 else n * np.dtype(fh.NP_DTYPE[t]).itemsize


def relayout_any(rt, src, sizes, views, t):
    """relayout() for any element type, 4-bit streams included."""
    ms = [fh.m(v, **sizes) for v in views]
    out = rt.upload(np.zeros(nbytes_of(t, mapping_size(ms[-1])), np.uint8))
    rt.transpose_chain(out, src, t, ms)
    return out


def encode(t, vals):
    """Integer values in [-8, 8) -> the kernel's storage encoding of them (exact in every type)."""
    if t == fh.I4:
        return emu.pack_nibbles(vals)
    if t == fh.I8:
        return vals.astype(np.int8)
    if t == BF16:
        return emu.f32_to_bf16(vals.astype(np.float32))
    return emu.f32_to_f8(vals.astype(np.float32), t)


def element_kernel_stream(rt, name, t, K, acc_t, x, w):
    """The seam calls of one contract_element_types kernel on encoded inputs x [A, K], w [R, K]."""
    s = dict(A=8, R=8, K=K)
    dm_a, dm_r = f"{ELEM_CC}, A, K", f"{ELEM_CC}, R, K"
    # to_dm (memory.rs:365-422) of both inputs; the padded cluster and slice cells stay zero
    x_dm = relayout_any(rt, rt.upload(x), s, ["A, K", dm_a], t)
    w_dm = relayout_any(rt, rt.upload(w), s, ["R, K", dm_r], t)
    n_a, n_r = mapping_size(fh.m(dm_a, **s)), mapping_size(fh.m(dm_r, **s))
    # sub: fetch -> fetch_cast::<D> (the identity map) -> collect -> to_trf, TRF [.., Lane = R, K]
    w_f = relayout_any(rt, w_dm, s, [dm_r, dm_r], t)
    w_c = rt.alloc(nbytes_of(t, n_r))
    rt.map(w_c, t, w_f, t, n_r, fh.op("CAST"))
    trf = relayout_any(rt, w_c, s, [dm_r, dm_r, dm_r], t)
    # main: fetch -> fetch_cast (or fetch_zero_point_sub, which widens as it subtracts) -> collect
    x_f = relayout_any(rt, x_dm, s, [dm_a, dm_a], t)
    if name == "zero_point_sub_contract":
        x_c = rt.alloc(n_a * 4)
        rt.map(x_c, fh.I32, x_f, t, n_a, fh.op("ZERO_POINT_SUB", 0, ZERO_POINT))
        lhs = relayout_any(rt, x_c, s, [dm_a, dm_a], fh.I32)
    else:
        x_c = rt.alloc(nbytes_of(t, n_a))
        rt.map(x_c, t, x_f, t, n_a, fh.op("CAST"))
        x_col = relayout_any(rt, x_c, s, [dm_a, dm_a], t)
        lhs = rt.alloc(n_a * 4)  # contract_outer's map(widen) of the stream operand
        rt.map(lhs, acc_t, x_col, t, n_a, fh.op("CAST"))
    rhs = rt.alloc(n_r * 4)      # ... and of the TRF operand
    rt.map(rhs, acc_t, trf, t, n_r, fh.op("CAST"))
    # contract_lane: contraction_prewidened onto [Chip, Cluster, Slice, Lane, Time = A, Packet = 1]
    pre, out_view = f"{ELEM_CC}, R, A, K", f"{ELEM_CC}, R, A"
    acc_np = np.int32 if acc_t == fh.I32 else np.float32
    acc = rt.upload(np.full(mapping_size(fh.m(out_view, **s)), 5, acc_np))  # dead cells must become 0
    rt.contraction(acc, lhs, rhs, acc_t, acc_t, *(fh.m(v, **s) for v in (dm_a, dm_r, pre, out_view)))
    raw = acc.read(acc_np)
    # the lane fold's transpose(false) to [.., A, R], commit_trim, commit, to_hbm [Chip, A, R]
    ct = f"{ELEM_CC}, A, R"
    out = relayout_any(rt, acc, s, [out_view, ct, ct, ct, "1, A, R"], acc_t)
    return raw, out.read(acc_np).reshape(8, 8)


def element_inputs(rng, t, K, lo, hi):
    xv, wv = rng.integers(lo, hi, 8 * K), rng.integers(lo, hi, 8 * K)
    return xv, wv, encode(t, xv), encode(t, wv)


@pytest.mark.parametrize("kernel", ELEMENT_KERNELS, ids=[k[0] for k in ELEMENT_KERNELS])
def test_element_type_kernel_seam_stream(rt, kernel):
    """Inputs in [-8, 8), as the answer key draws them (its SmallRng stream is Rust's, so the
    values here are numpy's, of the same distribution): every product and partial sum is a small
    integer, exact in f32 and i32, so the result is the hand-computed integer matmul
    out[a, r] = sum_k (x[a, k] - zp) * w[r, k] bit for bit, in any order the kernel folds."""
    name, t, K, acc_t = kernel
    rng = np.random.default_rng(42)
    xv, wv, x, w = element_inputs(rng, t, K, -8, 8)
    raw, got = element_kernel_stream(rt, name, t, K, acc_t, x, w)
    zp = ZERO_POINT if name == "zero_point_sub_contract" else 0
    want = (xv.reshape(8, K).astype(np.int64) - zp) @ wv.reshape(8, K).astype(np.int64).T
    assert np.array_equal(got, want.astype(got.dtype))
    # the contraction's own layout [cluster 2, slice 256, R, A]: one live cell, the rest zero
    cells = raw.reshape(2, 256, 8, 8)
    assert np.array_equal(cells[0, 0].T, want.astype(got.dtype))
    assert not cells.reshape(512, 64)[1:].any()


@pytest.mark.parametrize("kernel", ELEMENT_KERNELS, ids=[k[0] for k in ELEMENT_KERNELS])
def test_element_type_kernel_full_range(rt, kernel):
    """Every code of the type (the NaN codes of the 8-bit floats aside): the integer kernels are
    exact; bf16 matches the oracle's sequential f32 fold of the widened operands
    (contraction_prewidened, storage/buf.rs:401-447) to 1e-5; the 8-bit floats run on the f8f6f4
    MFMA, which multiplies exactly but sums each 64-wide k block at reduced internal precision, and
    are held to |got - ref| <= 2^-11 * sum_k |x_k * w_k| per cell (the bound of the f8 GEMM tests)."""
    name, t, K, acc_t = kernel
    rng = np.random.default_rng(43)
    if t in (fh.I8, fh.I4):
        lo, hi = (-128, 128) if t == fh.I8 else (-8, 8)
        xv, wv, x, w = element_inputs(rng, t, K, lo, hi)
        zp = ZERO_POINT if name == "zero_point_sub_contract" else 0
        want = (xv.reshape(8, K).astype(np.int64) - zp) @ wv.reshape(8, K).astype(np.int64).T
        _, got = element_kernel_stream(rt, name, t, K, acc_t, x, w)
        assert np.array_equal(got, want.astype(np.int32))
        return
    if t == BF16:
        x = emu.f32_to_bf16(rng.standard_normal(8 * K).astype(np.float32))
        w = emu.f32_to_bf16(rng.standard_normal(8 * K).astype(np.float32))
        xf, wf = emu.bf16_to_f32(x), emu.bf16_to_f32(w)
    else:
        finite = np.array([c for c in range(256) if np.isfinite(emu.f8_to_f32(np.array([c], np.uint8), t)[0])],
                          np.uint8)
        x, w = rng.choice(finite, 8 * K), rng.choice(finite, 8 * K)
        xf, wf = emu.f8_to_f32(x, t), emu.f8_to_f32(w, t)
    _, got = element_kernel_stream(rt, name, t, K, acc_t, x, w)
    maps = (mr.parse(v, dict(A=8, R=8, K=K)) for v in ("A, K", "R, K", "A, R, K", "A, R"))
    want = emu.contraction(xf, wf, F32, F32, *maps).reshape(8, 8)
    if t == BF16:
        close(got, want, rel=1e-5)
        return
    bound = 2.0 ** -11 * (np.abs(xf.reshape(8, K).astype(np.float64)) @ np.abs(wf.reshape(8, K).astype(np.float64)).T)
    err = np.abs(got.astype(np.float64) - want)
    assert np.all(err <= bound), f"worst excess {(err - bound).max()}"
