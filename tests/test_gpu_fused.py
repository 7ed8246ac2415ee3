"""GPU parity of the fused chains at the configs of BASELINE.json, through the C ABI.

Small shapes are compared whole against the oracle. At the full config shapes every output cell is
checked: against a vectorised numpy restatement of the same chain (f32 reductions in numpy's order,
the reference's rounding points), and a seeded sample against the oracle itself.

Tolerances. A single bf16 narrow after f32 accumulation: |got - ref| <= 1e-2 |ref| + 1e-2 rms(ref)
(`close`, the bar of the reference's transformer tests). The RMSNorm->softmax and attention chains
narrow to bf16 twice in sequence (y then the softmax output; o then o / l), and their f32 reductions
are reassociated on the GPU -- which the emulator's own contract allows (BufStorage::reduce,
storage/buf.rs:316-330) -- so an intermediate that differs in its last f32 bits can move the output
by up to one bf16 ulp per narrow. `close_chain` therefore holds each element to
max(1e-2 |ref| + 1e-2 rms(ref), 2 ulp_bf16(ref)), except a stated fraction of elements; every
element, exceptions included, must lie within a per-element bound derived from the one cause each
chain has:
  * RMSNorm: a reassociated sum of squares moves r by f32 ulps, which can flip any intermediate
    y = bf16(x g / r) by one bf16 ulp; that scales the element's exp by e^(+-ulp(y)) and the row sum
    by at most sum_j p_j (e^ulp(y_j) - 1) (`rmsnorm_bound`);
  * attention: the reference's max is taken over every key before masking (attention.rs:77-95)
    while the kernel scales p by a running max of the visible keys (updated lazily, when a block's
    max exceeds it by more than 8 ln 2), so bf16(p) rounds at a different scale; the shift of the
    weighted sum is at most 2^-8 times the element's weighted value mass (`attention_numpy`).

Every close_chain call records the measured error (max relative error, fraction beyond the 1e-2
bar, worst error in ulps); with FO_PARITY_REPORT set to a file path the records are appended to it
as JSON lines.
"""
import json
import os

import numpy as np
import pytest

import furiosa_hip as fh
from oracle import emulator as emu
from test_gpu_storage import close
from test_oracle_chains import first10_argmax, mnist_key, GOLDEN

pytestmark = pytest.mark.gpu


def bf16_ulp(v):
    a = np.abs(np.asarray(v, np.float64))
    e = np.floor(np.log2(np.where(a > 0, a, 2.0 ** -126)))
    return 2.0 ** (np.maximum(e, -126) - 7)


def report(name, got, ref, **extra):
    """Measured parity of one comparison: max |got - ref| / (|ref| + rms(ref)) (the normalised
    relative error), the fraction beyond 1e-2 |ref| + 1e-2 rms(ref), and the worst error in ulps."""
    got = np.asarray(got, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    rms = np.sqrt(np.mean(ref ** 2)) if ref.size else 0.0
    err = np.abs(got - ref)
    rec = dict(name=name, cells=int(ref.size),
               max_rel=float(np.max(err / (np.abs(ref) + rms + 1e-30))) if ref.size else 0.0,
               frac_beyond_1e2=float(np.mean(err > 1e-2 * np.abs(ref) + 1e-2 * rms)) if ref.size else 0.0,
               max_ulps=float(np.max(err / bf16_ulp(ref))) if ref.size else 0.0, **extra)
    path = os.environ.get("FO_PARITY_REPORT")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps(rec) + "\n")
    return rec


def close_chain(got, ref, hard, frac_beyond=0.0, name=""):
    """Every element within the per-element bound `hard`; at most a fraction `frac_beyond` of them
    beyond max(1e-2 |ref| + 1e-2 rms(ref), 2 ulp_bf16(ref))."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    rms = np.sqrt(np.mean(ref ** 2)) if ref.size else 0.0
    err = np.abs(got - ref)
    base = 1e-2 * np.abs(ref) + 1e-2 * rms
    ulp = bf16_ulp(ref)
    beyond = err > np.maximum(base, 2 * ulp)
    over = err > hard
    report(name, got, ref, frac_beyond_2ulp=float(beyond.mean()), cells_beyond_hard=int(over.sum()),
           worst_err_over_hard=float(np.max(err / np.maximum(hard, 1e-30))) if ref.size else 0.0)
    assert not over.any(), f"{over.sum()} of {over.size} beyond the hard bound; worst {err.max()}"
    assert beyond.mean() <= frac_beyond, f"{beyond.sum()} of {beyond.size} beyond 2 ulps (allowed {frac_beyond})"
    return float(beyond.mean())


SQRT_HEAD_DIM = np.float32(11.313708)  # attention.rs:10


def bf16(rng, n, scale=1.0, loc=0.0):
    return emu.f32_to_bf16((rng.standard_normal(n) * scale + loc).astype(np.float32))


# ---- RMSNorm -> softmax ------------------------------------------------------------------------------


@pytest.mark.parametrize("shape", [(64, 4096), (37, 1024), (5, 1000), (16, 8192), (33, 512), (19, 2048), (3000, 4096)])
def test_rmsnorm_softmax_small(rt, shape):
    rows, cols = shape
    rng = np.random.default_rng(30)
    x, g = bf16(rng, rows * cols), bf16(rng, cols, 0.1, 1.0)
    want = emu.rmsnorm_softmax(x, g, rows, cols, 1e-6)
    out = rt.alloc(rows * cols * 2)
    rt.rmsnorm_softmax(out, rt.upload(x), rt.upload(g), rows, cols, 1e-6)
    close_chain(emu.bf16_to_f32(out.read(np.uint16)).reshape(rows, cols), emu.bf16_to_f32(want).reshape(rows, cols),
                frac_beyond=1e-4, hard=rmsnorm_bound(x, g, rows, cols, 1e-6), name=f"rmsnorm_softmax {rows}x{cols} vs oracle")


@pytest.mark.parametrize("cols", [1024, 2048, 4096, 8192])
@pytest.mark.parametrize("gain_case", ["finite", "inf", "huge"])
def test_rmsnorm_softmax_nonfinite(rt, cols, gain_case):
    """Rows holding +-inf, NaN or a value whose square overflows take the per-element reference path
    (a NaN row stays NaN, an overflowed sum of squares gives the uniform row); so does every row when
    the gain holds inf or a magnitude of 2^121. Rows next to them keep the fast path."""
    rows = 8
    rng = np.random.default_rng(33)
    x = bf16(rng, rows * cols).reshape(rows, cols)
    g = emu.f32_to_bf16(rng.uniform(0.1, 1.0, cols).astype(np.float32))
    special = emu.f32_to_bf16(np.array([np.inf, np.nan, 1e20, -np.inf, 2.0 ** 121], np.float32))
    x[1, 5], x[2, 7], x[3, 0], x[4, 9] = special[:4]
    if gain_case == "inf":
        g[3] = special[0]
    elif gain_case == "huge":
        g[3] = special[4]
    want = emu.bf16_to_f32(emu.rmsnorm_softmax(x.ravel(), g, rows, cols, 1e-6)).reshape(rows, cols)
    out = rt.alloc(rows * cols * 2)
    rt.rmsnorm_softmax(out, rt.upload(x.ravel()), rt.upload(g), rows, cols, 1e-6)
    got = emu.bf16_to_f32(out.read(np.uint16)).reshape(rows, cols)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    fin = ~np.isnan(want)
    assert np.isnan(want[[1, 2, 4]]).all() and fin[[0, 3, 5, 6, 7]].any()
    bound = rmsnorm_bound(x.ravel(), g, rows, cols, 1e-6).reshape(rows, cols)
    assert np.isfinite(bound[fin]).all() or gain_case == "huge"  # 2^121 * x: one y ulp is unbounded
    close_chain(got[fin], want[fin], frac_beyond=1e-4, hard=bound[fin])


@pytest.mark.parametrize("cols", [1024, 4096])
def test_rmsnorm_softmax_subnormal_operands(rt, cols):
    """Subnormal inputs and gains read as zero (float/bf16.rs:16-40), also where a large gain would
    lift a subnormal product into the normal range: a row of subnormals only (y = 0, the uniform
    row), rows mixing them with normal values, and gains up to 2^63 with subnormal gains between."""
    rows = 6
    rng = np.random.default_rng(34)
    x = bf16(rng, rows * cols).reshape(rows, cols)
    sub = rng.integers(1, 0x80, (rows, cols)).astype(np.uint16) | (rng.integers(0, 2, (rows, cols)).astype(np.uint16) << 15)
    x[0] = sub[0]
    x[1:4, ::3] = sub[1:4, ::3]
    g = emu.f32_to_bf16(rng.uniform(0.5, 2.0, cols).astype(np.float32))
    g[::7] = emu.f32_to_bf16(np.float32(2.0 ** 63))
    g[3::11] = rng.integers(1, 0x80, len(g[3::11])).astype(np.uint16)  # subnormal gains
    want = emu.bf16_to_f32(emu.rmsnorm_softmax(x.ravel(), g, rows, cols, 1e-6)).reshape(rows, cols)
    out = rt.alloc(rows * cols * 2)
    rt.rmsnorm_softmax(out, rt.upload(x.ravel()), rt.upload(g), rows, cols, 1e-6)
    got = emu.bf16_to_f32(out.read(np.uint16)).reshape(rows, cols)
    assert np.all(want[0] == want[0, 0])  # the subnormal row is uniform
    bound = rmsnorm_bound(x.ravel(), g, rows, cols, 1e-6).reshape(rows, cols)
    close_chain(got, want, frac_beyond=1e-4, hard=bound)


def bf16r(x):
    """f32 -> bf16 -> f32 with the reference's rounding (float/bf16.rs:28-40)."""
    return emu.bf16_to_f32(emu.f32_to_bf16(np.asarray(x, np.float32)))


def rmsnorm_softmax_numpy(x, g, rows, cols, eps, with_y=False):
    """rmsnorm.rs:14-77 then the row softmax, vectorised in numpy f32 (numpy's summation order)."""
    xf = emu.bf16_to_f32(x).reshape(rows, cols)
    gf = emu.bf16_to_f32(g)
    ss = np.sum(xf * xf, axis=1, dtype=np.float32)
    r = np.sqrt(ss / np.float32(cols) + np.float32(eps)).astype(np.float32)
    y = bf16r((xf * gf) / r[:, None])
    e = np.exp(y - y.max(axis=1, keepdims=True)).astype(np.float32)
    out = bf16r(e / np.sum(e, axis=1, dtype=np.float32, keepdims=True))
    return (out, y) if with_y else out


def rmsnorm_bound(x, g, rows, cols, eps):
    """Per-element limit on how far a chain whose f32 sums are ordered differently can land from the
    reference's RMSNorm->softmax output ([rows, cols]). A different order moves r by a few f32 ulps,
    so each y_j = bf16(x_j g_j / r) either stays or moves to a neighbouring bf16 value (one ulp(y_j)).
    The output's e_i / s then changes by the factor e^(+-ulp(y_i)) of its own y and by the relative
    change of s, at most sum_j p_j (e^ulp(y_j) - 1); a common shift of the max cancels in e / s.
    Two bf16 ulps of the output cover the f32 roundings of exp, the sum and the quotient.
    Rows with non-finite values follow the same rule: an infinite y contributes e = 0 (or makes the
    row NaN, which the callers compare by pattern), and an element whose e is 0 stays 0."""
    with np.errstate(all="ignore"):
        out, y = rmsnorm_softmax_numpy(x, g, rows, cols, eps, with_y=True)
        out = out.astype(np.float64)
        fy = np.where(np.isfinite(y), np.expm1(bf16_ulp(y)), 0.0)
        term = np.where(out > 0, out * fy, 0.0)
        b = np.where(out > 0, out * fy + out * np.sum(term, axis=1, keepdims=True), 0.0)
    return b + 2 * bf16_ulp(out)


def test_rmsnorm_softmax_config(rt):
    rows, cols = 8192, 4096
    rng = np.random.default_rng(31)
    x, g = bf16(rng, rows * cols), bf16(rng, cols, 0.1, 1.0)
    out = rt.alloc(rows * cols * 2)
    rt.rmsnorm_softmax(out, rt.upload(x), rt.upload(g), rows, cols, 1e-6)
    y = emu.bf16_to_f32(out.read(np.uint16)).reshape(rows, cols)
    assert np.all(np.abs(y.sum(axis=1, dtype=np.float64) - 1.0) < 2e-2)  # every row a distribution
    # every cell against the numpy restatement
    bound = rmsnorm_bound(x, g, rows, cols, 1e-6)
    close_chain(y, rmsnorm_softmax_numpy(x, g, rows, cols, 1e-6), frac_beyond=1e-4, hard=bound,
                name="rmsnorm_softmax 8192x4096 all cells vs numpy")
    # a seeded sample of rows against the oracle
    sample = rng.choice(rows, 48, replace=False)
    xs = x.reshape(rows, cols)[sample].reshape(-1)
    want = emu.bf16_to_f32(emu.rmsnorm_softmax(xs, g, len(sample), cols, 1e-6)).reshape(len(sample), cols)
    close_chain(y[sample], want, frac_beyond=1e-4, hard=bound[sample], name="rmsnorm_softmax 8192x4096 48 rows vs oracle")


# ---- attention prefill ------------------------------------------------------------------------------


@pytest.mark.parametrize("shape", [(1, 2, 256, 128), (2, 1, 200, 64), (1, 1, 64, 128), (1, 3, 333, 128), (1, 2, 1000, 64)])
@pytest.mark.parametrize("causal", [True, False])
def test_attention_small(rt, shape, causal):
    b, h, s, d = shape
    rng = np.random.default_rng(32)
    q, k, v = (bf16(rng, b * h * s * d) for _ in range(3))
    sd = np.float32(np.sqrt(d)) if d != 128 else SQRT_HEAD_DIM
    want = emu.attention_prefill(q, k, v, b * h, s, d, float(sd), causal)
    want_cm = emu.attention_prefill(q, k, v, b * h, s, d, float(sd), causal, causal_max=True)
    out = rt.alloc(b * h * s * d * 2)
    rt.attention_prefill(out, rt.upload(q), rt.upload(k), rt.upload(v), b, h, s, d, float(sd), causal)
    got = emu.bf16_to_f32(out.read(np.uint16))
    cm = emu.bf16_to_f32(want_cm)
    bound = attention_bound(q, k, v, b * h, s, d, sd, causal)
    # The kernel's running max differs from the oracle's causal max by up to 8 ln 2 as well, so its
    # bf16(p) round at another scale: attention_numpy's bound covers that for any choice of max.
    cm_bar = np.maximum(bound, np.maximum(2 * bf16_ulp(cm), 1e-2 * np.abs(cm) +
                                          1e-2 * np.sqrt(np.mean(cm.astype(np.float64) ** 2))))
    close_chain(got, cm, frac_beyond=1e-3, hard=cm_bar, name=f"attention {shape} causal={causal} vs causal-max oracle")
    # Reference max before masking: bf16(p) rounds at another scale (attention_numpy's bound).
    close_chain(got, emu.bf16_to_f32(want), frac_beyond=1e-3, hard=bound,
                name=f"attention {shape} causal={causal} vs oracle")


def attention_numpy(q, k, v, s, d, sqrt_d, causal=True):
    """One head of the attention chain (attention.rs:53-206, 370-392) vectorised in numpy f32: the
    reference's rounding points and its row max over every key, taken before masking.

    Returns (out, bound): `bound` is the per-element limit on how far an implementation that scales
    p by another max (a causal or running max) can land from `out`. Both sides round each p_j to bf16
    with relative error <= 2^-9 at their own scale, so sum_j P_j v_je / l moves by at most
    2^-8 sum_j (p_j / l) |v_je| (the element's weighted value mass); the bf16 narrows of o and of
    o / l on both sides add up to 3 ulps, the epsilon the reference adds to l (6.25e-8) a relative
    eps / l, and one more ulp covers this restatement's own f32 sums (numpy's BLAS order)."""
    qf, kf, vf = (emu.bf16_to_f32(t).reshape(s, d) for t in (q, k, v))
    sc = bf16r((qf @ kf.T) / np.float32(sqrt_d))
    e = np.exp(sc - sc.max(axis=1, keepdims=True)).astype(np.float32)
    if causal:
        e = np.where(np.tri(s, dtype=bool), e, np.float32(0))
    l = np.sum(e, axis=1, dtype=np.float32) + np.float32(6.25e-8)
    o = bf16r(bf16r(e) @ vf)
    out = bf16r(o / l[:, None])
    mass = (e / l[:, None]) @ np.abs(vf)
    bound = 2.0 ** -8 * mass + 4 * bf16_ulp(out) + 2 * np.abs(out) * (6.25e-8 / l[:, None])
    return out, bound


def attention_bound(q, k, v, bh, s, d, sqrt_d, causal=True):
    """attention_numpy's per-element bound for every head, laid out like the output."""
    return np.concatenate([attention_numpy(q[h * s * d:(h + 1) * s * d], k[h * s * d:(h + 1) * s * d],
                                           v[h * s * d:(h + 1) * s * d], s, d, sqrt_d, causal)[1]
                           for h in range(bh)]).reshape(-1)


def test_attention_config(rt):
    b, h, s, d = 4, 32, 2048, 128
    rng = np.random.default_rng(33)
    q, k, v = (bf16(rng, b * h * s * d) for _ in range(3))
    out = rt.alloc(b * h * s * d * 2)
    rt.attention_prefill(out, rt.upload(q), rt.upload(k), rt.upload(v), b, h, s, d, float(SQRT_HEAD_DIM), True)
    got = emu.bf16_to_f32(out.read(np.uint16)).reshape(b * h, s, d)
    assert np.isfinite(got).all()
    # every cell of every head against the numpy restatement
    ref, bound = np.empty_like(got), np.empty(got.shape, np.float64)
    for hh in range(b * h):
        sl = slice(hh * s * d, (hh + 1) * s * d)
        ref[hh], bound[hh] = attention_numpy(q[sl], k[sl], v[sl], s, d, SQRT_HEAD_DIM)
    close_chain(got, ref, frac_beyond=1e-3, hard=bound, name="attention B4H32S2048D128 all cells vs numpy")
    # every head's first and last 64 queries against the oracle
    qh, kh, vh = (t.reshape(b * h, s * d) for t in (q, k, v))
    head = lambda t: np.ascontiguousarray(t).reshape(-1)
    w_first = emu.bf16_to_f32(emu.attention_prefill(head(qh), head(kh), head(vh), b * h, s, d, float(SQRT_HEAD_DIM),
                                                    True, 0, 64)).reshape(b * h, s, d)[:, :64]
    w_last = emu.bf16_to_f32(emu.attention_prefill(head(qh), head(kh), head(vh), b * h, s, d, float(SQRT_HEAD_DIM),
                                                   True, s - 64, s)).reshape(b * h, s, d)[:, s - 64:]
    close_chain(got[:, :64], w_first, frac_beyond=1e-3, hard=bound[:, :64],
                name="attention config first 64 queries vs oracle")
    close_chain(got[:, s - 64:], w_last, frac_beyond=1e-3, hard=bound[:, s - 64:],
                name="attention config last 64 queries vs oracle")


def given_max_report(got, want, name):
    """The 1e-2 bar with no exception, recorded like close_chain's comparisons."""
    rec = report(name, got, want)
    close(got, want)
    return rec


@pytest.mark.parametrize("shape", [(1, 2, 256, 128), (2, 1, 200, 64), (1, 3, 333, 128), (1, 2, 1000, 64)])
@pytest.mark.parametrize("causal", [True, False])
def test_attention_given_max_small(rt, shape, causal):
    """With the reference's row max given (the max over every key, before masking), the kernel's
    p = exp(s - m) is the reference's, and every output cell is within the 1e-2 bar of the oracle --
    no exception fraction (what remains is the MFMA's reassociated f32 sums)."""
    b, h, s, d = shape
    rng = np.random.default_rng(37)
    q, k, v = (bf16(rng, b * h * s * d) for _ in range(3))
    sd = np.float32(np.sqrt(d)) if d != 128 else SQRT_HEAD_DIM
    rm = np.empty(b * h * s, np.float32)
    want = emu.bf16_to_f32(emu.attention_prefill(q, k, v, b * h, s, d, float(sd), causal, row_max=rm))
    out = rt.alloc(b * h * s * d * 2)
    rt.attention_prefill(out, rt.upload(q), rt.upload(k), rt.upload(v), b, h, s, d, float(sd), causal,
                         row_max=rt.upload(rm))
    given_max_report(emu.bf16_to_f32(out.read(np.uint16)), want, f"attention {shape} causal={causal} given max vs oracle")


# Non-finite inputs (the kernel is built with -fno-honor-nans): NaN and infinity in one element of
# q, k or v, with the reference's row max given so that the semantics are the reference's (its max
# over every key before masking: an infinite logit of a key a row does not see still sets that
# row's max; its mask clip min(p, mask) turns a NaN p into 1). Every NaN and infinity lands where
# the oracle's do; the other cells are held to the 1e-2 bar. (An infinite v under causal masking is left out: a masked key's p = 0 times v = inf is
# NaN wherever the masked key is multiplied at all, which depends on how keys are blocked -- the
# reference's 512-key chunks, the oracle's visible keys only.)
NONFINITE = [
    ("q", (0, 10, 5), np.nan, True),      # one query row: all NaN
    ("k", (1, 100, 0), np.nan, True),     # one key: the rows that see it NaN
    ("k", (0, 30, 2), np.inf, True),      # +-inf logits: NaN rows, or the key's p = 0
    ("v", (0, 50, 7), np.inf, False),     # one value column: +inf for every row (no masking)
]


@pytest.mark.parametrize("case", NONFINITE, ids=lambda c: f"{c[0]}{c[1]}={c[2]}-causal{c[3]}")
def test_attention_nonfinite(rt, case):
    which, (hh, row, col), val, causal = case
    b, h, s, d = 1, 2, 256, 128
    rng = np.random.default_rng(43)
    q, k, v = (bf16(rng, b * h * s * d) for _ in range(3))
    clean = emu.bf16_to_f32(emu.attention_prefill(q, k, v, b * h, s, d, float(SQRT_HEAD_DIM), causal,
                                                  row_max=np.empty(b * h * s, np.float32)))
    arr = {"q": q, "k": k, "v": v}[which]
    arr[(hh * s + row) * d + col] = emu.f32_to_bf16(np.array([val], np.float32))[0]
    rm = np.empty(b * h * s, np.float32)
    want = emu.bf16_to_f32(emu.attention_prefill(q, k, v, b * h, s, d, float(SQRT_HEAD_DIM), causal, row_max=rm))
    print(f"attention non-finite {case}", flush=True)
    out = rt.alloc(b * h * s * d * 2)
    rt.attention_prefill(out, rt.upload(q), rt.upload(k), rt.upload(v), b, h, s, d, float(SQRT_HEAD_DIM), causal,
                         row_max=rt.upload(rm))
    got = emu.bf16_to_f32(out.read(np.uint16))
    assert not np.array_equal(want, clean, equal_nan=True)  # the injected value reaches the output
    for name, t in (("kernel", got), ("oracle", want)):
        cells = t.reshape(b * h, s, d)
        rows = sorted({(int(x), int(y)) for x, y, _ in np.argwhere(~np.isfinite(cells))})
        print(f"  {name}: {np.isnan(t).sum()} NaN, {np.isinf(t).sum()} inf; non-finite in {len(rows)} rows "
              f"{rows[:3]}..{rows[-3:]}", flush=True)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.isinf(got), np.isinf(want)) and np.array_equal(got[np.isinf(got)], want[np.isinf(want)])
    fin = np.isfinite(want)
    close(got[fin], want[fin])


def test_attention_config_given_max(rt):
    """The attention config with the reference's own row max given to the kernel: every head's first
    and last 64 queries and a seeded spread of 8 blocks of 16 queries (17,408 rows, 2.2 M cells)
    against the oracle, each cell within |got - ref| <= 1e-2 |ref| + 1e-2 rms(ref), no exception.
    The oracle supplies the exact max of the rows it computes; the other rows get numpy's, whose
    logits may differ from the reference's in a last bit -- those rows are not compared."""
    b, h, s, d = 4, 32, 2048, 128
    rng = np.random.default_rng(33)
    q, k, v = (bf16(rng, b * h * s * d) for _ in range(3))
    bh = b * h
    rm = np.empty((bh, s), np.float32)
    for hh in range(bh):  # every row's max over every key, from numpy's f32 sums
        sl = slice(hh * s * d, (hh + 1) * s * d)
        qf, kf = (emu.bf16_to_f32(t[sl]).reshape(s, d) for t in (q, k))
        rm[hh] = bf16r((qf @ kf.T) / SQRT_HEAD_DIM).max(axis=1)
    starts = [0, s - 64] + sorted(int(x) * 16 for x in rng.choice(np.arange(4, s // 16 - 4), 8, replace=False))
    ranges = [(a, a + (64 if a in (0, s - 64) else 16)) for a in starts]
    want = {}
    for a, e in ranges:  # the oracle's rows, with their exact maxima
        exact = np.full(bh * s, np.nan, np.float32)
        o = emu.attention_prefill(q, k, v, bh, s, d, float(SQRT_HEAD_DIM), True, a, e, row_max=exact)
        want[(a, e)] = emu.bf16_to_f32(o).reshape(bh, s, d)[:, a:e]
        rm[:, a:e] = exact.reshape(bh, s)[:, a:e]
    out = rt.alloc(bh * s * d * 2)
    rt.attention_prefill(out, rt.upload(q), rt.upload(k), rt.upload(v), b, h, s, d, float(SQRT_HEAD_DIM), True,
                         row_max=rt.upload(rm.ravel()))
    got = emu.bf16_to_f32(out.read(np.uint16)).reshape(bh, s, d)
    assert np.isfinite(got).all()
    for (a, e), w in want.items():
        given_max_report(got[:, a:e], w, f"attention config queries {a}..{e - 1} given max vs oracle")


# ---- W8A8 ------------------------------------------------------------------------------------------------


def test_w8a8_small_exact_acc(rt):
    m, n, k = 96, 160, 256
    rng = np.random.default_rng(34)
    a = rng.integers(-127, 128, m * k).astype(np.int8)
    w = rng.integers(-127, 128, n * k).astype(np.int8)
    scale = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
    want, acc = emu.w8a8(a, w, scale, m, n, k)
    out, accb = rt.alloc(m * n * 2), rt.alloc(m * n * 4)
    rt.gemm_w8a8_dequant(out, accb, rt.upload(a), rt.upload(w), rt.upload(scale), m, n, k)
    assert np.array_equal(accb.read(np.int32), acc)
    assert np.array_equal(out.read(np.uint16), want)  # exact acc -> exact dequant and narrow


def test_w8a8_config_sampled_rows(rt):
    m, n, k = 2048, 8192, 8192
    rng = np.random.default_rng(35)
    a = rng.integers(-127, 128, m * k, dtype=np.int8)
    w = rng.integers(-127, 128, n * k, dtype=np.int8)
    scale = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
    out, accb = rt.alloc(m * n * 2), rt.alloc(m * n * 4)
    rt.gemm_w8a8_dequant(out, accb, rt.upload(a), rt.upload(w), rt.upload(scale), m, n, k)
    got_acc = accb.read(np.int32).reshape(m, n)
    got = out.read(np.uint16).reshape(m, n)
    for r0 in (0, 1337, m - 2):
        want, acc = emu.w8a8(a, w, scale, m, n, k, r0, r0 + 2)
        assert np.array_equal(got_acc[r0:r0 + 2], acc.reshape(m, n)[r0:r0 + 2])
        assert np.array_equal(got[r0:r0 + 2], want.reshape(m, n)[r0:r0 + 2])
    # linearity: the column sums of acc equal (sum over rows of a) . w, exactly in int64
    colsum = got_acc.astype(np.int64).sum(axis=0)
    asum = a.reshape(m, k).astype(np.int64).sum(axis=0)
    assert np.array_equal(colsum, w.reshape(n, k).astype(np.int64) @ asum)


def test_w8a8_ragged_four_wave_tiles(rt):
    """Large enough for the four-wave 256x256 tiles, with M and N not multiples of 256 (partial
    tiles at both edges): every accumulator and output exact."""
    m, n, k = 2056, 4000, 512
    rng = np.random.default_rng(37)
    a = rng.integers(-127, 128, m * k, dtype=np.int8)
    w = rng.integers(-127, 128, n * k, dtype=np.int8)
    scale = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
    out, accb = rt.alloc(m * n * 2), rt.alloc(m * n * 4)
    rt.gemm_w8a8_dequant(out, accb, rt.upload(a), rt.upload(w), rt.upload(scale), m, n, k)
    want, acc = emu.w8a8(a, w, scale, m, n, k)
    assert np.array_equal(accb.read(np.int32), acc)
    assert np.array_equal(out.read(np.uint16), want)


# ---- mapped GEMM through the seam -------------------------------------------------------


def test_mapped_gemm_config(rt):
    M = N = K = 4096
    s = dict(M=M, N=N, K=K)
    rng = np.random.default_rng(36)
    a, b = bf16(rng, M * K), bf16(rng, N * K)
    out = rt.alloc(M * N * 2)
    rt.contraction(out, rt.upload(a), rt.upload(b), fh.BF16, fh.BF16, fh.m("M / 8, M % 8, K", **s), fh.m("N, K", **s),
                   fh.m("M / 8, M % 8, N, K", **s), fh.m("M / 8, M % 8, N", **s))
    got = emu.bf16_to_f32(out.read(np.uint16)).reshape(M, N)
    # all 16.8 M cells against numpy's f32 product of the same bf16 operands, narrowed once
    full = bf16r(emu.bf16_to_f32(a).reshape(M, K) @ emu.bf16_to_f32(b).reshape(N, K).T)
    close(got, full)
    report("mapped GEMM 4096^3 all cells vs numpy", got, full)
    # rows of every 256-row tile band against the oracle's sequential fold
    for r0 in range(0, M, 256):
        r = r0 + (r0 // 256) * 13 % 256
        want = emu.bf16_to_f32(emu.gemm_rows(a, b, M, N, K, r, r + 1)).reshape(1, N)
        close(got[r:r + 1], want)


@pytest.mark.parametrize("types", [(fh.BF16, fh.BF16), (fh.BF16, fh.F32)], ids=["bf16", "f32out"])
def test_mapped_gemm_large_tiles_ragged(rt, types):
    # Enough 256x256 tiles for the large-tile path, with a partial last tile in M and in N and a
    # K that ends inside a 64-element stage (its DMA chunks past K must read as zero).
    M, N, K = 2056, 4000, 200
    in_t, out_t = types
    s = dict(M=M, N=N, K=K)
    rng = np.random.default_rng(38)
    a, b = bf16(rng, M * K), bf16(rng, N * K)
    ob = 2 if out_t == fh.BF16 else 4
    out = rt.alloc(M * N * ob)
    rt.contraction(out, rt.upload(a), rt.upload(b), in_t, out_t, fh.m("M / 8, M % 8, K", **s), fh.m("N, K", **s),
                   fh.m("M / 8, M % 8, N, K", **s), fh.m("M / 8, M % 8, N", **s))
    got = out.read(np.uint16 if out_t == fh.BF16 else np.float32).reshape(M, N)
    for r0 in (0, 253, 2048, M - 3):
        want = emu.gemm_rows(a, b, M, N, K, r0, r0 + 3, out_t=out_t).reshape(3, N)
        if out_t == fh.BF16:
            close(emu.bf16_to_f32(got[r0:r0 + 3]), emu.bf16_to_f32(want))
        else:
            close(got[r0:r0 + 3], want, rel=1e-3)


# ---- MLP classifier ----------------------------------------------------------------------


@pytest.mark.parametrize("shape", [(64, 784, 128, 10), (1, 800, 256, 16), (7, 33, 40, 3)])
def test_mlp_exact(rt, shape):
    batch, in_f, hid, out_f = shape
    rng = np.random.default_rng(37)
    x = emu.f32_to_bf16(rng.uniform(0, 1, batch * in_f).astype(np.float32))
    w1, b1 = bf16(rng, hid * in_f, 0.05), bf16(rng, hid, 0.05)
    w2, b2 = bf16(rng, out_f * hid, 0.05), bf16(rng, out_f, 0.05)
    pred, logits = emu.mlp(x, w1, b1, w2, b2, batch, in_f, hid, out_f)
    pb, lb = rt.alloc(batch * 4), rt.alloc(batch * out_f * 2)
    rt.mlp(pb, lb, *(rt.upload(t) for t in (x, w1, b1, w2, b2)), batch, in_f, hid, out_f)
    assert np.array_equal(lb.read(np.uint16), logits)
    assert np.array_equal(pb.read(np.int32), pred)


@pytest.mark.parametrize("shape", [(64, 784, 128, 10), (7, 33, 40, 3)])
def test_mlp_special_values_exact(rt, shape):
    """Weights and inputs holding bf16 subnormals (the reference widen reads them as zero), signed
    zeros, and weights near 2^-70 whose products with small inputs are f32 subnormals (kept by the
    reference's f32 arithmetic): logits and predictions bit-exact against the oracle."""
    batch, in_f, hid, out_f = shape
    rng = np.random.default_rng(38)

    def special(n, scale):
        v = (rng.standard_normal(n) * scale).astype(np.float32)
        kind = rng.integers(0, 12, n)
        v[kind == 1] *= np.float32(2.0 ** -70)
        bits = emu.f32_to_bf16(v)
        sub = kind == 2
        bits[sub] = (rng.integers(1, 0x80, int(sub.sum())) | (rng.integers(0, 2, int(sub.sum())) << 15)).astype(np.uint16)
        bits[kind == 3] = 0x8000
        return bits
    x = special(batch * in_f, 1.0)
    w1, b1 = special(hid * in_f, 0.05), special(hid, 0.05)
    w2, b2 = special(out_f * hid, 0.05), special(out_f, 0.05)
    pred, logits = emu.mlp(x, w1, b1, w2, b2, batch, in_f, hid, out_f)
    pb, lb = rt.alloc(batch * 4), rt.alloc(batch * out_f * 2)
    rt.mlp(pb, lb, *(rt.upload(t) for t in (x, w1, b1, w2, b2)), batch, in_f, hid, out_f)
    assert np.array_equal(lb.read(np.uint16), logits)
    assert np.array_equal(pb.read(np.int32), pred)


def test_mnist_answer_key(rt):
    """furiosa-opt-examples/tests/mnist_tests.rs:7-53: the reference's weights and ten images, loaded
    through the safetensors entry point, one forward per image (batch 1, 800 -> 256 -> 16); the argmax
    over the first ten logits must equal the stored labels, and the logits the oracle's bit for bit."""
    x, w1, b1, w2, b2, labels = mnist_key()
    path = GOLDEN / "mnist_hw.safetensors"
    ax = dict(X=800, H=256, C=16)
    bufs = {}
    for name, text, n in (("hw.fc1.weight", "H, X", 256 * 800), ("fc1.bias", "H", 256),
                          ("hw.fc2.weight", "C, H", 16 * 256), ("hw.fc2.bias", "C", 16)):
        bufs[name] = rt.alloc(n * 2)
        rt.load_safetensors(bufs[name], path, name, fh.BF16, fh.m(text, **ax))
    assert np.array_equal(bufs["hw.fc1.weight"].read(np.uint16), w1)
    logits = []
    for i in range(10):
        img = rt.alloc(800 * 2)
        rt.load_safetensors(img, path, f"hw.image_{i}", fh.BF16, fh.m("X", **ax))
        pb, lb = rt.alloc(4), rt.alloc(16 * 2)
        rt.mlp(pb, lb, img, bufs["hw.fc1.weight"], bufs["fc1.bias"], bufs["hw.fc2.weight"], bufs["hw.fc2.bias"],
               1, 800, 256, 16)
        logits.append(lb.read(np.uint16))
    logits = np.concatenate(logits)
    _, want = emu.mlp(x, w1, b1, w2, b2, 10, 800, 256, 16)
    assert np.array_equal(logits, want)
    assert first10_argmax(logits) == labels


def test_mlp_argmax_ties_take_the_last(rt):
    # all logits equal (zero weights, equal biases): max_by keeps the last index.
    batch, in_f, hid, out_f = 2, 16, 8, 10
    z = np.zeros
    x = emu.f32_to_bf16(np.ones(batch * in_f, np.float32))
    b2 = emu.f32_to_bf16(np.full(out_f, 0.5, np.float32))
    pb = rt.alloc(batch * 4)
    rt.mlp(pb, None, rt.upload(x), rt.upload(z(hid * in_f, np.uint16)), rt.upload(z(hid, np.uint16)),
           rt.upload(z(out_f * hid, np.uint16)), rt.upload(b2), batch, in_f, hid, out_f)
    assert pb.read(np.int32).tolist() == [out_f - 1] * batch
