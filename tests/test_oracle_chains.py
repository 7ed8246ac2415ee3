"""Pins of the oracle's fused chains (oracle/fo_cpu.c ref_rmsnorm_softmax, ref_attention_prefill,
ref_w8a8, ref_mlp) against closed forms. The reference's own transformer tests need the closed
compiler, so the chain compositions are checked against what the mathematics fixes: inputs whose
every intermediate is exact (or rounds in a known way) give outputs computed here independently
with numpy, and a wrong order of the steps, a missing or misplaced rounding, a transposed operand
or a wrong mask fails one of them.
"""
import json
import struct
from pathlib import Path

import numpy as np
import pytest

from oracle import emulator as emu

bf = emu.f32_to_bf16
fl = emu.bf16_to_f32


def bf16_of(values):
    return bf(np.asarray(values, np.float32))


# ---- RMSNorm -> softmax (transformer/kernel/rmsnorm.rs:9-78, then a row softmax) --------------------


def test_rmsnorm_softmax_constant_row_is_uniform():
    # Every y equal: exp(0) = 1 everywhere, the sum is cols, and 1/cols is exact at a power of two.
    for cols in (512, 4096):
        x = bf16_of(np.full(2 * cols, 3.0))
        g = bf16_of(np.full(cols, 0.75))
        out = emu.rmsnorm_softmax(x, g, 2, cols, 1e-6)
        assert np.all(fl(out) == np.float32(1.0 / cols))


@pytest.mark.parametrize("a,b", [(1.0, 2.0), (2.0 ** -10, 2.0 ** -9)])
def test_rmsnorm_softmax_two_valued_row_closed_form(a, b):
    # Half the row is a, half b, gain 1: ss = (cols/2)(a^2 + b^2) is exact, r = sqrt(ss/cols + eps),
    # y = bf16(x / r); the softmax of the two values has a closed form. The division is by r (not
    # r^2, not a reciprocal); with the small pair ss/cols is comparable to eps, so eps must sit
    # inside the square root.
    cols = 1024
    x = bf16_of(np.array([a, b] * (cols // 2)))
    g = bf16_of(np.ones(cols))
    out = fl(emu.rmsnorm_softmax(x, g, 1, cols, 1e-6))
    ms = np.float32(np.float32((cols // 2) * (a * a + b * b)) / np.float32(cols)) + np.float32(1e-6)
    r = np.float32(np.sqrt(np.float64(ms)))  # sqrt of an f32 is never a tie: f64 rounding is correct
    ya, yb = float(fl(bf16_of(np.float32(a) / r))[0]), float(fl(bf16_of(np.float32(b) / r))[0])
    ea, eb = np.exp(np.float64(ya - yb)), 1.0
    s = (cols // 2) * (ea + eb)
    want = np.array([ea / s, eb / s] * (cols // 2))
    assert np.all(np.abs(out - want) <= 2.0 ** -8 * want)  # one bf16 rounding of e / s


def test_rmsnorm_softmax_gain_scales_y():
    # A constant row with a gain alternating 1 and 2 gives y alternating 1 and 2 (r rounds to 1 at
    # bf16), so the output alternates 1/(n(1+e)) and e/(n(1+e)) with e = exp(1).
    cols = 2048
    x = bf16_of(np.ones(cols))
    g = bf16_of(np.array([1.0, 2.0] * (cols // 2)))
    out = fl(emu.rmsnorm_softmax(x, g, 1, cols, 1e-6))
    ms = np.float32(np.float32(cols) / np.float32(cols)) + np.float32(1e-6)
    r = np.float32(np.sqrt(np.float64(ms)))
    y1, y2 = float(fl(bf16_of(np.float32(1.0) / r))[0]), float(fl(bf16_of(np.float32(2.0) / r))[0])
    assert (y1, y2) == (1.0, 2.0)
    e = np.exp(1.0)
    s = (cols // 2) * (1.0 + e)
    want = np.array([1.0 / s, e / s] * (cols // 2))
    assert np.all(np.abs(out - want) <= 2.0 ** -8 * want)


def test_rmsnorm_softmax_rows_are_distributions():
    rng = np.random.default_rng(5)
    rows, cols = 16, 1024
    x = bf16_of(rng.standard_normal(rows * cols))
    g = bf16_of(rng.uniform(0.5, 1.5, cols))
    out = fl(emu.rmsnorm_softmax(x, g, rows, cols, 1e-6)).reshape(rows, cols).astype(np.float64)
    assert np.all(out >= 0) and np.all(np.abs(out.sum(axis=1) - 1.0) < 1e-2)


# ---- attention (transformer/kernel/attention.rs:32-392) -----------------------------------------


def attn(q, k, v, s, d, causal):
    return fl(emu.attention_prefill(q, k, v, 1, s, d, float(np.sqrt(d)), causal=causal)).reshape(s, d)


@pytest.mark.parametrize("causal", [True, False])
def test_attention_zero_queries_average_the_visible_values(causal):
    # Q = 0 makes every logit 0 and every p = 1, so o_i is the plain sum of the visible V rows (small
    # integers: exact in f32), narrowed to bf16, and l = the count of visible keys:
    #   out_i = bf16( bf16(sum_{k visible to i} v_k) / (count + EPS) )   (attention.rs:167-176, 370-392).
    s, d = 96, 64
    rng = np.random.default_rng(6)
    q = bf16_of(np.zeros(s * d))
    k = bf16_of(rng.standard_normal(s * d))
    vi = rng.integers(-100, 101, (s, d))  # sums past 256 round at the bf16 narrow of o
    v = bf16_of(vi.astype(np.float32).ravel())
    got = attn(q, k, v, s, d, causal)
    eps = np.float32(6.25e-8)
    for i in range(s):
        n = i + 1 if causal else s
        o = fl(bf16_of(vi[:n].sum(axis=0).astype(np.float32)))
        want = fl(bf16_of(o / (np.float32(n) + eps)))
        assert np.array_equal(got[i], want), i


def test_attention_first_query_sees_only_the_first_key():
    # Causal: query 0 weighs key 0 alone, so out_0 = v_0 up to the bf16 roundings of p, o and the
    # quotient (p is taken against the max over all keys, before masking).
    s, d = 64, 128
    rng = np.random.default_rng(7)
    q, k, v = (bf16_of(rng.standard_normal(s * d)) for _ in range(3))
    got = attn(q, k, v, s, d, True)
    v0 = fl(v[:d])
    assert np.all(np.abs(got[0] - v0) <= 3 * 2.0 ** -8 * np.abs(v0))


def test_attention_weights_are_narrowed_to_bf16_before_pv():
    # Two keys per head with logits 0 and t < 0: p = (1, e^t), and with v = (0, 3) the output is
    # bf16( bf16(3 bf16(e^t)) / (1 + e^t + EPS) ) (weighted_sum casts p to bf16 before the product,
    # attention.rs:167-176, then o is narrowed) rather than bf16( bf16(3 e^t) / (1 + e^t + EPS) ).
    heads, s, d = 256, 2, 16
    t = -np.linspace(0.05, 6.0, heads).astype(np.float32)
    q = np.zeros((heads, s, d), np.float32)
    q[:, :, 0] = 1.0
    k = np.zeros((heads, s, d), np.float32)
    k[:, 1, 0] = t * np.float32(np.sqrt(d))
    v = np.zeros((heads, s, d), np.float32)
    v[:, 1, :] = 3.0
    got = fl(emu.attention_prefill(bf16_of(q.ravel()), bf16_of(k.ravel()), bf16_of(v.ravel()), heads, s, d,
                                   float(np.sqrt(d)), causal=False)).reshape(heads, s, d)[:, 0, 0]
    s1 = fl(bf16_of(fl(bf16_of(k[:, 1, 0])) / np.float32(np.sqrt(d))))  # the logit, as qk_scaled rounds it
    p1 = np.exp(s1.astype(np.float64)).astype(np.float32)
    den = np.float32(1.0) + p1 + np.float32(6.25e-8)
    narrowed = fl(bf16_of(fl(bf16_of(fl(bf16_of(p1)) * np.float32(3.0))) / den))
    plain = fl(bf16_of(fl(bf16_of(p1 * np.float32(3.0))) / den))
    assert np.mean(narrowed != plain) > 0.2  # the two readings are distinguishable here
    assert np.mean(got == narrowed) > 0.95  # (an f32 ulp of exp may flip a rare rounding)


def test_attention_equal_keys_are_weighted_equally():
    # Every key row equal: all logits of a query are equal, so the output is the mean of the visible
    # V rows within the bf16 roundings; with causal masking row i averages rows 0..i only.
    s, d = 64, 64
    rng = np.random.default_rng(8)
    q = bf16_of(rng.standard_normal(s * d))
    k = bf16_of(np.tile(rng.standard_normal(d), s))
    v = bf16_of(rng.standard_normal(s * d))
    vf = fl(v).reshape(s, d).astype(np.float64)
    got = attn(q, k, v, s, d, True)
    for i in (0, 1, 7, 63):
        want = vf[: i + 1].mean(axis=0)
        assert np.all(np.abs(got[i] - want) <= 2.0 ** -6 * np.abs(vf[: i + 1]).max()), i


def test_attention_causal_max_is_attention_over_the_prefix():
    # The oracle's causal-max mode (the max over the visible keys only) at query i is, by definition,
    # the reference's non-causal chain over the first i + 1 keys alone: with no masked key, the max
    # over every key is the max over the visible ones. Checked against the default (pinned) mode run
    # on the truncated sequence, bit for bit; and it differs from the default causal mode, whose max
    # includes the masked keys, on most rows.
    s, d = 48, 64
    rng = np.random.default_rng(10)
    q, k, v = (bf16_of(rng.standard_normal(s * d) * 2.0) for _ in range(3))
    cm = fl(emu.attention_prefill(q, k, v, 1, s, d, float(np.sqrt(d)), causal=True, causal_max=True)).reshape(s, d)
    dm = fl(emu.attention_prefill(q, k, v, 1, s, d, float(np.sqrt(d)), causal=True)).reshape(s, d)
    differ = 0
    for i in range(s):
        n = i + 1
        pre = fl(emu.attention_prefill(q.reshape(s, d)[:n].ravel(), k.reshape(s, d)[:n].ravel(),
                                       v.reshape(s, d)[:n].ravel(), 1, n, d, float(np.sqrt(d)),
                                       causal=False)).reshape(n, d)
        assert np.array_equal(cm[i].view(np.uint32), pre[i].view(np.uint32)), i
        differ += not np.array_equal(cm[i], dm[i])
    assert differ > s // 4
    # query 0 sees key 0 alone: p = e^0 = 1, l = 1 + EPS, o = v_0, so out_0 = v_0 exactly
    assert np.array_equal(cm[0], fl(v[:d]))


def test_attention_row_max_is_the_premask_max():
    # The oracle reports each computed row's max: over every key before masking by default (the
    # reference's row_max, attention.rs:77-95), over the visible keys in the causal-max mode; both
    # equal the max of the logits bf16(f32(q.k) / sqrt_d), whose f32 sums are exact here (small
    # integer inputs), computed in numpy.
    bh, s, d = 2, 40, 32
    rng = np.random.default_rng(11)
    q, k, v = (bf16_of(rng.integers(-3, 4, bh * s * d).astype(np.float32)) for _ in range(3))
    sd = float(np.sqrt(d))
    logits = np.stack([fl(bf16_of((fl(q).reshape(bh, s, d)[h] @ fl(k).reshape(bh, s, d)[h].T) / np.float32(sd)))
                       for h in range(bh)])
    for causal_max, want in ((False, logits.max(axis=2)),
                             (True, np.where(np.tri(s, dtype=bool), logits, -np.inf).max(axis=2))):
        rm = np.full(bh * s, np.nan, np.float32)
        emu.attention_prefill(q, k, v, bh, s, d, sd, causal=True, q_begin=3, q_end=30, causal_max=causal_max,
                              row_max=rm)
        rm = rm.reshape(bh, s)
        assert np.array_equal(rm[:, 3:30], want[:, 3:30].astype(np.float32))
        assert np.isnan(rm[:, :3]).all() and np.isnan(rm[:, 30:]).all()  # rows not computed are untouched


def test_attention_oracle_rejects_long_rows():
    # The oracle's per-row scratch holds 8192 keys; a longer sequence raises instead of leaving rows
    # unwritten.
    z = np.zeros(8200 * 8, np.uint16)
    with pytest.raises(ValueError):
        emu.attention_prefill(z, z, z, 1, 8200, 8, 2.0, q_begin=0, q_end=1)


# ---- W8A8 (i8 contraction, FxpToFp(31), MulF, cast to bf16) -----------------------------------------


def test_w8a8_is_the_integer_product_then_scale():
    # acc = A W^T in wrapping i32; out = bf16(f32(acc) * scale[col]) (fixedpoint_to_float(acc, 31)
    # is the nearest f32 of acc). Checked against numpy's integer matmul.
    rng = np.random.default_rng(9)
    m, n, k = 24, 40, 96
    a = rng.integers(-128, 128, (m, k)).astype(np.int8)
    w = rng.integers(-128, 128, (n, k)).astype(np.int8)
    scale = rng.uniform(1e-4, 1e-2, n).astype(np.float32)
    out, acc = emu.w8a8(a.ravel(), w.ravel(), scale, m, n, k)
    want_acc = a.astype(np.int64) @ w.astype(np.int64).T
    assert np.array_equal(acc.reshape(m, n), want_acc.astype(np.int32))
    want = bf(want_acc.astype(np.float32) * scale[None, :]).ravel()
    assert np.array_equal(out, want)


def test_w8a8_accumulator_wraps():
    # 127 * 127 * k past 2^31 wraps in the i32 accumulator, as the reference's wrapping add does.
    m, n, k = 2, 3, 140000
    a = np.full((m, k), 127, np.int8)
    w = np.full((n, k), 127, np.int8)
    _, acc = emu.w8a8(a.ravel(), w.ravel(), np.ones(n, np.float32), m, n, k)
    want = np.int64(127 * 127 * k)
    assert np.all(acc == np.int32(((want + 2 ** 31) % 2 ** 32) - 2 ** 31))


# ---- MLP (mnist/mod.rs:8-192) -----------------------------------------------------------------------


def mlp(x, w1, b1, w2, b2, batch, i, h, o):
    pred, logits = emu.mlp(bf16_of(x), bf16_of(w1), bf16_of(b1), bf16_of(w2), bf16_of(b2), batch, i, h, o)
    return pred, fl(logits).reshape(batch, o)


def test_mlp_zero_weights_give_the_output_bias():
    batch, i, h, o = 3, 20, 8, 10
    rng = np.random.default_rng(10)
    b2 = np.float32(np.round(rng.standard_normal(o), 2))
    b2[6] = 9.0
    pred, logits = mlp(rng.standard_normal(batch * i), np.zeros(h * i), rng.standard_normal(h), np.zeros(o * h), b2,
                       batch, i, h, o)
    assert np.all(logits == fl(bf16_of(b2))[None, :]) and np.all(pred == 6)


def test_mlp_relu_and_weight_orientation():
    # x one-hot at feature f, w1[j][f] = c_j: hidden j = relu(bf16(c_j) + b1_j); w2 a permutation
    # (w2[o][j] = 1 iff j == (o + 1) % h) and b2 = 0 route hidden (o + 1) % h to logit o. A
    # transposed w1 or w2, or a missing relu, changes the logits.
    batch, i, h = 2, 12, 6
    f = 5
    c = np.array([1.5, -2.0, 0.25, 3.0, -0.5, 0.75], np.float32)
    b1 = np.array([0.0, 1.0, -1.0, 0.5, 0.25, -0.75], np.float32)
    x = np.zeros((batch, i), np.float32)
    x[:, f] = 1.0
    w1 = np.zeros((h, i), np.float32)
    w1[:, f] = c
    w1[:, f + 1] = 7.0  # a feature the input does not hold
    w2 = np.roll(np.eye(h, dtype=np.float32), 1, axis=1)
    pred, logits = mlp(x.ravel(), w1.ravel(), b1, w2.ravel(), np.zeros(h), batch, i, h, h)
    want = np.roll(np.maximum(c + b1, 0.0), -1)
    assert np.all(logits == want[None, :]) and np.all(pred == int(np.argmax(want)))


# ---- the reference's MNIST answer key (furiosa-opt-examples/tests/mnist_tests.rs:7-53) -------------
GOLDEN = Path(__file__).resolve().parent / "golden"


def read_safetensors(path):
    """{name: (dtype string, shape, raw bytes)} of a safetensors file, parsed as plain data."""
    raw = Path(path).read_bytes()
    n = struct.unpack("<Q", raw[:8])[0]
    header = json.loads(raw[8:8 + n])
    return {k: (v["dtype"], v["shape"], raw[8 + n + v["data_offsets"][0]:8 + n + v["data_offsets"][1]])
            for k, v in header.items() if k != "__metadata__"}


def mnist_key():
    """The fixture's weights, the ten images stacked as a batch, and the labels."""
    t = read_safetensors(GOLDEN / "mnist_hw.safetensors")
    u16 = lambda name: np.frombuffer(t[name][2], np.uint16)
    x = np.concatenate([u16(f"hw.image_{i}") for i in range(10)])
    labels = [int(np.frombuffer(t[f"label_{i}"][2], np.int32)[0]) for i in range(10)]
    return x, u16("hw.fc1.weight"), u16("fc1.bias"), u16("hw.fc2.weight"), u16("hw.fc2.bias"), labels


def first10_argmax(logits):
    """mnist_tests.rs:38-48: max_by(total_cmp) over the first ten logits (the last maximum wins)."""
    rows = emu.bf16_to_f32(logits).reshape(10, 16)[:, :10]
    return [int(9 - np.argmax(r[::-1])) for r in rows]


def test_mnist_answer_key():
    x, w1, b1, w2, b2, labels = mnist_key()
    assert labels == [7, 2, 1, 0, 4, 1, 4, 9, 5, 9]
    _, logits = emu.mlp(x, w1, b1, w2, b2, 10, 800, 256, 16)
    assert first10_argmax(logits) == labels
