"""The decode-step chains (projection, decoder, final layer and one whole layer of mod.rs:29-131 and
transformer.py:495-562, stages in furiosa_hip/decode.py) through the C ABI against the oracle.

Every stage of the device chain is re-run on the oracle from the device's own inputs to that stage,
so each stage answers to its own bar rather than to the drift of the stages before it:
  * the GEMVs (q, k, v, o, lm_head) bit-exact: serial f32 folds of the widened bf16 operands, the
    oracle's order;
  * RoPE, the residuals, the attention norm, the cache rows bit-exact: f32 multiplies, adds and
    divides rounded once (no contraction into an FMA across seam ops), then a narrow, and copies;
  * RMSNorm: the rms within (n + 4) f32 ulps of the oracle's (two f32 sums of the same n
    non-negative squares, in any orders, lie within 2(n - 1) ulps of each other; the division, the
    EPS add and the square root add three roundings and halve the relative spread), then y
    bit-exact against the oracle's quotient by the device's own rms: the fold order of the sum is
    free, the rounding of y is not;
  * the MLP within the bar of test_gpu_decode (bit-exact on at least 99.9% of the elements, within 2
    bf16 ulps everywhere): its sigmoid goes through expf;
then the chain's end value passes the reference's acceptance test against the model.
"""
import numpy as np
import pytest

import decode_chain as dc
import furiosa_hip.decode as fd
from test_gpu_decode import near
from test_oracle_decode import accepted
from test_oracle_step import (D, G, H, N, ONE, T, model_decoder_inputs, model_projection_inputs, run_decoder,
                              step_case)

pytestmark = pytest.mark.gpu
BF16, F32 = fd.BF16, fd.F32
CPU = dc.CpuOps(dc.STEP_SIZES)


def host(ops, st):
    """The device stages as host arrays (f32 for the sums and rms, bf16 bits for the rest)."""
    return {k: ops.get(v, F32 if k == "sum" or k.endswith("_rms") else BF16) for k, v in st.items()}


def rms_stage(rms_got, y_got, x, w, rows, axis, n):
    rms_want, _ = fd.rmsnorm(CPU, x, w, rows, axis, n)
    np.testing.assert_allclose(rms_got, rms_want, rtol=(n + 4) * 2.0 ** -24, atol=0)
    _, y_want = fd.rmsnorm(CPU, x, w, rows, axis, n, rms=rms_got)
    assert np.array_equal(y_got, y_want)


def widen(x):
    return CPU.map(x, BF16, F32, "CAST")


def test_projection_stages_match_the_oracle(rt):
    a, kc0, vc0 = model_projection_inputs(100)
    pos = 5
    cos, sin = fd.rope_row(pos)
    print("projection seed 100 pos 5", flush=True)
    ops = fd.SeamOps(rt, fd.STEP_SIZES)
    st = {}
    q, kc, vc = fd.projection(ops, a["x"], a["wq"], a["wk"], a["wv"], a["g_in"], a["g_q"], a["g_k"],
                              pos * fd.ROW_STRIDE_ND, cos, sin, kc0, vc0, st)
    q, kc, vc, s = ops.get(q, BF16), ops.get(kc, BF16), ops.get(vc, BF16), host(ops, st)
    rms_stage(s["y_rms"], s["y"], a["x"], a["g_in"], "X", "H", H)
    yw = widen(s["y"])
    for name, w, rows in (("q", a["wq"], "Q"), ("k", a["wk"], "P"), ("v", a["wv"], "P")):
        assert np.array_equal(s[name], fd.proj(CPU, yw, w, rows)), name
    rms_stage(s["qn_rms"], s["qn"], s["q"], a["g_q"], "N, G", "D", D)
    rms_stage(s["kn_rms"], s["kn"], s["k"], a["g_k"], "N", "D", D)
    assert np.array_equal(q, fd.rope(CPU, s["qn"], cos, sin, "N, G"))
    assert np.array_equal(s["kr"], fd.rope(CPU, s["kn"], cos, sin, "N"))
    assert np.array_equal(kc, fd.cache_row(CPU, kc0, s["kr"], pos * fd.ROW_STRIDE_ND))
    assert np.array_equal(vc, fd.cache_row(CPU, vc0, s["v"], pos * fd.ROW_STRIDE_ND))
    qm, km, vm = dc.projection_model(a["x"], a["wq"], a["wk"], a["wv"], a["g_in"], a["g_q"], a["g_k"], pos)
    for want, got in ((qm, q), (km, kc.reshape(T, -1)[pos]), (vm, vc.reshape(T, -1)[pos])):
        ok, rate = accepted(want, dc.f64(got))
        assert ok, rate


def test_decoder_stages_match_the_oracle(rt):
    a = model_decoder_inputs(101)
    a["sum"] = np.random.default_rng(1).uniform(0.5, 4.0, N * G).astype(np.float32)  # a norm that divides
    print("decoder seed 101", flush=True)
    ops = fd.SeamOps(rt, fd.STEP_SIZES)
    st = {}
    out = ops.get(fd.decoder(ops, a["x"], a["sum"], a["rx"], a["wo"], a["g_post"], a["up"], a["gate"], a["down"],
                             st), BF16)
    s = host(ops, st)
    assert np.array_equal(s["a"], fd.norm(CPU, a["x"], a["sum"]))
    assert np.array_equal(s["o"], fd.proj(CPU, widen(s["a"]), a["wo"], "H", "Q"))
    assert np.array_equal(s["rx1"], fd.residual(CPU, s["o"], a["rx"]))
    rms_stage(s["y_rms"], s["y"], s["rx1"], a["g_post"], "X", "H", H)
    near(s["m"], fd.mlp_block(CPU, s["y"], a["up"], a["gate"], a["down"]))
    assert np.array_equal(out, fd.residual(CPU, s["m"], s["rx1"]))
    x_normed = dc.f64(a["x"], N * G, D) / a["sum"][:, None]  # the model's input: out / sum
    want = dc.decoder_model(dc.emu.f32_to_bf16(x_normed.reshape(-1).astype(np.float32)), a["rx"], a["wo"],
                            a["g_post"], a["up"], a["gate"], a["down"])
    ok, rate = accepted(want, dc.f64(out))
    assert ok, rate


def test_final_layer_stages_match_the_oracle(rt):
    rng = np.random.default_rng(102)
    x, g = dc.sample(rng, H), dc.layer_weights(rng)["post_norm"]
    lm = dc.linear_init(rng, fd.WP, H)
    print("final layer seed 102", flush=True)
    ops = fd.SeamOps(rt, fd.STEP_SIZES)
    st = {}
    got = ops.get(fd.final_layer(ops, x, g, lm, st), BF16)
    y = ops.get(st["y"], BF16)
    rms_stage(ops.get(st["y_rms"], F32), y, x, g, "X", "H", H)
    assert np.array_equal(got, fd.proj(CPU, widen(y), lm, "Wp"))
    ok, rate = accepted(dc.final_model(x, g, lm), dc.f64(got[:fd.W]))
    assert ok, rate


def test_decoder_step_wires_kernel_boundaries(rt):
    """transformer_tests.rs:405-526 through the C ABI: zero weights leave the residual stream as it was."""
    rng = np.random.default_rng(0xDEC0DE + 1)
    x, rx = dc.seeded(rng, H, 0.2), dc.seeded(rng, H, 0.2)
    ones = lambda n: np.full(n, ONE, np.uint16)
    zeros = lambda n: np.zeros(n, np.uint16)
    print("decoder step wiring", flush=True)
    ops = fd.SeamOps(rt, fd.STEP_SIZES)
    q, kc, vc = fd.projection(ops, x, zeros(fd.Q * H), zeros(fd.P * H), zeros(fd.P * H), ones(H), ones(D), ones(D),
                              0, ones(D), zeros(D), zeros(T * N * D), zeros(T * N * D))
    _, sm, out = fd.attend(ops, q, [kc], [vc], [np.ones(T, np.float32)])
    got = ops.get(fd.decoder(ops, out, sm, rx, zeros(H * fd.Q), zeros(H), zeros(fd.L * H), zeros(fd.L * H),
                             zeros(H * fd.L)), BF16)
    assert np.array_equal(got, rx)


@pytest.mark.parametrize("pos", [0, T - 1, T + 88, 2 * T])
def test_layer_step_matches_the_oracle(rt, pos):
    """One layer through the seam ops at the first token, the last row of a chunk, a row inside the
    second chunk and the first row of a third, against the same layer on the oracle: the new
    residual stream bit-exact on at least 99% of its elements and everywhere within the reference's
    per-element tolerance max(0.01 |e|, 2^-8) of the oracle's (the device regroups f32 sums and
    rounds exp within ulps, which a few bf16 narrows downstream can turn into ulp-sized steps); at
    T + 88 also under the reference's acceptance test against the float64 model. The earlier
    chunks' caches stay untouched and the written K and V rows are the device's own projection."""
    from test_oracle_step import step_model
    chunk, row = divmod(pos, T)
    lw, x, caches = step_case(103 + pos, pos)
    print("layer step seed", 103 + pos, "pos", pos, flush=True)
    ops = fd.SeamOps(rt, fd.STEP_SIZES)
    cs = [(ops.put(k), ops.put(v)) for k, v in caches]
    st = {}
    got = ops.get(fd.layer_step(ops, x, lw, pos, cs, *fd.rope_row(pos), st), BF16)
    want = CPU.get(fd.layer_step(CPU, x, lw, pos, list(caches), *fd.rope_row(pos)), BF16)
    g, w = dc.f64(got), dc.f64(want)
    assert np.mean(got == want) >= 0.99
    assert np.all(np.abs(g - w) <= np.maximum(0.01 * np.abs(w), 2.0 ** -8))
    if pos == T + 88:
        ok, rate = accepted(step_model(lw, x, caches, pos), g)
        assert ok, rate
    for c in range(chunk):
        assert np.array_equal(ops.get(cs[c][0], BF16), caches[c][0])
        assert np.array_equal(ops.get(cs[c][1], BF16), caches[c][1])
    for side, want_row in ((0, st["kr"]), (1, st["v"])):
        got_cache = ops.get(cs[chunk][side], BF16).reshape(T, -1)
        assert np.array_equal(got_cache[row], ops.get(want_row, BF16))
        assert np.array_equal(np.delete(got_cache, row, axis=0), np.delete(caches[chunk][side].reshape(T, -1), row, axis=0))


def test_pipeline_tokens_match_the_oracle(rt):
    """Pipeline.step (transformer.py:495-566) through the seam ops: two layers of random weights, a
    tied embedding, a two-token prompt and two greedy tokens, the same token sequence fed to the
    oracle's pipeline. Each step's logits are bit-exact on at least 99% of the vocabulary and all
    within max(0.01 |e|, 2^-8) of the oracle's; the greedy token is the oracle's wherever the
    oracle's best logit leads the next by more than two of its ulps."""
    from test_oracle_step import tied_model
    model = tied_model(111, layers=2, zero_layers=False)
    print("pipeline: 2 layers, 4 steps", flush=True)
    cpu, gpu = fd.Pipeline(CPU, model), fd.Pipeline(fd.SeamOps(rt, fd.STEP_SIZES), model)
    prompt, want = [5, 1234], None
    for pos in range(4):
        tok = prompt[pos] if pos < len(prompt) else fd.sample_token(want)
        want, got = cpu.step(tok, pos), gpu.step(tok, pos)
        w, g = dc.f64(want[:fd.W]), dc.f64(got[:fd.W])
        assert np.mean(got[:fd.W] == want[:fd.W]) >= 0.99, pos
        assert np.all(np.abs(g - w) <= np.maximum(0.01 * np.abs(w), 2.0 ** -8)), pos
        top2 = np.sort(w)[-2:]
        if top2[1] - top2[0] > 2 * 2.0 ** (np.floor(np.log2(abs(top2[1]))) - 7):
            assert fd.sample_token(got) == fd.sample_token(want), pos
