"""The oracle's decode-step chains (furiosa_hip/decode.py: projection, decoder and final layer of
mod.rs:29-131, and one whole layer of Pipeline.step, transformer.py:495-562) pinned on the CPU:

  * the reference's scalar tests (transformer_tests.rs:92-214, 405-526, 558-643, 663-695) with their
    own tolerances, on seeded inputs of their distributions (their SmallRng streams are not
    reproducible here, so the seeds are ours);
  * the reference's model checks (transformer.py:189-243, 284-341: the torch modules restated in
    float64 with torch's bf16 narrows) under its acceptance test, at a real RoPE position and with
    the KV caches holding other rows;
  * closed forms: the half swap, the cache row scatter at a byte offset, RoPE as one f32 rounding of
    two exact products, the tiled lm_head GEMV against the whole contraction;
  * planted mistakes (no half swap, an unscaled cache offset, a dropped residual) that the checks
    must reject.
"""
import numpy as np
import pytest

import decode_chain as dc
import furiosa_hip.decode as fd
from oracle import emulator as emu
from oracle import mapping_ref as mr
from test_oracle_decode import accepted

OPS = dc.CpuOps(dc.STEP_SIZES)
N, G, D, T, H, L = fd.N, fd.G, fd.D, fd.T, fd.H, fd.L
ONE = emu.f32_to_bf16(np.ones(1, np.float32))[0]


def test_gemv_tiles_match_the_whole_contraction():
    rng = np.random.default_rng(90)
    s = dict(R=2048, K=256)
    x = rng.standard_normal(256).astype(np.float32)
    w = rng.standard_normal(2048 * 256).astype(np.float32)
    tiled = dc.CpuOps(s, tile=512).gemv(x, w, "R", "K")
    v = lambda t: mr.parse(t, s)
    whole = emu.contraction(x, w, emu.F32, emu.F32, v("K"), v("R, K"), v("R, K"), v("R"))
    assert np.array_equal(tiled.view(np.uint32), whole.view(np.uint32))


def test_rotate_half_swaps_the_halves():
    x = np.arange(N * G * D, dtype=np.uint16)
    r = fd.rotate_half(OPS, x, "N, G").reshape(N * G, D)
    xx = x.reshape(N * G, D)
    assert np.array_equal(r[:, :D // 2], xx[:, D // 2:]) and np.array_equal(r[:, D // 2:], xx[:, :D // 2])


def test_cache_row_writes_one_row_at_a_byte_offset():
    rng = np.random.default_rng(91)
    cache = rng.integers(0, 1 << 16, T * N * D, dtype=np.uint64).astype(np.uint16)
    row = rng.integers(0, 1 << 16, N * D, dtype=np.uint64).astype(np.uint16)
    out = fd.cache_row(OPS, cache, row, 37 * fd.ROW_STRIDE_ND).reshape(T, N * D)
    want = cache.reshape(T, N * D).copy()
    want[37] = row
    assert np.array_equal(out, want)


@pytest.mark.parametrize("pos", [0, 5, 700, 4000])
def test_rope_is_one_rounding_of_exact_products(pos):
    """bf16 x bf16 products are exact in f32, so the kernel's value is the f32 rounding of the exact
    x cos + rotate_half(x) sin, narrowed: float64 arithmetic then the same two roundings."""
    rng = np.random.default_rng(92 + pos)
    x = emu.f32_to_bf16((2.0 * rng.standard_normal(N * G * D)).astype(np.float32))
    cos, sin = fd.rope_row(pos)
    got = fd.rope(OPS, x, cos, sin, "N, G")
    xf = dc.f64(x, N * G, D)
    sw = np.concatenate([xf[:, D // 2:], xf[:, :D // 2]], axis=1)
    want = emu.f32_to_bf16((xf * dc.f64(cos) + sw * dc.f64(sin)).astype(np.float32)).reshape(-1)
    assert np.array_equal(got, want)
    if pos == 0:  # cos = 1, sin = 0: the identity
        assert np.array_equal(got, x)


def test_rope_tables_match_the_model():
    """rope_row against the model's emb = [freqs, freqs] (transformer.py:88-94) in float64: within
    one bf16 ulp (the tables are f32 arithmetic narrowed to bf16), the sine's first half negated."""
    pos = 1234
    inv = 1.0 / (fd.ROPE_THETA ** (np.arange(0, D, 2) / D))
    emb = np.concatenate([pos * inv, pos * inv])
    cos, sin = fd.rope_row(pos)
    sign = np.concatenate([-np.ones(D // 2), np.ones(D // 2)])
    assert np.all(np.abs(dc.f64(cos) - np.cos(emb)) <= 2.0 ** -8 + 1e-4)
    assert np.all(np.abs(dc.f64(sin) - sign * np.sin(emb)) <= 2.0 ** -8 + 1e-4)


# ---- projection (mod.rs:29-58) ---------------------------------------------------------------------

def scalar_projection_inputs(seed):
    rng = np.random.default_rng(seed)
    return dict(x=dc.seeded(rng, H, 0.25), wq=dc.seeded(rng, fd.Q * H, 0.1), wk=dc.seeded(rng, fd.P * H, 0.1),
                wv=dc.seeded(rng, fd.P * H, 0.1), g_in=dc.seeded(rng, H, 1.0), g_q=dc.seeded(rng, D, 1.0),
                g_k=dc.seeded(rng, D, 1.0))


def run_projection(ops, a, pos, k_cache, v_cache):
    cos, sin = fd.rope_row(pos)
    return fd.projection(ops, a["x"], a["wq"], a["wk"], a["wv"], a["g_in"], a["g_q"], a["g_k"],
                         pos * fd.ROW_STRIDE_ND, cos, sin, k_cache, v_cache)


def test_projection_scalar_reference():
    """transformer_tests.rs:92-214: offset 0, cos = 1, sin = 0; q, k and v within 0.08 + 0.08 |e|."""
    a = scalar_projection_inputs(0x517E)
    zero = np.zeros(T * N * D, np.uint16)
    q, kc, vc = run_projection(OPS, a, 0, zero, zero)
    qe, ke, ve = dc.projection_scalar(a["x"], a["wq"], a["wk"], a["wv"], a["g_in"], a["g_q"], a["g_k"])
    dc.assert_close(q, qe, 0.08, 0.08, "q")
    dc.assert_close(kc[:N * D], ke, 0.08, 0.08, "k")
    dc.assert_close(vc[:N * D], ve, 0.08, 0.08, "v")
    assert not kc[N * D:].any() and not vc[N * D:].any()


def model_projection_inputs(seed):
    """verify_projection (transformer.py:189-243): x from sample(), nn.Linear weights, norms near 1,
    caches of random rows."""
    rng = np.random.default_rng(seed)
    w = dc.layer_weights(rng)
    a = dict(x=dc.sample(rng, H), wq=w["q"], wk=w["k"], wv=w["v"], g_in=w["input_norm"], g_q=w["q_norm"],
             g_k=w["k_norm"])
    return a, dc.sample(rng, T * N * D), dc.sample(rng, T * N * D)


def projection_verdicts(a, pos, k_cache, v_cache, q, kc, vc):
    qm, km, vm = dc.projection_model(a["x"], a["wq"], a["wk"], a["wv"], a["g_in"], a["g_q"], a["g_k"], pos)
    rows = lambda c: c.reshape(T, N * D)
    others = np.arange(T) != pos
    untouched = (np.array_equal(rows(kc)[others], rows(k_cache)[others])
                 and np.array_equal(rows(vc)[others], rows(v_cache)[others]))
    return [accepted(qm, dc.f64(q))[0], accepted(km, dc.f64(rows(kc)[pos]))[0],
            accepted(vm, dc.f64(rows(vc)[pos]))[0], untouched]


def test_projection_matches_the_model():
    a, kc0, vc0 = model_projection_inputs(93)
    q, kc, vc = run_projection(OPS, a, 5, kc0, vc0)
    assert all(projection_verdicts(a, 5, kc0, vc0, q, kc, vc))


def test_planted_projection_mistakes_are_rejected():
    a, kc0, vc0 = model_projection_inputs(94)
    good = fd.rotate_half
    try:
        fd.rotate_half = lambda ops, x, rows: x  # RoPE without the half swap
        q, kc, vc = run_projection(OPS, a, 5, kc0, vc0)
    finally:
        fd.rotate_half = good
    v = projection_verdicts(a, 5, kc0, vc0, q, kc, vc)
    assert not v[0] and not v[1] and v[2]
    cos, sin = fd.rope_row(5)
    q, kc, vc = fd.projection(OPS, a["x"], a["wq"], a["wk"], a["wv"], a["g_in"], a["g_q"], a["g_k"],
                              5 * N * D, cos, sin, kc0, vc0)  # an element offset, not bytes: row 2
    assert not all(projection_verdicts(a, 5, kc0, vc0, q, kc, vc)[1:])


# ---- decoder (mod.rs:89-116) ------------------------------------------------------------------------

def run_decoder(ops, a):
    return fd.decoder(ops, a["x"], a["sum"], a["rx"], a["wo"], a["g_post"], a["up"], a["gate"], a["down"])


def test_decoder_scalar_reference():
    """transformer_tests.rs:558-643: sum = 1; the residual stream within 0.25 + 0.2 |e|."""
    rng = np.random.default_rng(0xDEC0DE)
    a = dict(x=dc.seeded(rng, fd.Q, 0.05), rx=dc.seeded(rng, H, 0.05), wo=dc.seeded(rng, H * fd.Q, 0.02),
             g_post=dc.seeded(rng, H, 1.0), up=dc.seeded(rng, L * H, 0.01), gate=dc.seeded(rng, L * H, 0.01),
             down=dc.seeded(rng, H * L, 0.01), sum=np.ones(N * G, np.float32))
    got = OPS.get(run_decoder(OPS, a), fd.BF16)
    want = dc.decoder_scalar(a["x"], a["rx"], a["wo"], a["g_post"], a["up"], a["gate"], a["down"])
    dc.assert_close(got, want, 0.25, 0.2, "residual")


def model_decoder_inputs(seed):
    """verify_decoder (transformer.py:284-313): x, rx from sample(), sum = 1 (the norm a no-op)."""
    rng = np.random.default_rng(seed)
    w = dc.layer_weights(rng)
    return dict(x=dc.sample(rng, fd.Q), rx=dc.sample(rng, H), wo=w["o"], g_post=w["post_norm"], up=w["up"],
                gate=w["gate"], down=w["down"], sum=np.ones(N * G, np.float32))


def test_decoder_matches_the_model():
    a = model_decoder_inputs(95)
    got = OPS.get(run_decoder(OPS, a), fd.BF16)
    want = dc.decoder_model(a["x"], a["rx"], a["wo"], a["g_post"], a["up"], a["gate"], a["down"])
    ok, rate = accepted(want, dc.f64(got))
    assert ok, rate


def test_planted_decoder_mistake_is_rejected():
    a = model_decoder_inputs(96)
    good = fd.residual
    calls = []

    def second_residual_dropped(ops, x, r):
        calls.append(1)
        return good(ops, x, r) if len(calls) == 1 else x
    try:
        fd.residual = second_residual_dropped
        got = OPS.get(run_decoder(OPS, a), fd.BF16)
    finally:
        fd.residual = good
    want = dc.decoder_model(a["x"], a["rx"], a["wo"], a["g_post"], a["up"], a["gate"], a["down"])
    assert not accepted(want, dc.f64(got))[0]


def test_decoder_step_wires_kernel_boundaries():
    """transformer_tests.rs:405-526: projection, the first attention chunk (every key attended) and
    the decoder with zero weights leave the residual stream unchanged (there within 0.05 + 0.05 |e|;
    the chain's zeros make it exact)."""
    rng = np.random.default_rng(0xDEC0DE + 1)
    x, rx = dc.seeded(rng, H, 0.2), dc.seeded(rng, H, 0.2)
    ones = lambda n: np.full(n, ONE, np.uint16)
    zeros = lambda n: np.zeros(n, np.uint16)
    cos, sin = np.full(D, ONE, np.uint16), zeros(D)
    q, kc, vc = fd.projection(OPS, x, zeros(fd.Q * H), zeros(fd.P * H), zeros(fd.P * H), ones(H), ones(D), ones(D),
                              0, cos, sin, zeros(T * N * D), zeros(T * N * D))
    _, sm, out = fd.attend(OPS, q, [kc], [vc], [np.ones(T, np.float32)])
    got = OPS.get(fd.decoder(OPS, out, sm, rx, zeros(H * fd.Q), zeros(H), zeros(L * H), zeros(L * H),
                             zeros(H * L)), fd.BF16)
    dc.assert_close(got, dc.f64(rx), 0.05, 0.05, "residual")
    assert np.array_equal(got, rx)


# ---- final layer (mod.rs:118-131) ------------------------------------------------------------------

def test_final_layer_scalar_reference():
    """transformer_tests.rs:663-695: only column 0 of the lm_head weight set, (row % 17) 0.01 - 0.08;
    the W real logits within 0.08 + 0.08 |e|, the padding rows (zero weights) zero."""
    rng = np.random.default_rng(0xF1A1)
    x, g = dc.seeded(rng, H, 0.1), dc.seeded(rng, H, 1.0)
    lm = np.zeros(fd.WP * H, np.uint16)
    rows = np.arange(fd.W)
    lm[rows * H] = emu.f32_to_bf16(((rows % 17) * 0.01 - 0.08).astype(np.float32))
    got = OPS.get(fd.final_layer(OPS, x, g, lm), fd.BF16)
    xn = dc.rms_scalar(dc.f64(x), g)
    dc.assert_close(got[:fd.W], xn[0] * ((rows % 17) * 0.01 - 0.08), 0.08, 0.08, "logits")
    assert not got[fd.W:].any()


def test_final_layer_matches_the_model():
    """verify_final_layer (transformer.py:316-341): lm_head(rms(x)) over the W real rows."""
    rng = np.random.default_rng(97)
    x, g = dc.sample(rng, H), dc.layer_weights(rng)["post_norm"]
    lm = dc.linear_init(rng, fd.WP, H)
    got = OPS.get(fd.final_layer(OPS, x, g, lm), fd.BF16)
    ok, rate = accepted(dc.final_model(x, g, lm), dc.f64(got[:fd.W]))
    assert ok, rate


# ---- one layer of the decode step (transformer.py:495-562) ----------------------------------------

def step_case(seed, pos):
    """A layer's weights, the token's hidden state and the caches of chunks 0..pos // T: earlier
    tokens' rows random, the rows from the token's on zero (a fresh cache)."""
    rng = np.random.default_rng(seed)
    lw = dc.layer_weights(rng)
    chunk, row = divmod(pos, T)
    caches = []
    for c in range(chunk + 1):
        k = dc.seeded(rng, T * N * D, 1.0).reshape(T, N * D)
        v = dc.seeded(rng, T * N * D, 1.0).reshape(T, N * D)
        if c == chunk:
            k[row:], v[row:] = 0, 0
        caches.append((k.reshape(-1), v.reshape(-1)))
    return lw, dc.seeded(rng, H, 1.0), caches


def step_model(lw, x, caches, pos):
    """The model's layer (transformer.py:113-150) in float64: projection, softmax attention over every
    key up to pos (the new row included), Decoder."""
    chunk, row = divmod(pos, T)
    q, k, v = dc.projection_model(x, lw["q"], lw["k"], lw["v"], lw["input_norm"], lw["q_norm"], lw["k_norm"], pos)
    ks = [c[0].copy() for c in caches]
    vs = [c[1].copy() for c in caches]
    ks[chunk].reshape(T, N * D)[row] = emu.f32_to_bf16(k.astype(np.float32))
    vs[chunk].reshape(T, N * D)[row] = emu.f32_to_bf16(v.astype(np.float32))
    masks = [np.ones(T, np.float32)] * chunk + [fd.causal_mask(row)]
    attn = dc.softmax_attention(emu.f32_to_bf16(q.astype(np.float32)), ks, vs, masks, bf16_logits=True)
    a = emu.f32_to_bf16(attn.reshape(-1).astype(np.float32))
    return dc.decoder_model(a, x, lw["o"], lw["post_norm"], lw["up"], lw["gate"], lw["down"])


def test_layer_step_matches_the_model():
    """One layer at position T + 88 (the second chunk, row 88) against the float64 model under the
    reference's acceptance test. (At a chunk's first rows the reference's max, taken over the masked
    zero keys too, and its bf16(p) numerator over an f32 sum move single-key outputs by up to about
    1% from the model's softmax, so the model check is made where many keys are attended.)"""
    pos = T + 88
    lw, x, caches = step_case(98, pos)
    want = step_model(lw, x, caches, pos)
    cs = list(caches)
    got = OPS.get(fd.layer_step(OPS, x, lw, pos, cs, *fd.rope_row(pos)), fd.BF16)
    ok, rate = accepted(want, dc.f64(got))
    assert ok, rate
    assert np.array_equal(cs[0][0], caches[0][0]) and np.array_equal(cs[0][1], caches[0][1])


@pytest.mark.parametrize("pos", [0, T - 1, 2 * T])
def test_layer_step_edge_positions(pos):
    """The first token, the last row of a chunk and the first row of a third chunk: the new K and V
    rows are the projection's, at the token's row of its chunk, every other row and every earlier
    chunk untouched, and a chunk's first row attends to its one key: the attention output is that
    key's value row, scaled by the reference's bf16(p) / (p + EPS) with p = exp(s - max(s, 0))
    (the max over the masked zero keys too, attention.rs:77-134, 370-392)."""
    chunk, row = divmod(pos, T)
    lw, x, caches = step_case(98 + pos, pos)
    cs = list(caches)
    st = {}
    fd.layer_step(OPS, x, lw, pos, cs, *fd.rope_row(pos), st)
    for c in range(chunk):
        assert np.array_equal(cs[c][0], caches[c][0]) and np.array_equal(cs[c][1], caches[c][1])
    for side, new_row in ((0, st["kr"]), (1, st["v"])):
        got = cs[chunk][side].reshape(T, -1)
        assert np.array_equal(got[row], new_row)
        assert np.array_equal(np.delete(got, row, axis=0), np.delete(caches[chunk][side].reshape(T, -1), row, axis=0))
    if row == 0 and chunk == 0:
        # s = bf16(q.k0 / sqrt(D)) per (n, g); p = exp(s - max(s, 0)); out = bf16(bf16(p) v) then
        # bf16(out / (p + EPS)): closed form in float64 with the narrows at those points
        q = dc.f64(st["q_out"], N, G, D)
        k0 = dc.f64(st["kr"], N, D)
        v0 = dc.f64(st["v"], N, D)
        s = dc.r16(np.einsum("ngd,nd->ng", q, k0) / np.float32(fd.SQRT_HEAD_DIM))
        p = np.exp(s - np.maximum(s, 0.0))
        out = dc.r16(dc.r16(p)[..., None] * v0[:, None, :])
        want = dc.r16(out / (p + np.float32(fd.EPS))[..., None])
        got = dc.f64(st["a"], N, G, D)
        assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 2.0 ** -20)) <= 2 ** -7


# ---- the token loop (Pipeline.step, transformer.py:425-566) -----------------------------------------

def tied_model(seed, layers=1, zero_layers=True):
    """An embedding table of random rows, tied to the lm_head (its first W rows, the padding zero),
    RMSNorm gains of 1 and layers of zero weights (each then leaves the residual stream as it is)."""
    rng = np.random.default_rng(seed)
    embed = emu.f32_to_bf16(rng.standard_normal(fd.W * H).astype(np.float32))
    lm = np.zeros(fd.WP * H, np.uint16)
    lm[:fd.W * H] = embed
    one = lambda n: np.full(n, ONE, np.uint16)
    zero = lambda n: np.zeros(n, np.uint16)
    lw = dict(q=zero(fd.Q * H), k=zero(fd.P * H), v=zero(fd.P * H), o=zero(H * fd.Q), up=zero(L * H),
              gate=zero(L * H), down=zero(H * L), input_norm=one(H), q_norm=one(D), k_norm=one(D), post_norm=one(H))
    if not zero_layers:
        lws = [dc.layer_weights(rng) for _ in range(layers)]
    else:
        lws = [lw] * layers
    return dict(embed=embed, layers=lws, final_norm=one(H), lm_head=lm)


def test_pipeline_with_identity_layers_repeats_the_last_token():
    """With zero layer weights every layer leaves the embedding unchanged, so the tied lm_head scores
    each vocabulary row by its dot product with the normalised embedding of the current token: the
    token's own row wins, and greedy decoding repeats the prompt's last token."""
    pipe = fd.Pipeline(OPS, tied_model(110))
    new, logits = pipe.generate([5, 1234], 2)
    assert new == [1234, 1234]
    assert fd.sample_token(logits[0]) == 5
    assert len(pipe.caches[0]) == 1 and not dc.f64(pipe.caches[0][0][0]).any()  # zero K rows (q, k, v = 0)
