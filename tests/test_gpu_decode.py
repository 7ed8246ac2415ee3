"""The decode chains (attention.rs:226-392 and mlp.rs:9-150, stages in decode_chain.py) through the
C ABI at the reference's shapes against the oracle. Attention runs at N = 8, G = 2, D = 128, T = 512
keys per chunk, with the running max, sum and output kept in device buffers across the chunk
launches and compared after every chunk.

Bars, stage by stage:
  * max: bit-exact. The logits are exact (a serial f32 fold over D, an f32 division, one narrow) and
    a max does not depend on its order.
  * sum: relative 1e-5. The device exp is held to a tolerance, not bit parity (an ulp or two of
    expf), and the f32 sum over 512 keys is regrouped for parallelism (buf.rs:316-330 leaves the order
    of an f32 fold free); both are orders of magnitude inside 1e-5.
  * out: bit-exact on at least 99.9% of the outputs and within 2 bf16 ulps everywhere. An ulp of exp
    moves bf16(p) only when it crosses a rounding boundary of bf16 (about one key in 2^15), and
    then one partial product by an ulp.
and the normalised output passes the reference's own acceptance test (transformer.py:169-186)
against the model's softmax attention.
"""
import numpy as np
import pytest

import decode_chain as dc
from oracle import emulator as emu
from test_oracle_decode import accepted

pytestmark = pytest.mark.gpu


def ulp(x):
    """bf16 ulp of each value (the spacing at its exponent; 2^-133 below the normal range)."""
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -126)))
    return 2.0 ** (e - 7)


def near(got_bits, want_bits):
    g, w = emu.bf16_to_f32(got_bits).astype(np.float64), emu.bf16_to_f32(want_bits).astype(np.float64)
    exact = np.mean(got_bits == want_bits)
    worst = float(np.max(np.abs(g - w) / ulp(w)))
    assert exact >= 0.999 and worst <= 2.0, (exact, worst)


CASES = [
    dict(seed=60, chunks=1, valid=6, uniform=True),  # transformer.py:245-256's own check
    dict(seed=61, chunks=3, valid=300, scale=1.0),   # two full chunks, then the causal one
    dict(seed=62, chunks=2, valid=512, scale=1.0),   # every key of the last chunk attended
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"chunks{c['chunks']}_valid{c['valid']}")
def test_decode_chain_matches_the_oracle(rt, case):
    q, ks, vs, masks = dc.inputs(case["seed"], case["chunks"], case["valid"], scale=case.get("scale", 1.0),
                                 uniform=case.get("uniform", False))
    print(f"decode chain seed {case['seed']} chunks {case['chunks']} valid {case['valid']}", flush=True)
    got_stages, want_stages = [], []
    _, _, _, y = dc.decode(dc.GpuOps(rt), q, ks, vs, masks, got_stages)
    _, _, _, y_want = dc.decode(dc.CpuOps(), q, ks, vs, masks, want_stages)
    for c, ((gm, gs, go), (wm, ws, wo)) in enumerate(zip(got_stages, want_stages)):
        assert np.array_equal(gm.view(np.uint32), wm.view(np.uint32)), f"max after chunk {c}"
        np.testing.assert_allclose(gs, ws, rtol=1e-5, err_msg=f"sum after chunk {c}")
        near(go, wo)
    near(y, y_want)
    ok, rate = accepted(dc.softmax_attention(q, ks, vs, masks, bf16_logits=True), emu.bf16_to_f32(y))
    assert ok and rate == 1.0, rate


def test_mlp_matches_the_oracle(rt):
    """mlp.rs:9-150 at H = 1024, L = 3072: up, gate and the f32 down sums bit-exact (serial folds of
    the narrow sources); the device sigmoid (through expf) within ulps, so the product x and the
    output carry the exp bar above."""
    x, up_w, gate_w, down_w = dc.mlp_inputs(72)
    print("mlp chain seed 72", flush=True)
    got, want = {}, {}
    y = dc.mlp(dc.GpuOps(rt, dc.MLP_SIZES), x, up_w, gate_w, down_w, got)
    y_want = dc.mlp(dc.CpuOps(dc.MLP_SIZES), x, up_w, gate_w, down_w, want)
    assert np.array_equal(got["up"], want["up"]) and np.array_equal(got["gate"], want["gate"])
    near(got["x"], want["x"])
    if np.array_equal(got["x"], want["x"]):
        assert np.array_equal(got["down"].view(np.uint32), want["down"].view(np.uint32))
    near(y, y_want)
    ok, rate = accepted(dc.mlp_float(x, up_w, gate_w, down_w), emu.bf16_to_f32(y))
    assert ok and rate == 1.0, rate



@pytest.mark.parametrize("form", list(dc.RMS_FORMS))
def test_rmsnorm_forms_match_the_oracle(rt, form):
    """rmsnorm.rs forward (H = 1024), forward_q ([N, G, D]) and forward_k ([N, D]): the f32 sums of
    squares regrouped on the GPU (within 1e-6), so y = bf16(x w / rms) may move by one ulp where the
    quotient sits at a rounding boundary."""
    rows, axis, n, _ = dc.RMS_FORMS[form]
    x, w = dc.rms_inputs(82, form)
    print(f"rmsnorm {form}", flush=True)
    rms, y = dc.rmsnorm(dc.GpuOps(rt, dc.RMS_SIZES), x, w, rows, axis, n)
    rms_w, y_w = dc.rmsnorm(dc.CpuOps(dc.RMS_SIZES), x, w, rows, axis, n)
    rms, y = dc.GpuOps(rt).get(rms, dc.F32), dc.GpuOps(rt).get(y, dc.BF16)
    np.testing.assert_allclose(rms, rms_w, rtol=1e-6)
    near(y, y_w)
    # with the device's own rms the quotient's rounding leaves no freedom
    assert np.array_equal(y, dc.rmsnorm(dc.CpuOps(dc.RMS_SIZES), x, w, rows, axis, n, rms=rms)[1])



def test_reference_running_max_persists(rt):
    """transformer_tests.rs:252-289 through the seam ops: the max stored after the third chunk is
    sqrt(D), as the oracle's."""
    from test_oracle_decode import running_max_case
    case = running_max_case()
    mx, sm, out, _ = dc.decode(dc.GpuOps(rt), *case)
    mx_w, sm_w, out_w, _ = dc.decode(dc.CpuOps(), *case)
    assert np.array_equal(mx.view(np.uint32), mx_w.view(np.uint32))
    assert np.all(np.abs(mx - np.sqrt(dc.D)) < 0.05)
    np.testing.assert_allclose(sm, sm_w, rtol=1e-5)
    assert np.array_equal(out, out_w)
