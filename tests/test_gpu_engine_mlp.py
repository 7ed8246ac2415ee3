"""The decoder's RMSNorm and SiLU MLP (rmsnorm.rs:9-78, mlp.rs:9-150) at the engine's own layouts
through the C ABI (furiosa_hip/engine_mlp.py: SliceP4, the CustomBroadcast switch, SliceUG, the stash
passes, SliceD and the Broadcast1 switches), held to the bars of the logical-view chains
(test_gpu_decode.py) against those chains on the oracle:

  * rms within 1e-6 relative (an f32 sum of squares regrouped for parallelism), y within the
    `near` bar, and y bit-exact against the oracle's quotient by the device's own rms;
  * up and gate bit-exact, x = bf16(up * silu) within `near` (the device sigmoid goes through expf),
    the f32 down sums bit-exact when x is, and the output within `near`."""
import numpy as np
import pytest

import decode_chain as dc
import furiosa_hip.engine_mlp as em
from test_gpu_decode import near

pytestmark = pytest.mark.gpu


def test_engine_layout_rmsnorm_and_mlp_match_the_oracle(rt):
    x, w = dc.rms_inputs(83, "forward")
    _, up_w, gate_w, down_w = dc.mlp_inputs(84)
    print("engine-layout rmsnorm + mlp seeds 83, 84", flush=True)
    got = {}
    xn, y = em.decoder_tail(em.ops(rt), x, w, up_w, gate_w, down_w, got)
    rows, axis, n, _ = dc.RMS_FORMS["forward"]
    cpu = dc.CpuOps(dc.RMS_SIZES)
    rms_w, xn_w = dc.rmsnorm(cpu, x, w, rows, axis, n)
    np.testing.assert_allclose(got["rms"][:1], rms_w, rtol=1e-6)
    near(xn, xn_w)
    assert np.array_equal(xn, dc.rmsnorm(cpu, x, w, rows, axis, n, rms=got["rms"][:1])[1])
    want = {}
    y_w = dc.mlp(dc.CpuOps(dc.MLP_SIZES), xn, up_w, gate_w, down_w, want)
    assert np.array_equal(got["up"], want["up"]) and np.array_equal(got["gate"], want["gate"])
    near(got["x"], want["x"])
    if np.array_equal(got["x"], want["x"]):
        assert np.array_equal(got["down"].view(np.uint32), want["down"].view(np.uint32))
    near(y, y_w)
