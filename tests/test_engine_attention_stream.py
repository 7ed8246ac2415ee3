"""The engine-layout decode streams (furiosa_hip/engine_attention.py, furiosa_hip/engine_mlp.py) on the
oracle against the logical-view chains on the oracle. The attention stream (engine_attention.py) against
the logical-view chain on the oracle (furiosa_hip/decode.py through tests/decode_chain.py): the
transcription of attention.rs's stages into seam calls at the reference's layouts must give the
same bits, since no layout changes the order of any fold. The oracle's brute-force mapping resolver
walks every cell of the padded layouts (Slice m![1 # 256] keeps one live slice in 256), so the first
chunk takes about two and a half minutes here: marked slow."""
import numpy as np
import pytest

import decode_chain as dc
import furiosa_hip.engine_attention as ea
import furiosa_hip.engine_mlp as em
from engine_attention_cpu import CpuEngineOps


@pytest.mark.slow
def test_engine_layout_stream_equals_the_logical_chain_on_the_oracle():
    q, ks, vs, masks = dc.inputs(61, 1, 300, scale=1.0)
    e = CpuEngineOps()
    got, want = [], []
    mx, sm, out, y = ea.attend(e, q, ks, vs, masks, got)
    wm, ws, wo, wy = dc.decode(dc.CpuOps(), q, ks, vs, masks, want)
    assert np.array_equal(mx.view(np.uint32), wm.view(np.uint32))
    assert np.array_equal(sm.view(np.uint32), ws.view(np.uint32))
    assert np.array_equal(out, wo) and np.array_equal(y, wy)
    assert e.calls > 100  # every stage issued as its own seam call


@pytest.mark.slow
def test_engine_layout_rmsnorm_and_mlp_equal_the_logical_chains_on_the_oracle():
    """rmsnorm.rs forward and mlp.rs forward at their layouts: every sum in ascending order of its
    axis, as in the logical chains, so every stage is bit-exact."""
    x, w = dc.rms_inputs(83, "forward")
    _, up_w, gate_w, down_w = dc.mlp_inputs(84)
    got = {}
    xn, y = em.decoder_tail(CpuEngineOps(em.SIZES), x, w, up_w, gate_w, down_w, got)
    rows, axis, n, _ = dc.RMS_FORMS["forward"]
    rms_w, xn_w = dc.rmsnorm(dc.CpuOps(dc.RMS_SIZES), x, w, rows, axis, n)
    assert np.array_equal(got["rms"][:1].view(np.uint32), np.asarray(rms_w, np.float32).view(np.uint32))
    assert np.array_equal(xn, xn_w)
    want = {}
    y_w = dc.mlp(dc.CpuOps(dc.MLP_SIZES), xn, up_w, gate_w, down_w, want)
    for k in ("up", "gate", "x"):
        assert np.array_equal(got[k], want[k]), k
    assert np.array_equal(got["down"].view(np.uint32), want["down"].view(np.uint32))
    assert np.array_equal(y, y_w)
