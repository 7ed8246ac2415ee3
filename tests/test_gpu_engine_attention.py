"""The reference decode attention (attention.rs:18-392) at the engine's own layouts through the C
ABI: every fetch, switch, collect, commit, cast, tag and vector-engine pass of forward_first,
forward and norm on Cluster m![1 # 2], Slice m![1 # 256], SliceQK m![T / 8, 1 # 4] and SliceQV
m![N, T / 16] (furiosa_hip/engine_attention.py), held to the same bars as the logical-view chain
(test_gpu_decode.py) against that chain on the oracle:

  * max bit-exact; sum relative 1e-5; out and the normalised output bit-exact on >= 99.9% of the
    cells and within 2 bf16 ulps everywhere;
  * the normalised output passes the reference's own acceptance test (transformer.py:169-186).

The layouts move every value but change the order of no fold: the f32 sums over T and over the
T / 16 slices run in ascending key order, as in the logical chain. The stream itself was checked
on the oracle against the logical chain (tests/test_engine_attention_stream.py, bit-exact)."""
import numpy as np
import pytest

import decode_chain as dc
import furiosa_hip.engine_attention as ea
from oracle import emulator as emu
from test_gpu_decode import CASES, near
from test_oracle_decode import accepted

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"chunks{c['chunks']}_valid{c['valid']}")
def test_engine_layout_attention_matches_the_oracle(rt, case):
    q, ks, vs, masks = dc.inputs(case["seed"], case["chunks"], case["valid"], scale=case.get("scale", 1.0),
                                 uniform=case.get("uniform", False))
    print(f"engine-layout attention seed {case['seed']} chunks {case['chunks']} valid {case['valid']}", flush=True)
    got_stages, want_stages = [], []
    e = ea.EngineOps(rt)
    _, _, _, y = ea.attend(e, q, ks, vs, masks, got_stages)
    _, _, _, y_want = dc.decode(dc.CpuOps(), q, ks, vs, masks, want_stages)
    for c, ((gm, gs, go), (wm, ws, wo)) in enumerate(zip(got_stages, want_stages)):
        assert np.array_equal(gm.view(np.uint32), wm.view(np.uint32)), f"max after chunk {c}"
        np.testing.assert_allclose(gs, ws, rtol=1e-5, err_msg=f"sum after chunk {c}")
        near(go, wo)
    near(y, y_want)
    ok, rate = accepted(dc.softmax_attention(q, ks, vs, masks, bf16_logits=True), emu.bf16_to_f32(y))
    assert ok and rate == 1.0, rate
