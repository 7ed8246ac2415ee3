"""The engine-layout decode attention stream (furiosa_hip/engine_attention.py) on the oracle against
the logical-view chain on the oracle (furiosa_hip/decode.py through tests/decode_chain.py): the
transcription of attention.rs's stages into seam calls at the reference's layouts must give the
same bits, since no layout changes the order of any fold. The oracle's brute-force mapping resolver
walks every cell of the padded layouts (Slice m![1 # 256] keeps one live slice in 256), so the first
chunk takes about two and a half minutes here: marked slow."""
import numpy as np
import pytest

import decode_chain as dc
import furiosa_hip.engine_attention as ea
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
