"""Recorded op streams (fo_graph_begin / fo_graph_end / fo_graph_launch, the compile-once,
launch-per-call model of runtime.rs:157-177) on the decode step's seam calls.

A launch runs the kernels the recording issued, with the same arguments, so its results are those of
the same calls issued eagerly, bit for bit: every test below holds launches to the eager seam calls
on the same inputs, with eager work and synchronizations between launches, and each launch checked.
"""
import numpy as np
import pytest

import decode_chain as dc
import furiosa_hip as fh
import furiosa_hip.decode as fd
from oracle import emulator as emu
from test_oracle_step import step_case, tied_model

pytestmark = pytest.mark.gpu
BF16, F32, T, D = fd.BF16, fd.F32, fd.T, fd.D


@pytest.fixture(autouse=True)
def _no_open_recording(rt):
    """The session's runtime is shared: a test that fails while recording closes the recording."""
    yield
    try:
        rt.graph_end().free()
    except fh.FoError:
        pass


def _inputs(rt, pos, x):
    cos, sin = fd.rope_row(pos)
    row = pos % T
    return dict(x=rt.upload(x), cos=rt.upload(cos), sin=rt.upload(sin), mask=rt.upload(fd.causal_mask(row)),
                offset=rt.upload(np.array([row * fd.ROW_STRIDE_ND], np.int32)))


def _rewrite(inp, pos, x):
    cos, sin = fd.rope_row(pos)
    row = pos % T
    for name, v in (("x", x), ("cos", cos), ("sin", sin), ("mask", fd.causal_mask(row)),
                    ("offset", np.array([row * fd.ROW_STRIDE_ND], np.int32))):
        inp[name].write(v)


def test_recorded_layer_matches_eager_calls(rt):
    """One decode layer (projection with RoPE and both cache rows, attention over two chunks, decoder
    with the MLP: GEMVs, reduces, zips, maps, broadcast relayouts, tile copies into zeroed buffers,
    the cache scatters) recorded once at position T + 3, then launched for four positions of the same
    chunk against the eager layer on copies of the same caches: outputs and both caches bit-exact
    after every launch."""
    pos0 = T + 3
    lw, x0, caches = step_case(120, pos0)
    ops = fd.SeamOps(rt, fd.STEP_SIZES)
    w = {k: ops.put(v) for k, v in lw.items()}
    full = rt.upload(np.ones(T, np.float32))
    g_caches = [(rt.upload(k), rt.upload(v)) for k, v in caches]
    e_caches = [(rt.upload(k), rt.upload(v)) for k, v in caches]
    inp = _inputs(rt, pos0, x0)
    print("record one layer at pos", pos0, flush=True)
    rt.graph_begin()
    out = fd.layer_step(ops, inp["x"], w, pos0, list(g_caches), inp["cos"], inp["sin"], masks=[full, inp["mask"]],
                        offset=inp["offset"])
    graph = rt.graph_end()
    rng = np.random.default_rng(121)
    for pos in (pos0, pos0 + 1, T + 200, 2 * T - 1):
        x = dc.seeded(rng, fd.H, 1.0)
        _rewrite(inp, pos, x)
        print("launch at pos", pos, flush=True)
        graph.launch()
        got = ops.get(out, BF16)
        e_inp = _inputs(rt, pos, x)
        want = fd.layer_step(ops, e_inp["x"], w, pos, e_caches, e_inp["cos"], e_inp["sin"],
                             masks=[full, e_inp["mask"]], offset=e_inp["offset"])
        rt.sync()
        assert np.array_equal(got, ops.get(want, BF16)), pos
        for (gk, gv), (ek, ev) in zip(g_caches, e_caches):
            assert np.array_equal(ops.get(gk, BF16), ops.get(ek, BF16)), pos
            assert np.array_equal(ops.get(gv, BF16), ops.get(ev, BF16)), pos
    graph.free()


def test_recorded_pipeline_matches_eager_pipeline(rt):
    """Pipeline.step with graphs: one recording per chunk count (positions 0 and T open chunks 0 and
    1), launched for every later token of that count; the logits equal the eager pipeline's, bit for
    bit, over a prompt, greedy tokens and a jump across the chunk boundary."""
    model = tied_model(130, layers=2, zero_layers=False)
    eager = fd.Pipeline(fd.SeamOps(rt, fd.STEP_SIZES), model)
    graphed = fd.Pipeline(fd.SeamOps(rt, fd.STEP_SIZES), model, graphs=True)
    tok = 17
    for pos in (0, 1, 2, 3, T - 1, T, T + 1):
        print("pipeline pos", pos, flush=True)
        want, got = eager.step(tok, pos), graphed.step(tok, pos)
        assert np.array_equal(got, want), pos
        tok = fd.sample_token(want)
    assert sorted(graphed.graphs) == [0, 1]


def test_recording_memory_stays_with_the_graph(rt):
    """Blocks handed out while recording (the output, and intermediates freed inside the recording)
    are not given to buffers allocated after it: buffers of every size the recording used, allocated
    and filled after fo_graph_end, keep their contents across launches, and the launches' results
    stay right."""
    n = 4096
    a = rt.upload(np.arange(n, dtype=np.float32))
    b = rt.upload(np.full(n, 2.0, np.float32))
    rt.graph_begin()
    t1 = rt.alloc(n * 4)
    rt.map(t1, F32, a, F32, n, fh.op("EXP"))
    t2 = rt.alloc(n * 4)
    rt.zip_with(t2, F32, t1, b, F32, n, fh.op("MUL_F"))
    del t1
    out = rt.alloc(n * 4)
    rt.zip_with(out, F32, t2, a, F32, n, fh.op("ADD_F"))
    del t2
    graph = rt.graph_end()
    others = [rt.upload(np.full(n, 7.0 + i, np.float32)) for i in range(8)]
    for step in range(3):
        v = np.linspace(-3, 3, n, dtype=np.float32) + step
        a.write(v)
        graph.launch()
        t = rt.alloc(n * 4)
        rt.map(t, F32, a, F32, n, fh.op("EXP"))
        u = rt.alloc(n * 4)
        rt.zip_with(u, F32, t, b, F32, n, fh.op("MUL_F"))
        want = rt.alloc(n * 4)
        rt.zip_with(want, F32, u, a, F32, n, fh.op("ADD_F"))
        rt.sync()
        assert np.array_equal(out.read(F32), want.read(F32)), step
        for i, o in enumerate(others):
            assert np.all(o.read(F32) == 7.0 + i), (step, i)
    graph.free()


def test_recording_rejects_calls_that_wait(rt):
    """Calls that wait for the device fail while recording, and leave it open; a second begin and a
    launch fail too; fo_graph_end closes it, and a launch of the result then works."""
    x = rt.upload(np.ones(256, np.float32))
    y = rt.alloc(256 * 4)
    rt.graph_begin()
    other = rt.graph_end()
    rt.graph_begin()
    rt.map(y, F32, x, F32, 256, fh.op("EXP"))
    for call in (lambda: x.write(np.zeros(256, np.float32)), lambda: x.read(F32), rt.sync, rt.graph_begin,
                 lambda: rt.record(0), other.launch):
        with pytest.raises(fh.FoError, match="graph"):
            call()
    graph = rt.graph_end()
    with pytest.raises(fh.FoError, match="no graph"):
        rt.graph_end()
    graph.launch()
    assert np.allclose(y.read(F32), np.e, rtol=1e-6)
    graph.free()
    other.free()


def test_recorded_widen_of_a_dropped_narrow(rt):
    """Narrow into a temporary, widen it, drop the temporary, read the widen: once inside the
    recording, and once with the temporary dropped before fo_graph_begin and its widen read inside
    the recording. Launches for three inputs, each followed by buffers of both sizes allocated and
    written, equal the numpy result of the chain; the later buffers keep their contents."""
    n = 4096
    rng = np.random.default_rng(41)
    x = rt.upload(rng.standard_normal(n).astype(np.float32))
    b = rt.upload(rng.standard_normal(n).astype(np.float32))

    def narrow_widen(src):
        t = rt.alloc(2 * n)
        rt.map(t, BF16, src, F32, n, fh.op("CAST"))
        w = rt.alloc(4 * n)
        rt.map(w, F32, t, BF16, n, fh.op("CAST"))
        return w  # t dropped here

    x0 = rt.upload(rng.standard_normal(n).astype(np.float32))
    w0 = narrow_widen(x0)
    rt.graph_begin()
    w = narrow_widen(x)
    out = rt.alloc(4 * n)
    rt.zip_with(out, F32, w, b, F32, n, fh.op("MUL_F"))
    del w
    out0 = rt.alloc(4 * n)
    rt.zip_with(out0, F32, w0, b, F32, n, fh.op("ADD_F"))
    graph = rt.graph_end()  # w0 is an input of the graph: it stays alive while the graph does
    bv = b.read(F32)
    want0 = emu.bf16_to_f32(emu.f32_to_bf16(x0.read(F32))) + bv
    for step in range(3):
        v = rng.standard_normal(n).astype(np.float32) * (step + 1)
        x.write(v)
        print("launch", step, flush=True)
        graph.launch()
        others = [rt.upload(np.full(m, 0x3F80 + i, np.uint16)) for i, m in enumerate((n, 2 * n, n, 2 * n))]
        want = emu.bf16_to_f32(emu.f32_to_bf16(v)) * bv
        assert np.array_equal(out.read(F32), want), step
        assert np.array_equal(out0.read(F32), want0), step
        for i, o in enumerate(others):
            assert np.all(o.read(np.uint16) == 0x3F80 + i), (step, i)
    graph.free()
