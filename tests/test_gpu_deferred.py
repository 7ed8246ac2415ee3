"""The runtime's deferred forms (zero fills, widening and narrowing casts, f32 map chains, whole-buffer
broadcasts, read through by the ops that consume them) against a runtime that defers nothing.

`rt_eager` is created with FO_EAGER=1: every zero fill runs at allocation and every cast, map chain
and broadcast when it is issued, the plain reading of each Backend call (storage/buf.rs:203-447).
The same seeded sequences of seam calls run on both runtimes, interleaved with host writes, frees,
reads and recorded graphs launched between eager calls, and every live buffer must come out the same
bit for bit (NaNs compared as NaNs).

Also here: regressions for records that outlive a write they were not told of -- a graph launch
writes buffers without passing through the records, so a widen record whose cast has already run
must not survive a launch, nor be taken into a recording.
"""
import numpy as np
import pytest

import furiosa_hip as fh
from oracle import emulator as emu
from oracle import mapping_ref as mr

pytestmark = pytest.mark.gpu

BF16, F32 = fh.BF16, fh.F32
R, C = 16, 256
N = R * C
SIZES = dict(R=R, C=C, N=R, K=C)
# full views of the N-element buffers: consecutive relayouts between them compose (direct form)
VIEWS = ("R, C", "C, R", "R / 4, C, R % 4", "C / 64, R, C % 64")


def bf16_values(rng, n):
    """bf16 bits: N(0, 2) values, with zeros of both signs, subnormals (which the widen reads as
    zero) and an occasional NaN."""
    bits = emu.f32_to_bf16((2.0 * rng.standard_normal(n)).astype(np.float32))
    kind = rng.integers(0, 40, n)
    bits[kind == 1] = (rng.integers(1, 0x80, int((kind == 1).sum())) | 0x8000).astype(np.uint16)
    bits[kind == 2] = np.uint16(0x8000)
    bits[kind == 3] = np.uint16(0x7FC1)
    return bits


def f32_values(rng, n):
    v = (rng.standard_normal(n) * np.float32(10.0) ** rng.integers(-2, 3, n)).astype(np.float32)
    u = v.view(np.uint32)
    u[::11] = (u[::11] & 0xFFFF0000) | 0x8000  # ties of the bf16 narrow
    u[5::97] = 0x00000003  # f32 subnormal
    return v


def same_bits(a, b, dtype):
    a, b = np.asarray(a), np.asarray(b)
    if dtype == F32:
        nan = np.isnan(a) & np.isnan(b)
        return np.array_equal(a.view(np.uint32)[~nan], b.view(np.uint32)[~nan]) and np.array_equal(
            np.isnan(a), np.isnan(b))
    fa, fb = emu.bf16_to_f32(a), emu.bf16_to_f32(b)
    nan = np.isnan(fa) & np.isnan(fb)
    return np.array_equal(a[~nan], b[~nan]) and np.array_equal(np.isnan(fa), np.isnan(fb))


class Slot:
    def __init__(self, bufs, dtype, length):
        self.bufs, self.dtype, self.length = bufs, dtype, length
        self.view = VIEWS[0]  # the view a relayout last wrote it with (its next relayout reads it so)

    @property
    def nbytes(self):
        return self.length * (4 if self.dtype == F32 else 2)


UNARY = [("EXP", 0, 0.0), ("TANH", 0, 0.0), ("SIGMOID", 0, 0.0), ("SQRT", 0, 0.0), ("MUL_F", fh.RHS_IMM, 0.37),
         ("ADD_F", fh.RHS_IMM, 1e-6), ("DIV_F", fh.RHS_IMM, 3.0), ("NEG_EXP", 0, 0.0)]
BINARY = [("ADD_F", 0), ("SUB_F", 0), ("SUB_F", fh.SWAP), ("MUL_F", 0), ("DIV_F", 0)]


class Twin:
    """One sequence of seam calls issued on both runtimes (index 0: deferred, 1: eager)."""

    def __init__(self, rts, seed):
        self.rts = rts
        self.rng = np.random.default_rng(seed)
        self.slots = []
        self.pinned = set()
        self.recording = False  # no host writes while recording: src buffers must already exist
        self.log = []
        self.views = {t: fh.m(t, **SIZES) for t in ("R", "C", "R, C", "K", "N, K", "N") + VIEWS}

    # -- buffers --
    def new(self, dtype, length, data=True):
        assert not (data and self.recording), "a source is created before the recording"
        s = Slot([rt.alloc(length * (4 if dtype == F32 else 2)) for rt in self.rts], dtype, length)
        if data:
            self.write(s)
        self.slots.append(s)
        return s

    def write(self, s):
        v = bf16_values(self.rng, s.length) if s.dtype == BF16 else f32_values(self.rng, s.length)
        for b in s.bufs:
            b.write(v)

    def pick(self, dtype, length, exclude=()):
        c = [s for s in self.slots if s.dtype == dtype and s.length == length and s not in exclude]
        return c[self.rng.integers(len(c))] if c else None

    def src(self, dtype, length):
        s = self.pick(dtype, length)
        return s if s is not None else self.new(dtype, length)

    def dst(self, dtype, length, exclude=()):
        """An output: a fresh buffer (whose zero fill the op may drop) or an existing one."""
        s = None if self.rng.random() < 0.6 else self.pick(dtype, length, exclude)
        return s if s is not None else self.new(dtype, length, data=False)

    def check(self, s, what):
        got = [b.read(s.dtype, s.length) for b in s.bufs]
        assert same_bits(got[0], got[1], s.dtype), f"{what}: deferred and eager differ after {self.log[-12:]}"

    def check_all(self, what):
        for s in self.slots:
            self.check(s, what)

    # -- seam calls --
    def op(self, allowed):
        kind = allowed[self.rng.integers(len(allowed))]
        length = [N, R, C][self.rng.integers(3)]
        if kind == "widen":
            src = self.src(BF16, length)
            d = self.dst(F32, length)
            for i, rt in enumerate(self.rts):
                rt.map(d.bufs[i], F32, src.bufs[i], BF16, length, fh.op("CAST"))
        elif kind == "narrow":
            src = self.src(F32, length)
            d = self.dst(BF16, length)
            for i, rt in enumerate(self.rts):
                rt.map(d.bufs[i], BF16, src.bufs[i], F32, length, fh.op("CAST"))
        elif kind == "unary":
            src = self.src(F32, length)
            d = src if self.rng.random() < 0.1 else self.dst(F32, length)
            name, flags, imm = UNARY[self.rng.integers(len(UNARY))]
            o = fh.op(name, flags, imm)
            for i, rt in enumerate(self.rts):
                rt.map(d.bufs[i], F32, src.bufs[i], F32, length, o)
            kind += f":{name}"
        elif kind == "zip":
            a = self.src(F32, length)
            b = self.src(F32, length)
            d = self.dst(F32, length)
            name, flags = BINARY[self.rng.integers(len(BINARY))]
            o = fh.op(name, flags)
            for i, rt in enumerate(self.rts):
                rt.zip_with(d.bufs[i], F32, a.bufs[i], b.bufs[i], F32, length, o)
            kind += f":{name}"
        elif kind == "bcast":  # a per-row value over its row, or a row vector over every row
            sv = "R" if self.rng.random() < 0.5 else "C"
            src = self.src(F32, R if sv == "R" else C)
            d = self.dst(F32, N)
            for i, rt in enumerate(self.rts):
                rt.transpose(d.bufs[i], src.bufs[i], F32, self.views[sv], self.views["R, C"], allow_broadcast=True)
            kind += f":{sv}"
        elif kind == "reduce":
            src = self.src(F32, N)
            dv = "R" if self.rng.random() < 0.5 else "C"
            d = self.dst(F32, R if dv == "R" else C)
            red, ident = (fh.RED["ADD"], 0) if self.rng.random() < 0.7 else (fh.RED["MAX"], 0xFF800000)
            for i, rt in enumerate(self.rts):
                rt.reduce(d.bufs[i], src.bufs[i], F32, self.views["R, C"], self.views[dv], red, ident)
            kind += f":{dv}"
        elif kind == "gemv":  # the decode step's projection: one vector against weight rows
            x = self.src(F32, C)
            w = self.src(F32, N)
            d = self.dst(F32, R, exclude=(x, w))
            for i, rt in enumerate(self.rts):
                rt.contraction(d.bufs[i], x.bufs[i], w.bufs[i], F32, F32, self.views["K"], self.views["N, K"],
                               self.views["N, K"], self.views["N"])
        elif kind == "relayout":  # full-view transposes: consecutive ones compose into one pass
            dtype = BF16 if self.rng.random() < 0.5 else F32
            src = self.src(dtype, N)
            sv = src.view if self.rng.random() < 0.8 else VIEWS[self.rng.integers(len(VIEWS))]
            dv = VIEWS[self.rng.integers(len(VIEWS))]
            d = self.dst(dtype, N, exclude=(src,))
            for i, rt in enumerate(self.rts):
                rt.transpose(d.bufs[i], src.bufs[i], dtype, self.views[sv], self.views[dv])
            d.view = dv
            kind += f":{sv}->{dv}"
        elif kind == "write":
            s = self.slots[self.rng.integers(len(self.slots))]
            self.write(s)
        elif kind == "free":
            kinds = {}
            for s in self.slots:
                kinds.setdefault((s.dtype, s.length), []).append(s)
            # one buffer of each kind stays, so a recording always finds its sources
            free = [s for s in self.slots if s not in self.pinned and len(kinds[(s.dtype, s.length)]) > 1]
            if free:
                s = free[self.rng.integers(len(free))]
                self.slots.remove(s)
                for b in s.bufs:
                    b.free()
        elif kind == "read":
            self.check(self.slots[self.rng.integers(len(self.slots))], "read")
        self.log.append(kind)

    def graph(self):
        """A few calls recorded on both runtimes, launched, then launched again after eager calls and
        a host write into one of the buffers the recording reads."""
        before = set(self.slots)
        for rt in self.rts:
            rt.graph_begin()
        self.recording = True
        try:
            for _ in range(int(self.rng.integers(2, 7))):
                self.op(["widen", "narrow", "unary", "zip", "bcast", "reduce", "gemv", "relayout"])
        finally:
            self.recording = False
            graphs = [rt.graph_end() for rt in self.rts]
        self.log.append("graph")
        self.pinned = set(self.slots)  # the graphs may touch any of them
        for g in graphs:
            g.launch()
        self.check_all("first launch")
        for _ in range(int(self.rng.integers(0, 4))):
            self.op(["widen", "narrow", "unary", "zip", "bcast", "reduce", "gemv", "relayout", "read"])
        inputs = [s for s in before if s in self.slots]
        if inputs:
            self.write(inputs[self.rng.integers(len(inputs))])
        for g in graphs:
            g.launch()
        self.log.append("relaunch")
        self.check_all("second launch")
        for g in graphs:
            g.free()
        self.pinned = set()


@pytest.mark.parametrize("seed", range(6))
def test_deferred_matches_eager(rt, rt_eager, seed):
    """200 seeded seam calls (widens, narrows, f32 maps, zips, broadcasts, row and column reduces,
    GEMVs, full-view relayouts, host writes, frees, reads and recorded graphs) on the deferring runtime and on the eager
    one: every buffer equal, bit for bit, at every read and at the end."""
    print(f"deferred vs eager, seed {seed}", flush=True)
    tw = Twin((rt, rt_eager), 1000 + seed)
    for dtype, length in ((BF16, N), (F32, N), (BF16, C), (F32, C), (F32, R), (BF16, R)):
        tw.new(dtype, length)
    ops = ["widen"] * 4 + ["narrow"] * 3 + ["unary"] * 4 + ["zip"] * 4 + ["bcast"] * 2 + ["reduce"] * 2 + \
          ["gemv"] * 2 + ["relayout"] * 4 + ["write", "free", "free", "read"]
    for step in range(200):
        if tw.rng.random() < 0.04:
            tw.graph()
        else:
            tw.op(ops)
    tw.check_all("end")
    for s in tw.slots:
        for b in s.bufs:
            b.free()


def _gemv_case(rng):
    s = dict(N=16, K=64)
    maps = [fh.m(t, **s) for t in ("K", "N, K", "N, K", "N")]
    lo, ro, po, oo = (mr.parse(t, s) for t in ("K", "N, K", "N, K", "N"))
    x0 = emu.f32_to_bf16(rng.standard_normal(64).astype(np.float32))
    x1 = emu.f32_to_bf16(rng.standard_normal(64).astype(np.float32))
    w = emu.f32_to_bf16(rng.standard_normal(16 * 64).astype(np.float32))
    return maps, (lo, ro, po, oo), x0, x1, w


def test_graph_launch_rewriting_a_widen_source(rt):
    """A widen recorded after a graph that rewrites its source: the launch runs the widen first (the
    graph may read it), then rewrites the source; a contraction issued afterwards must read the
    widened copy of the old source, not the rewritten source."""
    maps, plan, x0, x1, w = _gemv_case(np.random.default_rng(5))
    s, x1b = rt.upload(x0), rt.upload(x1)
    rt.graph_begin()
    rt.map(s, BF16, x1b, BF16, 64, fh.op("CAST"))  # the graph overwrites s with x1
    g = rt.graph_end()
    d = rt.alloc(4 * 64)
    rt.map(d, F32, s, BF16, 64, fh.op("CAST"))  # d = widen(x0), deferred
    wd = rt.alloc(4 * 16 * 64)
    rt.map(wd, F32, rt.upload(w), BF16, 16 * 64, fh.op("CAST"))
    g.launch()
    out = rt.alloc(4 * 16)
    rt.contraction(out, d, wd, F32, F32, *maps)
    want = emu.contraction(x0, w, BF16, F32, *plan)
    assert np.array_equal(out.read(F32).view(np.uint32), want.view(np.uint32))
    assert np.array_equal(s.read(BF16), x1)
    g.free()


def test_graph_launch_rewriting_a_widen_output(rt):
    """The same with the graph writing the widen's output: the contraction reads what the graph
    wrote, not the widen's source."""
    rng = np.random.default_rng(6)
    maps, plan, x0, _, w = _gemv_case(rng)
    y = rng.standard_normal(64).astype(np.float32)
    d, yb = rt.alloc(4 * 64), rt.upload(y)
    rt.graph_begin()
    rt.map(d, F32, yb, F32, 64, fh.op("CAST"))  # the graph overwrites d with y
    g = rt.graph_end()
    s = rt.upload(x0)
    rt.map(d, F32, s, BF16, 64, fh.op("CAST"))  # d = widen(x0), deferred
    wd = rt.alloc(4 * 16 * 64)
    rt.map(wd, F32, rt.upload(w), BF16, 16 * 64, fh.op("CAST"))
    g.launch()
    out = rt.alloc(4 * 16)
    rt.contraction(out, d, wd, F32, F32, *maps)
    want = emu.contraction(y, emu.bf16_to_f32(w), F32, F32, *plan)
    assert np.array_equal(out.read(F32).view(np.uint32), want.view(np.uint32))
    g.free()


def test_recorded_contraction_of_a_run_widen(rt):
    """A widen whose cast ran before a recording: the recorded contraction must read the widened
    copy, so that a host write to the widen's source between launches does not change its result."""
    maps, plan, x0, x1, w = _gemv_case(np.random.default_rng(7))
    s = rt.upload(x0)
    d = rt.alloc(4 * 64)
    rt.map(d, F32, s, BF16, 64, fh.op("CAST"))
    wd = rt.alloc(4 * 16 * 64)
    rt.map(wd, F32, rt.upload(w), BF16, 16 * 64, fh.op("CAST"))
    d.read(F32)  # the cast runs; its record stays for contractions
    out = rt.alloc(4 * 16)
    rt.graph_begin()
    rt.contraction(out, d, wd, F32, F32, *maps)
    g = rt.graph_end()
    want = emu.contraction(x0, w, BF16, F32, *plan)
    for v in (x1, x0, x1):
        s.write(v)  # d keeps widen(x0)
        g.launch()
        assert np.array_equal(out.read(F32).view(np.uint32), want.view(np.uint32))
    g.free()
