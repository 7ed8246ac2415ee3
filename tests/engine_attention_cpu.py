"""The engine-layout decode attention stream (furiosa_hip/engine_attention.py) on the oracle: the
same stage functions with every seam call run by the CPU restatement, so the stream's transcription
can be held against the logical-view chain on the oracle without a GPU."""
import numpy as np

import furiosa_hip as fh
from furiosa_hip.engine_attention import ALL, NEVER, SIZES, Val
from oracle import emulator as emu
from oracle import mapping_ref as mr


def _bits(v):
    return int(np.float32(v).view(np.uint32)) if isinstance(v, float) else int(v) & 0xFFFFFFFF


class CpuEngineOps:
    """EngineOps' methods on numpy arrays through the oracle."""

    def __init__(self, sizes=SIZES):
        self.sizes = sizes
        self._views = {}
        self.calls = 0

    def view(self, text):
        v = self._views.get(text)
        if v is None:
            v = self._views[text] = mr.parse(text, self.sizes)
        return v

    def size(self, text):
        return mr.size(self.view(text))

    def put(self, arr, t, view):
        return Val(np.array(arr, dtype=fh.NP_DTYPE[t], copy=True), t, view)

    def get(self, x):
        return np.array(x.data, copy=True)

    def move(self, x, dst, broadcast):
        self.calls += 1
        out = np.zeros(self.size(dst), fh.NP_DTYPE[x.t])
        return Val(emu.transpose(out, x.data, self.view(x.view), self.view(dst)), x.t, dst)

    def move_into(self, dst, x):
        self.calls += 1
        dst.data[:] = emu.transpose(dst.data, x.data, self.view(x.view), self.view(dst.view))

    def zeros(self, view, t):
        return Val(np.zeros(self.size(view), fh.NP_DTYPE[t]), t, view)

    def read_tile(self, x, view, offset, dst=None, broadcast=False):
        self.calls += 1
        dst = dst or view
        out = np.zeros(self.size(dst), fh.NP_DTYPE[x.t])
        return Val(emu.transpose(out, x.data, self.view(view), self.view(dst), src_map=self.view(x.view),
                                 src_offset=offset), x.t, dst)

    def write_tile(self, dst, x, view, offset):
        self.calls += 1
        dst.data[:] = emu.transpose(dst.data, x.data, self.view(x.view), self.view(view), dst_map=self.view(dst.view),
                                    dst_offset=offset)

    def scatter(self, dst, x, index, key="1"):
        self.calls += 1
        k = self.view(key)
        dst.data[:] = emu.scatter(dst.data, x.data, index.data, np.dtype(fh.NP_DTYPE[x.t]).itemsize, self.view(x.view),
                                  k, self.view(dst.view), self.view(index.view), True)

    def map(self, x, dst_t, name, flags=0, imm=0):
        self.calls += 1
        return Val(emu.map_(x.data, x.t, dst_t, fh.OP[name], flags, _bits(imm)), dst_t, x.view)

    def tag(self, x):
        self.calls += 1
        return Val(emu.branch_tag(x.data, x.t, NEVER), fh.U8, x.view)

    def zero_tag(self, view):
        return Val(np.zeros(self.size(view), np.uint8), fh.U8, view)

    def reshape(self, x, view):
        assert self.size(view) == self.size(x.view), "reshape keeps the size"
        self.calls += 1
        return Val(np.array(x.data, copy=True), x.t, view)

    def slots(self, x, tag, name, const=None, port=None, flags=0):
        self.calls += 1
        regs = [ALL] if const is not None else []
        ops0 = [_bits(const)] if const is not None else []
        out = emu.zip3_slots(x.data, port.data if port is not None else None, tag.data, x.t, fh.OP[name], flags,
                             regs, ops0, [0] * len(regs), port is not None, ALL, 0)
        return Val(out, x.t, x.view)

    def unary(self, x, tag, name):
        return self.map(x, x.t, name)

    def reduce(self, x, dst, name, identity, broadcast):
        self.calls += 1
        return Val(emu.reduce(x.data, x.t, self.view(x.view), self.view(dst), fh.RED[name], identity), x.t, dst)

    def contraction(self, lhs, rhs, pre, out):
        self.calls += 1
        res = emu.contraction(lhs.data, rhs.data, fh.F32, fh.F32, self.view(lhs.view), self.view(rhs.view),
                              self.view(pre), self.view(out))
        return Val(res, fh.F32, out)
