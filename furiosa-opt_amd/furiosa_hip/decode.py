"""The decode chains of the reference transformer, stage by stage as Backend calls.

furiosa-opt-examples/src/transformer/kernel/attention.rs:226-365 (`forward_first`, `forward`) and
:370-392 (`norm`) attend one query token per (kv head n, group g) over one 512-key chunk of the KV
cache per launch; the running max, sum and unnormalised output stay in HBM between launches
(transformer.py:530-545 drives the chunks, the last one with a causal mask). Every stage below is one
seam op the engine issues for it, with the reference's rounding points:

  qk_scaled (:37-74)      widen q, k; f32 contraction over D; / sqrt(D) in f32; narrow to bf16
  row_max (:77-95)        widen; max over all T keys (before the mask)
  masked_exp (:98-134)    exp(x - max); min(., mask), mask[t] = 1 attends, 0 masks
  row_sum (:137-156)      sum over T, + EPS
  weighted_sum (:159-218) bf16(p) @ V as 32 partial products of 16 keys, each narrowed to bf16,
                          then an f32 sum over the 32 partials, narrowed to bf16
  forward (:248-365)      max' = max(block max, max); alpha = exp(max - max'); sum' = sum * alpha +
                          row_sum; out' = bf16(f32(bf16(f32(out) * alpha)) + f32(weighted_sum))
  norm (:370-392)         bf16(f32(out) / sum)

furiosa-opt-examples/src/transformer/kernel/mlp.rs:9-150 (`forward`, the SiLU MLP of one token):

  up, gate (:29-69)       widen; f32 contractions over H; narrow to bf16
  silu (:71-85)           g = f32(gate); sigmoid(g) * g in f32
  x (:94-108)             bf16(f32(up) * silu)
  down (:110-150)         widen; f32 contraction over L; narrow to bf16

Each chain is written once against a small adapter: `SeamOps` runs the stages on the HIP runtime;
the tests hold them against the same stages on the CPU oracle. The views are the logical layouts ([N, G, T], [T, N, D],
[L, H], ...); the reference's slice placements change where values sit, not the order of any fold.
"""
import json

import numpy as np

from . import BF16, F32, NP_DTYPE, RED, RHS_IMM, SWAP, Buffer, m, op

N, G, D, T = 8, 2, 128, 512
SIZES = dict(N=N, G=G, D=D, T=T)
H, L = 1024, 3072  # axes.rs: hidden and MLP widths
MLP_SIZES = dict(H=H, L=L)
# RMSNorm of one token: the hidden state [H] (X, a unit row axis), q [N, G, D] and k [N, D]
RMS_SIZES = dict(N=N, G=G, D=D, H=H, X=1)
RMS_EPS = 6.25e-8  # rmsnorm.rs:28 (and :104, :159)
SQRT_HEAD_DIM = 11.313708  # attention.rs:10
EPS = 6.25e-8              # attention.rs:13
NEG_INF_BITS = 0xFF800000



def mapping_size(js):
    """Mapping::size (furiosa-mapping-types/src/lib.rs:208-219) of a MappingSerde JSON string."""
    def size(node):
        (tag, b), = node.items()
        if tag == "Symbol":
            return b["size"]
        if tag == "Stride":
            return size(b["inner"]) // b["stride"]
        if tag == "Pair":
            return size(b["left"]) * size(b["right"])
        return b[{"Modulo": "modulo", "Resize": "resize", "Padding": "padding", "Broadcast": "size"}[tag]]
    return size(json.loads(js))


class SeamOps:
    """The stages through the C ABI (device buffers)."""

    def __init__(self, rt, sizes=SIZES):
        self.rt = rt
        self.sizes = sizes
        self.views = {}  # view text -> MappingSerde JSON (an engine builds these once per type)
        self.calls = 0   # seam calls issued (allocations excluded)

    def view(self, text):
        js = self.views.get(text)
        if js is None:
            js = self.views[text] = m(text, **self.sizes)
        return js

    def _size(self, text):
        return mapping_size(self.view(text))

    def put(self, arr):
        if isinstance(arr, Buffer):  # already resident
            return arr
        return self.rt.upload(np.ascontiguousarray(arr))

    def get(self, x, t):
        return x.read(NP_DTYPE[t])

    def _alloc(self, n, t):
        return self.rt.alloc(n * np.dtype(NP_DTYPE[t]).itemsize)

    def map(self, x, src_t, dst_t, name, flags=0, imm=0):
        self.calls += 1
        n = x.nbytes // np.dtype(NP_DTYPE[src_t]).itemsize
        out = self._alloc(n, dst_t)
        self.rt.map(out, dst_t, x, src_t, n, op(name, flags, imm))
        return out

    def zip(self, a, b, t, name, flags=0):
        self.calls += 1
        n = a.nbytes // np.dtype(NP_DTYPE[t]).itemsize
        out = self._alloc(n, t)
        self.rt.zip_with(out, t, a, b, t, n, op(name, flags))
        return out

    def reduce(self, x, t, src, dst, op, identity):
        self.calls += 1
        out = self._alloc(self._size(dst), t)
        self.rt.reduce(out, x, t, self.view(src), self.view(dst), RED[op], identity)
        return out

    def contraction(self, lhs, rhs, lv, rv, pre, out):
        self.calls += 1
        res = self._alloc(self._size(out), F32)
        self.rt.contraction(res, lhs, rhs, F32, F32, self.view(lv), self.view(rv), self.view(pre), self.view(out))
        return res

    def relayout(self, x, t, src, dst):
        self.calls += 1
        size = self._size(dst)
        out = self._alloc(size, t)  # to_dm / to_vrf: a fresh zeroed storage (fo_buffer_alloc zero-fills)
        self.rt.transpose(out, x, t, self.view(src), self.view(dst), allow_broadcast=True)
        return out


def qk_scaled(ops, q, k):
    """bf16 logits [N, G, T] (attention.rs:37-74)."""
    qw, kw = ops.map(q, BF16, F32, "CAST"), ops.map(k, BF16, F32, "CAST")
    acc = ops.contraction(qw, kw, "N, G, D", "T, N, D", "N, G, T, D", "N, G, T")
    acc = ops.map(acc, F32, F32, "DIV_F", RHS_IMM, float(np.float32(SQRT_HEAD_DIM)))
    return ops.map(acc, F32, BF16, "CAST")


def row_max(ops, qk):
    """f32 [N, G]: the max over every key of the chunk, the masked ones included (attention.rs:77-95)."""
    return ops.reduce(ops.map(qk, BF16, F32, "CAST"), F32, "N, G, T", "N, G", "MAX", NEG_INF_BITS)


def masked_exp(ops, qk, mx, mask):
    """f32 [N, G, T] = min(exp(f32(qk) - max), mask) (attention.rs:98-134)."""
    x = ops.map(qk, BF16, F32, "CAST")
    e = ops.map(ops.zip(x, ops.relayout(mx, F32, "N, G", "N, G, T"), F32, "SUB_F"), F32, F32, "EXP")
    return ops.zip(e, ops.relayout(mask, F32, "T", "N, G, T"), F32, "CLIP_MIN")


def row_sum(ops, e):
    """f32 [N, G] = sum over T + EPS (attention.rs:137-156)."""
    s = ops.reduce(e, F32, "N, G, T", "N, G", "ADD", 0)
    return ops.map(s, F32, F32, "CLIP_ADD", RHS_IMM, float(np.float32(EPS)))


def weighted_sum(ops, e, v):
    """bf16 [N, G, D] (attention.rs:159-218): 16-key partial products narrowed to bf16, then their f32
    sum over the 32 partials, narrowed again."""
    w = ops.map(ops.map(e, F32, BF16, "CAST"), BF16, F32, "CAST")
    vw = ops.map(v, BF16, F32, "CAST")
    part = ops.contraction(w, vw, "N, G, T", "T, N, D", "N, G, T / 16, D, T % 16", "N, G, T / 16, D")
    part = ops.map(ops.map(part, F32, BF16, "CAST"), BF16, F32, "CAST")
    total = ops.reduce(part, F32, "N, G, T / 16, D", "N, G, D", "ADD", 0)
    return ops.map(total, F32, BF16, "CAST")


def forward_first(ops, q, k, v, mask):
    """(max, sum, out) after the first chunk (attention.rs:226-246)."""
    qk = qk_scaled(ops, q, k)
    mx = row_max(ops, qk)
    e = masked_exp(ops, qk, mx, mask)
    return mx, row_sum(ops, e), weighted_sum(ops, e, v)


def forward(ops, q, k, v, mask, mx, sm, out):
    """(max, sum, out) folded over one more chunk (attention.rs:248-365)."""
    qk = qk_scaled(ops, q, k)
    new = ops.zip(row_max(ops, qk), mx, F32, "CLIP_MAX")
    alpha = ops.map(ops.zip(new, mx, F32, "SUB_F", SWAP), F32, F32, "EXP")  # exp(max - max')
    e = masked_exp(ops, qk, new, mask)
    sm = ops.zip(ops.zip(sm, alpha, F32, "MUL_F"), row_sum(ops, e), F32, "CLIP_ADD")
    result = ops.map(weighted_sum(ops, e, v), BF16, F32, "CAST")
    a = ops.relayout(alpha, F32, "N, G", "N, G, D")
    o = ops.map(ops.zip(ops.map(out, BF16, F32, "CAST"), a, F32, "MUL_F"), F32, BF16, "CAST")
    o = ops.zip(ops.map(o, BF16, F32, "CAST"), result, F32, "CLIP_ADD")
    return new, sm, ops.map(o, F32, BF16, "CAST")


def norm(ops, out, sm):
    """bf16 [N, G, D] = out / sum (attention.rs:370-392)."""
    s = ops.relayout(sm, F32, "N, G", "N, G, D")
    return ops.map(ops.zip(ops.map(out, BF16, F32, "CAST"), s, F32, "DIV_F"), F32, BF16, "CAST")


def decode(ops, q, ks, vs, masks, stages=None):
    """Every chunk in order (transformer.py:530-545), then norm; (max, sum, out, normalised out) as
    host arrays. `stages`, when a list, receives (max, sum, out) after each chunk."""
    q = ops.put(q)
    mx = sm = out = None
    for c, (k, v, mask) in enumerate(zip(ks, vs, masks)):
        k, v, mask = ops.put(k), ops.put(v), ops.put(mask)
        if c == 0:
            mx, sm, out = forward_first(ops, q, k, v, mask)
        else:
            mx, sm, out = forward(ops, q, k, v, mask, mx, sm, out)
        if stages is not None:
            stages.append((ops.get(mx, F32), ops.get(sm, F32), ops.get(out, BF16)))
    y = norm(ops, out, sm)
    return ops.get(mx, F32), ops.get(sm, F32), ops.get(out, BF16), ops.get(y, BF16)


def mlp(ops, x, up_w, gate_w, down_w, stages=None):
    """mlp.rs:9-150 for one token: x [H], up/gate weights [L, H], down weight [H, L] (bf16 bits);
    returns the bf16 output [H]. `stages`, when a dict, receives up, gate, x and the f32 down sums."""
    xw = ops.map(ops.put(x), BF16, F32, "CAST")
    up = ops.map(ops.contraction(xw, ops.map(ops.put(up_w), BF16, F32, "CAST"), "H", "L, H", "L, H", "L"),
                 F32, BF16, "CAST")
    gate = ops.map(ops.contraction(xw, ops.map(ops.put(gate_w), BF16, F32, "CAST"), "H", "L, H", "L, H", "L"),
                   F32, BF16, "CAST")
    g = ops.map(gate, BF16, F32, "CAST")
    silu = ops.zip(ops.map(g, F32, F32, "SIGMOID"), g, F32, "MUL_F")
    h = ops.map(ops.zip(ops.map(up, BF16, F32, "CAST"), silu, F32, "MUL_F"), F32, BF16, "CAST")
    hw = ops.map(h, BF16, F32, "CAST")
    down = ops.contraction(hw, ops.map(ops.put(down_w), BF16, F32, "CAST"), "L", "H, L", "H, L", "H")
    if stages is not None:
        stages.update(up=ops.get(up, BF16), gate=ops.get(gate, BF16), x=ops.get(h, BF16), down=ops.get(down, F32))
    return ops.get(ops.map(down, F32, BF16, "CAST"), BF16)


def rmsnorm(ops, x, w, rows, axis, n):
    """rmsnorm.rs `forward` (:9-78), `forward_q` (:80-150) and `forward_k` (:152-...): over the view
    `rows, axis` of x (bf16 bits), with a gain w over `axis`, n = the axis length:
    ms = sum_axis f32(x)^2 / n + EPS; rms = sqrt(ms); y = bf16(f32(x) * f32(w) / rms).
    Returns (rms, y)."""
    full = f"{rows}, {axis}"
    xf = ops.map(ops.put(x), BF16, F32, "CAST")
    ss = ops.reduce(ops.zip(xf, xf, F32, "MUL_F"), F32, full, rows, "ADD", 0)
    ms = ops.map(ops.map(ss, F32, F32, "DIV_F", RHS_IMM, float(n)), F32, F32, "CLIP_ADD", RHS_IMM,
                 float(np.float32(RMS_EPS)))
    rms = ops.map(ms, F32, F32, "SQRT")
    wf = ops.relayout(ops.map(ops.put(w), BF16, F32, "CAST"), F32, axis, full)
    y = ops.zip(ops.zip(xf, wf, F32, "MUL_F"), ops.relayout(rms, F32, rows, full), F32, "DIV_F")
    return rms, ops.map(y, F32, BF16, "CAST")
