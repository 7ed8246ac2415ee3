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

furiosa-opt-examples/src/transformer/mod.rs:29-131, the rest of one decode step:

  projection (:29-58)     rmsnorm(x); q, k, v = the GEMVs of projection.rs (widen; f32 contraction
                          over H; narrow); v to the V cache row; rmsnorm_q(q), rmsnorm_k(k); RoPE
                          (rope.rs: the half swap as two 64-element tile copies, then
                          bf16(f32(x) cos + f32(swapped) sin), the sign folded into sin); k to the
                          K cache row. The cache rows go through dma_scatter at a byte offset.
  decoder (:89-116)       norm(out, sum); proj_o over Q; residual (residual.rs: bf16(f32(a) +
                          f32(b))); rmsnorm; mlp; residual
  final_layer (:118-131)  rmsnorm; lm_head (lm_head.rs: the GEMV over Wp = 19 tiles of 8192 rows)

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
Q, P = N * G * D, N * D  # axes.rs: the query and key/value projection widths
W, WP, WT = 151936, 155648, 8192  # axes.rs: vocabulary, padded to 19 lm_head tiles of 8192 rows
ROW_STRIDE_ND = N * D * 2  # bytes of one [N, D] bf16 KV-cache row: dma_scatter offsets (transformer.py:44)
ROPE_THETA = 1_000_000.0   # transformer.py:41
# Every view of one decode step (a layer and the final layer)
STEP_SIZES = dict(N=N, G=G, D=D, T=T, H=H, L=L, Q=Q, P=P, X=1, Wp=WP, W=W)
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


_ITEM = {t: np.dtype(d).itemsize for t, d in NP_DTYPE.items()}  # element bytes per dtype code


class SeamOps:
    """The stages through the C ABI (device buffers)."""

    def __init__(self, rt, sizes=SIZES):
        self.rt = rt
        self.sizes = sizes
        self.views = {}  # view text -> MappingSerde JSON (an engine builds these once per type)
        self.ops = {}    # (name, flags, imm) -> op descriptor, built once
        self.sizes_of = {}  # view text -> its mapping's size
        self.calls = 0   # seam calls issued (allocations excluded)

    def view(self, text):
        js = self.views.get(text)
        if js is None:
            js = self.views[text] = m(text, **self.sizes)
        return js

    def _size(self, text):
        n = self.sizes_of.get(text)
        if n is None:
            n = self.sizes_of[text] = mapping_size(self.view(text))
        return n

    def put(self, arr):
        if isinstance(arr, Buffer):  # already resident
            return arr
        return self.rt.upload(np.ascontiguousarray(arr))

    def get(self, x, t):
        return x.read(NP_DTYPE[t])

    def _alloc(self, n, t):
        return self.rt.alloc(n * _ITEM[t])

    def _op(self, name, flags=0, imm=0):
        key = (name, flags, imm)
        o = self.ops.get(key)
        if o is None:
            o = self.ops[key] = op(name, flags, imm)
        return o

    def map(self, x, src_t, dst_t, name, flags=0, imm=0):
        self.calls += 1
        n = x.nbytes // _ITEM[src_t]
        out = self._alloc(n, dst_t)
        self.rt.map(out, dst_t, x, src_t, n, self._op(name, flags, imm))
        return out

    def zip(self, a, b, t, name, flags=0):
        self.calls += 1
        n = a.nbytes // _ITEM[t]
        out = self._alloc(n, t)
        self.rt.zip_with(out, t, a, b, t, n, self._op(name, flags))
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

    def gemv(self, xw, ww, rows, k):
        """f32 [rows] = sum over k of ww[rows, k] * xw[k]: one contraction over the whole weight."""
        return self.contraction(xw, ww, k, f"{rows}, {k}", f"{rows}, {k}", rows)

    def zeros(self, view, t):
        return self._alloc(self._size(view), t)  # DmTensor::new(): zero-filled

    def window(self, dst, x, t, view, base, src_offset, dst_offset):
        """A tile copy (Tensor::tile views, commit_view): the cells of `view` placed at src_offset in
        x's base mapping, written at dst_offset of dst's; dst is updated in place and returned."""
        self.calls += 1
        v, b = self.view(view), self.view(base)
        self.rt.transpose(dst, x, t, v, v, src_map=b, dst_map=b, src_offset=src_offset, dst_offset=dst_offset)
        return dst

    def row(self, table, i, t, rows, cols):
        """Row i of a [rows, cols] table: a gather of one index (the indexed axis `rows`, the
        payload `cols`) into a fresh [cols]. `i` is an int or a resident i32 [1]."""
        self.calls += 1
        out = self._alloc(self._size(cols), t)
        idx = i if isinstance(i, Buffer) else self.put(np.array([i], np.int32))
        self.rt.gather(out, self.put(table), idx, t, self.view(f"{rows}, {cols}"), self.view(f"X, {cols}"),
                       self.view("X"), False)
        return out

    def scatter(self, dst, src, index, t, src_map, key, dst_map, scaled):
        """dma_scatter into dst (updated in place and returned); `index` i32 over `key`."""
        self.calls += 1
        self.rt.scatter(dst, src, self.put(index), t, self.view(src_map), self.view(key), self.view(dst_map),
                        self.view(key), scaled)
        return dst


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


def attend(ops, q, ks, vs, masks, stages=None):
    """Every chunk in order (transformer.py:530-545); the running (max, sum, out) as device values.
    `stages`, when a list, receives (max, sum, out) after each chunk as host arrays."""
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
    return mx, sm, out


def decode(ops, q, ks, vs, masks, stages=None):
    """attend, then norm; (max, sum, out, normalised out) as host arrays."""
    mx, sm, out = attend(ops, q, ks, vs, masks, stages)
    y = norm(ops, out, sm)
    return ops.get(mx, F32), ops.get(sm, F32), ops.get(out, BF16), ops.get(y, BF16)


def proj(ops, xw, w, rows, k="H"):
    """bf16 [rows] = narrow(sum over k of f32(w[r, k]) * xw[k]): the GEMVs of projection.rs (proj_q
    :9-50, proj_p :53-93, proj_o :114-152), mlp.rs (:29-69, :110-150) and lm_head.rs (:18-49). xw is
    the widened input; w the bf16 weight [rows, k]."""
    return ops.map(ops.gemv(xw, ops.map(ops.put(w), BF16, F32, "CAST"), rows, k), F32, BF16, "CAST")


def mlp_block(ops, x, up_w, gate_w, down_w, stages=None):
    """mlp.rs:9-150 for one token: x [H], up/gate weights [L, H], down weight [H, L] (bf16 bits);
    returns the bf16 output [H] on the device. `stages`, when a dict, receives up, gate, x and the
    f32 down sums."""
    xw = ops.map(ops.put(x), BF16, F32, "CAST")
    up = proj(ops, xw, up_w, "L")
    gate = proj(ops, xw, gate_w, "L")
    g = ops.map(gate, BF16, F32, "CAST")
    silu = ops.zip(ops.map(g, F32, F32, "SIGMOID"), g, F32, "MUL_F")
    h = ops.map(ops.zip(ops.map(up, BF16, F32, "CAST"), silu, F32, "MUL_F"), F32, BF16, "CAST")
    down = ops.gemv(ops.map(h, BF16, F32, "CAST"), ops.map(ops.put(down_w), BF16, F32, "CAST"), "H", "L")
    if stages is not None:
        stages.update(up=ops.get(up, BF16), gate=ops.get(gate, BF16), x=ops.get(h, BF16), down=ops.get(down, F32))
    return ops.map(down, F32, BF16, "CAST")


def mlp(ops, x, up_w, gate_w, down_w, stages=None):
    """mlp_block with the output as a host array."""
    return ops.get(mlp_block(ops, x, up_w, gate_w, down_w, stages), BF16)


def rmsnorm(ops, x, w, rows, axis, n, rms=None):
    """rmsnorm.rs `forward` (:9-78), `forward_q` (:80-150) and `forward_k` (:152-...): over the view
    `rows, axis` of x (bf16 bits), with a gain w over `axis`, n = the axis length:
    ms = sum_axis f32(x)^2 / n + EPS; rms = sqrt(ms); y = bf16(f32(x) * f32(w) / rms).
    Returns (rms, y). A given `rms` (f32 per row) replaces the computed one: the sum's f32 fold
    order is free, and a check holds y to the rounding of the quotient by that rms."""
    full = f"{rows}, {axis}"
    xf = ops.map(ops.put(x), BF16, F32, "CAST")
    if rms is None:
        ss = ops.reduce(ops.zip(xf, xf, F32, "MUL_F"), F32, full, rows, "ADD", 0)
        ms = ops.map(ops.map(ss, F32, F32, "DIV_F", RHS_IMM, float(n)), F32, F32, "CLIP_ADD", RHS_IMM,
                     float(np.float32(RMS_EPS)))
        rms = ops.map(ms, F32, F32, "SQRT")
    rms = ops.put(rms)
    wf = ops.relayout(ops.map(ops.put(w), BF16, F32, "CAST"), F32, axis, full)
    y = ops.zip(ops.zip(xf, wf, F32, "MUL_F"), ops.relayout(rms, F32, rows, full), F32, "DIV_F")
    return rms, ops.map(y, F32, BF16, "CAST")


def residual(ops, a, b):
    """bf16 [H] = bf16(f32(a) + f32(b)) (residual.rs:9-31: a plus the residual stream b)."""
    s = ops.zip(ops.map(a, BF16, F32, "CAST"), ops.map(ops.put(b), BF16, F32, "CAST"), F32, "CLIP_ADD")
    return ops.map(s, F32, BF16, "CAST")


def rotate_half(ops, x, rows):
    """The half swap over D (rope.rs:37-73): the first 64 elements of every row copied to the second
    half of a zeroed [rows, D] tensor and the second half to the first, each as a tile copy of the
    view `rows, D = 64 # 128` at a D offset. No negation: the sign is in the sin table."""
    half, full = f"{rows}, D = {D // 2} # {D}", f"{rows}, D"
    out = ops.zeros(full, BF16)
    out = ops.window(out, x, BF16, half, full, {"D": 0}, {"D": D // 2})
    return ops.window(out, x, BF16, half, full, {"D": D // 2}, {"D": 0})


def rope(ops, x, cos, sin, rows):
    """rope.rs:75-173 for x [rows, D] (bf16): bf16(f32(x) * cos + f32(rotate_half(x)) * sin), each
    product an f32 multiply, their sum CLIP_ADD; cos, sin are bf16 [D] widened and broadcast."""
    full = f"{rows}, D"
    c = ops.relayout(ops.map(ops.put(cos), BF16, F32, "CAST"), F32, "D", full)
    s = ops.relayout(ops.map(ops.put(sin), BF16, F32, "CAST"), F32, "D", full)
    tc = ops.zip(ops.map(x, BF16, F32, "CAST"), c, F32, "MUL_F")
    ts = ops.zip(ops.map(rotate_half(ops, x, rows), BF16, F32, "CAST"), s, F32, "MUL_F")
    return ops.map(ops.zip(tc, ts, F32, "CLIP_ADD"), F32, BF16, "CAST")


def cache_row(ops, cache, row, offset):
    """dma_scatter::<m![1]> of one [N, D] row into a [T, N, D] cache (projection.rs:111, rope.rs:175):
    the key axis is the unit mapping, the indexed axis T, and `offset` the row's byte offset
    (row index * ROW_STRIDE_ND, transformer.py:432-435), an int or a resident i32 [1]. Returns the
    updated cache."""
    idx = offset if isinstance(offset, Buffer) else np.array([offset], np.int32)
    return ops.scatter(ops.put(cache), row, idx, BF16, "N, D", "1", "T, N, D", scaled=True)


def rope_row(pos):
    """cos and sin (bf16 bits [D]) at one absolute position, as the host builds its tables
    (transformer.py:452-472): inv_freq = 1 / theta^(2i / D) in f32, cos = cos(pos * inv_freq) on both
    halves, sin = [-sin, sin] (the rotation's sign folded in)."""
    inv_freq = np.float32(1.0) / (np.float32(ROPE_THETA) ** (np.arange(0, D, 2, dtype=np.float32) / np.float32(D)))
    f = np.float32(pos) * inv_freq.astype(np.float32)
    cos = np.concatenate([np.cos(f), np.cos(f)]).astype(np.float32)
    sin = np.concatenate([-np.sin(f), np.sin(f)]).astype(np.float32)

    def bf16(v):  # round to nearest even (finite values)
        u = v.view(np.uint32).astype(np.uint64)
        return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return bf16(cos), bf16(sin)


def projection(ops, x, wq, wk, wv, g_in, g_q, g_k, offset, cos, sin, k_cache, v_cache, stages=None):
    """ops::projection (mod.rs:29-58) for one token x [H]: returns (q [N, G, D], k_cache, v_cache),
    the caches with row `offset` (bytes) written. `stages`, when a dict, receives the device values
    y (the normed input), q, k, v (the GEMVs), qn, kn (their norms), kr (the roped k) and the rms of
    each norm (y_rms, qn_rms, kn_rms)."""
    y_rms, y = rmsnorm(ops, x, g_in, "X", "H", H)
    yw = ops.map(y, BF16, F32, "CAST")
    q, k, v = proj(ops, yw, wq, "Q"), proj(ops, yw, wk, "P"), proj(ops, yw, wv, "P")
    v_cache = cache_row(ops, v_cache, v, offset)
    qn_rms, qn = rmsnorm(ops, q, g_q, "N, G", "D", D)
    kn_rms, kn = rmsnorm(ops, k, g_k, "N", "D", D)
    qr, kr = rope(ops, qn, cos, sin, "N, G"), rope(ops, kn, cos, sin, "N")
    k_cache = cache_row(ops, k_cache, kr, offset)
    if stages is not None:
        stages.update(y=y, y_rms=y_rms, q=q, k=k, v=v, qn=qn, qn_rms=qn_rms, kn=kn, kn_rms=kn_rms, kr=kr)
    return qr, k_cache, v_cache


def decoder(ops, out, sm, rx, wo, g_post, up_w, gate_w, down_w, stages=None):
    """ops::decoder (mod.rs:89-116): the attention output normalised by its sum, proj_o over Q, the
    residual, the post-attention RMSNorm, the MLP and the second residual; returns the new residual
    stream [H]. `stages`, when a dict, receives a (the normed attention), o, rx1 (the first residual),
    y (its norm), y_rms and m (the MLP output)."""
    a = norm(ops, ops.put(out), ops.put(sm))  # [N, G, D], read as [Q]
    o = proj(ops, ops.map(a, BF16, F32, "CAST"), wo, "H", "Q")
    rx1 = residual(ops, o, rx)
    y_rms, y = rmsnorm(ops, rx1, g_post, "X", "H", H)
    mo = mlp_block(ops, y, up_w, gate_w, down_w)
    if stages is not None:
        stages.update(a=a, o=o, rx1=rx1, y=y, y_rms=y_rms, m=mo)
    return residual(ops, mo, rx1)


def final_layer(ops, x, g, lm_w, stages=None):
    """ops::final_layer (mod.rs:118-131): rmsnorm, then the lm_head GEMV over the padded vocabulary
    (lm_w [Wp, H]); returns the bf16 logits [Wp]."""
    y_rms, y = rmsnorm(ops, x, g, "X", "H", H)
    if stages is not None:
        stages.update(y=y, y_rms=y_rms)
    return proj(ops, ops.map(y, BF16, F32, "CAST"), lm_w, "Wp")


def causal_mask(row):
    """The mask of the chunk holding the query (transformer.py:437-450): keys up to `row` attended."""
    m_ = np.zeros(T, np.float32)
    m_[:row + 1] = 1.0
    return m_


def layer_step(ops, x, lw, pos, caches, cos, sin, stages=None, masks=None, offset=None):
    """One layer of Pipeline.step (transformer.py:495-562) for the token at absolute position pos:
    projection into the cache of chunk pos // T at row pos % T, attention over chunks 0..pos // T
    (the last one causal), decoder. `lw` holds the layer's weights by the names of mod.rs; `caches`
    a list of (k, v) per chunk, updated. `masks`, when given, are the chunks' masks already resident
    (the pipeline hoists them out of its layer loop, transformer.py:437-450); `offset`, when given,
    the cache row's byte offset already resident. Returns the new residual stream."""
    chunk, row = divmod(pos, T)
    kc, vc = caches[chunk]
    q, kc, vc = projection(ops, x, lw["q"], lw["k"], lw["v"], lw["input_norm"], lw["q_norm"], lw["k_norm"],
                           row * ROW_STRIDE_ND if offset is None else offset, cos, sin, kc, vc, stages)
    caches[chunk] = (kc, vc)
    if masks is None:
        full = ops.put(np.ones(T, np.float32))
        masks = [full] * chunk + [ops.put(causal_mask(row))]
    ks, vs = [c[0] for c in caches[:chunk + 1]], [c[1] for c in caches[:chunk + 1]]
    _, sm, out = attend(ops, q, ks, vs, masks)
    if stages is not None:
        stages.update(q_out=q, sum=sm, out=out)
    return decoder(ops, out, sm, x, lw["o"], lw["post_norm"], lw["up"], lw["gate"], lw["down"], stages)


def embedding(ops, table, token):
    """ops::embedding (mod.rs:23-27) on the token's row of the embedding table (transformer.py:507:
    `embedding_table[token]`): row `token` of the [W, H] table, as [H]."""
    return ops.row(table, token, BF16, "W", "H")


class Pipeline:
    """Pipeline.step (transformer.py:425-566) over the seam ops: per token the embedding, every
    layer's projection (K and V into the cache of chunk pos // T at row pos % T), attention over
    chunks 0..pos // T and decoder, then the final layer; greedy sampling of the first W logits
    (sample_token, transformer.py:489-490: the first index of the largest). `model` holds `embed`
    [W, H], `layers` (dicts of layer_step's weight names), `final_norm` [H] and `lm_head` [Wp, H],
    as bf16 bits or resident buffers. The KV caches are created zeroed per (layer, chunk), the masks
    and RoPE rows per position, as the reference's pipeline hoists them.

    With `graphs` (SeamOps only), the first token of each chunk count records the whole step (every
    seam call of the embedding, the layers and the final layer) into one graph, and every token of
    that chunk count launches it: the per-token inputs (token id, cache row offset, RoPE row, causal
    mask) sit in resident buffers that are rewritten before each launch, and everything else a
    step reads (weights, caches, the full mask) stays where it was when recorded. This is the
    NPU's compile-once, launch-per-call model (runtime.rs:157-177) on HIP graphs."""

    def __init__(self, ops, model, graphs=False):
        self.ops = ops
        self.model = {k: (ops.put(v) if k != "layers" else [{n: ops.put(w) for n, w in lw.items()} for lw in v])
                      for k, v in model.items()}
        self.caches = [[] for _ in self.model["layers"]]
        self.full = ops.put(np.ones(T, np.float32))
        self.graphs = {} if graphs else None  # chunk -> (graph, its logits buffer)
        if graphs:
            self.inputs = dict(token=ops.put(np.zeros(1, np.int32)), offset=ops.put(np.zeros(1, np.int32)),
                               cos=ops.put(np.zeros(D, np.uint16)), sin=ops.put(np.zeros(D, np.uint16)),
                               mask=ops.put(np.zeros(T, np.float32)))

    def _cache(self, layer, chunk):
        cs = self.caches[layer]
        while len(cs) <= chunk:
            cs.append((self.ops.zeros("T, N, D", BF16), self.ops.zeros("T, N, D", BF16)))
        return cs

    def _forward(self, token, pos, cos, sin, mask, offset):
        """The seam calls of one token; returns the logits buffer."""
        ops = self.ops
        chunk = pos // T
        masks = [self.full] * chunk + [mask]
        x = embedding(ops, self.model["embed"], token)
        for layer, lw in enumerate(self.model["layers"]):
            x = layer_step(ops, x, lw, pos, self._cache(layer, chunk), cos, sin, masks=masks, offset=offset)
        return final_layer(ops, x, self.model["final_norm"], self.model["lm_head"])

    def step(self, token, pos):
        """Runs one token at absolute position pos; returns the logits [Wp] as bf16 bits."""
        ops = self.ops
        chunk, row = divmod(pos, T)
        cos, sin = rope_row(pos)
        if self.graphs is None:
            logits = self._forward(token, pos, ops.put(cos), ops.put(sin), ops.put(causal_mask(row)),
                                   row * ROW_STRIDE_ND)
            return ops.get(logits, BF16)
        inp = self.inputs
        for name, v in (("token", np.array([token], np.int32)), ("offset", np.array([row * ROW_STRIDE_ND], np.int32)),
                        ("cos", cos), ("sin", sin), ("mask", causal_mask(row))):
            inp[name].write(v)
        rec = self.graphs.get(chunk)
        if rec is None:
            for layer in range(len(self.model["layers"])):
                self._cache(layer, chunk)  # created, and zeroed, before the recording
            ops.rt.graph_begin()
            try:
                logits = self._forward(inp["token"], pos, inp["cos"], inp["sin"], inp["mask"], inp["offset"])
            except BaseException:
                try:
                    ops.rt.graph_end().free()
                except RuntimeError:
                    pass
                raise
            rec = self.graphs[chunk] = (ops.rt.graph_end(), logits)
        rec[0].launch()
        return ops.get(rec[1], BF16)

    def generate(self, prompt, n_new):
        """Every prompt token in turn, then n_new greedy tokens; returns (new tokens, each step's
        logits)."""
        out, logs = [], []
        pos = 0
        for tok in prompt:
            logs.append(self.step(tok, pos))
            pos += 1
        for _ in range(n_new):
            nxt = sample_token(logs[-1])
            out.append(nxt)
            logs.append(self.step(nxt, pos))
            pos += 1
        return out, logs


def sample_token(logits):
    """The first index of the largest of the W real logits (bf16 bits; torch argmax semantics)."""
    u = np.asarray(logits[:W], np.uint32) << 16
    return int(np.argmax(u.view(np.float32)))
