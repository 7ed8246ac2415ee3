"""The decode chains of the reference transformer (furiosa_hip/decode.py: attention.rs:226-392,
mlp.rs:9-150) on both sides of the parity tests: `GpuOps` runs the stages through the C ABI,
`CpuOps` runs the same stages on the oracle. Also the float64 restatements of the model (softmax
attention, the SiLU MLP) and the seeded inputs at the reference's shapes.
"""
import numpy as np

import furiosa_hip as fh
import furiosa_hip.decode as fd
from furiosa_hip.decode import (BF16, D, EPS, F32, G, H, L, MLP_SIZES, N, RMS_EPS, RMS_SIZES, SIZES, T, decode, forward,
                                forward_first, masked_exp, mlp, norm, qk_scaled, rmsnorm, row_max, row_sum,
                                weighted_sum)
from oracle import emulator as emu
from oracle import mapping_ref as mr

GpuOps = fd.SeamOps

__all__ = ["BF16", "D", "EPS", "F32", "G", "H", "L", "MLP_SIZES", "N", "RMS_EPS", "RMS_SIZES", "SIZES", "T", "decode",
           "forward", "forward_first", "masked_exp", "mlp", "norm", "qk_scaled", "rmsnorm", "row_max", "row_sum",
           "weighted_sum"]

# The three RMSNorm forms of the decode step: (rows view, normed axis, its length, x shape)
RMS_FORMS = {"forward": ("X", "H", H, (1, H)), "forward_q": ("N, G", "D", D, (N * G, D)),
             "forward_k": ("N", "D", D, (N, D))}


def _bits(v):
    return int(np.float32(v).view(np.uint32)) if isinstance(v, float) else int(v)


class CpuOps:
    """The stages on the oracle (numpy arrays)."""

    def __init__(self, sizes=SIZES, tile=fd.WT):
        self.sizes = sizes
        self.tile = tile
        self._plans = {}

    def view(self, text):
        return mr.parse(text, self.sizes)

    def put(self, arr):
        return np.array(arr, copy=True)

    def get(self, x, t):
        return np.array(x, dtype=fh.NP_DTYPE[t], copy=True)

    def map(self, x, src_t, dst_t, name, flags=0, imm=0):
        return emu.map_(x, src_t, dst_t, fh.OP[name], flags, _bits(imm))

    def zip(self, a, b, t, name, flags=0):
        return emu.zip_(a, b, t, t, fh.OP[name], flags)

    def reduce(self, x, t, src, dst, op, identity):
        return emu.reduce(x, t, self.view(src), self.view(dst), fh.RED[op], identity)

    def contraction(self, lhs, rhs, lv, rv, pre, out):
        return emu.contraction(lhs, rhs, F32, F32, self.view(lv), self.view(rv), self.view(pre), self.view(out))

    def relayout(self, x, t, src, dst):
        size = mr.size(self.view(dst))
        return emu.transpose(np.zeros(size, fh.NP_DTYPE[t]), x, self.view(src), self.view(dst))

    def gemv(self, xw, ww, rows, k):
        """The contraction of SeamOps.gemv, resolved on row tiles of at most `tile` rows: row r reads
        only row r of the row-major weight, so every tile shares one read plan (resolved once and
        cached; test_oracle_decode pins the tiled result against the whole contraction)."""
        n, kk = self.sizes[rows], self.sizes[k]
        t = min(n, self.tile)
        if n % t:
            raise ValueError("gemv rows must split into whole tiles")
        key = (rows, k, t)
        plan = self._plans.get(key)
        if plan is None:
            s = {rows: t, k: kk}
            v = lambda text: mr.parse(text, s)
            plan = self._plans[key] = emu.contraction_plan(v(k), v(f"{rows}, {k}"), v(f"{rows}, {k}"), v(rows))
        w = np.asarray(ww).reshape(n // t, t * kk)
        return np.concatenate([emu.contraction_run(plan, xw, w[i], F32, F32) for i in range(n // t)])

    def zeros(self, view, t):
        return np.zeros(mr.size(self.view(view)), fh.NP_DTYPE[t])

    def window(self, dst, x, t, view, base, src_offset, dst_offset):
        v, b = self.view(view), self.view(base)
        return emu.transpose(dst, x, v, v, src_map=b, dst_map=b, src_offset=src_offset, dst_offset=dst_offset)

    def row(self, table, i, t, rows, cols):
        """Row i of the row-major [rows, cols] table (the gather's closed form: its index picks one
        row, scatter_gather_tests.rs:3-11)."""
        n = self.sizes[cols]
        if not 0 <= i < self.sizes[rows]:
            raise IndexError("row index past the table")
        return np.array(table[i * n:(i + 1) * n], copy=True)

    def scatter(self, dst, src, index, t, src_map, key, dst_map, scaled):
        k = self.view(key)
        return emu.scatter(dst, src, index, np.dtype(fh.NP_DTYPE[t]).itemsize, self.view(src_map), k,
                           self.view(dst_map), k, scaled)


def softmax_attention(q, ks, vs, masks, bf16_logits=False):
    """The model's attention for the one query (float64, transformer.py:255-263): softmax over every
    attended key of every chunk, then the weighted sum of V; [N, G, D]. `bf16_logits` rounds the
    scaled logits to bf16 first, as qk_scaled does (attention.rs:63-70): with logits of a few units
    that rounding alone moves p by a few percent, beyond the acceptance test's 1%."""
    qf = emu.bf16_to_f32(q).astype(np.float64).reshape(N, G, D)
    k = np.concatenate([emu.bf16_to_f32(x).reshape(T, N, D) for x in ks]).astype(np.float64)
    v = np.concatenate([emu.bf16_to_f32(x).reshape(T, N, D) for x in vs]).astype(np.float64)
    m = np.concatenate(masks)
    s = np.einsum("ngd,tnd->ngt", qf, k) / np.sqrt(D)
    if bf16_logits:
        s = emu.bf16_to_f32(emu.f32_to_bf16(s.astype(np.float32))).astype(np.float64)
    s = np.where(m[None, None, :] == 0, -np.inf, s)
    w = np.exp(s - s.max(axis=-1, keepdims=True))
    w /= w.sum(axis=-1, keepdims=True)
    return np.einsum("ngt,tnd->ngd", w, v)


def inputs(seed, chunks, valid_last, scale=1.0, uniform=False):
    """q [N, G, D], per-chunk k, v [T, N, D] (bf16 bits) and masks [T]; earlier chunks fully
    attended, the last one up to `valid_last` keys (the causal row of transformer.py:437-450)."""
    rng = np.random.default_rng(seed)

    def sample(n):
        x = rng.uniform(0, 1, n) if uniform else scale * rng.standard_normal(n)
        return emu.f32_to_bf16(x.astype(np.float32))
    q = sample(N * G * D)
    ks = [sample(T * N * D) for _ in range(chunks)]
    vs = [sample(T * N * D) for _ in range(chunks)]
    masks = [np.ones(T, np.float32) for _ in range(chunks)]
    masks[-1][valid_last:] = 0.0
    return q, ks, vs, masks


def mlp_float(x, up_w, gate_w, down_w):
    """The model's MLP in float64 (down(silu(gate x) * up x)), with the chain's three bf16 narrows
    (up, gate, the product) kept: at H = 1024 a dot product of unit-scale values rounds to bf16 with
    errors near 1%, which the narrows of the chain make on the same values."""
    f = lambda t, *shape: emu.bf16_to_f32(t).astype(np.float64).reshape(*shape)
    r = lambda v: emu.bf16_to_f32(emu.f32_to_bf16(np.asarray(v, np.float32))).astype(np.float64)
    xf = f(x, H)
    up, gate = r(f(up_w, L, H) @ xf), r(f(gate_w, L, H) @ xf)
    h = r(up * gate / (1.0 + np.exp(-gate)))
    return f(down_w, H, L) @ h


def mlp_inputs(seed):
    """x, up, gate, down weights (bf16 bits) at the reference's shapes; weights scaled by 1/sqrt(fan-in)."""
    rng = np.random.default_rng(seed)
    b = lambda a: emu.f32_to_bf16(a.astype(np.float32))
    x = b(rng.standard_normal(H))
    return (x, b(rng.standard_normal(L * H) / np.sqrt(H)), b(rng.standard_normal(L * H) / np.sqrt(H)),
            b(rng.standard_normal(H * L) / np.sqrt(L)))


def rms_inputs(seed, form):
    """x and the gain (bf16 bits) of one RMSNorm form; gains near 1 as the model's are."""
    rng = np.random.default_rng(seed)
    _, _, n, shape = RMS_FORMS[form]
    x = emu.f32_to_bf16((2.0 * rng.standard_normal(shape[0] * shape[1])).astype(np.float32))
    w = emu.f32_to_bf16((1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32))
    return x, w


def rmsnorm_float(x, w, form):
    """rmsnorm.rs in float64 with its one bf16 narrow: (rms per row, y)."""
    _, _, n, shape = RMS_FORMS[form]
    xf = emu.bf16_to_f32(x).astype(np.float64).reshape(shape)
    rms = np.sqrt((xf * xf).sum(axis=1) / n + RMS_EPS)
    y = emu.f32_to_bf16((xf * emu.bf16_to_f32(w).astype(np.float64) / rms[:, None]).astype(np.float32))
    return rms, y.reshape(-1)


# ---- the rest of the decode step (mod.rs:29-131) -------------------------------------------------

STEP_SIZES = fd.STEP_SIZES


def seeded(rng, n, scale):
    """seeded_bf16 (transformer_tests.rs:13-17): uniform(-scale, scale) rounded to bf16 (bits)."""
    return emu.f32_to_bf16(rng.uniform(-scale, scale, n).astype(np.float32))


def sample(rng, n):
    """sample (transformer.py:161-162): uniform [0, 1) in bf16 (bits)."""
    return emu.f32_to_bf16(rng.uniform(0.0, 1.0, n).astype(np.float32))


def linear_init(rng, rows, cols):
    """nn.Linear's default weight init, uniform(+-1/sqrt(fan_in)), in bf16 (bits) [rows, cols]."""
    b = 1.0 / np.sqrt(cols)
    return emu.f32_to_bf16(rng.uniform(-b, b, rows * cols).astype(np.float32))


def f64(bits, *shape):
    v = emu.bf16_to_f32(np.asarray(bits)).astype(np.float64)
    return v.reshape(*shape) if shape else v


def r16(v):
    """Round float64 values to bf16 (through f32, as torch's .to(bfloat16) of an f32 tensor)."""
    return emu.bf16_to_f32(emu.f32_to_bf16(np.asarray(v, np.float64).astype(np.float32))).astype(np.float64)


def assert_close(actual_bits, expected, abs_, rel, name=""):
    """assert_close (transformer_tests.rs:19-29): |a - e| <= abs + rel |e| for every element."""
    a = f64(actual_bits)
    e = np.asarray(expected, np.float64).reshape(-1)
    assert a.shape == e.shape
    bad = np.abs(a - e) > abs_ + rel * np.abs(e)
    assert not bad.any(), f"{name}: {int(bad.sum())} elements, first {np.argmax(bad)}"


def rms_scalar(values, weight):
    """rms (transformer_tests.rs:31-40) in float64: value / sqrt(mean(v^2) + eps) * weight."""
    v = np.asarray(values, np.float64)
    return v / np.sqrt(np.mean(v * v) + RMS_EPS) * f64(weight)


def projection_scalar(x, wq, wk, wv, g_in, g_q, g_k):
    """transformer_tests.rs:166-194 (cos = 1, sin = 0): (q [Q], k [P], v [P]) with no narrows."""
    xn = rms_scalar(f64(x), g_in)
    q, k, v = f64(wq, fd.Q, H) @ xn, f64(wk, fd.P, H) @ xn, f64(wv, fd.P, H) @ xn
    q = np.concatenate([rms_scalar(q[h * D:(h + 1) * D], g_q) for h in range(N * G)])
    k = np.concatenate([rms_scalar(k[h * D:(h + 1) * D], g_k) for h in range(N)])
    return q, k, v


def decoder_scalar(x, rx, wo, g_post, up_w, gate_w, down_w):
    """transformer_tests.rs:591-634 (sum = 1): the new residual stream [H] with no narrows."""
    after = f64(rx) + f64(wo, H, fd.Q) @ f64(x)
    xn = rms_scalar(after, g_post)
    up, gate = f64(up_w, L, H) @ xn, f64(gate_w, L, H) @ xn
    return after + f64(down_w, H, L) @ (gate / (1.0 + np.exp(-gate)) * up)


def model_rms(x, w, axis_len):
    """RMSNorm (transformer.py:73-83) over the last axis of length axis_len: the normalised f32 value
    narrowed to bf16, then times the bf16 weight, narrowed again."""
    v = np.asarray(x, np.float64).reshape(-1, axis_len)
    n = r16(v / np.sqrt(np.mean(v * v, axis=1, keepdims=True) + RMS_EPS))
    return r16(f64(w)[None, :] * n).reshape(-1)


def projection_model(x, wq, wk, wv, g_in, g_q, g_k, pos):
    """Attention.projection (transformer.py:113-128) after the input RMSNorm, in float64 with torch's
    bf16 narrows: every Linear output, each RMSNorm, and the RoPE products and sum, with the model's
    own tables (cos, sin of emb = [freqs, freqs]) and rotate_half = [-x2, x1]. (q [Q], k [P], v [P])."""
    xn = model_rms(f64(x), g_in, H)
    q, k, v = r16(f64(wq, fd.Q, H) @ xn), r16(f64(wk, fd.P, H) @ xn), r16(f64(wv, fd.P, H) @ xn)
    q, k = model_rms(q, g_q, D).reshape(-1, D), model_rms(k, g_k, D).reshape(-1, D)
    cos_b, sin_b = fd.rope_row(pos)
    c, s = f64(cos_b), f64(sin_b)
    s = np.concatenate([-s[:D // 2], s[D // 2:]])  # undo the sign the kernel's table folds in

    def rot(t):
        return np.concatenate([-t[:, D // 2:], t[:, :D // 2]], axis=1)
    q = r16(r16(q * c) + r16(rot(q) * s))
    k = r16(r16(k * c) + r16(rot(k) * s))
    return q.reshape(-1), k.reshape(-1), v


def decoder_model(x, rx, wo, g_post, up_w, gate_w, down_w):
    """Decoder.forward (transformer.py:146-150) in float64 with torch's narrows: rx + o_proj(x), then
    that plus mlp(post_norm(.))."""
    h1 = r16(f64(rx) + r16(f64(wo, H, fd.Q) @ f64(x)))
    xn = model_rms(h1, g_post, H)
    up, gate = r16(f64(up_w, L, H) @ xn), r16(f64(gate_w, L, H) @ xn)
    act = r16(r16(gate / (1.0 + np.exp(-gate))) * up)
    return r16(h1 + r16(f64(down_w, H, L) @ act))


def final_model(x, g, lm_w):
    """lm_head(rms(x)) (transformer.py:316-341) over the W real rows, float64 with the narrows."""
    xn = model_rms(f64(x), g, H)
    return r16(f64(lm_w[:fd.W * H], fd.W, H) @ xn)


def layer_weights(rng, ones=True):
    """One layer's weights by the names layer_step reads: nn.Linear's init, and the RMSNorm gains
    the modules start with (ones, transformer.py:76) or, with ones=False, gains near 1. The model's
    narrows round the normalised value before the gain (model_rms), the kernels once after it: with
    gains of 1 the two agree, with others they differ by an ulp on up to half the elements, which the
    GEMVs after them sum to about 1% of a projection."""
    if ones:
        gain = lambda n: np.full(n, emu.f32_to_bf16(np.ones(1, np.float32))[0], np.uint16)
    else:
        gain = lambda n: emu.f32_to_bf16((1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32))
    return dict(q=linear_init(rng, fd.Q, H), k=linear_init(rng, fd.P, H), v=linear_init(rng, fd.P, H),
                o=linear_init(rng, H, fd.Q), up=linear_init(rng, L, H), gate=linear_init(rng, L, H),
                down=linear_init(rng, H, L), input_norm=gain(H), q_norm=gain(D), k_norm=gain(D),
                post_norm=gain(H))
