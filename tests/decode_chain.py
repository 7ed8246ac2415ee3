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

    def __init__(self, sizes=SIZES):
        self.sizes = sizes

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
