"""Python binding of the MI355X backend's C ABI (include/furiosa_hip.h), over ctypes.

This is the harness the tests and the benchmark drive the library through; a Rust `Hip: Backend`
would bind the same header with bindgen. Nothing here computes: every call goes to
`libfuriosa_hip.so`, and importing raises if the library has not been built.

Mappings are passed as `m![...]` text plus axis sizes (parsed by the library into MappingSerde
JSON) or as MappingSerde JSON directly.
"""
from __future__ import annotations

import ctypes as C
import json
import os
from pathlib import Path
from typing import Dict, Optional, Sequence

import numpy as np

_HERE = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("FO_HIP_LIB", _HERE.parent / "libfuriosa_hip.so"))

if not LIB_PATH.exists():
    raise ImportError(
        f"{LIB_PATH} is not built; run `python furiosa-opt_amd/build.py` (or __graft_entry__.build())"
    )

_lib = C.CDLL(str(LIB_PATH))

# ---- dtypes / ops (mirrors furiosa_hip.h) -------------------------------------------------------
I8, U8, I16, I32, BF16, F32, F8E4M3, F8E5M2, I4, F4E2M1 = 0, 1, 2, 3, 4, 5, 6, 7, 8, 9
# bf16 and the 8-bit floats travel as their raw bit patterns; the 4-bit types as packed bytes
# (element 2k in the low nibble of byte k)
NP_DTYPE = {I8: np.int8, U8: np.uint8, I16: np.int16, I32: np.int32, BF16: np.uint16, F32: np.float32,
            F8E4M3: np.uint8, F8E5M2: np.uint8, I4: np.uint8, F4E2M1: np.uint8}
NAMES = {"i8": I8, "u8": U8, "i16": I16, "i32": I32, "bf16": BF16, "f32": F32, "f8e4m3": F8E4M3, "f8e5m2": F8E5M2,
         "i4": I4, "f4e2m1": F4E2M1}

OP = dict(
    CAST=0, CAST_RELU=1, TABLE_LOOKUP=2, ZERO_POINT_SUB=3,
    EXP=10, NEG_EXP=11, SQRT=12, TANH=13, SIGMOID=14, LOG=15, SIN=16, COS=17,
    ADD_F=30, SUB_F=31, MUL_F=32, DIV_F=33, CLIP_ADD=40, CLIP_MIN=41, CLIP_MAX=42, CLIP_ABS_MIN=43,
    CLIP_ABS_MAX=44, FMA_F=50, FXP_TO_FP=60, FP_TO_FXP=61, ADD_FXP=70, ADD_FXP_SAT=71, SUB_FXP=72,
    SUB_FXP_SAT=73, MUL_FXP=74, MUL_INT=75, MIN_I=76, MAX_I=77, SHL=78, LSHR=79, ASHR=80,
    BIT_AND=81, BIT_OR=82, BIT_XOR=83, SHL_SAT=84, ABS_MIN_I=85, ABS_MAX_I=86,
)
CMP = dict(EQUAL=0, LESS=1, GREATER=2, LESS_UNSIGNED=3, GREATER_UNSIGNED=4, TRUE=5, FALSE=6)
RHS_IMM, SWAP = 1, 2
RED = dict(ADD=0, MAX=1, MIN=2, MUL=3, ADD_SAT=4)


class FoOp(C.Structure):
    _fields_ = [("code", C.c_int32), ("flags", C.c_uint32), ("imm0", C.c_uint32), ("imm1", C.c_uint32)]


class FoSlots(C.Structure):
    _fields_ = [
        ("op", FoOp),
        ("n_regs", C.c_int32),
        ("reg_guard", C.c_uint32 * 3),
        ("reg_operand0", C.c_uint32 * 3),
        ("reg_operand1", C.c_uint32 * 3),
        ("has_port", C.c_int32),
        ("port_guard", C.c_uint32),
        ("port_operand1", C.c_uint32),
    ]


class FoCmp(C.Structure):
    _fields_ = [("kind", C.c_int32), ("boundary", C.c_uint32)]


_P = C.c_void_p
TRACE_SINK = C.CFUNCTYPE(None, C.c_void_p, C.POINTER(C.c_char), C.c_uint64, C.c_uint64, C.c_uint64)
TRACE_DONE = C.CFUNCTYPE(None, C.c_void_p)
_sig = {
    "fo_last_error": (C.c_char_p, []),
    "fo_runtime_init": (C.c_int32, [C.c_int32, C.POINTER(_P)]),
    "fo_runtime_free": (None, [_P]),
    "fo_runtime_synchronize": (C.c_int32, [_P]),
    "fo_runtime_set_trace": (C.c_int32, [_P, TRACE_SINK, TRACE_DONE, _P]),
    "fo_runtime_device_info": (C.c_int32, [_P, C.POINTER(C.c_int32), C.c_char_p, C.c_uint64]),
    "fo_buffer_alloc": (C.c_int32, [_P, C.c_uint64, C.POINTER(_P)]),
    "fo_buffer_free": (None, [_P]),
    "fo_buffer_clone": (C.c_int32, [_P, _P, C.POINTER(_P)]),
    "fo_buffer_bytes": (C.c_uint64, [_P]),
    "fo_buffer_flush": (C.c_int32, [_P, _P]),
    "fo_write": (C.c_int32, [_P, _P, C.c_uint64, _P]),
    "fo_read": (C.c_int32, [_P, _P, _P, C.c_uint64]),
    "fo_event_record": (C.c_int32, [_P, C.c_int32]),
    "fo_event_elapsed_ms": (C.c_int32, [_P, C.c_int32, C.c_int32, C.POINTER(C.c_float)]),
    "fo_graph_begin": (C.c_int32, [_P]),
    "fo_graph_end": (C.c_int32, [_P, C.POINTER(_P)]),
    "fo_graph_launch": (C.c_int32, [_P, _P]),
    "fo_graph_free": (None, [_P]),
    "fo_mapping_parse": (C.c_int64, [C.c_char_p, C.c_char_p, C.c_char_p, C.c_uint64]),
    "fo_mapping_sequence": (
        C.c_int32,
        [C.c_char_p, C.c_char_p, C.c_int32, C.POINTER(C.c_int64), C.POINTER(C.c_int64), C.POINTER(C.c_int64), C.c_int32],
    ),
    "fo_mapping_carve": (C.c_int64, [C.c_char_p, C.c_char_p, C.c_char_p, C.c_uint64]),
    "fo_mapping_window_base": (C.c_int64, [C.c_char_p, C.c_char_p]),
    "fo_map": (C.c_int32, [_P, _P, C.c_int32, _P, C.c_int32, C.c_uint64, C.POINTER(FoOp)]),
    "fo_zip_with": (C.c_int32, [_P, _P, C.c_int32, _P, _P, C.c_int32, C.c_uint64, C.POINTER(FoOp)]),
    "fo_zip3_slots": (C.c_int32, [_P, _P, _P, _P, _P, C.c_int32, C.c_uint64, C.POINTER(FoSlots)]),
    "fo_branch_tag": (C.c_int32, [_P, _P, _P, C.c_int32, C.c_uint64, C.POINTER(FoCmp)]),
    "fo_transpose": (
        C.c_int32,
        [_P, _P, _P, C.c_int32, C.c_char_p, C.c_char_p, C.c_char_p, C.c_char_p, C.c_char_p, C.c_char_p, C.c_int32],
    ),
    "fo_transpose_chain": (C.c_int32, [_P, _P, _P, C.c_int32, C.c_int32, C.POINTER(C.c_char_p),
                                       C.POINTER(C.c_int32)]),
    "fo_safetensors_load": (C.c_int32, [_P, _P, C.c_char_p, C.c_char_p, C.c_int32, C.c_char_p]),
    "fo_safetensors_info": (C.c_int32, [C.c_char_p, C.c_char_p, C.POINTER(C.c_int32), C.POINTER(C.c_int64), C.c_int32,
                                        C.POINTER(C.c_int32), C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
    "fo_reduce": (C.c_int32, [_P, _P, _P, C.c_int32, C.c_char_p, C.c_char_p, C.c_int32, C.c_uint32, C.c_int32]),
    "fo_contraction": (
        C.c_int32,
        [_P, _P, _P, _P, C.c_int32, C.c_int32, C.c_char_p, C.c_char_p, C.c_char_p, C.c_char_p],
    ),
    "fo_contraction_noalloc": (
        C.c_int32,
        [_P, _P, _P, _P, C.c_int32, C.c_int32, C.c_char_p, C.c_char_p, C.c_char_p, C.c_char_p],
    ),
    "fo_transmute": (C.c_int32, [_P, _P, _P, C.c_int32, C.c_char_p, C.c_char_p]),
    "fo_scatter": (C.c_int32, [_P, _P, _P, _P, C.c_int32, C.c_char_p, C.c_char_p, C.c_char_p, C.c_char_p,
                               C.c_int32]),
    "fo_gather": (C.c_int32, [_P, _P, _P, _P, C.c_int32, C.c_char_p, C.c_char_p, C.c_char_p, C.c_int32]),
    "fo_rmsnorm_softmax": (C.c_int32, [_P, _P, _P, _P, C.c_int64, C.c_int64, C.c_float]),
    "fo_attention_prefill": (
        C.c_int32,
        [_P, _P, _P, _P, _P, C.c_int64, C.c_int64, C.c_int64, C.c_int64, C.c_float, C.c_int32, _P],
    ),
    "fo_gemm_w8a8_dequant": (C.c_int32, [_P, _P, _P, _P, _P, _P, C.c_int64, C.c_int64, C.c_int64]),
    "fo_mlp": (
        C.c_int32,
        [_P, _P, _P, _P, _P, _P, _P, _P, C.c_int64, C.c_int64, C.c_int64, C.c_int64],
    ),
}
for _name, (_res, _args) in _sig.items():
    _f = getattr(_lib, _name)
    _f.restype = _res
    _f.argtypes = _args

EXPORTED = tuple(_sig)


class FoError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"[{status}] {msg}")
        self.status = status


def _check(st: int):
    if st < 0:
        raise FoError(st, _lib.fo_last_error().decode())
    return st


def _b(s: Optional[str]) -> Optional[bytes]:
    return None if s is None else s.encode()


# ---- mapping utilities (host only) ----------------------------------------------------------------


def m(text: str, **sizes: int) -> str:
    """`m![text]` with axis sizes -> MappingSerde JSON (parsed by the library)."""
    axes = json.dumps(sizes).encode()
    n = _check(_lib.fo_mapping_parse(text.encode(), axes, None, 0))
    buf = C.create_string_buffer(n + 1)
    _check(_lib.fo_mapping_parse(text.encode(), axes, buf, n + 1))
    return buf.value.decode()


def sequence(memory: str, stream: str, mode: int = 0):
    """Wheels (size, live, stride) innermost-first of sequence([memory],[stream],mode)."""
    cap = 64
    s, l, st = (C.c_int64 * cap)(), (C.c_int64 * cap)(), (C.c_int64 * cap)()
    n = _check(_lib.fo_mapping_sequence(memory.encode(), stream.encode(), mode, s, l, st, cap))
    return [(s[i], l[i], st[i]) for i in range(n)]


def carve(self_map: str, piece: str) -> str:
    n = _check(_lib.fo_mapping_carve(self_map.encode(), piece.encode(), None, 0))
    buf = C.create_string_buffer(n + 1)
    _check(_lib.fo_mapping_carve(self_map.encode(), piece.encode(), buf, n + 1))
    return buf.value.decode()


def window_base(base_map: str, offset: Optional[Dict[str, int]]) -> int:
    return _check(_lib.fo_mapping_window_base(base_map.encode(), _b(json.dumps(offset or {}))))


# ---- runtime / buffers -------------------------------------------------------------------------------


class Runtime:
    def __init__(self, device: int = 0):
        h = _P()
        _check(_lib.fo_runtime_init(device, C.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            _lib.fo_runtime_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def sync(self):
        _check(_lib.fo_runtime_synchronize(self.h))

    def info(self):
        cus = C.c_int32()
        arch = C.create_string_buffer(128)
        _check(_lib.fo_runtime_device_info(self.h, C.byref(cus), arch, 128))
        return {"compute_units": cus.value, "arch": arch.value.decode()}

    def alloc(self, nbytes: int) -> "Buffer":
        return Buffer(self, nbytes)

    def upload(self, arr: np.ndarray) -> "Buffer":
        arr = np.ascontiguousarray(arr)
        b = Buffer(self, arr.nbytes)
        _check(_lib.fo_write(self.h, arr.ctypes.data, arr.nbytes, b.h))
        return b

    def record(self, slot: int):
        _check(_lib.fo_event_record(self.h, slot))

    def graph_begin(self):
        """Ops issued from here to graph_end() are recorded into a graph instead of running."""
        _check(_lib.fo_graph_begin(self.h))

    def graph_end(self) -> "Graph":
        h = _P()
        _check(_lib.fo_graph_end(self.h, C.byref(h)))
        return Graph(self, h)

    def elapsed_ms(self, a: int, b: int) -> float:
        ms = C.c_float()
        _check(_lib.fo_event_elapsed_ms(self.h, a, b, C.byref(ms)))
        return ms.value

    # -- seam ops --
    def transpose(self, dst: "Buffer", src: "Buffer", dtype: int, src_view: str, dst_view: str,
                  src_map: Optional[str] = None, dst_map: Optional[str] = None,
                  src_offset: Optional[Dict[str, int]] = None, dst_offset: Optional[Dict[str, int]] = None,
                  allow_broadcast: bool = False):
        _check(_lib.fo_transpose(self.h, dst.h, src.h, dtype, src_view.encode(), dst_view.encode(), _b(src_map),
                                 _b(dst_map), _b(json.dumps(src_offset) if src_offset else None),
                                 _b(json.dumps(dst_offset) if dst_offset else None), int(allow_broadcast)))

    def transpose_chain(self, dst: "Buffer", src: "Buffer", dtype: int, views: Sequence[str],
                        allow_broadcast: Optional[Sequence[bool]] = None):
        """The full-view transposes views[0] -> views[1] -> ... as one pass; only the last is written."""
        arr = (C.c_char_p * len(views))(*[v.encode() for v in views])
        bc = None
        if allow_broadcast is not None:
            bc = (C.c_int32 * (len(views) - 1))(*[int(b) for b in allow_broadcast])
        _check(_lib.fo_transpose_chain(self.h, dst.h, src.h, dtype, len(views), arr, bc))

    def set_trace(self, on_span=None, on_done=None):
        """on_span(name, begin_ns, end_ns) per executed op, delivered at sync(); None turns tracing off."""
        if on_span is None:
            self._trace = None
            _check(_lib.fo_runtime_set_trace(self.h, TRACE_SINK(), TRACE_DONE(), None))
            return
        sink = TRACE_SINK(lambda ctx, name, n, b, e: on_span(C.string_at(name, n).decode(), b, e))
        done = TRACE_DONE(lambda ctx: on_done() if on_done else None)
        self._trace = (sink, done)  # the callbacks live as long as the runtime uses them
        _check(_lib.fo_runtime_set_trace(self.h, sink, done, None))

    def load_safetensors(self, dst: "Buffer", path: str, name: str, dtype: int, element_map: str):
        _check(_lib.fo_safetensors_load(self.h, dst.h, str(path).encode(), name.encode(), dtype, element_map.encode()))

    def map(self, dst: "Buffer", dst_t: int, src: "Buffer", src_t: int, n: int, op: FoOp):
        _check(_lib.fo_map(self.h, dst.h, dst_t, src.h, src_t, n, C.byref(op)))

    def zip_with(self, dst: "Buffer", dst_t: int, a: "Buffer", b: "Buffer", in_t: int, n: int, op: FoOp):
        _check(_lib.fo_zip_with(self.h, dst.h, dst_t, a.h, b.h, in_t, n, C.byref(op)))

    def zip3_slots(self, dst: "Buffer", data: "Buffer", port: Optional["Buffer"], tag: "Buffer", dtype: int, n: int,
                   slots: FoSlots):
        _check(_lib.fo_zip3_slots(self.h, dst.h, data.h, port.h if port else None, tag.h, dtype, n, C.byref(slots)))

    def branch_tag(self, tag: "Buffer", src: "Buffer", dtype: int, n: int, cmps):
        """cmps: four (kind name, boundary) pairs, e.g. ("LESS", 0.0); boundary as a float or an int."""
        _check(_lib.fo_branch_tag(self.h, tag.h, src.h, dtype, n, cmp_array(cmps)))

    def reduce(self, dst: "Buffer", src: "Buffer", dtype: int, src_map: str, dst_map: str, op: int, identity_bits: int,
               allow_broadcast: bool = False):
        _check(_lib.fo_reduce(self.h, dst.h, src.h, dtype, src_map.encode(), dst_map.encode(), op, identity_bits,
                              int(allow_broadcast)))

    def contraction(self, out: "Buffer", lhs: "Buffer", rhs: "Buffer", in_t: int, out_t: int, lhs_map: str,
                    rhs_map: str, pre_reduce: str, out_map: str):
        _check(_lib.fo_contraction(self.h, out.h, lhs.h, rhs.h, in_t, out_t, lhs_map.encode(), rhs_map.encode(),
                                   pre_reduce.encode(), out_map.encode()))

    def contraction_noalloc(self, out: "Buffer", lhs: "Buffer", rhs: "Buffer", in_t: int, out_t: int, lhs_map: str,
                            rhs_map: str, pre_reduce: str, out_map: str):
        _check(_lib.fo_contraction_noalloc(self.h, out.h, lhs.h, rhs.h, in_t, out_t, lhs_map.encode(),
                                           rhs_map.encode(), pre_reduce.encode(), out_map.encode()))

    def transmute(self, dst: "Buffer", src: "Buffer", dtype: int, src_map: str, dst_map: str):
        _check(_lib.fo_transmute(self.h, dst.h, src.h, dtype, src_map.encode(), dst_map.encode()))

    def scatter(self, dst: "Buffer", src: "Buffer", index: "Buffer", dtype: int, src_map: str, key_map: str,
                dst_map: str, idx_map: str, scaled: bool):
        _check(_lib.fo_scatter(self.h, dst.h, src.h, index.h, dtype, src_map.encode(), key_map.encode(),
                               dst_map.encode(), idx_map.encode(), int(scaled)))

    def gather(self, dst: "Buffer", src: "Buffer", index: "Buffer", dtype: int, src_map: str, dst_map: str,
               idx_map: str, scaled: bool):
        _check(_lib.fo_gather(self.h, dst.h, src.h, index.h, dtype, src_map.encode(), dst_map.encode(),
                              idx_map.encode(), int(scaled)))

    # -- fused chains --
    def rmsnorm_softmax(self, out: "Buffer", x: "Buffer", gain: "Buffer", rows: int, cols: int, eps: float):
        _check(_lib.fo_rmsnorm_softmax(self.h, out.h, x.h, gain.h, rows, cols, eps))

    def attention_prefill(self, out, q, k, v, batch, heads, seq, head_dim, sqrt_d, causal=True, row_max=None):
        """row_max: optional f32 buffer of one max per query row ([B, H, S]) for p = exp(s - m)."""
        _check(_lib.fo_attention_prefill(self.h, out.h, q.h, k.h, v.h, batch, heads, seq, head_dim, sqrt_d,
                                         int(causal), row_max.h if row_max is not None else None))

    def gemm_w8a8_dequant(self, out, acc_out, a, w, scale, m_, n_, k_):
        _check(_lib.fo_gemm_w8a8_dequant(self.h, out.h, acc_out.h if acc_out else None, a.h, w.h, scale.h, m_, n_,
                                         k_))

    def mlp(self, pred, logits, x, w1, b1, w2, b2, batch, in_f, hidden, out_f):
        _check(_lib.fo_mlp(self.h, pred.h, logits.h if logits else None, x.h, w1.h, b1.h, w2.h, b2.h, batch, in_f,
                           hidden, out_f))


class Buffer:
    def __init__(self, rt: Runtime, nbytes: int):
        h = _P()
        _check(_lib.fo_buffer_alloc(rt.h, nbytes, C.byref(h)))
        self.h = h
        self.rt = rt
        self.nbytes = nbytes

    def free(self):
        if self.h:
            _lib.fo_buffer_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def write(self, arr: np.ndarray):
        arr = np.ascontiguousarray(arr)
        _check(_lib.fo_write(self.rt.h, arr.ctypes.data, arr.nbytes, self.h))

    def flush(self):
        """Runs whatever the runtime still owes this buffer (zero fill, deferred cast or relayout)."""
        _check(_lib.fo_buffer_flush(self.rt.h, self.h))

    def clone(self) -> "Buffer":
        """Storage: Clone, and Backend::reshape: a device copy of the same bytes in a new buffer."""
        h = _P()
        _check(_lib.fo_buffer_clone(self.rt.h, self.h, C.byref(h)))
        b = Buffer.__new__(Buffer)
        b.h, b.rt, b.nbytes = h, self.rt, self.nbytes
        return b

    def read(self, dtype, count: Optional[int] = None) -> np.ndarray:
        dt = np.dtype(NP_DTYPE[dtype] if isinstance(dtype, int) else dtype)
        n = self.nbytes // dt.itemsize if count is None else count
        out = np.empty(n, dtype=dt)
        _check(_lib.fo_read(self.rt.h, self.h, out.ctypes.data, out.nbytes))
        return out


class Graph:
    """A recorded op stream (fo_graph_begin .. fo_graph_end); launch() runs it on the runtime's stream."""

    def __init__(self, rt: Runtime, h):
        self.rt = rt  # the runtime outlives its graphs
        self.h = h

    def launch(self):
        _check(_lib.fo_graph_launch(self.rt.h, self.h))

    def free(self):
        if self.h:
            _lib.fo_graph_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def safetensors_info(path: str, name: str):
    """(dtype code or -1, shape, (data_begin, data_end)) of one tensor of a safetensors file; host only."""
    dt, rank = C.c_int32(), C.c_int32()
    shape = (C.c_int64 * 16)()
    b, e = C.c_uint64(), C.c_uint64()
    _check(_lib.fo_safetensors_info(str(path).encode(), name.encode(), C.byref(dt), shape, 16, C.byref(rank),
                                    C.byref(b), C.byref(e)))
    return dt.value, [shape[i] for i in range(min(rank.value, 16))], (b.value, e.value)


def op(code: str, flags: int = 0, imm0=0, imm1=0) -> FoOp:
    """An elementwise op descriptor; float immediates are passed as their f32 bit patterns."""
    def bits(v):
        if isinstance(v, float):
            return int(np.float32(v).view(np.uint32))
        return int(np.int64(v) & 0xFFFFFFFF)
    return FoOp(OP[code], flags, bits(imm0), bits(imm1))


def cmp_array(cmps):
    """Four (kind, boundary) comparisons as an fo_cmp[4]; float boundaries pass as f32 bit patterns."""
    if len(cmps) != 4:
        raise ValueError("the tag unit takes exactly four comparisons")
    arr = (FoCmp * 4)()
    for i, (kind, bnd) in enumerate(cmps):
        bits = f32_bits(bnd) if isinstance(bnd, float) else int(np.int64(bnd) & 0xFFFFFFFF)
        arr[i] = FoCmp(CMP[kind], bits)
    return arr


def slots(op_: FoOp, regs=(), port=None) -> FoSlots:
    """A slot layout: `regs` up to three (guard mask, operand0[, operand1]) immediate slots in priority
    order, `port` an optional (guard mask[, operand1]) register-file slot. Float operands pass as f32
    bit patterns."""
    def bits(v):
        return f32_bits(v) if isinstance(v, float) else int(np.int64(v) & 0xFFFFFFFF)
    s = FoSlots()
    s.op = op_
    s.n_regs = len(regs)
    for k, r in enumerate(regs):
        s.reg_guard[k] = r[0]
        s.reg_operand0[k] = bits(r[1])
        s.reg_operand1[k] = bits(r[2]) if len(r) > 2 else 0
    if port is not None:
        s.has_port = 1
        s.port_guard = port[0]
        s.port_operand1 = bits(port[1]) if len(port) > 1 else 0
    return s


def f32_bits(v: float) -> int:
    return int(np.float32(v).view(np.uint32))
