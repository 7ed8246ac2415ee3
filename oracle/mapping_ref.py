"""CPU restatement of furiosa-opt's mapping semantics -- TEST INFRASTRUCTURE ONLY.

This module is part of the parity oracle. Only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` may import it, and only as the checker. The product (the HIP
library under `furiosa-opt_amd/`) never routes through it.

What it restates, and from where (paths relative to the reference repository root):

* `parse(text, sizes)` -- the `m![...]` grammar, `furiosa-mapping-macro/src/parser/parser.lalrpop:37-82`:
  `,` is a right-associative Pair; `/ % = # #{*} #{!} #{0}` are left-associative postfix operators
  binding tighter than `,`; a bare natural number is a `Broadcast`; `(..)` / `[..]` group.
* Mapping values are the MappingSerde JSON form (`furiosa-mapping-types/src/lib.rs:433-543`,
  serde's externally tagged enum), e.g. `{"Stride": {"inner": {"Symbol": {...}}, "stride": 8}}`.
* `size(m)` -- `Mapping::size`, `furiosa-mapping-types/src/lib.rs:208-219`.
* `cells(m, positions)` -- the open position semantics `M::map` of every DSL node,
  `furiosa-mapping-types/src/dsl.rs:35-277`, vectorised over an array of positions. It returns the
  per-symbol coordinate sums (an `Index` finalised to absolute coordinates: contributions of one
  symbol add up, `docs/src/mapping-tensors/mapping-expressions.md:284-333`) and a status code per
  position (live, padding kind, out of bounds). Pair gives the major (left) side's padding
  precedence, exactly as `Pair::map` (`dsl.rs:257-276`).
* `relayout_offsets(src, dst)` -- the brute-force meaning of `sequence([src],[dst],Carve)` used by
  `BufStorage::transpose` (`furiosa-opt-std/src/storage/buf.rs:257-313`): for each live dst
  position, the src position whose coordinates equal the dst position's on every src symbol.
  This is computed by coordinate matching, never from strides, so it checks the product's
  wheel resolver independently.
* `read_plan(operand, out, residue)` -- the brute-force `ReadPlan` (`buf.rs:680-753`): the
  operand position each `(out cell, live residue cell)` pair reads.
* `carve(self, piece)` -- `MappingExt::carve` (`furiosa-mapping/src/lib.rs:154-167`) restated on
  coordinates: the self factors that `piece` backs become `Top` pads.

Where this module is pinned (see tests/test_oracle_golden.py): the doc examples of
`mapping-expressions.md` (e.g. `m![B / 64, B % 32, B / 32 % 2]`: position 67 maps to `B = 97`),
the `m![C, D # 64]` padding table, the `pseudo.rs:92-151` stream vectors, the transpose and
reduce vectors of `furiosa-opt-std/src/tensor/mod.rs:359-549`, and the sequencer stride tables of
`docs/src/moving-tensors/sequencer.md:306-497` (each table entry is a closed form the brute-force
offsets must reproduce).
"""
from __future__ import annotations

import re
from typing import Dict, List, Tuple

import numpy as np

LIVE = 0
PAD_TOP = 1
PAD_ZERO = 2
PAD_BOTTOM = 3
OOB = 4

_KIND_CODE = {"Top": PAD_TOP, "Zero": PAD_ZERO, "Bottom": PAD_BOTTOM}

# ----------------------------------------------------------------------------------------------
# m![...] text -> MappingSerde JSON value
# ----------------------------------------------------------------------------------------------

_TOKEN = re.compile(r"\s*(?:(#\{[*!0]\})|([A-Z][A-Za-z0-9_]*)|(\d+)|([/%=#,()\[\]]))")


def _tokenize(text: str) -> List[Tuple[str, object]]:
    out = []
    pos = 0
    text = text.strip()
    while pos < len(text):
        mt = _TOKEN.match(text, pos)
        if not mt or mt.end() == pos:
            raise ValueError(f"m![{text}]: unexpected character at {pos}: {text[pos:]!r}")
        fill, sym, nat, punct = mt.groups()
        if fill:
            out.append(("fill", {"#{*}": "Top", "#{!}": "Bottom", "#{0}": "Zero"}[fill]))
        elif sym:
            out.append(("sym", sym))
        elif nat:
            out.append(("nat", int(nat)))
        else:
            out.append(("p", punct))
        pos = mt.end()
    return out


def parse(text: str, sizes: Dict[str, int]) -> dict:
    """Parse `m![text]` with axis sizes `sizes` (the `axes![A = 4, ...]` declaration)."""
    toks = _tokenize(text)
    i = 0

    def peek():
        return toks[i] if i < len(toks) else (None, None)

    def take():
        nonlocal i
        t = toks[i]
        i += 1
        return t

    def mapping0():
        left = mapping1()
        if peek() == ("p", ","):
            take()
            if peek()[0] is None or peek() in (("p", ")"), ("p", "]")):
                return left  # trailing comma
            right = mapping0()
            return {"Pair": {"left": left, "right": right}}
        return left

    def num():
        kind, v = take()
        if kind != "nat":
            raise ValueError(f"m![{text}]: expected a number, got {v!r}")
        return v

    def mapping1():
        node = mapping2()
        while True:
            kind, v = peek()
            if kind == "p" and v in ("/", "%", "=", "#"):
                take()
                n = num()
                if v == "/":
                    node = {"Stride": {"inner": node, "stride": n}}
                elif v == "%":
                    node = {"Modulo": {"inner": node, "modulo": n}}
                elif v == "=":
                    node = {"Resize": {"inner": node, "resize": n}}
                else:
                    node = {"Padding": {"inner": node, "padding": n, "kind": "Top"}}
            elif kind == "fill":
                take()
                n = num()
                node = {"Padding": {"inner": node, "padding": n, "kind": v}}
            else:
                return node

    def mapping2():
        kind, v = take()
        if kind == "sym":
            if v not in sizes:
                raise ValueError(f"m![{text}]: axis {v} has no declared size")
            return {"Symbol": {"symbol": v, "size": int(sizes[v])}}
        if kind == "nat":
            return {"Broadcast": {"size": v}}
        if kind == "p" and v in ("(", "["):
            inner = mapping0()
            close = take()
            if close != ("p", ")" if v == "(" else "]"):
                raise ValueError(f"m![{text}]: unbalanced {v}")
            return inner
        raise ValueError(f"m![{text}]: unexpected token {v!r}")

    node = mapping0()
    if i != len(toks):
        raise ValueError(f"m![{text}]: trailing tokens {toks[i:]}")
    return node


# ----------------------------------------------------------------------------------------------
# size and position semantics (dsl.rs)
# ----------------------------------------------------------------------------------------------


def _tag(m: dict) -> Tuple[str, dict]:
    (k, v), = m.items()
    return k, v


def size(m: dict) -> int:
    """`Mapping::size` (lib.rs:208-219)."""
    k, v = _tag(m)
    if k == "Symbol":
        return v["size"]
    if k == "Stride":
        return size(v["inner"]) // v["stride"]
    if k == "Modulo":
        return v["modulo"]
    if k == "Resize":
        return v["resize"]
    if k == "Padding":
        return v["padding"]
    if k == "Pair":
        return size(v["left"]) * size(v["right"])
    if k == "Broadcast":
        return v["size"]
    raise ValueError(f"unknown mapping node {k}")


def symbols(m: dict) -> List[str]:
    """`Mapping::idents` (lib.rs:359-383): unique symbols in first-encounter order."""
    out: List[str] = []

    def walk(n):
        k, v = _tag(n)
        if k == "Symbol":
            if v["symbol"] not in out:
                out.append(v["symbol"])
        elif k in ("Stride", "Modulo", "Resize", "Padding"):
            walk(v["inner"])
        elif k == "Pair":
            walk(v["left"])
            walk(v["right"])

    walk(m)
    return out


def cells(m: dict, pos: np.ndarray) -> Tuple[Dict[str, np.ndarray], np.ndarray]:
    """Vectorised `M::map` (dsl.rs:35-277) over int64 positions.

    Returns `(coords, status)`: `coords[S]` is the summed coordinate of symbol `S` (valid where
    `status == LIVE`), `status` is LIVE / PAD_* / OOB per position.
    """
    pos = np.asarray(pos, dtype=np.int64)
    k, v = _tag(m)
    n = size(m)
    status = np.where(pos >= n, OOB, LIVE).astype(np.int8)
    inb = pos < n
    if k == "Symbol":
        return {v["symbol"]: np.where(inb, pos, 0)}, status
    if k == "Broadcast":
        return {}, status
    if k == "Stride":
        c, s = cells(v["inner"], np.where(inb, pos * v["stride"], 0))
        return c, np.where(inb, s, OOB).astype(np.int8)
    if k == "Modulo":
        inner_n = size(v["inner"])
        c, s = cells(v["inner"], np.where(inb, pos % inner_n, 0))
        return c, np.where(inb, s, OOB).astype(np.int8)
    if k == "Resize":
        c, s = cells(v["inner"], np.where(inb, pos, 0))
        return c, np.where(inb, s, OOB).astype(np.int8)
    if k == "Padding":
        inner_n = size(v["inner"])
        in_inner = pos < inner_n
        c, s = cells(v["inner"], np.where(in_inner, pos, 0))
        st = np.where(in_inner, s, _KIND_CODE[v["kind"]])
        return c, np.where(inb, st, OOB).astype(np.int8)
    if k == "Pair":
        rn = size(v["right"])
        lc, ls = cells(v["left"], np.where(inb, pos // rn, 0))
        rc, rs = cells(v["right"], np.where(inb, pos % rn, 0))
        st = np.where(ls != LIVE, ls, rs)
        coords = dict(lc)
        for sym, arr in rc.items():
            coords[sym] = coords[sym] + arr if sym in coords else arr
        return coords, np.where(inb, st, OOB).astype(np.int8)
    raise ValueError(f"unknown mapping node {k}")


def liveness(m: dict) -> np.ndarray:
    """`iter_positions()` liveness (storage/par_iters.rs:8-16): True where the wire cell is live."""
    _, st = cells(m, np.arange(size(m), dtype=np.int64))
    return st == LIVE


# ----------------------------------------------------------------------------------------------
# brute-force relayout / read plans
# ----------------------------------------------------------------------------------------------


def _coord_key(coords: Dict[str, np.ndarray], syms: List[str], n: int, radix: int) -> np.ndarray:
    key = np.zeros(n, dtype=np.int64)
    for s in syms:
        c = coords.get(s)
        key = key * radix + (c if c is not None else 0)
    return key


def _inverse_table(memory: dict):
    """Map from a memory's live coordinate tuple (its own symbols) to its wire position."""
    msyms = symbols(memory)
    mn = size(memory)
    mpos = np.arange(mn, dtype=np.int64)
    mc, ms = cells(memory, mpos)
    radix = 1 + max([int(mc[s].max()) if s in mc and mn else 0 for s in msyms] + [0])
    live = ms == LIVE
    keys = _coord_key(mc, msyms, mn, radix)[live]
    order = np.argsort(keys, kind="stable")
    return msyms, radix, keys[order], mpos[live][order]


def _project(memory: dict, s: str, c: np.ndarray) -> np.ndarray:
    """Symbol s's coordinate restricted to the digits `memory` holds: a digit of s the memory's
    mapping does not cover is read with stride 0 (a broadcast), as the sequencer reads a stream
    piece that no memory piece covers. A covered digit (weight w, radix p) keeps its value
    (c // w) % p; a symbol the memory covers whole keeps c."""
    spans = [(x["w"], x["p"]) for x in factors(memory) if x["kind"] == "T" and x["sym"] == s]
    top = _tiled_to(spans)
    if top is not None and top >= _sym_sizes(memory)[s]:
        return c
    out = np.zeros_like(c)
    for w, p in spans:
        out += ((c // w) % p) * w
    return out


def _tiled_to(spans):
    """The coordinate bound the digits (weight, radix) cover when they tile it from weight 1
    without a gap, else None."""
    cur = 1
    for w, p in sorted(spans):
        if w != cur:
            return None
        cur = w * p
    return cur


def lookup(memory: dict, coords: Dict[str, np.ndarray], n: int) -> np.ndarray:
    """For each of `n` coordinate tuples, the memory position holding those coordinates
    (restricted to the memory's own symbols, and to the digits of each it holds), or -1 where the
    memory holds no such live cell."""
    msyms, radix, keys, positions = _inverse_table(memory)
    q = np.zeros(n, dtype=np.int64)
    bad = np.zeros(n, dtype=bool)
    for s in msyms:
        c = coords.get(s)
        c = np.zeros(n, dtype=np.int64) if c is None else _project(memory, s, c)
        bad |= c >= radix
        q = q * radix + np.minimum(c, radix - 1)
    idx = np.searchsorted(keys, q)
    idx_c = np.minimum(idx, max(len(keys) - 1, 0))
    found = (~bad) & (len(keys) > 0) & (keys[idx_c] == q) if len(keys) else np.zeros(n, bool)
    return np.where(found, positions[idx_c] if len(keys) else 0, -1)


def relayout_offsets(src: dict, dst: dict) -> Tuple[np.ndarray, np.ndarray]:
    """Brute-force `BufStorage::transpose` addressing (buf.rs:257-313) for whole tensors.

    Returns `(live, src_pos)` over dst wire positions: `live[p]` is the dst liveness
    (`iter_positions`), `src_pos[p]` the src wire position read for a live `p`.
    """
    # Every src axis must be covered by the dst stream (buf.rs:280-281: `sequence(...)` under Carve
    # "expect"s it); a dst without one of src's symbols would leave its coordinate undetermined.
    missing = set(symbols(src)) - set(symbols(dst))
    if missing:
        raise ValueError(f"relayout: src axes {sorted(missing)} are not covered by the dst stream")
    dn = size(dst)
    dc, dsn = cells(dst, np.arange(dn, dtype=np.int64))
    live = dsn == LIVE
    sp = lookup(src, dc, dn)
    if np.any(live & (sp < 0)):
        raise ValueError("relayout: a live dst cell has no src cell with equal coordinates")
    return live, sp


# ----------------------------------------------------------------------------------------------
# digit factors (used only by carve): a mapping as a product of per-symbol digits. Checked against
# `cells` by brute force in the tests, so it carries no semantics of its own.
# ----------------------------------------------------------------------------------------------


def factors(m: dict) -> List[dict]:
    """Outer -> inner digit factors: dicts with kind ('T' term / 'B' broadcast / 'P' pad), and for
    terms sym, w (coordinate weight), p (span period), n (live count), e (wire extent)."""
    k, v = _tag(m)
    if k == "Symbol":
        n = v["size"]
        return [dict(kind="T", sym=v["symbol"], w=1, p=n, n=n, e=n)]
    if k == "Broadcast":
        return [] if v["size"] == 1 else [dict(kind="B", n=v["size"], e=v["size"])]
    if k == "Pair":
        return factors(v["left"]) + factors(v["right"])
    if k == "Stride":
        f = [dict(x) for x in factors(v["inner"])]
        r = v["stride"]
        while r > 1:
            x = f[-1]
            if r % x["e"] == 0:
                r //= x["e"]
                f.pop()
            elif x["e"] % r == 0:
                if x["kind"] == "T":
                    assert x["p"] % r == 0, "composite stride"
                    x.update(w=x["w"] * r, p=x["p"] // r, n=-(-x["n"] // r))
                elif x["kind"] == "B":
                    x["n"] = x["e"] // r
                else:
                    x["n"] = 1
                x["e"] //= r
                r = 1
            else:
                raise ValueError("composite stride")
        return f
    if k in ("Modulo", "Resize"):
        f = [dict(x) for x in factors(v["inner"])]
        r = v["modulo"] if k == "Modulo" else v["resize"]
        total = int(np.prod([x["e"] for x in f])) if f else 1
        if r == total:
            return f
        keep = []
        for x in reversed(f):
            if r == 1:
                break
            if r % x["e"] == 0:
                keep.insert(0, x)
                r //= x["e"]
            elif r < x["e"]:
                if x["kind"] == "T" and k == "Modulo":
                    assert x["p"] % r == 0, "composite modulo"
                    x["p"] = r
                x["n"] = min(x["n"], r) if x["kind"] != "B" else r
                x["e"] = r
                keep.insert(0, x)
                r = 1
            else:
                raise ValueError("composite modulo/resize")
        return keep
    if k == "Padding":
        f = [dict(x) for x in factors(v["inner"])]
        n = v["padding"]
        total = int(np.prod([x["e"] for x in f])) if f else 1
        if n == total:
            return f
        if not f:
            return [dict(kind="P", n=1, e=n)]
        inner = int(np.prod([x["e"] for x in f[1:]])) if len(f) > 1 else 1
        if n % inner:
            raise ValueError("composite padding")
        f[0]["e"] = n // inner
        return f
    raise ValueError(k)


def _unfactor(f: List[dict], sizes: Dict[str, int]) -> dict:
    out = None
    for x in reversed(f):
        if x["kind"] == "T":
            node = {"Symbol": {"symbol": x["sym"], "size": sizes[x["sym"]]}}
            if x["w"] != 1:
                node = {"Stride": {"inner": node, "stride": x["w"]}}
            if x["p"] != sizes[x["sym"]] // x["w"]:
                node = {"Modulo": {"inner": node, "modulo": x["p"]}}
            if x["n"] < x["p"]:
                node = {"Resize": {"inner": node, "resize": x["n"]}}
        elif x["kind"] == "B":
            node = {"Broadcast": {"size": x["n"]}}
        else:
            node = {"Broadcast": {"size": 1}}
        if x["e"] > x["n"]:
            node = {"Padding": {"inner": node, "padding": x["e"], "kind": "Top"}}
        out = node if out is None else {"Pair": {"left": node, "right": out}}
    return out if out is not None else {"Broadcast": {"size": 1}}


def _sym_sizes(*ms: dict) -> Dict[str, int]:
    out: Dict[str, int] = {}

    def walk(n):
        k, v = _tag(n)
        if k == "Symbol":
            out[v["symbol"]] = v["size"]
        elif k == "Pair":
            walk(v["left"])
            walk(v["right"])
        elif "inner" in v:
            walk(v["inner"])

    for m in ms:
        walk(m)
    return out


def carve(self_m: dict, piece: dict) -> dict:
    """`MappingExt::carve` (furiosa-mapping/src/lib.rs:154-167): `self` sequenced as the stream
    against `piece`; each self digit `piece` backs becomes a `Top` pad of its size (position 0
    live), any other digit stays. Digits are split at the union of both sides' span boundaries."""
    fs, fp = factors(self_m), factors(piece)
    breaks: Dict[str, set] = {}
    for x in fs + fp:
        if x["kind"] == "T":
            breaks.setdefault(x["sym"], set()).update({x["w"], x["w"] * x["p"]})
    backed = set()
    for x in fp:
        if x["kind"] == "T":
            b = sorted(bp for bp in breaks[x["sym"]] if x["w"] <= bp <= x["w"] * x["p"])
            backed.update((x["sym"], b[j]) for j in range(len(b) - 1))
    out: List[dict] = []
    for x in fs:
        if x["kind"] != "T":
            out.append(x)
            continue
        b = sorted(bp for bp in breaks[x["sym"]] if x["w"] <= bp <= x["w"] * x["p"])
        q = [b[j + 1] // b[j] for j in range(len(b) - 1)]
        if not q:  # a one-value digit: only its wire extent remains
            if x["e"] > 1:
                out.append(dict(kind="P", n=1, e=x["e"]))
            continue
        L, prod = 0, 1
        while L < len(q) and prod < x["n"]:
            prod *= q[L]
            L += 1
        L = max(L, 1)
        inner = int(np.prod(q[: L - 1])) if L > 1 else 1
        sub = []
        for j in range(L):
            outer = j == L - 1
            e = x["e"] // inner if outer else q[j]
            n = x["n"] // inner if outer else q[j]
            if (x["sym"], b[j]) in backed:
                sub.append(dict(kind="P", n=1, e=e))
            else:
                sub.append(dict(kind="T", sym=x["sym"], w=b[j], p=q[j], n=n, e=e))
        out.extend(reversed(sub))
    return _unfactor(out, _sym_sizes(self_m, piece))


def pair(a: dict, b: dict) -> dict:
    return {"Pair": {"left": a, "right": b}}


def is_identity(m: dict) -> bool:
    k, v = _tag(m)
    return k == "Broadcast" and v["size"] == 1


def remove_padding(m: dict) -> dict:
    """`Mapping::remove_padding` (furiosa-mapping-types/src/lib.rs:324-337): the Padding wrappers of
    the left spine go; a left side that becomes the identity hands over to the right side."""
    k, v = _tag(m)
    if k == "Padding":
        return remove_padding(v["inner"])
    if k == "Pair":
        left = remove_padding(v["left"])
        if is_identity(left):
            return remove_padding(v["right"])
        return pair(left, v["right"])
    return m


def first_axis(m: dict) -> dict:
    """The first live axis term of `m`, outer to inner, as a mapping of its own (`axes().next()`,
    then `AxisTerm::to_term`; backend/op_prep.rs:45-89 picks the indexed axis this way)."""
    sizes = _sym_sizes(m)
    for x in factors(m):
        if x["kind"] == "T" and x["n"] > 0:
            return _unfactor([dict(x, e=x["n"])], sizes)
    raise ValueError("mapping has no live axis term")


def stream_offsets(memory: dict, stream: dict, padded: bool = False) -> np.ndarray:
    """`sequence(&[memory], &[stream], Read)[0].iter()` by brute force: for every stream position,
    the memory wire position holding the cell with equal coordinates. A stream with interior padding
    raises unless `padded`; then a padding position gets -1. (SequencerConfig::iter,
    furiosa-mapping-types/src/lib.rs:866-905, walks every position; a stream pad that no memory
    cell backs is a wheel of memory stride 0, so its positions repeat the offsets of the pad's
    first, live, position.)"""
    n = size(stream)
    coords, st = cells(stream, np.arange(n, dtype=np.int64))
    dead = st != LIVE
    if np.any(dead) and not padded:
        raise ValueError("stream_offsets: padded stream")
    pos = lookup(memory, {k: v[~dead] for k, v in coords.items()}, int(np.count_nonzero(~dead)))
    if np.any(pos < 0):
        raise ValueError("stream_offsets: a stream cell is absent from memory")
    out = np.full(n, -1, dtype=np.int64)
    out[~dead] = pos
    return out


def read_plan(operand: dict, out: dict, residue: dict):
    """Brute-force `ReadPlan` (buf.rs:680-753).

    Returns `(out_live, live_r, pos)`: `out_live[o]` the out liveness, `live_r` the live residue
    positions in wire order (the fold order), and `pos[o, j]` the operand wire position that out
    cell `o` reads for live residue cell `live_r[j]` (-1 when the operand holds no such cell).
    """
    on, rn = size(out), size(residue)
    oc, ost = cells(out, np.arange(on, dtype=np.int64))
    rc, rst = cells(residue, np.arange(rn, dtype=np.int64))
    live_r = np.nonzero(rst == LIVE)[0]
    nr = len(live_r)
    coords = {}
    for s in set(oc) | set(rc):
        a = oc.get(s, np.zeros(on, np.int64))[:, None]
        b = rc.get(s, np.zeros(rn, np.int64))[live_r][None, :]
        coords[s] = (a + b).reshape(-1)
    pos = lookup(operand, coords, on * nr).reshape(on, nr)
    return ost == LIVE, live_r, pos
