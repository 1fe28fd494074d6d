"""HTile front end: bind an HTile flash-attention tile program to the backend.

The reference lowers its HTile tile program
(tests/data/flash_attention_htile.mlir:26-146 in Evan-Zhao/mlir-toy) to
Triton/TileLang/cuTile source with ``translate_file``
(src/neptune_mlir/translators/triton.py:479-487), which a caller executes and
launches as ``kernel[grid](q, k, v, out)`` (tests/test_translators.py:184-194).
This module is the same entry for the MI355X backend: ``translate_file(path)``
parses the program (no MLIR installation needed: a small parser for the op
subset the tile program uses), checks that its dataflow is the online-softmax
attention recurrence, and returns a module whose attribute named after the
kernel function launches ``neptune_attn_fwd`` with the program's shapes,
scale and coverage.

Recognised forms: the program as written (``htile.dot {transpose_b}`` on a
row-major K tile) and after the reference's ``htile-dot-transpose-to-load-
order`` pass (K loaded with ``dimension_order = array<i64: 1, 0>``,
lib/HTile/HTilePasses.cpp:91-140), with canonicalised constants (a block id
of a grid dimension of size 1 folded to 0). Unsupported ops raise
``NotImplementedError`` naming the op, as the reference's translators do
(src/neptune_mlir/translators/common.py:187-197); a program that parses but
is not the attention recurrence raises ``NotImplementedError`` too.
"""

from __future__ import annotations

import json
import math
import re
import sys
import types
from dataclasses import asdict, dataclass, field
from pathlib import Path

# ---------------------------------------------------------------- tokens

_TYPE_HEADS = ("memref", "tensor", "vector", "array", "dense")


@dataclass
class Tok:
    kind: str  # ssa, sym, ident, num, str, punct, type, alias
    text: str
    line: int


def _balanced(src: str, i: int) -> int:
    """Index just past the '>' closing the '<' at src[i]."""
    depth = 0
    while i < len(src):
        c = src[i]
        if c == "<":
            depth += 1
        elif c == ">":
            depth -= 1
            if depth == 0:
                return i + 1
        elif c == '"':
            j = src.index('"', i + 1)
            i = j
        i += 1
    raise ValueError("unbalanced '<' in type or attribute")


_NUM = re.compile(r"-?(0x[0-9a-fA-F]+|\d+\.\d*(?:[eE][-+]?\d+)?|\d+(?:[eE][-+]?\d+)?)")
_IDENT = re.compile(r"[A-Za-z_][A-Za-z0-9_.$]*")
_SSA = re.compile(r"%[A-Za-z0-9_$.\-]+(?:#\d+)?(?::\d+)?")


def tokenize(src: str) -> list[Tok]:
    toks: list[Tok] = []
    i, line = 0, 1
    n = len(src)
    while i < n:
        c = src[i]
        if c == "\n":
            line += 1
            i += 1
            continue
        if c.isspace():
            i += 1
            continue
        if src.startswith("//", i):
            while i < n and src[i] != "\n":
                i += 1
            continue
        if c == "%":
            m = _SSA.match(src, i)
            if not m:
                raise ValueError(f"line {line}: bad SSA name")
            toks.append(Tok("ssa", m.group(0), line))
            i = m.end()
            continue
        if c == "@":
            m = _IDENT.match(src, i + 1)
            toks.append(Tok("sym", "@" + m.group(0), line))
            i = m.end()
            continue
        if c == "#":
            m = _IDENT.match(src, i + 1)
            j = m.end()
            if j < n and src[j] == "<":
                j = _balanced(src, j)
            toks.append(Tok("alias", src[i:j], line))
            i = j
            continue
        if c == '"':
            j = src.index('"', i + 1)
            toks.append(Tok("str", src[i + 1:j], line))
            i = j + 1
            continue
        if src.startswith("->", i):
            toks.append(Tok("punct", "->", line))
            i += 2
            continue
        if c.isdigit() or (c == "-" and i + 1 < n and src[i + 1].isdigit()):
            m = _NUM.match(src, i)
            toks.append(Tok("num", m.group(0), line))
            i = m.end()
            continue
        if c.isalpha() or c == "_":
            m = _IDENT.match(src, i)
            j = m.end()
            word = m.group(0)
            if j < n and src[j] == "<" and word in _TYPE_HEADS:
                j = _balanced(src, j)
                toks.append(Tok("type", src[i:j], line))
            else:
                toks.append(Tok("ident", word, line))
            i = j
            continue
        if c in "()[]{},:=<>*":
            toks.append(Tok("punct", c, line))
            i += 1
            continue
        raise ValueError(f"line {line}: unexpected character {c!r}")
    return toks


# -------------------------------------------------------------------- IR


@dataclass
class Op:
    name: str
    results: list[str]
    operands: list[str]
    attrs: dict
    types: list[str]
    regions: list[list["Op"]] = field(default_factory=list)
    extra: dict = field(default_factory=dict)  # op-specific pieces
    line: int = 0


class Parser:
    def __init__(self, toks: list[Tok]):
        self.t = toks
        self.i = 0
        self.aliases: dict[str, str] = {}

    # -- token helpers
    def peek(self, k: int = 0) -> Tok | None:
        j = self.i + k
        return self.t[j] if j < len(self.t) else None

    def at(self, text: str) -> bool:
        p = self.peek()
        return p is not None and p.text == text and p.kind in ("punct", "ident")

    def take(self, text: str | None = None, kind: str | None = None) -> Tok:
        p = self.peek()
        if p is None:
            raise ValueError("unexpected end of input")
        if text is not None and p.text != text:
            raise ValueError(f"line {p.line}: expected {text!r}, found {p.text!r}")
        if kind is not None and p.kind != kind:
            raise ValueError(f"line {p.line}: expected {kind}, found {p.text!r}")
        self.i += 1
        return p

    def accept(self, text: str) -> bool:
        if self.at(text):
            self.i += 1
            return True
        return False

    # -- pieces
    def ssa_list(self, close: str) -> list[str]:
        out = []
        while not self.at(close):
            out.append(self.take(kind="ssa").text)
            if not self.accept(","):
                break
        return out

    def type_(self) -> str:
        p = self.take()
        if p.kind in ("type", "ident"):
            return p.text
        raise ValueError(f"line {p.line}: expected a type, found {p.text!r}")

    def attr_value(self):
        p = self.peek()
        if p.kind == "str":
            self.i += 1
            return p.text
        if p.kind == "num":
            self.i += 1
            v = float(p.text) if any(ch in p.text for ch in ".eE") and not p.text.startswith(
                ("0x", "-0x")) else int(p.text, 0)
            if self.accept(":"):
                self.type_()
            return v
        if p.kind == "type" and p.text.startswith("array<"):
            self.i += 1
            body = p.text[len("array<"):-1]
            vals = body.split(":", 1)[1] if ":" in body else ""
            return [int(x) for x in vals.replace(" ", "").split(",") if x]
        if p.text == "[":
            self.i += 1
            vals = []
            while not self.at("]"):
                vals.append(self.attr_value())
                if not self.accept(","):
                    break
            self.take("]")
            return vals
        if p.kind in ("ident", "alias", "type"):
            self.i += 1
            return p.text
        raise ValueError(f"line {p.line}: cannot parse attribute value {p.text!r}")

    def attr_dict(self) -> dict:
        attrs: dict = {}
        if not self.accept("{"):
            return attrs
        while not self.at("}"):
            key = self.take().text
            if self.accept("="):
                attrs[key] = self.attr_value()
            else:
                attrs[key] = True
            if not self.accept(","):
                break
        self.take("}")
        return attrs

    # -- structure
    def module(self) -> list[Op]:
        funcs: list[Op] = []
        while self.peek() is not None:
            p = self.peek()
            if p.kind == "alias" and self.peek(1) is not None and self.peek(1).text == "=":
                self.i += 2
                self.aliases[p.text] = self.take().text
                continue
            if p.text == "module":
                self.i += 1
                if self.peek().kind == "sym":
                    self.i += 1
                self.attr_dict() if self.at("attributes") and self.accept("attributes") else None
                self.take("{")
                while not self.at("}"):
                    funcs.append(self.func())
                self.take("}")
                continue
            if p.text in ("func.func", "func"):
                funcs.append(self.func())
                continue
            raise ValueError(f"line {p.line}: expected a module or func.func, found {p.text!r}")
        return funcs

    def func(self) -> Op:
        line = self.take().line  # func.func
        name = self.take(kind="sym").text[1:]
        self.take("(")
        args, arg_types = [], []
        while not self.at(")"):
            args.append(self.take(kind="ssa").text)
            self.take(":")
            arg_types.append(self.type_())
            if self.peek().text == "{":  # argument attributes
                self.attr_dict()
            if not self.accept(","):
                break
        self.take(")")
        if self.accept("->"):
            self._skip_types()
        if self.accept("attributes"):
            self.attr_dict()
        body = self.block()
        return Op("func.func", [], args, {"sym_name": name}, arg_types, [body], line=line)

    def _skip_types(self):
        if self.accept("("):
            while not self.at(")"):
                self.type_()
                if not self.accept(","):
                    break
            self.take(")")
        else:
            self.type_()

    def block(self) -> list[Op]:
        self.take("{")
        ops = []
        while not self.at("}"):
            ops.append(self.op())
        self.take("}")
        return ops

    def op(self) -> Op:
        results: list[str] = []
        if self.peek().kind == "ssa":
            while True:
                r = self.take(kind="ssa").text
                if ":" in r and "#" not in r:  # %r:3 packs 3 results
                    base, cnt = r.rsplit(":", 1)
                    results += [f"{base}#{k}" for k in range(int(cnt))]
                else:
                    results.append(r)
                if not self.accept(","):
                    break
            self.take("=")
        tok = self.take()
        name = tok.text
        fn = _OP_PARSERS.get(name)
        if fn is None:
            raise NotImplementedError(f"HTile front end: unsupported op {name!r} (line {tok.line})")
        op = fn(self, name, results)
        op.line = tok.line
        return op


def _binary(p: Parser, name, results):
    a = p.take(kind="ssa").text
    p.take(",")
    b = p.take(kind="ssa").text
    attrs = p.attr_dict()
    p.take(":")
    return Op(name, results, [a, b], attrs, [p.type_()])


def _unary(p: Parser, name, results):
    a = p.take(kind="ssa").text
    attrs = p.attr_dict()
    p.take(":")
    t = p.type_()
    types_ = [t]
    if p.accept("to"):
        types_.append(p.type_())
    return Op(name, results, [a], attrs, types_)


def _constant(p: Parser, name, results):
    v = p.attr_value()
    if p.accept(":"):
        t = p.type_()
    else:
        t = "index"
    return Op(name, results, [], {"value": v}, [t])


def _load(p: Parser, name, results):
    m = p.take(kind="ssa").text
    p.take("[")
    idx = p.ssa_list("]")
    p.take("]")
    attrs = p.attr_dict()
    p.take(":")
    src = p.type_()
    p.take("->")
    dst = p.type_()
    return Op(name, results, [m] + idx, attrs, [src, dst])


def _store(p: Parser, name, results):
    v = p.take(kind="ssa").text
    p.take(",")
    m = p.take(kind="ssa").text
    p.take("[")
    idx = p.ssa_list("]")
    p.take("]")
    attrs = p.attr_dict()
    p.take(":")
    vt = p.type_()
    p.take(",")
    mt = p.type_()
    return Op(name, results, [v, m] + idx, attrs, [vt, mt])


def _full(p: Parser, name, results):
    v = p.take(kind="ssa").text
    attrs = p.attr_dict()
    p.take(":")
    st = p.type_()
    p.take("->")
    return Op(name, results, [v], attrs, [st, p.type_()])


def _dot(p: Parser, name, results):
    a = p.take(kind="ssa").text
    p.take(",")
    b = p.take(kind="ssa").text
    attrs = p.attr_dict()
    p.take(":")
    ta = p.type_()
    p.take(",")
    tb = p.type_()
    p.take("->")
    return Op(name, results, [a, b], attrs, [ta, tb, p.type_()])


def _reduce(p: Parser, name, results):
    a = p.take(kind="ssa").text
    attrs = {}
    while p.peek().text in ("axis", "kind"):
        key = p.take().text
        attrs[key] = p.attr_value()
    attrs.update(p.attr_dict())
    p.take(":")
    ta = p.type_()
    p.take("->")
    return Op(name, results, [a], attrs, [ta, p.type_()])


def _empty(p: Parser, name, results):
    p.take("(")
    dyn = p.ssa_list(")")
    p.take(")")
    p.take(":")
    return Op(name, results, dyn, {}, [p.type_()])


def _broadcast(p: Parser, name, results):
    p.take("ins")
    p.take("(")
    a = p.take(kind="ssa").text
    p.take(":")
    ta = p.type_()
    p.take(")")
    p.take("outs")
    p.take("(")
    b = p.take(kind="ssa").text
    p.take(":")
    tb = p.type_()
    p.take(")")
    p.take("dimensions")
    p.take("=")
    dims = p.attr_value()
    attrs = p.attr_dict()
    attrs["dimensions"] = dims
    return Op(name, results, [a, b], attrs, [ta, tb])


def _for(p: Parser, name, results):
    iv = p.take(kind="ssa").text
    p.take("=")
    lb = p.take(kind="ssa").text
    p.take("to")
    ub = p.take(kind="ssa").text
    p.take("step")
    st = p.take(kind="ssa").text
    iter_args, inits = [], []
    if p.accept("iter_args"):
        p.take("(")
        while not p.at(")"):
            iter_args.append(p.take(kind="ssa").text)
            p.take("=")
            inits.append(p.take(kind="ssa").text)
            if not p.accept(","):
                break
        p.take(")")
        if p.accept("->"):
            p._skip_types()
    body = p.block()
    attrs = p.attr_dict()
    op = Op(name, results, [lb, ub, st] + inits, attrs, [], [body])
    op.extra = {"iv": iv, "iter_args": iter_args}
    return op


def _yield(p: Parser, name, results):
    vals = []
    while p.peek().kind == "ssa":
        vals.append(p.take().text)
        if not p.accept(","):
            break
    if p.accept(":"):
        while True:
            p.type_()
            if not p.accept(","):
                break
    return Op(name, results, vals, {}, [])


def _launch(p: Parser, name, results):
    def group(kw):
        p.take(kw)
        p.take("(")
        ids = p.ssa_list(")")
        p.take(")")
        p.take("in")
        p.take("(")
        sizes = []
        while not p.at(")"):
            p.take(kind="ssa")
            p.take("=")
            sizes.append(p.take(kind="ssa").text)
            if not p.accept(","):
                break
        p.take(")")
        return ids, sizes

    bids, bsz = group("blocks")
    tids, tsz = group("threads")
    attrs = p.attr_dict() if p.accept("attributes") else {}
    body = p.block()
    op = Op(name, results, bsz + tsz, attrs, [], [body])
    op.extra = {"block_ids": bids, "thread_ids": tids}
    return op


def _term(p: Parser, name, results):
    vals = []
    while p.peek() is not None and p.peek().kind == "ssa":
        vals.append(p.take().text)
        if not p.accept(","):
            break
    if vals and p.accept(":"):
        while True:
            p.type_()
            if not p.accept(","):
                break
    return Op(name, results, vals, {}, [])


_OP_PARSERS = {
    "arith.constant": _constant,
    "arith.muli": _binary, "arith.addi": _binary, "arith.subi": _binary,
    "arith.mulf": _binary, "arith.addf": _binary, "arith.subf": _binary,
    "arith.divf": _binary, "arith.maximumf": _binary, "arith.maxnumf": _binary,
    "arith.truncf": _unary, "math.exp2": _unary,
    "htile.load": _load, "htile.store": _store, "htile.full": _full,
    "htile.dot": _dot, "htile.reduce": _reduce,
    "tensor.empty": _empty, "linalg.broadcast": _broadcast,
    "scf.for": _for, "scf.yield": _yield,
    "gpu.launch": _launch, "gpu.terminator": _term,
    "func.return": _term, "return": _term,
}

# ----------------------------------------------------------------- types

_SHAPED = re.compile(r"^(memref|tensor)<([^,>]*?)(?:,.*)?>$")


def shaped(t: str) -> tuple[list[int], str]:
    m = _SHAPED.match(t.replace(" ", ""))
    if not m:
        raise ValueError(f"not a shaped type: {t}")
    parts = m.group(2).split("x")
    return [int(d) for d in parts[:-1]], parts[-1]


# ------------------------------------------------- symbolic evaluation

_COMMUTATIVE = {"add", "mul", "max"}


def _norm(e):
    """Canonical form of an expression tree: commutative operands sorted."""
    if isinstance(e, tuple) and e and e[0] in _COMMUTATIVE:
        a, b = _norm(e[1]), _norm(e[2])
        return (e[0],) + tuple(sorted((a, b), key=repr))
    if isinstance(e, tuple):
        return tuple(_norm(x) for x in e)
    return e


class NotAttention(NotImplementedError):
    pass


def _fail(msg: str):
    raise NotAttention(f"HTile front end: not a flash-attention tile program: {msg}")


@dataclass
class AttentionProgram:
    """What the tile program computes, as the backend needs it."""

    name: str
    shape: tuple[int, int, int, int]      # memref shape [B, H, S, D]
    dtype: str                            # f16 / bf16 / f32
    block_m: int                          # query rows per program
    block_n: int                          # keys per iteration
    trip_count: int                       # iterations of the key loop
    grid: tuple[int, int, int]            # (x = query block, y = head, z = batch)
    threads: tuple[int, int, int]
    scale_log2: float                     # score scale in the exp2 domain
    pipeline_stages: int | None           # htile.pipeline_stages (bound to the kernel)
    k_dimension_order: tuple[int, int]    # (1, 0): K tile loaded transposed
    neg_init: float                       # running-max initial value
    k_dim_order: int = 0                  # K memref: 0 = [B, H, S, D], 1 = [B, H, D, S]


def _recognize(func: Op) -> AttentionProgram:
    name = func.attrs["sym_name"]
    args = func.operands
    if len(args) != 4:
        _fail(f"{name} takes {len(args)} arguments, expected q, k, v, out")
    mshapes = [shaped(t) for t in func.types]
    if any(s != mshapes[0] for s in (mshapes[2], mshapes[3])):
        _fail("q, v and out memrefs must share one shape and element type")
    shape, dtype = mshapes[0]
    if len(shape) != 4 or dtype not in ("f16", "bf16", "f32"):
        _fail(f"memref<{shape}x{dtype}> is not [B, H, S, D] in f16/bf16/f32")
    kshape, kdtype = mshapes[1]
    kt_shape = [shape[0], shape[1], shape[3], shape[2]]
    if kdtype != dtype or (kshape != shape and kshape != kt_shape):
        _fail("the k memref must be [B, H, S, D] or [B, H, D, S] of the q element type")
    q, k, v, out = args

    env: dict[str, object] = {q: ("arg", "q"), k: ("arg", "k"), v: ("arg", "v"), out: ("arg", "out")}
    consts: dict[str, object] = {}
    launches = [op for op in func.regions[0] if op.name == "gpu.launch"]
    for op in func.regions[0]:
        if op.name == "arith.constant":
            consts[op.results[0]] = op.attrs["value"]
    if len(launches) != 1:
        _fail("expected exactly one gpu.launch")
    launch = launches[0]

    def cval(ssa):
        if ssa not in consts:
            _fail(f"{ssa} is not a constant")
        return consts[ssa]

    grid = tuple(int(cval(s)) for s in launch.operands[:3])
    threads = tuple(int(cval(s)) for s in launch.operands[3:6])
    bx, by, bz = launch.extra["block_ids"]
    # a block id of a size-1 grid dimension is 0 (canonicalisation folds it)
    env[bx] = ("bid", "x") if grid[0] > 1 else 0
    env[by] = ("bid", "y") if grid[1] > 1 else 0
    env[bz] = ("bid", "z") if grid[2] > 1 else 0
    for t in launch.extra["thread_ids"]:
        env[t] = ("tid",)

    info: dict = {"loads": [], "stores": [], "loops": [], "full": {}}

    def val(ssa):
        if ssa in env:
            return env[ssa]
        if ssa in consts:
            return consts[ssa]
        _fail(f"use of undefined value {ssa}")

    def run(ops: list[Op]):
        for op in ops:
            n = op.name
            if n == "arith.constant":
                consts[op.results[0]] = op.attrs["value"]
                env[op.results[0]] = op.attrs["value"]
            elif n in ("arith.muli", "arith.addi", "arith.subi"):
                a, b = val(op.operands[0]), val(op.operands[1])
                if isinstance(a, (int, float)) and isinstance(b, (int, float)):
                    r = {"arith.muli": a * b, "arith.addi": a + b, "arith.subi": a - b}[n]
                else:
                    r = ({"arith.muli": "mul", "arith.addi": "add", "arith.subi": "sub"}[n], a, b)
                env[op.results[0]] = r
            elif n in ("arith.mulf", "arith.addf", "arith.subf", "arith.divf",
                       "arith.maximumf", "arith.maxnumf"):
                tag = {"arith.mulf": "mul", "arith.addf": "add", "arith.subf": "sub",
                       "arith.divf": "div", "arith.maximumf": "max", "arith.maxnumf": "max"}[n]
                env[op.results[0]] = (tag, val(op.operands[0]), val(op.operands[1]))
            elif n == "math.exp2":
                env[op.results[0]] = ("exp2", val(op.operands[0]))
            elif n == "arith.truncf":
                env[op.results[0]] = ("trunc", val(op.operands[0]))
            elif n == "htile.full":
                c = val(op.operands[0])
                env[op.results[0]] = ("full", c)
            elif n == "tensor.empty":
                env[op.results[0]] = ("empty",)
            elif n == "linalg.broadcast":
                env[op.results[0]] = ("bcast", val(op.operands[0]))
            elif n == "htile.reduce":
                kind = op.attrs.get("kind")
                if op.attrs.get("axis") != 1 or kind not in ("max", "sum"):
                    _fail(f"reduce axis {op.attrs.get('axis')} kind {kind}")
                env[op.results[0]] = ("red" + kind, val(op.operands[0]))
            elif n == "htile.load":
                mem = val(op.operands[0])
                idx = tuple(val(s) for s in op.operands[1:])
                dims, _ = shaped(op.types[1])
                order = tuple(op.attrs.get("dimension_order", [0, 1]))
                term = ("load", mem[1] if isinstance(mem, tuple) else mem, idx, tuple(dims), order)
                info["loads"].append(term)
                env[op.results[0]] = term
            elif n == "htile.dot":
                a, b = val(op.operands[0]), val(op.operands[1])
                env[op.results[0]] = ("dot", a, b, bool(op.attrs.get("transpose_b", False)))
            elif n == "htile.store":
                info["stores"].append((val(op.operands[0]), val(op.operands[1]),
                                       tuple(val(s) for s in op.operands[2:])))
            elif n == "scf.for":
                lb, ub, st = (val(s) for s in op.operands[:3])
                inits = [val(s) for s in op.operands[3:]]
                iv = op.extra["iv"]
                env[iv] = ("iv",)
                for i, a in enumerate(op.extra["iter_args"]):
                    env[a] = ("iter", i)
                body = op.regions[0]
                run(body[:-1])
                y = body[-1]
                if y.name != "scf.yield":
                    _fail("scf.for body does not end in scf.yield")
                ys = [val(s) for s in y.operands]
                info["loops"].append({"lb": lb, "ub": ub, "step": st, "inits": inits,
                                      "yields": ys, "attrs": op.attrs})
                for i, r in enumerate(op.results):
                    env[r] = ("final", len(info["loops"]) - 1, i)
            elif n in ("gpu.terminator", "func.return", "return", "scf.yield"):
                pass
            elif n == "gpu.launch":
                run(op.regions[0])
            else:
                raise NotImplementedError(f"HTile front end: unsupported op {n!r}")

    run(func.regions[0])

    if len(info["loops"]) != 1:
        _fail("expected one scf.for over key blocks")
    loop = info["loops"][0]
    if loop["lb"] != 0 or loop["step"] != 1 or not isinstance(loop["ub"], int):
        _fail("the key loop must run 0 .. N step 1 with a constant N")
    trip = loop["ub"]
    if len(loop["yields"]) != 3:
        _fail("the key loop must carry (row sum, accumulator, row max)")

    # identify the loads
    qloads = [t for t in info["loads"] if t[1] == "q"]
    kloads = [t for t in info["loads"] if t[1] == "k"]
    vloads = [t for t in info["loads"] if t[1] == "v"]
    if not (len(qloads) == len(kloads) == len(vloads) == 1):
        _fail("expected one tile load each of q, k and v")
    qt, kt, vt = qloads[0], kloads[0], vloads[0]
    B, H, S, D = shape
    block_m, dq = qt[3]
    if dq != D:
        _fail("the q tile must span head_dim")
    # K's memref stores [S, D] or [D, S]; the tile load may transpose it
    # (dimension_order [1, 0]) and the dot may transpose its operand: QK^T
    # needs a [D, block_n] operand, i.e. an odd number of the three flips
    # ([D, S] storage, [1, 0] load, transpose_b). When S == D the index
    # pattern tells the storage order.
    k_order = tuple(kt[4])
    if k_order not in ((0, 1), (1, 0)):
        _fail(f"K dimension_order {k_order}")
    X, Y, Z = env[bx], env[by], env[bz]
    mrow = _norm(("mul", X, block_m)) if X != 0 else 0
    kidx = _norm(kt[2])
    k_stored_t = kshape != shape or (kshape == kt_shape and kidx[2] == 0 and kidx[3] != 0)
    tile_t = k_stored_t != (k_order == (1, 0))  # tile is [D, block_n]
    if tile_t:
        dk, block_n = kt[3]
    else:
        block_n, dk = kt[3]
    bnv, dv = vt[3]
    if dk != D or dv != D or bnv != block_n or tuple(vt[4]) != (0, 1):
        _fail("K and V tiles must be block_n x head_dim")

    jrow = _norm(("mul", ("iv",), block_n))
    if _norm(qt[2]) != (Z, Y, mrow, 0):
        _fail("q tile is not q[b, h, block_x * block_m, 0]")
    if _norm(vt[2]) != (Z, Y, jrow, 0):
        _fail("the v tile is not v[b, h, j * block_n, 0]")
    if kidx != ((Z, Y, 0, jrow) if k_stored_t else (Z, Y, jrow, 0)):
        _fail("the k tile is not k[b, h, j * block_n, 0] (or k[b, h, 0, j * block_n] for a "
              "[B, H, D, S] memref)")

    # the recurrence, with the loop-carried values as ("iter", i)
    ys = loop["yields"]
    inits = loop["inits"]
    # which iter arg is which: the row max is the one compared by maximumf
    s_i, a_i, m_i = None, None, None
    for i, y in enumerate(ys):
        if isinstance(y, tuple) and y[0] == "max":
            m_i = i
    if m_i is None:
        _fail("no running row max")
    score = None
    qk = ("dot", qt, kt, not tile_t)
    for i, y in enumerate(ys):
        if i == m_i:
            continue
        y = _norm(y)
        if y[0] == "add" and any(isinstance(x, tuple) and x[0] == "redsum" for x in y[1:]):
            s_i = i
        elif y[0] == "add":
            a_i = i
    if s_i is None or a_i is None:
        _fail("cannot identify the row-sum and accumulator recurrences")
    M, L, A = ("iter", m_i), ("iter", s_i), ("iter", a_i)
    ymax = ys[m_i]
    # score = qk * full(scale)
    red = [x for x in ymax[1:] if isinstance(x, tuple) and x[0] == "redmax"]
    if len(red) != 1 or M not in ymax[1:]:
        _fail("row max is not max(m_prev, rowmax(score))")
    score = red[0][1]
    if not (isinstance(score, tuple) and score[0] == "mul"):
        _fail("score is not a scaled QK^T")
    fulls = [x for x in score[1:] if isinstance(x, tuple) and x[0] == "full"]
    rest = [x for x in score[1:] if not (isinstance(x, tuple) and x[0] == "full")]
    if len(fulls) != 1 or len(rest) != 1 or _norm(rest[0]) != _norm(qk):
        _fail("score is not QK^T (transpose folded into the dot or the K load) times a scale")
    scale_log2 = float(fulls[0][1])
    mnext = ymax
    p = ("exp2", ("sub", score, ("bcast", mnext)))
    want_sum = ("add", ("mul", L, ("exp2", ("sub", M, mnext))), ("redsum", p))
    want_acc = ("add", ("mul", A, ("exp2", ("sub", ("bcast", M), ("bcast", mnext)))),
                ("dot", ("trunc", p), vt, False))
    if _norm(ys[s_i]) != _norm(want_sum):
        _fail("row sum is not l*exp2(m_prev - m_next) + rowsum(exp2(score - m_next))")
    if _norm(ys[a_i]) != _norm(want_acc):
        _fail("accumulator is not acc*exp2(m_prev - m_next) + trunc(p) . V")
    neg = inits[m_i]
    if not (isinstance(neg, tuple) and neg[0] == "full" and isinstance(neg[1], float)):
        _fail("the running max must start from a constant")
    if inits[s_i] != ("full", 0.0) or inits[a_i] != ("full", 0.0):
        _fail("row sum and accumulator must start from 0")

    # epilogue: out[b, h, block_x * block_m, 0] = trunc(acc_final / bcast(l_final))
    if len(info["stores"]) != 1:
        _fail("expected one htile.store")
    sval, smem, sidx = info["stores"][0]
    want_out = ("trunc", ("div", ("final", 0, a_i), ("bcast", ("final", 0, s_i))))
    if smem != ("arg", "out") or _norm(sval) != _norm(want_out) or _norm(sidx) != (Z, Y, mrow, 0):
        _fail("the output is not trunc(acc / l) stored at out[b, h, block_x * block_m, 0]")
    stages = loop["attrs"].get("htile.pipeline_stages")
    if stages is not None and int(stages) not in (1, 2, 3):
        raise NotImplementedError(f"HTile front end: htile.pipeline_stages = {stages}: the HIP "
                                  "kernel stages 1, 2 or 3 K/V tiles in LDS")
    return AttentionProgram(
        name=name, shape=(B, H, S, D), dtype=dtype, block_m=block_m, block_n=block_n,
        trip_count=trip, grid=grid, threads=threads, scale_log2=scale_log2,
        pipeline_stages=int(stages) if stages is not None else None,
        k_dimension_order=k_order, neg_init=float(neg[1]), k_dim_order=int(k_stored_t))


# ------------------------------------------------------------- binding

_TORCH_DTYPES = {"f16": "float16", "bf16": "bfloat16", "f32": "float32"}


class HTileKernel:
    """The tile program bound to ``neptune_attn_fwd``.

    ``kernel[grid](q, k, v, out)`` computes what the program computes for that
    launch grid: program (bx, by, bz) writes rows [bx*block_m, +block_m) of
    out[bz, by] from q[bz, by] attending to keys [0, trip_count*block_n) of
    k/v[bz, by]. Tensors are CUDA tensors of the memref shapes and dtype with
    the memrefs' identity (row-major) layout; a [B, H, D, S] k memref binds
    to the kernel's k_dim_order 1 and the loop's htile.pipeline_stages to
    its pipeline_stages."""

    def __init__(self, program: AttentionProgram):
        self.program = program

    def __repr__(self):
        return f"HTileKernel({json.dumps(asdict(self.program))})"

    def __getitem__(self, grid):
        grid = tuple(int(g) for g in (grid if isinstance(grid, (tuple, list)) else (grid,)))
        grid = grid + (1,) * (3 - len(grid))
        return lambda *args: self._launch(grid, *args)

    def __call__(self, *args):
        return self._launch(self.program.grid, *args)

    def _launch(self, grid, q, k, v, out):
        import torch

        from . import ops

        prog = self.program
        want_dtype = getattr(torch, _TORCH_DTYPES[prog.dtype])
        B, H, S, D = prog.shape
        kshape = (B, H, D, S) if prog.k_dim_order else prog.shape
        for name, t in (("q", q), ("k", k), ("v", v), ("out", out)):
            want = kshape if name == "k" else prog.shape
            if tuple(t.shape) != want or t.dtype != want_dtype:
                raise ValueError(f"{name}: expected {list(want)} {prog.dtype}, "
                                 f"got {list(t.shape)} {t.dtype}")
            if not t.is_contiguous():
                raise ValueError(f"{name}: the memref layout is row-major contiguous")
        gx, gy, gz = grid
        rows, keys = gx * prog.block_m, prog.trip_count * prog.block_n
        if gz > B or gy > H or rows > S or keys > S:
            raise ValueError(f"grid {grid} with block_m {prog.block_m} and {prog.trip_count} "
                             f"key blocks of {prog.block_n} reads outside the memrefs {prog.shape}")
        if min(grid) <= 0:
            return out
        kk = k[:gz, :gy, :, :keys] if prog.k_dim_order else k[:gz, :gy, :keys]
        ops.attention(q[:gz, :gy, :rows], kk, v[:gz, :gy, :keys], causal=False,
                      out=out[:gz, :gy, :rows], scale_log2=prog.scale_log2,
                      pipeline_stages=prog.pipeline_stages or 0, k_dim_order=prog.k_dim_order)
        return out


def translate_source(text: str) -> types.ModuleType:
    """Parse an HTile module and bind each attention function in it."""
    funcs = Parser(tokenize(text)).module()
    mod = types.ModuleType("neptune_hip_htile_program")
    bound = []
    for f in funcs:
        kern = HTileKernel(_recognize(f))
        setattr(mod, f.attrs["sym_name"], kern)
        bound.append(f.attrs["sym_name"])
    mod.__all__ = bound
    return mod


def translate_file(path: str, plugin: str | None = None) -> types.ModuleType:
    """``translate_file`` of the reference's translators
    (src/neptune_mlir/translators/triton.py:479-487), bound to this backend:
    returns a module whose attributes are the program's kernels. ``plugin`` is
    accepted for signature compatibility; no MLIR plugin is needed."""
    return translate_source(Path(path).read_text())


def main(argv: list[str] | None = None) -> int:
    import argparse

    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("mlir_file")
    ap.add_argument("--plugin", default=None)
    args = ap.parse_args(argv)
    mod = translate_file(args.mlir_file, args.plugin)
    for name in mod.__all__:
        print(json.dumps({name: asdict(getattr(mod, name).program)}, indent=1))
    return 0


if __name__ == "__main__":
    sys.exit(main())
