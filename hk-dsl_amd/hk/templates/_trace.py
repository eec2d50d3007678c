"""Epilogue capture: run a user's epilogue on symbolic tiles and compile what it did.

The reference traces the epilogue into its kernel's store through its DSL
(python/hk/templates/gemm.py:290-339, `rewrite` + `_call`). Here the callable runs once,
at bind time, on `Sym` values that record every operation into an expression graph
(hash-consed, so a value used twice is computed once). The graph is then compiled to
one of the two forms libhkx.so runs (include/hkx.h):

* the fused form -- act(acc * col_scale[m] * row_scale[n] * cmul + row_add[n] +
  tile_add[m, n] + cadd), act one of none / gelu(tanh) / silu / relu -- which the GEMM
  kernels apply in registers before their one store: bias, the activations, per-token x
  per-channel dequant, a residual, a scale;
* anything else, as a register program (HKX_OP_*) the reduction pass interprets once
  per element on the fp32 sum (the reference's separate pass for an epilogue that does
  not fit its kernel, templates/gemm.py:616-634).

Semantics follow the reference's tiles, element by element: `acc` is C's fp32
accumulator; operands are converted to fp32 where they are loaded (:212-226); `ctx.row`
and `ctx.col` are C's coordinates (this build evaluates every element as its own 1 x 1
tile, so a fill such as `acc.right_fill_(1000 - ctx.col, 0.0)` -- columns at or past
the index -- means column >= 1000, exactly as on the reference's tiles).
"""

from __future__ import annotations

import math
from typing import Dict, List, Optional, Tuple

# node kinds (shapes against C): what the value varies along
SCALAR, ROWV, COLV, TILEV = 0, 1, 2, 3  # ROWV: one value per column (a row vector)

UNARY = {"EXP", "EXP2", "LOG", "LOG2", "ABS", "RELU", "GELU", "SILU", "SQRT", "RSQRT", "NEG",
         "STEP", "TANH", "SIGMOID", "SQUARE", "MOV"}
BINARY = {"ADD", "SUB", "MUL", "DIV", "MAX", "MIN"}
LEAVES = {"ACC", "LOAD", "CONST", "ROW", "COL", "M"}


class Node:
    __slots__ = ("op", "args", "imm", "name", "kind", "key")

    def __init__(self, op, args=(), imm=0.0, name=None, kind=SCALAR):
        self.op, self.args, self.imm, self.name, self.kind = op, tuple(args), imm, name, kind
        self.key = (op, tuple(id(a) for a in self.args), imm, name)


def _join(*kinds) -> int:
    k = 0
    for x in kinds:
        k |= x
    return k


class Graph:
    """The nodes of one trace, hash-consed."""

    def __init__(self):
        self.nodes: Dict[tuple, Node] = {}

    def make(self, op, args=(), imm=0.0, name=None, kind=None) -> Node:
        if kind is None:
            kind = _join(*(a.kind for a in args))
        n = Node(op, args, imm, name, kind)
        got = self.nodes.get(n.key)
        if got is None:
            self.nodes[n.key] = got = n
        return got

    def const(self, v: float) -> Node:
        return self.make("CONST", imm=float(v), kind=SCALAR)


class Sym:
    """A traced value: a tile of C (acc, a tile operand, anything made from them), a row
    or column vector, or a coordinate. Arithmetic and the tile methods of the reference's
    DSL (python/hk/dsl/values.py:1183-1350) record into the graph; the in-place forms
    (`+=`, `exp2_()`, ...) rebind this object, as they overwrite the tile in the DSL."""

    __slots__ = ("g", "node")

    def __init__(self, g: Graph, node: Node):
        self.g, self.node = g, node

    # -- plumbing
    def _lift(self, o) -> Node:
        if isinstance(o, Sym):
            if o.g is not self.g:
                raise TypeError("an epilogue mixed values from two traces")
            return o.node
        if isinstance(o, bool) or not isinstance(o, (int, float)):
            raise TypeError(f"an epilogue combines tiles with tiles, vectors and Python "
                            f"numbers, not {type(o).__name__}")
        return self.g.const(o)

    def _bin(self, op, a, b) -> "Sym":
        return Sym(self.g, self.g.make(op, (a, b)))

    def _un(self, op) -> "Sym":
        return Sym(self.g, self.g.make(op, (self.node,)))

    def _set(self, s: "Sym") -> "Sym":
        self.node = s.node
        return self

    # -- arithmetic
    def __add__(self, o): return self._bin("ADD", self.node, self._lift(o))
    def __radd__(self, o): return self._bin("ADD", self._lift(o), self.node)
    def __sub__(self, o): return self._bin("SUB", self.node, self._lift(o))
    def __rsub__(self, o): return self._bin("SUB", self._lift(o), self.node)
    def __mul__(self, o): return self._bin("MUL", self.node, self._lift(o))
    def __rmul__(self, o): return self._bin("MUL", self._lift(o), self.node)
    def __truediv__(self, o): return self._bin("DIV", self.node, self._lift(o))
    def __rtruediv__(self, o): return self._bin("DIV", self._lift(o), self.node)
    def __neg__(self): return self._un("NEG")
    def __pos__(self): return self
    def __abs__(self): return self._un("ABS")
    def __iadd__(self, o): return self._set(self + o)
    def __isub__(self, o): return self._set(self - o)
    def __imul__(self, o): return self._set(self * o)
    def __itruediv__(self, o): return self._set(self / o)

    def __bool__(self):
        raise TypeError("an epilogue value has no truth value on the host: it is per element "
                        "of C. Select with a fill (right_fill_, left_fill_, ...) or step()")

    def __eq__(self, o):  # identity, as the reference's tiles outside index maps
        return self is o

    __hash__ = object.__hash__

    # -- the tile methods
    def maximum(self, o): return self._bin("MAX", self.node, self._lift(o))
    def minimum(self, o): return self._bin("MIN", self.node, self._lift(o))
    def exp(self): return self._un("EXP")
    def exp2(self): return self._un("EXP2")
    def log(self): return self._un("LOG")
    def log2(self): return self._un("LOG2")
    def abs(self): return self._un("ABS")
    def relu(self): return self._un("RELU")
    def gelu(self): return self._un("GELU")
    def silu(self): return self._un("SILU")
    def sqrt(self): return self._un("SQRT")
    def rsqrt(self): return self._un("RSQRT")
    def sigmoid(self): return self._un("SIGMOID")
    def tanh(self): return self._un("TANH")
    def step(self): return self._un("STEP")
    def copy(self): return Sym(self.g, self.node)
    def exp_(self): return self._set(self.exp())
    def exp2_(self): return self._set(self.exp2())
    def rsqrt_(self): return self._set(self.rsqrt())
    def relu_(self): return self._set(self.relu())
    def gelu_(self): return self._set(self.gelu())
    def silu_(self): return self._set(self.silu())
    def zero_(self): return self._set(Sym(self.g, self.g.make("MUL", (self.node, self.g.const(0.0)))))
    def fill_(self, v): return self._set(Sym(self.g, self.g.make(
        "ADD", (self.g.make("MUL", (self.node, self.g.const(0.0))), self._lift(v)))))

    def to(self, dtype=None):
        """A conversion inside the epilogue: the value stays fp32 here (C's conversion is
        the store's)."""
        return Sym(self.g, self.node)

    # Fills: every element is its own 1 x 1 tile, at local row 0 and column 0. So
    # right_fill_(i) (columns >= i) fills where 0 >= i, left_fill_(i) (columns < i) where
    # 0 < i; lower_fill_ / upper_fill_ are the same on rows.
    def _fill(self, idx, value, at_or_past: bool) -> "Sym":
        i = self._lift(idx)
        v = self._lift(value)
        if at_or_past:
            n = self.g.make("SELLE", (i, v, self.node))
        else:
            n = self.g.make("SELLE", (i, self.node, v))
        return self._set(Sym(self.g, n))

    def right_fill_(self, idx, value=0.0): return self._fill(idx, value, True)
    def lower_fill_(self, idx, value=0.0): return self._fill(idx, value, True)
    def left_fill_(self, idx, value=0.0): return self._fill(idx, value, False)
    def upper_fill_(self, idx, value=0.0): return self._fill(idx, value, False)

    def triu_(self, idx, value=0.0):
        raise NotImplementedError("triu_/tril_ in a GEMM epilogue are not supported: select "
                                  "on ctx.row and ctx.col with the fills instead")

    tril_ = triu_


# ------------------------------------------------------------------ compilation

class Compiled:
    """What a trace compiles to: `form` "none" | "fused" | "program", with the fused
    fields or the program (instructions over operand names)."""

    def __init__(self):
        self.form = "none"
        self.act = "none"
        self.col_scale: Optional[str] = None
        self.row_scale: Optional[str] = None
        self.row_add: Optional[str] = None
        self.tile_add: Optional[str] = None
        self.cmul = 1.0
        self.cadd = 0.0
        self.ins: List[Tuple[str, int, int, int, int, float]] = []  # op, dst, a, b, c, imm
        self.out_reg = 0
        self.uses_coords = False

    def describe(self) -> str:
        if self.form == "none":
            return "acc"
        if self.form == "fused":
            x = "acc"
            for what, name in (("*", self.col_scale), ("*", self.row_scale)):
                if name:
                    x = f"{x} {what} {name}"
            if self.cmul != 1.0:
                x = f"{x} * {self.cmul:g}"
            for name in (self.row_add, self.tile_add):
                if name:
                    x = f"{x} + {name}"
            if self.cadd:
                x = f"{x} + {self.cadd:g}"
            return x if self.act == "none" else f"{self.act}({x})"
        return f"program of {len(self.ins)} instructions"


_ACTS = {"GELU": "gelu_tanh", "SILU": "silu", "RELU": "relu"}


def _flat(n: Node, op: str) -> List[Node]:
    if n.op == op:
        return [t for a in n.args for t in _flat(a, op)]
    return [n]


def _has_acc(n: Node, memo=None) -> bool:
    memo = {} if memo is None else memo
    if id(n) in memo:
        return memo[id(n)]
    r = n.op == "ACC" or any(_has_acc(a, memo) for a in n.args)
    memo[id(n)] = r
    return r


def match_fused(out: Node, kinds: Dict[str, str]) -> Optional[Compiled]:
    """The fused form of `out`, or None if it is not one. `kinds`: operand name -> its
    kind ("row" / "col" / "tile")."""
    c = Compiled()
    x = out
    if x.op in _ACTS:
        c.act = _ACTS[x.op]
        x = x.args[0]
    terms = _flat(x, "ADD")
    acc_terms = [t for t in terms if _has_acc(t)]
    if len(acc_terms) != 1:
        return None
    for t in terms:
        if t is acc_terms[0]:
            continue
        if t.op == "CONST":
            c.cadd += t.imm
        elif t.op == "LOAD" and kinds[t.name] == "row" and c.row_add is None:
            c.row_add = t.name
        elif t.op == "LOAD" and kinds[t.name] == "tile" and c.tile_add is None:
            c.tile_add = t.name
        else:
            return None
    n_acc = 0
    for f in _flat(acc_terms[0], "MUL"):
        if f.op == "ACC":
            n_acc += 1
        elif f.op == "CONST":
            c.cmul *= f.imm
        elif f.op == "LOAD" and kinds[f.name] == "col" and c.col_scale is None:
            c.col_scale = f.name
        elif f.op == "LOAD" and kinds[f.name] == "row" and c.row_scale is None:
            c.row_scale = f.name
        else:
            return None
    if n_acc != 1:
        return None
    trivial = (c.act == "none" and c.cmul == 1.0 and c.cadd == 0.0 and
               not (c.col_scale or c.row_scale or c.row_add or c.tile_add))
    c.form = "none" if trivial else "fused"
    return c


def compile_program(out: Node, operand_index: Dict[str, int], max_regs: int,
                    max_ins: int) -> Compiled:
    """`out` as a register program: nodes in dependency order, R0 holding the
    accumulator, registers reused after a value's last use."""
    order: List[Node] = []
    seen = set()

    def visit(n: Node):
        stack = [(n, False)]
        while stack:
            x, done = stack.pop()
            if done:
                if id(x) not in seen:
                    seen.add(id(x))
                    order.append(x)
                continue
            if id(x) in seen:
                continue
            stack.append((x, True))
            for a in reversed(x.args):
                stack.append((a, False))

    visit(out)
    last: Dict[int, int] = {}
    for i, x in enumerate(order):
        for a in x.args:
            last[id(a)] = i
    last[id(out)] = len(order)
    reg: Dict[int, int] = {}
    free = list(range(max_regs - 1, 0, -1))  # R0 is the accumulator's
    acc_live = True
    c = Compiled()
    c.form = "program"
    for i, x in enumerate(order):
        if x.op == "ACC":
            reg[id(x)] = 0
            continue
        srcs = [reg[id(a)] for a in x.args]
        # registers whose last use is this instruction can be the destination
        for a in x.args:
            if last.get(id(a)) == i:
                r = reg[id(a)]
                if r == 0:
                    acc_live = False
                    free.append(0)
                elif r not in free:
                    free.append(r)
        if not free:
            raise ValueError(f"the epilogue holds more than {max_regs} values at once")
        dst = free.pop()
        reg[id(x)] = dst
        a = srcs[0] if srcs else 0
        b = srcs[1] if len(srcs) > 1 else 0
        cc = srcs[2] if len(srcs) > 2 else 0
        if x.op == "LOAD":
            a = operand_index[x.name]
        if x.op in ("ROW", "COL"):
            c.uses_coords = True
        c.ins.append((x.op, dst, a, b, cc, x.imm if x.op == "CONST" else 0.0))
    del acc_live
    c.out_reg = reg[id(out)]
    if len(c.ins) > max_ins:
        raise ValueError(f"the epilogue compiles to {len(c.ins)} instructions; at most "
                         f"{max_ins} are taken")
    return c


def fmt_const(v: float) -> str:
    return repr(v) if math.isfinite(v) else str(v)


__all__ = ["Graph", "Sym", "Node", "Compiled", "match_fused", "compile_program",
           "SCALAR", "ROWV", "COLV", "TILEV"]
