"""Affine expressions, maps and integer sets used by KTIR access descriptors.

An expression is a nested tuple:

    ("const", n)            integer literal
    ("dim", i)              i-th dimension variable (d0, d1, ...)
    ("sym", i)              i-th symbol (s0, ...)
    ("ssa", "%name")        outer SSA scalar (only in ktdp subscripts)
    ("add", a, b)  ("sub", a, b)  ("neg", a)  ("mul", a, b)
    ("floordiv", a, n)  ("ceildiv", a, n)  ("mod", a, n)

``evaluate`` works on Python ints and on NumPy integer arrays alike, so the
GPU planner evaluates one expression for every lane at once.  Division and
modulo follow MLIR: floor division and a non-negative remainder for positive
divisors (reference: ``parser_ast.py:464-490``).

A set whose constraints pin every axis on both sides with unit coefficients
lowers to a ``Box`` (reference ``affine.py:440-507``); anything else stays an
``AffineSet`` and is enumerated by brute force over ``[0, shape)``
(reference ``parser_ast.py:525-545``).
"""

from __future__ import annotations

import itertools
import re
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

import numpy as np

Expr = tuple

_TOKEN_RE = re.compile(
    r"\s*(?:(?P<num>\d+)|(?P<name>%?[A-Za-z_][\w$.]*(?:#\d+)?)|(?P<op>>=|<=|==|->|[-+*(),\[\]:]))"
)
_KEYWORDS = {"floordiv", "ceildiv", "mod"}


def tokenize(text: str) -> List[str]:
    toks: List[str] = []
    pos = 0
    text = text.strip()
    while pos < len(text):
        m = _TOKEN_RE.match(text, pos)
        if not m or m.end() == pos:
            if text[pos:].strip() == "":
                break
            raise ValueError(f"affine: cannot tokenize {text[pos:]!r} in {text!r}")
        tok = m.group("num") or m.group("name") or m.group("op")
        toks.append(tok)
        pos = m.end()
    return toks


class _ExprParser:
    """Recursive-descent parser for affine expressions.

    Grammar: expr := term (('+'|'-') term)* ;
             term := unary (('*' unary) | ('floordiv'|'ceildiv'|'mod') INT)* ;
             unary := '-' unary | atom ; atom := INT | name | '(' expr ')'
    Names resolve to dims, symbols or (with ``ssa_ok``) outer SSA values.
    """

    def __init__(self, toks, dims=(), syms=(), ssa_vars=None):
        self.toks = toks
        self.i = 0
        self.dims = {n: k for k, n in enumerate(dims)}
        self.syms = {n: k for k, n in enumerate(syms)}
        self.ssa_vars = ssa_vars  # list of intermediate-variable names or None

    def peek(self, k=0):
        j = self.i + k
        return self.toks[j] if j < len(self.toks) else None

    def take(self, expect=None):
        tok = self.peek()
        if tok is None or (expect is not None and tok != expect):
            raise ValueError(f"affine: expected {expect!r}, got {tok!r} in {' '.join(self.toks)!r}")
        self.i += 1
        return tok

    def expr(self) -> Expr:
        node = self.term()
        while self.peek() in ("+", "-"):
            op = self.take()
            rhs = self.term()
            node = ("add", node, rhs) if op == "+" else ("sub", node, rhs)
        return node

    def term(self) -> Expr:
        node = self.unary()
        while True:
            tok = self.peek()
            if tok == "*":
                self.take()
                node = ("mul", node, self.unary())
            elif tok in _KEYWORDS:
                self.take()
                rhs = self.unary()
                if rhs[0] != "const" or rhs[1] <= 0:
                    raise ValueError(f"affine: {tok} needs a positive integer constant divisor")
                node = (tok, node, rhs[1])
            else:
                return node

    def unary(self) -> Expr:
        if self.peek() == "-":
            self.take()
            inner = self.unary()
            if inner[0] == "const":
                return ("const", -inner[1])
            return ("neg", inner)
        return self.atom()

    def atom(self) -> Expr:
        tok = self.take()
        if tok == "(":
            node = self.expr()
            self.take(")")
            return node
        if tok.isdigit():
            return ("const", int(tok))
        bare = tok.lstrip("%")
        if self.ssa_vars is not None:
            if bare in self.ssa_vars:
                return ("dim", self.ssa_vars.index(bare))
            if tok.startswith("%"):
                return ("ssa", tok)
        if tok in self.dims:
            return ("dim", self.dims[tok])
        if tok in self.syms:
            return ("sym", self.syms[tok])
        if not self.dims and re.fullmatch(r"d\d+", tok):
            return ("dim", int(tok[1:]))
        if not self.syms and re.fullmatch(r"s\d+", tok):
            return ("sym", int(tok[1:]))
        raise ValueError(f"affine: unknown identifier {tok!r}")


def evaluate(node: Expr, dims: Sequence = (), syms: Sequence = (), ssa=None):
    """Evaluate *node*; operands may be ints or NumPy int arrays (broadcasting)."""
    tag = node[0]
    if tag == "const":
        return node[1]
    if tag == "dim":
        return dims[node[1]]
    if tag == "sym":
        return syms[node[1]]
    if tag == "ssa":
        if ssa is None:
            raise ValueError(f"affine: unresolved SSA reference {node[1]}")
        return ssa(node[1])
    if tag == "add":
        return evaluate(node[1], dims, syms, ssa) + evaluate(node[2], dims, syms, ssa)
    if tag == "sub":
        return evaluate(node[1], dims, syms, ssa) - evaluate(node[2], dims, syms, ssa)
    if tag == "neg":
        return -evaluate(node[1], dims, syms, ssa)
    if tag == "mul":
        return evaluate(node[1], dims, syms, ssa) * evaluate(node[2], dims, syms, ssa)
    if tag == "floordiv":
        return evaluate(node[1], dims, syms, ssa) // node[2]
    if tag == "ceildiv":
        return -((-evaluate(node[1], dims, syms, ssa)) // node[2])
    if tag == "mod":
        return evaluate(node[1], dims, syms, ssa) % node[2]
    raise ValueError(f"affine: unknown node {tag!r}")


def substitute_ssa(node: Expr, resolve) -> Expr:
    """Replace ("ssa", name) leaves by ``resolve(name)`` (an Expr)."""
    tag = node[0]
    if tag == "ssa":
        return resolve(node[1])
    if tag in ("add", "sub", "mul"):
        return (tag, substitute_ssa(node[1], resolve), substitute_ssa(node[2], resolve))
    if tag == "neg":
        return ("neg", substitute_ssa(node[1], resolve))
    if tag in ("floordiv", "ceildiv", "mod"):
        return (tag, substitute_ssa(node[1], resolve), node[2])
    return node


def depends_on_dims(node: Expr) -> set:
    tag = node[0]
    if tag == "dim":
        return {node[1]}
    if tag in ("add", "sub", "mul"):
        return depends_on_dims(node[1]) | depends_on_dims(node[2])
    if tag in ("neg", "floordiv", "ceildiv", "mod"):
        return depends_on_dims(node[1])
    return set()


def linearize(node: Expr, n_dims: int) -> Optional[Tuple[List[int], int]]:
    """Return (coeffs, const) if *node* is linear in dims with constant terms.

    ``("const", v)`` leaves may hold NumPy arrays (per-lane constants); such
    arrays may only appear additively.  Returns None for non-linear forms.
    """
    tag = node[0]
    if tag == "const":
        return [0] * n_dims, node[1]
    if tag == "dim":
        c = [0] * n_dims
        c[node[1]] = 1
        return c, 0
    if tag in ("add", "sub"):
        a = linearize(node[1], n_dims)
        b = linearize(node[2], n_dims)
        if a is None or b is None:
            return None
        s = 1 if tag == "add" else -1
        return [x + s * y for x, y in zip(a[0], b[0])], a[1] + s * b[1]
    if tag == "neg":
        a = linearize(node[1], n_dims)
        if a is None:
            return None
        return [-x for x in a[0]], -a[1]
    if tag == "mul":
        a = linearize(node[1], n_dims)
        b = linearize(node[2], n_dims)
        if a is None or b is None:
            return None
        a_const = not any(a[0]) and np.ndim(a[1]) == 0
        b_const = not any(b[0]) and np.ndim(b[1]) == 0
        if a_const:
            k = int(a[1])
            return [k * y for y in b[0]], k * b[1]
        if b_const:
            k = int(b[1])
            return [k * x for x in a[0]], k * a[1]
        return None
    return None


@dataclass(frozen=True)
class AffineMap:
    n_dims: int
    n_syms: int
    exprs: Tuple[Expr, ...]
    source: str = ""

    def eval(self, dims: Sequence, syms: Sequence = ()) -> Tuple:
        return tuple(evaluate(e, dims, syms) for e in self.exprs)

    def permutation(self) -> Optional[Tuple[int, ...]]:
        """Output k reads input dim perm[k]; None unless a pure permutation."""
        if len(self.exprs) != self.n_dims:
            return None
        perm = []
        for e in self.exprs:
            lin = linearize(e, self.n_dims)
            if lin is None or lin[1] != 0 or sum(1 for c in lin[0] if c) != 1:
                return None
            k = next(i for i, c in enumerate(lin[0]) if c)
            if lin[0][k] != 1:
                return None
            perm.append(k)
        if sorted(perm) != list(range(self.n_dims)):
            return None
        return tuple(perm)

    def is_identity(self) -> bool:
        p = self.permutation()
        return p is not None and p == tuple(range(self.n_dims))

    def is_permutation(self) -> bool:
        return self.permutation() is not None

    @staticmethod
    def identity(n: int) -> "AffineMap":
        return AffineMap(n, 0, tuple(("dim", i) for i in range(n)), f"identity({n})")


@dataclass(frozen=True)
class AffineSet:
    """``{p : c(p) >= 0 for ge-constraints, c(p) == 0 for eq-constraints}``."""
    n_dims: int
    n_syms: int
    constraints: Tuple[Tuple[str, Expr], ...]
    source: str = ""

    def contains(self, pt: Sequence[int], syms: Sequence[int] = ()) -> bool:
        for kind, e in self.constraints:
            v = evaluate(e, pt, syms)
            if (kind == "ge" and v < 0) or (kind == "eq" and v != 0):
                return False
        return True

    def mask(self, grids: Sequence[np.ndarray], syms: Sequence[int] = ()) -> np.ndarray:
        ok = np.ones(np.broadcast(*grids).shape if grids else (), dtype=bool)
        for kind, e in self.constraints:
            v = evaluate(e, grids, syms)
            ok &= (v >= 0) if kind == "ge" else (v == 0)
        return ok

    def enumerate(self, shape: Sequence[int], syms: Sequence[int] = ()) -> List[Tuple[int, ...]]:
        """All points of ``[0, shape)`` inside the set, row-major."""
        if len(shape) != self.n_dims:
            raise ValueError("AffineSet.enumerate: rank mismatch")
        grids = np.indices(tuple(shape)) if shape else []
        m = self.mask(list(grids), syms) if self.n_dims else np.array(True)
        pts = np.argwhere(m)
        return [tuple(int(x) for x in p) for p in pts]


@dataclass(frozen=True)
class Box:
    """Axis-aligned ``{p : lo[d] <= p[d] < hi[d]}``; bounds may be symbolic Exprs."""
    lo: Tuple
    hi: Tuple
    source: str = ""

    @property
    def n_dims(self) -> int:
        return len(self.lo)

    @property
    def is_concrete(self) -> bool:
        return all(isinstance(b, int) for b in self.lo + self.hi)

    def specialize(self, syms: Sequence[int]) -> "Box":
        f = lambda b: b if isinstance(b, int) else int(evaluate(b, (), syms))
        return Box(tuple(f(b) for b in self.lo), tuple(f(b) for b in self.hi), self.source)

    @property
    def extent(self) -> Tuple[int, ...]:
        return tuple(h - l for l, h in zip(self.lo, self.hi))

    def contains(self, pt: Sequence[int], syms: Sequence[int] = ()) -> bool:
        b = self if self.is_concrete else self.specialize(syms)
        return len(pt) == b.n_dims and all(l <= p < h for l, p, h in zip(b.lo, pt, b.hi))

    def enumerate(self, shape: Optional[Sequence[int]] = None, syms: Sequence[int] = ()):
        """Row-major points; *shape* must bound ``hi`` (reference ``affine.py:294-324``)."""
        b = self if self.is_concrete else self.specialize(syms)
        if shape is not None:
            if len(shape) != b.n_dims:
                raise ValueError("Box.enumerate: rank mismatch")
            for d in range(b.n_dims):
                if b.hi[d] > shape[d]:
                    raise ValueError(
                        f"Box.enumerate: hi[{d}]={b.hi[d]} exceeds shape[{d}]={shape[d]}")
        return list(itertools.product(*(range(l, h) for l, h in zip(b.lo, b.hi))))

    def is_full(self, shape: Sequence[int]) -> bool:
        return self.is_concrete and tuple(self.lo) == (0,) * len(shape) and tuple(self.hi) == tuple(shape)


def _split_dims_syms(toks, p: _ExprParser):
    dims: List[str] = []
    syms: List[str] = []
    p.take("(")
    while p.peek() != ")":
        dims.append(p.take())
        if p.peek() == ",":
            p.take()
    p.take(")")
    if p.peek() == "[":
        p.take("[")
        while p.peek() != "]":
            syms.append(p.take())
            if p.peek() == ",":
                p.take()
        p.take("]")
    return dims, syms


def _strip(text: str, kw: str) -> str:
    t = text.strip()
    if t.startswith(kw + "<"):
        if not t.endswith(">"):
            raise ValueError(f"{kw}: unterminated {text!r}")
        t = t[len(kw) + 1:-1]
    return t


def parse_affine_map(text: str) -> AffineMap:
    body = _strip(text, "affine_map")
    toks = tokenize(body)
    p = _ExprParser(toks)
    dims, syms = _split_dims_syms(toks, p)
    p.take("->")
    q = _ExprParser(toks, dims, syms)
    q.i = p.i
    q.take("(")
    exprs = []
    while q.peek() != ")":
        exprs.append(q.expr())
        if q.peek() == ",":
            q.take()
    q.take(")")
    if q.peek() is not None:
        raise ValueError(f"affine_map: trailing tokens in {text!r}")
    return AffineMap(len(dims), len(syms), tuple(exprs), text.strip())


def parse_affine_set_raw(text: str) -> AffineSet:
    body = _strip(text, "affine_set")
    toks = tokenize(body)
    p = _ExprParser(toks)
    dims, syms = _split_dims_syms(toks, p)
    p.take(":")
    q = _ExprParser(toks, dims, syms)
    q.i = p.i
    q.take("(")
    cons = []
    while q.peek() != ")":
        lhs = q.expr()
        op = q.take()
        rhs = q.expr()
        if op == ">=":
            cons.append(("ge", ("sub", lhs, rhs)))
        elif op == "<=":
            cons.append(("ge", ("sub", rhs, lhs)))
        elif op == "==":
            cons.append(("eq", ("sub", lhs, rhs)))
        else:
            raise ValueError(f"affine_set: unsupported relation {op!r}")
        if q.peek() == ",":
            q.take()
    q.take(")")
    return AffineSet(len(dims), len(syms), tuple(cons), text.strip())


def _sym_linear(node: Expr, n_dims: int, n_syms: int):
    """Split into (dim_coeffs, sym_coeffs, const) or None."""
    tag = node[0]
    if tag == "const":
        return [0] * n_dims, [0] * n_syms, node[1]
    if tag == "dim":
        d = [0] * n_dims
        d[node[1]] = 1
        return d, [0] * n_syms, 0
    if tag == "sym":
        s = [0] * n_syms
        s[node[1]] = 1
        return [0] * n_dims, s, 0
    if tag in ("add", "sub"):
        a = _sym_linear(node[1], n_dims, n_syms)
        b = _sym_linear(node[2], n_dims, n_syms)
        if a is None or b is None:
            return None
        k = 1 if tag == "add" else -1
        return ([x + k * y for x, y in zip(a[0], b[0])],
                [x + k * y for x, y in zip(a[1], b[1])], a[2] + k * b[2])
    if tag == "neg":
        a = _sym_linear(node[1], n_dims, n_syms)
        if a is None:
            return None
        return [-x for x in a[0]], [-x for x in a[1]], -a[2]
    if tag == "mul":
        a = _sym_linear(node[1], n_dims, n_syms)
        b = _sym_linear(node[2], n_dims, n_syms)
        if a is None or b is None:
            return None
        for x, y in ((a, b), (b, a)):
            if not any(x[0]) and not any(x[1]):
                k = x[2]
                return [k * v for v in y[0]], [k * v for v in y[1]], k * y[2]
        return None
    return None


def _sym_term(coeffs: List[int], const: int):
    if not any(coeffs):
        return const
    node: Expr = ("const", const)
    for j, c in enumerate(coeffs):
        if c:
            node = ("add", node, ("mul", ("const", c), ("sym", j)))
    return node


def _bound_add(a, k):
    return a + k if isinstance(a, int) else ("add", a, ("const", k))


def _bound_neg(a):
    return -a if isinstance(a, int) else ("neg", a)


def box_from_set(aset: AffineSet) -> Optional[Box]:
    """Lower an axis-aligned set to a Box (every axis bounded on both sides).

    Mirrors the lowering rule of reference ``affine.py:440-507``: each
    constraint must involve exactly one dim with coefficient +/-1; repeated
    bounds on an axis combine by max (lower) / min (upper), which is only
    decided here for concrete bounds.  Concrete empty boxes stay sets.
    """
    n = aset.n_dims
    los: List = [None] * n
    his: List = [None] * n
    for kind, e in aset.constraints:
        lin = _sym_linear(e, n, aset.n_syms)
        if lin is None:
            return None
        dc, sc, const = lin
        nz = [i for i, c in enumerate(dc) if c]
        if len(nz) != 1 or abs(dc[nz[0]]) != 1:
            return None
        i = nz[0]
        term = _sym_term(sc, const)
        if kind == "eq":
            pin = _bound_neg(term) if dc[i] == 1 else term
            lo_c, hi_c = pin, _bound_add(pin, 1)
            cands = [("lo", lo_c), ("hi", hi_c)]
        elif dc[i] == 1:
            cands = [("lo", _bound_neg(term))]
        else:
            cands = [("hi", _bound_add(term, 1))]
        for which, val in cands:
            arr = los if which == "lo" else his
            if arr[i] is None:
                arr[i] = val
            elif isinstance(arr[i], int) and isinstance(val, int):
                arr[i] = max(arr[i], val) if which == "lo" else min(arr[i], val)
            else:
                return None
    if any(v is None for v in los + his):
        return None
    if all(isinstance(v, int) for v in los + his) and any(l >= h for l, h in zip(los, his)):
        return None
    return Box(tuple(los), tuple(his), aset.source)


def parse_affine_set(text: str):
    """Box when axis-aligned and bounded, else AffineSet (reference ``parser_ast.py:440-461``)."""
    aset = parse_affine_set_raw(text)
    box = box_from_set(aset)
    return box if box is not None else aset


def parse_subscript(text: str, var_names: Sequence[str]) -> Expr:
    """Parse an indirect-access subscript; bare vars become dims, others SSA refs."""
    toks = tokenize(text)
    p = _ExprParser(toks, ssa_vars=list(var_names))
    node = p.expr()
    if p.peek() is not None:
        raise ValueError(f"subscript: trailing tokens in {text!r}")
    return node
