"""KTIR (MLIR text) parser.

A hand-written lexer turns the text into tokens (type/attribute payloads such
as ``tensor<...>`` or ``affine_set<...>`` become single tokens), a statement
splitter groups tokens into operations with nested regions, and one small
interpreter per op family reads each statement.  It accepts the KTIR surface
the reference's regex parser accepts for the hot path (reference
``parser.py:85-147``, ``dialects/*::parse_*``) and yields the same semantic
content: operand order, ``shape``/``strides``/``dtype`` of memory views,
access-tile sets and orders, indirect subscripts, reduce/generic regions.
"""

from __future__ import annotations

import re
from dataclasses import dataclass
from typing import Any, Dict, List, Optional, Tuple

import numpy as np

from .affine import AffineMap, parse_affine_map, parse_affine_set, parse_subscript
from .ir import IRFunction, IRModule, Operation, Region, ScalarType, ShapedType, canonical_dtype


class KTIRParseError(ValueError):
    pass


# ---------------------------------------------------------------------------
# Lexer
# ---------------------------------------------------------------------------

@dataclass
class Tok:
    kind: str   # ssa sym caret num str ident blob alias punct region
    text: str
    value: Any = None

    def __repr__(self):
        return f"{self.kind}:{self.text}"


_PUNCT2 = ("->", ">=", "<=", "==", "::")
_PUNCT1 = "()[]{},:=+-*<>?!|"
_IDENT_RE = re.compile(r"[A-Za-z_][\w$.]*")
_NUM_RE = re.compile(r"0[xX][0-9a-fA-F]+|(?:\d+\.?\d*|\.\d+)(?:[eE][+-]?\d+)?")


def _match_angle(text: str, i: int) -> int:
    """Given text[i] == '<', return the index just past the matching '>'."""
    depth = 0
    n = len(text)
    while i < n:
        two = text[i:i + 2]
        if two in ("->", ">=", "<="):
            i += 2
            continue
        c = text[i]
        if c == "<":
            depth += 1
        elif c == ">":
            depth -= 1
            if depth == 0:
                return i + 1
        i += 1
    raise KTIRParseError("unterminated '<' payload")


def lex(text: str) -> List[Tok]:
    text = re.sub(r"//[^\n]*", "", text)
    toks: List[Tok] = []
    i, n = 0, len(text)
    while i < n:
        c = text[i]
        if c.isspace():
            i += 1
            continue
        if c == '"':
            j = text.index('"', i + 1)
            toks.append(Tok("str", text[i + 1:j]))
            i = j + 1
            continue
        if c in "%@^":
            m = re.compile(r"[\w$.]+(?:#\d+)?").match(text, i + 1)
            if not m:
                raise KTIRParseError(f"bad name at {text[i:i + 20]!r}")
            kind = {"%": "ssa", "@": "sym", "^": "caret"}[c]
            toks.append(Tok(kind, c + m.group(0)))
            i = m.end()
            continue
        if c in "#!":
            m = _IDENT_RE.match(text, i + 1)
            if m:
                j = m.end()
                if j < n and text[j] == "<":
                    k = _match_angle(text, j)
                    toks.append(Tok("blob", text[i:k]))
                    i = k
                else:
                    toks.append(Tok("alias" if c == "#" else "blob", text[i:j]))
                    i = j
                continue
        if c.isdigit() or (c == "-" and i + 1 < n and (text[i + 1].isdigit()) and _neg_allowed(toks)):
            m = _NUM_RE.match(text, i + 1 if c == "-" else i)
            s = (("-" if c == "-" else "") + m.group(0))
            toks.append(Tok("num", s))
            i = m.end()
            continue
        m = _IDENT_RE.match(text, i)
        if m:
            j = m.end()
            word = m.group(0)
            if j < n and text[j] == "<" and word in _BLOB_WORDS:
                k = _match_angle(text, j)
                toks.append(Tok("blob", text[i:k]))
                i = k
            else:
                toks.append(Tok("ident", word))
                i = j
            continue
        two = text[i:i + 2]
        if two in _PUNCT2:
            toks.append(Tok("punct", two))
            i += 2
            continue
        if c in _PUNCT1:
            toks.append(Tok("punct", c))
            i += 1
            continue
        raise KTIRParseError(f"unexpected character {c!r} near {text[i:i + 30]!r}")
    return toks


_BLOB_WORDS = {
    "tensor", "memref", "vector", "affine_map", "affine_set", "dense", "array",
    "complex", "tuple", "dense_resource", "sparse", "strided",
}


def _neg_allowed(toks: List[Tok]) -> bool:
    if not toks:
        return True
    t = toks[-1]
    if t.kind in ("ssa", "num", "blob"):
        return False
    if t.kind == "punct" and t.text in (")", "]"):
        return False
    if t.kind == "ident" and "." not in t.text:
        return False
    return True


# ---------------------------------------------------------------------------
# Types and attribute values
# ---------------------------------------------------------------------------

_SHAPED_RE = re.compile(r"^(!ktdp\.access_tile|tensor|memref|vector)<(.*)>$", re.S)


def parse_type(text: str):
    text = text.strip()
    m = _SHAPED_RE.match(text)
    if m:
        kind = {"!ktdp.access_tile": "access_tile"}.get(m.group(1), m.group(1))
        body = m.group(2).strip()
        # drop layout / memory-space suffix (", strided<...>", ", #space")
        depth = 0
        for k, ch in enumerate(body):
            if ch == "<":
                depth += 1
            elif ch == ">":
                depth -= 1
            elif ch == "," and depth == 0:
                body = body[:k].strip()
                break
        parts = body.split("x")
        dims: List[Optional[int]] = []
        k = 0
        while k < len(parts) - 1 and (parts[k].strip().isdigit() or parts[k].strip() == "?"):
            p = parts[k].strip()
            dims.append(None if p == "?" else int(p))
            k += 1
        elem = "x".join(parts[k:]).strip()
        return ShapedType(kind, tuple(dims), canonical_dtype(elem))
    if text.startswith("!") or text.startswith("#"):
        return ShapedType("other", (), text)
    return ScalarType(canonical_dtype(text))


def parse_number(s: str, dtype: Optional[str] = None):
    """Literal → Python int/float; hex literals of float types are bit patterns.

    Reference: ``parser_utils.py:188-230``.
    """
    s = s.strip()
    neg = s.startswith("-")
    body = s[1:] if neg else s
    if body[:2].lower() == "0x":
        bits = int(body, 16)
        if dtype == "f32":
            v = float(np.array([bits & 0xFFFFFFFF], dtype=np.uint32).view(np.float32)[0])
        elif dtype == "f16":
            v = float(np.array([bits & 0xFFFF], dtype=np.uint16).view(np.float16)[0])
        elif dtype == "bf16":
            v = float(np.array([(bits & 0xFFFF) << 16], dtype=np.uint32).view(np.float32)[0])
        else:
            v = bits
        return -v if neg else v
    try:
        return int(s)
    except ValueError:
        return float(s)


def _dense_payload(text: str, elem: Optional[str]):
    """``dense<...>`` → (value, is_list)."""
    inner = text[text.index("<") + 1:-1].strip()
    if inner.startswith("["):
        flat = re.findall(r"-?0[xX][0-9a-fA-F]+|-?[\d.]+(?:[eE][+-]?\d+)?|true|false|-?inf|nan", inner)
        vals = [_lit(v, elem) for v in flat]
        return vals, True
    return _lit(inner, elem), False


def _lit(v: str, elem):
    v = v.strip()
    if v == "true":
        return 1
    if v == "false":
        return 0
    if v in ("inf", "-inf", "nan"):
        return float(v)
    return parse_number(v, elem)


# ---------------------------------------------------------------------------
# Statement splitter
# ---------------------------------------------------------------------------

@dataclass
class Stmt:
    results: List[str]
    name: str
    toks: List[Tok]        # tokens after the op name; regions as Tok("region", value=Region)


class _Splitter:
    def __init__(self, toks: List[Tok], aliases: Dict[str, str]):
        self.t = toks
        self.i = 0
        self.aliases = aliases

    def peek(self, k=0) -> Optional[Tok]:
        j = self.i + k
        return self.t[j] if j < len(self.t) else None

    def _is_result_list(self, k=0) -> bool:
        j = self.i + k
        t = self.t
        if j >= len(t) or t[j].kind != "ssa":
            return False
        j += 1
        while True:
            if j < len(t) and t[j].text == "=" and t[j].kind == "punct":
                return True
            if j + 1 < len(t) and t[j].text == ":" and t[j + 1].kind == "num":
                j += 2
                continue
            if j + 1 < len(t) and t[j].text == "," and t[j + 1].kind == "ssa":
                j += 2
                continue
            return False

    def _is_op_name(self, tok: Optional[Tok]) -> bool:
        return tok is not None and tok.kind == "ident" and (
            ("." in tok.text and not tok.text[0].isdigit()) or tok.text == "return")

    def parse_region_body(self) -> Region:
        """Parse statements until the closing '}' (consumed)."""
        region = Region()
        while True:
            tok = self.peek()
            if tok is None:
                raise KTIRParseError("unexpected end of input inside region")
            if tok.kind == "punct" and tok.text == "}":
                self.i += 1
                return region
            if tok.kind == "caret":
                region.args.extend(self._block_label())
                continue
            region.ops.append(self.parse_statement())

    def _block_label(self):
        self.i += 1  # ^bb0
        args = []
        if self.peek() and self.peek().text == "(":
            self.i += 1
            while self.peek().text != ")":
                name = self.peek().text
                self.i += 1
                ty = None
                if self.peek().text == ":":
                    self.i += 1
                    ty = parse_type(self.peek().text)
                    self.i += 1
                args.append((name, ty))
                if self.peek().text == ",":
                    self.i += 1
            self.i += 1
        if self.peek() and self.peek().text == ":":
            self.i += 1
        return args

    def parse_statement(self) -> Operation:
        results: List[str] = []
        if self._is_result_list():
            while True:
                name = self.peek().text
                self.i += 1
                if self.peek().text == ":" and self.peek(1).kind == "num":
                    count = int(self.peek(1).text)
                    self.i += 2
                    results.extend(f"{name}#{k}" for k in range(count))
                else:
                    results.append(name)
                if self.peek().text == ",":
                    self.i += 1
                    continue
                break
            assert self.peek().text == "="
            self.i += 1
        head = self.peek()
        if head is None or head.kind != "ident":
            raise KTIRParseError(f"expected an operation name, got {head}")
        name = head.text
        self.i += 1
        body: List[Tok] = []
        depth = 0
        first = True
        while True:
            tok = self.peek()
            if tok is None:
                break
            if depth == 0:
                if tok.kind == "punct" and tok.text == "}":
                    break
                if tok.kind == "caret":
                    break
                if self._is_result_list() and not (first and name == "scf.for"):
                    break
                if self._is_op_name(tok) and not first:
                    break
                if tok.kind == "punct" and tok.text == "{":
                    if self._brace_is_region():
                        self.i += 1
                        body.append(Tok("region", "{...}", self.parse_region_body()))
                        first = False
                        continue
                    body.extend(self._attr_dict_tokens())
                    first = False
                    continue
            if tok.kind == "punct" and tok.text in "([":
                depth += 1
            elif tok.kind == "punct" and tok.text in ")]":
                depth -= 1
            body.append(tok)
            self.i += 1
            first = False
        text = name + " " + " ".join(t.text for t in body)
        return _build_op(Stmt(results, name, body), self.aliases, text)

    def _brace_is_region(self) -> bool:
        nxt = self.peek(1)
        if nxt is None:
            return False
        if nxt.kind == "punct" and nxt.text == "}":
            return False
        if nxt.kind in ("ident", "str"):
            after = self.peek(2)
            if after is not None and after.kind == "punct" and after.text == "=":
                return False
            if nxt.kind == "ident" and "." not in nxt.text and nxt.text != "return":
                # unit attribute such as {foo}
                return False
        return True

    def _attr_dict_tokens(self) -> List[Tok]:
        out = []
        depth = 0
        while True:
            tok = self.peek()
            if tok is None:
                raise KTIRParseError("unterminated attribute dictionary")
            out.append(tok)
            self.i += 1
            if tok.kind == "punct" and tok.text in "{([":
                depth += 1
            elif tok.kind == "punct" and tok.text in "})]":
                depth -= 1
                if depth == 0:
                    return out


# ---------------------------------------------------------------------------
# Token-list helpers used by the per-op builders
# ---------------------------------------------------------------------------

def _idx(toks: List[Tok], text: str, start=0, kind=None) -> int:
    depth = 0
    for k in range(start, len(toks)):
        t = toks[k]
        if t.kind == "punct" and t.text in "{":
            depth += 1
        elif t.kind == "punct" and t.text in "}":
            depth -= 1
        if depth == 0 and t.text == text and (kind is None or t.kind == kind):
            return k
    return -1


def _group(toks: List[Tok], k: int) -> Tuple[List[Tok], int]:
    """toks[k] is '(' or '['; return inner tokens and index past the closer."""
    opener = toks[k].text
    closer = {"(": ")", "[": "]", "{": "}"}[opener]
    depth = 0
    for j in range(k, len(toks)):
        t = toks[j]
        if t.kind == "punct" and t.text in "([{":
            depth += 1
        elif t.kind == "punct" and t.text in ")]}":
            depth -= 1
            if depth == 0:
                if t.text != closer:
                    raise KTIRParseError("mismatched brackets")
                return toks[k + 1:j], j + 1
    raise KTIRParseError("unterminated group")


def _split_commas(toks: List[Tok]) -> List[List[Tok]]:
    out, cur, depth = [], [], 0
    for t in toks:
        if t.kind == "punct" and t.text in "([{":
            depth += 1
        elif t.kind == "punct" and t.text in ")]}":
            depth -= 1
        if depth == 0 and t.kind == "punct" and t.text == ",":
            out.append(cur)
            cur = []
        else:
            cur.append(t)
    if cur:
        out.append(cur)
    return out


def _attr_value(toks: List[Tok], aliases):
    if not toks:
        return None
    if toks[0].kind == "punct" and toks[0].text == "[":
        inner, _ = _group(toks, 0)
        return [_attr_value(p, aliases) for p in _split_commas(inner)]
    t = toks[0]
    if t.kind == "alias":
        return aliases.get(t.text, t.text)
    if t.kind == "num":
        return parse_number(t.text)
    if t.kind == "str":
        return t.text
    return " ".join(x.text for x in toks)


def _parse_attr_dicts(toks: List[Tok], aliases) -> Dict[str, Any]:
    """Parse every top-level ``{k = v, ...}`` dict in *toks*."""
    attrs: Dict[str, Any] = {}
    k = 0
    while k < len(toks):
        t = toks[k]
        if t.kind == "punct" and t.text == "{":
            inner, k2 = _group(toks, k)
            for part in _split_commas(inner):
                if not part:
                    continue
                key = part[0].text
                if len(part) >= 2 and part[1].text == "=":
                    attrs[key] = _attr_value(part[2:], aliases)
                else:
                    attrs[key] = True
            k = k2
        else:
            k += 1
    return attrs


def _strip_attr_dicts(toks: List[Tok]) -> List[Tok]:
    out = []
    k = 0
    while k < len(toks):
        t = toks[k]
        if t.kind == "punct" and t.text == "{":
            _, k = _group(toks, k)
        else:
            out.append(t)
            k += 1
    return out


def _types_after(toks: List[Tok], k: int) -> List[Any]:
    """Comma-separated types starting at toks[k] (stops at '->'/'to'/'into')."""
    out = []
    j = k
    while j < len(toks):
        t = toks[j]
        if t.kind == "punct" and t.text == "(":
            inner, j = _group(toks, j)
            out.extend(parse_type(p[0].text) for p in _split_commas(inner) if p)
            continue
        if t.kind in ("blob", "ident"):
            if t.kind == "ident" and t.text in ("to", "into", "iter_args", "step", "else"):
                break
            out.append(parse_type(t.text))
            j += 1
            if j < len(toks) and toks[j].text == ",":
                j += 1
                continue
            break
        break
    return out


def _result_types(toks: List[Tok]) -> List[Any]:
    clean = _strip_attr_dicts([t for t in toks if t.kind != "region"])
    k = _last_top(clean, "->")
    if k >= 0:
        return _types_after(clean, k + 1)
    k = _last_top(clean, ":")
    if k >= 0:
        return _types_after(clean, k + 1)
    return []


def _last_top(toks: List[Tok], text: str) -> int:
    depth = 0
    best = -1
    for k, t in enumerate(toks):
        if t.kind == "punct" and t.text in "([":
            depth += 1
        elif t.kind == "punct" and t.text in ")]":
            depth -= 1
        elif depth == 0 and t.kind == "punct" and t.text == text:
            best = k
    return best


def _ins_outs(toks: List[Tok]):
    """Parse ``ins(%a, %b : t, t) outs(%c : t)`` → (ins, in_types, outs, out_types)."""
    res = {}
    for key in ("ins", "outs"):
        k = _idx(toks, key, kind="ident")
        names, types = [], []
        if k >= 0 and k + 1 < len(toks) and toks[k + 1].text == "(":
            inner, _ = _group(toks, k + 1)
            c = _last_top(inner, ":")
            head = inner if c < 0 else inner[:c]
            names = [t.text for t in head if t.kind == "ssa"]
            if c >= 0:
                types = [parse_type(p[0].text) for p in _split_commas(inner[c + 1:]) if p]
        res[key] = (names, types)
    return res["ins"][0], res["ins"][1], res["outs"][0], res["outs"][1]


def _int_list_after(toks: List[Tok], key: str) -> Optional[List[int]]:
    k = _idx(toks, key, kind="ident")
    if k < 0:
        return None
    j = k + 1
    if j < len(toks) and toks[j].text == "=":
        j += 1
    if j < len(toks) and toks[j].text == "[":
        inner, _ = _group(toks, j)
        return [int(t.text) for t in inner if t.kind == "num"]
    return None


def _regions(toks: List[Tok]) -> List[Region]:
    return [t.value for t in toks if t.kind == "region"]


def _ssa(toks: List[Tok]) -> List[str]:
    return [t.text for t in _strip_attr_dicts(toks) if t.kind == "ssa"]


# ---------------------------------------------------------------------------
# Per-op builders
# ---------------------------------------------------------------------------

def _build_op(st: Stmt, aliases, text: str) -> Operation:
    name = st.name
    if name == "func.return":
        name = "return"
    builder = _BUILDERS.get(name)
    if builder is None:
        for prefix, b in _PREFIX_BUILDERS:
            if name.startswith(prefix):
                builder = b
                break
    op = Operation(op_type=name, results=list(st.results), text=text)
    (builder or _generic)(op, st.toks, aliases)
    return op


def _generic(op: Operation, toks: List[Tok], aliases):
    op.operands = _ssa([t for t in toks if t.kind != "region"])
    op.attributes.update(_parse_attr_dicts(toks, aliases))
    op.result_types = _result_types(toks)
    op.regions = _regions(toks)


def _b_tile_id(op, toks, aliases):
    k = _idx(toks, ":")
    op.result_types = _types_after(toks, k + 1) if k >= 0 else []
    if len(op.result_types) != len(op.results):
        raise KTIRParseError(
            f"ktdp.get_compute_tile_id: {len(op.results)} result name(s) but "
            f"{len(op.result_types)} result type(s)")


def _b_memory_view(op, toks, aliases):
    ptr = next(t.text for t in toks if t.kind == "ssa")
    dyn: List[str] = []

    def _list(key):
        k = _idx(toks, key, kind="ident")
        if k < 0:
            return None
        j = k + 1
        if toks[j].text == ":":
            j += 1
        inner, _ = _group(toks, j)
        vals = []
        for part in _split_commas(inner):
            t = part[0]
            if t.kind == "ssa":
                vals.append(t.text)
                if t.text not in dyn:
                    dyn.append(t.text)
            else:
                vals.append(int(t.text))
        return vals

    sizes = _list("sizes")
    strides = _list("strides")
    attrs = _parse_attr_dicts(toks, aliases)
    rtypes = _result_types(toks)
    mt = next((t for t in rtypes if isinstance(t, ShapedType) and t.kind == "memref"), None)
    if mt is None:
        raise KTIRParseError("construct_memory_view: could not parse dtype from memref<> type")
    if sizes is not None:
        if len(sizes) != len(mt.shape):
            raise KTIRParseError("construct_memory_view: sizes count does not match memref rank")
        for s, d in zip(sizes, mt.shape):
            if d is not None and isinstance(s, int) and s != d:
                raise KTIRParseError(f"construct_memory_view: sizes {s} does not match memref dim {d}")
            if d is None and isinstance(s, int):
                raise KTIRParseError("construct_memory_view: dynamic dim requires an SSA size")
        shape = tuple(sizes)
    else:
        if any(d is None for d in mt.shape):
            raise KTIRParseError("construct_memory_view: dynamic dims need sizes")
        shape = tuple(mt.shape)
    space, ct = "HBM", None
    ms = attrs.get("memory_space")
    if isinstance(ms, str):
        m = re.search(r"memory_space<\s*(\w+)(?:\s*,\s*ct_id\s*=\s*(\d+))?\s*>", ms)
        if m:
            kind = m.group(1)
            if kind not in ("global", "ct_local"):
                raise KTIRParseError(f"Unknown #ktdp.memory_space kind {kind!r}")
            space = "HBM" if kind == "global" else "LX"
            ct = int(m.group(2)) if m.group(2) else None
    cs = attrs.get("coordinate_set")
    op.operands = [ptr] + dyn
    op.attributes = {
        "shape": shape,
        "strides": strides if strides is not None else [1],
        "memory_space": space,
        "dtype": mt.elem,
        "coordinate_set": parse_affine_set(cs) if isinstance(cs, str) else None,
        "lx_core_id": ct,
    }
    op.result_types = [mt]


def _b_dist_view(op, toks, aliases):
    """``ktdp.construct_distributed_memory_view (%p0, %p1 : memref, memref) : memref<GxH..>``:
    the partition views and the global shape (``None`` for ``?``) and dtype
    of the result type (reference dialects/ktdp_ops.py:109-140)."""
    _generic(op, toks, aliases)
    mt = op.result_types[0] if op.result_types else None
    if not isinstance(mt, ShapedType) or mt.kind != "memref":
        raise KTIRParseError("construct_distributed_memory_view: missing memref<> result type")
    op.attributes["shape"] = tuple(mt.shape)
    op.attributes["dtype"] = mt.elem


def _named_set(toks: List[Tok], key: str, aliases, what: str, required: bool = True):
    """`key = #alias` or `key = affine_set<...>` among the op's own tokens."""
    k = _idx(toks, key, kind="ident")
    if k < 0 or k + 2 >= len(toks) or toks[k + 1].text != "=":
        if required:
            raise KTIRParseError(f"{what}: missing {key}")
        return None
    v = toks[k + 2]
    text = aliases.get(v.text) if v.kind == "alias" else v.text
    if not isinstance(text, str) or not text.startswith("affine_set"):
        raise KTIRParseError(f"{what}: {key} is not an affine_set ({v.text!r})")
    return parse_affine_set(text)


def _future_groups(toks: List[Tok], aliases, what: str):
    """The `groups = <set>` inside the tile_future type, in either spelling:
    `!ktdp.tile_future<T, groups = S>` or the shortened `<(T), groups = S>`
    (reference dialects/ktdp_ops.py:1034-1080)."""
    for t in toks:
        if t.kind == "blob" and t.text.startswith("!ktdp.tile_future<"):
            m = re.search(r"groups\s*=\s*(affine_set<.*>|#[\w$.-]+)\s*>\s*$", t.text, re.S)
            if m is None:
                raise KTIRParseError(f"{what}: missing groups inside !ktdp.tile_future<...> type")
            text = aliases.get(m.group(1), m.group(1)) if m.group(1).startswith("#") else m.group(1)
            return parse_affine_set(text)
    return _named_set(toks, "groups", aliases, what + " (groups inside the tile_future type)")


def _b_inter_tile_produce(op, toks, aliases):
    """``%f = ktdp.inter_tile_produce producer_tiles_per_group = S -> <(T), groups = G> { ^bb0(%gid): ... }``
    (reference dialects/ktdp_ops.py:1083-1130)."""
    op.regions = _regions(toks)
    top = [t for t in toks if t.kind != "region"]
    op.attributes["producer_tiles_per_group"] = _named_set(top, "producer_tiles_per_group", aliases,
                                                           "ktdp.inter_tile_produce")
    op.attributes["groups"] = _future_groups(top, aliases, "ktdp.inter_tile_produce")
    op.operands = []


def _b_inter_tile_reduce(op, toks, aliases):
    """``%r = ktdp.inter_tile_reduce(%f) consumer_tiles_per_group = S, identity(%id : T) : <future> -> T_r {...}``:
    operands [future, identity...], the consumer set, the future's groups,
    the optional dependency set and the result shape (reference
    dialects/ktdp_ops.py:1234-1307)."""
    op.regions = _regions(toks)
    top = [t for t in toks if t.kind != "region"]
    what = "ktdp.inter_tile_reduce"
    if len(top) < 3 or top[0].text != "(" or top[1].kind != "ssa" or top[2].text != ")":
        raise KTIRParseError(f"{what}: expected ( %future ) after the op name")
    operands = [top[1].text]
    k = _idx(top, "identity", kind="ident")
    if k >= 0 and k + 1 < len(top) and top[k + 1].text == "(":
        j = k + 2
        depth = 1
        while j < len(top) and depth:
            t = top[j]
            if t.kind == "punct" and t.text == "(":
                depth += 1
            elif t.kind == "punct" and t.text == ")":
                depth -= 1
            elif t.kind == "ssa" and depth == 1:
                operands.append(t.text)
            j += 1
    op.operands = operands
    op.attributes["consumer_tiles_per_group"] = _named_set(top, "consumer_tiles_per_group", aliases, what)
    op.attributes["groups"] = _future_groups(top, aliases, what)
    dep = _named_set(top, "producer_dependency_per_consumer", aliases, what, required=False)
    if dep is not None:
        op.attributes["producer_dependency_per_consumer"] = dep
    arrows = [i for i, t in enumerate(top) if t.kind == "punct" and t.text == "->"]
    if arrows and arrows[-1] + 1 < len(top):
        rt_ = parse_type(top[arrows[-1] + 1].text)
        if isinstance(rt_, ShapedType):
            op.result_types = [rt_]
            op.attributes["_result_shape"] = tuple(rt_.shape)


def _b_yield_values(op, toks, aliases):
    """``ktdp.yield_partial`` / ``ktdp.yield_reduced``: the yielded SSA values."""
    op.operands = _ssa([t for t in toks if t.kind != "region"])
    k = _idx(toks, ":")
    if k >= 0:
        op.operands = _ssa(toks[:k])


def _b_access_tile(op, toks, aliases):
    view = next(t.text for t in toks if t.kind == "ssa")
    k = _idx(toks, "[")
    inner, _ = _group(toks, k)
    indices = [t.text for t in inner if t.kind == "ssa"]
    attrs = _parse_attr_dicts(toks, aliases)
    rtypes = _result_types(toks)
    at = next((t for t in rtypes if isinstance(t, ShapedType) and t.kind == "access_tile"), None)
    if at is None:
        raise KTIRParseError("construct_access_tile: missing !ktdp.access_tile<> result type")
    if at.elem != "index":
        raise KTIRParseError(f"AccessTileType element type must be 'index', got {at.elem!r}")
    bm = attrs.get("base_map")
    n = max(1, len(indices))
    base_map = parse_affine_map(bm) if isinstance(bm, str) else AffineMap.identity(n)
    cs = attrs.get("access_tile_set")
    if not isinstance(cs, str):
        raise KTIRParseError("construct_access_tile: access_tile_set is required")
    order = attrs.get("access_tile_order")
    order_map = parse_affine_map(order) if isinstance(order, str) else None
    if order_map is not None and order_map.is_identity():
        order_map = None
    op.operands = [view] + indices
    op.attributes = {
        "shape": tuple(at.shape),
        "base_map": base_map,
        "coordinate_set": parse_affine_set(cs),
        "coordinate_order": order_map,
    }
    op.result_types = [at]


def _b_indirect_tile(op, toks, aliases):
    k = _idx(toks, "intermediate_variables", kind="ident")
    if k < 0:
        raise KTIRParseError("construct_indirect_access_tile: missing intermediate_variables")
    ivs, j = _group(toks, k + 1)
    var_names = [t.text.lstrip("%") for t in ivs if t.kind == "ssa"]
    primary = toks[j].text
    sub_toks, j2 = _group(toks, j + 1)
    operands = [primary]
    subs = []
    for part in _split_commas(sub_toks):
        if part and part[0].kind == "ident" and part[0].text == "ind":
            inner, _ = _group(part, 1)
            view = inner[0].text
            idx_inner, _ = _group(inner, 1)
            exprs = [parse_subscript(" ".join(t.text for t in p), var_names)
                     for p in _split_commas(idx_inner)]
            subs.append({"kind": "indirect", "index_view_idx": len(operands) - 1, "idx_exprs": exprs})
            operands.append(view)
        else:
            subs.append({"kind": "direct_expr",
                         "subscript": parse_subscript(" ".join(t.text for t in part), var_names)})
    attrs = _parse_attr_dicts(toks[j2:], aliases)
    vss = attrs.get("variables_space_set")
    if not isinstance(vss, str):
        raise KTIRParseError("construct_indirect_access_tile: variables_space_set is required")
    vso = attrs.get("variables_space_order")
    vso_map = parse_affine_map(vso) if isinstance(vso, str) else None
    if vso_map is not None and vso_map.is_identity():
        vso_map = None
    rtypes = _result_types(toks)
    at = next((t for t in rtypes if isinstance(t, ShapedType) and t.kind == "access_tile"), None)
    if at is None:
        raise KTIRParseError("construct_indirect_access_tile: missing !ktdp.access_tile<> result type")
    op.operands = operands
    op.attributes = {
        "shape": tuple(at.shape),
        "dim_subscripts": subs,
        "intermediate_vars": var_names,
        "variables_space_set": parse_affine_set(vss),
        "variables_space_order": vso_map,
    }
    op.result_types = [at]


def _b_load(op, toks, aliases):
    op.operands = _ssa(toks)
    op.result_types = _result_types(toks)
    rt = op.result_type
    if isinstance(rt, ShapedType) and rt.kind == "tensor":
        op.attributes["_result_shape"] = tuple(rt.shape)
        op.attributes["_result_dtype"] = rt.elem


def _b_simple(op, toks, aliases):
    """``op %a, %b ... : type`` or ``op %a : t1 to t2`` (casts)."""
    clean = _strip_attr_dicts(toks)
    op.attributes.update(_parse_attr_dicts(toks, aliases))
    if clean and clean[0].kind == "ident" and op.op_type in ("arith.cmpi", "arith.cmpf"):
        op.attributes["predicate"] = clean[0].text
        clean = clean[1:]
    op.operands = [t.text for t in clean if t.kind == "ssa"]
    c = _idx(clean, ":")
    if c >= 0:
        t_idx = _idx(clean, "to", kind="ident")
        if t_idx >= 0:
            op.operand_types = _types_after(clean, c + 1)
            op.result_types = _types_after(clean, t_idx + 1)
        else:
            types = _types_after(clean, c + 1)
            op.operand_types = types
            if op.op_type in ("arith.cmpi", "arith.cmpf"):
                base = types[-1] if types else None
                if isinstance(base, ShapedType):
                    op.result_types = [ShapedType(base.kind, base.shape, "i1")]
                else:
                    op.result_types = [ScalarType("i1")]
            elif op.op_type == "arith.select":
                op.result_types = types[-1:] if types else []
            else:
                op.result_types = types[-1:] if types else []
    if op.op_type == "arith.bitcast" and op.result_types:
        rt = op.result_types[0]
        op.attributes["dst_type"] = rt.elem if isinstance(rt, ShapedType) else rt.name


def _b_constant(op, toks, aliases):
    clean = _strip_attr_dicts(toks)
    braced = _parse_attr_dicts(toks, aliases)
    c = _last_top(clean, ":")
    rtypes = _types_after(clean, c + 1) if c >= 0 else []
    rt = rtypes[0] if rtypes else None
    elem = rt.elem if isinstance(rt, ShapedType) else (rt.name if rt else None)
    payload = clean[:c] if c >= 0 else clean
    attrs: Dict[str, Any] = {}
    if not payload and "value" in braced:
        v = braced["value"]
        payload = lex(v if isinstance(v, str) else str(v))
    if payload:
        p = payload[0]
        if p.kind == "blob" and p.text.startswith("dense"):
            val, is_list = _dense_payload(p.text, elem)
            attrs["value"] = val
            if is_list:
                attrs["dense_list"] = True
        elif p.kind == "num":
            attrs["value"] = parse_number(p.text, elem)
        elif p.kind == "ident" and p.text in ("true", "false"):
            attrs["value"] = p.text == "true"
        else:
            attrs["value"] = 0
    else:
        attrs["value"] = 0
    if isinstance(rt, ShapedType) and rt.kind == "tensor":
        attrs["shape"] = tuple(rt.shape)
        attrs["dtype"] = rt.elem
        attrs["is_tensor"] = True
    op.attributes = attrs
    op.result_types = rtypes[:1]


def _b_linalg(op, toks, aliases):
    ins, in_t, outs, out_t = _ins_outs(toks)
    op.operands = ins + outs
    op.operand_types = in_t + out_t
    op.attributes.update(_parse_attr_dicts(toks, aliases))
    op.attributes["n_ins"] = len(ins)
    op.attributes["outs"] = outs
    rt = _result_types([t for t in toks if t.kind != "region"])
    arrow = _last_top(_strip_attr_dicts([t for t in toks if t.kind != "region"]), "->")
    op.result_types = rt if arrow >= 0 else list(out_t)
    for key in ("dimensions", "permutation"):
        v = _int_list_after(toks, key)
        if v is not None:
            op.attributes[key] = v
    op.regions = _regions(toks)
    if op.op_type == "linalg.reduce":
        _finish_reduce(op, toks)
    elif op.op_type == "linalg.generic":
        maps = op.attributes.get("indexing_maps")
        if isinstance(maps, list):
            op.attributes["indexing_maps"] = [parse_affine_map(m) if isinstance(m, str) else m for m in maps]
        it = op.attributes.get("iterator_types")
        if isinstance(it, list):
            op.attributes["iterator_types"] = [s.strip('"').split(".")[-1].strip(">") if isinstance(s, str) else s
                                               for s in it]


def _finish_reduce(op, toks):
    """Normalise both ``linalg.reduce`` surfaces to one region with 2 block args."""
    region = op.regions[0] if op.regions else None
    # explicit block args: "(%a : f32, %b : f32) { ... }"
    explicit_args = []
    for k, t in enumerate(toks):
        if t.kind == "punct" and t.text == "(" and k + 1 < len(toks) and toks[k + 1].kind == "ssa":
            prev = toks[k - 1] if k > 0 else None
            if prev is not None and prev.kind == "ident" and prev.text in ("ins", "outs"):
                continue
            inner, _ = _group(toks, k)
            names = [x.text for x in inner if x.kind == "ssa"]
            if names:
                explicit_args = names
    if region is not None and region.ops and not region.ops[0].operands and len(region.ops) == 1 \
            and not region.args and not explicit_args:
        fn = region.ops[0].op_type
        op.attributes["reduce_fn"] = fn
        region = None
    if region is None:
        fn = op.attributes.get("reduce_fn", "arith.addf")
        a, b = "%__reduce_in__", "%__reduce_acc__"
        body = [Operation(fn, ["%__reduce_combined__"], [a, b]),
                Operation("linalg.yield", [], ["%__reduce_combined__"])]
        region = Region([(a, None), (b, None)], body)
    else:
        if not region.args:
            names = explicit_args or list(next((o for o in region.ops if o.op_type != "linalg.yield"),
                                               Operation("x")).operands)
            region.args = [(n, None) for n in names]
        op.attributes.setdefault(
            "reduce_fn", next((o.op_type for o in region.ops if o.op_type != "linalg.yield"), "arith.addf"))
    op.regions = [region]


def _b_linalg_index(op, toks, aliases):
    nums = [t for t in toks if t.kind == "num"]
    op.attributes["dim"] = int(nums[0].text) if nums else 0
    op.result_types = _result_types(toks)


def _b_tensor_empty(op, toks, aliases):
    op.operands = _ssa(toks)
    op.result_types = _result_types(toks)
    rt = op.result_type
    op.attributes["shape"] = tuple(rt.shape)
    op.attributes["dtype"] = rt.elem


def _b_splat(op, toks, aliases):
    op.operands = _ssa(toks)
    op.result_types = _result_types(toks)
    rt = op.result_type
    if isinstance(rt, ShapedType):
        op.attributes["shape"] = tuple(rt.shape)
        op.attributes["dtype"] = rt.elem


def _b_extract(op, toks, aliases):
    op.operands = _ssa(toks)
    c = _last_top(toks, ":")
    op.operand_types = _types_after(toks, c + 1) if c >= 0 else []
    src = op.operand_types[0] if op.operand_types else None
    op.result_types = [ScalarType(src.elem)] if isinstance(src, ShapedType) else []


def _b_reshape(op, toks, aliases):
    op.operands = _ssa(toks)[:1]
    c = _last_top(toks, ":")
    into = _idx(toks, "into", kind="ident")
    if into < 0:
        into = _idx(toks, "to", kind="ident")
    if into < 0 and c >= 0:
        # tensor.reshape %src(%shape) : (T, tensor<Nxindex>) -> T'
        into = _idx(toks, "->", start=c + 1)
    op.operand_types = _types_after(toks, c + 1) if c >= 0 else []
    op.result_types = _types_after(toks, into + 1) if into >= 0 else []
    if not op.result_types:
        raise KTIRParseError(f"{op.op_type}: missing result type")
    k = _idx(toks, "[")
    if k >= 0 and k < (c if c >= 0 else len(toks)):
        inner, _ = _group(toks, k)
        op.attributes["reassociation"] = [[int(x.text) for x in g if x.kind == "num"]
                                          for g in _split_commas(inner)]
    op.attributes["target_shape"] = tuple(op.result_types[0].shape)
    if op.op_type == "tensor.reshape":
        op.operands = _ssa(toks)


def _b_slice(op, toks, aliases):
    """``tensor.extract_slice %src[offs] [sizes] [strides] : T to T`` and insert_slice."""
    ssa_head = []
    k = 0
    groups = []
    while k < len(toks):
        t = toks[k]
        if t.kind == "punct" and t.text == "[":
            inner, k = _group(toks, k)
            groups.append([p for p in _split_commas(inner)])
            continue
        if t.kind == "ssa" and not groups:
            ssa_head.append(t.text)
        if t.kind == "punct" and t.text == ":":
            break
        k += 1
    dyn = []
    statics = []
    for g in groups[:3]:
        vals = []
        for p in g:
            if p[0].kind == "ssa":
                vals.append(-(1 << 63))
                dyn.append(p[0].text)
            else:
                vals.append(int(p[0].text))
        statics.append(vals)
    c = _last_top(toks, ":")
    # the type separator after the colon (insert_slice also has the
    # `%src into %dst` before it)
    to = _idx(toks, "to", start=c + 1, kind="ident")
    into = _idx(toks, "into", start=c + 1, kind="ident")
    sep = to if to >= 0 else into
    op.operand_types = _types_after(toks, c + 1)
    op.result_types = _types_after(toks, sep + 1) if sep >= 0 else op.operand_types[-1:]
    op.operands = ssa_head + dyn
    rt = op.result_types[0]
    op.attributes.update({"static_offsets": statics[0], "static_sizes": statics[1],
                          "static_strides": statics[2], "result_shape": tuple(rt.shape),
                          "dtype": rt.elem})


def _b_from_elements(op, toks, aliases):
    op.operands = _ssa(toks)
    op.result_types = _result_types(toks)
    rt = op.result_type
    op.attributes["shape"] = tuple(rt.shape)
    op.attributes["dtype"] = rt.elem


def _b_generate(op, toks, aliases):
    op.operands = _ssa([t for t in toks if t.kind != "region"])
    op.regions = _regions(toks)
    op.result_types = _result_types(toks)
    rt = op.result_type
    op.attributes["shape"] = tuple(rt.shape)
    op.attributes["dtype"] = rt.elem


def _b_scf_for(op, toks, aliases):
    iv = toks[0].text
    assert toks[1].text == "="
    lb = toks[2].text
    to = _idx(toks, "to", kind="ident")
    st = _idx(toks, "step", kind="ident")
    ub = toks[to + 1].text
    step = toks[st + 1].text
    iter_names, inits = [], []
    k = _idx(toks, "iter_args", kind="ident")
    if k >= 0:
        inner, _ = _group(toks, k + 1)
        for part in _split_commas(inner):
            iter_names.append(part[0].text)
            inits.append(part[2].text)
    regions = _regions(toks)
    op.operands = [lb, ub, step] + inits
    op.attributes = {"iter_var": iv, "iter_args": iter_names}
    arrow = _last_top([t for t in toks if t.kind != "region"], "->")
    op.result_types = _types_after([t for t in toks if t.kind != "region"], arrow + 1) if arrow >= 0 else []
    op.regions = regions
    for r in regions:
        if not r.args:
            r.args = [(iv, ScalarType("index"))] + [(n, None) for n in iter_names]


def _b_scf_if(op, toks, aliases):
    op.operands = [toks[0].text]
    op.regions = _regions(toks)
    arrow = _last_top([t for t in toks if t.kind != "region"], "->")
    op.result_types = _types_after([t for t in toks if t.kind != "region"], arrow + 1) if arrow >= 0 else []


def _b_yield(op, toks, aliases):
    clean = _strip_attr_dicts(toks)
    c = _idx(clean, ":")
    head = clean if c < 0 else clean[:c]
    op.operands = [t.text for t in head if t.kind == "ssa"]
    op.operand_types = _types_after(clean, c + 1) if c >= 0 else []


_BUILDERS = {
    "ktdp.get_compute_tile_id": _b_tile_id,
    "ktdp.construct_memory_view": _b_memory_view,
    "ktdp.construct_distributed_memory_view": _b_dist_view,
    "ktdp.construct_access_tile": _b_access_tile,
    "ktdp.inter_tile_produce": _b_inter_tile_produce,
    "ktdp.inter_tile_reduce": _b_inter_tile_reduce,
    "ktdp.yield_partial": _b_yield_values,
    "ktdp.yield_reduced": _b_yield_values,
    "ktdp.construct_indirect_access_tile": _b_indirect_tile,
    "ktdp.load": _b_load,
    "ktdp.store": _b_load,
    "arith.constant": _b_constant,
    "linalg.index": _b_linalg_index,
    "tensor.empty": _b_tensor_empty,
    "tensor.splat": _b_splat,
    "tensor.extract": _b_extract,
    "tensor.collapse_shape": _b_reshape,
    "tensor.expand_shape": _b_reshape,
    "tensor.reshape": _b_reshape,
    "tensor.extract_slice": _b_slice,
    "tensor.insert_slice": _b_slice,
    "tensor.from_elements": _b_from_elements,
    "tensor.generate": _b_generate,
    "scf.for": _b_scf_for,
    "scf.if": _b_scf_if,
    "scf.yield": _b_yield,
    "linalg.yield": _b_yield,
    "tensor.yield": _b_yield,
    "return": _b_yield,
}
_PREFIX_BUILDERS = [("arith.", _b_simple), ("math.", _b_simple), ("linalg.", _b_linalg)]


# ---------------------------------------------------------------------------
# Module level
# ---------------------------------------------------------------------------

class KTIRParser:
    """Parse KTIR text into an :class:`IRModule` (reference ``parser.py:85-147``)."""

    def parse_file(self, path: str) -> IRModule:
        with open(path) as f:
            return self.parse_module(f.read())

    def parse_module(self, text: str) -> IRModule:
        toks = lex(text)
        module = IRModule()
        # top-level aliases: "#name = value"
        k = 0
        while k + 2 < len(toks):
            if toks[k].kind == "alias" and toks[k + 1].text == "=" and (k == 0 or toks[k - 1].kind != "punct"
                                                                        or toks[k - 1].text not in ",{("):
                module.aliases[toks[k].text] = toks[k + 2].text
                k += 3
                continue
            k += 1
        k = 0
        while k < len(toks):
            t = toks[k]
            if t.kind == "ident" and t.text == "func.func":
                fn, k = self._parse_func(toks, k + 1, module.aliases)
                module.add_function(fn)
                continue
            k += 1
        return module

    def _parse_func(self, toks: List[Tok], k: int, aliases) -> Tuple[IRFunction, int]:
        name = toks[k].text.lstrip("@")
        inner, k = _group(toks, k + 1)
        args = []
        for part in _split_commas(inner):
            if part and part[0].kind == "ssa":
                ty = parse_type(part[2].text) if len(part) > 2 else None
                args.append((part[0].text, ty))
        grid = (1, 1, 1)
        # header: optional "-> type", "attributes {...}", then body "{"
        while k < len(toks):
            t = toks[k]
            if t.kind == "punct" and t.text == "{":
                if k > 0 and toks[k - 1].kind == "ident" and toks[k - 1].text == "attributes":
                    inner_attr, k = _group(toks, k)
                    for part in _split_commas(inner_attr):
                        if part and part[0].text == "grid":
                            nums = [int(x.text) for x in part if x.kind == "num"]
                            nums = (nums + [1, 1, 1])[:3]
                            grid = tuple(nums)
                    continue
                break
            k += 1
        sp = _Splitter(toks, aliases)
        sp.i = k + 1
        body = sp.parse_region_body()
        fn = IRFunction(name, args, body.ops, grid)
        return fn, sp.i
