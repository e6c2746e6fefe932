"""Julia-subset -> C transpiler: the CPU oracle for STADE-generated derivative code.

TEST INFRASTRUCTURE ONLY.  Nothing in the product path (the `stade_hip` package, the
HIP library, the generated Julia host code) imports or calls this module.  Only the
tests, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` use it, as
the checker and as the reported CPU baseline.

What it restates.  STADE writes its tangent / adjoint / HVP code as plain Julia text
(`agen_emit` /root/reference/src/STADE.jl:3390-3419, `tgen_emit` 3271-3278, `hvp_emit`
6729-6782; committed snapshots in /root/reference/test/val-corpus/*_{b,d,hv}.jl).  Julia
is not installed here, so this module executes that text by translating it
mechanically, statement for statement, into sequential C that keeps Julia's
semantics for the subset STADE emits (the kernel language of
/root/reference/claude/skill-stade.md and the relaxed generated-code forms accepted by
`cgen_parse_generated` /root/reference/src/STADE.jl:6984-7002):

* 1-based indexing, column-major multi-dimensional arrays (`a[i, j]` ->
  `a[(i-1) + (j-1)*size(a,1)]`);
* `mod` floored (sign of the divisor), `div` truncated toward zero;
* `x ^ p` with an integer literal p is `Base.literal_pow` (p = 2 -> `x*x`, 3 -> `x*x*x`,
  -1 -> `inv(x)`, -2 -> `inv(x)*inv(x)`); other powers call `pow`;
* juxtaposition `2x` = `2 * x` binding tighter than `*` and `/` (`1/2x` = `1/(2x)`);
* Int64 / Int64 is Float64; Int64 op Float promotes to the float type;
* `max` / `min` on floats propagate NaN and order -0.0 < 0.0; `sign(0.0) = 0.0`;
* range bounds evaluated once at loop entry; an empty range runs zero trips; a `for`
  variable is local to its loop;
* `Vector{T}(undef, n)` allocates without zeroing (stacks are filled with a NaN
  pattern so a read-before-write shows up);
* `precision="f32"` mirrors `cgen_convert_precision` (/root/reference/src/STADE.jl:
  15351-15365): float literals and Float64 stacks become Float32, Int64 is untouched.

Type inference follows the four shapes of STADE's `shape_infer` (/root/reference/src/
STADE.jl:936): Float, Int, Array{Float}, Array{Int}, decided from use (index
positions, loop bounds, `div`/`mod` operands and integer literals make Int; a local assigned
only Ints, itself included, is an Int, as Julia types `c = 0; c = c + 1`).  What a file's
`initstacks_*` returns types the trailing arguments of its `_b` / `_hv` functions (arrays
with their element type, counts as Int), also where the body never reads them.
"""
from __future__ import annotations

import re
from dataclasses import dataclass, field
from typing import Any

# ----------------------------------------------------------------------------------------------
# tokens
# ----------------------------------------------------------------------------------------------

_TOKEN_RE = re.compile(
    r"""
    (?P<ws>[ \t\r]+)
  | (?P<comment>\#[^\n]*)
  | (?P<nl>\n)
  | (?P<num>0x[0-9a-fA-F]+|(?:\d+\.\d*|\.\d+|\d+)(?:[eEf][+-]?\d+)?)
  | (?P<ident>[A-Za-z_][A-Za-z_0-9!]*)
  | (?P<op>\+=|-=|\*=|/=|\^=|==|!=|<=|>=|&&|\|\||::|\.\.\.|[-+*/^<>=!(),\[\]{}:;%@.])
    """,
    re.VERBOSE,
)

KEYWORDS = {"function", "end", "for", "in", "while", "if", "elseif", "else", "return",
            "break", "continue", "local", "global", "begin"}


@dataclass
class Tok:
    kind: str  # num ident op nl kw eof
    text: str
    line: int
    juxt: bool = False  # a number immediately followed by an identifier or '(' (Julia juxtaposition)


def tokenize(src: str) -> list[Tok]:
    toks: list[Tok] = []
    pos, line, depth = 0, 1, 0
    n = len(src)
    while pos < n:
        m = _TOKEN_RE.match(src, pos)
        if not m:
            raise SyntaxError(f"line {line}: cannot tokenize {src[pos:pos + 20]!r}")
        kind = m.lastgroup
        text = m.group(kind)
        end = m.end()
        if kind == "nl":
            line += 1
            if depth == 0:
                toks.append(Tok("nl", "\n", line - 1))
        elif kind in ("ws", "comment"):
            pass
        elif kind == "num":
            j = end < n and (src[end].isalpha() or src[end] == "_" or src[end] == "(")
            toks.append(Tok("num", text, line, juxt=bool(j)))
        elif kind == "ident":
            toks.append(Tok("kw" if text in KEYWORDS else "ident", text, line))
        else:
            if text in "([{":
                depth += 1
            elif text in ")]}":
                depth -= 1
            toks.append(Tok("op", text, line))
        pos = end
    toks.append(Tok("nl", "\n", line))
    toks.append(Tok("eof", "", line))
    # a binary operator at the end of a line continues the expression on the next line
    out: list[Tok] = []
    for t in toks:
        if t.kind == "nl" and out and out[-1].kind == "op" and out[-1].text in (
                "+", "-", "*", "/", "^", "&&", "||", "==", "!=", "<", ">", "<=", ">=", "=", ","):
            continue
        out.append(t)
    return out


# ----------------------------------------------------------------------------------------------
# AST (tuples keep it small):
#   ("num", text) ("var", name) ("call", fname, [args]) ("ref", name, [idx]) ("bin", op, a, b)
#   ("un", op, a) ("tuple", [items]) ("range", lo, step|None, hi) ("alloc", T, nexpr) ("nothing",)
# statements:
#   ("assign", lhs, rhs) ("for", var, range, body) ("while", cond, body)
#   ("if", [(cond, body)...], else_body|None) ("return", expr|None) ("break",) ("continue",)
# ----------------------------------------------------------------------------------------------

@dataclass
class Func:
    name: str
    args: list[str]
    body: list
    arg_annot: dict = field(default_factory=dict)


class Parser:
    def __init__(self, toks: list[Tok]):
        self.t = toks
        self.i = 0

    # -- helpers
    def peek(self, k=0) -> Tok:
        return self.t[self.i + k]

    def next(self) -> Tok:
        tok = self.t[self.i]
        self.i += 1
        return tok

    def accept(self, kind, text=None) -> Tok | None:
        tok = self.peek()
        if tok.kind == kind and (text is None or tok.text == text):
            self.i += 1
            return tok
        return None

    def expect(self, kind, text=None) -> Tok:
        tok = self.accept(kind, text)
        if tok is None:
            p = self.peek()
            raise SyntaxError(f"line {p.line}: expected {text or kind}, got {p.text!r}")
        return tok

    def skip_nl(self):
        while self.peek().kind == "nl" or (self.peek().kind == "op" and self.peek().text == ";"):
            self.i += 1

    # -- file
    def parse_file(self) -> list[Func]:
        funcs = []
        self.skip_nl()
        while self.peek().kind != "eof":
            if self.peek().kind == "kw" and self.peek().text == "function":
                funcs.append(self.parse_function())
            else:
                # anything outside a function (a `using` line, a stray expression) is skipped to the end of line
                while self.peek().kind not in ("nl", "eof"):
                    self.i += 1
            self.skip_nl()
        return funcs

    def parse_function(self) -> Func:
        self.expect("kw", "function")
        name = self.expect("ident").text
        self.expect("op", "(")
        args, annot = [], {}
        while not self.accept("op", ")"):
            a = self.expect("ident").text
            if self.accept("op", "::"):
                annot[a] = self.parse_type_text()
            args.append(a)
            if not self.accept("op", ","):
                self.expect("op", ")")
                break
        body = self.parse_block(("end",))
        self.expect("kw", "end")
        return Func(name, args, body, annot)

    def parse_type_text(self) -> str:
        name = self.expect("ident").text
        if self.accept("op", "{"):
            inner = []
            while not self.accept("op", "}"):
                inner.append(self.next().text)
            name += "{" + "".join(inner) + "}"
        return name

    def parse_block(self, terminators) -> list:
        stmts = []
        self.skip_nl()
        while not (self.peek().kind == "kw" and self.peek().text in terminators):
            if self.peek().kind == "eof":
                raise SyntaxError("unexpected end of file inside a block")
            s = self.parse_stmt()
            if s is not None:
                stmts.append(s)
            self.skip_nl()
        return stmts

    def parse_stmt(self):
        tok = self.peek()
        if tok.kind == "op" and tok.text == "@":  # a macro prefix such as @inbounds: dropped
            self.next()
            self.expect("ident")
            if self.peek().kind == "kw" and self.peek().text == "begin":
                self.next()
                body = self.parse_block(("end",))
                self.expect("kw", "end")
                return ("block", body)
            return self.parse_stmt()
        if tok.kind == "kw":
            kw = tok.text
            if kw == "for":
                self.next()
                var = self.expect("ident").text
                if not (self.accept("op", "=") or self.accept("kw", "in")):
                    raise SyntaxError(f"line {tok.line}: bad for header")
                rng = self.parse_expr()
                if rng[0] != "range":
                    raise SyntaxError(f"line {tok.line}: for loop over a non-range")
                body = self.parse_block(("end",))
                self.expect("kw", "end")
                return ("for", var, rng, body)
            if kw == "while":
                self.next()
                cond = self.parse_expr()
                body = self.parse_block(("end",))
                self.expect("kw", "end")
                return ("while", cond, body)
            if kw == "if":
                self.next()
                arms = []
                cond = self.parse_expr()
                body = self.parse_block(("elseif", "else", "end"))
                arms.append((cond, body))
                els = None
                while True:
                    k = self.next()
                    if k.text == "elseif":
                        c = self.parse_expr()
                        b = self.parse_block(("elseif", "else", "end"))
                        arms.append((c, b))
                    elif k.text == "else":
                        els = self.parse_block(("end",))
                        self.expect("kw", "end")
                        break
                    else:
                        break
                return ("if", arms, els)
            if kw == "return":
                self.next()
                if self.peek().kind in ("nl", "eof") or (self.peek().kind == "kw" and self.peek().text == "end"):
                    return ("return", None)
                e = self.parse_expr()
                if e[0] == "nothing":
                    return ("return", None)
                return ("return", e)
            if kw == "break":
                self.next()
                return ("break",)
            if kw == "continue":
                self.next()
                return ("continue",)
            if kw in ("local", "global"):
                self.next()
                while self.peek().kind not in ("nl", "eof"):
                    self.i += 1
                return None
            if kw == "begin":
                self.next()
                body = self.parse_block(("end",))
                self.expect("kw", "end")
                return ("block", body)
            raise SyntaxError(f"line {tok.line}: unexpected keyword {kw}")
        lhs = self.parse_expr()
        op = self.peek()
        if op.kind == "op" and op.text in ("=", "+=", "-=", "*=", "/=", "^="):
            self.next()
            rhs = self.parse_expr()
            if op.text != "=":
                rhs = ("bin", op.text[0], lhs, rhs)
            if lhs[0] not in ("var", "ref"):
                raise SyntaxError(f"line {op.line}: unsupported assignment target")
            return ("assign", lhs, rhs)
        if lhs[0] == "nothing":
            return None
        return ("expr", lhs)

    # -- expressions (precedence climbing, Julia order)
    def parse_expr(self):
        return self.parse_or()

    def parse_or(self):
        a = self.parse_and()
        while self.accept("op", "||"):
            a = ("bin", "||", a, self.parse_and())
        return a

    def parse_and(self):
        a = self.parse_cmp()
        while self.accept("op", "&&"):
            a = ("bin", "&&", a, self.parse_cmp())
        return a

    def parse_cmp(self):
        a = self.parse_range()
        tok = self.peek()
        if tok.kind == "op" and tok.text in ("==", "!=", "<", ">", "<=", ">="):
            self.next()
            b = self.parse_range()
            nxt = self.peek()
            if nxt.kind == "op" and nxt.text in ("==", "!=", "<", ">", "<=", ">="):
                raise SyntaxError(f"line {tok.line}: chained comparison not supported")
            return ("bin", tok.text, a, b)
        return a

    def parse_range(self):
        a = self.parse_add()
        if self.accept("op", ":"):
            b = self.parse_add()
            if self.accept("op", ":"):
                c = self.parse_add()
                return ("range", a, b, c)
            return ("range", a, None, b)
        return a

    def parse_add(self):
        a = self.parse_mul()
        while True:
            tok = self.peek()
            if tok.kind == "op" and tok.text in ("+", "-"):
                self.next()
                a = ("bin", tok.text, a, self.parse_mul())
            else:
                return a

    def parse_mul(self):
        a = self.parse_unary()
        while True:
            tok = self.peek()
            if tok.kind == "op" and tok.text in ("*", "/", "%"):
                self.next()
                a = ("bin", tok.text, a, self.parse_unary())
            else:
                return a

    def parse_unary(self):
        tok = self.peek()
        if tok.kind == "op" and tok.text in ("-", "+", "!"):
            self.next()
            inner = self.parse_unary()
            if tok.text == "+":
                return inner
            return ("un", tok.text, inner)
        return self.parse_juxt()

    def parse_juxt(self):
        tok = self.peek()
        if tok.kind == "num" and tok.juxt:
            self.next()
            rhs = self.parse_pow()
            return ("bin", "*", ("num", tok.text), rhs)
        return self.parse_pow()

    def parse_pow(self):
        a = self.parse_postfix()
        if self.accept("op", "^"):
            if self.peek().kind == "op" and self.peek().text in ("-", "+"):
                sgn = self.next().text
                b = self.parse_pow()
                b = ("un", "-", b) if sgn == "-" else b
            else:
                b = self.parse_pow()
            return ("bin", "^", a, b)
        return a

    def parse_postfix(self):
        a = self.parse_primary()
        while True:
            if self.accept("op", "("):
                args = self.parse_args(")")
                if a[0] == "var":
                    a = ("call", a[1], args)
                elif a[0] == "typeapp":
                    if len(args) != 2 or args[0] != ("var", "undef"):
                        raise SyntaxError("only Vector{T}(undef, n) allocations are supported")
                    a = ("alloc", a[2], args[1])
                else:
                    raise SyntaxError("unsupported call target")
            elif self.peek().kind == "op" and self.peek().text == "[" and a[0] == "var":
                self.next()
                idx = self.parse_args("]")
                a = ("ref", a[1], idx)
            elif self.peek().kind == "op" and self.peek().text == "{" and a[0] == "var":
                self.next()
                inner = []
                while not self.accept("op", "}"):
                    inner.append(self.next().text)
                a = ("typeapp", a[1], "".join(inner))
            else:
                return a

    def parse_args(self, close):
        args = []
        if self.accept("op", close):
            return args
        while True:
            args.append(self.parse_expr())
            if self.accept("op", close):
                return args
            self.expect("op", ",")

    def parse_primary(self):
        tok = self.next()
        if tok.kind == "num":
            return ("num", tok.text)
        if tok.kind == "ident":
            if tok.text == "nothing":
                return ("nothing",)
            if tok.text in ("true", "false"):
                return ("num", "1" if tok.text == "true" else "0")
            return ("var", tok.text)
        if tok.kind == "op" and tok.text == "(":
            if self.accept("op", ")"):
                return ("tuple", [])
            e = self.parse_expr()
            if self.accept("op", ","):
                items = [e]
                while not self.accept("op", ")"):
                    items.append(self.parse_expr())
                    if not self.accept("op", ","):
                        self.expect("op", ")")
                        break
                return ("tuple", items)
            self.expect("op", ")")
            return e
        raise SyntaxError(f"line {tok.line}: unexpected token {tok.text!r}")


def parse(src: str) -> list[Func]:
    return Parser(tokenize(src)).parse_file()


# ----------------------------------------------------------------------------------------------
# type inference: 'i' Int64, 'f' float (Float64 or Float32), 'b' Bool; arrays are ('A', elem)
# ----------------------------------------------------------------------------------------------

FLOAT_FUNCS = {"abs", "sqrt", "exp", "log", "log10", "sin", "cos", "tan", "asin", "acos", "atan",
               "sinh", "cosh", "tanh", "floor", "ceil", "trunc", "sign", "max", "min", "mod", "div"}
INT_RESULT = {"length", "div", "mod"}


def _is_int_literal(t: str) -> bool:
    return re.fullmatch(r"\d+|0x[0-9a-fA-F]+", t) is not None


class FuncTypes:
    """Shapes of every variable of one function (Float / Int / Array{Float} / Array{Int})."""

    def __init__(self, f: Func, known_arrays: dict[str, str] | None = None,
                 arg_types: dict[str, str] | None = None):
        self.f = f
        self.arrays: dict[str, str] = {}   # name -> elem type 'f' | 'i'
        self.scalars: dict[str, str] = {}  # name -> 'f' | 'i'
        self.loopvars: set[str] = set()
        self.allocs: dict[str, str] = {}
        known_arrays = known_arrays or {}
        arg_types = arg_types or {}
        # arrays: anything indexed, or allocated
        self._walk(f.body, self._collect_arrays)
        for a, t in arg_types.items():
            if t in ("Af", "Ai"):
                self.arrays[a] = t[1]
            elif t in ("f", "i"):
                self.scalars[a] = t
        for a in list(self.arrays):
            if a in known_arrays and a not in arg_types:
                self.arrays[a] = known_arrays[a]
        for a, t in self.allocs.items():
            self.arrays[a] = t
        # annotations: x::Float64, n::Int64, a::Vector{Float64} ...
        for a, ann in f.arg_annot.items():
            if a in arg_types:
                continue
            if "Int" in ann and ("Vector" in ann or "Array" in ann):
                self.arrays[a] = "i"
            elif "Vector" in ann or "Array" in ann or "Matrix" in ann:
                self.arrays.setdefault(a, "f")
            elif "Int" in ann:
                self.scalars[a] = "i"
            elif "Float" in ann:
                self.scalars[a] = "f"
        self.fixed = set(self.scalars) | {a for a in arg_types}
        self._infer()

    # collect array names
    def _collect_arrays(self, s):
        def visit(e):
            if e[0] == "ref":
                self.arrays.setdefault(e[1], "f")
            if e[0] == "call" and e[1] == "length" and e[2] and e[2][0][0] == "var":
                self.arrays.setdefault(e[2][0][1], "f")
            for c in _children(e):
                visit(c)
        if s[0] == "assign":
            visit(s[1])
            rhs = s[2]
            if rhs[0] == "alloc":
                self.allocs[s[1][1]] = "i" if "Int" in rhs[1] else "f"
                visit(rhs[2])
            else:
                visit(rhs)
        elif s[0] == "for":
            self.loopvars.add(s[1])
            visit(s[2])
        elif s[0] in ("while",):
            visit(s[1])
        elif s[0] == "if":
            for c, _ in s[1]:
                visit(c)
        elif s[0] in ("return", "expr") and s[1] is not None:
            visit(s[1])

    def _walk(self, body, fn):
        for s in body:
            fn(s)
            if s[0] == "for":
                self._walk(s[3], fn)
            elif s[0] == "while":
                self._walk(s[2], fn)
            elif s[0] == "if":
                for _, b in s[1]:
                    self._walk(b, fn)
                if s[2] is not None:
                    self._walk(s[2], fn)
            elif s[0] == "block":
                self._walk(s[1], fn)

    def etype(self, e) -> str:
        k = e[0]
        if k == "num":
            return "i" if _is_int_literal(e[1]) else "f"
        if k == "var":
            if e[1] in self.loopvars and e[1] not in self.scalars:
                return "i"
            return self.scalars.get(e[1], "?")
        if k == "ref":
            return self.arrays.get(e[1], "f")
        if k == "un":
            if e[1] == "!":
                return "b"
            return self.etype(e[2])
        if k == "bin":
            op = e[1]
            if op in ("==", "!=", "<", ">", "<=", ">=", "&&", "||"):
                return "b"
            ta, tb = self.etype(e[2]), self.etype(e[3])
            if op == "/":
                return "f"
            if op == "^":
                return "f" if "f" in (ta, tb) else ("i" if ta == tb == "i" else "?")
            if "f" in (ta, tb):
                return "f"
            if ta == "i" and tb == "i":
                return "i"
            return "?"
        if k == "call":
            fn = e[1]
            if fn == "length":
                return "i"
            ts = [self.etype(a) for a in e[2]]
            if fn in ("div", "mod", "fld", "max", "min", "abs", "sign"):
                if "f" in ts:
                    return "f"
                if all(t == "i" for t in ts):
                    return "i"
                return "?"
            if fn in ("floor", "ceil", "trunc", "round"):
                return "f"
            return "f"
        if k == "tuple":
            return "t"
        if k == "nothing":
            return "n"
        return "?"

    def _int_context_vars(self):
        """Variables used where only an Int fits: index positions, loop bounds, allocation sizes,
        and (to a fixed point) everything an Int-context variable is computed from.  An array
        read inside such an expression is an Array{Int} (a connectivity table, a tripcount)."""
        out: set[str] = set()
        int_arrays: set[str] = set()

        def mark_int_expr(e):
            if e[0] == "var":
                out.add(e[1])
            elif e[0] == "bin" and e[1] not in ("/", "^", "==", "!=", "<", ">", "<=", ">=", "&&", "||"):
                mark_int_expr(e[2])
                mark_int_expr(e[3])
            elif e[0] == "un" and e[1] == "-":
                mark_int_expr(e[2])
            elif e[0] == "call" and e[1] in ("div", "mod", "fld", "max", "min", "abs", "sign"):
                for a in e[2]:
                    mark_int_expr(a)
            elif e[0] == "ref":
                int_arrays.add(e[1])

        def visit(e):
            if e[0] == "ref":
                for ix in e[2]:
                    mark_int_expr(ix)
            if e[0] == "call" and e[1] in ("div", "mod", "fld"):
                # a literal div/mod call is one of shape_infer's Int64 signals (skill-stade rule 11)
                for a in e[2]:
                    mark_int_expr(a)
            if e[0] == "range":
                for part in (e[1], e[2], e[3]):
                    if part is not None:
                        mark_int_expr(part)
            if e[0] == "alloc":
                mark_int_expr(e[2])
            for c in _children(e):
                visit(c)

        assigns = []

        def stmt(s):
            if s[0] == "assign":
                visit(s[1])
                visit(s[2])
                if s[1][0] == "var":
                    assigns.append((s[1][1], s[2]))
            elif s[0] == "for":
                visit(s[2])
            elif s[0] == "while":
                visit(s[1])
            elif s[0] == "if":
                for c, _ in s[1]:
                    visit(c)
            elif s[0] in ("return", "expr") and s[1] is not None:
                visit(s[1])
        self._walk(self.f.body, stmt)
        while True:
            n0 = (len(out), len(int_arrays))
            for v, rhs in assigns:
                if v in out and rhs[0] != "alloc":
                    mark_int_expr(rhs)
            if (len(out), len(int_arrays)) == n0:
                break
        for a in int_arrays:
            if a in self.arrays and a not in self.allocs and a not in self.fixed:
                self.arrays[a] = "i"
        return out

    def _infer(self):
        intctx = self._int_context_vars()
        assigns: dict[str, list] = {}
        arr_writes: dict[str, list] = {}

        def collect(s):
            if s[0] == "assign":
                if s[1][0] == "var":
                    if s[2][0] != "alloc":
                        assigns.setdefault(s[1][1], []).append(s[2])
                else:
                    arr_writes.setdefault(s[1][1], []).append(s[2])
        self._walk(self.f.body, collect)
        names = set(self.f.args) | set(assigns) | intctx
        names -= set(self.arrays)
        for nm in names:
            if nm in self.fixed or nm in self.loopvars and nm not in assigns:
                continue
            self.scalars.setdefault(nm, "i" if nm in intctx else "?")
        # fixed point over local assignments
        for _ in range(50):
            changed = False
            for nm, rhss in assigns.items():
                if nm in self.fixed or nm in self.arrays:
                    continue
                cur = self.scalars.get(nm, "?")
                # a counter (`c = 0`, then `c = c + 1`) is an Int in Julia: while its type is
                # open, its own reads count as Int (the type only widens, so this settles)
                if cur == "?":
                    self.scalars[nm] = "i"
                    ts = {self.etype(r) for r in rhss}
                    self.scalars[nm] = cur
                else:
                    ts = {self.etype(r) for r in rhss}
                if "f" in ts:
                    new = "f"
                elif ts <= {"i"}:
                    new = "i"
                elif nm in intctx:
                    new = "i"
                else:
                    new = cur
                if new != cur and not (cur == "f" and new == "i"):
                    self.scalars[nm] = new
                    changed = True
            # an argument array written with Int values is an Int array (branch / tripcount stacks)
            for arr, rhss in arr_writes.items():
                if arr in self.allocs:
                    continue
                ts = {self.etype(r) for r in rhss}
                if ts and ts <= {"i"} and self.arrays.get(arr) == "f" and arr not in self.fixed:
                    self.arrays[arr] = "i"
                    changed = True
            if not changed:
                break
        for nm, t in list(self.scalars.items()):
            if t == "?":
                self.scalars[nm] = "f"


def _children(e):
    k = e[0]
    if k in ("bin",):
        return [e[2], e[3]]
    if k == "un":
        return [e[2]]
    if k in ("call", "ref"):
        return list(e[2])
    if k == "tuple":
        return list(e[1])
    if k == "range":
        return [x for x in (e[1], e[2], e[3]) if x is not None]
    if k == "alloc":
        return [e[2]]
    return []


# ----------------------------------------------------------------------------------------------
# C code generation
# ----------------------------------------------------------------------------------------------

RUNTIME = r"""
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>
#include <stdio.h>

typedef struct { void *data; int64_t ndim; int64_t dims[4]; } jl_arr;

static inline int64_t jl_len(const jl_arr *a) {
    int64_t n = 1;
    for (int64_t k = 0; k < a->ndim; ++k) n *= a->dims[k];
    return n;
}
/* floored modulus (Julia `mod`): the result has the sign of the divisor */
static inline int64_t jl_mod(int64_t a, int64_t b) {
    int64_t r = a % b;
    if (r != 0 && ((r < 0) != (b < 0))) r += b;
    return r;
}
/* truncated division (Julia `div` on Int64) */
static inline int64_t jl_div(int64_t a, int64_t b) { return a / b; }
/* floored division (Julia `fld`) */
static inline int64_t jl_fld(int64_t a, int64_t b) { int64_t q = a / b; if ((a % b != 0) && ((a < 0) != (b < 0))) q -= 1; return q; }
static inline int64_t jl_ipow(int64_t x, int64_t p) {
    int64_t r = 1;
    while (p > 0) { if (p & 1) r *= x; x *= x; p >>= 1; }
    return r;
}
/* Julia max/min on floats: NaN propagates, -0.0 < 0.0 */
static inline double jl_fmax(double x, double y) {
    int pick_y = (y > x) || (signbit(y) < signbit(x));
    return pick_y ? (isnan(x) ? x : y) : (isnan(y) ? y : x);
}
static inline double jl_fmin(double x, double y) {
    int pick_y = (y < x) || (signbit(y) > signbit(x));
    return pick_y ? (isnan(x) ? x : y) : (isnan(y) ? y : x);
}
static inline float jl_fmaxf(float x, float y) {
    int pick_y = (y > x) || (signbit(y) < signbit(x));
    return pick_y ? (isnan(x) ? x : y) : (isnan(y) ? y : x);
}
static inline float jl_fminf(float x, float y) {
    int pick_y = (y < x) || (signbit(y) > signbit(x));
    return pick_y ? (isnan(x) ? x : y) : (isnan(y) ? y : x);
}
static inline long double jl_fmaxl(long double x, long double y) {
    int pick_y = (y > x) || (signbit(y) < signbit(x));
    return pick_y ? (isnan(x) ? x : y) : (isnan(y) ? y : x);
}
static inline long double jl_fminl(long double x, long double y) {
    int pick_y = (y < x) || (signbit(y) > signbit(x));
    return pick_y ? (isnan(x) ? x : y) : (isnan(y) ? y : x);
}
static inline long double jl_fsignl(long double x) { return x > 0.0L ? 1.0L : (x < 0.0L ? -1.0L : x); }
static inline long double jl_fmod_flooredl(long double a, long double b) {
    long double r = fmodl(a, b);
    if (r != 0.0L && ((r < 0.0L) != (b < 0.0L))) r += b;
    return r;
}
static inline int64_t jl_imax(int64_t a, int64_t b) { return a > b ? a : b; }
static inline int64_t jl_imin(int64_t a, int64_t b) { return a < b ? a : b; }
static inline int64_t jl_iabs(int64_t a) { return a < 0 ? -a : a; }
static inline int64_t jl_isign(int64_t a) { return (a > 0) - (a < 0); }
static inline double jl_fsign(double x) { return x > 0.0 ? 1.0 : (x < 0.0 ? -1.0 : x); }
static inline float jl_fsignf(float x) { return x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : x); }
static inline double jl_fmod_floored(double a, double b) {
    double r = fmod(a, b);
    if (r != 0.0 && ((r < 0.0) != (b < 0.0))) r += b;
    return r;
}
static inline float jl_fmod_flooredf(float a, float b) {
    float r = fmodf(a, b);
    if (r != 0.0f && ((r < 0.0f) != (b < 0.0f))) r += b;
    return r;
}

static int jl_bounds_error = 0;
static void jl_oob(const char *name, int64_t i, int64_t n) {
    if (!jl_bounds_error) fprintf(stderr, "BoundsError: %s[%lld] of length %lld\n", name, (long long)i, (long long)n);
    jl_bounds_error = 1;
}
static void *jl_alloc(int64_t n, size_t esz, int is_int) {
    if (n < 0) n = 0;
    void *p = malloc((size_t)(n > 0 ? n : 1) * esz);
    if (!p) { fprintf(stderr, "allocation of %lld elements failed\n", (long long)n); abort(); }
    if (n > 0 && n <= (1 << 26)) {
        if (is_int) { int64_t *q = (int64_t *)p; for (int64_t k = 0; k < n; ++k) q[k] = (int64_t)0x7ff4dead7ff4deadLL; }
        else memset(p, 0xff, (size_t)n * esz);  /* NaN pattern: a read before the first write shows up */
    }
    return p;
}
int jl_get_bounds_error(void) { int e = jl_bounds_error; jl_bounds_error = 0; return e; }
"""


class CGen:
    def __init__(self, f: Func, types: FuncTypes, precision: str, bounds_check: bool):
        self.f = f
        self.ty = types
        # f80 ("long double", 64-bit significand) runs the same text as a higher-precision truth
        self.fp = {"f32": "float", "f64": "double", "f80": "long double"}[precision]
        self.f32 = precision == "f32"
        self.lsfx = {"f32": "f", "f64": "", "f80": "L"}[precision]  # float literal suffix
        self.msfx = {"f32": "f", "f64": "", "f80": "l"}[precision]  # libm / helper suffix
        self.bc = bounds_check
        self.lines: list[str] = []
        self.ind = 1
        self.tmp = 0
        self.local_arrays: list[str] = []
        self.ret_kinds: list[str] | None = None
        self.ret_names: list = []

    # expression -> (C text, type)
    def ex(self, e) -> tuple[str, str]:
        k = e[0]
        ty = self.ty
        if k == "num":
            t = e[1]
            if _is_int_literal(t):
                return (f"((int64_t){int(t, 0)})", "i")
            if "f" in t and not t.startswith("0x"):
                # a Float32 literal (`1.0f-8`): the decimal rounded once, to Float32
                mant, ex_ = t.split("f")
                return (f"({mant}e{ex_}f)", "f")
            txt = t if ("." in t or "e" in t or "E" in t) else t + ".0"
            if txt.startswith("."):
                txt = "0" + txt
            if txt.endswith("."):
                txt += "0"
            if self.fp == "double":
                return (txt, "f")
            # a Float64 literal in another precision keeps its Float64 value and is then
            # converted, as `cgen_convert_precision`'s T(expr) converts the parsed literal
            # (/root/reference/src/STADE.jl:15353-15354): decimal -> Float64 -> Float32 rounds
            # twice, which can differ from the single rounding of a C float literal
            return (f"(({self.fp}){txt})", "f")
        if k == "var":
            t = ty.etype(e)
            if e[1] in ty.arrays:
                return (e[1], "A")
            return (e[1], t)
        if k == "ref":
            return (self.ref(e), ty.arrays.get(e[1], "f"))
        if k == "un":
            a, ta = self.ex(e[2])
            if e[1] == "!":
                return (f"(!{a})", "b")
            return (f"(-{a})", ta)
        if k == "bin":
            return self.binop(e)
        if k == "call":
            return self.call(e)
        if k == "tuple":
            raise SyntaxError("tuple outside return")
        raise SyntaxError(f"unsupported expression {e[0]}")

    def tofp(self, txt, t):
        return txt if t == "f" else f"(({self.fp}){txt})"

    def binop(self, e):
        op = e[1]
        if op in ("&&", "||"):
            a, _ = self.ex(e[2])
            b, _ = self.ex(e[3])
            return (f"({a} {op} {b})", "b")
        if op in ("==", "!=", "<", ">", "<=", ">="):
            a, ta = self.ex(e[2])
            b, tb = self.ex(e[3])
            return (f"({a} {op} {b})", "b")
        if op == "^":
            return self.power(e)
        a, ta = self.ex(e[2])
        b, tb = self.ex(e[3])
        if op == "/":
            if ta == "i" and tb == "i":
                # Julia: Int64 / Int64 is a Float64 quotient in every precision mode (the
                # reference's BigFloat rerun keeps it so too: only inputs are promoted)
                return (f"((double){a} / (double){b})", "f")
            return (f"({self.tofp(a, ta)} / {self.tofp(b, tb)})", "f")
        if op == "%":
            if ta == "i" and tb == "i":
                return (f"({a} % {b})", "i")
            return (f"fmod{self.msfx}({self.tofp(a, ta)}, {self.tofp(b, tb)})", "f")
        rt = "f" if "f" in (ta, tb) else "i"
        if rt == "f":
            a, b = self.tofp(a, ta), self.tofp(b, tb)
        return (f"({a} {op} {b})", rt)

    def power(self, e):
        base, tb = self.ex(e[2])
        pe = e[3]
        lit = None
        if pe[0] == "num" and _is_int_literal(pe[1]):
            lit = int(pe[1], 0)
        elif pe[0] == "un" and pe[1] == "-" and pe[2][0] == "num" and _is_int_literal(pe[2][1]):
            lit = -int(pe[2][1], 0)
        if tb == "i":
            p, tp = self.ex(pe)
            if tp == "i":
                return (f"jl_ipow({base}, {p})", "i")
            return (f"pow((double){base}, {p})", "f")
        if lit is not None:
            self.tmp += 1
            one = f"1.0{self.lsfx}"
            if lit == 2:
                return (f"({{{self.fp} __p = {base}; __p * __p;}})", "f")
            if lit == 3:
                return (f"({{{self.fp} __p = {base}; __p * __p * __p;}})", "f")
            if lit == 1:
                return (f"({base})", "f")
            if lit == 0:
                return (one, "f")
            if lit == -1:
                return (f"({one} / ({base}))", "f")
            if lit == -2:
                return (f"({{{self.fp} __p = {one} / ({base}); __p * __p;}})", "f")
        p, tp = self.ex(pe)
        fn = "pow" + self.msfx
        return (f"{fn}({base}, {self.tofp(p, tp)})", "f")

    def call(self, e):
        fn, args = e[1], e[2]
        if fn == "length":
            a = args[0]
            if a[0] != "var" or a[1] not in self.ty.arrays:
                raise SyntaxError("length of a non-array")
            return (f"jl_len(&{a[1]})", "i")
        cs = [self.ex(a) for a in args]
        ts = [t for _, t in cs]
        txt = [c for c, _ in cs]
        allint = all(t == "i" for t in ts)
        sfx = self.msfx
        if fn in ("div", "mod", "fld"):
            if allint:
                return (f"jl_{fn}({txt[0]}, {txt[1]})", "i")
            if fn == "fld":
                return (f"floor{sfx}({self.tofp(txt[0], ts[0])} / {self.tofp(txt[1], ts[1])})", "f")
            a0, a1 = self.tofp(txt[0], ts[0]), self.tofp(txt[1], ts[1])
            if fn == "div":
                return (f"trunc{sfx}({a0} / {a1})", "f")
            return (f"jl_fmod_floored{sfx}({a0}, {a1})", "f")
        if fn in ("max", "min"):
            if allint:
                return (f"jl_i{fn}({txt[0]}, {txt[1]})", "i")
            a0, a1 = self.tofp(txt[0], ts[0]), self.tofp(txt[1], ts[1])
            return (f"jl_f{fn}{sfx}({a0}, {a1})", "f")
        if fn == "abs":
            if allint:
                return (f"jl_iabs({txt[0]})", "i")
            return (f"fabs{sfx}({txt[0]})", "f")
        if fn == "sign":
            if allint:
                return (f"jl_isign({txt[0]})", "i")
            return (f"jl_fsign{sfx}({txt[0]})", "f")
        math1 = {"sqrt", "exp", "log", "log10", "sin", "cos", "tan", "asin", "acos", "atan",
                 "sinh", "cosh", "tanh", "floor", "ceil", "trunc"}
        if fn in math1:
            if len(args) != 1:
                raise SyntaxError(f"{fn} takes one argument")
            if ts[0] == "i" and self.fp == "long double":
                # Julia: sqrt(::Int64), exp(::Int64), ... return Float64; the reference's
                # BigFloat rerun promotes inputs only, so that value stays a Float64
                return (f"((long double){fn}((double){txt[0]}))", "f")
            return (f"{fn}{sfx}({self.tofp(txt[0], ts[0])})", "f")
        raise SyntaxError(f"call to unsupported function {fn}")

    def ref(self, e) -> str:
        name, idx = e[1], e[2]
        if name not in self.ty.arrays:
            raise SyntaxError(f"indexing non-array {name}")
        parts = []
        for ix in idx:
            c, t = self.ex(ix)
            if t != "i":
                raise SyntaxError(f"non-integer index into {name}")
            parts.append(c)
        if len(parts) == 1:
            lin = f"({parts[0]} - 1)"
        else:
            lin = f"({parts[0]} - 1)"
            stride = f"{name}.dims[0]"
            for k, p in enumerate(parts[1:], start=1):
                lin = f"({lin} + ({p} - 1) * {stride})"
                stride = f"{stride} * {name}.dims[{k}]"
        ct = "int64_t" if self.ty.arrays[name] == "i" else self.fp
        if self.bc:
            return f"(*({{int64_t __k = {lin}; if (__k < 0 || __k >= jl_len(&{name})) jl_oob(\"{name}\", __k + 1, jl_len(&{name})); (__k < 0 || __k >= jl_len(&{name})) ? &(({ct} *){name}.data)[0] : &(({ct} *){name}.data)[__k];}}))"
        return f"(({ct} *){name}.data)[{lin}]"

    def emit(self, s: str):
        self.lines.append("    " * self.ind + s)

    def stmts(self, body):
        for s in body:
            self.stmt(s)

    def stmt(self, s):
        k = s[0]
        if k == "assign":
            lhs, rhs = s[1], s[2]
            if rhs[0] == "alloc":
                nm = lhs[1]
                n, _ = self.ex(rhs[2])
                isint = "Int" in rhs[1]
                ct = "int64_t" if isint else ("float" if (self.f32 or "Float32" in rhs[1]) else self.fp)
                self.emit(f"if ({nm}.data) free({nm}.data);")
                self.emit(f"{nm}.ndim = 1; {nm}.dims[0] = {n} > 0 ? {n} : 0; {nm}.data = jl_alloc({nm}.dims[0], sizeof({ct}), {1 if isint else 0});")
                return
            if lhs[0] == "var" and lhs[1] in self.ty.arrays:
                if rhs[0] == "var" and rhs[1] in self.ty.arrays:
                    self.emit(f"{lhs[1]} = {rhs[1]};")
                    return
                raise SyntaxError(f"array binding {lhs[1]} from an expression")
            r, tr = self.ex(rhs)
            if lhs[0] == "var":
                tl = self.ty.scalars.get(lhs[1], "f")
                if tl == "i" and tr == "f":
                    raise SyntaxError(f"Float assigned to Int variable {lhs[1]}")
                self.emit(f"{lhs[1]} = {r};")
            else:
                l = self.ref(lhs)
                self.emit(f"{l} = {r};")
        elif k == "for":
            var, rng, body = s[1], s[2], s[3]
            lo, _ = self.ex(rng[1])
            hi, _ = self.ex(rng[3])
            self.tmp += 1
            t = self.tmp
            if rng[2] is None:
                self.emit(f"{{ int64_t __lo{t} = {lo}, __hi{t} = {hi};")
                self.emit(f"for (int64_t {var} = __lo{t}; {var} <= __hi{t}; ++{var}) {{")
            else:
                st, _ = self.ex(rng[2])
                self.emit(f"{{ int64_t __lo{t} = {lo}, __st{t} = {st}, __hi{t} = {hi};")
                self.emit(f"for (int64_t {var} = __lo{t}; __st{t} > 0 ? {var} <= __hi{t} : {var} >= __hi{t}; {var} += __st{t}) {{")
            self.ind += 1
            self.stmts(body)
            self.ind -= 1
            self.emit("} }")
        elif k == "while":
            c, _ = self.ex(s[1])
            self.emit(f"while ({c}) {{")
            self.ind += 1
            self.stmts(s[2])
            self.ind -= 1
            self.emit("}")
        elif k == "if":
            for j, (cond, body) in enumerate(s[1]):
                c, _ = self.ex(cond)
                self.emit(("if" if j == 0 else "} else if") + f" ({c}) {{")
                self.ind += 1
                self.stmts(body)
                self.ind -= 1
            if s[2] is not None:
                self.emit("} else {")
                self.ind += 1
                self.stmts(s[2])
                self.ind -= 1
            self.emit("}")
        elif k == "block":
            self.stmts(s[1])
        elif k == "return":
            self.ret(s[1])
        elif k == "break":
            self.emit("break;")
        elif k == "continue":
            self.emit("continue;")
        elif k == "expr":
            c, _ = self.ex(s[1])
            self.emit(f"(void){c};")
        else:
            raise SyntaxError(f"unsupported statement {k}")

    def ret(self, e):
        items = [] if e is None else (e[1] if e[0] == "tuple" else [e])
        kinds = []
        for j, it in enumerate(items):
            if it[0] == "var" and it[1] in self.ty.arrays:
                # an array returned by initstacks: its length and element type go back, the buffer is freed
                kinds.append("A" + self.ty.arrays[it[1]])
                self.emit(f"((long double *)__ret)[{j}] = (long double)jl_len(&{it[1]});")
            else:
                c, t = self.ex(it)
                kinds.append(t)
                self.emit(f"((long double *)__ret)[{j}] = (long double){c};")
        if self.ret_kinds is None:
            self.ret_kinds = kinds
            self.ret_names = [it[1] if it[0] == "var" else None for it in items]
        self.emit("goto __done;")

    def generate(self) -> str:
        f, ty = self.f, self.ty
        head = f"int64_t {f.name}(void **__argv, void *__ret)"
        self.lines.append(head + " {")
        self.emit("int64_t __nret = 0; (void)__nret;")
        # arguments
        for j, a in enumerate(f.args):
            if a in ty.arrays:
                self.emit(f"jl_arr {a} = *(jl_arr *)__argv[{j}];")
            else:
                t = ty.scalars.get(a, "f")
                ct = "int64_t" if t == "i" else self.fp
                self.emit(f"{ct} {a} = *({ct} *)__argv[{j}];")
        # locals
        for nm, t in sorted(ty.scalars.items()):
            if nm in f.args:
                continue
            ct = "int64_t" if t == "i" else self.fp
            self.emit(f"{ct} {nm} = 0; (void){nm};")
        for nm in sorted(ty.arrays):
            if nm in f.args:
                continue
            self.emit(f"jl_arr {nm}; memset(&{nm}, 0, sizeof({nm}));")
            self.local_arrays.append(nm)
        self.stmts(f.body)
        nret = len(self.ret_kinds) if self.ret_kinds is not None else 0
        self.emit("__done:;")
        for nm in self.local_arrays:
            self.emit(f"if ({nm}.data) free({nm}.data);")
        self.emit(f"return {nret};")
        self.lines.append("}")
        return "\n".join(self.lines)


@dataclass
class FuncInfo:
    name: str
    args: list[tuple[str, str]]  # (name, 'f'|'i'|'Af'|'Ai')
    ret: list[str]
    ret_names: list = field(default_factory=list)


def transpile(src: str, precision: str = "f64", bounds_check: bool = False,
              arg_types: dict[str, dict[str, str]] | None = None) -> tuple[str, dict[str, FuncInfo]]:
    """Translate every function of a generated `.jl` text into C.

    Returns the C source (one `int64_t NAME(void **argv, void *ret)` per Julia function,
    in file order; a duplicate name, such as the primal repeated after the adjoint, is
    emitted once) and a table of argument shapes and returned scalars for the ctypes
    runner.  `arg_types` optionally pins argument shapes per function.
    """
    funcs = parse(src)
    arg_types = arg_types or {}
    # stacks allocated by initstacks_* keep their element type when they are arguments of *_b / *_hv
    known: dict[str, str] = {}
    # everything initstacks_* returns is a trailing argument of *_b / *_hv: arrays with their
    # element type, and Int64 counts (`__tot_*`, `__len_*`), typed so even where unread
    init_ret: dict[str, str] = {}
    for f in funcs:
        if f.name.startswith("initstacks_"):
            ft = FuncTypes(f)
            for a, t in ft.allocs.items():
                known[a] = t
            for st in f.body:
                if st[0] == "return" and st[1] is not None:
                    items = st[1][1] if st[1][0] == "tuple" else [st[1]]
                    for it in items:
                        if it[0] != "var":
                            continue
                        nm = it[1]
                        if nm in ft.arrays:
                            init_ret[nm] = "A" + ft.arrays[nm]
                        else:
                            init_ret[nm] = ft.scalars.get(nm, "i")
    # a shadow argument (`xd`, `xb`, `xbd`) has the shape of its primal even where the derivative
    # code never touches it (a dead tangent): first pass collects every array name in the file
    arrays_by_name: dict[str, str] = dict(known)
    for f in funcs:
        ft = FuncTypes(f, known_arrays=known, arg_types=arg_types.get(f.name))
        for a, t in ft.arrays.items():
            arrays_by_name.setdefault(a, t)
    seen = set()
    chunks = [RUNTIME]
    infos: dict[str, FuncInfo] = {}
    for f in funcs:
        if f.name in seen:
            continue
        seen.add(f.name)
        hints = dict(arg_types.get(f.name) or {})
        if not f.name.startswith("initstacks_"):
            for a in f.args:
                if a in init_ret and a not in hints:
                    hints[a] = init_ret[a]
        probe = FuncTypes(f, known_arrays=known, arg_types=hints)
        for a in f.args:
            if a in probe.arrays or a in hints:
                continue
            for suf in ("bd", "d", "b"):
                base = a[: -len(suf)]
                if a.endswith(suf) and base in arrays_by_name and base in f.args:
                    hints[a] = "A" + arrays_by_name[base]
                    break
        ft = FuncTypes(f, known_arrays=known, arg_types=hints) if hints else probe
        g = CGen(f, ft, precision, bounds_check)
        chunks.append(g.generate())
        args = []
        for a in f.args:
            if a in ft.arrays:
                args.append((a, "A" + ft.arrays[a]))
            else:
                args.append((a, ft.scalars.get(a, "f")))
        infos[f.name] = FuncInfo(f.name, args, g.ret_kinds or [], g.ret_names)
    return "\n\n".join(chunks) + "\n", infos
