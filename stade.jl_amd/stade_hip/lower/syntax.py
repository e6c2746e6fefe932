"""Front end of the general lowering: the Julia subset that STADE's generators write, parsed
into a small AST.

The subset is the generated derivative code of `stade_adjoint_file`, `stade_tangent_file`
and `stade_hvp_file` (`agen_emit` /root/reference/src/STADE.jl:3390-3419, `tgen_emit`
3271-3278, `hvp_emit` 6729-6782) and the kernel language they read
(/root/reference/claude/skill-stade.md; the generated-code forms accepted by
`cgen_parse_generated` /root/reference/src/STADE.jl:6984-7002): `function ... end` with
positional arguments, `for v = lo:hi` / `lo:step:hi`, `while`, `if / elseif / else`,
assignments (`=`, `+=`, `-=`, `*=`, `/=`), 1-based indexing `a[i]`, `a[i, j]`, calls,
`return`, `break`, `continue`, `Vector{T}(undef, n)` allocations, Julia's operator
precedence including juxtaposition (`2x` is `2 * x` binding tighter than `*`; `1/2x` is
`1/(2x)`) and right-associative `^`.
"""
from __future__ import annotations

import re
from dataclasses import dataclass, field


class LowerError(ValueError):
    """Generated text the lowering cannot take, with the cause."""


# ------------------------------------------------------------------------------------------
# AST
# ------------------------------------------------------------------------------------------

@dataclass(frozen=True)
class Num:
    text: str
    is_int: bool
    f32: bool = False          # a Float32 literal (`1.0f0`)


@dataclass(frozen=True)
class Var:
    name: str


@dataclass(frozen=True)
class Call:
    fn: str
    args: tuple


@dataclass(frozen=True)
class Ref:
    name: str
    idx: tuple


@dataclass(frozen=True)
class Bin:
    op: str
    a: object
    b: object


@dataclass(frozen=True)
class Un:
    op: str
    a: object


@dataclass(frozen=True)
class Range:
    lo: object
    step: object               # None: 1
    hi: object


@dataclass(frozen=True)
class Alloc:
    eltype: str                # "Float64" | "Float32" | "Int64"
    n: object


@dataclass(frozen=True)
class Tup:
    items: tuple


@dataclass(frozen=True)
class Nothing_:
    pass


@dataclass
class Assign:
    lhs: object                # Var | Ref
    rhs: object


@dataclass
class For:
    var: str
    rng: Range
    body: list


@dataclass
class While:
    cond: object
    body: list


@dataclass
class If:
    branches: list             # [(cond, body)]
    orelse: list | None


@dataclass
class Return:
    value: object | None


@dataclass
class Break:
    pass


@dataclass
class Continue:
    pass


@dataclass
class ExprStmt:
    e: object


@dataclass
class GemmSeg:
    """One product of a Gemm: A(m, k) = a[a_off + (k + m * lda if a_km else m + k * lda)],
    B(k, n) = b[b_off + (k + n * ldb if b_km else n + k * ldb)], k < K (0-based offsets;
    every expression an Int expression of the function's Int arguments)."""
    a: str
    a_off: object
    a_km: bool
    lda: object
    b: str
    b_off: object
    b_km: bool
    ldb: object
    K: object


@dataclass
class Gemm:
    """A statement the general lowering makes of a contraction (contract.py), not Julia text:
    out[out_off + m * out_sm + n * out_sn] (+)= sum over segments of sum_k A(m, k) B(k, n) for
    m < M, n < N (`acc`: added to the element, else stored)."""
    out: str
    out_off: object
    out_sm: object
    out_sn: object
    acc: bool
    M: object
    N: object
    segs: list


@dataclass
class TabDim:
    """An offset along one dimension of a GemmT operand: table[i] (a local Int64 array of
    0-based element offsets) or, with no table, i * stride."""
    table: str | None
    stride: object


@dataclass
class GemmT:
    """A table-addressed product the general lowering makes of a contraction whose factors are
    gathers (contract.py), not Julia text:
    out[out_off + ro(m) + co(n)] (+)= sum_{k < K} a[a_off + ar(m) + ak(k)] * b[b_off + bk(k) + bc(n)]
    for m < M, n < N (0-based); mode 0 stores, 1 adds, 2 adds atomically (elements that
    several (m, n) share)."""
    out: str
    out_off: object
    ro: TabDim
    co: TabDim
    mode: int
    M: object
    N: object
    K: object
    a: str
    a_off: object
    ar: TabDim
    ak: TabDim
    b: str
    b_off: object
    bk: TabDim
    bc: TabDim
    a_km: bool = False         # a's k are adjacent in memory (else its rows): how to gather it
    b_km: bool = False         # b's k are adjacent (else its columns)


@dataclass
class Func:
    name: str
    args: list
    body: list
    annot: dict = field(default_factory=dict)


# ------------------------------------------------------------------------------------------
# tokens
# ------------------------------------------------------------------------------------------

_TOK = re.compile(
    r"""(?P<ws>[ \t\r]+)|(?P<comment>\#[^\n]*)|(?P<nl>\n)
      |(?P<num>(?:\d+\.\d*|\.\d+|\d+)(?:[eEf][+-]?\d+)?)
      |(?P<id>[A-Za-z_][A-Za-z_0-9!]*)
      |(?P<op>\+=|-=|\*=|/=|==|!=|<=|>=|&&|\|\||::|[-+*/^<>=!(),\[\]{}:;.])""",
    re.X,
)
_KW = {"function", "end", "for", "in", "while", "if", "elseif", "else", "return", "break", "continue", "local",
       "global", "begin"}
_CONT = {"+", "-", "*", "/", "^", "&&", "||", "==", "!=", "<", ">", "<=", ">=", "=", ",", "+=", "-=", "*=", "/="}


@dataclass
class Tok:
    kind: str                  # num id kw op nl eof
    text: str
    line: int
    juxt: bool = False         # a number directly followed by an identifier or '('


def tokenize(src: str) -> list[Tok]:
    out: list[Tok] = []
    pos, line, depth = 0, 1, 0
    while pos < len(src):
        m = _TOK.match(src, pos)
        if not m:
            raise LowerError(f"line {line}: cannot read {src[pos:pos + 16]!r}")
        k, t, pos = m.lastgroup, m.group(m.lastgroup), m.end()
        if k == "nl":
            if depth == 0 and not (out and out[-1].kind == "op" and out[-1].text in _CONT):
                out.append(Tok("nl", "\n", line))
            line += 1
        elif k in ("ws", "comment"):
            continue
        elif k == "num":
            nxt = src[pos] if pos < len(src) else ""
            out.append(Tok("num", t, line, juxt=nxt.isalpha() or nxt in "_("))
        elif k == "id":
            out.append(Tok("kw" if t in _KW else "id", t, line))
        else:
            depth += t in "([{"
            depth -= t in ")]}"
            out.append(Tok("op", t, line))
    out.append(Tok("nl", "\n", line))
    out.append(Tok("eof", "", line))
    return out


# ------------------------------------------------------------------------------------------
# parser
# ------------------------------------------------------------------------------------------

class _P:
    def __init__(self, toks):
        self.t, self.i = toks, 0

    def peek(self, k=0):
        return self.t[min(self.i + k, len(self.t) - 1)]

    def take(self):
        tok = self.t[self.i]
        self.i += 1
        return tok

    def at(self, kind, text=None):
        tok = self.peek()
        return tok.kind == kind and (text is None or tok.text == text)

    def accept(self, kind, text=None):
        if self.at(kind, text):
            return self.take()
        return None

    def expect(self, kind, text=None):
        tok = self.take()
        if tok.kind != kind or (text is not None and tok.text != text):
            raise LowerError(f"line {tok.line}: expected {text or kind}, found {tok.text!r}")
        return tok

    def skip_nl(self):
        while self.at("nl") or self.at("op", ";"):
            self.take()

    # -- file and functions
    def file(self) -> list[Func]:
        fs = []
        self.skip_nl()
        while not self.at("eof"):
            if self.at("kw", "function"):
                fs.append(self.function())
            else:
                raise LowerError(f"line {self.peek().line}: only function definitions may appear at top level")
            self.skip_nl()
        return fs

    def function(self) -> Func:
        self.expect("kw", "function")
        name = self.expect("id").text
        self.expect("op", "(")
        args, annot = [], {}
        while not self.at("op", ")"):
            a = self.expect("id").text
            if self.accept("op", "::"):
                annot[a] = self.type_text()
            args.append(a)
            if not self.accept("op", ","):
                break
        self.expect("op", ")")
        body = self.block({"end"})
        self.expect("kw", "end")
        return Func(name, args, body, annot)

    def type_text(self) -> str:
        s = self.expect("id").text
        if self.accept("op", "{"):
            inner = []
            while not self.at("op", "}"):
                inner.append(self.take().text)
            self.expect("op", "}")
            s += "{" + "".join(inner) + "}"
        return s

    def block(self, ends) -> list:
        out = []
        self.skip_nl()
        while not (self.at("kw") and self.peek().text in ends):
            if self.at("eof"):
                raise LowerError("unexpected end of text inside a block")
            st = self.stmt()
            if st is not None:
                out.append(st)
            self.skip_nl()
        return out

    def stmt(self):
        tok = self.peek()
        if tok.kind == "kw":
            k = tok.text
            if k == "for":
                self.take()
                var = self.expect("id").text
                if not (self.accept("op", "=") or self.accept("kw", "in")):
                    raise LowerError(f"line {tok.line}: expected = or in after the loop variable")
                rng = self.expr()
                if not isinstance(rng, Range):
                    raise LowerError(f"line {tok.line}: a for loop must run over a range lo:hi or lo:step:hi")
                body = self.block({"end"})
                self.expect("kw", "end")
                return For(var, rng, body)
            if k == "while":
                self.take()
                cond = self.expr()
                body = self.block({"end"})
                self.expect("kw", "end")
                return While(cond, body)
            if k == "if":
                self.take()
                branches = [(self.expr(), None)]
                orelse = None
                body = self.block({"elseif", "else", "end"})
                branches[0] = (branches[0][0], body)
                while self.accept("kw", "elseif"):
                    c = self.expr()
                    branches.append((c, self.block({"elseif", "else", "end"})))
                if self.accept("kw", "else"):
                    orelse = self.block({"end"})
                self.expect("kw", "end")
                return If(branches, orelse)
            if k == "begin":
                self.take()
                body = self.block({"end"})
                self.expect("kw", "end")
                return If([(Num("true", False), body)], None) if body else None
            if k == "return":
                self.take()
                if self.at("nl") or self.at("kw", "end") or self.at("op", ";"):
                    return Return(None)
                e = self.expr()
                if self.at("op", ","):
                    items = [e]
                    while self.accept("op", ","):
                        items.append(self.expr())
                    e = Tup(tuple(items))
                return Return(e)
            if k == "break":
                self.take()
                return Break()
            if k == "continue":
                self.take()
                return Continue()
            if k in ("local", "global"):
                self.take()
                return self.stmt()
            raise LowerError(f"line {tok.line}: unexpected {k!r}")
        lhs = self.expr()
        if self.at("op") and self.peek().text in ("=", "+=", "-=", "*=", "/="):
            op = self.take().text
            rhs = self.expr()
            if not isinstance(lhs, (Var, Ref)):
                raise LowerError(f"line {tok.line}: cannot assign to this expression")
            if op != "=":
                rhs = Bin(op[0], lhs, rhs)
            return Assign(lhs, rhs)
        return ExprStmt(lhs)

    # -- expressions (Julia precedence, lowest first)
    def expr(self):
        e = self.orx()
        if self.at("op", ":"):
            self.take()
            b = self.orx()
            if self.accept("op", ":"):
                c = self.orx()
                return Range(e, b, c)
            return Range(e, None, b)
        return e

    def orx(self):
        e = self.andx()
        while self.accept("op", "||"):
            e = Bin("||", e, self.andx())
        return e

    def andx(self):
        e = self.cmp()
        while self.accept("op", "&&"):
            e = Bin("&&", e, self.cmp())
        return e

    def cmp(self):
        e = self.add()
        while self.at("op") and self.peek().text in ("==", "!=", "<", ">", "<=", ">="):
            op = self.take().text
            e = Bin(op, e, self.add())
        return e

    def add(self):
        e = self.mul()
        while self.at("op") and self.peek().text in ("+", "-"):
            op = self.take().text
            e = Bin(op, e, self.mul())
        return e

    def mul(self):
        e = self.unary()
        while self.at("op") and self.peek().text in ("*", "/"):
            op = self.take().text
            e = Bin(op, e, self.unary())
        return e

    def unary(self):
        if self.at("op") and self.peek().text in ("-", "+", "!"):
            op = self.take().text
            a = self.unary()
            if op == "+":
                return a
            if op == "-" and isinstance(a, Num):
                return Num("-" + a.text, a.is_int, a.f32)
            return Un(op, a)
        return self.juxt()

    def juxt(self):
        tok = self.peek()
        if tok.kind == "num" and tok.juxt:
            n = self.atom_num(self.take())
            return Bin("*", n, self.power())
        return self.power()

    def power(self):
        base = self.postfix()
        if self.accept("op", "^"):
            # right associative; a unary minus binds to the exponent (`x^-2`)
            if self.at("op") and self.peek().text in ("-", "+"):
                op = self.take().text
                ex = self.power()
                ex = ex if op == "+" else (Num("-" + ex.text, ex.is_int, ex.f32) if isinstance(ex, Num) else Un("-", ex))
            else:
                ex = self.power()
            return Bin("^", base, ex)
        return base

    def postfix(self):
        e = self.primary()
        while True:
            if self.at("op", "["):
                self.take()
                idx = self.args("]")
                if not isinstance(e, Var):
                    raise LowerError(f"line {self.peek().line}: only named arrays may be indexed")
                e = Ref(e.name, tuple(idx))
            elif self.at("op", "(") and isinstance(e, (Var, Alloc)):
                self.take()
                args = self.args(")")
                if isinstance(e, Alloc):
                    if len(args) != 2 or not (isinstance(args[0], Var) and args[0].name == "undef"):
                        raise LowerError("only Vector{T}(undef, n) allocations are supported")
                    e = Alloc(e.eltype, args[1])
                else:
                    e = Call(e.name, tuple(args))
            else:
                return e

    def args(self, close):
        out = []
        while not self.at("op", close):
            out.append(self.expr())
            if not self.accept("op", ","):
                break
        self.expect("op", close)
        return out

    def atom_num(self, tok):
        t = tok.text
        if "f" in t:
            return Num(t.replace("f", "e"), False, True)
        is_int = not any(c in t for c in ".eE")
        return Num(t, is_int)

    def primary(self):
        tok = self.take()
        if tok.kind == "num":
            return self.atom_num(tok)
        if tok.kind == "id":
            if tok.text in ("true", "false"):
                return Num(tok.text, False)
            if tok.text == "nothing":
                return Nothing_()
            if tok.text in ("Vector", "Array") and self.at("op", "{"):
                self.take()
                et = self.expect("id").text
                while not self.at("op", "}"):
                    self.take()
                self.expect("op", "}")
                if et not in ("Float64", "Float32", "Int64", "Int"):
                    raise LowerError(f"line {tok.line}: arrays of {et} are not supported")
                return Alloc("Int64" if et == "Int" else et, None)
            return Var(tok.text)
        if tok.kind == "op" and tok.text == "(":
            if self.accept("op", ")"):
                return Tup(())
            e = self.expr()
            if self.at("op", ","):
                items = [e]
                while self.accept("op", ","):
                    if self.at("op", ")"):
                        break
                    items.append(self.expr())
                self.expect("op", ")")
                return Tup(tuple(items))
            self.expect("op", ")")
            return e
        raise LowerError(f"line {tok.line}: unexpected {tok.text!r}")


def parse(src: str) -> list[Func]:
    return _P(tokenize(src)).file()


# ------------------------------------------------------------------------------------------
# walking
# ------------------------------------------------------------------------------------------

def children(e):
    if isinstance(e, (Call,)):
        return e.args
    if isinstance(e, Ref):
        return e.idx
    if isinstance(e, Bin):
        return (e.a, e.b)
    if isinstance(e, Un):
        return (e.a,)
    if isinstance(e, Range):
        return tuple(x for x in (e.lo, e.step, e.hi) if x is not None)
    if isinstance(e, Alloc):
        return (e.n,) if e.n is not None else ()
    if isinstance(e, Tup):
        return e.items
    return ()


def walk_expr(e):
    yield e
    for c in children(e):
        yield from walk_expr(c)


def stmt_exprs(s):
    """The expressions a statement evaluates itself (not those of nested statements)."""
    if isinstance(s, Assign):
        return [s.rhs] + (list(s.lhs.idx) if isinstance(s.lhs, Ref) else [])
    if isinstance(s, For):
        return [s.rng]
    if isinstance(s, While):
        return [s.cond]
    if isinstance(s, If):
        return [c for c, _ in s.branches]
    if isinstance(s, Return):
        return [s.value] if s.value is not None else []
    if isinstance(s, ExprStmt):
        return [s.e]
    if isinstance(s, GemmT):
        return [s.out_off, s.M, s.N, s.K, s.a_off, s.b_off] + [d.stride for d in (s.ro, s.co, s.ar, s.ak, s.bk, s.bc)
                                                                if d.table is None]
    if isinstance(s, Gemm):
        out = [s.out_off, s.out_sm, s.out_sn, s.M, s.N]
        for g in s.segs:
            out += [g.a_off, g.lda, g.b_off, g.ldb, g.K]
        return out
    return []


def sub_blocks(s):
    if isinstance(s, (For, While)):
        return [s.body]
    if isinstance(s, If):
        return [b for _, b in s.branches] + ([s.orelse] if s.orelse is not None else [])
    return []


def walk_stmts(body):
    for s in body:
        yield s
        for b in sub_blocks(s):
            yield from walk_stmts(b)
