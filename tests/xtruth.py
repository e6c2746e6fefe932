"""A second executor of STADE-generated Julia text, in decimal arithmetic with 50 significant
digits: the known answer that the oracle's 80-bit truth mode is checked against.

TEST INFRASTRUCTURE ONLY.  Nothing in the product path uses it.

It is independent of the oracle.  It parses the text with the lowering's front end
(`stade_hip.lower.syntax`), not with `oracle/jl2c.py`, and it evaluates the syntax tree
directly in Python.  No C compiler, no long double and no ctypes marshalling are involved.
Each arithmetic operation rounds to 50 digits, about 1e-50 relative, so its results are
exact to far below the 1e-19 of the 80-bit format.

The reference's own truth is the same generated code rerun on BigFloat copies of the inputs
(`val_gpu_parity_script` /root/reference/src/STADE.jl:19045-19113): the inputs are promoted
exactly, and the text's Float64 constants keep their Float64 values (`BigFloat * 0.1` promotes
the Float64 0.1 exactly; `Int / Int` is a Float64 quotient).  This executor follows those rules:

* float literals are their Float64 values, promoted exactly (`0.1` is 0.1000000000000000055...);
* `Int / Int` is rounded once to Float64, as Julia's `/` on two Int64 does, then promoted;
* inputs are the callers' numpy values, promoted exactly;
* everything else is Julia's semantics for the subset STADE writes: 1-based column-major
  arrays, floored `mod`, truncated `div`, `x ^ p` with a literal integer `p` as repeated
  multiplication (`Base.literal_pow`), `sign(0) = 0`, a `for` variable local to its loop,
  range bounds evaluated once, `Vector{T}(undef, n)` unset until written (reading an unset
  element raises).

Entry point: `run(text, fname, args) -> (arrays, returned)`, where `args` are numpy arrays
(float or Int64) and Python scalars in the function's order.  Float arrays come back as lists
of `Decimal` in column-major order, Int64 arrays as lists of `int`.
"""
from __future__ import annotations

import decimal
from decimal import Decimal
from fractions import Fraction

import numpy as np

from stade_hip.lower import syntax as S

CTX = decimal.Context(prec=50, rounding=decimal.ROUND_HALF_EVEN, Emax=10**6, Emin=-10**6,
                      traps=[decimal.InvalidOperation, decimal.DivisionByZero, decimal.Overflow])


class JArr:
    __slots__ = ("data", "dims", "isint")

    def __init__(self, data, dims, isint):
        self.data, self.dims, self.isint = data, tuple(dims), isint


class _Break(Exception):
    pass


class _Continue(Exception):
    pass


class _Return(Exception):
    def __init__(self, value):
        self.value = value


def dec(x) -> Decimal:
    """Exact promotion of a binary float, an int or a numpy scalar (long double included)."""
    if isinstance(x, Decimal):
        return x
    if isinstance(x, (bool, np.bool_)):
        raise TypeError("a Bool used as a number")
    if isinstance(x, (int, np.integer)):
        return Decimal(int(x))
    if isinstance(x, np.longdouble) and np.finfo(np.longdouble).nmant > 52:
        fr = Fraction(*x.as_integer_ratio())
        return CTX.divide(Decimal(fr.numerator), Decimal(fr.denominator))
    return Decimal(float(x))


def _isf(v):
    return isinstance(v, Decimal)


def _add(a, b):
    return a + b if not (_isf(a) or _isf(b)) else CTX.add(dec(a), dec(b))


def _sub(a, b):
    return a - b if not (_isf(a) or _isf(b)) else CTX.subtract(dec(a), dec(b))


def _mul(a, b):
    return a * b if not (_isf(a) or _isf(b)) else CTX.multiply(dec(a), dec(b))


def _div(a, b):
    if not (_isf(a) or _isf(b)):
        # Julia: Int64 / Int64 is the Float64 quotient (Python's int / int rounds once, too)
        return Decimal(a / b)
    return CTX.divide(dec(a), dec(b))


def _pow(a, b, literal):
    if not _isf(a) and not _isf(b):
        if b < 0:
            raise ValueError("Int ^ negative Int")
        return a ** b
    if literal is not None:
        # Base.literal_pow: x^2 = x*x, x^3 = x*x*x, x^-1 = inv(x), x^-2 = inv(x)*inv(x), ...
        x = dec(a) if literal >= 0 else CTX.divide(Decimal(1), dec(a))
        r = Decimal(1)
        for _ in range(abs(literal)):
            r = CTX.multiply(r, x)
        return r
    return CTX.power(dec(a), dec(b))


def _tanh(x):
    x = dec(x)
    if abs(x) > 60:
        return Decimal(1 if x > 0 else -1)
    e = CTX.exp(CTX.multiply(Decimal(2), x))
    return CTX.divide(CTX.subtract(e, Decimal(1)), CTX.add(e, Decimal(1)))


def _sincos(x, want_sin):
    """Taylor series at 60 digits after reducing by 2*pi."""
    with decimal.localcontext(CTX) as c:
        c.prec = 70
        x = dec(x)
        pi = _pi(c.prec + 5)
        x = x - 2 * pi * (x / (2 * pi)).to_integral_value(rounding=decimal.ROUND_FLOOR)
        term = x if want_sin else Decimal(1)
        s, k = term, (1 if want_sin else 0)
        while True:
            term = -term * x * x / ((k + 1) * (k + 2))
            k += 2
            if abs(term) < Decimal(10) ** -(c.prec + 2):
                break
            s += term
    return CTX.plus(s)


def _pi(prec):
    with decimal.localcontext() as c:
        c.prec = prec + 5
        # Machin: pi = 16 atan(1/5) - 4 atan(1/239)
        def atan_inv(m):
            x = Decimal(1) / m
            x2, term, s, k = x * x, x, x, 1
            while True:
                term = -term * x2
                k += 2
                t = term / k
                if abs(t) < Decimal(10) ** -(prec + 3):
                    return s
                s += t
        return 16 * atan_inv(5) - 4 * atan_inv(239)


def _sign(x):
    if _isf(x):
        return Decimal(0) if x == 0 else Decimal(1 if x > 0 else -1)
    return (x > 0) - (x < 0)


def _jdiv(a, b):
    if _isf(a) or _isf(b):
        return CTX.divide(dec(a), dec(b)).to_integral_value(rounding=decimal.ROUND_DOWN)
    q = abs(a) // abs(b)
    return q if (a >= 0) == (b >= 0) else -q


def _jmod(a, b):
    if _isf(a) or _isf(b):
        a, b = dec(a), dec(b)
        return CTX.subtract(a, CTX.multiply(b, CTX.divide(a, b).to_integral_value(rounding=decimal.ROUND_FLOOR)))
    return a % b      # Python's % is floored: the sign of the divisor, as Julia's mod


def _jmax(a, b):
    if _isf(a) or _isf(b):
        a, b = dec(a), dec(b)
        return b if b > a else a
    return max(a, b)


def _jmin(a, b):
    if _isf(a) or _isf(b):
        a, b = dec(a), dec(b)
        return b if b < a else a
    return min(a, b)


def _jfld(a, b):
    """Julia's fld: the quotient rounded toward minus infinity."""
    if _isf(a) or _isf(b):
        return CTX.divide(dec(a), dec(b)).to_integral_value(rounding=decimal.ROUND_FLOOR)
    return a // b


_CALLS = {
    "div": _jdiv, "mod": _jmod, "fld": _jfld, "max": _jmax, "min": _jmin, "sign": _sign,
    "abs": lambda x: abs(x) if not _isf(x) else CTX.copy_abs(x),
    "sqrt": lambda x: CTX.sqrt(dec(x)), "exp": lambda x: CTX.exp(dec(x)),
    "log": lambda x: CTX.ln(dec(x)), "tanh": _tanh,
    "sin": lambda x: _sincos(x, True), "cos": lambda x: _sincos(x, False),
    "floor": lambda x: dec(x).to_integral_value(rounding=decimal.ROUND_FLOOR),
    "ceil": lambda x: dec(x).to_integral_value(rounding=decimal.ROUND_CEILING),
}


def _lin(arr: JArr, idx):
    k, stride = 0, 1
    for d, i in zip(arr.dims, idx):
        if not isinstance(i, int):
            raise TypeError("a non-integer index")
        k += (i - 1) * stride
        stride *= d
    if len(idx) == 1:
        k = idx[0] - 1
    if k < 0 or k >= len(arr.data):
        raise IndexError(f"index {idx} out of bounds for an array of {len(arr.data)}")
    return k


class Tracer:
    """Array accesses of the iterations of the loops a plan runs in parallel, one logical
    thread per iteration: which element each iteration plainly wrote, plainly read or added to
    atomically (`record`), set up by `run_func(..., tracer=...)`.

    parallel: {id(For): {array: kind}} for the loops run one iteration per thread, with the
    plan's kind of each array ('atomic' accumulations become atomic additions; everything else
    is a plain read or write)."""

    def __init__(self, parallel: dict):
        self.parallel = parallel
        self.thread = None
        self.log: dict = {}
        self.violations: list = []
        self.loops_checked = 0

    def note(self, name, k, slot):
        if self.thread is None:
            return
        e = self.log.setdefault((name, k), (set(), set(), set()))
        e[slot].add(self.thread)

    def close(self, label):
        """The checks of `ownership_shim.jl` (/root/reference/test/ownership_shim.jl:1-20) on
        one loop's log: an element two threads write; one written by a thread and read or
        added to by another; one read by a thread and added to by another."""
        for (name, k), (w, r, a) in self.log.items():
            if len(w) >= 2:
                self.violations.append((label, name, k + 1, "multi_writer"))
            elif w and ((r | a) - w):
                self.violations.append((label, name, k + 1, "write_vs_other"))
            elif r and a and (len(r | a) > 1):
                self.violations.append((label, name, k + 1, "read_vs_atomic"))
        self.log = {}
        self.loops_checked += 1


class _Compiler:
    """Syntax tree -> Python closures over an environment dict."""

    def __init__(self, tracer: Tracer | None = None):
        self.tracer = tracer
        self.kinds: dict = {}     # the innermost parallel loop's array kinds, while compiling it

    def expr(self, e):
        if isinstance(e, S.Num):
            if e.text in ("true", "false"):
                v = e.text == "true"
                return lambda env: v
            if e.is_int:
                v = int(e.text)
                return lambda env: v
            v = Decimal(float(np.float32(float(e.text)))) if e.f32 else Decimal(float(e.text))
            return lambda env: v
        if isinstance(e, S.Var):
            nm = e.name
            return lambda env: env[nm]
        if isinstance(e, S.Ref):
            nm, ix = e.name, [self.expr(i) for i in e.idx]

            tr = self.tracer

            def ref(env):
                a = env[nm]
                k = _lin(a, [f(env) for f in ix])
                v = a.data[k]
                if v is None:
                    raise ValueError(f"read of an unset element of {nm}")
                if tr is not None:
                    tr.note(nm, k, 1)
                return v
            return ref
        if isinstance(e, S.Un):
            a = self.expr(e.a)
            if e.op == "!":
                return lambda env: not a(env)
            return lambda env: (lambda v: CTX.minus(v) if _isf(v) else -v)(a(env))
        if isinstance(e, S.Bin):
            op = e.op
            a = self.expr(e.a)
            if op == "^":
                lit = None
                if isinstance(e.b, S.Num) and e.b.is_int:
                    lit = int(e.b.text)
                b = self.expr(e.b)
                return lambda env: _pow(a(env), b(env), lit)
            b = self.expr(e.b)
            if op == "&&":
                return lambda env: bool(a(env)) and bool(b(env))
            if op == "||":
                return lambda env: bool(a(env)) or bool(b(env))
            fn = {"+": _add, "-": _sub, "*": _mul, "/": _div,
                  "==": lambda x, y: x == y, "!=": lambda x, y: x != y, "<": lambda x, y: x < y,
                  ">": lambda x, y: x > y, "<=": lambda x, y: x <= y, ">=": lambda x, y: x >= y}[op]
            return lambda env: fn(a(env), b(env))
        if isinstance(e, S.Call):
            if e.fn == "length":
                nm = e.args[0].name
                return lambda env: len(env[nm].data)
            if e.fn not in _CALLS:
                raise NotImplementedError(f"call to {e.fn}")
            f, args = _CALLS[e.fn], [self.expr(a) for a in e.args]
            return lambda env: f(*[g(env) for g in args])
        if isinstance(e, S.Alloc):
            n, isint = self.expr(e.n), e.eltype == "Int64"
            return lambda env: (lambda k: JArr([None] * max(k, 0), (max(k, 0),), isint))(n(env))
        if isinstance(e, S.Tup):
            items = [self.expr(i) for i in e.items]
            return lambda env: tuple(f(env) for f in items)
        if isinstance(e, S.Nothing_):
            return lambda env: None
        raise NotImplementedError(type(e).__name__)

    def block(self, body):
        fs = [self.stmt(s) for s in body]

        def run(env):
            for f in fs:
                f(env)
        return run

    def stmt(self, s):
        if isinstance(s, S.Assign):
            rhs = self.expr(s.rhs)
            if isinstance(s.lhs, S.Var):
                nm = s.lhs.name

                def assign(env):
                    env[nm] = rhs(env)
                return assign
            nm, ix = s.lhs.name, [self.expr(i) for i in s.lhs.idx]
            tr = self.tracer
            r = s.rhs
            if (tr is not None and self.kinds.get(nm) == "atomic" and isinstance(r, S.Bin) and r.op in ("+", "-")
                    and s.lhs in (r.a, r.b)):
                # an accumulation the plan makes atomic: the element's read is part of the addition
                other = self.expr(r.b if r.a == s.lhs else r.a)
                neg = r.op == "-" and r.a == s.lhs
                first = r.a == s.lhs

                def atomic(env):
                    a = env[nm]
                    v = other(env)
                    k = _lin(a, [f(env) for f in ix])
                    old = a.data[k]
                    if old is None:
                        raise ValueError(f"read of an unset element of {nm}")
                    if neg:
                        nv = _sub(old, v)
                    else:
                        nv = _add(old, v) if first else _add(v, old)
                    a.data[k] = nv if not a.isint else int(nv)
                    tr.note(nm, k, 2)
                return atomic

            def store(env):
                a = env[nm]
                v = rhs(env)
                if a.isint:
                    if _isf(v):
                        if v != v.to_integral_value():
                            raise ValueError(f"InexactError storing {v} into Int64 array {nm}")
                        v = int(v)
                elif not _isf(v):
                    v = dec(v)
                k = _lin(a, [f(env) for f in ix])
                a.data[k] = v
                if tr is not None:
                    tr.note(nm, k, 0)
            return store
        if isinstance(s, S.For):
            var, lo, hi = s.var, self.expr(s.rng.lo), self.expr(s.rng.hi)
            st = self.expr(s.rng.step) if s.rng.step is not None else (lambda env: 1)
            tr = self.tracer
            par = tr is not None and id(s) in tr.parallel
            if par:
                saved, self.kinds = self.kinds, tr.parallel[id(s)]
            body = self.block(s.body)
            if par:
                self.kinds = saved
            label = f"for {var}"

            def loop(env):
                a, step, b = lo(env), st(env), hi(env)
                had, old = var in env, env.get(var)
                rng = range(a, b + 1, step) if step > 0 else range(a, b - 1, step)
                try:
                    for it, v in enumerate(rng):
                        if par:
                            tr.thread = it
                        env[var] = v
                        try:
                            body(env)
                        except _Continue:
                            continue
                except _Break:
                    pass
                finally:
                    if had:
                        env[var] = old
                    else:
                        env.pop(var, None)
                    if par:
                        tr.thread = None
                        tr.close(label)
            return loop
        if isinstance(s, S.While):
            cond, body = self.expr(s.cond), self.block(s.body)

            def wloop(env):
                try:
                    while cond(env):
                        try:
                            body(env)
                        except _Continue:
                            continue
                except _Break:
                    pass
            return wloop
        if isinstance(s, S.If):
            brs = [(self.expr(c), self.block(b)) for c, b in s.branches]
            orelse = self.block(s.orelse) if s.orelse is not None else None

            def ifs(env):
                for c, b in brs:
                    if c(env):
                        b(env)
                        return
                if orelse is not None:
                    orelse(env)
            return ifs
        if isinstance(s, S.Return):
            v = self.expr(s.value) if s.value is not None else (lambda env: None)

            def ret(env):
                raise _Return(v(env))
            return ret
        if isinstance(s, S.Break):
            def brk(env):
                raise _Break()
            return brk
        if isinstance(s, S.Continue):
            def cont(env):
                raise _Continue()
            return cont
        if isinstance(s, S.ExprStmt):
            f = self.expr(s.e)
            return lambda env: (f(env), None)[1]
        if isinstance(s, S.Gemm):
            return self.gemm(s)
        if isinstance(s, S.GemmT):
            return self.gemm_tab(s)
        raise NotImplementedError(type(s).__name__)

    def gemm_tab(self, s):
        """A table-addressed product of the lowering by its definition (every offset through
        its table or stride; an address outside an array, or an unset element, raises)."""
        ex = self.expr
        head = [ex(e) for e in (s.out_off, s.M, s.N, s.K, s.a_off, s.b_off)]
        dims = [(d.table, ex(d.stride) if d.table is None else None) for d in (s.ro, s.co, s.ar, s.ak, s.bk, s.bc)]

        def elem(arr, k, nm):
            if k < 0 or k >= len(arr.data):
                raise IndexError(f"matrix product: {nm}[{k}] outside an array of {len(arr.data)}")
            v = arr.data[k]
            if v is None:
                raise ValueError(f"matrix product: read of an unset element of {nm}")
            return v

        def gemm(env):
            c0, M, N, K, a0, b0 = (f(env) for f in head)

            def at(d):
                tab, st = d
                if tab is None:
                    sv = st(env)
                    return lambda i: i * sv
                arr = env[tab]
                return lambda i: int(elem(arr, i, tab))
            ro, co, ar, ak, bk, bc = (at(d) for d in dims)
            A, B, C = env[s.a], env[s.b], env[s.out]
            akv = [ak(k) for k in range(K)]
            bkv = [bk(k) for k in range(K)]
            for m in range(M):
                am = a0 + ar(m)
                for n in range(N):
                    bn = b0 + bc(n)
                    t = Decimal(0)
                    for k in range(K):
                        t = _add(t, _mul(elem(A, am + akv[k], s.a), elem(B, bkv[k] + bn, s.b)))
                    ic = c0 + ro(m) + co(n)
                    C.data[ic] = t if s.mode == 0 else _add(elem(C, ic, s.out), t)
        return gemm

    def gemm(self, s):
        """A matrix product of the lowering (stade_hip.lower.contract) by its definition:
        out[off + m sm + n sn] (+)= sum over segments of sum_k A(m, k) B(k, n), every element
        addressed as the statement's offsets and leading dimensions say (an address outside
        an array, or an unset element, raises)."""
        ex = self.expr
        head = [ex(e) for e in (s.out_off, s.out_sm, s.out_sn, s.M, s.N)]
        segs = [(g.a, ex(g.a_off), g.a_km, ex(g.lda), g.b, ex(g.b_off), g.b_km, ex(g.ldb), ex(g.K)) for g in s.segs]

        def elem(arr, k, nm):
            if k < 0 or k >= len(arr.data):
                raise IndexError(f"matrix product: {nm}[{k}] outside an array of {len(arr.data)}")
            v = arr.data[k]
            if v is None:
                raise ValueError(f"matrix product: read of an unset element of {nm}")
            return v

        def gemm(env):
            off, sm, sn, M, N = (f(env) for f in head)
            C = env[s.out]
            sv = [(a, env[a], ao(env), akm, la(env), b, env[b], bo(env), bkm, lb(env), K(env))
                  for a, ao, akm, la, b, bo, bkm, lb, K in segs]
            for m in range(M):
                for n in range(N):
                    t = Decimal(0)
                    for a, A, ao, akm, la, b, B, bo, bkm, lb, K in sv:
                        for k in range(K):
                            x = elem(A, ao + (k + m * la if akm else m + k * la), a)
                            y = elem(B, bo + (k + n * lb if bkm else n + k * lb), b)
                            t = _add(t, _mul(x, y))
                    ic = off + m * sm + n * sn
                    C.data[ic] = _add(elem(C, ic, s.out), t) if s.acc else t
        return gemm


def _to_j(v):
    if isinstance(v, np.ndarray):
        if v.dtype == np.int64:
            return JArr([int(x) for x in v.ravel(order="F")], v.shape or (1,), True)
        return JArr([dec(x) for x in v.ravel(order="F")], v.shape or (1,), False)
    if isinstance(v, (int, np.integer)) and not isinstance(v, bool):
        return int(v)
    return dec(v)


def run(text: str, fname: str, args):
    """Execute generated function `fname` of `text` on `args`; returns (arrays, returned):
    the final contents of every array argument (None for scalars) and the returned values
    as a tuple (empty for `nothing`)."""
    funcs = {f.name: f for f in S.parse(text)}
    return run_func(funcs[fname], args)


def run_func(f, args, tracer: Tracer | None = None):
    """`run` on a parsed function (a syntax tree, transformed or not); with a tracer, the
    accesses of its parallel loops' iterations are recorded and checked (`Tracer`)."""
    fname = f.name
    if len(args) != len(f.args):
        raise TypeError(f"{fname} takes {len(f.args)} arguments, got {len(args)}")
    env = {a: _to_j(v) for a, v in zip(f.args, args)}
    body = _Compiler(tracer).block(f.body)
    ret = None
    try:
        body(env)
    except _Return as r:
        ret = r.value
    arrays = [env[a].data if isinstance(v, np.ndarray) else None for a, v in zip(f.args, args)]
    if ret is None:
        rets = ()
    elif isinstance(ret, tuple):
        rets = ret
    else:
        rets = (ret,)
    return arrays, rets
