"""Contractions of the generated code onto the matrix cores.

A dense layer's generated code sums products in a sequential loop nested in a parallel flat
loop.  The forward form (one iteration per output element (i, j), a sum over k):

    for idx = 1:R * N                       # i = div(idx - 1, N) + 1, j = mod(idx - 1, N) + 1
        s = b[j]
        for k = 1:K
            s = s + w[(k - 1) * N + j] * x[(i - 1) * K + k]
        end
        h[...] = tanh(s)
    end

and the adjoint form, whose inner loop scatters products of a per-iteration scalar into two
arrays, each summed over the other coordinate:

    for idx = R * N:-1:1
        ... sb = ... ;
        for k = K:-1:1
            wb[(k - 1) * N + j] = wb[(k - 1) * N + j] + x[(i - 1) * K + k] * sb
            xb[(i - 1) * K + k] = xb[(i - 1) * K + k] + w[(k - 1) * N + j] * sb
        end
    end

On the vector units these run one thread per (i, j) with K-long dot products or K atomics
per thread.  Here the inner loop becomes matrix products on the fp32 matrix cores
(csrc/gemm_f32.hpp) around a loop that keeps the rest of the body:
- forward: a product T(j, i) = sum_k A(j, k) B(k, i) of the two factors, run before the
  loop, and `s = s + T[j, i]` in place of the inner loop (one per accumulated scalar; a
  term list `A1 B1 + A2 B2` is a two-segment product);
- adjoint: the loop stores each scalar the products scale into a scratch array V[j, i] in
  place of the inner loop, and a product per accumulated array after the loop adds
  sum over the other coordinate of V times the factor into it (`C(j, k) += sum_i V(j, i)
  x(k, i)`).

The reference's AMDGPU path has no such rewrite: its `stade_gpu` runs these loops as
written (`cgen_body` /root/reference/src/STADE.jl:11937); the hand-written configs
(csrc/mlp2_ce.hip, conv3x3.hip) are this build's products of the same loops.  The sums are
reassociated (a product sums K terms in its own order, and s adds the whole sum to its
initial value), so results match the loops to fp32 rounding, not bit for bit: fp32 only (the
configs' fp32 tolerance), and only with unchecked accesses (a product reads exactly the
elements the loops read, without the per-access range checks).

Conditions, all checked, else the loop stays as it is:
- the loop is at the function's top level, a flat loop over 1:R*N (either direction) with
  i = div(idx - 1, N) + 1 and j = mod(idx - 1, N) + 1 and R, N expressions of Int arguments;
- the inner loop runs k over all of 1:K (either direction), K an expression of Int
  arguments, and holds only Int index temporaries, float temporaries that name one element,
  and accumulations (all scalar `s = s + E`, or all array `C[e] = C[e] + E`);
- each term of E is a product of two elements (forward) or of an element and a scalar the
  inner loop does not assign (adjoint), every index affine in k and in one of i, j with
  coefficients of Int arguments and a unit stride in k or in that coordinate;
- forward: no array a product reads is written anywhere in the loop; adjoint: an accumulated
  array is touched by nothing else in the loop, and no factor array is written in it;
- the inner loop's temporaries are read nowhere else.
"""
from __future__ import annotations

import os
from dataclasses import dataclass

from .analysis import (NotAffine, Types, _derived, _freeze, _linear_index, _mul, _reads_of, _upward_exposed, linear_in,
                       to_poly)
from .syntax import (Alloc, Assign, Bin, Call, For, Func, Gemm, GemmSeg, GemmT, Num, Range, Ref, TabDim, Un, Var,
                     stmt_exprs, walk_expr, walk_stmts)

ONE = {(): 1}


class _No(Exception):
    pass


def _num(v: int) -> Num:
    return Num(str(v), True)


def poly_expr(p: dict):
    """The Int expression of a polynomial over Int-argument atoms."""
    terms = []
    for m, c in sorted(p.items()):
        if c == 0:
            continue
        e = None
        for a in m:
            if a[0] != "v":
                raise _No("a coefficient that is not a product of Int arguments")
            e = Var(a[1]) if e is None else Bin("*", e, Var(a[1]))
        if e is None:
            e = _num(c)
        elif c != 1:
            e = Bin("*", _num(c), e)
        terms.append(e)
    if not terms:
        return _num(0)
    out = terms[0]
    for t in terms[1:]:
        out = Bin("+", out, t)
    return out


def _host_poly(p: dict, host_ints: set) -> bool:
    return all(a[0] == "v" and a[1] in host_ints for m in p for a in m)


@dataclass
class Affine:
    """A reference's 0-based element offset as off + sk (k - 1) + sc (c - 1), c the one outer
    coordinate it depends on (None: neither)."""
    array: str
    off: dict
    sk: dict
    coord: str | None
    sc: dict


@dataclass
class Flat:
    var: str
    iv: str
    jv: str
    R: object
    N: object


def flat_of(loop: For, host_ints: set) -> Flat | None:
    """The flat decomposition of `for idx = 1:R*N` (or `R*N:-1:1`) with i = div(idx - 1, N) + 1
    and j = mod(idx - 1, N) + 1 assigned once each at the top of the body."""
    r = loop.rng
    step = 1 if r.step is None else (int(r.step.text) if isinstance(r.step, Num) and r.step.is_int else 0)
    one = lambda e: isinstance(e, Num) and e.is_int and int(e.text) == 1
    if step == 1 and one(r.lo):
        trip = r.hi
    elif step == -1 and one(r.hi):
        trip = r.lo
    else:
        return None
    v = loop.var
    count = {}
    for s in loop.body:
        if isinstance(s, Assign) and isinstance(s.lhs, Var):
            count[s.lhs.name] = count.get(s.lhs.name, 0) + 1
    vm1 = {s.lhs.name for s in loop.body if isinstance(s, Assign) and isinstance(s.lhs, Var)
           and isinstance(s.rhs, Bin) and s.rhs.op == "-" and s.rhs.a == Var(v) and one(s.rhs.b)
           and count[s.lhs.name] == 1}
    der = [d for d in (_derived(s, v, vm1) for s in loop.body) if d is not None]
    divs = [d for d in der if d[1] == "div"]
    mods = [d for d in der if d[1] == "mod"]
    if len(divs) != 1 or len(mods) != 1 or divs[0][2] != mods[0][2]:
        return None
    iv, jv, N = divs[0][0], mods[0][0], divs[0][2]
    if count.get(iv) != 1 or count.get(jv) != 1:
        return None
    if not (isinstance(trip, Bin) and trip.op == "*"):
        return None
    if trip.b == N:
        R = trip.a
    elif trip.a == N:
        R = trip.b
    else:
        return None
    names = lambda e: {x.name for x in walk_expr(e) if isinstance(x, Var)}
    if not (names(N) | names(R)) <= host_ints:
        return None
    return Flat(v, iv, jv, R, N)


@dataclass
class Digit:
    """One digit of a flat loop variable: name = mod(div(idx - 1, P), R) + 1 (the top digit:
    div(idx - 1, P) + 1, its range the trip count / P)."""
    name: str
    P: dict
    R: dict
    Re: object


def _mono_div(p: dict, q: dict):
    """p / q for single monomials with an exact quotient, else None."""
    if len(p) != 1 or len(q) != 1:
        return None
    (mp, cp), = p.items()
    (mq, cq), = q.items()
    if cq == 0 or cp % cq:
        return None
    rest = list(mp)
    for a in mq:
        if a not in rest:
            return None
        rest.remove(a)
    return {tuple(rest): cp // cq}


def digits_of(loop: For, T: Types, host_ints: set) -> list | None:
    """The digits of `for idx = 1:trip` (or `trip:-1:1`) in increasing place value, when the
    body's top Int temporaries decompose idx - 1 into a complete mixed radix
    (idx - 1 = sum (d - 1) P_d, P of the first 1, each next P the product of those before and
    their ranges, the trip count the product of all), else None."""
    r = loop.rng
    step = 1 if r.step is None else (int(r.step.text) if isinstance(r.step, Num) and r.step.is_int else 0)
    one = lambda e: isinstance(e, Num) and e.is_int and int(e.text) == 1
    if step == 1 and one(r.lo):
        trip = r.hi
    elif step == -1 and one(r.hi):
        trip = r.lo
    else:
        return None
    v = loop.var
    count = {}
    for s in loop.body:
        if isinstance(s, Assign) and isinstance(s.lhs, Var):
            count[s.lhs.name] = count.get(s.lhs.name, 0) + 1
    vm1 = {s.lhs.name for s in loop.body if isinstance(s, Assign) and isinstance(s.lhs, Var)
           and isinstance(s.rhs, Bin) and s.rhs.op == "-" and s.rhs.a == Var(v) and one(s.rhs.b)
           and count[s.lhs.name] == 1}
    is_e0 = lambda x: (isinstance(x, Var) and x.name in vm1) or (isinstance(x, Bin) and x.op == "-" and x.a == Var(v)
                                                                   and one(x.b))

    def poly(e):
        try:
            p = to_poly(e, {}, T)
        except NotAffine:
            return None
        return p if _host_poly(p, host_ints) and p else None
    found = []
    for s in loop.body:
        if not (isinstance(s, Assign) and isinstance(s.lhs, Var) and count.get(s.lhs.name) == 1):
            continue
        e = s.rhs
        if not (isinstance(e, Bin) and e.op == "+" and one(e.b) and isinstance(e.a, Call) and len(e.a.args) == 2):
            continue
        c = e.a
        if c.fn == "mod" and is_e0(c.args[0]):
            P, R, Re = {(): 1}, poly(c.args[1]), c.args[1]
        elif (c.fn == "mod" and isinstance(c.args[0], Call) and c.args[0].fn == "div" and len(c.args[0].args) == 2
              and is_e0(c.args[0].args[0])):
            P, R, Re = poly(c.args[0].args[1]), poly(c.args[1]), c.args[1]
        elif c.fn == "div" and is_e0(c.args[0]):
            P, R, Re = poly(c.args[1]), None, None
        else:
            continue
        if P is None or (Re is not None and R is None):
            return None
        found.append(Digit(s.lhs.name, P, R, Re))
    if len(found) < 2:
        return None
    tp = poly(trip)
    if tp is None:
        return None
    out, cur, left = [], {(): 1}, list(found)
    while left:
        nxt = [d for d in left if _freeze(d.P) == _freeze(cur)]
        if len(nxt) != 1:
            return None
        d = nxt[0]
        left.remove(d)
        out.append(d)
        if d.R is None:
            if left:
                return None
            q = _mono_div(tp, d.P)
            if q is None:
                return None
            d.R = q
            d.Re = poly_expr(q)
            return out
        cur = _mul(cur, d.R)
    return out if _freeze(cur) == _freeze(tp) else None


def _rename_expr(e, ren: dict):
    if isinstance(e, Ref):
        return Ref(ren.get(e.name, e.name), tuple(_rename_expr(x, ren) for x in e.idx))
    if isinstance(e, Bin):
        return Bin(e.op, _rename_expr(e.a, ren), _rename_expr(e.b, ren))
    if isinstance(e, Un):
        return Un(e.op, _rename_expr(e.a, ren))
    if isinstance(e, Call):
        return Call(e.fn, tuple(_rename_expr(x, ren) for x in e.args))
    return e


def _rename_refs(st, ren: dict) -> None:
    """Rename the arrays `ren` maps in the references of a statement and its nested ones, in
    place (the statements keep their identity)."""
    for x in walk_stmts([st]):
        if isinstance(x, Assign):
            x.rhs = _rename_expr(x.rhs, ren)
            if isinstance(x.lhs, Ref):
                x.lhs = _rename_expr(x.lhs, ren)


BIG = 1 << 30      # the run of a digit whose range is an argument (taken as long)


def _run_of(R) -> int:
    """A digit's range as a run length: its value when a literal, else BIG."""
    return int(R.text) if isinstance(R, Num) and R.is_int else BIG


def _subst(e, f):
    """e with every Var replaced by f(name) (an expression)."""
    if isinstance(e, Var):
        return f(e.name)
    if isinstance(e, Bin):
        return Bin(e.op, _subst(e.a, f), _subst(e.b, f))
    if isinstance(e, Un):
        return Un(e.op, _subst(e.a, f))
    if isinstance(e, Call):
        return Call(e.fn, tuple(_subst(x, f) for x in e.args))
    if isinstance(e, Ref):
        return Ref(e.name, tuple(_subst(x, f) for x in e.idx))
    return e


@dataclass
class Split:
    """A reference's 0-based offset as outer(digits) + inner(k) + const - 1, the two parts
    polynomials in disjoint variables."""
    array: str
    outer: dict
    inner: dict
    uses: set


class _Tables:
    """The table form of one inner loop: splitting of references, and the loops that fill the
    offset tables (over a set of digits, or over the inner index)."""

    def __init__(self, rw, digits, inner: For, k: str, K, outer_env: dict, var: str):
        self.rw, self.digits, self.k, self.K, self.var = rw, digits, k, K, var
        self.loops, self.allocs, self.cache = [], [], {}
        T = rw.T
        # inner Int temporaries: those with div / mod stay variables of the inner offset (their
        # definitions, in order, are copied into the inner tables' loops); the rest substitute
        self.int_stmts, self.atoms, env = [], set(), dict(outer_env)
        for s in inner.body:
            if isinstance(s, Assign) and isinstance(s.lhs, Var) and T.scalars.get(s.lhs.name) == "i":
                self.int_stmts.append(s)
                if any(isinstance(x, Call) and x.fn in ("div", "mod") for x in walk_expr(s.rhs)):
                    self.atoms.add(s.lhs.name)
                else:
                    env[s.lhs.name] = s.rhs
        self.env = env
        # the inner index's fastest digit: a temporary mod(k - 1, R) + 1 (or k itself)
        km1 = {s.lhs.name for s in self.int_stmts if isinstance(s.rhs, Bin) and s.rhs.op == "-"
               and s.rhs.a == Var(k) and isinstance(s.rhs.b, Num) and s.rhs.b.text == "1"}
        self.fast, self.fast_run = k, BIG
        for s in self.int_stmts:
            e = s.rhs
            if (isinstance(e, Bin) and e.op == "+" and isinstance(e.b, Num) and e.b.text == "1"
                    and isinstance(e.a, Call) and e.a.fn == "mod"
                    and (e.a.args[0] in [Var(x) for x in km1] or e.a.args[0] == Bin("-", Var(k), Num("1", True)))):
                self.fast = s.lhs.name
                self.fast_run = _run_of(e.a.args[1])
        # the inner tables' loops recompute the div / mod temporaries and what they read; those
        # may depend on nothing of the outer loop
        inner_names = {s.lhs.name for s in self.int_stmts}
        need = set(self.atoms)
        for s in reversed(self.int_stmts):
            if s.lhs.name in need:
                need |= _reads_of(s.rhs) & inner_names
        self.int_stmts = [s for s in self.int_stmts if s.lhs.name in need]
        for s in self.int_stmts:
            if not _reads_of(s.rhs) <= inner_names | {k} | rw.host_ints:
                raise _No("an inner index temporary reads the outer loop")

    def split(self, ref: Ref) -> Split:
        T = self.rw.T
        try:
            p = to_poly(_linear_index(ref, T), self.env, T)
        except NotAffine:
            raise _No(f"{ref.name}: index not a polynomial")
        dn = {d.name for d in self.digits}
        inner_v = self.atoms | {self.k}
        outer, inner, const = {}, {}, {}
        for m, c in p.items():
            if any(a[0] != "v" for a in m):
                raise _No(f"{ref.name}: a div / mod outside the digits")
            names = {a[1] for a in m}
            o, i = names & dn, names & inner_v
            if not names - dn - inner_v <= self.rw.host_ints:
                raise _No(f"{ref.name}: reads a variable of neither loop")
            if o and i:
                raise _No(f"{ref.name}: the offset does not split into outer and inner parts")
            (outer if o else inner if i else const)[m] = c
        inner = dict(inner)
        for m, c in const.items():
            inner[m] = inner.get(m, 0) + c
        inner[()] = inner.get((), 0) - 1
        inner = {m: c for m, c in inner.items() if c}
        return Split(ref.name, outer, inner, {a[1] for m in outer for a in m} & dn)

    def size(self, D):
        out = None
        for d in D:
            out = d.Re if out is None else Bin("*", out, d.Re)
        return out if out is not None else _num(1)

    def unit_t(self, poly: dict) -> int:
        """How many adjacent k are adjacent elements: the run of the inner index's fastest
        digit when its coefficient is 1, else 0."""
        if poly.get(((("v", self.k),)), 0) == 1:
            return BIG
        return self.fast_run if poly.get(((("v", self.fast),)), 0) == 1 else 0

    @staticmethod
    def unit_rows(D, poly: dict) -> int:
        """How many adjacent rows over digits D are adjacent elements (0: none)."""
        return _run_of(D[0].Re) if D and poly.get(((("v", D[0].name),)), 0) == 1 else 0

    def place(self, D) -> dict:
        """The digits' share of idx - 1: sum over D of (d - 1) P_d."""
        out = {}
        for d in D:
            for m, c in _mul({(("v", d.name),): 1}, d.P).items():
                out[m] = out.get(m, 0) + c
            for m, c in d.P.items():
                out[m] = out.get(m, 0) - c
        return {m: c for m, c in out.items() if c}

    def row_table(self, D, sp) -> TabDim:
        """A table over the mixed radix of digits D of a polynomial in them (a Split's outer
        part, or a polynomial)."""
        poly = sp.outer if isinstance(sp, Split) else sp
        key = ("row", tuple(d.name for d in D), _freeze(poly))
        if key in self.cache:
            return self.cache[key]
        rw = self.rw
        name, q, r0 = rw.fresh("R"), rw.fresh("q"), rw.fresh("r")
        stmts = [Assign(Var(r0), Bin("-", Var(q), _num(1)))]
        ren, Q = {}, None
        for j, d in enumerate(D):
            dv = rw.fresh("d")
            x = Var(r0) if Q is None else Call("div", (Var(r0), Q))
            val = x if j == len(D) - 1 else Call("mod", (x, d.Re))
            stmts.append(Assign(Var(dv), Bin("+", val, _num(1))))
            ren[d.name] = dv
            Q = d.Re if Q is None else Bin("*", Q, d.Re)
        stmts.append(Assign(Ref(name, (Var(q),)), _subst(poly_expr(poly), lambda n: Var(ren.get(n, n)))))
        n_ = self.size(D)
        self.allocs.append(Assign(Var(name), Alloc("Int64", n_)))
        self.loops.append(For(q, Range(_num(1), None, n_), stmts))
        self.cache[key] = TabDim(name, _num(0))
        return self.cache[key]

    def t_table(self, sp: Split) -> TabDim:
        key = ("t", _freeze(sp.inner))
        if key in self.cache:
            return self.cache[key]
        rw = self.rw
        name, kv = rw.fresh("K"), rw.fresh("k")
        ren = {self.k: kv}
        stmts = []
        for s in self.int_stmts:
            nv = rw.fresh("t")
            stmts.append(Assign(Var(nv), _subst(s.rhs, lambda n: Var(ren.get(n, n)))))
            ren[s.lhs.name] = nv
        stmts.append(Assign(Ref(name, (Var(kv),)), _subst(poly_expr(sp.inner), lambda n: Var(ren.get(n, n)))))
        self.allocs.append(Assign(Var(name), Alloc("Int64", self.K)))
        self.loops.append(For(kv, Range(_num(1), None, self.K), stmts))
        self.cache[key] = TabDim(name, _num(0))
        return self.cache[key]


class _Rewriter:
    def __init__(self, f: Func, T: Types, host_ints: set, is_parallel):
        self.f = f
        self.T = T
        self.host_ints = host_ints
        self.is_parallel = is_parallel
        self.n = 0
        self.rec = {"forward": 0, "adjoint": 0, "gemms": 0, "loops": []}
        # Int names the function sets once, at its top level, from its Int arguments (`i_wp =
        # i_w + 2`): substituted into indices like the arguments themselves
        count = {}
        for s in walk_stmts(f.body):
            if isinstance(s, Assign) and isinstance(s.lhs, Var):
                count[s.lhs.name] = count.get(s.lhs.name, 0) + 1
        self.fenv = {s.lhs.name: s.rhs for s in f.body if isinstance(s, Assign) and isinstance(s.lhs, Var)
                     and count[s.lhs.name] == 1 and T.scalars.get(s.lhs.name) == "i"
                     and {x.name for x in walk_expr(s.rhs) if isinstance(x, Var)} <= host_ints
                     and not any(isinstance(x, Ref) for x in walk_expr(s.rhs))}

    def fresh(self, stem: str) -> str:
        self.n += 1
        return f"__gemm_{stem}{self.n}"

    # -- index analysis ------------------------------------------------------------------------
    def affine(self, ref: Ref, env: dict, k: str, fl: Flat) -> Affine:
        try:
            p = to_poly(_linear_index(ref, self.T), env, self.T)
        except NotAffine:
            raise _No(f"{ref.name}: index not affine")
        lk = linear_in(p, k)
        if lk is None:
            raise _No(f"{ref.name}: not linear in {k}")
        sk, rest = lk
        li = linear_in(rest, fl.iv)
        lj = linear_in(li[1] if li else {}, fl.jv) if li else None
        if li is None or lj is None:
            raise _No(f"{ref.name}: not linear in the coordinates")
        si, (sj, off) = li[0], lj
        for q in (sk, si, sj, off):
            if not _host_poly(q, self.host_ints):
                raise _No(f"{ref.name}: a coefficient the host cannot evaluate")
        if si and sj:
            raise _No(f"{ref.name}: depends on both coordinates")
        coord, sc = (fl.iv, si) if si else ((fl.jv, sj) if sj else (None, {}))
        # 0-based offset at k = 1, c = 1: (p - 1) = off + sk + sc - 1 + sk (k - 1) + sc (c - 1)
        off0 = dict(off)
        for q in (sk, sc):
            for m, c in q.items():
                off0[m] = off0.get(m, 0) + c
        off0[()] = off0.get((), 0) - 1
        off0 = {m: c for m, c in off0.items() if c}
        return Affine(ref.name, off0, sk, coord, sc)

    # -- the inner loop ---------------------------------------------------------------------------
    def inner_parts(self, inner: For, outer_env: dict, fl: Flat):
        k = inner.var
        r = inner.rng
        one = lambda e: isinstance(e, Num) and e.is_int and int(e.text) == 1
        step = 1 if r.step is None else (int(r.step.text) if isinstance(r.step, Num) and r.step.is_int else 0)
        if step == 1 and one(r.lo):
            K = r.hi
        elif step == -1 and one(r.hi):
            K = r.lo
        else:
            raise _No("inner range not 1:K")
        if not {x.name for x in walk_expr(K) if isinstance(x, Var)} <= self.host_ints:
            raise _No("inner bound not host-evaluable")
        env = dict(outer_env)
        alias = {}
        temps = set()
        accs = []
        assigned = set()
        for s in inner.body:
            if not isinstance(s, Assign):
                raise _No("inner loop holds a non-assignment")
            if isinstance(s.lhs, Var):
                nm = s.lhs.name
                if nm in assigned:
                    raise _No(f"{nm} assigned twice in the inner loop")
                r_ = s.rhs
                if isinstance(r_, Bin) and r_.op == "+" and Var(nm) in (r_.a, r_.b):
                    other = r_.b if r_.a == Var(nm) else r_.a
                    if nm in _reads_of(other):
                        raise _No("accumulation reads itself twice")
                    accs.append(("s", Var(nm), other))
                    assigned.add(nm)
                    continue
                if self.T.scalars.get(nm) == "i":
                    env[nm] = r_
                elif isinstance(r_, Ref) and self.T.arrays.get(r_.name) == "f":
                    alias[nm] = r_
                else:
                    raise _No(f"inner temporary {nm} is not an index or an element")
                temps.add(nm)
                assigned.add(nm)
                continue
            ref = s.lhs
            r_ = s.rhs
            if not (isinstance(r_, Bin) and r_.op == "+" and ref in (r_.a, r_.b)):
                raise _No(f"store to {ref.name} is not an accumulation")
            other = r_.b if r_.a == ref else r_.a
            if any(isinstance(x, Ref) and x.name == ref.name for x in walk_expr(other)):
                raise _No("accumulation reads its own array")
            accs.append(("c", ref, other))
        if not accs or len({a[0] for a in accs}) != 1:
            raise _No("no accumulation, or scalar and array accumulations mixed")
        acc_names = {a[1].name for a in accs if a[0] == "s"}
        for _, _, e in accs:
            if _reads_of(e) & acc_names:
                raise _No("a product reads an accumulated scalar")
        return k, K, env, alias, temps, accs

    def terms(self, e) -> list:
        if isinstance(e, Bin) and e.op == "+":
            return self.terms(e.a) + self.terms(e.b)
        if isinstance(e, Bin) and e.op == "*":
            return [(e.a, e.b)]
        raise _No("a term that is not a product")

    def resolve(self, x, alias):
        if isinstance(x, Var) and x.name in alias:
            return alias[x.name]
        return x

    # -- products ------------------------------------------------------------------------------------
    @staticmethod
    def layout(a: Affine):
        """(km, ld) of an element factor as a gemm operand over (its coordinate, the summed
        index): km when the summed index is contiguous (X[s + c ld], ld the coordinate's
        stride), else the coordinate is (X[c + s ld], ld the summed index's stride).  The
        same flag means A_KM for the gemm's A operand (rows the coordinate) and B_KM for its
        B operand (columns the coordinate)."""
        if a.sk == ONE:
            return True, a.sc
        if a.sc == ONE:
            return False, a.sk
        raise _No(f"{a.array}: no unit stride")

    def seg(self, A: Affine, B: Affine, K) -> GemmSeg:
        a_km, lda = self.layout(A)
        b_km, ldb = self.layout(B)
        return GemmSeg(A.array, poly_expr(A.off), a_km, poly_expr(lda), B.array, poly_expr(B.off), b_km,
                       poly_expr(ldb), K)

    def written_in(self, body) -> set:
        out = set()
        for s in walk_stmts(body):
            if isinstance(s, Assign) and isinstance(s.lhs, Ref):
                out.add(s.lhs.name)
        return out

    def refs_in(self, stmts) -> set:
        out = set()
        for s in walk_stmts(stmts):
            for e in stmt_exprs(s):
                out |= {x.name for x in walk_expr(e) if isinstance(x, Ref)}
            if isinstance(s, Assign) and isinstance(s.lhs, Ref):
                out.add(s.lhs.name)
        return out

    def live_after(self, names: set, loop: For, inner: For) -> bool:
        """Any of `names` (assigned in `inner`, a top-level statement of `loop`'s body) read
        after `inner` before being assigned again: in the rest of the iteration, the next
        iteration, or the statements after `loop` in the function."""
        pos = next(j for j, x in enumerate(loop.body) if x is inner)
        top = next(j for j, x in enumerate(self.f.body) if x is loop)
        cont = loop.body[pos + 1:] + loop.body + self.f.body[top + 1:]
        return any(_upward_exposed(cont, n) for n in names)

    def rewrite_loop(self, loop: For):
        """(statements before, the new loop, statements after) or raises _No.  Each inner loop
        is tried in the strided form (a two-coordinate flat loop, operands with a unit
        stride: the tuned GEMM), then in the table form (any mixed-radix flat loop, factors
        that are sums of an outer and an inner offset)."""
        fl = flat_of(loop, self.host_ints)
        dg = digits_of(loop, self.T, self.host_ints)
        if fl is None and dg is None:
            raise _No("not a flat loop")
        # outer Int temporaries (assigned once, not the coordinates) substitute into indices
        count = {}
        for s in walk_stmts(loop.body):
            if isinstance(s, Assign) and isinstance(s.lhs, Var):
                count[s.lhs.name] = count.get(s.lhs.name, 0) + 1
        coords = {fl.iv, fl.jv} if fl is not None else set()
        digit_names = {d.name for d in dg} if dg is not None else set()
        outer_ints = {s.lhs.name: s.rhs for s in loop.body if isinstance(s, Assign) and isinstance(s.lhs, Var)
                      and self.T.scalars.get(s.lhs.name) == "i" and count[s.lhs.name] == 1}
        outer_env = dict(self.fenv, **{n: e for n, e in outer_ints.items() if n not in coords})
        outer_env_t = dict(self.fenv, **{n: e for n, e in outer_ints.items() if n not in digit_names})
        inners = [s for s in loop.body if isinstance(s, For)]
        if not inners:
            raise _No("no inner loop")
        written = self.written_in(loop.body)
        before, after, new_body = [], [], []
        done = 0
        for s in loop.body:
            if not isinstance(s, For):
                new_body.append(s)
                continue
            try:
                k, K, env, alias, temps, accs = self.inner_parts(s, outer_env, fl)
                # (k itself is the loop's own: a Julia loop variable is a new local of the loop)
                if self.live_after(temps, loop, s):
                    raise _No("an inner temporary is read outside the inner loop")
                pre = repl = post = None
                if fl is not None:
                    lin = Bin("+", Var(fl.jv), Bin("*", Bin("-", Var(fl.iv), _num(1)), fl.N))   # (j, i), j fastest
                    size = Bin("*", fl.R, fl.N)
                    try:
                        if accs[0][0] == "s":
                            pre, repl = self.forward(s, k, K, env, alias, accs, fl, written, lin, size)
                            post = []
                        else:
                            repl, post = self.adjoint(loop, s, k, K, env, alias, accs, fl, written, lin, size)
                            pre = []
                    except _No:
                        pre = None
                if pre is None:
                    if dg is None:
                        raise _No("no strided form and no digits")
                    tb = _Tables(self, dg, s, k, K, outer_env_t, loop.var)
                    if accs[0][0] == "s":
                        pre, repl = self.forward_tab(tb, accs, alias, written)
                        post = []
                    else:
                        repl, post = self.adjoint_tab(tb, loop, s, accs, alias, written)
                        pre = []
                    pre = tb.loops + pre
                    self._allocs += tb.allocs
                before += pre
                new_body += repl
                after += post
                self.rec["forward" if accs[0][0] == "s" else "adjoint"] += 1
                self.rec["gemms"] += sum(1 for x in pre + post if isinstance(x, (Gemm, GemmT)))
                done += 1
            except _No:
                new_body.append(s)
        if not done:
            raise _No("no inner loop is a contraction")
        return before, For(loop.var, loop.rng, new_body), after

    # -- the table form -------------------------------------------------------------------------------
    def forward_tab(self, tb, accs, alias, written):
        pre, repl = [], []
        for _, acc, e in accs:
            parts = None
            launches = []
            for a, b in self.terms(e):
                a, b = self.resolve(a, alias), self.resolve(b, alias)
                if not (isinstance(a, Ref) and isinstance(b, Ref)):
                    raise _No("a forward term that is not a product of two elements")
                sa, sb = tb.split(a), tb.split(b)
                if sa.array in written or sb.array in written:
                    raise _No("a factor is written in the loop")
                fast = tb.digits[0].name
                X, Y = (sa, sb) if fast in sa.uses else (sb, sa)
                if fast not in X.uses:
                    raise _No("no factor runs over the fastest digit")
                Dm = [d for d in tb.digits if d.name in X.uses]
                Dn = [d for d in tb.digits if d.name not in X.uses]
                if not Y.uses <= {d.name for d in Dn}:
                    raise _No("the factors share a digit")
                if parts is not None and parts != (tuple(d.name for d in Dm), tuple(d.name for d in Dn)):
                    raise _No("the terms split the digits differently")
                parts = (tuple(d.name for d in Dm), tuple(d.name for d in Dn))
                launches.append((X, Y, Dm, Dn))
            _, _, Dm, Dn = launches[0]
            Mm, Mn = tb.size(Dm), tb.size(Dn)
            # T in the loop's own order: T(m, n) at the idx whose digits they are, read as T[idx]
            tname = self.fresh("T")
            pre.append(Assign(Var(tname), Alloc("Float32", Bin("*", Mm, Mn))))
            ro, co = tb.row_table(Dm, tb.place(Dm)), tb.row_table(Dn, tb.place(Dn))
            for j, (X, Y, _, _) in enumerate(launches):
                pre.append(GemmT(tname, _num(0), ro, co, 0 if j == 0 else 1, Mm, Mn, tb.K, X.array, _num(0),
                                 tb.row_table(Dm, X), tb.t_table(X), Y.array, _num(0), tb.t_table(Y), tb.row_table(Dn, Y),
                                 a_km=tb.unit_t(X.inner) > tb.unit_rows(Dm, X.outer),
                                 b_km=tb.unit_t(Y.inner) > tb.unit_rows(Dn, Y.outer)))
            repl.append(Assign(acc, Bin("+", acc, Ref(tname, (Var(tb.var),)))))
        return pre, repl

    def adjoint_tab(self, tb, loop, inner, accs, alias, written):
        inner_ids = {id(x) for x in walk_stmts([inner])}
        rest = [x for x in loop.body if id(x) not in inner_ids]
        touched_elsewhere = self.refs_in(rest)
        allnames = {d.name for d in tb.digits}
        fast = tb.digits[0].name
        vnames, post = {}, []
        D1 = D2 = None
        for _, acc, e in accs:
            sc = tb.split(acc)
            if sc.array in touched_elsewhere:
                raise _No(f"{sc.array} is touched elsewhere in the loop")
            if not sc.inner:
                raise _No("an accumulated array that does not run over the inner index")
            DC = [d for d in tb.digits if d.name in sc.uses]
            DR = [d for d in tb.digits if d.name not in sc.uses]
            for a, b in self.terms(e):
                a, b = self.resolve(a, alias), self.resolve(b, alias)
                if isinstance(a, Var) and isinstance(b, Ref):
                    a, b = b, a
                if not (isinstance(a, Ref) and isinstance(b, Var)):
                    raise _No("an adjoint term that is not an element times a scalar")
                if b.name == tb.k or b.name in alias or self.T.scalars.get(b.name) != "f":
                    raise _No("the scalar factor varies in the inner loop or is not a float")
                sr = tb.split(a)
                if sr.array in written:
                    raise _No("a factor is written in the loop")
                if not sr.inner or sr.uses & sc.uses or (sr.uses | sc.uses) != allnames:
                    raise _No("the accumulation and its factor do not split the digits")
                d1 = [d for d in tb.digits if d.name in (sc.uses if fast in sc.uses else sr.uses)]
                d2 = [d for d in tb.digits if d.name not in {x.name for x in d1}]
                if D1 is not None and [d.name for d in d1] != [d.name for d in D1]:
                    raise _No("the accumulations split the digits differently")
                D1, D2 = d1, d2
                vn = vnames.setdefault(b.name, self.fresh("V"))
                # V in the loop's own order (V[idx]): V(m, s) at the place of C's digits m plus
                # the place of the factor's digits s
                post.append(GemmT(sc.array, _num(0), tb.row_table(DC, sc), tb.t_table(sc), 2, tb.size(DC), tb.K,
                                  tb.size(DR), vn, _num(0), tb.row_table(DC, tb.place(DC)), tb.row_table(DR, tb.place(DR)),
                                  sr.array, _num(0), tb.row_table(DR, sr), tb.t_table(sr),
                                  a_km=tb.unit_rows(DR, tb.place(DR)) > tb.unit_rows(DC, tb.place(DC)),
                                  b_km=tb.unit_rows(DR, sr.outer) > tb.unit_t(sr.inner)))
        repl = [Assign(Ref(vn, (Var(tb.var),)), Var(sname)) for sname, vn in vnames.items()]
        size = Bin("*", tb.size(D1), tb.size(D2))
        tb.allocs += [Assign(Var(vn), Alloc("Float32", size)) for vn in vnames.values()]
        return repl, post

    def forward(self, inner, k, K, env, alias, accs, fl, written, lin, size):
        pre, repl = [], []
        for _, acc, e in accs:
            segs = []
            for a, b in self.terms(e):
                a, b = self.resolve(a, alias), self.resolve(b, alias)
                if not (isinstance(a, Ref) and isinstance(b, Ref)):
                    raise _No("a forward term that is not a product of two elements")
                fa, fb = self.affine(a, env, k, fl), self.affine(b, env, k, fl)
                if {fa.coord, fb.coord} != {fl.iv, fl.jv}:
                    raise _No("the factors do not split the coordinates")
                if fa.array in written or fb.array in written:
                    raise _No("a factor is written in the loop")
                A, B = (fa, fb) if fa.coord == fl.jv else (fb, fa)   # T(j, i): rows j
                segs.append(self.seg(A, B, K))
            tname = self.fresh("T")
            pre.append(Assign(Var(tname), Alloc("Float32", size)))
            pre += self.gemms(tname, _num(0), _num(1), fl.N, False, fl.N, fl.R, segs)
            repl.append(Assign(acc, Bin("+", acc, Ref(tname, (lin,)))))
        return pre, repl

    def adjoint(self, loop, inner, k, K, env, alias, accs, fl, written, lin, size):
        inner_ids = {id(s) for s in walk_stmts([inner])}
        rest = [s for s in loop.body if id(s) not in inner_ids]
        touched_elsewhere = self.refs_in(rest)
        vnames = {}
        repl, post = [], []
        for _, acc, e in accs:
            c = self.affine(acc, env, k, fl)
            if c.coord is None or not c.sk:
                raise _No("an accumulated array that does not run over k and one coordinate")
            if c.array in touched_elsewhere:
                raise _No(f"{c.array} is touched elsewhere in the loop")
            other = fl.iv if c.coord == fl.jv else fl.jv       # summed over
            srange = fl.R if other == fl.iv else fl.N
            # output rows: C's coordinate when its stride there is 1, else k when that is 1
            rows_coord = c.sc == ONE or c.sk != ONE
            segs = []
            for a, b in self.terms(e):
                a, b = self.resolve(a, alias), self.resolve(b, alias)
                if isinstance(a, Var) and isinstance(b, Ref):
                    a, b = b, a
                if not (isinstance(a, Ref) and isinstance(b, Var)):
                    raise _No("an adjoint term that is not an element times a scalar")
                if b.name == k or b.name in alias or self.T.scalars.get(b.name) != "f":
                    raise _No("the scalar factor varies in the inner loop or is not a float")
                fa = self.affine(a, env, k, fl)
                if fa.coord != other or not fa.sk:
                    raise _No("the element factor does not run over k and the summed coordinate")
                if fa.array in written:
                    raise _No("a factor is written in the loop")
                vn = vnames.setdefault(b.name, self.fresh("V"))
                # the factor over (summed index s = `other`, k): km when s is contiguous
                f_km, f_ld = (True, fa.sk) if fa.sc == ONE else ((False, fa.sc) if fa.sk == ONE else (None, None))
                if f_km is None:
                    raise _No(f"{fa.array}: no unit stride")
                if rows_coord:
                    # A(m = C's coordinate, s) = V: V(j, i) = V[(j - 1) + (i - 1) N], so s
                    # contiguous when the coordinate is i;  B(s, n = k) = the factor
                    segs.append(GemmSeg(vn, _num(0), c.coord == fl.iv, fl.N, fa.array, poly_expr(fa.off), f_km,
                                        poly_expr(f_ld), srange))
                else:
                    # A(m = k, s) = the factor;  B(s, n = C's coordinate) = V, s contiguous
                    # when s is j
                    segs.append(GemmSeg(fa.array, poly_expr(fa.off), f_km, poly_expr(f_ld), vn, _num(0),
                                        other == fl.jv, fl.N, srange))
            crange = fl.R if c.coord == fl.iv else fl.N
            if rows_coord:
                M_, N_, sm, sn = crange, K, c.sc, c.sk
            else:
                M_, N_, sm, sn = K, crange, c.sk, c.sc
            post += self.gemms(c.array, poly_expr(c.off), poly_expr(sm), poly_expr(sn), True, M_, N_, segs)
        for sname, vn in vnames.items():
            repl.append(Assign(Ref(vn, (lin,)), Var(sname)))
        allocs = [Assign(Var(vn), Alloc("Float32", size)) for vn in vnames.values()]
        self._allocs += allocs
        return repl, post

    def gemms(self, out, off, sm, sn, acc, M, N, segs):
        """Gemm statements for the segments: two to a launch when they share a layout, the
        first storing (unless acc) and the rest adding."""
        out_stmts = []
        groups = []
        for g in segs:
            if groups and len(groups[-1]) < 2 and (groups[-1][0].a_km, groups[-1][0].b_km) == (g.a_km, g.b_km):
                groups[-1].append(g)
            else:
                groups.append([g])
        for n_, grp in enumerate(groups):
            out_stmts.append(Gemm(out, off, sm, sn, acc or n_ > 0, M, N, grp))
        return out_stmts

    def run(self, exclude: set) -> Func:
        self._allocs = []
        self.pairs = []
        body = []
        for s in self.f.body:
            if isinstance(s, For) and id(s) not in exclude and self.is_parallel(s):
                try:
                    before, loop, after = self.rewrite_loop(s)
                except _No:
                    body.append(s)
                    continue
                body += before + [loop] + after
                self.pairs.append((s, loop))
                self.rec["loops"].append(s.var)
                continue
            body.append(s)
        body = self.reuse(body)
        return Func(self.f.name, self.f.args, self._allocs + body, self.f.annot)

    def reuse(self, body: list) -> list:
        """A forward product computed again with operands unchanged since (the adjoint's
        backward loop recomputes the forward sums): the later loop reads the first product's
        sums, and the second product and its scratch go."""
        groups, j = [], 0
        while j < len(body):     # runs of products into one scratch sums array, first one storing
            g = body[j]
            if isinstance(g, Gemm) and g.out.startswith("__gemm_T") and not g.acc:
                k = j + 1
                while k < len(body) and isinstance(body[k], Gemm) and body[k].out == g.out:
                    k += 1
                groups.append((j, k))
                j = k
            else:
                j += 1
        if len(groups) < 2:
            return body
        sig = lambda g: repr((g.acc, g.M, g.N, g.out_off, g.out_sm, g.out_sn, g.segs))
        drop, rename, avail = set(), {}, {}
        starts = {a: b for a, b in groups}
        j = 0
        while j < len(body):
            if j in starts:
                run = body[j:starts[j]]
                key = tuple(sig(g) for g in run)
                reads = {x for g in run for sg in g.segs for x in (sg.a, sg.b)}
                if key in avail:
                    rename[run[0].out] = avail[key][0]
                    drop |= set(range(j, starts[j]))
                else:
                    avail[key] = (run[0].out, reads)
                j = starts[j]
                continue
            written = self.written_in([body[j]]) | ({body[j].out} if isinstance(body[j], (Gemm, GemmT)) else set())
            avail = {k: v for k, v in avail.items() if not (v[1] & written)}
            j += 1
        if not rename:
            return body
        out = []
        for j, st in enumerate(body):
            if j in drop or (isinstance(st, Assign) and isinstance(st.lhs, Var) and st.lhs.name in rename):
                continue
            _rename_refs(st, rename)
            out.append(st)
        self.rec["gemms"] -= len(drop)
        self.rec["reused"] = len(rename)
        return out


def transform(f: Func, T: Types, is_parallel, retype, host_ints: set | None = None) -> tuple[Func, dict, Types]:
    """(f with its contractions on the matrix cores, a record {forward, adjoint, gemms, loops},
    the rewritten function's types); f, {} and T unchanged when there is none or
    `STADE_LOWER_GEMM=0`.  is_parallel(loop, func, types): the planner's verdict on a loop of
    func; retype(func): the types of a rewritten function.  A rewritten loop that the planner
    would no longer run in parallel is left as written."""
    if os.environ.get("STADE_LOWER_GEMM", "1") == "0":
        return f, {}, T
    if host_ints is None:
        assigned = {s.lhs.name for s in walk_stmts(f.body) if isinstance(s, Assign) and isinstance(s.lhs, Var)}
        host_ints = {a for a in f.args if T.scalars.get(a) == "i" and a not in assigned and a not in T.arrays}
    exclude: set = set()
    while True:
        rw = _Rewriter(f, T, host_ints, lambda loop: is_parallel(loop, f, T))
        g = rw.run(exclude)
        if not rw.rec["gemms"]:
            return f, {}, T
        T2 = retype(g)
        bad = {id(orig) for orig, new in rw.pairs if not is_parallel(new, g, T2)}
        if not bad:
            return g, rw.rec, T2
        exclude |= bad
