"""Owner-computes form of periodic scatters: the general lowering's counterpart of the
reference's level-3 gather (`cgen_gather_loop`, `cgen_gather_periodic_inverse`
/root/reference/src/STADE.jl:7343-7712).

An adjoint loop of a periodic stencil scatters each iteration's contributions into its
neighbours' shadows:

    for idx = 1:n*n                       (or n*n:-1:1)
        i = mod(idx - 1, n) + 1; j = div(idx - 1, n) + 1
        ip = mod(i, n) + 1; ...
        old = unb[idx]; unb[idx] = 0.0
        ub[idx] = ub[idx] + old
        ub[(j - 1) * n + ip] = ub[(j - 1) * n + ip] + 0.1 old
        ...

Run as written on the GPU, every scattered `+=` is an atomic.  Each index map here is a
bijection of 1..N (per coordinate a periodic shift), so the loop can instead run over the
targets: target t takes, for each scattered statement k, the value that iteration
src_k(t) = map_k^-1(t) adds, recomputed from that iteration's own inputs.  This rewrites the
loop into two loops:

  G: for t in the same range: the body as written without its scattered statements and
     without its constant resets of arrays the body reads (those neighbours read them), then,
     per scattered statement k, src_k(t) from t's coordinates shifted back, the statements
     that compute k's value copied with the loop variable bound to src_k(t), and
     `A[t] = A[t] + value`: every write of A at the iteration's own index, no atomics;
  R: for t in the same range: the deferred resets (`unb[t] = 0.0`), in order.

The rewrite applies only where it can be shown exact:
* the loop runs over 1..N (either direction), its body straight-line assignments;
* coordinates are `mod(v - 1, E) + 1` / `div(v - 1, S) + 1` forms of the loop variable v
  (or v itself, in one dimension) whose strides and extents tile 1..N exactly, and every
  scattered index is sum_c (X_c - 1) * S_c + 1 with X_c the coordinate or a periodic shift
  `mod(c + k, E_c) + 1` of it;
* the gathered array is written only by such `A[e] = A[e] + value` statements and not read
  otherwise; the value's statements are single assignments of scalars that read only arrays
  the loop never writes or arrays whose only write is a constant reset after every read, at
  the iteration's own index.
Anything else keeps the loop as written (atomics).
"""
from __future__ import annotations

from .analysis import NotAffine, Types, _add, _freeze, _mul, to_poly
from .syntax import Assign, Bin, Call, For, If, Num, Range, Ref, Var, While, walk_expr


class _No(Exception):
    pass


def _is_num(e, value: int) -> bool:
    return isinstance(e, Num) and e.is_int and int(e.text, 0) == value


def _reads(e) -> set:
    return {x.name for x in walk_expr(e) if isinstance(x, Var)}


def _refs(e) -> list:
    return [x for x in walk_expr(e) if isinstance(x, Ref)]


def _subst(e, m: dict):
    """e with the variables named in m replaced (Var -> expression; Ref names renamed when m
    maps them to a Var)."""
    if isinstance(e, Var):
        return m.get(e.name, e)
    if isinstance(e, Num):
        return e
    if isinstance(e, Ref):
        return Ref(e.name, tuple(_subst(x, m) for x in e.idx))
    if isinstance(e, Bin):
        return Bin(e.op, _subst(e.a, m), _subst(e.b, m))
    if hasattr(e, "op") and hasattr(e, "a") and not hasattr(e, "b"):   # Un
        return type(e)(e.op, _subst(e.a, m))
    if isinstance(e, Call):
        return Call(e.fn, tuple(_subst(x, m) for x in e.args))
    raise _No


def _acc_value(s: Assign):
    """The added value of `A[e] = A[e] + value` (either operand order), else None."""
    if not isinstance(s.lhs, Ref) or not isinstance(s.rhs, Bin) or s.rhs.op != "+":
        return None
    if s.rhs.a == s.lhs:
        return s.rhs.b
    if s.rhs.b == s.lhs:
        return s.rhs.a
    return None


def _poly_eq(p, q) -> bool:
    return _freeze(p) == _freeze(q)


def gather_loop(loop: For, n_loop: int):
    """[G, R] replacing `loop` (R omitted when nothing is deferred), or None."""
    try:
        return _gather(loop, n_loop)
    except (_No, NotAffine, KeyError, ValueError):
        return None


def _gather(loop: For, n_loop: int):
    v, body, r = loop.var, loop.body, loop.rng
    if not body or not all(isinstance(s, Assign) for s in body):
        raise _No
    step = 1 if r.step is None else (int(r.step.text, 0) if isinstance(r.step, Num) and r.step.is_int else 0)
    if step == 1 and _is_num(r.lo, 1):
        N = r.hi
    elif step == -1 and _is_num(r.hi, 1):
        N = r.lo
    else:
        raise _No
    defs: dict[str, list[int]] = {}
    for k, s in enumerate(body):
        if isinstance(s.lhs, Var):
            defs.setdefault(s.lhs.name, []).append(k)
    if _reads(N) & set(defs) or v in defs:
        raise _No
    single = {n for n, ks in defs.items() if len(ks) == 1}
    # index arithmetic is Int: every name polynomial-valued
    names = {v} | set(defs) | _reads(N)
    for s in body:
        for e in ([s.rhs] + (list(s.lhs.idx) if isinstance(s.lhs, Ref) else [])):
            names |= _reads(e)
    T = Types(scalars={n: "i" for n in names})
    pN = to_poly(N, {}, T)
    pv = {(("v", v),): 1}
    # scalars whose definitions are pure index arithmetic (no array element)
    pure = {n for n in single if not _refs(body[defs[n][0]].rhs)}

    def rhs(n):
        return body[defs[n][0]].rhs

    # coordinates: name -> (stride poly, extent poly or None), from v - 1
    env_all = {n: rhs(n) for n in pure}

    def poly(e, keep=()):
        return to_poly(e, {n: x for n, x in env_all.items() if n not in keep}, T)

    vm1 = _add(pv, {(): -1})
    coords: dict[str, tuple] = {}   # name -> (stride poly, extent poly or None, operand expression)
    for n in sorted(pure):
        e = rhs(n)
        if not (isinstance(e, Bin) and e.op == "+" and _is_num(e.b, 1) and isinstance(e.a, Call) and len(e.a.args) == 2):
            continue
        c = e.a
        try:
            if c.fn == "mod" and _poly_eq(poly(c.args[0]), vm1):
                if _poly_eq(poly(c.args[1]), pN):   # mod(v - 1, N) + 1 is v itself
                    continue
                coords[n] = ({(): 1}, poly(c.args[1]), c.args[1])
            elif c.fn == "div" and _poly_eq(poly(c.args[0]), vm1):
                coords[n] = (poly(c.args[1]), None, c.args[1])
        except NotAffine:
            continue
    # shifts: name -> (coordinate, d, extent) with name - 1 = mod((c - 1) + d, extent)
    shifts: dict[str, tuple] = {}
    atoms_keep = set(coords) | {v}
    for n in sorted(pure - set(coords)):
        e = rhs(n)
        if not (isinstance(e, Bin) and e.op == "+" and _is_num(e.b, 1) and isinstance(e.a, Call)
                and e.a.fn == "mod" and len(e.a.args) == 2):
            continue
        try:
            z = poly(e.a.args[0], keep=atoms_keep)
            E = poly(e.a.args[1])
        except NotAffine:
            continue
        for c in list(coords) + [v]:
            rest = _add(z, {(("v", c),): 1}, -1)
            if set(rest) <= {()}:
                shifts[n] = (c, rest.get((), 0) + 1, E, e.a.args[1])
                break
    # the coordinate system: v alone (one dimension) or the coordinates found, tiling 1..N
    if coords:
        order = sorted(coords, key=lambda c: (0 if coords[c][0] == {(): 1} else 1, len(coords[c][0])))
        ext, ext_e, stride_e = {}, {}, {}
        for c in order:
            E, Ee = coords[c][1], coords[c][2]
            if E is None:   # the last coordinate: its extent from its shifts
                es = [s for s in shifts.values() if s[0] == c]
                if not es or not all(_poly_eq(x[2], es[0][2]) for x in es):
                    raise _No
                E, Ee = es[0][2], es[0][3]
                stride_e[c] = coords[c][2]
            ext[c], ext_e[c] = E, Ee
        stride = {}
        acc = {(): 1}
        for c in order:
            if not _poly_eq(coords[c][0], acc):
                raise _No
            stride[c] = acc
            acc = _mul(acc, ext[c])
        # (only two-level decompositions are written back: stride 1 and one div stride)
        if len(order) != 2 or order[1] not in stride_e:
            raise _No
        if not _poly_eq(acc, pN):
            raise _No
        for s_ in shifts.values():
            if s_[0] == v or not _poly_eq(s_[2], ext[s_[0]]):
                raise _No
    else:
        order, ext, stride = [v], {v: pN}, {v: {(): 1}}
        ext_e, stride_e = {v: N}, {}
        for s_ in shifts.values():
            if s_[0] != v or not _poly_eq(s_[2], pN):
                raise _No

    def index_map(e):
        """{coordinate: shift d} if e = sum_c (X_c - 1) S_c + 1, X_c = c or a shift of c (the
        loop variable itself: no shift)."""
        if _poly_eq(poly(e), pv):
            return {c: 0 for c in order}
        p = poly(e, keep=atoms_keep | set(shifts))
        got = {}
        for c in order:
            cands = [c] + [s for s, x in shifts.items() if x[0] == c]
            hit = None
            for a in cands:
                coef = {}
                for m, k in p.items():
                    if ("v", a) in m:
                        rest = list(m)
                        rest.remove(("v", a))
                        coef[tuple(rest)] = coef.get(tuple(rest), 0) + k
                if coef:
                    if hit is not None or not _poly_eq(coef, stride[c]):
                        raise _No
                    hit = a
            if hit is None:
                raise _No
            got[c] = 0 if hit == c else shifts[hit][1]
            p = _add(p, _mul({(("v", hit),): 1}, stride[c]), -1)
        const = {(): 1}
        for c in order:
            const = _add(const, stride[c], -1)
        if not _poly_eq(p, const):
            raise _No
        return got

    def is_own(e) -> bool:
        try:
            return _poly_eq(poly(e), pv)
        except NotAffine:
            return False

    written = {}
    for k, s in enumerate(body):
        if isinstance(s.lhs, Ref):
            written.setdefault(s.lhs.name, []).append(k)
    reads_at = {}
    for k, s in enumerate(body):
        for x in _refs(s.rhs) + [y for i in (s.lhs.idx if isinstance(s.lhs, Ref) else ()) for y in _refs(i)]:
            reads_at.setdefault(x.name, []).append((k, x))
    # gathered arrays: written only by accumulations at recognised maps, at least one shifted
    gathered, scattered = set(), []
    for a, ks in written.items():
        vals = [_acc_value(body[k]) for k in ks]
        if any(x is None for x in vals) or any(len(body[k].lhs.idx) != 1 for k in ks):
            continue
        if any(not (k2 in ks and x == body[k2].lhs) for k2, x in reads_at.get(a, [])):
            continue
        try:
            maps = [index_map(body[k].lhs.idx[0]) for k in ks]
        except (_No, NotAffine):
            continue
        if all(all(d == 0 for d in m.values()) for m in maps):
            continue
        gathered.add(a)
        for k, m in zip(ks, maps):
            if any(d != 0 for d in m.values()):
                scattered.append((k, a, m))
    if not gathered:
        raise _No
    # constant resets of arrays the body reads, after every read, at the own index
    deferred = []
    for a, ks in written.items():
        if a in gathered or a not in reads_at:
            continue
        if len(ks) != 1:
            continue
        s = body[ks[0]]
        if not (isinstance(s.rhs, Num) and len(s.lhs.idx) == 1 and is_own(s.lhs.idx[0])):
            continue
        if all(k < ks[0] and len(x.idx) == 1 and is_own(x.idx[0]) for k, x in reads_at[a]):
            deferred.append(ks[0])
    deferred_arrays = {body[k].lhs.name for k in deferred}
    readonly = {a for a in reads_at if a not in written}
    # G: the body without its scattered statements and deferred resets, then one gathered
    # contribution per scattered statement
    drop = {k for k, _, _ in scattered} | set(deferred)
    g_body = [s for k, s in enumerate(body) if k not in drop]
    for q, (k, a, m) in enumerate(scattered):
        value = _acc_value(body[k])
        # the statements computing the value, in body order (single scalar assignments)
        need, sl = set(_reads(value)), []
        for kk in range(k - 1, -1, -1):
            s = body[kk]
            if isinstance(s.lhs, Var) and s.lhs.name in need:
                if s.lhs.name not in single:
                    raise _No
                sl.append(kk)
                need |= _reads(s.rhs)
        sl.reverse()
        for kk in sl:
            for x in _refs(body[kk].rhs):
                if x.name not in readonly and x.name not in deferred_arrays:
                    raise _No
        for x in _refs(value):
            if x.name not in readonly and x.name not in deferred_arrays:
                raise _No
        if need & {n for n in defs if n not in single}:
            raise _No
        # every body scalar the value reads is computed by the slice, before the statement: a
        # name the body assigns only later carries the previous iteration's value, which the
        # source iteration's recomputation would not reproduce (sums and end-of-iteration
        # resets elsewhere in the body keep their order in the rewritten loop)
        if (need & set(defs)) - {body[kk].lhs.name for kk in sl}:
            raise _No
        tag = f"__g{n_loop}_{q}"
        # the source iteration: t's coordinates shifted back
        src_c = {}
        for c in order:
            d = m[c]
            cv = Var(c)
            if d == 0:
                src_c[c] = cv
            else:
                nm = f"{tag}_{c}"
                g_body.append(Assign(Var(nm), Bin("+", Call("mod", (Bin("-", cv, Num(str(d + 1), True)), ext_e[c])),
                                                  Num("1", True))))
                src_c[c] = Var(nm)
        if coords:
            flat = None
            for c in order:
                term = Bin("-", src_c[c], Num("1", True))
                term = term if c not in stride_e else Bin("*", term, stride_e[c])
                flat = term if flat is None else Bin("+", flat, term)
            src = Bin("+", flat, Num("1", True))
        else:
            src = src_c[v]
        srcn = f"{tag}_src"
        g_body.append(Assign(Var(srcn), src))
        ren = {v: Var(srcn)}
        for kk in sl:
            ren[body[kk].lhs.name] = Var(f"{body[kk].lhs.name}{tag}")
        for kk in sl:
            s = body[kk]
            g_body.append(Assign(Var(f"{s.lhs.name}{tag}"), _subst(s.rhs, ren)))
        own = Ref(a, (Var(v),))
        g_body.append(Assign(own, Bin("+", own, _subst(value, ren))))
    out = [For(v, r, g_body)]
    if deferred:
        out.append(For(v, r, [Assign(Ref(body[k].lhs.name, (Var(v),)), body[k].rhs) for k in deferred]))
    return out


def transform(body: list, counter: list | None = None) -> list:
    """The statements of `body` with every loop that qualifies rewritten (recursively)."""
    counter = counter if counter is not None else [0]
    out = []
    for s in body:
        if isinstance(s, For):
            g = gather_loop(s, counter[0])
            if g is not None:
                counter[0] += 1
                out.extend(g)
                continue
            out.append(For(s.var, s.rng, transform(s.body, counter)))
        elif isinstance(s, If):
            out.append(If([(c, transform(b, counter)) for c, b in s.branches],
                          None if s.orelse is None else transform(s.orelse, counter)))
        elif isinstance(s, While):
            out.append(While(s.cond, transform(s.body, counter)))
        else:
            out.append(s)
    return out
