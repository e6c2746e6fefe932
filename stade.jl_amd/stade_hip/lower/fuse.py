"""Fusion of consecutive parallel loops over the same iterations.

Generated adjoints often run several loops over one index space back to back (the forward
values, the loss, the seed of a shadow; `for k = 1:n*n` then `for k = n*n:-1:1`).  Lowered one
kernel per loop, each re-reads what the previous one wrote.  Two adjacent loops become one
loop whose iteration runs the first body and then the second when that is the same
computation:

* both loops run over the same set of iterations (1:n and n:-1:1 alike) and each is a
  parallel loop on its own;
* every array that either loop writes and both access is accessed, in both, at one index
  expression (the loop variables identified): iteration v of the second loop reads or writes
  only what iteration v of the first wrote or read, so no iteration of one depends on another
  iteration of the other;
* no scalar is written by one body and read or written by the other, and, unless both run in
  the same direction, neither body writes a scalar that is read after them (a value left by
  the last iteration would come from the other end of the range);
* the fused loop is itself a parallel loop (checked by the same classification);
* both bodies are straight-line assignments (a loop with inner loops keeps its own launch
  shape).
Anything else keeps the loops apart.
"""
from __future__ import annotations

from .analysis import NotAffine, Types, _freeze, to_poly
from .syntax import Assign, For, If, Num, Range, Ref, Var, While, stmt_exprs, walk_expr, walk_stmts


def _rename(e, old: str, new: str):
    from .gather import _subst
    return _subst(e, {old: Var(new)})


def _rename_stmt(s, old: str, new: str):
    if isinstance(s, Assign):
        lhs = s.lhs if isinstance(s.lhs, Var) else Ref(s.lhs.name, tuple(_rename(x, old, new) for x in s.lhs.idx))
        if isinstance(lhs, Var) and lhs.name == old:
            raise ValueError("assigns the loop variable")
        return Assign(lhs, _rename(s.rhs, old, new))
    if isinstance(s, For):
        if s.var == old:
            raise ValueError("shadows the loop variable")
        rng = Range(_rename(s.rng.lo, old, new), None if s.rng.step is None else _rename(s.rng.step, old, new),
                    _rename(s.rng.hi, old, new))
        return For(s.var, rng, [_rename_stmt(t, old, new) for t in s.body])
    if isinstance(s, If):
        return If([(_rename(c, old, new), [_rename_stmt(t, old, new) for t in b]) for c, b in s.branches],
                  None if s.orelse is None else [_rename_stmt(t, old, new) for t in s.orelse])
    if isinstance(s, While):
        return While(_rename(s.cond, old, new), [_rename_stmt(t, old, new) for t in s.body])
    raise ValueError("statement kind")


def _span(loop: For, T: Types):
    """(first, last, direction) polynomials of the iteration set, or None."""
    r = loop.rng
    if r.step is None:
        st = 1
    elif isinstance(r.step, Num) and r.step.is_int:
        st = int(r.step.text, 0)
    else:
        return None
    if st not in (1, -1):
        return None
    try:
        lo, hi = _freeze(to_poly(r.lo, {}, T)), _freeze(to_poly(r.hi, {}, T))
    except NotAffine:
        return None
    return (lo, hi, 1) if st == 1 else (hi, lo, -1)


def _scalars(body, arrays: set):
    written, read = set(), set()
    for s in walk_stmts(body):
        if isinstance(s, Assign) and isinstance(s.lhs, Var):
            written.add(s.lhs.name)
        if isinstance(s, For):
            written.add(s.var)
        for e in stmt_exprs(s):
            read |= {x.name for x in walk_expr(e) if isinstance(x, Var) and x.name not in arrays}
    return written, read


def _accesses(body) -> dict:
    out: dict[str, list] = {}
    for s in walk_stmts(body):
        for e in stmt_exprs(s):
            for x in walk_expr(e):
                if isinstance(x, Ref):
                    out.setdefault(x.name, []).append(("r", x))
        if isinstance(s, Assign) and isinstance(s.lhs, Ref):
            out.setdefault(s.lhs.name, []).append(("w", s.lhs))
    return out


def fuse_pair(a: For, b: For, T: Types, after: list, is_parallel) -> For | None:
    """The loop that runs a's body then b's per iteration, or None.  `after`: the statements
    that run after b (for the scalars a value of the last iteration would reach)."""
    from .analysis import _upward_exposed
    # straight-line bodies only: a body with inner loops keeps its own launch shape (the
    # narrow-output form, where each iteration is a wave, measured far slower fused with an
    # elementwise loop)
    if not all(isinstance(s, Assign) for s in a.body + b.body):
        return None
    sa, sb = _span(a, T), _span(b, T)
    if sa is None or sb is None or sa[:2] != sb[:2]:
        return None
    arrays = set(T.arrays)
    if a.var != b.var and any(isinstance(x, Var) and x.name == a.var for s in walk_stmts(b.body)
                              for e in stmt_exprs(s) for x in walk_expr(e)):
        return None   # b reads a scalar named like a's loop variable
    try:
        bbody = b.body if b.var == a.var else [_rename_stmt(s, b.var, a.var) for s in b.body]
    except ValueError:
        return None
    wa, ra = _scalars(a.body, arrays)
    wb, rb = _scalars(bbody, arrays)
    if (wa & (rb | wb)) or (wb & ra):
        return None
    if sa[2] != sb[2] and any(_upward_exposed(after, n) for n in (wa | wb)):
        return None
    acc_a, acc_b = _accesses(a.body), _accesses(bbody)
    for x in set(acc_a) & set(acc_b):
        uses = acc_a[x] + acc_b[x]
        if not any(k == "w" for k, _ in uses):
            continue
        if len({repr(r.idx) for _, r in uses}) != 1:
            return None
    fused = For(a.var, a.rng, list(a.body) + list(bbody))
    return fused if is_parallel(fused) else None


def transform(body: list, T: Types, is_parallel, after: list | None = None) -> list:
    """body with adjacent fusable loops fused (recursively in nested blocks); `after`: the
    statements that run after this block (an enclosing loop's body included)."""
    after = after or []
    out: list = []
    for k, s in enumerate(body):
        rest = body[k + 1:] + after
        if isinstance(s, For):
            s = For(s.var, s.rng, transform(s.body, T, is_parallel, rest + s.body))
            prev = out[-1] if out else None
            if isinstance(prev, For) and is_parallel(prev) and is_parallel(s):
                f = fuse_pair(prev, s, T, rest, is_parallel)
                if f is not None:
                    out[-1] = f
                    continue
            out.append(s)
        elif isinstance(s, If):
            out.append(If([(c, transform(b, T, is_parallel, rest)) for c, b in s.branches],
                          None if s.orelse is None else transform(s.orelse, T, is_parallel, rest)))
        elif isinstance(s, While):
            out.append(While(s.cond, transform(s.body, T, is_parallel, rest + s.body)))
        else:
            out.append(s)
    return out
