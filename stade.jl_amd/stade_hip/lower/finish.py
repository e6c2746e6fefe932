"""Kernel finishing passes of the general lowering, on the syntax tree of one generated function.

The reference runs these on what it emits for a GPU (`stade_gpu` /root/reference/src/STADE.jl:
18522-18560, with `stade_amdgpu_file`'s defaults `inbounds = true, dead_scalars = true`):

* `dead_pops` -- `cgen_dead_pops` (12356): a restore of a scalar from one of STADE's own stacks
  (`s = s_stack[k]`) whose value the code overwrites before it reads it is deleted, and then
  every store to such a stack whose slot no remaining read takes (the index formula compared
  after substituting the scalars' definitions, `cgen_dp_stores` 12343) is deleted too.
* `merge_accum` -- `cgen_merge_accum` (18144, `cgen_merge_accum_block` 18102): two additions
  into the same element, `A[e] = A[e] + e1` and later `A[e] = A[e] + e2`, with only scalar
  assignments between them that leave A, the index and e1 alone, become one
  `A[e] = A[e] + (e1 + e2)` at the second one's place (one atomic instead of two where the
  element is shared).
* `dead_scalars` -- `cgen_dead_scalars` (12369) over `cgen_dead_walk` (12151): a backward
  liveness walk that deletes a scalar assignment whose target no later statement reads and
  whose right side has no effect (`cgen_dead_pure_calls` 12126; an array read only under
  `inbounds`, where it cannot raise).  The reference runs it per kernel; the lowering keeps a
  function's scalars in one device frame, so it runs over the whole function, with what the
  function returns as its live-out set.

`inbounds` itself (`cgen_inbounds_wrap` 12376) is a code-generation switch of hipgen: without
it every access is checked and an index out of range is reported as a BoundsError.
"""
from __future__ import annotations

from .syntax import (Alloc, Assign, Bin, Break, Call, Continue, ExprStmt, For, Func, If, Num, Ref, Return, Tup, Un,
                     Var, While, walk_expr, walk_stmts)

# calls with no effect other than their value (`cgen_dead_pure_calls` /root/reference/src/STADE.jl:12126)
PURE_CALLS = {"div", "mod", "rem", "fld", "cld", "abs", "sqrt", "exp", "log", "log10", "sin", "cos", "tan", "asin",
              "acos", "atan", "sinh", "cosh", "tanh", "max", "min", "sign", "floor", "ceil", "trunc", "ifelse"}


def names(e) -> set[str]:
    """Every variable and array name an expression mentions."""
    out = set()
    for x in walk_expr(e):
        if isinstance(x, Var):
            out.add(x.name)
        elif isinstance(x, Ref):
            out.add(x.name)
    return out


def stmt_names(s) -> set[str]:
    """Every name a statement mentions, nested statements included."""
    out = set()
    if isinstance(s, Assign):
        out |= names(s.rhs) | names(s.lhs)
    elif isinstance(s, (For,)):
        out |= {s.var} | names(s.rng)
    elif isinstance(s, While):
        out |= names(s.cond)
    elif isinstance(s, If):
        for c, _ in s.branches:
            out |= names(c)
    elif isinstance(s, Return) and s.value is not None:
        out |= names(s.value)
    elif isinstance(s, ExprStmt):
        out |= names(s.e)
    for b in _blocks(s):
        for t in b:
            out |= stmt_names(t)
    return out


def _blocks(s):
    if isinstance(s, (For, While)):
        return [s.body]
    if isinstance(s, If):
        return [b for _, b in s.branches] + ([s.orelse] if s.orelse is not None else [])
    return []


def pure(e, refs_ok: bool) -> bool:
    """`cgen_dead_pure` (12130): no effect besides the value."""
    if isinstance(e, (Num, Var)):
        return True
    if isinstance(e, Ref):
        return refs_ok and all(pure(i, refs_ok) for i in e.idx)
    if isinstance(e, (Bin, Un)):
        return all(pure(x, refs_ok) for x in ((e.a, e.b) if isinstance(e, Bin) else (e.a,)))
    if isinstance(e, Call):
        return e.fn in PURE_CALLS and all(pure(a, refs_ok) for a in e.args)
    return False


# ---------------------------------------------------------------------------------------------
# dead scalars: backward liveness
# ---------------------------------------------------------------------------------------------

def _walk(stmts, live_out: set, refs_ok: bool, droppable, loop_ctx):
    """(statements kept, live-in).  loop_ctx: (live at the innermost loop's exit, live at its
    head) for `break` and `continue`, or None outside loops."""
    live = set(live_out)
    out = []
    for s in reversed(stmts):
        if isinstance(s, Assign) and isinstance(s.lhs, Var):
            v = s.lhs.name
            if v not in live and pure(s.rhs, refs_ok) and (droppable is None or droppable(v, s.rhs)):
                continue
            live.discard(v)
            live |= names(s.rhs)
            out.append(s)
        elif isinstance(s, (For, While)):
            head_names = names(s.rng) if isinstance(s, For) else names(s.cond)
            head = live | head_names
            while True:
                _, bin_ = _walk(s.body, head, refs_ok, droppable, (live, head))
                if isinstance(s, For):
                    bin_ = bin_ - {s.var}
                nh = live | head_names | bin_
                if nh == head:
                    break
                head = nh
            nb, _ = _walk(s.body, head, refs_ok, droppable, (live, head))
            out.append(For(s.var, s.rng, nb) if isinstance(s, For) else While(s.cond, nb))
            live = head
        elif isinstance(s, If):
            nl = set()
            brs = []
            for c, b in s.branches:
                nb, bl = _walk(b, live, refs_ok, droppable, loop_ctx)
                brs.append((c, nb))
                nl |= bl | names(c)
            if s.orelse is not None:
                ne, el = _walk(s.orelse, live, refs_ok, droppable, loop_ctx)
                nl |= el
            else:
                ne = None
                nl |= live
            out.append(If(brs, ne))
            live = nl
        elif isinstance(s, Break):
            out.append(s)
            live = set(loop_ctx[0]) if loop_ctx else set(live)
        elif isinstance(s, Continue):
            out.append(s)
            live = set(loop_ctx[1]) if loop_ctx else set(live)
        elif isinstance(s, Return):
            out.append(s)
            live = names(s.value) if s.value is not None else set()
        else:
            # an element store, an expression statement: everything it mentions stays live
            live |= stmt_names(s)
            out.append(s)
    out.reverse()
    return out, live


def dead_scalars(body: list, refs_ok: bool) -> list:
    """The body without its dead scalar assignments (one walk: a deleted statement adds no
    reads, so what fed it is found dead in the same sweep, as `cgen_dead_scalars` notes)."""
    return _walk(body, set(), refs_ok, None, None)[0]


# ---------------------------------------------------------------------------------------------
# merged accumulations
# ---------------------------------------------------------------------------------------------

def _accum(s):
    """(lhs Ref, added value) of `A[e] = A[e] + v`, else None (`cgen_accum_parts` 18094)."""
    if isinstance(s, Assign) and isinstance(s.lhs, Ref) and isinstance(s.rhs, Bin) and s.rhs.op == "+" \
            and s.rhs.a == s.lhs:
        return s.lhs, s.rhs.b
    return None


def merge_block(stmts: list) -> tuple[list, int]:
    out = list(stmts)
    merged = 0
    changed = True
    while changed:
        changed = False
        for i in range(len(out)):
            p1 = _accum(out[i])
            if p1 is None:
                continue
            lhs, e1 = p1
            arr = lhs.name
            syms1 = names(lhs) | names(e1)
            k = i + 1
            while k < len(out):
                st = out[k]
                p2 = _accum(st)
                if p2 is not None and p2[0] == lhs:
                    if arr not in names(p2[1]):
                        out[k] = Assign(lhs, Bin("+", lhs, Bin("+", e1, p2[1])))
                        del out[i]
                        changed = True
                        merged += 1
                    break
                # between the two: only a scalar assignment that leaves the array, the index
                # and e1 alone
                if not (isinstance(st, Assign) and isinstance(st.lhs, Var)):
                    break
                if st.lhs.name in syms1 or arr in names(st.rhs):
                    break
                k += 1
            if changed:
                break
    return out, merged


def merge_accum(body: list, counter: list | None = None) -> list:
    counter = counter if counter is not None else [0]
    out = []
    for s in body:
        if isinstance(s, For):
            s = For(s.var, s.rng, merge_accum(s.body, counter))
        elif isinstance(s, While):
            s = While(s.cond, merge_accum(s.body, counter))
        elif isinstance(s, If):
            s = If([(c, merge_accum(b, counter)) for c, b in s.branches],
                   None if s.orelse is None else merge_accum(s.orelse, counter))
        out.append(s)
    out, n = merge_block(out)
    counter[0] += n
    return out


# ---------------------------------------------------------------------------------------------
# dead pops, and the stack stores nothing reads then
# ---------------------------------------------------------------------------------------------

def stack_params(f: Func, allocated: set[str]) -> set[str]:
    """The function's stack parameters (`cgen_dead_pops_stacks` 12213): a parameter that an
    `initstacks_*` of the file allocates, or the HVP's `<stack>_d` of one."""
    return {a for a in f.args if a in allocated or (a.endswith("_d") and a[:-2] in allocated)}


class _Canon:
    """Index formulas with every scalar replaced by its definition, in program order
    (`cgen_dp_canon` 12270): a scalar assigned in a loop or a branch is a fresh token after it,
    and so is one a loop body assigns, inside the body."""

    def __init__(self, stacks):
        self.stacks = stacks
        self.ctr = 0
        self.stores: set = set()
        self.reads: set = set()
        self.bad: set = set()
        self.eligible: set = set()
        self.drop = False
        self.dropped = 0
        self.lost: set = set()

    def token(self):
        self.ctr += 1
        return Var(f"__dp{self.ctr}")

    def subst(self, e, env):
        if isinstance(e, Var):
            return env.get(e.name, e)
        if isinstance(e, Ref):
            return Ref(e.name, tuple(self.subst(i, env) for i in e.idx))
        if isinstance(e, Bin):
            return Bin(e.op, self.subst(e.a, env), self.subst(e.b, env))
        if isinstance(e, Un):
            return Un(e.op, self.subst(e.a, env))
        if isinstance(e, Call):
            return Call(e.fn, tuple(self.subst(a, env) for a in e.args))
        if isinstance(e, Tup):
            return Tup(tuple(self.subst(a, env) for a in e.items))
        return e

    def canon(self, e, env):
        c = self.subst(e, env)
        return self.token() if sum(1 for _ in walk_expr(c)) > 4000 else c

    def note_reads(self, e, env):
        if isinstance(e, Var):
            if e.name in self.stacks:
                self.bad.add(e.name)
            return
        if isinstance(e, Ref) and e.name in self.stacks:
            if len(e.idx) == 1:
                self.reads.add((e.name, repr(self.canon(e.idx[0], env))))
            else:
                self.bad.add(e.name)
            for i in e.idx:
                self.note_reads(i, env)
            return
        if isinstance(e, Ref):
            for i in e.idx:
                self.note_reads(i, env)
            return
        if isinstance(e, Bin):
            self.note_reads(e.a, env)
            self.note_reads(e.b, env)
        elif isinstance(e, Un):
            self.note_reads(e.a, env)
        elif isinstance(e, Call):
            for a in e.args:
                self.note_reads(a, env)
        elif isinstance(e, Tup):
            for a in e.items:
                self.note_reads(a, env)
        elif isinstance(e, Alloc) and e.n is not None:
            self.note_reads(e.n, env)

    def block(self, stmts, env):
        out = []
        for s in stmts:
            r = self.stmt(s, env)
            if r is not None:
                out.append(r)
        return out

    def stmt(self, s, env):
        if isinstance(s, Assign):
            self.note_reads(s.rhs, env)
            if isinstance(s.lhs, Ref):
                for i in s.lhs.idx:
                    self.note_reads(i, env)
                if s.lhs.name in self.stacks:
                    if len(s.lhs.idx) != 1:
                        self.bad.add(s.lhs.name)
                    else:
                        key = (s.lhs.name, repr(self.canon(s.lhs.idx[0], env)))
                        self.stores.add(key)
                        if self.drop and s.lhs.name in self.eligible and key not in self.reads:
                            self.dropped += 1
                            self.lost.add(s.lhs.name)
                            return None
            else:
                env[s.lhs.name] = self.canon(s.rhs, env)
            return s
        if isinstance(s, (For, While)):
            self.note_reads(s.rng if isinstance(s, For) else s.cond, env)
            assigned = _assigned(s)
            inner = dict(env)
            for v in assigned:
                inner[v] = self.token()
            if isinstance(s, For):
                inner.pop(s.var, None)
            body = self.block(s.body, inner)
            for v in assigned:
                env[v] = self.token()
            return For(s.var, s.rng, body) if isinstance(s, For) else While(s.cond, body)
        if isinstance(s, If):
            for c, _ in s.branches:
                self.note_reads(c, env)
            assigned = _assigned(s)
            brs = [(c, self.block(b, dict(env))) for c, b in s.branches]
            orelse = None if s.orelse is None else self.block(s.orelse, dict(env))
            for v in assigned:
                env[v] = self.token()
            return If(brs, orelse)
        if isinstance(s, Return) and s.value is not None:
            self.note_reads(s.value, env)
        elif isinstance(s, ExprStmt):
            self.note_reads(s.e, env)
        return s


def _assigned(s) -> set[str]:
    out = set()
    for t in walk_stmts([s]):
        if isinstance(t, Assign) and isinstance(t.lhs, Var):
            out.add(t.lhs.name)
        elif isinstance(t, For):
            out.add(t.var)
    return out


def dead_pops(body: list, stacks: set[str]) -> tuple[list, int, set[str]]:
    """(body, restores deleted, stacks that lost stores)."""
    if not stacks:
        return body, 0, set()

    def restore(v, rhs):
        return isinstance(rhs, Ref) and rhs.name in stacks and len(rhs.idx) == 1
    before = sum(1 for _ in walk_stmts(body))
    kept, _ = _walk(body, set(), True, restore, None)
    n_restores = before - sum(1 for _ in walk_stmts(kept))
    c = _Canon(stacks)
    c.block(kept, {})
    for k in stacks:
        if k not in c.bad and all(r in c.stores for r in c.reads if r[0] == k):
            c.eligible.add(k)
    c2 = _Canon(stacks)
    c2.reads, c2.eligible, c2.drop = c.reads, c.eligible, True
    out = c2.block(kept, {})
    return out, n_restores, c2.lost


def finish(f: Func, stacks_allocated: set[str], inbounds: bool = True, dead: bool = True,
           merge: bool = True) -> tuple[Func, dict]:
    """The passes in the reference's order (dead pops, merged accumulations, then dead scalars),
    with a record of what each did."""
    body = f.body
    rec = {"dead_restores": 0, "dead_stacks": [], "merged": 0, "dead_scalars": 0}
    if dead:
        body, rec["dead_restores"], lost = dead_pops(body, stack_params(f, stacks_allocated))
        rec["dead_stacks"] = sorted(lost)
    if merge:
        cnt = [0]
        body = merge_accum(body, cnt)
        rec["merged"] = cnt[0]
    if dead:
        n0 = sum(1 for _ in walk_stmts(body))
        body = dead_scalars(body, refs_ok=inbounds)
        rec["dead_scalars"] = n0 - sum(1 for _ in walk_stmts(body))
    return Func(f.name, f.args, body, f.annot), rec
