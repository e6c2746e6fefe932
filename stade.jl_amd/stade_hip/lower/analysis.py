"""Analysis for the general lowering: types, and which loops may run one iteration per GPU
thread.

Types follow the four shapes of STADE's own inference (`shape_infer`
/root/reference/src/STADE.jl:936): Float, Int, Array{Float}, Array{Int}, decided from use: an
index position, a range bound or a `div`/`mod` operand makes an Int; an array whose element
lands in such a position is an Int array.  Arrays declared `Vector{Int64}` are Int arrays.

Loop classification is the GPU half of `cgen_body` (/root/reference/src/STADE.jl:10409-10640),
redesigned: a `for` loop runs one iteration per thread when every scalar it assigns is
iteration-private (defined before use, or reset to a constant at the end of every
iteration, `agen_backward_assign`'s `xb = 0.0`, 6605-6656) or a sum (`s = s + e`), and
every array it writes is either owned (one element per iteration: all accesses at one index
expression, injective in the loop variable, `cgen_expr_injective_ok` 11148-11158) or only
accumulated (`A[e] = A[e] + t`, the adjoint's scatter, `cgen_device_assign` 11941-11969).
Accumulations at indices that are not injective become atomics (wave-aggregated when a wave
shares the index, `11834-11922`; LDS-privatised for small targets, `11576-11832`).
Anything else runs in order on one GPU thread, which keeps Julia's sequential semantics.
"""
from __future__ import annotations

from dataclasses import dataclass, field

from .syntax import (Alloc, Assign, Bin, Break, Call, Continue, ExprStmt, For, Func, Gemm, GemmT, If, LowerError, Num,
                     Range, Ref, Return, Tup, Un, Var, While, children, stmt_exprs, sub_blocks, walk_expr, walk_stmts)

FLOAT_FNS = {"exp", "log", "tanh", "sin", "cos", "tan", "sqrt", "sinh", "cosh", "atan", "asin", "acos", "log10", "log2",
             "exp2", "expm1", "log1p", "cbrt", "float", "Float64", "Float32", "inv"}
INT_FNS = {"div", "mod", "rem", "fld", "cld", "length", "size", "Int", "Int64"}
POLY_FNS = {"abs", "max", "min", "sign", "ifelse", "floor", "ceil", "round", "trunc"}


@dataclass
class Types:
    arrays: dict = field(default_factory=dict)       # name -> 'f' | 'i'
    ndim: dict = field(default_factory=dict)         # name -> number of indices used (>= 1)
    scalars: dict = field(default_factory=dict)      # name -> 'f' | 'i' | 'b'
    allocs: dict = field(default_factory=dict)       # local array name -> Alloc

    def etype(self, e) -> str:
        """'f', 'i' or 'b' of an expression (arrays as a whole: 'A')."""
        if isinstance(e, Num):
            if e.text in ("true", "false"):
                return "b"
            return "i" if e.is_int else "f"
        if isinstance(e, Var):
            if e.name in self.arrays:
                return "A"
            return self.scalars.get(e.name, "f")
        if isinstance(e, Ref):
            return self.arrays.get(e.name, "f")
        if isinstance(e, Bin):
            if e.op in ("==", "!=", "<", ">", "<=", ">=", "&&", "||"):
                return "b"
            ta, tb = self.etype(e.a), self.etype(e.b)
            if e.op == "/":
                return "f"
            if e.op == "^":
                return "i" if ta == "i" and tb == "i" else "f"
            return "f" if "f" in (ta, tb) else "i"
        if isinstance(e, Un):
            return "b" if e.op == "!" else self.etype(e.a)
        if isinstance(e, Call):
            fn = e.fn
            if fn in ("length", "size", "Int", "Int64"):
                return "i"
            if fn in ("div", "mod", "rem", "fld", "cld"):
                return "f" if any(self.etype(a) == "f" for a in e.args) else "i"
            if fn in FLOAT_FNS:
                return "f"
            if fn in ("floor", "ceil", "round", "trunc") and len(e.args) == 2:
                return "i"   # floor(Int, x)
            if fn == "ifelse":
                return "f" if "f" in (self.etype(e.args[1]), self.etype(e.args[2])) else self.etype(e.args[1])
            if fn in POLY_FNS:
                return "f" if any(self.etype(a) == "f" for a in e.args) else "i"
            raise LowerError(f"call to unsupported function {fn}")
        raise LowerError(f"cannot type {e!r}")


def _int_context(f: Func) -> tuple[set, set]:
    """(scalar names, array names whose elements) appear where Julia needs an Int."""
    names, arrays = set(), set()

    def mark(e):
        for x in walk_expr(e):
            if isinstance(x, Var):
                names.add(x.name)
            elif isinstance(x, Ref):
                arrays.add(x.name)

    for s in walk_stmts(f.body):
        for e in stmt_exprs(s):
            for x in walk_expr(e):
                if isinstance(x, Ref):
                    for i in x.idx:
                        mark(i)
                elif isinstance(x, Range):
                    for y in (x.lo, x.step, x.hi):
                        if y is not None:
                            mark(y)
                elif isinstance(x, Call) and x.fn in ("div", "mod", "rem", "fld", "cld") and len(x.args) == 2:
                    # both operands of an integer division taken as Ints when they read no float
                    pass
                elif isinstance(x, Alloc) and x.n is not None:
                    mark(x.n)
        if isinstance(s, Assign) and isinstance(s.lhs, Ref):
            for i in s.lhs.idx:
                mark(i)
        if isinstance(s, For):
            names.add(s.var)
    return names, arrays


def infer_types(f: Func, arg_types: dict | None = None, precision: str = "f64") -> Types:
    """Types of every name of f.  arg_types: caller's kinds ('f', 'i', 'Af', 'Ai') by name."""
    T = Types()
    arg_types = dict(arg_types or {})
    # arrays: indexed names, allocated names, names passed to length / size
    for s in walk_stmts(f.body):
        for e in stmt_exprs(s):
            for x in walk_expr(e):
                if isinstance(x, Ref):
                    T.ndim[x.name] = max(T.ndim.get(x.name, 1), len(x.idx))
                    T.arrays.setdefault(x.name, "f")
                if isinstance(x, Call) and x.fn in ("length", "size") and x.args and isinstance(x.args[0], Var):
                    T.arrays.setdefault(x.args[0].name, "f")
                    T.ndim.setdefault(x.args[0].name, 1)
        if isinstance(s, (Gemm, GemmT)):   # (a contraction's operands and output are float arrays)
            names = [s.out] + ([x for g in s.segs for x in (g.a, g.b)] if isinstance(s, Gemm) else [s.a, s.b])
            for nm in names:
                T.arrays.setdefault(nm, "f")
                T.ndim.setdefault(nm, 1)
        if isinstance(s, Assign):
            if isinstance(s.lhs, Ref):
                T.ndim[s.lhs.name] = max(T.ndim.get(s.lhs.name, 1), len(s.lhs.idx))
                T.arrays.setdefault(s.lhs.name, "f")
            if isinstance(s.rhs, Alloc) and isinstance(s.lhs, Var):
                T.arrays[s.lhs.name] = "i" if s.rhs.eltype == "Int64" else "f"
                T.ndim.setdefault(s.lhs.name, 1)
                T.allocs[s.lhs.name] = s.rhs
    for a, k in arg_types.items():
        if k in ("Af", "Ai"):
            T.arrays[a] = "i" if k == "Ai" else "f"
            T.ndim.setdefault(a, 1)
        elif a in T.arrays:
            raise LowerError(f"argument {a} is indexed but declared a scalar")
    int_names, int_arrays = _int_context(f)
    # an array whose element is assigned to a name Julia needs as an Int is an Int array
    # (`i_l = lab[i_s]` with i_l an index); likewise a name assigned such an element
    changed = True
    while changed:
        changed = False
        for s in walk_stmts(f.body):
            if isinstance(s, Assign) and isinstance(s.lhs, Var) and s.lhs.name in int_names:
                # the value flows into an Int: its operands are Ints (an index inside a
                # reference is one already)
                stack = [s.rhs]
                while stack:
                    x = stack.pop()
                    if isinstance(x, Ref):
                        if x.name not in int_arrays:
                            int_arrays.add(x.name)
                            changed = True
                        continue
                    if isinstance(x, Var) and x.name not in int_names:
                        int_names.add(x.name)
                        changed = True
                    if isinstance(x, Call) and x.fn in ("length", "size"):
                        continue
                    stack.extend(children(x))
    for a in int_arrays:
        if a in T.arrays and arg_types.get(a) != "Af":
            T.arrays[a] = "i"
    # a shadow or tangent argument has its primal's shape even where the body never indexes it
    # (an input the loss does not depend on): the generated signatures follow each float
    # argument with its shadow (`agen_signature_args` /root/reference/src/STADE.jl:3455-3464,
    # x, xb), tangent (`tgen_signature_args` 3306-3315, x, xd) and HVP pair (`hvp_emit`
    # 6750-6756, xd, xbd)
    for a in f.args:
        if a in T.arrays or arg_types.get(a) in ("f", "i"):
            continue
        for suf in ("bd", "b", "d"):
            p0 = a[:-len(suf)]
            if a.endswith(suf) and p0 in f.args and T.arrays.get(p0) == "f":
                T.arrays[a] = "f"
                T.ndim[a] = T.ndim.get(p0, 1)
                break
    # scalars: fixed point over assignments; a name in an Int context, or assigned only Ints, is an Int
    assigns: dict[str, list] = {}
    for s in walk_stmts(f.body):
        if isinstance(s, Assign) and isinstance(s.lhs, Var) and not isinstance(s.rhs, Alloc):
            assigns.setdefault(s.lhs.name, []).append(s.rhs)
    names = set(assigns) | {a for a in f.args if a not in T.arrays} | {s.var for s in walk_stmts(f.body) if isinstance(s, For)}
    # arguments: from the caller's kinds, else Int where Julia needs an Int; locals start as
    # Int and widen to Float when an assignment is Float (monotone, so the iteration ends)
    for a in names:
        if a in T.arrays:
            continue
        k = arg_types.get(a)
        if a in f.args:
            T.scalars[a] = k if k in ("f", "i") else ("i" if a in int_names else "f")
        else:
            T.scalars[a] = "i"
    loopvars = {s.var for s in walk_stmts(f.body) if isinstance(s, For)}
    for v in loopvars:
        T.scalars[v] = "i"
    for _ in range(2 * len(names) + 4):
        changed = False
        for a, rhss in assigns.items():
            if a in T.arrays or a in loopvars or arg_types.get(a) in ("f", "i"):
                continue
            ts = {T.etype(r) for r in rhss}
            want = "b" if ts == {"b"} else ("f" if "f" in ts else "i")
            cur = T.scalars.get(a)
            if cur == "f" or cur == want:
                continue
            T.scalars[a] = want
            changed = True
        if not changed:
            break
    for a in int_names:
        if T.scalars.get(a) == "f" and a not in T.arrays:
            raise LowerError(f"{a} is used as an index or bound but holds a float")
    return T


# ------------------------------------------------------------------------------------------
# integer expressions in normal form (polynomials over atoms), for injectivity
# ------------------------------------------------------------------------------------------
# A polynomial is a dict {monomial: coefficient}; a monomial a sorted tuple of atoms; an atom
# ('v', name) or ('div', X, N) / ('mod', X, N) with X, N polynomials frozen as sorted tuples.

def _freeze(p: dict) -> tuple:
    return tuple(sorted((m, c) for m, c in p.items() if c != 0))


def _thaw(t: tuple) -> dict:
    return {m: c for m, c in t}


def _add(p, q, s=1):
    r = dict(p)
    for m, c in q.items():
        r[m] = r.get(m, 0) + s * c
        if r[m] == 0:
            del r[m]
    return r


def _mul(p, q):
    r = {}
    for m1, c1 in p.items():
        for m2, c2 in q.items():
            m = tuple(sorted(m1 + m2))
            r[m] = r.get(m, 0) + c1 * c2
            if r[m] == 0:
                del r[m]
    return r


class NotAffine(Exception):
    pass


def to_poly(e, env: dict, types: Types) -> dict:
    """Polynomial of an Int expression; env substitutes iteration-private Int scalars by
    their defining expressions.  Raises NotAffine for anything else."""
    if isinstance(e, Num):
        if not e.is_int:
            raise NotAffine
        return {(): int(e.text, 0)} if int(e.text, 0) else {}
    if isinstance(e, Var):
        if e.name in env:
            return to_poly(env[e.name], env, types)
        if types.scalars.get(e.name) != "i":
            raise NotAffine
        return {(("v", e.name),): 1}
    if isinstance(e, Bin) and e.op in ("+", "-", "*"):
        a, b = to_poly(e.a, env, types), to_poly(e.b, env, types)
        return _add(a, b) if e.op == "+" else (_add(a, b, -1) if e.op == "-" else _mul(a, b))
    if isinstance(e, Un) and e.op == "-":
        return _add({}, to_poly(e.a, env, types), -1)
    if isinstance(e, Call) and e.fn in ("div", "mod") and len(e.args) == 2:
        x, n = to_poly(e.args[0], env, types), to_poly(e.args[1], env, types)
        return {(("div" if e.fn == "div" else "mod", _freeze(x), _freeze(n)),): 1}
    if isinstance(e, Call) and e.fn in ("length", "size"):
        return {(("v", f"{e.fn}({','.join(_key(a) for a in e.args)})"),): 1}
    raise NotAffine


def _key(e) -> str:
    if isinstance(e, Var):
        return e.name
    if isinstance(e, Num):
        return e.text
    raise NotAffine


def fold_divmod(p: dict) -> tuple[dict, list]:
    """Apply n * div(x, n) + mod(x, n) = x wherever both terms appear with the same
    coefficient.  Returns the folded polynomial and the conditions (x, n) it assumed: the
    identity holds for x >= 0, n > 0 (Julia's div truncates and mod floors)."""
    conds = []
    changed = True
    while changed:
        changed = False
        for m, c in list(p.items()):
            mods = [a for a in m if a[0] == "mod"]
            if len(m) != 1 or not mods:
                continue
            _, X, N = mods[0]
            n = _thaw(N)
            d_atom = ("div", X, N)
            # the matching term: c * n * div(x, n)
            want = _mul({(d_atom,): c}, n)
            if all(p.get(mm) == cc for mm, cc in want.items()):
                for mm in want:
                    del p[mm]
                del p[m]
                p = _add(p, _mul({(): c}, _thaw(X)))
                conds.append((_thaw(X), n))
                changed = True
                break
    return p, conds


def depends_on(p: dict, name: str) -> bool:
    def atom_dep(a):
        if a[0] == "v":
            return a[1] == name
        return depends_on(_thaw(a[1]), name) or depends_on(_thaw(a[2]), name)
    return any(atom_dep(a) for m in p for a in m)


def linear_in(p: dict, name: str):
    """(coefficient polynomial, rest) with p = coeff * name + rest, coeff and rest free of
    name; None if p is not of that form."""
    coef, rest = {}, {}
    v = ("v", name)
    for m, c in p.items():
        k = sum(1 for a in m if a == v)
        others = tuple(a for a in m if a != v)
        if k == 0:
            if depends_on({m: c}, name):
                return None
            rest[m] = c
        elif k == 1:
            if depends_on({others: c}, name):
                return None
            coef[others] = coef.get(others, 0) + c
        else:
            return None
    return {m: c for m, c in coef.items() if c}, rest


# ------------------------------------------------------------------------------------------
# loop classification
# ------------------------------------------------------------------------------------------

@dataclass
class ArrayUse:
    name: str
    kind: str                  # 'read' | 'owned' | 'acc' | 'atomic'
    index: object = None       # the common index expression (owned / injective acc; hoisted atomic)
    hoist: bool = False        # atomic at one index that no iteration changes: summed in a register


@dataclass
class ParallelLoop:
    loop: For
    private: list              # scalars private to an iteration (assigned in the body)
    reset: dict                # scalar -> constant it holds at the start of iterations after the first
    reductions: dict           # scalar -> '+' (sum of the body's s = s + e terms)
    arrays: dict               # name -> ArrayUse
    guards: list               # (kind, poly...) conditions the host checks before using this form
    live_out: list             # private scalars read after the loop (written back by the last iteration)
    reads: set                 # scalars read (frame values) in the loop


def _reads_of(e) -> set:
    return {x.name for x in walk_expr(e) if isinstance(x, Var)}


def _assigned(body) -> set:
    out = set()
    for s in walk_stmts(body):
        if isinstance(s, Assign) and isinstance(s.lhs, Var):
            out.add(s.lhs.name)
        if isinstance(s, For):
            out.add(s.var)
    return out


def _upward_exposed(body, name: str) -> bool:
    """Is `name` read in an iteration before that iteration assigns it (on some path)?"""
    def block(stmts, assigned: bool) -> tuple[bool, bool]:
        # returns (exposed, definitely assigned after the block)
        for s in stmts:
            reads = set()
            for e in stmt_exprs(s):
                reads |= _reads_of(e)
            if name in reads and not assigned:
                return True, assigned
            if isinstance(s, Assign) and isinstance(s.lhs, Var) and s.lhs.name == name:
                assigned = True
            elif isinstance(s, If):
                outs = []
                for _, b in s.branches:
                    ex, a = block(b, assigned)
                    if ex:
                        return True, assigned
                    outs.append(a)
                if s.orelse is not None:
                    ex, a = block(s.orelse, assigned)
                    if ex:
                        return True, assigned
                    outs.append(a)
                else:
                    outs.append(assigned)
                assigned = all(outs)
            elif isinstance(s, (For, While)):
                ex, _ = block(s.body, assigned)
                if ex:
                    return True, assigned
                # a loop body may run zero times: assignments inside do not count
        return False, assigned
    return block(body, False)[0]


def _last_top_assign(body, name: str):
    """The constant that the last top-level statement assigning `name` gives it, when nothing
    after that statement assigns it again (at any depth); None otherwise."""
    idx = None
    for k, s in enumerate(body):
        if isinstance(s, Assign) and isinstance(s.lhs, Var) and s.lhs.name == name:
            idx = k
    if idx is None:
        return None
    s = body[idx]
    if not isinstance(s.rhs, Num) or s.rhs.text in ("true", "false"):
        return None
    for t in body[idx + 1:]:
        if name in _assigned([t]):
            return None
    return s.rhs


def _is_sum_update(s, name) -> bool:
    """s is `name = name + e`, `name = e + name` or `name = name - e` with e free of name."""
    if not (isinstance(s, Assign) and isinstance(s.lhs, Var) and s.lhs.name == name and isinstance(s.rhs, Bin)):
        return False
    r = s.rhs
    if r.op == "+":
        if isinstance(r.a, Var) and r.a.name == name and name not in _reads_of(r.b):
            return True
        if isinstance(r.b, Var) and r.b.name == name and name not in _reads_of(r.a):
            return True
    if r.op == "-" and isinstance(r.a, Var) and r.a.name == name and name not in _reads_of(r.b):
        return True
    return False


def _linear_index(ref: Ref, types: Types) -> object:
    """The 1-based linear index expression of a reference (column-major)."""
    if len(ref.idx) == 1:
        return ref.idx[0]
    e = ref.idx[0]
    stride = None
    for d, i in enumerate(ref.idx[1:], start=1):
        dim = Call("size", (Var(ref.name), Num(str(d), True)))
        stride = dim if stride is None else Bin("*", stride, dim)
        e = Bin("+", e, Bin("*", Bin("-", i, Num("1", True)), stride))
    return e


def _is_acc(s, ref: Ref) -> bool:
    """s is `A[e] = A[e] + t` (or `t + A[e]`) with t free of A."""
    if not isinstance(s, Assign) or s.lhs != ref or not isinstance(s.rhs, Bin) or s.rhs.op not in ("+", "-"):
        return False
    r = s.rhs
    other = None
    if r.a == ref:
        other = r.b
    elif r.op == "+" and r.b == ref:
        other = r.a
    if other is None:
        return False
    return not any(isinstance(x, Ref) and x.name == ref.name for x in walk_expr(other))


def classify(loop: For, types: Types, later_reads: set, frame_written_outside: set) -> tuple[ParallelLoop | None, str]:
    """A ParallelLoop for `loop`, or (None, reason) when it must run in order."""
    body = loop.body
    v = loop.var
    for s in walk_stmts(body):
        if isinstance(s, (Return, Break)):
            return None, "the body returns or breaks out of the loop"
        if isinstance(s, ExprStmt):
            return None, "a bare expression statement"
        if isinstance(s, Assign) and isinstance(s.rhs, Alloc):
            return None, "an allocation inside the loop"
    if loop.rng.step is not None and not (isinstance(loop.rng.step, Num) and loop.rng.step.is_int
                                          and int(loop.rng.step.text) != 0):
        return None, "a step that is not a nonzero integer literal"
    has_continue = any(isinstance(s, Continue) for s in walk_stmts(body))
    bound_reads = _reads_of(loop.rng)
    assigned = _assigned(body) - {v}
    inner_vars = {s.var for s in walk_stmts(body) if isinstance(s, For)}
    if bound_reads & assigned:
        return None, "the loop bounds read a scalar the body assigns"
    private, reset, reductions, live_out = [], {}, {}, []
    for name in sorted(assigned):
        if name in inner_vars and name not in {x.lhs.name for x in walk_stmts(body) if isinstance(x, Assign) and isinstance(x.lhs, Var)}:
            continue
        occ = [s for s in walk_stmts(body) if any(name in _reads_of(e) for e in stmt_exprs(s))
               or (isinstance(s, Assign) and isinstance(s.lhs, Var) and s.lhs.name == name)]
        if occ and all(_is_sum_update(s, name) for s in occ) and types.scalars.get(name) in ("f", "i"):
            reductions[name] = "+"
            continue
        if _upward_exposed(body, name):
            c = None if has_continue else _last_top_assign(body, name)
            if c is None:
                return None, f"{name} is carried from one iteration to the next"
            reset[name] = c
        private.append(name)
        if name in later_reads:
            # the last iteration's value survives the loop: it must be written on every path
            top = any(isinstance(s, Assign) and isinstance(s.lhs, Var) and s.lhs.name == name for s in body)
            if not top or has_continue:
                return None, f"{name} is read after the loop but not assigned in every iteration"
            live_out.append(name)
    # iteration-private Int scalars with a single top-level definition, for index analysis
    env = {}
    for s in body:
        if (isinstance(s, Assign) and isinstance(s.lhs, Var) and s.lhs.name in private
                and types.scalars.get(s.lhs.name) == "i" and s.lhs.name not in reset):
            n_defs = sum(1 for t in walk_stmts(body) if isinstance(t, Assign) and isinstance(t.lhs, Var)
                         and t.lhs.name == s.lhs.name)
            if n_defs == 1:
                env[s.lhs.name] = s.rhs
    guards = []
    arrays = {}
    refs_by_array: dict[str, list] = {}
    for s in walk_stmts(body):
        for e in stmt_exprs(s):
            for x in walk_expr(e):
                if isinstance(x, Ref):
                    refs_by_array.setdefault(x.name, []).append(("r", x, s))
        if isinstance(s, Assign) and isinstance(s.lhs, Ref):
            refs_by_array.setdefault(s.lhs.name, []).append(("w", s.lhs, s))
    inner_depth = {}

    def in_inner(stmt):
        for t in walk_stmts(body):
            if isinstance(t, (For, While)) and any(u is stmt for u in walk_stmts(t.body)):
                return True
        return False

    def injective(ref: Ref):
        try:
            p = to_poly(_linear_index(ref, types), env, types)
        except NotAffine:
            return None
        p, conds = fold_divmod(p)
        lin = linear_in(p, v)
        if lin is None:
            return None
        coef, _ = lin
        if not coef:
            return None
        for m in coef:
            if any(a[0] != "v" or a[1] in assigned or a[1] in inner_vars for a in m):
                return None
        g = [("nonzero", coef)]
        for X, N in conds:
            lx = linear_in(X, v)
            if lx is None or any(depends_on({m: 1}, w) for m in list(lx[0]) + list(lx[1]) for w in inner_vars | assigned):
                return None
            g.append(("nonneg_over_range", X))
            g.append(("positive", N))
        return g

    for name, uses in refs_by_array.items():
        writes = [(r, s) for k, r, s in uses if k == "w"]
        if not writes:
            arrays[name] = ArrayUse(name, "read")
            continue
        reads = [(r, s) for k, r, s in uses if k == "r"]
        # accumulate-only: every write is A[e] = A[e] + t and the only reads are those
        acc_stmts = [s for r, s in writes if _is_acc(s, r)]
        if len(acc_stmts) == len(writes):
            read_ok = all(any(s is a for a in acc_stmts) and r == s.lhs for r, s in reads)
            if read_ok:
                idxs = {str(r) for r, _ in writes}
                if len(idxs) == 1 and not any(in_inner(s) for _, s in writes):
                    g = injective(writes[0][0])
                    if g is not None:
                        arrays[name] = ArrayUse(name, "owned", writes[0][0])
                        guards += g
                        continue
                # every accumulation at one index expression that no iteration changes (the
                # loss of a reduction loop, a bias gradient): a register sum per thread,
                # added once per block (`cgen_hoistable_atomic_keys` 11501-11519)
                varying = assigned | inner_vars | {v}
                if len(idxs) == 1 and all(not isinstance(x, (Ref, Call)) and not (isinstance(x, Var) and x.name in varying)
                                          for e in writes[0][0].idx for x in walk_expr(e)):
                    arrays[name] = ArrayUse(name, "atomic", writes[0][0], hoist=True)
                    continue
                arrays[name] = ArrayUse(name, "atomic")
                continue
        # owned: one index expression for every access, injective in the loop variable
        all_refs = [r for _, r, _ in uses]
        if len({str(r) for r in all_refs}) == 1 and not any(in_inner(s) for _, _, s in uses):
            g = injective(all_refs[0])
            if g is not None:
                arrays[name] = ArrayUse(name, "owned", all_refs[0])
                guards += g
                continue
        return None, f"array {name} is written at indices other iterations may read or write"
    reads_all = set()
    for s in walk_stmts(body):
        for e in stmt_exprs(s):
            reads_all |= _reads_of(e)
    reads_all |= bound_reads
    frame_reads = {n for n in reads_all if n not in types.arrays and n != v and n not in inner_vars}
    return ParallelLoop(loop, private, reset, reductions, arrays, guards, live_out, frame_reads), ""


# ------------------------------------------------------------------------------------------
# narrow outputs: lanes that share one iteration's inner loop
# ------------------------------------------------------------------------------------------

def split_loops(pl: ParallelLoop, types: Types) -> dict:
    """The inner loops of a parallel loop's body that the lanes of a wave can share when the
    loop has few iterations and long inner loops (the narrow-output twin, `cgen_split_*`
    /root/reference/src/STADE.jl:13155-13200, redone for 64-lane waves).

    Returns {id(inner For): [sum targets]} for the direct children of the body that qualify:
    every scalar the inner body assigns is either a sum target (only `s = s + e` / `s = e + s`
    / `s = s - e` updates of a scalar declared outside, combined across lanes after the loop)
    or local to an inner iteration (defined before it is read, not read after the loop, not
    carried to the next outer iteration); the inner body writes only accumulate-only arrays
    (order-free, so lanes add atomically); no break or return.  Empty when the body reads an
    element of an array after a statement that stores into that array (the stores are made
    by one lane of the wave; the other lanes would not see them)."""
    body = pl.loop.body
    owned = {n for n, u in pl.arrays.items() if u.kind == "owned"}
    written = set()
    for s in walk_stmts(body):     # statements in program order (owned stores are never in inner loops)
        for e in stmt_exprs(s):
            if any(isinstance(x, Ref) and x.name in written for x in walk_expr(e)):
                return {}
        if isinstance(s, Assign) and isinstance(s.lhs, Ref) and s.lhs.name in owned:
            written.add(s.lhs.name)
    out = {}
    for k, L in enumerate(body):
        if not isinstance(L, For):
            continue
        if any(isinstance(t, (Break, Return)) for t in walk_stmts(L.body)):
            continue
        inner_vars = {t.var for t in walk_stmts(L.body) if isinstance(t, For)} | {L.var}
        assigned = _assigned(L.body) - inner_vars
        after_reads = set()
        for t in body[k + 1:]:
            for e in stmt_exprs(t):
                after_reads |= _reads_of(e)
            for u in walk_stmts([t]):
                for e in stmt_exprs(u):
                    after_reads |= _reads_of(e)
        targets, ok = [], True
        for name in sorted(assigned):
            occ = [t for t in walk_stmts(L.body) if any(name in _reads_of(e) for e in stmt_exprs(t))
                   or (isinstance(t, Assign) and isinstance(t.lhs, Var) and t.lhs.name == name)]
            if occ and all(_is_sum_update(t, name) for t in occ) and types.scalars.get(name) in ("f", "i"):
                if name in pl.reductions:
                    continue          # the parallel loop's own sum: per-lane partials already
                targets.append(name)
                continue
            if (_upward_exposed(L.body, name) or name in after_reads or name in pl.reset or name in pl.live_out
                    or name in pl.reductions):
                ok = False
                break
        if not ok:
            continue
        for t in walk_stmts(L.body):
            if isinstance(t, Assign) and isinstance(t.lhs, Ref):
                u = pl.arrays.get(t.lhs.name)
                if u is None or u.kind != "atomic":
                    ok = False
                    break
        if ok:
            out[id(L)] = targets
    return out


@dataclass
class FlatTwin:
    """A flat loop over the elements of an R x N row-major range whose accumulations all
    target the row (kind 'row') or all the column (kind 'col'): see `flat_twin`."""
    kind: str                  # 'row' | 'col'
    N: object                  # the row length (an expression of Int arguments)
    sites: list                # the accumulated arrays
    iv: str                    # the row variable, i = div(idx - 1, N) + 1
    jv: str                    # the column variable, j = mod(idx - 1, N) + 1


def _derived(s, v, idxm1_names):
    """(var, 'div'|'mod', N) of `x = div(r, N) + 1` / `x = mod(r, N) + 1` with r = v - 1 (or
    a scalar holding it), else None (`cgen_rowblock_derived` /root/reference/src/STADE.jl:18162)."""
    if not (isinstance(s, Assign) and isinstance(s.lhs, Var)):
        return None
    r = s.rhs
    if not (isinstance(r, Bin) and r.op == "+" and isinstance(r.b, Num) and r.b.is_int and int(r.b.text) == 1):
        return None
    d = r.a
    if not (isinstance(d, Call) and d.fn in ("div", "mod") and len(d.args) == 2):
        return None
    x = d.args[0]
    is_vm1 = (isinstance(x, Bin) and x.op == "-" and x.a == Var(v) and isinstance(x.b, Num) and x.b.is_int
              and int(x.b.text) == 1)
    if not (is_vm1 or (isinstance(x, Var) and x.name in idxm1_names)):
        return None
    return s.lhs.name, d.fn, d.args[1]


def flat_twin(pl: ParallelLoop, int_args: set) -> FlatTwin | None:
    """The row-block or column-block twin of a parallel loop, or None.

    The reference's twins (`cgen_rowblock_kernel` /root/reference/src/STADE.jl:18187,
    `cgen_colblock_kernel` 18371) match a flat loop `for idx = 1:R*N` (ascending from 1, or
    descending to 1) with `i = div(idx - 1, N) + 1` and `j = mod(idx - 1, N) + 1` whose body is
    straight-line (scalar assignments, stores, accumulations) and whose accumulations go to at
    most four arrays, each touched by nothing else in the body:
    - 'row' when every accumulation's index reads i and nothing that depends on the column
      (idx, j, or a scalar computed from them): the N iterations of a row add into one element;
    - 'col' when every accumulation's index is j itself: the R iterations of a column do.
    N must be an expression of the function's Int arguments (the host checks at run time that
    the range is whole rows).  Loops with sums into scalars' last values read after the loop
    (live-out scalars) are left to the ordinary form."""
    loop = pl.loop
    body = loop.body
    v = loop.var
    if not body or not all(isinstance(s, Assign) for s in body) or pl.live_out:
        return None
    r = loop.rng
    step = 1 if r.step is None else (int(r.step.text) if isinstance(r.step, Num) and r.step.is_int else 0)
    one = lambda e: isinstance(e, Num) and e.is_int and int(e.text) == 1
    if not ((step == 1 and one(r.lo)) or (step == -1 and one(r.hi))):
        return None
    count = {}
    for s in body:
        if isinstance(s.lhs, Var):
            count[s.lhs.name] = count.get(s.lhs.name, 0) + 1
    vm1 = {s.lhs.name for s in body if isinstance(s.lhs, Var) and isinstance(s.rhs, Bin) and s.rhs.op == "-"
           and s.rhs.a == Var(v) and isinstance(s.rhs.b, Num) and s.rhs.b.is_int and int(s.rhs.b.text) == 1
           and count[s.lhs.name] == 1}
    der = [d for d in (_derived(s, v, vm1) for s in body) if d is not None]
    divs = [d for d in der if d[1] == "div"]
    mods = [d for d in der if d[1] == "mod"]
    if len(divs) != 1 or len(mods) != 1 or divs[0][2] != mods[0][2]:
        return None
    iv, jv, N = divs[0][0], mods[0][0], divs[0][2]
    nn = {x.name for x in walk_expr(N) if isinstance(x, Var)}
    if not nn or not nn <= int_args:
        return None
    if count.get(iv) != 1 or count.get(jv) != 1 or v in count:
        return None
    atomic = {n for n, u in pl.arrays.items() if u.kind == "atomic"}
    if not atomic or len(atomic) > 4 or pl.reductions or any(u.hoist for u in pl.arrays.values()):
        return None
    # names whose value depends on the column: idx, j, and scalars computed from them, in order
    tainted = {v, jv} | vm1
    site_idx = {}
    for s in body:
        if isinstance(s.lhs, Var):
            if s.lhs.name in (iv, jv) or s.lhs.name in vm1:
                continue          # the row, the column and idx - 1 themselves
            if _reads_of(s.rhs) & tainted:
                tainted.add(s.lhs.name)
            continue
        if s.lhs.name in atomic:
            if not (isinstance(s.rhs, Bin) and s.rhs.op in ("+", "-") and s.lhs in (s.rhs.a, s.rhs.b)):
                return None
            site_idx.setdefault(s.lhs.name, []).append(s.lhs)
    # each accumulated array is touched only by its accumulations
    for s in body:
        for e in stmt_exprs(s):
            for x in walk_expr(e):
                if isinstance(x, Ref) and x.name in atomic and not (isinstance(s.lhs, Ref) and s.lhs.name == x.name):
                    return None
    refs = [ref for refs in site_idx.values() for ref in refs]
    if len(site_idx) != len(atomic):
        return None
    if all(len(ref.idx) == 1 and ref.idx[0] == Var(jv) for ref in refs):
        return FlatTwin("col", N, sorted(atomic), iv, jv)
    if all(not (set().union(*(_reads_of(i) for i in ref.idx)) & tainted)
           and iv in set().union(*(_reads_of(i) for i in ref.idx)) for ref in refs):
        return FlatTwin("row", N, sorted(atomic), iv, jv)
    return None
