"""Code generation of the general lowering: one HIP source per generated file, one C entry
point per generated function.

Execution model (designed for one MI355X, not a translation of the reference's per-loop
AMDGPU.jl kernels, `cgen_kernel_def` /root/reference/src/STADE.jl:11106-11126):

* The function's scalars (arguments and locals) live in a per-function frame in device
  memory, so the host never waits for a device value: scalar statements run in small
  single-thread kernels, stream-ordered with the loops around them.
* A loop that `analysis.classify` accepts runs one iteration per thread (a grid-stride loop
  over the trip count, bounds read on the device).  Its index conditions (a nonzero stride,
  non-negative `div`/`mod` operands) are checked by the kernel; if one fails, the kernel runs
  the loop in order on one thread instead.  Iteration-private scalars are registers; sums
  into scalars are per-thread partials, summed across the wave and added once per wave;
  owned array elements are plain loads and stores; accumulations at shared indices are
  wave-aggregated atomics, or, for a small target with many contributions, atomics into a
  block-private LDS copy flushed once per block.
* A loop that cannot run that way but contains such loops, and whose bounds the host can
  evaluate (Int arguments, sizes, enclosing host loops), stays on the host (the time loop of
  an explicit scheme, as `cgen_body` keeps it, 10613-10615); one without parallel loops inside
  runs on one thread.
* An `if` around loops is evaluated on the device into a frame flag; the kernels of its
  branches test the flags (no host round trip).
* Returned scalars are copied back at the end: the only synchronisation of a call.
"""
from __future__ import annotations

import os
import re

from dataclasses import dataclass, field

from .analysis import ArrayUse, ParallelLoop, Types, classify, flat_twin, infer_types, split_loops, _reads_of, _thaw
from . import contract, finish, fuse, gather
from .syntax import (Alloc, Assign, Bin, Break, Call, Continue, ExprStmt, For, Func, Gemm, GemmT, If, LowerError,
                     Nothing_, Num, Range, Ref, Return, Tup, Un, Var, While, stmt_exprs, sub_blocks, walk_expr, walk_stmts)

MAX_BLOCKS = 8192          # grid of a parallel loop whose trip count the host cannot evaluate
                           # (and at most the fold's slots: FOLD_NT x FOLD_PER in lowered_rt.hpp)
FOLD_MIN_BLOCKS = 256      # a loop's block sums: atomics up to this many blocks, a fold kernel above
PRIV_MAX_BYTES = 48 * 1024  # LDS-privatised accumulation target, at most
PRIV_RATIO = 32            # and at least this many iterations per target element
TWIN_MIN_N = 256           # flat twins: rows of at least this many iterations (`row_block`, `col_block`
TWIN_MIN_ROWS = 64         # defaults of stade_gpu); the column twin at least this many rows (`cgen_colblock_min_rows`)
ROWBLOCK_GRID = 4096       # the row twin splits few rows over several blocks: about this many blocks,
ROWBLOCK_CHUNK = 2048      # each at least this many iterations of its row (the block's one atomic amortised)
COLBLOCK_ROWS = 128        # rows of a column-block tile (`cgen_colblock_rows`), 8 row lanes x 32 columns
XSPLIT_NW = 16             # waves of a block of the lanes-over-iterations form (16 to 64 iterations a block)
SPLIT_MAX_TRIP = 16384     # a parallel loop with at most this many iterations (64 blocks of 256 threads)
SPLIT_MIN_INNER = 256      # whose shared inner loop runs at least this many iterations (when the host
SPLIT_MAX_TRIP_UNKNOWN = 4096  # can evaluate it; otherwise at most this many outer iterations) gives
                               # each iteration a wave


def cname(n: str) -> str:
    return n.replace("!", "_bang_")


# ------------------------------------------------------------------------------------------
# plan
# ------------------------------------------------------------------------------------------

@dataclass
class SerialOp:
    stmts: list
    pred: tuple
    kid: int = 0


@dataclass
class ParOp:
    pl: ParallelLoop
    pred: tuple
    kid: int = 0
    types: Types | None = None


@dataclass
class HostLoopOp:
    loop: For
    ops: list
    slot: int = 0


@dataclass
class IfOp:
    node: If
    flags: list                # flag slot of each branch (and of else when present)
    branches: list             # ops per branch (else last)
    pred: tuple
    kid: int = 0


@dataclass
class AllocOp:
    name: str
    alloc: Alloc


@dataclass
class ReturnOp:
    value: object
    pred: tuple
    kid: int = 0


@dataclass
class GemmOp:
    g: object                  # Gemm | GemmT


class FuncLower:
    def __init__(self, f: Func, precision: str, arg_types: dict | None = None, stacks_allocated: set | None = None,
                 inbounds: bool = True, dead_scalars: bool = True, merge_accum: bool = True):
        # kernel finishing (finish.py, as `stade_gpu` runs it before and after planning): dead
        # restores and the stack stores nothing reads then, merged accumulations, dead scalars
        f, self.finish_rec = finish.finish(f, stacks_allocated or set(), inbounds=inbounds, dead=dead_scalars,
                                           merge=merge_accum)
        # inbounds (`stade_amdgpu_file`'s default): no check on array accesses; otherwise an
        # index out of range raises the frame's flag and is reported as a BoundsError
        self.inbounds = inbounds
        # periodic scatters into owner-computes gathers where the index maps are bijections
        # (gather.py); STADE_LOWER_GATHER=0 keeps every loop as written
        if os.environ.get("STADE_LOWER_GATHER", "1") != "0":
            f = Func(f.name, f.args, gather.transform(f.body), f.annot)
            # the owner's replayed terms add into its one element: merged as the finishing pass
            # merges the text's own (`stade_gpu` finishes after planning too), so that an
            # iteration loads and stores the element once
            if merge_accum:
                cnt = [0]
                f = Func(f.name, f.args, finish.merge_accum(f.body, cnt), f.annot)
                self.finish_rec["merged_gathered"] = cnt[0]
        self.f = f
        self.precision = precision
        self.T: Types = infer_types(f, arg_types, precision)
        # adjacent parallel loops over the same iterations as one loop (fuse.py);
        # STADE_LOWER_FUSE=0 keeps them apart
        if os.environ.get("STADE_LOWER_FUSE", "1") != "0":
            f = self._fused(f)
            self.f = f
        # contractions onto the fp32 matrix cores (contract.py): fp32 texts with unchecked
        # accesses; STADE_LOWER_GEMM=0 keeps the loops
        self.contract_rec: dict = {}
        if precision == "f32" and inbounds:
            f = self._contracted(f, arg_types, precision)
            self.f = f
        self.fty = "float" if precision == "f32" else "double"
        self.arrays = self.T.arrays
        self.scalars = {n: t for n, t in self.T.scalars.items() if n not in self.arrays}
        self.loopvars = {s.var for s in walk_stmts(f.body) if isinstance(s, For)}
        self.nflags = 0
        self.nhl = 0
        self.kernels: list[str] = []
        self.reasons: list[str] = []
        self.twins: list = []          # (loop variable, 'row' | 'col', sites) of the flat twins
        self.xsplits: list = []        # loop variables taking the lanes-over-iterations form
        self.refuse_reasons()
        self.ops = self.plan()

    @staticmethod
    def _parallel(loop: For, f: Func, T: Types) -> bool:
        """The planner's verdict on a top-level loop of f: its live-out scalars are those it
        assigns that the statements after it may read before assigning them."""
        from .analysis import _assigned, _upward_exposed
        pos = next((j for j, x in enumerate(f.body) if x is loop), None)
        if pos is None:
            return False
        cont = f.body[pos + 1:]
        live = {n for n in _assigned(loop.body) if _upward_exposed(cont, n)}
        pl, _ = classify(loop, T, live, set())
        return pl is not None

    def _contracted(self, f: Func, arg_types, precision) -> Func:
        def retype(g: Func) -> Types:
            # every array keeps its kind and rank (an operand only the products read is still
            # an argument of the same signature)
            T2 = infer_types(g, arg_types, precision)
            for n, kind in self.T.arrays.items():
                T2.arrays.setdefault(n, kind)
                T2.ndim[n] = max(T2.ndim.get(n, 1), self.T.ndim.get(n, 1))
            return T2
        g, rec, T2 = contract.transform(f, self.T, self._parallel, retype)
        if rec:
            self.T = T2
            self.contract_rec = rec
        return g

    def _fused(self, f: Func) -> Func:
        from .analysis import _upward_exposed

        def is_parallel(loop: For) -> bool:
            # (live-out scalars: every scalar the loop assigns that is read anywhere else in
            # the function, a superset of what the planner computes)
            outside = set()
            for s in walk_stmts(f.body):
                if s is loop or any(t is s for t in walk_stmts(loop.body)):
                    continue
                for e in stmt_exprs(s):
                    outside |= _reads_of(e)
            pl, _ = classify(loop, self.T, outside, set())
            return pl is not None
        return Func(f.name, f.args, fuse.transform(f.body, self.T, is_parallel), f.annot)

    # -- refusals ---------------------------------------------------------------------------
    def refuse_reasons(self):
        for s in walk_stmts(self.f.body):
            for e in stmt_exprs(s):
                for x in walk_expr(e):
                    if isinstance(x, Call) and x.fn in ("push!", "pop!"):
                        raise LowerError(f"{self.f.name}: push!/pop! stacks are not lowered (generate with indexed stacks)")
                    if isinstance(x, Ref) and x.name not in self.arrays:
                        raise LowerError(f"{self.f.name}: {x.name} is indexed but not an array")
            if isinstance(s, ExprStmt):
                raise LowerError(f"{self.f.name}: a bare expression statement")
            if isinstance(s, Assign) and isinstance(s.lhs, Var) and s.lhs.name in self.arrays and not isinstance(s.rhs, Alloc):
                raise LowerError(f"{self.f.name}: array {s.lhs.name} rebound by assignment")

    # -- host-evaluable expressions ----------------------------------------------------------
    def host_ok(self, e, hl: set) -> bool:
        assigned = {s.lhs.name for s in walk_stmts(self.f.body) if isinstance(s, Assign) and isinstance(s.lhs, Var)}
        for x in walk_expr(e):
            if isinstance(x, Var):
                if x.name in hl:
                    continue
                if x.name in self.arrays:
                    continue
                if x.name not in self.f.args or x.name in assigned or self.scalars.get(x.name) != "i":
                    return False
            elif isinstance(x, Ref):
                return False
            elif isinstance(x, Call) and x.fn not in ("div", "mod", "max", "min", "abs", "length", "size"):
                return False
            elif isinstance(x, Num) and not x.is_int:
                return False
            elif isinstance(x, Bin) and x.op not in ("+", "-", "*"):
                return False
        return True

    # -- planning ----------------------------------------------------------------------------
    def plan(self):
        body = self.f.body
        rets = [s for s in walk_stmts(body) if isinstance(s, Return)]
        tail_return = bool(body) and isinstance(body[-1], Return)
        if any(r is not body[-1] for r in rets) or any(isinstance(s, (Break, Continue)) for s in body):
            # a return before the end (or control flow at the top level): the whole function in
            # order on one thread
            return [SerialOp(list(body), ())]
        stmts = body[:-1] if tail_return else body
        ops = self.lower_block(stmts, (), set(), top=True)
        if tail_return and body[-1].value is not None and not isinstance(body[-1].value, Nothing_):
            ops.append(ReturnOp(body[-1].value, ()))
        return ops

    def _later_reads(self) -> set:
        out = set()
        for s in walk_stmts(self.f.body):
            for e in stmt_exprs(s):
                out |= _reads_of(e)
        return out

    def contains_parallel(self, body, hl) -> bool:
        for s in walk_stmts(body):
            if isinstance(s, For):
                pl, _ = classify(s, self.T, self._reads_outside(s), set())
                if pl is not None:
                    return True
        return False

    def _parents(self):
        if not hasattr(self, "_par"):
            par = {}

            def visit(block, enclosing):
                for k, s in enumerate(block):
                    par[id(s)] = (block, k, enclosing)
                    for b in sub_blocks(s):
                        visit(b, s)
            visit(self.f.body, None)
            self._par = par
        return self._par

    def _reads_outside(self, loop: For) -> set:
        """The scalars the loop assigns that are live after it: read on some path from the
        loop's exit before being assigned again (the statements after it, then after each
        enclosing statement, and one more pass over every enclosing loop's body)."""
        from .analysis import _assigned, _upward_exposed
        par = self._parents()
        cont = []
        node = loop
        while node is not None:
            block, k, enclosing = par[id(node)]
            cont += block[k + 1:]
            if isinstance(enclosing, (For, While)):
                cont += enclosing.body
            node = enclosing
        out = set()
        for name in _assigned(loop.body):
            if _upward_exposed(cont, name):
                out.add(name)
        return out

    def lower_block(self, stmts, pred, hl: set, top=False):
        ops = []
        cur = []

        def flush():
            if cur:
                ops.append(SerialOp(list(cur), pred))
                cur.clear()
        for s in stmts:
            if isinstance(s, (Gemm, GemmT)):
                if not top or pred:
                    raise LowerError(f"{self.f.name}: a matrix product below the top level")
                flush()
                ops.append(GemmOp(s))
                continue
            if isinstance(s, Assign) and isinstance(s.rhs, Alloc):
                if not (top and isinstance(s.lhs, Var) and self.host_ok(s.rhs.n, hl)):
                    raise LowerError(f"{self.f.name}: allocation of {s.lhs} needs a size the host can evaluate, "
                                     f"at the top level of the function")
                flush()
                ops.append(AllocOp(s.lhs.name, s.rhs))
                continue
            if isinstance(s, For):
                pl, why = classify(s, self.T, self._reads_outside(s), set())
                if pl is not None:
                    flush()
                    ops.append(ParOp(pl, pred, types=self.T))
                    continue
                self.reasons.append(f"loop over {s.var}: {why}")
                if self.contains_parallel(s.body, hl) and self.host_ok(s.rng, hl) and not any(
                        isinstance(t, (Break, Continue, Return)) for t in walk_stmts(s.body)):
                    flush()
                    slot = self.nhl
                    self.nhl += 1
                    inner = self.lower_block(s.body, pred, hl | {s.var})
                    ops.append(HostLoopOp(s, inner, slot))
                    continue
                cur.append(s)
                continue
            if isinstance(s, If) and self.contains_parallel([s], hl) and not any(
                    isinstance(t, (Break, Continue, Return)) for t in walk_stmts([s])):
                flush()
                nb = len(s.branches) + (1 if s.orelse is not None else 0)
                flags = list(range(self.nflags, self.nflags + nb))
                self.nflags += nb
                branches = []
                for k, (_, b) in enumerate(s.branches):
                    branches.append(self.lower_block(b, pred + (flags[k],), hl))
                if s.orelse is not None:
                    branches.append(self.lower_block(s.orelse, pred + (flags[-1],), hl))
                ops.append(IfOp(s, flags, branches, pred))
                continue
            cur.append(s)
        flush()
        return ops

    # -- names ---------------------------------------------------------------------------------
    def cty(self, t: str) -> str:
        return {"i": "int64_t", "b": "bool", "f": self.fty}[t]

    def frame_scalars(self):
        # every scalar (a name may be a loop variable in one place and a plain variable in
        # another; unused slots cost nothing)
        return sorted(self.scalars)

    # -- expressions -----------------------------------------------------------------------------
    def ex(self, e, ctx) -> tuple[str, str]:
        """C code and type ('i', 'b', 'f' precision float, 'd' double) of an expression."""
        if isinstance(e, Num):
            if e.text in ("true", "false"):
                return e.text, "b"
            if e.is_int:
                return f"((int64_t){int(e.text, 0)}LL)", "i"
            if e.f32:
                return f"({e.text}f)", "f" if self.fty == "float" else "F"
            txt = e.text if ("." in e.text or "e" in e.text or "E" in e.text) else e.text + ".0"
            if self.fty == "float":
                return f"((float){txt})", "f"
            return f"({txt})", "f"
        if isinstance(e, Var):
            return ctx.var(e.name), ctx.vtype(e.name)
        if isinstance(e, Ref):
            return ctx.ref(e), ("i" if self.arrays[e.name] == "i" else "f")
        if isinstance(e, Un):
            a, t = self.ex(e.a, ctx)
            if e.op == "!":
                return f"(!{a})", "b"
            return f"(-{a})", t
        if isinstance(e, Bin):
            return self.binop(e, ctx)
        if isinstance(e, Call):
            return self.call(e, ctx)
        raise LowerError(f"{self.f.name}: cannot lower expression {e!r}")

    def binop(self, e, ctx):
        op = e.op
        if op == "^":
            return self.power(e, ctx)
        a, ta = self.ex(e.a, ctx)
        b, tb = self.ex(e.b, ctx)
        if op in ("&&", "||"):
            return f"({a} {op} {b})", "b"
        if op in ("==", "!=", "<", ">", "<=", ">="):
            return f"({a} {op} {b})", "b"
        if op == "/":
            if ta == "i" and tb == "i":
                return f"((double){a} / (double){b})", "d"
            return f"({a} / {b})", self._join(ta, tb)
        return f"({a} {op} {b})", self._join(ta, tb)

    def _join(self, ta, tb):
        if "d" in (ta, tb):
            return "d"
        if "f" in (ta, tb) or "F" in (ta, tb):
            return "f" if self.fty == "float" or "f" in (ta, tb) and self.fty == "double" else "f"
        if "b" in (ta, tb):
            return "i"
        return "i"

    def power(self, e, ctx):
        base, tb = self.ex(e.a, ctx)
        pe = e.b
        if isinstance(pe, Num) and pe.is_int:
            p = int(pe.text, 0)
            if tb == "i":
                return f"stade_lowered::jl_ipow({base}, {p})", "i"
            ct = "double" if tb == "d" else self.fty
            if p == 2:
                return f"([&]() {{ const {ct} _b = {base}; return _b * _b; }}())", tb
            if p == 3:
                return f"([&]() {{ const {ct} _b = {base}; return _b * _b * _b; }}())", tb
            if p == 1:
                return base, tb
            if p == 0:
                return f"(({ct})1)", tb
            if p == -1:
                return f"(({ct})1 / {base})", tb
            if p == -2:
                return f"([&]() {{ const {ct} _b = ({ct})1 / {base}; return _b * _b; }}())", tb
            return f"pow({base}, ({ct}){p})", tb
        x, tx = self.ex(pe, ctx)
        if tb == "i" and tx == "i":
            return f"stade_lowered::jl_ipow({base}, {x})", "i"
        return f"pow({base}, {x})", self._join(tb, tx) if tb != "i" else (tx if tx != "i" else "d")

    def call(self, e, ctx):
        fn, args = e.fn, e.args
        if fn == "length":
            return ctx.length(args[0].name), "i"
        if fn == "size":
            d = int(args[1].text) if len(args) > 1 else 1
            return ctx.dim(args[0].name, d - 1), "i"
        xs = [self.ex(a, ctx) for a in args]
        codes = [c for c, _ in xs]
        tys = [t for _, t in xs]
        if fn in ("div", "mod", "rem", "fld", "cld"):
            a, b = codes
            if all(t == "i" for t in tys):
                return {"div": f"({a} / {b})", "rem": f"({a} % {b})", "mod": f"stade_lowered::jl_mod({a}, {b})",
                        "fld": f"stade_lowered::jl_fld({a}, {b})", "cld": f"stade_lowered::jl_cld({a}, {b})"}[fn], "i"
            t = self._join(*tys)
            ct = "double" if t == "d" else self.fty
            a, b = f"({ct}){a}", f"({ct}){b}"
            if fn == "mod":
                return f"stade_lowered::jl_mod({a}, {b})", t
            if fn == "rem":
                return f"fmod({a}, {b})", t
            if fn == "div":
                return f"trunc({a} / {b})", t
            if fn == "fld":
                return f"floor({a} / {b})", t
            return f"ceil({a} / {b})", t
        if fn in ("max", "min"):
            t = "i" if all(t == "i" for t in tys) else self._join(*tys)
            ct = {"i": "int64_t", "d": "double"}.get(t, self.fty)
            out = f"(({ct}){codes[0]})"
            for c in codes[1:]:
                out = f"stade_lowered::jl_{fn}({out}, ({ct}){c})"
            return out, t
        if fn == "abs":
            return (f"llabs({codes[0]})", "i") if tys[0] == "i" else (f"fabs({codes[0]})", tys[0])
        if fn == "sign":
            return f"stade_lowered::jl_sign({codes[0]})", tys[0]
        if fn == "ifelse":
            t = self._join(tys[1], tys[2]) if "i" not in (tys[1], tys[2]) or tys[1] != tys[2] else tys[1]
            return f"(({codes[0]}) ? ({codes[1]}) : ({codes[2]}))", t
        if fn in ("Float64", "float"):
            return f"((double){codes[0]})", "d"
        if fn == "Float32":
            return f"((float){codes[0]})", "f" if self.fty == "float" else "F"
        if fn in ("Int", "Int64"):
            return f"((int64_t){codes[0]})", "i"
        if fn in ("floor", "ceil", "round", "trunc"):
            cfn = {"floor": "floor", "ceil": "ceil", "round": "rint", "trunc": "trunc"}[fn]
            if len(args) == 2:   # floor(Int, x)
                return f"((int64_t){cfn}({codes[1]}))", "i"
            return f"{cfn}({codes[0]})", tys[0]
        if fn == "inv":
            return f"(1 / {codes[0]})", tys[0]
        if fn in ("exp", "log", "tanh", "sin", "cos", "tan", "sqrt", "sinh", "cosh", "atan", "asin", "acos", "log10",
                  "log2", "exp2", "expm1", "log1p", "cbrt"):
            t = tys[0] if tys[0] != "i" else "d"
            a = codes[0] if tys[0] != "i" else f"(double){codes[0]}"
            return f"{fn}({a})", t
        raise LowerError(f"{self.f.name}: call to unsupported function {fn}")


# ------------------------------------------------------------------------------------------
# emission contexts
# ------------------------------------------------------------------------------------------

class Ctx:
    """How names read and write inside one kernel (or the host)."""

    def __init__(self, fl: FuncLower, locals_: dict, hl_names: dict, acc: dict | None = None, serial_acc=True,
                 reductions: dict | None = None, lds: str | None = None, hoist: dict | None = None):
        self.fl = fl
        self.hoist = hoist or {}       # array -> register summing its accumulations (one index)
        self.locals = locals_          # scalar -> C local name
        self.hl = hl_names             # host loop var -> slot
        self.acc = acc or {}           # array -> 'atomic' (accumulations through wave_add / lds)
        self.serial_acc = serial_acc   # accumulations as plain read-modify-writes
        self.reductions = reductions or {}
        self.lds = lds                 # array privatised in LDS (its accumulations go to lds_priv)
        self.site_ix = {}              # hoisted array -> local recording its index (the flat twins)

    def var(self, n):
        if n in self.locals:
            return self.locals[n]
        if n in self.hl:
            return f"a.hl[{self.hl[n]}]"
        if n in self.fl.arrays:
            raise LowerError(f"{self.fl.f.name}: array {n} used as a value")
        return f"fr.v_{cname(n)}"

    def vtype(self, n):
        t = self.fl.scalars.get(n, "f")
        return t

    def dim(self, name, d):
        return f"a.D_{cname(name)}[{d}]"

    def length(self, name):
        nd = self.fl.T.ndim.get(name, 1)
        return "(" + " * ".join(f"a.D_{cname(name)}[{d}]" for d in range(nd)) + ")"

    def lin(self, ref: Ref) -> str:
        parts = []
        stride = None
        for d, i in enumerate(ref.idx):
            c, t = self.fl.ex(i, self)
            if t != "i":
                c = f"(int64_t)({c})"
            term = f"(({c}) - 1)"
            parts.append(term if stride is None else f"{term} * {stride}")
            s = f"a.D_{cname(ref.name)}[{d}]"
            stride = s if stride is None else f"{stride} * {s}"
        return " + ".join(parts)

    def ref(self, ref: Ref) -> str:
        # inbounds: a plain load; otherwise bounds-checked: an index outside the array raises
        # the frame's flag (the call then reports Julia's BoundsError) and reads 0 instead of
        # touching memory
        if self.fl.inbounds:
            return f"a.A_{cname(ref.name)}[{self.lin(ref)}]"
        return f"rd(a.A_{cname(ref.name)}, {self.lin(ref)}, a.N_{cname(ref.name)})"


class Emitter:
    def __init__(self, fl: FuncLower, ctx: Ctx):
        self.fl, self.ctx = fl, ctx
        # labels unique across the emitters of one function, numbered in emission order so the
        # generated source (whose hash names the built library) is the same in every process
        fl.n_emitters = getattr(fl, "n_emitters", 0) + 1
        self.u = fl.n_emitters
        self.lines: list[str] = []
        self.ind = 1
        self.loop_labels = []
        self.nlabel = 0
        # the split form (a wave per iteration): inner loops shared by the lanes, their sum
        # targets' per-lane partials, and stores made by lane 0 outside those loops
        self.split_loops: dict = {}
        self.partials: dict = {}
        self.lane0 = False
        self.in_split = 0
        # who shares a split loop: the wave's lanes (`_lane`, 64 of them, combined by a wave
        # sum), or, in the lanes-over-iterations form, the block's waves (`_wv`, XSPLIT_NW of
        # them, combined through LDS), whose inactive lanes (`act`) store nothing
        self.share_var, self.share_n, self.xsum = "_lane", "64", None
        self.act = None
        # the lanes-over-iterations form's iterations a block (a template parameter of its
        # kernel): accumulations inside shared loops aggregate per lane group (group_add)
        self.group = None

    def one_lane(self) -> bool:
        return self.lane0 and not self.in_split

    def who(self) -> str:
        """The guard of a store: lane (or wave) 0 outside split loops, active lanes only."""
        conds = []
        if self.one_lane():
            conds.append(f"{self.share_var} == 0")
        if self.act:
            conds.append(self.act)
        return f"if ({' && '.join(conds)}) " if conds else ""

    def emit(self, s):
        self.lines.append("    " * self.ind + s)

    def block(self, stmts):
        for s in stmts:
            self.stmt(s)

    def stmt(self, s):
        fl, ctx = self.fl, self.ctx
        if isinstance(s, Assign):
            if isinstance(s.lhs, Var):
                n = s.lhs.name
                acc_name = self.partials.get(n) if self.in_split else None
                if acc_name is None and n in ctx.reductions:
                    acc_name = ctx.reductions[n]
                if acc_name is not None and isinstance(s.rhs, Bin):
                    r = s.rhs
                    if isinstance(r.a, Var) and r.a.name == n:
                        c, _ = fl.ex(r.b, ctx)
                        line = f"{acc_name} {'+' if r.op == '+' else '-'}= {c};"
                    else:
                        c, _ = fl.ex(r.a, ctx)
                        line = f"{acc_name} += {c};"
                    # (a sum of the parallel loop outside the shared inner loops: lane 0's)
                    self.emit(f"{self.who()}{{ {line} }}" if (self.one_lane() or self.act) and n in ctx.reductions
                              else line)
                    return
                c, _ = fl.ex(s.rhs, ctx)
                self.emit(f"{ctx.var(n)} = ({fl.cty(fl.scalars.get(n, 'f'))})({c});")
                return
            ref = s.lhs
            et = "int64_t" if fl.arrays[ref.name] == "i" else fl.fty
            if ref.name in ctx.acc and not ctx.serial_acc:
                r = s.rhs
                other, sign = (r.b, "+") if r.a == ref else (r.a, "+")
                if r.op == "-":
                    sign = "-"
                c, _ = fl.ex(other, ctx)
                val = f"({et})({c})" if sign == "+" else f"(-({et})({c}))"
                nm = cname(ref.name)
                chk = "" if fl.inbounds else f"if ((uint64_t)_i < (uint64_t)a.N_{nm}) "
                els = "" if fl.inbounds else " else oob();"
                if ref.name in ctx.hoist:
                    self.emit(f"{{ const int64_t _i = {ctx.lin(ref)};")
                    track = f" {ctx.site_ix[ref.name]} = _i;" if ref.name in ctx.site_ix else ""
                    self.emit(f"  {chk}{ctx.hoist[ref.name]} += {val};{els}{track} }}")
                    return
                if self.act and self.one_lane():
                    self.emit("__syncthreads();")
                self.emit(self.who() + f"{{ const int64_t _i = {ctx.lin(ref)};")
                if ctx.lds == ref.name:
                    self.emit(f"  {chk}stade_lowered::lds_add(&lds_priv[_i], {val});{els} }}")
                else:
                    add = f"group_add<{self.group}>" if self.group and self.in_split else "wave_add"
                    self.emit(f"  {chk}stade_lowered::{add}(&a.A_{nm}[_i], {val}, a.st);{els} }}")
                return
            c, _ = fl.ex(s.rhs, ctx)
            if self.act and self.one_lane():
                # (the lanes-over-iterations form: every wave has read the element before wave 0
                # stores it)
                self.emit("__syncthreads();")
            if fl.inbounds:
                self.emit(self.who() + f"a.A_{cname(ref.name)}[{ctx.lin(ref)}] = ({et})({c});")
            else:
                self.emit(self.who() + f"wr(a.A_{cname(ref.name)}, {ctx.lin(ref)}, a.N_{cname(ref.name)}, ({et})({c}));")
            return
        if isinstance(s, For) and id(s) in self.split_loops:
            self.split_for(s)
            return
        if isinstance(s, For):
            lo, _ = fl.ex(s.rng.lo, ctx)
            hi, _ = fl.ex(s.rng.hi, ctx)
            st = "1" if s.rng.step is None else fl.ex(s.rng.step, ctx)[0]
            v = f"l_{cname(s.var)}"
            saved = ctx.locals.get(s.var)
            k = self.nlabel
            self.nlabel += 1
            self.emit("{")
            self.ind += 1
            self.emit(f"const int64_t _lo{k} = {lo}, _st{k} = {st}, _n{k} = stade_lowered::jl_trip(_lo{k}, _st{k}, {hi});")
            self.emit(f"for (int64_t _k{k} = 0; _k{k} < _n{k}; ++_k{k}) {{")
            self.ind += 1
            self.emit(f"const int64_t {v} = _lo{k} + _k{k} * _st{k};")
            ctx.locals[s.var] = v
            self.loop_labels.append(k)
            self.block(s.body)
            self.loop_labels.pop()
            self.emit(f"_cont{self.u}_{k}:;")
            self.ind -= 1
            self.emit("}")
            self.emit(f"_brk{self.u}_{k}:;")
            self.ind -= 1
            self.emit("}")
            if saved is None:
                ctx.locals.pop(s.var, None)
            else:
                ctx.locals[s.var] = saved
            return
        if isinstance(s, While):
            k = self.nlabel
            self.nlabel += 1
            c, _ = fl.ex(s.cond, ctx)
            self.emit(f"while ({c}) {{")
            self.ind += 1
            self.loop_labels.append(k)
            self.block(s.body)
            self.loop_labels.pop()
            self.emit(f"_cont{self.u}_{k}:;")
            self.ind -= 1
            self.emit("}")
            self.emit(f"_brk{self.u}_{k}:;")
            return
        if isinstance(s, If):
            for j, (cond, body) in enumerate(s.branches):
                c, _ = fl.ex(cond, ctx)
                self.emit(("if" if j == 0 else "} else if") + f" ({c}) {{")
                self.ind += 1
                self.block(body)
                self.ind -= 1
            if s.orelse is not None:
                self.emit("} else {")
                self.ind += 1
                self.block(s.orelse)
                self.ind -= 1
            self.emit("}")
            return
        if isinstance(s, Break):
            self.emit(f"goto _brk{self.u}_{self.loop_labels[-1]};")
            return
        if isinstance(s, Continue):
            if self.loop_labels:
                self.emit(f"goto _cont{self.u}_{self.loop_labels[-1]};")
            else:
                self.emit(f"goto _next_iter{self.u};")
            return
        if isinstance(s, Return):
            self.ret(s.value)
            self.emit("goto _fn_end;")
            return
        raise LowerError(f"{fl.f.name}: cannot lower statement {s!r}")

    def split_for(self, s: For):
        """An inner loop shared by the lanes of the wave: lane l runs iterations l, l + 64, ...;
        each sum target gets a per-lane partial, added to the target (the same value in every
        lane) after the loop.  The last bits of such a sum differ from the loop in order."""
        fl, ctx = self.fl, self.ctx
        lo, _ = fl.ex(s.rng.lo, ctx)
        hi, _ = fl.ex(s.rng.hi, ctx)
        st = "1" if s.rng.step is None else fl.ex(s.rng.step, ctx)[0]
        v = f"l_{cname(s.var)}"
        saved = ctx.locals.get(s.var)
        k = self.nlabel
        self.nlabel += 1
        targets = self.split_loops[id(s)]
        self.emit("{")
        self.ind += 1
        saved_partials = dict(self.partials)
        for t in targets:
            pn = f"p{k}_{cname(t)}"
            self.emit(f"{fl.cty(fl.scalars[t])} {pn} = 0;")
            self.partials[t] = pn
        self.emit(f"const int64_t _lo{k} = {lo}, _st{k} = {st}, _n{k} = stade_lowered::jl_trip(_lo{k}, _st{k}, {hi});")
        self.emit(f"for (int64_t _k{k} = {self.share_var}; _k{k} < _n{k}; _k{k} += {self.share_n}) {{")
        self.ind += 1
        self.emit(f"const int64_t {v} = _lo{k} + _k{k} * _st{k};")
        ctx.locals[s.var] = v
        self.loop_labels.append(k)
        self.in_split += 1
        self.block(s.body)
        self.in_split -= 1
        self.loop_labels.pop()
        self.emit(f"_cont{self.u}_{k}:;")
        self.ind -= 1
        self.emit("}")
        self.emit(f"_brk{self.u}_{k}:;")
        for t in targets:
            tot = (f"stade_lowered::wave_sum({self.partials[t]})" if self.xsum is None
                   else self.xsum(self.partials[t], fl.scalars[t]))
            self.emit(f"{ctx.var(t)} = {ctx.var(t)} + {tot};")
        self.partials = saved_partials
        self.ind -= 1
        self.emit("}")
        if saved is None:
            ctx.locals.pop(s.var, None)
        else:
            ctx.locals[s.var] = saved

    def ret(self, value):
        fl = self.fl
        if value is None or isinstance(value, Nothing_):
            return
        items = value.items if isinstance(value, Tup) else (value,)
        if len(items) > 16:
            # the frame holds 16 returned values (r, ri, rk) and the host copies back as many
            raise LowerError(f"{fl.f.name}: returns {len(items)} values; the lowering returns at most 16")
        for k, it in enumerate(items):
            c, t = fl.ex(it, self.ctx)
            if t == "i":
                self.emit(f"fr.ri[{k}] = {c}; fr.rk[{k}] = 1;")
            else:
                self.emit(f"fr.r[{k}] = (double)({c}); fr.rk[{k}] = 0;")
        self.emit(f"fr.nret = {len(items)};")


# ------------------------------------------------------------------------------------------
# kernels and the entry point of one function
# ------------------------------------------------------------------------------------------

def _stmt_scalars(fl: FuncLower, stmts) -> tuple[set, set]:
    """(scalars read, scalars assigned) by statements, excluding their own loop variables."""
    reads, writes, inner = set(), set(), set()
    for s in walk_stmts(stmts):
        for e in stmt_exprs(s):
            reads |= {n for n in _reads_of(e) if n not in fl.arrays}
        if isinstance(s, Assign) and isinstance(s.lhs, Var):
            writes.add(s.lhs.name)
        if isinstance(s, For):
            inner.add(s.var)
    return reads - inner, writes - inner


class FuncGen:
    """HIP source of one lowered function: namespace gen_<name> with its frame, kernels and
    the extern "C" entry point stade_hip_gen_<name>."""

    def __init__(self, fl: FuncLower):
        self.fl = fl
        self.ns = f"gen_{cname(fl.f.name)}"
        self.kern: list[str] = []
        self.host: list[str] = []
        self.nk = 0
        self.hind = 1
        self.nalloc = 0
        self.ngemm = 0
        self.uses_gemm = False
        self.hlv: dict[str, int] = {}   # host loop variables in scope -> their slot in Args.hl
        self.serial_kernels: set[str] = set()

    def pred_code(self, pred) -> str:
        return " && ".join(f"fr.flag[{k}]" for k in pred) if pred else "true"

    def hemit(self, line):
        self.host.append("    " * self.hind + line)

    def launch(self, kname, grid="1", block="1", shmem="0", tmpl=""):
        self.hemit(f"{kname}{tmpl}<<<{grid}, {block}, {shmem}, stream>>>(a);")
        self.hemit(f"if ((_e = hipGetLastError()) != hipSuccess) return _fail(_e, \"{kname}\");")

    # -- serial kernels ---------------------------------------------------------------------
    def serial(self, stmts, pred, ret_value=None) -> None:
        fl = self.fl
        k = self.nk
        self.nk += 1
        reads, writes = _stmt_scalars(fl, stmts)
        if ret_value is not None:
            reads |= {n for n in _reads_of(ret_value) if n not in fl.arrays}
        hl = self.hlv
        names = sorted(n for n in (reads | writes) if n not in hl and n in fl.scalars)
        ctx = Ctx(fl, {n: f"x_{cname(n)}" for n in names}, hl, serial_acc=True)
        em = Emitter(fl, ctx)
        em.emit(f"if (!({self.pred_code(pred)})) return;")
        for n in names:
            em.emit(f"{fl.cty(fl.scalars[n])} x_{cname(n)} = fr.v_{cname(n)};")
        em.block(stmts)
        if ret_value is not None:
            em.ret(ret_value)
        em.emit("goto _fn_end;")
        em.emit("_fn_end:;")
        for n in sorted(writes):
            if n in names:
                em.emit(f"fr.v_{cname(n)} = x_{cname(n)};")
        self.one_thread_kernel(k, em.lines)
        self.launch(f"k{k}")

    def one_thread_kernel(self, k: int, lines: list) -> None:
        """A one-thread kernel k<k>, its body a device function, so that launches of
        consecutive one-thread kernels can be merged into one (merge_serial_launches)."""
        self.kern.append(f"__device__ __forceinline__ void k{k}_body(const Args& a) {{\n" + "\n".join(lines) + "\n}\n"
                         f"__global__ __launch_bounds__(1) void k{k}(const Args a) {{ k{k}_body(a); }}\n")
        self.serial_kernels.add(f"k{k}")

    def merge_serial_launches(self) -> None:
        """Launches of one-thread kernels that follow each other with no host
        statement between them become one launch of a kernel that runs their bodies in order:
        the same statements in the same order on the same thread, with the same arguments
        (`a` changes only at host statements), one kernel boundary instead of several."""
        launch_re = re.compile(r"^(\s*)(k\d+)<<<1, 1, 0, stream>>>\(a\);$")
        out, i, h = [], 0, self.host
        while i < len(h):
            m = launch_re.match(h[i])
            run = []
            j = i
            while j + 1 < len(h):
                mj = launch_re.match(h[j])
                if not (mj and mj.group(2) in self.serial_kernels and (not run or mj.group(1) == m.group(1))
                        and h[j + 1].strip().startswith("if ((_e = hipGetLastError())")):
                    break
                run.append(mj.group(2))
                j += 2
            if len(run) >= 2:
                name = "km" + "_".join(r[1:] for r in run)
                self.kern.append(f"__global__ __launch_bounds__(1) void {name}(const Args a) {{ "
                                 + " ".join(f"{r}_body(a);" for r in run) + " }\n")
                out.append(f"{m.group(1)}{name}<<<1, 1, 0, stream>>>(a);")
                out.append(f"{m.group(1)}if ((_e = hipGetLastError()) != hipSuccess) return _fail(_e, \"{name}\");")
                i = j
            else:
                out.append(h[i])
                i += 1
        self.host = out

    # -- flat twins ----------------------------------------------------------------------------
    def twin_kernel(self, k: int, tw, head: list, guards: str, body_lines, n_dev: str) -> str:
        """k<k>t, the row-block or column-block twin of a flat loop (`cgen_rowblock_kernel`
        /root/reference/src/STADE.jl:18187, `cgen_colblock_kernel` 18371): the same iterations,
        mapped so that the accumulations of a row (a column) meet in one block (one thread).
        - row: block b runs the N iterations _k = b N .. b N + N - 1, which for an ascending
          loop from 1, or a descending one to 1, are exactly row b + 1 (or R - b) of the range;
          each thread sums its iterations' values per site in a register, the block adds them
          in a fixed order and makes one atomic addition per site.
        - col: a block of 32 columns x 8 row lanes takes COLBLOCK_ROWS rows; a thread sums its
          column's rows in a register, the 8 lanes of a column add up in a fixed order through
          LDS and one thread adds the tile's total, one atomic per column and tile.
        The host launches it only when the range is whole rows (checked at run time)."""
        fl = self.fl
        sites = tw.sites
        acc = {n: f"t_{cname(n)}" for n in sites}
        ix = {n: f"ti_{cname(n)}" for n in sites}
        et = lambda n: "int64_t" if fl.arrays[n] == "i" else fl.fty
        out = list(head)
        out.append(f"    if (!({guards})) {{")
        out.append("        if (blockIdx.x != 0 || blockIdx.y != 0 || threadIdx.x != 0) return;")
        out.append("        for (int64_t _k = 0; _k < _trip; ++_k) {")
        out += body_lines(False, None)
        out.append("        }")
        out.append("        return;")
        out.append("    }")
        out.append(f"    const int64_t _tn = {n_dev};")
        for n in sites:
            out.append(f"    {et(n)} {acc[n]} = 0;")
            out.append(f"    int64_t {ix[n]} = 0;")
        lines = body_lines(True, None, twin_sites=acc, twin_ix=ix)
        if tw.kind == "row":
            # S = gridDim.x / rows blocks a row, each a chunk of ceil(N / S) >= 256 iterations
            out.append("    if (threadIdx.x == 0) stade_lowered::count(a.st, stade_lowered::ST_ROW_BLOCK);")
            out.append("    const int64_t _tr = _trip / _tn, _ts = (int64_t)gridDim.x / _tr;")
            out.append("    const int64_t _row = (int64_t)blockIdx.x / _ts, _cs = (_tn + _ts - 1) / _ts;")
            out.append("    const int64_t _t0 = ((int64_t)blockIdx.x % _ts) * _cs, _t1 = _t0 + _cs < _tn ? _t0 + _cs : _tn;")
            out.append("    for (int64_t _t = _t0 + threadIdx.x; _t < _t1; _t += blockDim.x) {")
            out.append("        const int64_t _k = _row * _tn + _t;")
            out += lines
            out.append("    }")
            out.append(f"    __shared__ double _blk[16];")
            for n in sites:
                # thread 0 ran the chunk's first iteration (every chunk has one): its index is the row's
                out.append(f"    stade_lowered::block_add(&a.A_{cname(n)}[{ix[n]}], {acc[n]}, "
                           f"reinterpret_cast<{et(n)}*>(_blk), a.st);")
        else:
            out.append("    if (threadIdx.x == 0) stade_lowered::count(a.st, stade_lowered::ST_COL_BLOCK);")
            out.append("    const int _tx = threadIdx.x & 31, _ty = threadIdx.x >> 5;")
            out.append("    const int64_t _tr = _trip / _tn, _col = (int64_t)blockIdx.x * 32 + _tx;")
            out.append(f"    const int64_t _r0 = (int64_t)blockIdx.y * {COLBLOCK_ROWS}, "
                       f"_r1 = _r0 + {COLBLOCK_ROWS} < _tr ? _r0 + {COLBLOCK_ROWS} : _tr;")
            out.append("    if (_col < _tn) {")
            out.append("        for (int64_t _row = _r0 + _ty; _row < _r1; _row += 8) {")
            out.append("            const int64_t _q = _row * _tn + _col;   // idx - 1")
            out.append("            const int64_t _k = _st > 0 ? _q : _trip - 1 - _q;")
            out += lines
            out.append("        }")
            out.append("    }")
            for q, n in enumerate(sites):
                out.append(f"    __shared__ {et(n)} _cb{q}[8][32];")
                out.append(f"    _cb{q}[_ty][_tx] = {acc[n]};")
            out.append("    __syncthreads();")
            out.append("    if (_ty == 0 && _col < _tn) {")
            for q, n in enumerate(sites):
                terms = " + ".join(f"_cb{q}[{l}][_tx]" for l in range(8))
                out.append(f"        const {et(n)} _v{q} = {terms};")
                out.append(f"        if (_v{q} != ({et(n)})0) stade_lowered::atomic_add(&a.A_{cname(n)}[{ix[n]}], _v{q});")
            out.append("    }")
        return f"__global__ __launch_bounds__(256) void k{k}t(const Args a) {{\n" + "\n".join(out) + "\n}\n"

    # -- parallel loops -----------------------------------------------------------------------
    def parallel(self, op: ParOp) -> None:
        fl, pl = self.fl, op.pl
        loop = pl.loop
        k = self.nk
        self.nk += 1
        hl = self.hlv
        v = loop.var
        inner = {s.var for s in walk_stmts(loop.body) if isinstance(s, For)}
        priv = [n for n in pl.private if n not in hl]
        reds = {n: f"r_{cname(n)}" for n in pl.reductions}
        inv = sorted(n for n in pl.reads if n not in priv and n not in reds and n not in hl and n != v and n in fl.scalars)
        atomic = [n for n, u in pl.arrays.items() if u.kind == "atomic"]
        # accumulations at one index no iteration changes: a register per thread, added once
        # per block after the loop (not in the narrow-output form, whose lanes share the work)
        hoist = {n: f"h_{cname(n)}" for n, u in sorted(pl.arrays.items()) if u.kind == "atomic" and u.hoist}
        # LDS-privatised variants: PRIV = c + 1 takes candidate c's accumulations into a
        # block-private copy (the host picks the first candidate small enough, with enough
        # iterations per element); PRIV = 0 uses wave-aggregated global atomics only
        cands = sorted(n for n in atomic if n not in hoist)
        locals_ = {n: f"x_{cname(n)}" for n in priv + inv}
        locals_[v] = f"l_{cname(v)}"

        split = split_loops(pl, fl.T)
        # the flat loops' row-block and column-block twins (launched when the host proves the
        # range whole rows of at least TWIN_MIN_N, at least TWIN_MIN_ROWS of them)
        int_args = {a for a in fl.f.args if a not in fl.arrays and fl.scalars.get(a) == "i"}
        twin = None if split or os.environ.get("STADE_LOWER_TWINS", "1") == "0" else flat_twin(pl, int_args)
        if twin is not None and not fl.host_ok(loop.rng, set(hl)):
            twin = None
        if twin is not None:
            fl.twins.append((v, twin.kind, list(twin.sites)))

        def body_lines(parallel: bool, lds: str | None, wave: bool = False, twin_sites: dict | None = None,
                       twin_ix: dict | None = None, xs: bool = False) -> list[str]:
            ctx = Ctx(fl, dict(locals_), hl, acc={n: "atomic" for n in atomic}, serial_acc=not parallel,
                      reductions=reds, lds=lds,
                      hoist=twin_sites if twin_sites is not None else (hoist if parallel and not wave else None))
            ctx.site_ix = twin_ix or {}
            em = Emitter(fl, ctx)
            if wave:
                em.split_loops = split
                em.lane0 = True
            if xs:
                em.share_var, em.share_n = "_sh", "_nsh"
                em.xsum = lambda part, t: f"stade_lowered::xgroup_sum<{XSPLIT_NW}, XG>({part}, {xs_lds[t]})"
                em.act = "_act"
                em.group = "XG"
            em.ind = 3
            em.emit(f"const int64_t l_{cname(v)} = _lo + _k * _st;")
            for n in priv:
                ct = fl.cty(fl.scalars[n])
                if n in pl.reset:
                    c, _ = fl.ex(pl.reset[n], ctx)
                    em.emit(f"{ct} x_{cname(n)} = _k == 0 ? f0_{cname(n)} : ({ct})({c});")
                else:
                    em.emit(f"{ct} x_{cname(n)} = ({ct})0;")
            em.block(loop.body)
            em.emit(f"goto _next_iter{em.u};")
            em.emit(f"_next_iter{em.u}:;")
            if pl.live_out:
                em.emit("if (_k == _trip - 1) {")
                for n in pl.live_out:
                    em.emit(f"    wb.v_{cname(n)} = x_{cname(n)};")
                em.emit("}")
            return em.lines

        ctx0 = Ctx(fl, dict(locals_), hl)
        lo, _ = fl.ex(loop.rng.lo, ctx0)
        hi, _ = fl.ex(loop.rng.hi, ctx0)
        st = "1" if loop.rng.step is None else fl.ex(loop.rng.step, ctx0)[0]
        guards = self.guard_code(pl, ctx0)
        head = [f"    if (!({self.pred_code(op.pred)})) return;"]
        for n in inv:
            head.append(f"    const {fl.cty(fl.scalars[n])} x_{cname(n)} = fr.v_{cname(n)};")
        for n in priv:
            if n in pl.reset:
                head.append(f"    const {fl.cty(fl.scalars[n])} f0_{cname(n)} = fr.v_{cname(n)};")
        head.append(f"    const int64_t _lo = {lo}, _st = {st}, _trip = stade_lowered::jl_trip(_lo, _st, {hi});")
        red_decl = [f"    {fl.cty(fl.scalars[n])} {r} = 0;" for n, r in reds.items()]
        out = list(head)
        out.append(f"    if (!({guards})) {{")
        out.append("        // an index condition of the one-thread-per-iteration form fails: the loop in order")
        out.append("        if (blockIdx.x != 0 || threadIdx.x != 0) return;")
        out += ["    " + x for x in red_decl]
        out.append("        for (int64_t _k = 0; _k < _trip; ++_k) {")
        out += body_lines(False, None)
        out.append("        }")
        for n, r in reds.items():
            out.append(f"        fr.v_{cname(n)} += {r};")
        out.append("        return;")
        out.append("    }")
        out += red_decl

        def et_of(n):
            return "int64_t" if fl.arrays[n] == "i" else fl.fty
        out += [f"    {et_of(n)} {r} = 0;" for n, r in hoist.items()]
        for c, n in enumerate(cands):
            n_len = Ctx(fl, {}, hl).length(n)
            out.append(f"    if constexpr (PRIV == {c + 1}) {{")
            out.append(f"        {et_of(n)}* lds_priv = reinterpret_cast<{et_of(n)}*>(lds_raw);")
            out.append(f"        for (int64_t _j = threadIdx.x; _j < {n_len}; _j += blockDim.x) lds_priv[_j] = ({et_of(n)})0;")
            out.append("        __syncthreads();")
            out.append("    }")
        out.append("    for (int64_t _k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; _k < _trip; _k += (int64_t)gridDim.x * blockDim.x) {")
        if cands:
            out.append("        if constexpr (PRIV == 0) {")
            out += ["    " + x for x in body_lines(True, None)]
            for c, n in enumerate(cands):
                out.append(f"        }} else if constexpr (PRIV == {c + 1}) {{")
                out.append(f"            {et_of(n)}* lds_priv = reinterpret_cast<{et_of(n)}*>(lds_raw);")
                out += ["    " + x for x in body_lines(True, n)]
            out.append("        }")
        else:
            out += body_lines(True, None)
        out.append("    }")
        for c, n in enumerate(cands):
            n_len = Ctx(fl, {}, hl).length(n)
            out.append(f"    if constexpr (PRIV == {c + 1}) {{")
            out.append(f"        {et_of(n)}* lds_priv = reinterpret_cast<{et_of(n)}*>(lds_raw);")
            out.append("        __syncthreads();")
            out.append(f"        for (int64_t _j = threadIdx.x; _j < {n_len}; _j += blockDim.x)")
            out.append(f"            if (lds_priv[_j] != ({et_of(n)})0) stade_lowered::atomic_add(&a.A_{cname(n)}[_j], lds_priv[_j]);")
            out.append("        if (threadIdx.x == 0) stade_lowered::count(a.st, stade_lowered::ST_PRIV_BLOCK);")
            out.append("    }")
        # the block's sums: with few blocks one atomic addition per block; with more, stored per
        # block (no atomics) and added in block order into their targets by the one-block fold
        # kernel k<k>f that the host then launches after this one (same-address atomics
        # serialise: thousands of them cost more than a launch)
        parts = []   # (C type, slot array, register, the fold's addition of its total `_s`, target)
        for n, r in reds.items():
            parts.append((fl.cty(fl.scalars[n]), f"g_p{k}_{len(parts)}", r, f"fr.v_{cname(n)} += _s;",
                          f"&fr.v_{cname(n)}"))
        for n, r in hoist.items():
            ix = Ctx(fl, dict(locals_), hl).lin(pl.arrays[n].index)
            add = (f"a.A_{cname(n)}[_i] += _s;" if fl.inbounds else
                   f"if ((uint64_t)_i < (uint64_t)a.N_{cname(n)}) a.A_{cname(n)}[_i] += _s;")
            tgt = (f"&a.A_{cname(n)}[_i]" if fl.inbounds else
                   f"(uint64_t)_i < (uint64_t)a.N_{cname(n)} ? &a.A_{cname(n)}[_i] : nullptr")
            parts.append((et_of(n), f"g_p{k}_{len(parts)}", r, f"{{ const int64_t _i = {ix}; {add} }}",
                          (ix, tgt)))
        if parts:
            out.append(f"    if (gridDim.x <= {FOLD_MIN_BLOCKS}) {{")
            for ct, arr, r, _, tgt in parts:
                if isinstance(tgt, tuple):
                    out.append(f"        {{ const int64_t _i = {tgt[0]};")
                    out.append(f"          stade_lowered::block_add({tgt[1]}, {r}, reinterpret_cast<{ct}*>(_blk), a.st); }}")
                else:
                    out.append(f"        stade_lowered::block_add({tgt}, {r}, reinterpret_cast<{ct}*>(_blk), a.st);")
            out.append("    } else {")
            for ct, arr, r, _, _ in parts:
                self.kern.append(f"__device__ {ct} {arr}[{MAX_BLOCKS}];   // k{k}'s block sums (at most {MAX_BLOCKS} blocks)\n")
                out.append(f"        stade_lowered::block_part({arr}, {r}, reinterpret_cast<{ct}*>(_blk), a.st);")
            out.append("    }")
        pre = "    extern __shared__ __align__(16) unsigned char lds_raw[];\n    (void)lds_raw;\n" if cands else ""
        if parts:
            pre += "    __shared__ double _blk[16];  // the waves' sums of block_part\n"
        self.kern.append(f"template <int PRIV>\n__global__ __launch_bounds__(256) void k{k}(const Args a) {{\n" + pre +
                         "\n".join(out) + "\n}\n")
        if parts:
            fo = list(head)
            # the loop's last values committed here (when it ran), instead of by a one-thread
            # kernel of their own; in either form the last iteration left them in `wb`
            if pl.live_out:
                fo.append("    if (threadIdx.x == 0 && _trip > 0) {")
                for n in pl.live_out:
                    fo.append(f"        fr.v_{cname(n)} = wb.v_{cname(n)};")
                fo.append("    }")
            # (a failed index condition ran the loop in order on one thread, which added its sums)
            fo.append(f"    if (!({guards})) return;")
            # every slot's load in flight at once, then the sums
            for c, (ct, arr, r, add, _) in enumerate(parts):
                fo.append(f"    {ct} _v{c}[stade_lowered::FOLD_PER];")
                fo.append(f"    stade_lowered::fold_load({arr}, _nb, _v{c});")
            for c, (ct, arr, r, add, _) in enumerate(parts):
                fo.append(f"    {{ const {ct} _s = stade_lowered::fold_sum(_v{c}, reinterpret_cast<{ct}*>(_blk));")
                fo.append(f"      if (threadIdx.x == 0 && _s != ({ct})0) {add} }}")
            self.kern.append(f"__global__ __launch_bounds__(stade_lowered::FOLD_NT) void k{k}f(const Args a, const unsigned _nb) {{\n"
                             "    __shared__ double _blk[16];\n" + "\n".join(fo) + "\n}\n")

        # `_cm<k>`: the fold ran and committed the loop's last values (live_out)
        commit_in_fold = bool(parts) and bool(pl.live_out)
        if commit_in_fold:
            self.hemit(f"bool _cm{k} = false;")

        def fold(nb):
            if parts:
                self.hemit(f"if ({nb} > {FOLD_MIN_BLOCKS}) {{")
                self.hemit(f"    k{k}f<<<1, stade_lowered::FOLD_NT, 0, stream>>>(a, {nb});")
                self.hemit(f"    if ((_e = hipGetLastError()) != hipSuccess) return _fail(_e, \"k{k}f\");")
                if commit_in_fold:
                    self.hemit(f"    _cm{k} = true;")
                self.hemit("}")
        # the lanes-over-iterations variant of the narrow-output form, for inner loops whose
        # accesses run along the outer loop (a column-major matrix read by rows)
        xsplit = bool(split) and os.environ.get("STADE_LOWER_XSPLIT", "1") != "0" and self.xsplit_ok(pl, split)
        if xsplit:
            fl.xsplits.append(v)
            tys = sorted({fl.scalars[t] for ts in split.values() for t in ts})
            xs_lds = {}
            pre_x = []
            for t in tys:
                ct = fl.cty(t)
                nm = f"_xs{t}"
                pre_x.append(f"    __shared__ {ct} {nm}[{XSPLIT_NW} * 64];")
                xs_lds[t] = nm
            sp = list(head)
            sp.append(f"    if (!({guards})) {{")
            sp.append("        if (blockIdx.x != 0 || threadIdx.x != 0) return;")
            sp += ["    " + x for x in red_decl]
            sp.append("        for (int64_t _k = 0; _k < _trip; ++_k) {")
            sp += body_lines(False, None)
            sp.append("        }")
            for n, r in reds.items():
                sp.append(f"        fr.v_{cname(n)} += {r};")
            sp.append("        return;")
            sp.append("    }")
            sp += red_decl
            # XG consecutive outer iterations a block (16, 32 or 64, chosen by the host from the
            # trip count so that few rows still fill the CUs): lane l of wave w takes iteration
            # l % XG and share l / XG + (64 / XG) w of the shared inner loops
            sp.append(f"    constexpr int _nsh = {XSPLIT_NW} * 64 / XG;")
            sp.append("    const int _ln = threadIdx.x & 63, _wv = threadIdx.x >> 6;")
            sp.append("    const int _r = _ln & (XG - 1), _sh = _ln / XG + (64 / XG) * _wv;")
            sp.append("    if (threadIdx.x == 0) stade_lowered::count(a.st, stade_lowered::ST_XSPLIT_BLOCK);")
            # block-uniform steps of XG iterations: every thread reaches the waves' barriers
            # (a lane past the range computes the last iteration again and stores nothing)
            sp.append("    for (int64_t _base = (int64_t)blockIdx.x * XG; _base < _trip; _base += (int64_t)gridDim.x * XG) {")
            sp.append("        const bool _act = _base + _r < _trip;")
            sp.append("        const int64_t _k = _act ? _base + _r : _trip - 1;")
            sp += body_lines(True, None, wave=True, xs=True)
            sp.append("    }")
            for n, r in reds.items():
                sp.append(f"    {r} = stade_lowered::wave_sum({r});")
                sp.append(f"    if (_ln == 0 && {r} != 0) stade_lowered::atomic_add(&fr.v_{cname(n)}, {r});")
            self.kern.append(f"template <int XG>\n__global__ __launch_bounds__({64 * XSPLIT_NW}) void k{k}s(const Args a) {{\n"
                             + "\n".join(pre_x) + "\n" + "\n".join(sp) + "\n}\n")
        if split and not xsplit:
            # the narrow-output form: a wave per iteration, its lanes sharing the inner loops
            sp = list(head)
            sp.append(f"    if (!({guards})) {{")
            sp.append("        if (blockIdx.x != 0 || threadIdx.x != 0) return;")
            sp += ["    " + x for x in red_decl]
            sp.append("        for (int64_t _k = 0; _k < _trip; ++_k) {")
            sp += body_lines(False, None)
            sp.append("        }")
            for n, r in reds.items():
                sp.append(f"        fr.v_{cname(n)} += {r};")
            sp.append("        return;")
            sp.append("    }")
            sp += red_decl
            sp.append("    const int _lane = threadIdx.x & 63;")
            sp.append("    if (threadIdx.x == 0) stade_lowered::count(a.st, stade_lowered::ST_SPLIT_BLOCK);")
            sp.append("    for (int64_t _k = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6; _k < _trip;"
                      " _k += ((int64_t)gridDim.x * blockDim.x) >> 6) {")
            sp += body_lines(True, None, wave=True)
            sp.append("    }")
            for n, r in reds.items():
                sp.append(f"    {r} = stade_lowered::wave_sum({r});")
                sp.append(f"    if ((threadIdx.x & 63) == 0 && {r} != 0) stade_lowered::atomic_add(&fr.v_{cname(n)}, {r});")
            self.kern.append(f"__global__ __launch_bounds__(256) void k{k}s(const Args a) {{\n" + "\n".join(sp) + "\n}\n")
        if twin is not None:
            self.kern.append(self.twin_kernel(k, twin, head, guards, body_lines, fl.ex(twin.N, ctx0)[0]))
        # host: grid from the trip count when the host can evaluate it
        if fl.host_ok(loop.rng, set(hl)):
            hctx = HostCtx(fl, self.hlv)
            hlo, hhi = hctx.ex(loop.rng.lo), hctx.ex(loop.rng.hi)
            hst = "1" if loop.rng.step is None else hctx.ex(loop.rng.step)
            self.hemit("{")
            self.hind += 1
            self.hemit(f"const int64_t _trip = stade_lowered::jl_trip({hlo}, {hst}, {hhi});")
            if split:
                # few iterations with long inner loops: a wave per iteration
                first = next(t for t in walk_stmts(loop.body) if isinstance(t, For) and id(t) in split)
                if fl.host_ok(first.rng, set(hl)):
                    ilo, ihi = hctx.ex(first.rng.lo), hctx.ex(first.rng.hi)
                    ist = "1" if first.rng.step is None else hctx.ex(first.rng.step)
                    cond = (f"_trip > 0 && _trip <= {SPLIT_MAX_TRIP} && "
                            f"stade_lowered::jl_trip({ilo}, {ist}, {ihi}) >= {SPLIT_MIN_INNER}")
                else:
                    cond = f"_trip > 0 && _trip <= {SPLIT_MAX_TRIP_UNKNOWN}"
                self.hemit(f"if ({cond}) {{")
                self.hind += 1
                if xsplit:
                    # rows a block: 64 when that still gives 256 blocks, else 32, else 16 (a
                    # wave's loads then cover 16 rows of 4 columns: 128-byte segments)
                    for g, cond in ((64, f"_trip >= {64 * 256}"), (32, f"_trip >= {32 * 256}"), (16, None)):
                        if cond:
                            self.hemit(f"if ({cond}) {{")
                        else:
                            self.hemit("{")
                        self.hind += 1
                        self.launch(f"k{k}s", f"(unsigned)std::min<int64_t>((_trip + {g - 1}) / {g}, {MAX_BLOCKS})",
                                    str(64 * XSPLIT_NW), "0", f"<{g}>")
                        self.hind -= 1
                        self.hemit("} else" if cond else "}")
                else:
                    self.launch(f"k{k}s", f"(unsigned)std::min<int64_t>((_trip + 3) / 4, {MAX_BLOCKS})", "256", "0")
                self.hind -= 1
                self.hemit("} else")
            if twin is not None:
                hN = hctx.ex(twin.N)
                self.hemit(f"const int64_t _tn = {hN}, _tr = _tn > 0 ? _trip / _tn : 0;")
                if twin.kind == "row":
                    # blocks a row: about ROWBLOCK_GRID blocks in all, each at least ROWBLOCK_CHUNK iterations
                    self.hemit(f"const int64_t _ts = std::max<int64_t>(1, std::min<int64_t>((_tn + {ROWBLOCK_CHUNK - 1}) / "
                               f"{ROWBLOCK_CHUNK}, ({ROWBLOCK_GRID} + _tr - 1) / "
                               f"std::max<int64_t>(_tr, 1)));")
                    cond = (f"_tn >= {TWIN_MIN_N} && _trip > 0 && _trip % _tn == 0 && _tr >= 1 && "
                            f"_tr * _ts <= (int64_t)2147483647")
                else:
                    cond = (f"_tn >= {TWIN_MIN_N} && _trip > 0 && _trip % _tn == 0 && _tr >= {TWIN_MIN_ROWS}"
                            f" && _tr <= (int64_t)65535 * {COLBLOCK_ROWS}")
                self.hemit(f"if ({cond}) {{")
                self.hind += 1
                if twin.kind == "row":
                    self.launch(f"k{k}t", "(unsigned)(_tr * _ts)", "256", "0")
                else:
                    self.launch(f"k{k}t", f"dim3((unsigned)((_tn + 31) / 32), (unsigned)((_tr + {COLBLOCK_ROWS - 1}) / {COLBLOCK_ROWS}))",
                                "256", "0")
                self.hind -= 1
                self.hemit("} else")
            self.hemit("if (_trip > 0) {")
            self.hind += 1
            self.hemit(f"const unsigned _g = (unsigned)std::min<int64_t>((_trip + 255) / 256, {MAX_BLOCKS});")
            if cands:
                self.hemit("int _priv = 0;")
                self.hemit("size_t _lds = 0;")
                for c, n in enumerate(cands):
                    es = 8 if fl.arrays[n] == "i" or fl.fty == "double" else 4
                    hlen = hctx.length(n)
                    cond = f"{hlen} > 0 && {hlen} * {es} <= {PRIV_MAX_BYTES} && _trip >= {PRIV_RATIO} * {hlen}"
                    self.hemit(("if" if c == 0 else "else if") + f" ({cond}) {{ _priv = {c + 1}; _lds = (size_t){hlen} * {es}; }}")
                self.hemit("switch (_priv) {")
                for c in range(len(cands) + 1):
                    self.hemit(f"case {c}:")
                    self.hind += 1
                    self.launch(f"k{k}", "_g", "256", "_lds", f"<{c}>")
                    self.hemit("break;")
                    self.hind -= 1
                self.hemit("}")
            else:
                self.launch(f"k{k}", "_g", "256", "0", "<0>")
            fold("_g")
            self.hind -= 1
            self.hemit("}")
            self.hind -= 1
            self.hemit("}")
        else:
            self.launch(f"k{k}", str(MAX_BLOCKS), "256", "0", "<0>")
            fold(f"{MAX_BLOCKS}u")
        if pl.live_out:
            kc = self.nk
            self.nk += 1
            lines = [f"    if (!({self.pred_code(op.pred)})) return;"]
            for n in inv:
                lines.append(f"    const {fl.cty(fl.scalars[n])} x_{cname(n)} = fr.v_{cname(n)};")
            lines.append(f"    const int64_t _lo = {lo}, _st = {st}, _trip = stade_lowered::jl_trip(_lo, _st, {hi});")
            lines.append("    if (_trip <= 0) return;")
            for n in pl.live_out:
                lines.append(f"    fr.v_{cname(n)} = wb.v_{cname(n)};")
            self.one_thread_kernel(kc, lines)
            if commit_in_fold:
                self.hemit(f"if (!_cm{k}) {{")
                self.hind += 1
                self.launch(f"k{kc}")
                self.hind -= 1
                self.hemit("}")
            else:
                self.launch(f"k{kc}")

    def xsplit_ok(self, pl: ParallelLoop, split: dict) -> bool:
        """The lanes-over-iterations form: every shared inner loop at the top of the body (the
        waves meet at a barrier after each), no break, continue or return, and fewer stores and
        accumulations in those loops that step along the outer loop with a stride other than 1
        than ones that step along their own index with a stride other than 1 (the lanes then
        update adjacent elements: a column-major matrix updated by rows).  Reads alone do not
        choose it: the lanes' scattered reads of a wave-per-iteration loop share cache lines with
        the neighbouring waves' (measured on the affine row sums: 9.8 against 19 µs), while
        scattered atomic updates do not combine."""
        from .analysis import NotAffine, _linear_index, linear_in, to_poly
        fl, loop = self.fl, pl.loop
        if any(isinstance(t, (Break, Continue, Return)) for t in walk_stmts(loop.body)):
            return False
        tops = {id(t) for t in loop.body if isinstance(t, For)}
        if not set(split) <= tops:
            return False
        # stores outside the shared loops are wave 0's, each after a barrier that orders every
        # wave's earlier reads of the element before it: only straight-line, top-level ones
        inside = {id(x) for L in loop.body if id(L) in split for x in walk_stmts([L])}
        top = {id(t) for t in loop.body}
        for t in walk_stmts(loop.body):
            if (isinstance(t, Assign) and isinstance(t.lhs, Ref) and id(t) not in inside and id(t) not in top):
                return False
        count = {}
        for t in walk_stmts(loop.body):
            if isinstance(t, Assign) and isinstance(t.lhs, Var):
                count[t.lhs.name] = count.get(t.lhs.name, 0) + 1
        env = {t.lhs.name: t.rhs for t in walk_stmts(loop.body) if isinstance(t, Assign) and isinstance(t.lhs, Var)
               and fl.T.scalars.get(t.lhs.name) == "i" and count[t.lhs.name] == 1}
        unit = lambda c: c is not None and c[0] in ({(): 1}, {(): -1})
        bad_x = bad_s = 0
        for L in loop.body:
            if id(L) not in split:
                continue
            for t in walk_stmts(L.body):
                refs = [t.lhs] if isinstance(t, Assign) and isinstance(t.lhs, Ref) else []
                for ref in refs:
                    try:
                        p = to_poly(_linear_index(ref, fl.T), env, fl.T)
                    except NotAffine:
                        continue
                    co, ci = linear_in(p, loop.var), linear_in(p, L.var)
                    if co is None or ci is None:
                        continue
                    if co[0] and not unit(co):
                        bad_x += 1
                    if ci[0] and not unit(ci):
                        bad_s += 1
        return bad_x < bad_s

    def guard_code(self, pl: ParallelLoop, ctx) -> str:
        conds = []
        for g in pl.guards:
            kind = g[0]
            if kind == "nonzero":
                conds.append(f"({self.poly(g[1], ctx)}) != 0")
            elif kind == "positive":
                conds.append(f"({self.poly(g[1], ctx)}) > 0")
            elif kind == "nonneg_over_range":
                v = pl.loop.var
                at_lo = self.poly(g[1], ctx, {v: "_lo"})
                at_hi = self.poly(g[1], ctx, {v: "(_lo + (_trip - 1) * _st)"})
                conds.append(f"(_trip <= 0 || (({at_lo}) >= 0 && ({at_hi}) >= 0))")
        return " && ".join(conds) if conds else "true"

    def poly(self, p: dict, ctx, subst: dict | None = None) -> str:
        subst = subst or {}
        if not p:
            return "((int64_t)0)"
        terms = []
        for m, c in sorted(p.items()):
            fs = [f"((int64_t){c}LL)"]
            for a in m:
                fs.append(self.atom(a, ctx, subst))
            terms.append(" * ".join(fs))
        return "(" + " + ".join(terms) + ")"

    def atom(self, a, ctx, subst):
        if a[0] == "v":
            n = a[1]
            if n in subst:
                return subst[n]
            if n.startswith("size(") or n.startswith("length("):
                inner = n[n.index("(") + 1:-1].split(",")
                if n.startswith("length("):
                    return ctx.length(inner[0])
                return ctx.dim(inner[0], int(inner[1]) - 1 if len(inner) > 1 else 0)
            return ctx.var(n) if n not in ctx.locals else ctx.locals[n]
        X, N = _thaw(a[1]), _thaw(a[2])
        x, n = self.poly(X, ctx, subst), self.poly(N, ctx, subst)
        return f"({x} / {n})" if a[0] == "div" else f"stade_lowered::jl_mod({x}, {n})"

    # -- structure ------------------------------------------------------------------------------
    def ops(self, ops):
        fl = self.fl
        for op in ops:
            if isinstance(op, SerialOp):
                self.serial(op.stmts, op.pred)
            elif isinstance(op, ParOp):
                self.parallel(op)
            elif isinstance(op, ReturnOp):
                self.serial([], op.pred, op.value)
            elif isinstance(op, GemmOp):
                if isinstance(op.g, GemmT):
                    self.gemm_tab(op.g)
                else:
                    self.gemm(op.g)
            elif isinstance(op, AllocOp):
                hctx = HostCtx(fl, self.hlv)
                et = 8 if fl.arrays[op.name] == "i" or fl.fty == "double" else 4
                slot = self.nalloc
                self.nalloc += 1
                self.hemit(f"a.D_{cname(op.name)}[0] = std::max<int64_t>(0, {hctx.ex(op.alloc.n)});")
                self.hemit(f"a.N_{cname(op.name)} = a.D_{cname(op.name)}[0];")
                self.hemit(f"if (!(a.A_{cname(op.name)} = reinterpret_cast<decltype(a.A_{cname(op.name)})>("
                           f"_buf({slot}, (size_t)a.D_{cname(op.name)}[0] * {et})))) return _fail(hipErrorOutOfMemory, \"{op.name}\");")
            elif isinstance(op, HostLoopOp):
                hctx = HostCtx(fl, self.hlv)
                lo, hi = hctx.ex(op.loop.rng.lo), hctx.ex(op.loop.rng.hi)
                st = "1" if op.loop.rng.step is None else hctx.ex(op.loop.rng.step)
                self.hemit("{")
                self.hind += 1
                self.hemit(f"const int64_t _lo{op.slot} = {lo}, _st{op.slot} = {st}, "
                           f"_n{op.slot} = stade_lowered::jl_trip(_lo{op.slot}, _st{op.slot}, {hi});")
                self.hemit(f"for (int64_t _k{op.slot} = 0; _k{op.slot} < _n{op.slot}; ++_k{op.slot}) {{")
                self.hind += 1
                self.hemit(f"a.hl[{op.slot}] = _lo{op.slot} + _k{op.slot} * _st{op.slot};")
                saved = dict(self.hlv)
                self.hlv[op.loop.var] = op.slot
                self.ops(op.ops)
                self.hlv = saved
                self.hind -= 1
                self.hemit("}")
                self.hind -= 1
                self.hemit("}")
            elif isinstance(op, IfOp):
                k = self.nk
                self.nk += 1
                reads = set()
                for c, _ in op.node.branches:
                    reads |= {n for n in _reads_of(c) if n not in fl.arrays}
                names = sorted(n for n in reads if n in fl.scalars and n not in self.hlv)
                ctx = Ctx(fl, {n: f"x_{cname(n)}" for n in names}, self.hlv)
                lines = [f"    if (!({self.pred_code(op.pred)})) return;"]
                for n in names:
                    lines.append(f"    const {fl.cty(fl.scalars[n])} x_{cname(n)} = fr.v_{cname(n)};")
                for f in op.flags:
                    lines.append(f"    fr.flag[{f}] = 0;")
                for j, (c, _) in enumerate(op.node.branches):
                    cc, _ = fl.ex(c, ctx)
                    lines.append(("    if" if j == 0 else "    else if") + f" ({cc}) fr.flag[{op.flags[j]}] = 1;")
                if op.node.orelse is not None:
                    lines.append(f"    else fr.flag[{op.flags[-1]}] = 1;")
                self.one_thread_kernel(k, lines)
                self.launch(f"k{k}")
                for b in op.branches:
                    self.ops(b)

    def gemm(self, g: Gemm) -> None:
        """Host code of a matrix product (contract.py) on the fp32 matrix-core GEMM: the plan's
        tile width and K split (an accumulating product adds its split's slices by atomics, a
        stored one reduces them from a partials buffer)."""
        fl = self.fl
        hctx = HostCtx(fl, self.hlv)
        self.uses_gemm = True
        n = self.ngemm
        self.ngemm += 1
        km = {(x.a_km, x.b_km) for x in g.segs}
        assert len(g.segs) in (1, 2) and len(km) == 1
        a_km, b_km = km.pop()
        tf = lambda b: "true" if b else "false"
        self.hemit("{")
        self.hind += 1
        self.hemit(f"const int64_t _gm = {hctx.ex(g.M)}, _gn = {hctx.ex(g.N)};")
        ks = []
        for j, x in enumerate(g.segs):
            self.hemit(f"const int64_t _gk{j} = {hctx.ex(x.K)};")
            ks.append(f"_gk{j}")
        kt = " + ".join(ks)
        self.hemit(f"if (_gm > 0x7fffffff || _gn > 0x7fffffff || {kt} > 0x7fffffff) "
                   f"return _fail(hipErrorInvalidValue, \"matrix product {n} into {g.out}: a dimension past 2^31\");")
        self.hemit("if (_gm > 0 && _gn > 0) {")
        self.hind += 1
        self.hemit("stade::gemm::Args _g{};")
        self.hemit(f"_g.nseg = {len(g.segs)};")
        self.hemit("_g.M = (int)_gm;")
        self.hemit("_g.N = (int)_gn;")
        for j, x in enumerate(g.segs):
            self.hemit(f"_g.seg[{j}] = stade::gemm::Seg{{a.A_{cname(x.a)} + ({hctx.ex(x.a_off)}), "
                       f"a.A_{cname(x.b)} + ({hctx.ex(x.b_off)}), (long)({hctx.ex(x.lda)}), (long)({hctx.ex(x.ldb)}), "
                       f"(int)_gk{j}}};")
        self.hemit(f"const stade::gemm::Plan _p = stade::gemm::plan(_g.M, _g.N, (int)({kt}), stade::gemm::device_cus(), 1, "
                   f"{tf(g.acc)});")
        if not g.acc:
            slot = self.nalloc
            self.nalloc += 1
            self.hemit(f"if (_p.ksplit > 1 && !(_g.part = (float*)_buf({slot}, (size_t)_p.ksplit * (size_t)_gm * (size_t)_gn * 4)))")
            self.hemit(f"    return _fail(hipErrorOutOfMemory, \"matrix product {n}: partial sums\");")
        self.hemit(f"const stade_lowered::GemmOut<{tf(g.acc)}> _ep{{a.A_{cname(g.out)} + ({hctx.ex(g.out_off)}), "
                   f"(long)({hctx.ex(g.out_sm)}), (long)({hctx.ex(g.out_sn)})}};")
        self.hemit(f"if ((_e = stade::gemm::launch<{tf(a_km)}, {tf(b_km)}>(_g, _ep, stream, _p)) != hipSuccess) "
                   f"return _fail(_e, \"matrix product {n} into {g.out}\");")
        self.hind -= 1
        self.hemit("}")
        self.hind -= 1
        self.hemit("}")

    def gemm_tab(self, g: GemmT) -> None:
        """Host code of a table-addressed product (contract.py's table form) on the matrix
        cores (stade_lowered::gemm_tab)."""
        fl = self.fl
        hctx = HostCtx(fl, self.hlv)
        self.uses_gemm = True
        n = self.ngemm
        self.ngemm += 1
        dim = lambda d: (f"stade_lowered::TabDim{{a.A_{cname(d.table)}, 0}}" if d.table is not None
                         else f"stade_lowered::TabDim{{nullptr, (long)({hctx.ex(d.stride)})}}")
        self.hemit("{")
        self.hind += 1
        self.hemit(f"const int64_t _gm = {hctx.ex(g.M)}, _gn = {hctx.ex(g.N)}, _gk = {hctx.ex(g.K)};")
        self.hemit(f"if (_gm > 0x7fffffff || _gn > 0x7fffffff || _gk > 0x7fffffff) "
                   f"return _fail(hipErrorInvalidValue, \"matrix product {n} into {g.out}: a dimension past 2^31\");")
        self.hemit("stade_lowered::GemmTabArgs _g{};")
        self.hemit(f"_g.A = a.A_{cname(g.a)} + ({hctx.ex(g.a_off)});")
        self.hemit(f"_g.ar = {dim(g.ar)};")
        self.hemit(f"_g.ak = {dim(g.ak)};")
        self.hemit(f"_g.B = a.A_{cname(g.b)} + ({hctx.ex(g.b_off)});")
        self.hemit(f"_g.bk = {dim(g.bk)};")
        self.hemit(f"_g.bc = {dim(g.bc)};")
        self.hemit(f"_g.C = a.A_{cname(g.out)} + ({hctx.ex(g.out_off)});")
        self.hemit(f"_g.ro = {dim(g.ro)};")
        self.hemit(f"_g.co = {dim(g.co)};")
        self.hemit("_g.M = (int)_gm;")
        self.hemit("_g.N = (int)_gn;")
        self.hemit("_g.K = (int)_gk;")
        tf = lambda b: "true" if b else "false"
        self.hemit(f"if ((_e = stade_lowered::gemm_tab<{g.mode}, {tf(g.a_km)}, {tf(g.b_km)}>(_g, stream)) != hipSuccess) "
                   f"return _fail(_e, \"matrix product {n} into {g.out}\");")
        self.hind -= 1
        self.hemit("}")

    def source(self) -> str:
        fl = self.fl
        f = fl.f
        fr_fields = []
        for n in fl.frame_scalars():
            fr_fields.append(f"    {fl.cty(fl.scalars[n])} v_{cname(n)};")
        args_fields = []
        for n in sorted(fl.arrays):
            et = "int64_t" if fl.arrays[n] == "i" else fl.fty
            args_fields.append(f"    {et}* A_{cname(n)};")
            args_fields.append(f"    int64_t D_{cname(n)}[{fl.T.ndim.get(n, 1)}];")
            args_fields.append(f"    int64_t N_{cname(n)};   // elements (the product of the dimensions)")
        for n in f.args:
            if n not in fl.arrays:
                args_fields.append(f"    {fl.cty(fl.scalars.get(n, 'f'))} s_{cname(n)};")
        args_fields.append(f"    int64_t hl[{max(1, fl.nhl)}];")
        args_fields.append("    unsigned long long* st;   // path statistics (null: not counted)")
        self.ops(fl.ops)
        self.merge_serial_launches()
        init = ["    fr.nret = 0;", "    fr.oob = 0;"] + [f"    fr.v_{cname(n)} = a.s_{cname(n)};" for n in f.args if n not in fl.arrays]
        init += [f"    fr.flag[{k}] = 0;" for k in range(fl.nflags)]
        params, fill = [], []
        for n in f.args:   # (parameters prefixed: a Julia name may be any C identifier)
            if n in fl.arrays:
                et = "int64_t" if fl.arrays[n] == "i" else fl.fty
                params.append(f"{et}* p_{cname(n)}")
                fill.append(f"    a.A_{cname(n)} = p_{cname(n)};")
                for d in range(fl.T.ndim.get(n, 1)):
                    params.append(f"int64_t p_{cname(n)}_d{d}")
                    fill.append(f"    a.D_{cname(n)}[{d}] = p_{cname(n)}_d{d};")
                nd = fl.T.ndim.get(n, 1)
                fill.append(f"    a.N_{cname(n)} = " + " * ".join(f"p_{cname(n)}_d{d}" for d in range(nd)) + ";")
                fill.append(f"    if (a.N_{cname(n)} < 0) return _fail(hipErrorInvalidValue, \"negative dimension of {n}\");")
            else:
                params.append(f"{fl.cty(fl.scalars.get(n, 'f'))} p_{cname(n)}")
                fill.append(f"    a.s_{cname(n)} = p_{cname(n)};")
        params += ["double* ret", "int64_t* iret", "hipStream_t stream"]
        nb = max(1, self.nalloc)
        return "\n".join([
            f"namespace {self.ns} {{",
            "using namespace stade_lowered;",
            "struct Frame {",
            *fr_fields,
            f"    int32_t flag[{max(1, fl.nflags)}];",
            "    double r[16];",
            "    int64_t ri[16];",
            "    int32_t rk[16];",
            "    int32_t nret;",
            "    int32_t oob;      // an index was outside its array",
            "};",
            "__device__ Frame fr;   // the function's scalars (one per device: calls that overlap race)",
            "__device__ Frame wb;   // values of the last iteration of a parallel loop, committed after it",
            "__device__ __forceinline__ void oob() { fr.oob = 1; }",
            "template <class T>",
            "__device__ __forceinline__ T rd(const T* p, int64_t i, int64_t n) {",
            "    if ((uint64_t)i < (uint64_t)n) return p[i];",
            "    oob();",
            "    return T(0);",
            "}",
            "template <class T>",
            "__device__ __forceinline__ void wr(T* p, int64_t i, int64_t n, T v) {",
            "    if ((uint64_t)i < (uint64_t)n) p[i] = v;",
            "    else oob();",
            "}",
            "struct Args {",
            *args_fields,
            "};",
            "__global__ __launch_bounds__(1) void kinit(const Args a) {",
            *init,
            "}",
            *self.kern,
            f"static void* g_buf[{nb}];",
            f"static size_t g_bytes[{nb}];",
            "// the launch sequences replayed as HIP graphs (functions with host loops; lowered_rt.hpp)",
            "static LaunchGraphs<Args> g_graphs;",
            "// local arrays (allocated inside the generated function): kept per process, grown on demand",
            "// (a reallocation drops the captured graphs, which hold the old address)",
            "static void* _buf(int slot, size_t bytes) {",
            "    if (bytes == 0) bytes = 8;   // an empty array still gets an address (nothing reads it)",
            "    if (g_bytes[slot] < bytes) {",
            "        if (g_buf[slot]) { (void)hipDeviceSynchronize(); g_graphs.clear(); (void)hipFree(g_buf[slot]); g_buf[slot] = nullptr; g_bytes[slot] = 0; }",
            "        if (hipMalloc(&g_buf[slot], bytes) != hipSuccess) return nullptr;",
            "        g_bytes[slot] = bytes;",
            "    }",
            "    return g_buf[slot];",
            "}",
            "// where the kernels count their accumulation paths (stade_lowered::ST_*; null: nowhere)",
            "static unsigned long long* g_stats = nullptr;",
            "// the function's launches in order on `stream` (the caller's, or a private stream under",
            "// capture): the host statements read and write nothing but the frame `a`",
            "static int32_t _launches(Args a, hipStream_t stream) {",
            "    hipError_t _e;",
            "    kinit<<<1, 1, 0, stream>>>(a);",
            "    if ((_e = hipGetLastError()) != hipSuccess) return _fail(_e, \"kinit\");",
            *self.host,
            "    return 0;",
            "}",
            "}  // namespace",
            "",
            "// Test hook, not part of the generated function's ABI: until it is called again with null,",
            "// every call of this function adds its path counts into stats[0..ST_N) (device memory).",
            f"extern \"C\" void stade_hip_gen_{cname(f.name)}_set_stats(unsigned long long* stats) {{",
            f"    {self.ns}::g_stats = stats;",
            "}",
            "// Test hook: the launch sequences captured into graphs so far, and the graph launches.",
            f"extern \"C\" void stade_hip_gen_{cname(f.name)}_graphs(int64_t* out) {{",
            f"    {self.ns}::g_graphs.counts(out);",
            "}",
            "",
            f"extern \"C\" int32_t stade_hip_gen_{cname(f.name)}({', '.join(params)}) {{",
            f"    using namespace {self.ns};",
            "    Args a;",
            "    std::memset(&a, 0, sizeof a);   // (padding too: frames are compared bytewise)",
            "    a.st = g_stats;",
            *fill,
            # a host loop issues its launches once per iteration: replayed as a graph when the
            # same frame comes back
            f"    const int32_t _rc = {'g_graphs.run(a, stream, _launches)' if fl.nhl else '_launches(a, stream)'};",
            "    if (_rc != 0) return _rc;",
            "    hipError_t _e;",
            "    Frame h;",
            "    if ((_e = hipMemcpyFromSymbolAsync(&h, HIP_SYMBOL(fr), sizeof(Frame), 0, hipMemcpyDeviceToHost, stream)) != hipSuccess)",
            "        return _fail(_e, \"returned values\");",
            "    if ((_e = hipStreamSynchronize(stream)) != hipSuccess) return _fail(_e, \"hipStreamSynchronize\");",
            f"    if (h.oob) return _bounds(\"{f.name}\");",
            "    for (int k = 0; k < h.nret && k < 16; ++k) {",
            "        if (ret) ret[k] = h.r[k];",
            "        if (iret) iret[k] = h.ri[k];",
            "    }",
            "    return h.nret;",
            "}",
            "",
        ])


class HostCtx:
    """Host-side C of an expression the host can evaluate (Int arguments, array sizes, host
    loop variables in scope)."""

    def __init__(self, fl: FuncLower, hlv: dict):
        self.fl = fl
        self.hlv = hlv

    def length(self, name):
        nd = self.fl.T.ndim.get(name, 1)
        return "(" + " * ".join(f"a.D_{cname(name)}[{d}]" for d in range(nd)) + ")"

    def ex(self, e) -> str:
        fl = self.fl
        if isinstance(e, Num):
            return f"((int64_t){int(e.text, 0)}LL)"
        if isinstance(e, Var):
            if e.name in self.hlv:
                return f"a.hl[{self.hlv[e.name]}]"
            return f"a.s_{cname(e.name)}"
        if isinstance(e, Un):
            return f"(-{self.ex(e.a)})"
        if isinstance(e, Bin):
            return f"({self.ex(e.a)} {e.op} {self.ex(e.b)})"
        if isinstance(e, Call):
            if e.fn == "length":
                return self.length(e.args[0].name)
            if e.fn == "size":
                d = int(e.args[1].text) if len(e.args) > 1 else 1
                return f"a.D_{cname(e.args[0].name)}[{d - 1}]"
            xs = [self.ex(x) for x in e.args]
            if e.fn == "div":
                return f"({xs[0]} / {xs[1]})"
            if e.fn == "mod":
                return f"stade_lowered::jl_mod_h({xs[0]}, {xs[1]})"
            if e.fn in ("max", "min"):
                out = xs[0]
                for x in xs[1:]:
                    out = f"std::{e.fn}<int64_t>({out}, {x})"
                return out
            if e.fn == "abs":
                return f"std::llabs({xs[0]})"
        raise LowerError(f"{fl.f.name}: the host cannot evaluate {e!r}")


PRELUDE = r"""// Generated by stade_hip.lower from STADE-generated Julia text: HIP for gfx950.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <algorithm>
#include <cstdlib>
#include "lowered_rt.hpp"
namespace stade_lowered {
inline int64_t jl_mod_h(int64_t a, int64_t b) { int64_t r = a % b; return (r != 0 && ((r < 0) != (b < 0))) ? r + b : r; }
}
static char g_gen_err[256];
static int32_t _fail(hipError_t e, const char* what) {
    snprintf(g_gen_err, sizeof g_gen_err, "%s: %s", what, hipGetErrorString(e));
    return -(int32_t)(e > 0 ? e : 1) - 100;
}
static int32_t _bounds(const char* fn) {
    snprintf(g_gen_err, sizeof g_gen_err, "%s: an array index out of bounds (Julia raises a BoundsError)", fn);
    return -3;
}
extern "C" const char* stade_hip_gen_last_error(void) { return g_gen_err; }
"""


GEMM_INCLUDE = '#include "lowered_gemm.hpp"'


def generate(text: str, precision: str = "f64", arg_types: dict | None = None, inbounds: bool = True,
             dead_scalars: bool = True, merge_accum: bool = True) -> tuple[str, dict]:
    """HIP source for every generated function of `text` (the initstacks_* functions stay on
    the host) and, per function, its signature: [(name, kind, ndim)] with kind 'Af', 'Ai',
    'f', 'i'.  `inbounds`, `dead_scalars` and `merge_accum` are `stade_gpu`'s switches
    (/root/reference/src/STADE.jl:18522), on by default as `stade_amdgpu_file` has them."""
    from .syntax import parse
    funcs = parse(text)
    src = [PRELUDE]
    sigs = {}
    stack_kinds = _stack_kinds(funcs, precision)
    for f in funcs:
        if f.name.startswith("initstacks_"):
            continue
        fl = _func_lower(f, stack_kinds, precision, arg_types, inbounds, dead_scalars, merge_accum)
        gen = FuncGen(fl)
        src.append(gen.source())
        if gen.uses_gemm and GEMM_INCLUDE not in src:
            src.insert(1, GEMM_INCLUDE)
        sig = []
        for n in f.args:
            if n in fl.arrays:
                sig.append((n, "Ai" if fl.arrays[n] == "i" else "Af", fl.T.ndim.get(n, 1)))
            else:
                sig.append((n, fl.scalars.get(n, "f"), 0))
        sigs[f.name] = dict(args=sig, plan=describe(fl.ops), reasons=list(fl.reasons), finish=fl.finish_rec,
                            inbounds=inbounds, twins=list(fl.twins), contract=fl.contract_rec,
                            xsplit=list(fl.xsplits))
    return "\n".join(src), sigs


def _func_lower(f, stack_kinds, precision, arg_types, inbounds, dead_scalars, merge_accum):
    kinds = {a: k for a, k in stack_kinds.items() if a in f.args}
    kinds.update((arg_types or {}).get(f.name) or {})
    return FuncLower(f, precision, kinds, stacks_allocated={a for a, k in stack_kinds.items() if k in ("Ai", "Af")},
                     inbounds=inbounds, dead_scalars=dead_scalars, merge_accum=merge_accum)


def lower_function(text: str, fname: str, precision: str = "f64", arg_types: dict | None = None,
                   inbounds: bool = True, dead_scalars: bool = True, merge_accum: bool = True) -> FuncLower:
    """The plan of one generated function of `text`, built as `generate` builds it (the same
    stack types from the file's initstacks_*, the same passes): its transformed syntax tree is
    `.f` and its operations `.ops`."""
    from .syntax import parse
    funcs = parse(text)
    f = next(g for g in funcs if g.name == fname)
    return _func_lower(f, _stack_kinds(funcs, precision), precision, arg_types, inbounds, dead_scalars, merge_accum)


def _stack_kinds(funcs, precision) -> dict:
    """The element types of the stacks that the file's initstacks_* allocate (Int64 branch and
    tripcount stacks, Float64 value stacks), which type the stack arguments of its functions,
    and the kinds of the other values they return."""
    stack_kinds = {}
    for f in funcs:
        if f.name.startswith("initstacks_"):
            for s in walk_stmts(f.body):
                if isinstance(s, Assign) and isinstance(s.lhs, Var) and isinstance(s.rhs, Alloc):
                    stack_kinds[s.lhs.name] = "Ai" if s.rhs.eltype == "Int64" else "Af"
            # what it returns besides arrays are Int64 counts (`__tot_*`, `__mult_*`, `__len_*`),
            # passed on as the trailing arguments even where the body never reads them
            ti = infer_types(f, None, precision)
            for s in walk_stmts(f.body):
                if isinstance(s, Return) and s.value is not None:
                    for it in (s.value.items if isinstance(s.value, Tup) else (s.value,)):
                        if isinstance(it, Var) and it.name not in stack_kinds and it.name not in ti.arrays:
                            stack_kinds[it.name] = ti.scalars.get(it.name, "i")
    return stack_kinds


def describe(ops, depth=0) -> list[str]:
    out = []
    for op in ops:
        pad = "  " * depth
        if isinstance(op, SerialOp):
            nloops = sum(1 for t in walk_stmts(op.stmts) if isinstance(t, (For, While)))
            out.append(pad + f"serial ({len(op.stmts)} statements" + (f", {nloops} loops in order)" if nloops else ")"))
        elif isinstance(op, ParOp):
            pl = op.pl
            kinds = ", ".join(f"{n}:{u.kind}" for n, u in sorted(pl.arrays.items()))
            nsplit = len(split_loops(pl, op.types)) if getattr(op, "types", None) is not None else 0
            out.append(pad + f"parallel over {pl.loop.var} [{kinds}]"
                       + (f" sums {sorted(pl.reductions)}" if pl.reductions else "")
                       + (f"; with few iterations a wave each, lanes sharing {nsplit} inner loop(s)" if nsplit else ""))
        elif isinstance(op, HostLoopOp):
            out.append(pad + f"host loop over {op.loop.var}")
            out += describe(op.ops, depth + 1)
        elif isinstance(op, IfOp):
            out.append(pad + "device if")
            for b in op.branches:
                out += describe(b, depth + 1)
        elif isinstance(op, AllocOp):
            out.append(pad + f"allocate {op.name}")
        elif isinstance(op, ReturnOp):
            out.append(pad + "return")
        elif isinstance(op, GemmOp) and isinstance(op.g, GemmT):
            g = op.g
            out.append(pad + f"matrix product into {g.out} ({('stored', 'added', 'added atomically')[g.mode]}; "
                       f"{g.a} x {g.b}, offset tables)")
        elif isinstance(op, GemmOp):
            g = op.g
            out.append(pad + f"matrix product into {g.out} ({'added' if g.acc else 'stored'}; "
                       + " + ".join(f"{x.a} x {x.b}" for x in g.segs) + ")")
    return out
