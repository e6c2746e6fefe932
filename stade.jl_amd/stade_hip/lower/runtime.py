"""Building and calling the libraries that the general lowering writes.

`lower(text_or_path, precision)` turns a generated `.jl` into HIP source (`hipgen.generate`),
compiles it for gfx950 once (hipcc, the build flags of libstade_hip: floating-point
contraction off, packed FP32 off) into `stade.jl_amd/lib/gen/<stem>_<hash>.so`, and returns a
`LoweredLib`.  A library already built for the same source is loaded as it is, so the GPU
box, which receives the tree with its built libraries, does not compile.

`LoweredLib.call(name, *args)` runs one generated function with Julia's argument convention:
arrays are flat, contiguous torch tensors on the GPU (a matrix argument passes its Julia
dimensions through `shapes=`), mutated in place; Int64 and float scalars are passed by value;
the function's returned scalars come back as a tuple.  There is no CPU path: a tensor that is
not on a GPU raises.
"""
from __future__ import annotations

import ctypes
import hashlib
import os
import shutil
import subprocess
import threading
from pathlib import Path

from . import hipgen
from .syntax import (Alloc, Assign, Bin, Break, Call, Continue, ExprStmt, For, If, LowerError, Nothing_, Num, Ref,
                     Return, Tup, Un, Var, While, parse)

PKG = Path(__file__).resolve().parent.parent.parent
GEN_LIB = PKG / "lib" / "gen"
CSRC = PKG / "csrc"
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
ARCH = os.environ.get("STADE_HIP_ARCH", "gfx950")
FLAGS = [f"--offload-arch={ARCH}", "-O3", "-fPIC", "-shared", "-std=c++17", "-ffp-contract=off",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wno-unused-label", "-Wno-unused-variable",
         "-Wno-unused-command-line-argument", "-I", str(CSRC)]
_lock = threading.Lock()
_cache: dict[str, "LoweredLib"] = {}


def _src_key(src: str) -> str:
    # the flags without the include directory's absolute path: the key (and so the library's
    # file name) must not depend on where the tree sits, or a copied tree would rebuild
    # (the device runtime header is part of the source, and so are the matrix-product headers
    # where the source includes them)
    flags = " ".join(f for f in FLAGS[1:] if f != str(CSRC))
    rt = (CSRC / "lowered_rt.hpp").read_text()
    if '#include "lowered_gemm.hpp"' in src:
        rt += (CSRC / "lowered_gemm.hpp").read_text() + (CSRC / "gemm_f32.hpp").read_text()
    return hashlib.sha256((src + flags + rt).encode()).hexdigest()[:16]


_so_locks: dict = {}


def build_source(src: str, stem: str, out_dir: Path | None = None) -> Path:
    """Compile HIP source into the generated-library directory (or `out_dir`), once per source
    text; one lock per library, so that different sources compile in parallel threads."""
    out_dir = Path(out_dir) if out_dir is not None else GEN_LIB
    out_dir.mkdir(parents=True, exist_ok=True)
    so = out_dir / f"{stem}_{_src_key(src)}.so"
    with _lock:
        lk = _so_locks.setdefault(so, threading.Lock())
    with lk:
        if so.exists():
            return so
        hip = so.with_suffix(".hip")
        hip.write_text(src)
        tmp = so.with_suffix(f".so.tmp{os.getpid()}")
        r = subprocess.run([HIPCC, *FLAGS, "-o", str(tmp), str(hip)], capture_output=True, text=True)
        if r.returncode != 0:
            raise LowerError(f"hipcc failed on the lowered {stem}:\n{r.stderr[-3000:]}")
        os.replace(tmp, so)
    return so


class LoweredLib:
    def __init__(self, so: Path, sigs: dict, precision: str, text: str):
        self.path = so
        self.sigs = sigs
        self.precision = precision
        self.text = text
        self._lib = None
        self._fns = {}

    @property
    def lib(self):
        """The library, loaded at first use (after torch's HIP runtime: `hip_runtime_first`)."""
        if self._lib is None:
            from ..api import hip_runtime_first
            hip_runtime_first()
            self._lib = ctypes.CDLL(str(self.path))
            self._lib.stade_hip_gen_last_error.restype = ctypes.c_char_p
        return self._lib

    def plan(self, name: str) -> list[str]:
        return self.sigs[name]["plan"]

    def set_stats(self, name: str, counters=None):
        """Count the accumulation paths of function `name`'s launches into `counters` (an int64
        CUDA tensor of at least 8 elements, added to, never cleared) until called with None.
        Slots: 0 wave-aggregated atomics (one per wave), 1 per-lane atomics (one per wave), 2
        blocks of an LDS-privatised variant, 3 blocks of the wave-per-iteration form, 4 block
        sums added, 5 blocks of a flat loop's row-block twin, 6 of its column-block twin, 7
        blocks of the lanes-over-iterations form (`csrc/lowered_rt.hpp`, ST_*).  A test hook: the calls of the generated
        function are unchanged."""
        f = getattr(self.lib, f"stade_hip_gen_{hipgen.cname(name)}_set_stats")
        f.restype = None
        f.argtypes = [ctypes.c_void_p]
        if counters is None:
            f(None)
            return
        import torch
        if not (isinstance(counters, torch.Tensor) and counters.is_cuda and counters.dtype == torch.int64
                and counters.is_contiguous() and counters.numel() >= 8):
            raise ValueError("counters must be a contiguous int64 CUDA tensor of at least 8 elements")
        f(ctypes.c_void_p(counters.data_ptr()))

    def graphs(self, name: str) -> tuple[int, int]:
        """(launch sequences of function `name` captured into HIP graphs, graph launches) so far
        in this process.  A function with host loops replays its launches as a graph when a
        call repeats an earlier call's frame (device, array addresses, sizes and scalars alike;
        `csrc/lowered_rt.hpp`, LaunchGraphs).  A test hook."""
        f = getattr(self.lib, f"stade_hip_gen_{hipgen.cname(name)}_graphs")
        f.restype = None
        f.argtypes = [ctypes.c_void_p]
        out = (ctypes.c_int64 * 2)()
        f(ctypes.cast(out, ctypes.c_void_p))
        return int(out[0]), int(out[1])

    def _fn(self, name):
        if name not in self._fns:
            f = getattr(self.lib, f"stade_hip_gen_{hipgen.cname(name)}")
            f.restype = ctypes.c_int32
            ft = ctypes.c_float if self.precision == "f32" else ctypes.c_double
            at = []
            for a, kind, nd in self.sigs[name]["args"]:
                if kind in ("Af", "Ai"):
                    at += [ctypes.c_void_p] + [ctypes.c_int64] * nd
                elif kind == "i":
                    at.append(ctypes.c_int64)
                elif kind == "b":
                    at.append(ctypes.c_bool)
                else:
                    at.append(ft)
            at += [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int64), ctypes.c_void_p]
            f.argtypes = at
            self._fns[name] = f
        return self._fns[name]

    def call(self, name: str, *args, shapes: dict | None = None, stream=None):
        import torch
        sig = self.sigs[name]["args"]
        if len(args) != len(sig):
            raise TypeError(f"{name} takes {len(sig)} arguments, got {len(args)}")
        shapes = shapes or {}
        fdt = torch.float32 if self.precision == "f32" else torch.float64
        cargs = []
        dev = None
        for (a, kind, nd), v in zip(sig, args):
            if kind in ("Af", "Ai"):
                want = torch.int64 if kind == "Ai" else fdt
                if not isinstance(v, torch.Tensor) or not v.is_cuda:
                    raise ValueError(f"{name}: {a} must be a torch tensor on a GPU (there is no CPU path)")
                if v.dtype != want:
                    raise TypeError(f"{name}: {a} has dtype {v.dtype}, expected {want}")
                if not v.is_contiguous():
                    raise ValueError(f"{name}: {a} must be contiguous")
                dims = tuple(shapes.get(a, (v.numel(),)))
                if len(dims) < nd:
                    raise ValueError(f"{name}: {a} is indexed with {nd} subscripts; pass its Julia dimensions in shapes")
                if len(dims) > nd:   # trailing dimensions fold into the last one used
                    head = list(dims[:nd - 1])
                    tail = 1
                    for d in dims[nd - 1:]:
                        tail *= d
                    dims = tuple(head + [tail])
                n = 1
                for d in dims:
                    n *= d
                if n != v.numel():
                    raise ValueError(f"{name}: {a} has {v.numel()} elements, dimensions {dims} need {n}")
                cargs += [ctypes.c_void_p(v.data_ptr())] + [int(d) for d in dims]
                dev = dev or v.device
            elif kind == "i":
                cargs.append(int(v))
            elif kind == "b":
                cargs.append(bool(v))
            else:
                cargs.append(float(v))
        if stream is None:
            stream = torch.cuda.current_stream(dev).cuda_stream if dev is not None else 0
        ret = (ctypes.c_double * 16)()
        iret = (ctypes.c_int64 * 16)()
        rc = self._fn(name)(*cargs, ret, iret, ctypes.c_void_p(stream))
        if rc < 0:
            raise RuntimeError(f"{name}: {self.lib.stade_hip_gen_last_error().decode(errors='replace')}")
        kinds = self.sigs[name].get("ret", [])
        return tuple(int(iret[k]) if k < len(kinds) and kinds[k] == "i" else float(ret[k]) for k in range(rc))


def _ret_kinds(text: str, precision: str, arg_types) -> dict:
    out = {}
    arg_types = dict(arg_types or {})
    for f in parse(text):
        if f.name.startswith("initstacks_"):
            for s in f.body:
                if isinstance(s, Assign) and isinstance(s.lhs, Var) and isinstance(s.rhs, Alloc):
                    for g in parse(text):
                        if s.lhs.name in g.args:
                            arg_types.setdefault(g.name, {})[s.lhs.name] = "Ai" if s.rhs.eltype == "Int64" else "Af"
    for f in parse(text):
        if f.name.startswith("initstacks_"):
            continue
        if f.body and isinstance(f.body[-1], Return) and f.body[-1].value is not None \
                and not isinstance(f.body[-1].value, Nothing_):
            v = f.body[-1].value
            items = v.items if isinstance(v, Tup) else (v,)
            fl = hipgen.FuncLower(f, precision, (arg_types or {}).get(f.name))
            out[f.name] = ["i" if fl.T.etype(x) == "i" else "f" for x in items]
    return out


def lower(src, precision: str = "f64", arg_types: dict | None = None, tag: str | None = None,
          out_dir: Path | None = None, inbounds: bool = True, dead_scalars: bool = True,
          merge_accum: bool = True) -> LoweredLib:
    """Lower a generated file (path or text), build it once (into stade.jl_amd/lib/gen, or
    `out_dir`), load it.  `inbounds`, `dead_scalars` and `merge_accum` are the reference's
    switches of the same names (on by default, as `stade_amdgpu_file` has them): with
    `inbounds=False` every array access is checked and an index out of range raises
    StadeHipBoundsError; with `inbounds=True` such an index is undefined behaviour, as under
    Julia's @inbounds."""
    p = Path(src) if not (isinstance(src, str) and "\n" in src) else None
    text = p.read_text() if p is not None else str(src)
    key = (text, precision, repr(sorted((arg_types or {}).items())), str(out_dir), inbounds, dead_scalars, merge_accum)
    ck = hashlib.sha256(repr(key).encode()).hexdigest()
    if ck in _cache:
        return _cache[ck]
    hip, sigs = hipgen.generate(text, precision, arg_types, inbounds=inbounds, dead_scalars=dead_scalars,
                                merge_accum=merge_accum)
    for name, kinds in _ret_kinds(text, precision, arg_types).items():
        sigs[name]["ret"] = kinds
    so = build_source(hip, tag or (p.stem if p is not None else "inline"), out_dir)
    lib = LoweredLib(so, sigs, precision, text)
    _cache[ck] = lib
    return lib


# ------------------------------------------------------------------------------------------
# initstacks_* on the host: the stack sizes are Int arithmetic of the Int arguments
# ------------------------------------------------------------------------------------------

def _ival(e, env):
    if isinstance(e, Num):
        return int(e.text, 0)
    if isinstance(e, Var):
        return env[e.name]
    if isinstance(e, Un) and e.op == "-":
        return -_ival(e.a, env)
    if isinstance(e, Bin):
        a, b = _ival(e.a, env), _ival(e.b, env)
        if e.op == "+":
            return a + b
        if e.op == "-":
            return a - b
        if e.op == "*":
            return a * b
    if isinstance(e, Call):
        xs = [_ival(x, env) for x in e.args]
        if e.fn == "div":
            q = abs(xs[0]) // abs(xs[1])
            return q if (xs[0] >= 0) == (xs[1] >= 0) else -q
        if e.fn == "mod":
            return xs[0] % xs[1]
        if e.fn == "max":
            return max(xs)
        if e.fn == "min":
            return min(xs)
    raise LowerError(f"initstacks: cannot evaluate {e!r} on the host")


def initstacks(text: str, name: str, *int_args) -> list[tuple[str, str, int]]:
    """[(stack name, element type, length)] that `initstacks_<k>_b(int_args...)` allocates,
    in the order it returns them (`agen_init_emit` /root/reference/src/STADE.jl:4011-4097)."""
    f = next((g for g in parse(text) if g.name == name), None)
    if f is None:
        raise LowerError(f"no function {name}")
    env = dict(zip(f.args, (int(v) for v in int_args)))
    allocs = {}
    ret = []
    for s in f.body:
        if isinstance(s, Assign) and isinstance(s.lhs, Var):
            if isinstance(s.rhs, Alloc):
                allocs[s.lhs.name] = (s.rhs.eltype, max(0, _ival(s.rhs.n, env)))
            else:
                env[s.lhs.name] = _ival(s.rhs, env)
        elif isinstance(s, Return) and s.value is not None:
            items = s.value.items if isinstance(s.value, Tup) else (s.value,)
            for it in items:
                if isinstance(it, Var) and it.name in allocs:
                    ret.append((it.name, *allocs[it.name]))
    return ret


# ------------------------------------------------------------------------------------------
# initstacks_* run on the host in full: loops, branches, index arrays and scalar returns
# ------------------------------------------------------------------------------------------

class _Return(Exception):
    def __init__(self, value):
        self.value = value


class _Break(Exception):
    pass


class _Continue(Exception):
    pass


def initstacks_returns(text: str, name: str) -> list[str]:
    """Names of what `initstacks_<k>_b` returns, in order: the trailing arguments of the
    generated `<k>_b` / `<k>_hv` (stacks, then any index arrays and Int64 counts)."""
    f = next((g for g in parse(text) if g.name == name), None)
    if f is None:
        raise LowerError(f"no function {name}")
    for st in f.body:
        if isinstance(st, Return) and st.value is not None and not isinstance(st.value, Nothing_):
            items = st.value.items if isinstance(st.value, Tup) else (st.value,)
            if not all(isinstance(it, Var) for it in items):
                raise LowerError(f"{name}: returns an expression, not named values")
            return [it.name for it in items]
    return []


def run_initstacks(text: str, name: str, args: dict, max_iters: int = 1 << 26) -> list[tuple[str, object]]:
    """Run `initstacks_<k>_b` on the host with its arguments' values (`args`: Int64 and float
    scalars by name, arrays as numpy arrays where it takes their `length`), and return its
    returned values [(name, value)] in order: stacks as zero-filled numpy arrays (the
    generated code writes every slot before reading it), index arrays (`prefix_*`, `val_*`)
    with the values it computed, Int64 counts as ints.  Julia's semantics for what these
    functions use: Int64 and Float64 arithmetic, `div` (truncating), `mod` (the divisor's
    sign), `max`, `min`, `length`, 1-based element stores, counted loops, `if`/`elseif`.
    Same role as the generated function in the reference (`agen_init_emit`
    /root/reference/src/STADE.jl:4011-4097); its calls run there in Julia on the host."""
    import numpy as np
    f = next((g for g in parse(text) if g.name == name), None)
    if f is None:
        raise LowerError(f"no function {name}")
    missing = [a for a in f.args if a not in args]
    if missing:
        raise LowerError(f"{name}: no value for {', '.join(missing)}")
    env = {a: args[a] for a in f.args}
    budget = [max_iters]

    def num(e: Num):
        if e.text in ("true", "false"):
            return e.text == "true"
        t = e.text.replace("_", "")
        return int(t, 0) if e.is_int else float(t)

    def idiv(a, b):
        if isinstance(a, int) and isinstance(b, int):
            q = abs(a) // abs(b)
            return q if (a >= 0) == (b >= 0) else -q
        import math
        return math.trunc(a / b)

    def call(e: Call):
        fn = e.fn
        if fn == "length":
            return int(np.size(ev(e.args[0])))
        if fn == "size":
            return int(np.shape(ev(e.args[0]))[ev(e.args[1]) - 1])
        xs = [ev(x) for x in e.args]
        if fn == "div":
            return idiv(*xs)
        if fn == "mod":
            return xs[0] % xs[1]
        if fn == "rem":
            return xs[0] - idiv(xs[0], xs[1]) * xs[1]
        if fn in ("max", "min"):
            return (max if fn == "max" else min)(xs)
        if fn == "abs":
            return abs(xs[0])
        if fn in ("Int", "Int64") and len(xs) == 1:
            v = xs[0]
            if isinstance(v, float) and not v.is_integer():
                raise LowerError(f"{name}: InexactError converting {v} to Int64")
            return int(v)
        if fn in ("floor", "ceil", "round", "trunc"):
            import math
            v = xs[-1]
            r = {"floor": math.floor, "ceil": math.ceil, "trunc": math.trunc,
                 "round": lambda x: int(np.round(x))}[fn](v)
            return int(r) if len(xs) == 2 else float(r)
        if fn in ("Float64", "float"):
            return float(xs[0])
        raise LowerError(f"{name}: cannot run {fn}(...) on the host")

    def ev(e):
        if isinstance(e, Num):
            return num(e)
        if isinstance(e, Var):
            if e.name not in env:
                raise LowerError(f"{name}: {e.name} is read before it is set")
            return env[e.name]
        if isinstance(e, Ref):
            a = env[e.name]
            ix = [ev(x) for x in e.idx]
            return a.ravel(order="F")[_linear(a, ix)].item()
        if isinstance(e, Un):
            v = ev(e.a)
            return (not v) if e.op == "!" else -v
        if isinstance(e, Bin):
            if e.op == "&&":
                return bool(ev(e.a)) and bool(ev(e.b))
            if e.op == "||":
                return bool(ev(e.a)) or bool(ev(e.b))
            x, y = ev(e.a), ev(e.b)
            op = e.op
            if op == "+":
                return x + y
            if op == "-":
                return x - y
            if op == "*":
                return x * y
            if op == "/":
                return x / y
            if op == "^":
                return x ** y
            return {"==": x == y, "!=": x != y, "<": x < y, ">": x > y, "<=": x <= y, ">=": x >= y}[op]
        if isinstance(e, Call):
            return call(e)
        if isinstance(e, Alloc):
            n = ev(e.n)
            return np.zeros(max(0, int(n)), dtype=np.int64 if e.eltype == "Int64" else np.float64)
        if isinstance(e, Tup):
            return tuple(ev(x) for x in e.items)
        if isinstance(e, Nothing_):
            return None
        raise LowerError(f"{name}: cannot evaluate {type(e).__name__} on the host")

    def _linear(a, ix):
        k, stride = 0, 1
        shape = a.shape if a.ndim else (1,)
        for d, i in enumerate(ix):
            ext = shape[d] if d < len(shape) else 1
            if not 1 <= i <= (ext if d < len(ix) - 1 else int(np.prod(shape[d:]))):
                raise LowerError(f"{name}: index {i} out of bounds for {a.shape}")
            k += (i - 1) * stride
            stride *= ext
        return k

    def tick():
        budget[0] -= 1
        if budget[0] < 0:
            raise LowerError(f"{name}: more than {max_iters} loop iterations")

    def run(stmts):
        for st in stmts:
            if isinstance(st, Assign):
                v = ev(st.rhs)
                if isinstance(st.lhs, Var):
                    env[st.lhs.name] = v
                else:
                    a = env[st.lhs.name]
                    ix = [ev(x) for x in st.lhs.idx]
                    flat = a.reshape(-1, order="F")
                    if not np.shares_memory(flat, a):
                        raise LowerError(f"{name}: {st.lhs.name} is not contiguous")
                    flat[_linear(a, ix)] = v
            elif isinstance(st, For):
                r = st.rng
                lo, hi = ev(r.lo), ev(r.hi)
                step = 1 if r.step is None else ev(r.step)
                i = lo
                while (step > 0 and i <= hi) or (step < 0 and i >= hi):
                    tick()
                    env[st.var] = i
                    try:
                        run(st.body)
                    except _Continue:
                        pass
                    except _Break:
                        break
                    i += step
            elif isinstance(st, While):
                while ev(st.cond):
                    tick()
                    try:
                        run(st.body)
                    except _Continue:
                        pass
                    except _Break:
                        break
            elif isinstance(st, If):
                for cond, body in st.branches:
                    if ev(cond):
                        run(body)
                        break
                else:
                    if st.orelse:
                        run(st.orelse)
            elif isinstance(st, Return):
                raise _Return(None if st.value is None else ev(st.value))
            elif isinstance(st, Break):
                raise _Break()
            elif isinstance(st, Continue):
                raise _Continue()
            elif isinstance(st, ExprStmt):
                ev(st.e)
            else:
                raise LowerError(f"{name}: cannot run {type(st).__name__} on the host")

    try:
        run(f.body)
        value = None
    except _Return as r:
        value = r.value
    names = initstacks_returns(text, name)
    vals = value if isinstance(value, tuple) else (() if value is None else (value,))
    if len(vals) != len(names):
        raise LowerError(f"{name}: returned {len(vals)} values for {len(names)} names")
    return list(zip(names, vals))

