"""Compile transpiled STADE-generated code with gcc and call it on numpy arrays.

TEST INFRASTRUCTURE ONLY (see oracle/jl2c.py): the checker and the CPU baseline.

`load(path_or_text, precision=..., bounds_check=...)` returns an `OracleLib`; its
`call(name, *args)` runs one generated Julia function with Julia's argument
convention: arrays are mutated in place (numpy, Fortran order for matrices), scalar
arguments are passed by value, and the function's `return` values come back as a
tuple (an adjoint returns its scalar shadows, `agen_emit` /root/reference/src/
STADE.jl:3672; an HVP returns `(xb, xbd)` pairs, 6772-6779).  `stacks(name, *args)`
runs an `initstacks_*` function and allocates the stacks it sizes, with the element
types it declares (`agen_init_emit` /root/reference/src/STADE.jl:4011-4097).

Build flags: `gcc -O2 -fno-fast-math -ffp-contract=off`, single-threaded, matching
the sequential Julia the generator writes.
"""
from __future__ import annotations

import ctypes
import hashlib
import os
import subprocess
import threading
from pathlib import Path

import numpy as np

from . import jl2c

GEN_DIR = Path(__file__).resolve().parent / "_gen"
CFLAGS = ["-O2", "-fno-fast-math", "-ffp-contract=off", "-fPIC", "-shared", "-std=gnu11",
          "-Wno-unused-variable", "-Wno-unused-label", "-Wno-unused-but-set-variable"]
_locks: dict[str, threading.Lock] = {}
_locks_mu = threading.Lock()


def _lock_for(path: Path) -> threading.Lock:
    with _locks_mu:
        return _locks.setdefault(str(path), threading.Lock())


class JlArr(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("ndim", ctypes.c_int64), ("dims", ctypes.c_int64 * 4)]


_DT = {"Af": None, "Ai": np.int64}


def _ld_from_buffer(buf, n):
    """The first n values of a ctypes c_longdouble array as numpy long doubles.  Indexing the
    ctypes array itself would return Python floats and drop the 80-bit values' last 11 bits (and
    Int64 values above 2^53)."""
    assert ctypes.sizeof(ctypes.c_longdouble) == np.dtype(np.longdouble).itemsize
    return np.frombuffer(buf, dtype=np.longdouble, count=max(n, 0))


class OracleLib:
    def __init__(self, so_path: Path, infos: dict, precision: str):
        self.path = so_path
        self.lib = ctypes.CDLL(str(so_path))
        self.infos = infos
        self.precision = precision
        self.fdt = {"f32": np.float32, "f64": np.float64, "f80": np.longdouble}[precision]
        self.lib.jl_get_bounds_error.restype = ctypes.c_int
        self._fns = {}

    def _fn(self, name):
        if name not in self._fns:
            f = getattr(self.lib, name)
            f.restype = ctypes.c_int64
            f.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_void_p]
            self._fns[name] = f
        return self._fns[name]

    def call(self, name: str, *args):
        info = self.infos[name]
        if len(args) != len(info.args):
            raise TypeError(f"{name} takes {len(info.args)} arguments, got {len(args)}")
        keep = []
        argv = (ctypes.c_void_p * max(1, len(args)))()
        for j, ((an, kind), v) in enumerate(zip(info.args, args)):
            if kind.startswith("A"):
                want = np.int64 if kind == "Ai" else self.fdt
                if not isinstance(v, np.ndarray):
                    raise TypeError(f"{name}: argument {an} must be a numpy array")
                if v.dtype != want:
                    raise TypeError(f"{name}: argument {an} has dtype {v.dtype}, expected {np.dtype(want)}")
                if v.ndim > 1 and not v.flags.f_contiguous:
                    raise TypeError(f"{name}: matrix argument {an} must be Fortran-ordered (Julia column-major)")
                if v.ndim <= 1 and not v.flags.c_contiguous:
                    raise TypeError(f"{name}: argument {an} must be contiguous")
                s = JlArr()
                s.data = v.ctypes.data
                s.ndim = max(1, v.ndim)
                shape = v.shape if v.ndim else (1,)
                for k, d in enumerate(shape):
                    s.dims[k] = d
                keep.append(s)
                argv[j] = ctypes.cast(ctypes.pointer(s), ctypes.c_void_p)
            else:
                if kind == "i":
                    if isinstance(v, (float, np.floating)):
                        raise TypeError(f"{name}: argument {an} is an Int64, got a float")
                    c = ctypes.c_int64(int(v))
                elif self.precision == "f32":
                    c = ctypes.c_float(float(v))
                elif self.precision == "f80":
                    # through a numpy buffer: ctypes.c_longdouble(v) converts v via a Python float
                    c = np.array([v], dtype=np.longdouble)
                    keep.append(c)
                    argv[j] = ctypes.c_void_p(c.ctypes.data)
                    continue
                else:
                    c = ctypes.c_double(float(v))
                keep.append(c)
                argv[j] = ctypes.cast(ctypes.pointer(c), ctypes.c_void_p)
        ret = (ctypes.c_longdouble * 64)()
        n = self._fn(name)(argv, ret)
        if self.lib.jl_get_bounds_error():
            raise IndexError(f"{name}: out-of-bounds array access (see stderr)")
        rv = _ld_from_buffer(ret, n)
        out = []
        for k in range(n):
            kind = info.ret[k] if k < len(info.ret) else "f"
            if kind == "i":
                out.append(int(rv[k]))
            elif kind.startswith("A"):
                out.append((int(rv[k]), kind))
            else:
                out.append(self.fdt(rv[k]) if self.precision == "f80" else float(self.fdt(rv[k])))
        return tuple(out)

    def stacks(self, name: str, *args, fill_nan: bool = True):
        """Run `initstacks_*` and allocate what it sizes: a tuple of numpy arrays."""
        res = self.call(name, *args)
        arrs = []
        for length, kind in res:
            if kind == "Ai":
                a = np.full(length, np.int64(0x7FF4DEAD7FF4DEAD), dtype=np.int64)
            else:
                a = np.full(length, np.nan, dtype=self.fdt) if fill_nan else np.empty(length, self.fdt)
            arrs.append(a)
        return tuple(arrs)


_cache: dict[tuple, OracleLib] = {}


def load(src: str | os.PathLike, precision: str = "f64", bounds_check: bool = True,
         arg_types: dict | None = None, tag: str | None = None) -> OracleLib:
    """Transpile a generated `.jl` (path or text), compile it once, and load it."""
    p = Path(src) if not (isinstance(src, str) and "\n" in src) else None
    text = p.read_text() if p is not None else str(src)
    stem = tag or (p.stem if p is not None else "inline")
    c_src, infos = jl2c.transpile(text, precision=precision, bounds_check=bounds_check, arg_types=arg_types)
    key = hashlib.sha256((c_src + " ".join(CFLAGS)).encode()).hexdigest()[:12]
    ck = (key,)
    if ck in _cache:
        return _cache[ck]
    # builds of the reference's own corpus and of inline test texts are CPU-test only: kept
    # apart from the config builds that the GPU box uses
    gen = GEN_DIR if (p is not None and "/root/reference" not in str(p.resolve())) else GEN_DIR / "cpu_only"
    gen.mkdir(parents=True, exist_ok=True)
    so = gen / f"{stem}_{precision}{'_bc' if bounds_check else ''}_{key}.so"
    with _lock_for(so):
        if not so.exists():
            c_path = so.with_suffix(".c")
            c_path.write_text(c_src)
            tmp = so.with_suffix(f".so.tmp{os.getpid()}")
            subprocess.run(["gcc", *CFLAGS, "-o", str(tmp), str(c_path), "-lm"], check=True)
            os.replace(tmp, so)
    lib = OracleLib(so, infos, precision)
    _cache[ck] = lib
    return lib
