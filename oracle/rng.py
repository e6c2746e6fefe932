"""Julia's scalar random stream, restated -- TEST INFRASTRUCTURE ONLY (the checker).

Pinned bit-for-bit against the known answers of
/root/reference/test/validate_seed_stable.jl:37-56 (tests/test_oracle_rng.py):

* `val_stable_seed(s)`: FNV-1a64 over the UTF-8 bytes (/root/reference/src/STADE.jl:16619-16625);
* `Random.Xoshiro(seed)`: Julia 1.10 seeding (SHA-256 of the seed's 32-bit little-endian
  words, first four UInt64 of the digest) and the xoshiro256++ step; `rand(rng)` is
  `(next >>> 11) * 2^-53` (Julia's Float64 sampler for Xoshiro);
* `val_normal(rng)`: Box-Muller, cosine branch, u1 = 1 - rand(), u2 = rand()
  (/root/reference/src/STADE.jl:16628-16637).

The scalar draws are pure Python.  Array fills longer than `_C_FILL_MIN` run the same
stream through `oracle/rng_fill.c` (gcc, built into `oracle/_gen/`), bit-identical to the
scalar loop; the full-size parity tests need tens of millions of draws.  The product
library has its own C++ copy (`stade_hip_rng_*` in libstade_hip.so); tests compare them.
"""
from __future__ import annotations

import ctypes
import hashlib
import math
import os
import struct
import subprocess
import threading
from pathlib import Path

import numpy as np

_M = (1 << 64) - 1


def val_stable_seed(s: str) -> int:
    h = 0xCBF29CE484222325
    for b in s.encode("utf-8"):
        h = ((h ^ b) * 0x00000100000001B3) & _M
    return h


def _hash_seed(seed: int) -> bytes:
    ctx = hashlib.sha256()
    neg = seed < 0
    if neg:
        seed = ~seed
    while True:
        ctx.update(struct.pack("<I", seed & 0xFFFFFFFF))
        seed >>= 32
        if seed == 0:
            break
    if neg:
        ctx.update(b"\x01")
    return ctx.digest()


class Xoshiro:
    """Julia's `Random.Xoshiro(seed)` scalar draws."""

    def __init__(self, seed: int):
        self.s = list(struct.unpack("<4Q", _hash_seed(seed)))

    def next_u64(self) -> int:
        s0, s1, s2, s3 = self.s
        tmp = (s0 + s3) & _M
        res = ((((tmp << 23) | (tmp >> 41)) & _M) + s0) & _M
        t = (s1 << 17) & _M
        s2 ^= s0
        s3 ^= s1
        s1 ^= s2
        s0 ^= s3
        s2 ^= t
        s3 = ((s3 << 45) | (s3 >> 19)) & _M
        self.s = [s0, s1, s2, s3]
        return res

    def rand(self) -> float:
        return (self.next_u64() >> 11) * 2.0 ** -53


def val_normal(rng: Xoshiro) -> float:
    u1 = 1.0 - rng.rand()
    u2 = rng.rand()
    return math.sqrt(-2.0 * math.log(u1)) * math.cos(2.0 * math.pi * u2)


_C_FILL_MIN = 256
_SRC = Path(__file__).resolve().parent / "rng_fill.c"
_SO = Path(__file__).resolve().parent / "_gen" / "rng_fill.so"
_fill_lib = None
_fill_mu = threading.Lock()


def fill_lib(rebuild: bool = False):
    """Compile (when missing, stale, or `rebuild`) and load oracle/rng_fill.c."""
    global _fill_lib
    with _fill_mu:
        if _fill_lib is not None and not rebuild:
            return _fill_lib
        stale = not _SO.exists() or _SO.stat().st_mtime < _SRC.stat().st_mtime
        if rebuild or stale:
            _SO.parent.mkdir(parents=True, exist_ok=True)
            tmp = _SO.with_suffix(f".so.tmp{os.getpid()}")
            subprocess.run(["gcc", "-O2", "-fno-fast-math", "-ffp-contract=off", "-fPIC", "-shared",
                            "-o", str(tmp), str(_SRC), "-lm"], check=True)
            os.replace(tmp, _SO)
        lib = ctypes.CDLL(str(_SO))
        st = ctypes.POINTER(ctypes.c_uint64)
        dp = ctypes.POINTER(ctypes.c_double)
        lib.oracle_rng_normal.argtypes = [st, dp, ctypes.c_int64]
        lib.oracle_rng_normal.restype = None
        lib.oracle_rng_uniform.argtypes = [st, dp, ctypes.c_int64, ctypes.c_double, ctypes.c_double]
        lib.oracle_rng_uniform.restype = None
        _fill_lib = lib
        return lib


def _c_fill(rng: Xoshiro, n: int, fn: str, *extra) -> np.ndarray:
    out = np.empty(n, dtype=np.float64)
    st = (ctypes.c_uint64 * 4)(*rng.s)
    getattr(fill_lib(), fn)(st, out.ctypes.data_as(ctypes.POINTER(ctypes.c_double)), n, *extra)
    rng.s = [int(v) for v in st]
    return out


def val_randn(rng: Xoshiro, n: int, c_fill: bool | None = None) -> np.ndarray:
    """n draws of `val_normal(rng)` in order (`c_fill` forces or forbids the C fill)."""
    if c_fill if c_fill is not None else n >= _C_FILL_MIN:
        return _c_fill(rng, n, "oracle_rng_normal")
    return np.array([val_normal(rng) for _ in range(n)], dtype=np.float64)


def rand_uniform(rng: Xoshiro, n: int, lo: float = 0.0, hi: float = 1.0, c_fill: bool | None = None) -> np.ndarray:
    """`lo + (hi - lo) * rand(rng)`, n scalar draws in order."""
    if c_fill if c_fill is not None else n >= _C_FILL_MIN:
        return _c_fill(rng, n, "oracle_rng_uniform", float(lo), float(hi))
    return np.array([lo + (hi - lo) * rng.rand() for _ in range(n)], dtype=np.float64)
