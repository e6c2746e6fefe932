"""The reference's numerical oracles for generated derivative code, restated.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Every generated function works in one flattened space: all float arguments of the
primal, scalars and arrays, in signature order.  The primal maps that space to itself
in place (an untouched argument is the identity); `<k>_d` maps an initial tangent `xd`
to the final tangents `J xd`; `<k>_b` maps an initial shadow `yb` to the final shadows
`J' yb` (scalar shadows come back as return values); `<k>_hv` does both at once.

* `dotprod`  -- `<yb, J xd> = <J' yb, xd>` to rtol 1e-11
  (`val_validate_dotprod` /root/reference/src/STADE.jl:17108-17131);
* `fd_adjoint` -- central difference of `<seed, F(x)>` against `<xb, d>`, eps 1e-6,
  rtol 1e-3 (`val_finite_diff_check` 16334-16351, `val_validate_adjoint` 17080);
* `fd_tangent` -- central difference of F against `J d` (`val_finite_diff_check_jvp`
  16376, `val_validate_tangent` 17064);
* `fd_hvp` -- central difference of the gradient against the HVP's `xbd`
  (`val_validate_hvp` 17133-17153).

Argument orders: tangent interleaves `x, xd` (`tgen_signature_args` 3306-3315); adjoint
interleaves `x, xb`, Int64 arguments once, then stacks (`agen_signature_args`
3455-3464, 3649); HVP is the adjoint list, then `(xd, xbd)` per float argument, then
stacks (`hvp_emit` 6750-6756).  The adjoint returns the float scalars' shadows, the
HVP returns `(xb, xbd)` pairs (3672, 6772-6779).
"""
from __future__ import annotations

import copy
from dataclasses import dataclass, field

import numpy as np

from . import rng as jrng
from .runner import OracleLib


@dataclass
class Kernel:
    """A primal signature plus concrete sizes: enough to call its generated code."""
    name: str
    args: list[tuple[str, str]]                 # (name, 'f'|'i'|'Af'|'Ai') from the primal
    ints: dict[str, int]                        # Int64 scalar arguments
    shapes: dict[str, tuple]                    # array arguments -> Julia dims
    int_arrays: dict[str, np.ndarray] = field(default_factory=dict)
    init_scalars: dict[str, float] = field(default_factory=dict)
    fdt: type = np.float64

    @property
    def float_args(self):
        return [(a, k) for a, k in self.args if k in ("f", "Af")]

    def flat_len(self):
        n = 0
        for a, k in self.float_args:
            n += 1 if k == "f" else int(np.prod(self.shapes[a]))
        return n


def kernel_from_lib(lib: OracleLib, name: str, ints: dict, shapes: dict, int_arrays=None,
                    init_scalars=None) -> Kernel:
    info = lib.infos[name]
    return Kernel(name, list(info.args), dict(ints), {k: tuple(v) if isinstance(v, (tuple, list)) else (v,)
                                                      for k, v in shapes.items()},
                  dict(int_arrays or {}), dict(init_scalars or {}), lib.fdt)


def _arr(shape, vals, dt):
    a = np.asarray(vals, dtype=dt)
    return np.asfortranarray(a.reshape(shape, order="F")) if len(shape) > 1 else np.ascontiguousarray(a.reshape(shape))


def random_values(k: Kernel, g: jrng.Xoshiro, base: bool = False) -> dict:
    """N(0,1) for every float argument, scalars included (`val_random_values_like`).
    With `base=True` the kernel's fixed scalar values (a physical time step, a final
    time) replace the draws; directions and seeds are always N(0,1)."""
    out = {}
    for a, kind in k.float_args:
        if kind == "f":
            z = jrng.val_normal(g)
            out[a] = k.init_scalars[a] if (base and a in k.init_scalars) else z
        else:
            n = int(np.prod(k.shapes[a]))
            out[a] = _arr(k.shapes[a], jrng.val_randn(g, n), k.fdt)
    return out


def zeros_like(k: Kernel) -> dict:
    out = {}
    for a, kind in k.float_args:
        out[a] = 0.0 if kind == "f" else _arr(k.shapes[a], np.zeros(int(np.prod(k.shapes[a]))), k.fdt)
    return out


def flatten(k: Kernel, vals: dict) -> np.ndarray:
    parts = []
    for a, kind in k.float_args:
        v = vals[a]
        parts.append(np.array([v], dtype=np.float64) if kind == "f" else np.asarray(v, dtype=np.float64).ravel(order="F"))
    return np.concatenate(parts) if parts else np.zeros(0)


def unflatten(k: Kernel, x: np.ndarray) -> dict:
    out, pos = {}, 0
    for a, kind in k.float_args:
        if kind == "f":
            out[a] = float(x[pos])
            pos += 1
        else:
            n = int(np.prod(k.shapes[a]))
            out[a] = _arr(k.shapes[a], x[pos:pos + n], k.fdt)
            pos += n
    return out


def _int_value(k: Kernel, a: str, kind: str):
    if kind == "i":
        return k.ints[a]
    return k.int_arrays[a]


def call_primal(lib: OracleLib, k: Kernel, vals: dict) -> np.ndarray:
    vals = copy.deepcopy(vals)
    args = [vals[a] if kind in ("f", "Af") else _int_value(k, a, kind) for a, kind in k.args]
    lib.call(k.name, *args)
    return flatten(k, vals)


def _stack_args(lib: OracleLib, k: Kernel, fname: str, stack_fn: str | None):
    if stack_fn is None or stack_fn not in lib.infos:
        return ()
    sargs = [k.ints[a] for a, kind in lib.infos[stack_fn].args]
    return lib.stacks(stack_fn, *sargs)


def call_tangent(lib: OracleLib, k: Kernel, vals: dict, xd: dict, fname: str | None = None) -> np.ndarray:
    fname = fname or f"{k.name}_d"
    vals, xd = copy.deepcopy(vals), copy.deepcopy(xd)
    args = []
    for a, kind in k.args:
        if kind in ("f", "Af"):
            args += [vals[a], xd[a]]
        else:
            args.append(_int_value(k, a, kind))
    ret = lib.call(fname, *args)
    names = lib.infos[fname].ret_names
    for nm, v in zip(names, ret):
        if nm is not None and nm.endswith("d") and nm[:-1] in xd:
            xd[nm[:-1]] = v
    return flatten(k, xd)


def call_adjoint(lib: OracleLib, k: Kernel, vals: dict, yb: dict, fname: str | None = None,
                 return_state: bool = False):
    fname = fname or f"{k.name}_b"
    vals, yb = copy.deepcopy(vals), copy.deepcopy(yb)
    args = []
    for a, kind in k.args:
        if kind in ("f", "Af"):
            args += [vals[a], yb[a]]
        else:
            args.append(_int_value(k, a, kind))
    stacks = _stack_args(lib, k, fname, f"initstacks_{k.name}_b")
    ret = lib.call(fname, *args, *stacks)
    scal = [a for a, kind in k.args if kind == "f"]
    for a, v in zip(scal, ret):
        yb[a] = v
    if return_state:
        return flatten(k, yb), vals, yb, stacks
    return flatten(k, yb)


def call_hvp(lib: OracleLib, k: Kernel, vals: dict, yb: dict, xd: dict, ybd: dict, fname: str | None = None):
    fname = fname or f"{k.name}_hv"
    vals, yb, xd, ybd = (copy.deepcopy(v) for v in (vals, yb, xd, ybd))
    args = []
    for a, kind in k.args:
        if kind in ("f", "Af"):
            args += [vals[a], yb[a]]
        else:
            args.append(_int_value(k, a, kind))
    for a, kind in k.float_args:
        args += [xd[a], ybd[a]]
    stacks = _stack_args(lib, k, fname, f"initstacks_{k.name}_b")
    ret = lib.call(fname, *args, *stacks)
    scal = [a for a, kind in k.args if kind == "f"]
    for j, a in enumerate(scal):
        yb[a] = ret[2 * j]
        ybd[a] = ret[2 * j + 1]
    return flatten(k, yb), flatten(k, ybd)


# ---------------------------------------------------------------------------------------------
# the oracles
# ---------------------------------------------------------------------------------------------

def dotprod(lib_d: OracleLib, lib_b: OracleLib, k: Kernel, base: dict, seed: int, trials: int = 3):
    """max over trials of |<yb, J xd> - <J' yb, xd>| / max(|lhs|, |rhs|, 1)."""
    g = jrng.Xoshiro(seed)
    worst = 0.0
    for _ in range(trials):
        xd = random_values(k, g)
        yb = random_values(k, g)
        yd = call_tangent(lib_d, k, base, xd)
        xb = call_adjoint(lib_b, k, base, yb)
        lhs = float(np.dot(flatten(k, yb), yd))
        rhs = float(np.dot(xb, flatten(k, xd)))
        worst = max(worst, abs(lhs - rhs) / max(abs(lhs), abs(rhs), 1.0))
    return worst


def _unit(g, n):
    d = jrng.val_randn(g, n)
    return d / np.sqrt(np.sum(d * d))


def fd_adjoint(lib_p: OracleLib, lib_b: OracleLib, k: Kernel, base: dict, seed: int, trials: int = 3,
               eps: float = 1e-6):
    g = jrng.Xoshiro(seed)
    x0 = flatten(k, base)
    sd = random_values(k, g)
    sflat = flatten(k, sd)
    grad = call_adjoint(lib_b, k, base, sd)
    worst = 0.0
    for _ in range(trials):
        d = _unit(g, len(x0))
        fp = float(np.dot(sflat, call_primal(lib_p, k, unflatten(k, x0 + eps * d))))
        fm = float(np.dot(sflat, call_primal(lib_p, k, unflatten(k, x0 - eps * d))))
        fd = (fp - fm) / (2 * eps)
        ad = float(np.dot(grad, d))
        worst = max(worst, abs(fd - ad) / max(abs(fd), abs(ad), 1e-12))
    return worst


def fd_tangent(lib_p: OracleLib, lib_d: OracleLib, k: Kernel, base: dict, seed: int, trials: int = 3,
               eps: float = 1e-6):
    g = jrng.Xoshiro(seed)
    x0 = flatten(k, base)
    worst = 0.0
    for _ in range(trials):
        d = _unit(g, len(x0))
        fd = (call_primal(lib_p, k, unflatten(k, x0 + eps * d)) - call_primal(lib_p, k, unflatten(k, x0 - eps * d))) / (2 * eps)
        jv = call_tangent(lib_d, k, base, unflatten(k, d))
        denom = max(np.max(np.abs(fd)), np.max(np.abs(jv)), 1e-12)
        worst = max(worst, float(np.max(np.abs(fd - jv)) / denom))
    return worst


def fd_hvp(lib_b: OracleLib, lib_hv: OracleLib, k: Kernel, base: dict, seed: int, trials: int = 3,
           eps: float = 1e-6):
    g = jrng.Xoshiro(seed)
    x0 = flatten(k, base)
    sd = random_values(k, g)
    zero = zeros_like(k)
    worst = 0.0
    for _ in range(trials):
        v = _unit(g, len(x0))
        gp = call_adjoint(lib_b, k, unflatten(k, x0 + eps * v), sd)
        gm = call_adjoint(lib_b, k, unflatten(k, x0 - eps * v), sd)
        fd = (gp - gm) / (2 * eps)
        _, hv = call_hvp(lib_hv, k, base, sd, unflatten(k, v), zero)
        denom = max(np.max(np.abs(fd)), np.max(np.abs(hv)), 1e-12)
        worst = max(worst, float(np.max(np.abs(fd - hv)) / denom))
    return worst
