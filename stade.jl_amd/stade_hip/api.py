"""ctypes bindings of libstade_hip.so and the generated-function mirrors built on them."""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

_PKG = Path(__file__).resolve().parent.parent
_DEFAULT_LIB = _PKG / "lib" / "libstade_hip.so"


class StadeHipError(RuntimeError):
    """A nonzero return code of a libstade_hip entry point, with the library's message."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed with code {code}: {msg}")
        self.code = code


class StadeHipBoundsError(IndexError):
    """An index the generated code would reject with a BoundsError (a label outside
    1..i_out), seen by a kernel and reported through the device error flag."""


def lib_path() -> Path:
    return Path(os.environ.get("STADE_HIP_LIB", str(_DEFAULT_LIB)))


_lib = None

P = ctypes.c_void_p
I64 = ctypes.c_int64
F64 = ctypes.c_double
F64P = ctypes.POINTER(ctypes.c_double)
U64P = ctypes.POINTER(ctypes.c_uint64)

# C signatures: argument kinds in generated-function order.
#   'a' device array pointer, 'i' Int64 by value, 'f' Float64 by value, 'r' host in/out
#   Float64 (a scalar shadow), 's' stream (appended by the caller)
ENTRY_POINTS: dict[str, str] = {
    "stade_hip_affine_lsq_b": "aaaaaaaaaaaaii",
    "stade_hip_affine_lsq_d": "aaaaaaaaaaaaii",
    "stade_hip_affine_lsq_hv": "aaaaaaaaaaaaii" + "aaaaaaaaaaaa",
    "stade_hip_diffusion2d_b": "aaaaaai",
    "stade_hip_diffusion2d_d": "aaaaaai",
    "stade_hip_diffusion2d_hv": "aaaaaai" + "aaaaaa",
    "stade_hip_burgers1d_b": "aaaaaa" + "frfrfrfr" + "ii" + "aa",
    "stade_hip_burgers1d_d": "aaaaaa" + "ffffffff" + "ii",
    "stade_hip_burgers1d_hv": "aaaaaa" + "frfrfrfr" + "ii" + "aaaaaa" + "frfrfrfr" + "aa",
    "stade_hip_burgers1d_b_ckpt": "aaaaaa" + "frfrfrfr" + "ii" + "aa" + "i",
    "stade_hip_burgers1d_hv_ckpt": "aaaaaa" + "frfrfrfr" + "ii" + "aaaaaa" + "frfrfrfr" + "aa" + "i",
    "stade_hip_mlp2_ce_b": "a" * 17 + "iiii",
    "stade_hip_mlp2_ce_d": "a" * 17 + "iiii",
    "stade_hip_mlp2_ce_hv": "a" * 17 + "iiii" + "a" * 16,
    "stade_hip_conv3x3_b": "a" * 8 + "iiiii",
    "stade_hip_conv3x3_d": "a" * 8 + "iiiii",
    "stade_hip_conv3x3_hv": "a" * 8 + "iiiii" + "a" * 8,
}

_CT = {"a": P, "i": I64, "f": F64, "r": F64P}


def hip_runtime_first():
    """Load torch (and with it the HIP runtime it carries) before any library of this package.

    The libraries link libamdhip64.so.7; loaded first, they would bring in /opt/rocm's copy,
    and torch would then load its own next to it.  Two HIP runtimes in one process do not
    share the device (the second one's launches fail with "no ROCm-capable device"), so the
    runtime torch carries is loaded first and the libraries resolve to it."""
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


def lib():
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        hip_runtime_first()
        path = lib_path()
        if not path.exists():
            raise RuntimeError(f"libstade_hip.so not found at {path}: build it with "
                               f"`python stade.jl_amd/build.py` (or __graft_entry__.build())")
        L = ctypes.CDLL(str(path))
        L.stade_hip_last_error.restype = ctypes.c_char_p
        L.stade_hip_version.restype = ctypes.c_char_p
        L.stade_hip_stable_seed.restype = ctypes.c_uint64
        L.stade_hip_stable_seed.argtypes = [ctypes.c_char_p]
        L.stade_hip_rng_seed.argtypes = [ctypes.c_uint64, U64P]
        L.stade_hip_rng_normal_f64.argtypes = [U64P, P, I64]
        L.stade_hip_rng_uniform_f64.argtypes = [U64P, P, I64, F64, F64]
        L.stade_hip_rng_int_range.argtypes = [U64P, P, I64, I64, I64]
        for nm in ("stade_hip_rng_seed", "stade_hip_rng_normal_f64", "stade_hip_rng_uniform_f64",
                   "stade_hip_rng_int_range", "stade_hip_free", "stade_hip_synchronize", "stade_hip_device_error"):
            getattr(L, nm).restype = ctypes.c_int32
        L.stade_hip_device_error.argtypes = [ctypes.POINTER(ctypes.c_int32)]
        L.stade_hip_free.argtypes = [P]
        L.stade_hip_workspace_info.argtypes = [ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64)]
        L.stade_hip_synchronize.argtypes = [P]
        for nm, kinds in ENTRY_POINTS.items():
            f = getattr(L, nm)
            f.restype = ctypes.c_int32
            f.argtypes = [_CT[k] for k in kinds] + [P]
        _lib = L
    return _lib


def _check(fn: str, rc: int):
    if rc != 0:
        msg = lib().stade_hip_last_error().decode(errors="replace")
        raise StadeHipError(fn, rc, msg)


# ------------------------------------------------------------------------------------------
# inputs: Julia's Xoshiro stream (host)
# ------------------------------------------------------------------------------------------

def stable_seed(name: str) -> int:
    """`val_stable_seed(name)`: FNV-1a64 of the UTF-8 bytes."""
    return int(lib().stade_hip_stable_seed(name.encode()))


class Rng:
    """`Random.Xoshiro(seed)` scalar draws (host, C++)."""

    def __init__(self, seed: int):
        self.state = (ctypes.c_uint64 * 4)()
        _check("stade_hip_rng_seed", lib().stade_hip_rng_seed(ctypes.c_uint64(seed), self.state))


def rng_normal(rng: Rng, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float64)
    _check("stade_hip_rng_normal_f64", lib().stade_hip_rng_normal_f64(rng.state, out.ctypes.data, n))
    return out


def rng_uniform(rng: Rng, n: int, lo: float = 0.0, hi: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float64)
    _check("stade_hip_rng_uniform_f64", lib().stade_hip_rng_uniform_f64(rng.state, out.ctypes.data, n, lo, hi))
    return out


def rng_int_range(rng: Rng, n: int, lo: int, hi: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int64)
    _check("stade_hip_rng_int_range", lib().stade_hip_rng_int_range(rng.state, out.ctypes.data, n, lo, hi))
    return out


# ------------------------------------------------------------------------------------------
# argument marshalling
# ------------------------------------------------------------------------------------------

def _stream_of(t):
    """The raw HIP stream that torch's current stream of t's device wraps (an int).  torch's
    raw-stream query is used where it exists (it skips building a Stream object per call)."""
    import torch
    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if raw is not None:
        return raw(t.get_device())
    return torch.cuda.current_stream(t.device).cuda_stream


def _arr(name: str, t, dtype, numel: int | None):
    """Device pointer (an int) of a flat contiguous GPU tensor of the given dtype and length.
    The accepted case is tested first in one expression (an evaluation passes a dozen arrays,
    so the checks are a visible part of a small call); anything else falls through to the
    checks that name what is wrong."""
    import torch
    if (isinstance(t, torch.Tensor) and t.is_cuda and t.dtype is dtype and t.is_contiguous()
            and (numel is None or t.numel() == numel)):
        return t.data_ptr()
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a torch tensor on a GPU, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise ValueError(f"{name}: tensor is on {t.device}, not on a GPU (there is no CPU path)")
    if t.dtype != dtype:
        raise TypeError(f"{name}: dtype {t.dtype}, expected {dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: tensor must be contiguous (Julia column-major data, flat)")
    if numel is not None and t.numel() != numel:
        raise ValueError(f"{name}: length {t.numel()}, expected {numel}")
    return t.data_ptr()


def _int(name: str, v) -> int:
    if isinstance(v, bool) or not isinstance(v, (int, np.integer)):
        raise TypeError(f"{name}: expected an Int64, got {type(v).__name__}")
    return int(v)


def _call(fn: str, args: list, stream):
    _check(fn, getattr(lib(), fn)(*args, stream))


def device_error() -> int:
    """Read and clear the device error flag (`stade_hip_device_error`): nonzero if a kernel
    saw an index the generated code would reject since the flag was last read.  Waits for
    the device."""
    flag = ctypes.c_int32(0)
    _check("stade_hip_device_error", lib().stade_hip_device_error(ctypes.byref(flag)))
    return int(flag.value)


def workspace_info() -> tuple[int, int]:
    """(bytes of scratch held, scratch buffers retired) of the current device's library
    workspace (`stade_hip_workspace_info`): a buffer is retired, not freed, when a larger call
    needs more scratch after a graph captured a call that used it."""
    b, r = ctypes.c_int64(0), ctypes.c_int64(0)
    _check("stade_hip_workspace_info", lib().stade_hip_workspace_info(ctypes.byref(b), ctypes.byref(r)))
    return int(b.value), int(r.value)


def _bounds(fn: str, check: bool):
    """`check=True` is the generated code's bounds checking (`stade_amdgpu_file(...;
    inbounds=false)`, /root/reference/src/STADE.jl:18604-18605): the flag is read after the
    call, at the cost of one synchronisation, and a raised flag is a BoundsError.  The default
    matches the reference's GPU default, `inbounds=true`: no check, and an out-of-range label
    contributes no term."""
    if check and device_error():
        raise StadeHipBoundsError(f"{fn}: a label is outside 1..i_out (the generated code raises a BoundsError)")


# ------------------------------------------------------------------------------------------
# config 1: affine_lsq(loss, w, x, b, t, r, i_m, i_n)
# ------------------------------------------------------------------------------------------

def _f64():
    import torch
    return torch.float64


def affine_lsq_b(loss, lossb, w, wb, x, xb, b, bb, t, tb, r, rb, i_m, i_n):
    """Adjoint of affine_lsq (corpus/affine_lsq_b.jl); returns nothing."""
    m, n = _int("i_m", i_m), _int("i_n", i_n)
    d = _f64()
    a = [_arr("loss", loss, d, 1), _arr("lossb", lossb, d, 1), _arr("w", w, d, m * n), _arr("wb", wb, d, m * n),
         _arr("x", x, d, n), _arr("xb", xb, d, n), _arr("b", b, d, m), _arr("bb", bb, d, m),
         _arr("t", t, d, m), _arr("tb", tb, d, m), _arr("r", r, d, m), _arr("rb", rb, d, m), m, n]
    _call("stade_hip_affine_lsq_b", a, _stream_of(w))


def affine_lsq_d(loss, lossd, w, wd, x, xd, b, bd, t, td, r, rd, i_m, i_n):
    """Tangent of affine_lsq (corpus/affine_lsq_d.jl); returns nothing."""
    m, n = _int("i_m", i_m), _int("i_n", i_n)
    d = _f64()
    a = [_arr("loss", loss, d, 1), _arr("lossd", lossd, d, 1), _arr("w", w, d, m * n), _arr("wd", wd, d, m * n),
         _arr("x", x, d, n), _arr("xd", xd, d, n), _arr("b", b, d, m), _arr("bd", bd, d, m),
         _arr("t", t, d, m), _arr("td", td, d, m), _arr("r", r, d, m), _arr("rd", rd, d, m), m, n]
    _call("stade_hip_affine_lsq_d", a, _stream_of(w))


def affine_lsq_hv(loss, lossb, w, wb, x, xb, b, bb, t, tb, r, rb, i_m, i_n,
                  lossd, lossbd, wd, wbd, xd, xbd, bd, bbd, td, tbd, rd, rbd):
    """HVP of affine_lsq (corpus/affine_lsq_hv.jl); returns nothing."""
    m, n = _int("i_m", i_m), _int("i_n", i_n)
    d = _f64()
    a = [_arr("loss", loss, d, 1), _arr("lossb", lossb, d, 1), _arr("w", w, d, m * n), _arr("wb", wb, d, m * n),
         _arr("x", x, d, n), _arr("xb", xb, d, n), _arr("b", b, d, m), _arr("bb", bb, d, m),
         _arr("t", t, d, m), _arr("tb", tb, d, m), _arr("r", r, d, m), _arr("rb", rb, d, m), m, n,
         _arr("lossd", lossd, d, 1), _arr("lossbd", lossbd, d, 1), _arr("wd", wd, d, m * n), _arr("wbd", wbd, d, m * n),
         _arr("xd", xd, d, n), _arr("xbd", xbd, d, n), _arr("bd", bd, d, m), _arr("bbd", bbd, d, m),
         _arr("td", td, d, m), _arr("tbd", tbd, d, m), _arr("rd", rd, d, m), _arr("rbd", rbd, d, m)]
    _call("stade_hip_affine_lsq_hv", a, _stream_of(w))


# ------------------------------------------------------------------------------------------
# config 2: diffusion2d(loss, u, un, n)
# ------------------------------------------------------------------------------------------

def diffusion2d_b(loss, lossb, u, ub, un, unb, n):
    """Adjoint of diffusion2d (corpus/diffusion2d_b.jl); returns nothing."""
    n = _int("n", n)
    d, c = _f64(), n * n
    a = [_arr("loss", loss, d, 1), _arr("lossb", lossb, d, 1), _arr("u", u, d, c), _arr("ub", ub, d, c),
         _arr("un", un, d, c), _arr("unb", unb, d, c), n]
    _call("stade_hip_diffusion2d_b", a, _stream_of(u))


def diffusion2d_d(loss, lossd, u, ud, un, und, n):
    """Tangent of diffusion2d (corpus/diffusion2d_d.jl); returns nothing."""
    n = _int("n", n)
    d, c = _f64(), n * n
    a = [_arr("loss", loss, d, 1), _arr("lossd", lossd, d, 1), _arr("u", u, d, c), _arr("ud", ud, d, c),
         _arr("un", un, d, c), _arr("und", und, d, c), n]
    _call("stade_hip_diffusion2d_d", a, _stream_of(u))


def diffusion2d_hv(loss, lossb, u, ub, un, unb, n, lossd, lossbd, ud, ubd, und, unbd):
    """HVP of diffusion2d (corpus/diffusion2d_hv.jl); returns nothing."""
    n = _int("n", n)
    d, c = _f64(), n * n
    a = [_arr("loss", loss, d, 1), _arr("lossb", lossb, d, 1), _arr("u", u, d, c), _arr("ub", ub, d, c),
         _arr("un", un, d, c), _arr("unb", unb, d, c), n,
         _arr("lossd", lossd, d, 1), _arr("lossbd", lossbd, d, 1), _arr("ud", ud, d, c), _arr("ubd", ubd, d, c),
         _arr("und", und, d, c), _arr("unbd", unbd, d, c)]
    _call("stade_hip_diffusion2d_hv", a, _stream_of(u))


# ------------------------------------------------------------------------------------------
# config 5: burgers1d(loss, u, un, nu, dt, dx, tend, n, nsteps)
# ------------------------------------------------------------------------------------------

def burgers1d_stack_lengths(n: int, nsteps: int) -> tuple[int, int]:
    """Lengths of initstacks_burgers1d_b's (branch_stack, u_stack)."""
    out = (ctypes.c_int64 * 2)()
    L = lib()
    L.stade_hip_burgers1d_stack_lengths.argtypes = [I64, I64, ctypes.POINTER(ctypes.c_int64)]
    _check("stade_hip_burgers1d_stack_lengths", L.stade_hip_burgers1d_stack_lengths(_int("n", n), _int("nsteps", nsteps), out))
    return int(out[0]), int(out[1])


def initstacks_burgers1d_b(n, nsteps, device=None):
    """initstacks_burgers1d_b (corpus/burgers1d_b.jl): (branch_stack Int64, u_stack Float64),
    allocated uninitialised on the GPU as the generated code allocates them with `undef`."""
    import torch
    lb, lu = burgers1d_stack_lengths(n, nsteps)
    dev = device or torch.device("cuda", torch.cuda.current_device())
    return (torch.empty(lb, dtype=torch.int64, device=dev), torch.empty(lu, dtype=torch.float64, device=dev))


def _r(v) -> ctypes.c_double:
    if isinstance(v, bool) or not isinstance(v, (int, float, np.floating, np.integer)):
        raise TypeError(f"expected a Float64, got {type(v).__name__}")
    return ctypes.c_double(float(v))


def burgers1d_b(loss, lossb, u, ub, un, unb, nu, nub, dt, dtb, dx, dxb, tend, tendb, n, nsteps, branch_stack, u_stack):
    """Adjoint of burgers1d (corpus/burgers1d_b.jl); returns (nub, dtb, dxb, tendb)."""
    import torch
    n, T = _int("n", n), _int("nsteps", nsteps)
    lb, lu = burgers1d_stack_lengths(n, T)
    d = _f64()
    rs = [_r(v) for v in (nub, dtb, dxb, tendb)]
    a = [_arr("loss", loss, d, 1), _arr("lossb", lossb, d, 1), _arr("u", u, d, n), _arr("ub", ub, d, n),
         _arr("un", un, d, n), _arr("unb", unb, d, n),
         float(nu), ctypes.byref(rs[0]), float(dt), ctypes.byref(rs[1]), float(dx), ctypes.byref(rs[2]),
         float(tend), ctypes.byref(rs[3]), n, T,
         _arr("branch_stack", branch_stack, torch.int64, lb), _arr("u_stack", u_stack, d, lu)]
    _call("stade_hip_burgers1d_b", a, _stream_of(u))
    return tuple(r.value for r in rs)


def burgers1d_d(loss, lossd, u, ud, un, und, nu, nud, dt, dtd, dx, dxd, tend, tendd, n, nsteps):
    """Tangent of burgers1d (corpus/burgers1d_d.jl); returns nothing."""
    n, T = _int("n", n), _int("nsteps", nsteps)
    d = _f64()
    a = [_arr("loss", loss, d, 1), _arr("lossd", lossd, d, 1), _arr("u", u, d, n), _arr("ud", ud, d, n),
         _arr("un", un, d, n), _arr("und", und, d, n),
         float(nu), float(nud), float(dt), float(dtd), float(dx), float(dxd), float(tend), float(tendd), n, T]
    _call("stade_hip_burgers1d_d", a, _stream_of(u))


def burgers1d_hv(loss, lossb, u, ub, un, unb, nu, nub, dt, dtb, dx, dxb, tend, tendb, n, nsteps,
                 lossd, lossbd, ud, ubd, und, unbd, nud, nubd, dtd, dtbd, dxd, dxbd, tendd, tendbd,
                 branch_stack, u_stack):
    """HVP of burgers1d (corpus/burgers1d_hv.jl); returns (nub, nubd, dtb, dtbd, dxb, dxbd, tendb, tendbd)."""
    import torch
    n, T = _int("n", n), _int("nsteps", nsteps)
    lb, lu = burgers1d_stack_lengths(n, T)
    d = _f64()
    rs = [_r(v) for v in (nub, dtb, dxb, tendb)]
    rd = [_r(v) for v in (nubd, dtbd, dxbd, tendbd)]
    a = [_arr("loss", loss, d, 1), _arr("lossb", lossb, d, 1), _arr("u", u, d, n), _arr("ub", ub, d, n),
         _arr("un", un, d, n), _arr("unb", unb, d, n),
         float(nu), ctypes.byref(rs[0]), float(dt), ctypes.byref(rs[1]), float(dx), ctypes.byref(rs[2]),
         float(tend), ctypes.byref(rs[3]), n, T,
         _arr("lossd", lossd, d, 1), _arr("lossbd", lossbd, d, 1), _arr("ud", ud, d, n), _arr("ubd", ubd, d, n),
         _arr("und", und, d, n), _arr("unbd", unbd, d, n),
         float(nud), ctypes.byref(rd[0]), float(dtd), ctypes.byref(rd[1]), float(dxd), ctypes.byref(rd[2]),
         float(tendd), ctypes.byref(rd[3]),
         _arr("branch_stack", branch_stack, torch.int64, lb), _arr("u_stack", u_stack, d, lu)]
    _call("stade_hip_burgers1d_hv", a, _stream_of(u))
    return (rs[0].value, rd[0].value, rs[1].value, rd[1].value, rs[2].value, rd[2].value, rs[3].value, rd[3].value)


def burgers1d_ckpt_lengths(n: int, nsteps: int, every: int) -> tuple[int, int]:
    """Lengths of (branch_stack, u_ckpt) under the checkpoint policy (every `every`-th state)."""
    L = lib()
    out = (ctypes.c_int64 * 2)()
    L.stade_hip_burgers1d_ckpt_lengths.argtypes = [I64, I64, I64, ctypes.POINTER(ctypes.c_int64)]
    _check("stade_hip_burgers1d_ckpt_lengths",
           L.stade_hip_burgers1d_ckpt_lengths(_int("n", n), _int("nsteps", nsteps), _int("every", every), out))
    return int(out[0]), int(out[1])


def burgers1d_b_ckpt(loss, lossb, u, ub, un, unb, nu, nub, dt, dtb, dx, dxb, tend, tendb, n, nsteps, branch_stack, u_ckpt,
                     every):
    """burgers1d_b under the checkpoint tape policy: u_ckpt (every `every`-th state) instead of
    u_stack, the segments recomputed in the reverse sweep; the other outputs are burgers1d_b's.
    Returns (nub, dtb, dxb, tendb)."""
    import torch
    n, T, every = _int("n", n), _int("nsteps", nsteps), _int("every", every)
    lb, lc = burgers1d_ckpt_lengths(n, T, every)
    d = _f64()
    rs = [_r(v) for v in (nub, dtb, dxb, tendb)]
    a = [_arr("loss", loss, d, 1), _arr("lossb", lossb, d, 1), _arr("u", u, d, n), _arr("ub", ub, d, n),
         _arr("un", un, d, n), _arr("unb", unb, d, n),
         float(nu), ctypes.byref(rs[0]), float(dt), ctypes.byref(rs[1]), float(dx), ctypes.byref(rs[2]),
         float(tend), ctypes.byref(rs[3]), n, T,
         _arr("branch_stack", branch_stack, torch.int64, lb), _arr("u_ckpt", u_ckpt, d, lc), every]
    _call("stade_hip_burgers1d_b_ckpt", a, _stream_of(u))
    return tuple(r.value for r in rs)


def burgers1d_hv_ckpt(loss, lossb, u, ub, un, unb, nu, nub, dt, dtb, dx, dxb, tend, tendb, n, nsteps,
                      lossd, lossbd, ud, ubd, und, unbd, nud, nubd, dtd, dtbd, dxd, dxbd, tendd, tendbd,
                      branch_stack, u_ckpt, every):
    """burgers1d_hv under the checkpoint tape policy (see burgers1d_b_ckpt).  Returns (nub, nubd,
    dtb, dtbd, dxb, dxbd, tendb, tendbd)."""
    import torch
    n, T, every = _int("n", n), _int("nsteps", nsteps), _int("every", every)
    lb, lc = burgers1d_ckpt_lengths(n, T, every)
    d = _f64()
    rs = [_r(v) for v in (nub, dtb, dxb, tendb)]
    rd = [_r(v) for v in (nubd, dtbd, dxbd, tendbd)]
    a = [_arr("loss", loss, d, 1), _arr("lossb", lossb, d, 1), _arr("u", u, d, n), _arr("ub", ub, d, n),
         _arr("un", un, d, n), _arr("unb", unb, d, n),
         float(nu), ctypes.byref(rs[0]), float(dt), ctypes.byref(rs[1]), float(dx), ctypes.byref(rs[2]),
         float(tend), ctypes.byref(rs[3]), n, T,
         _arr("lossd", lossd, d, 1), _arr("lossbd", lossbd, d, 1), _arr("ud", ud, d, n), _arr("ubd", ubd, d, n),
         _arr("und", und, d, n), _arr("unbd", unbd, d, n),
         float(nud), ctypes.byref(rd[0]), float(dtd), ctypes.byref(rd[1]), float(dxd), ctypes.byref(rd[2]),
         float(tendd), ctypes.byref(rd[3]),
         _arr("branch_stack", branch_stack, torch.int64, lb), _arr("u_ckpt", u_ckpt, d, lc), every]
    _call("stade_hip_burgers1d_hv_ckpt", a, _stream_of(u))
    return (rs[0].value, rd[0].value, rs[1].value, rd[1].value, rs[2].value, rd[2].value, rs[3].value, rd[3].value)


# ------------------------------------------------------------------------------------------
# config 3: mlp2_ce(loss, x, lab, w1, b1, w2, b2, h1, z, i_b, i_in, i_h, i_out)   (Float32)
# ------------------------------------------------------------------------------------------

def _f32():
    import torch
    return torch.float32


def _mlp_sizes(i_b, i_in, i_h, i_out):
    B, I, H, O = (_int(n, v) for n, v in (("i_b", i_b), ("i_in", i_in), ("i_h", i_h), ("i_out", i_out)))
    return B, I, H, O, dict(loss=1, x=I * B, w1=H * I, b1=H, w2=O * H, b2=O, h1=H * B, z=O * B)



def mlp2_ce_b(loss, lossb, x, xb, lab, w1, w1b, b1, b1b, w2, w2b, b2, b2b, h1, h1b, z, zb, i_b, i_in, i_h, i_out, check=False):
    """Adjoint of mlp2_ce (corpus/mlp2_ce_b.jl); returns nothing.  check=True raises
    StadeHipBoundsError for a label outside 1..i_out (one synchronisation)."""
    import torch
    B, I, H, O, s = _mlp_sizes(i_b, i_in, i_h, i_out)
    f = _f32()
    a = [_arr("loss", loss, f, 1), _arr("lossb", lossb, f, 1), _arr("x", x, f, s["x"]), _arr("xb", xb, f, s["x"]),
         _arr("lab", lab, torch.int64, B), _arr("w1", w1, f, s["w1"]), _arr("w1b", w1b, f, s["w1"]),
         _arr("b1", b1, f, H), _arr("b1b", b1b, f, H), _arr("w2", w2, f, s["w2"]), _arr("w2b", w2b, f, s["w2"]),
         _arr("b2", b2, f, O), _arr("b2b", b2b, f, O), _arr("h1", h1, f, s["h1"]), _arr("h1b", h1b, f, s["h1"]),
         _arr("z", z, f, s["z"]), _arr("zb", zb, f, s["z"]), B, I, H, O]
    _call("stade_hip_mlp2_ce_b", a, _stream_of(x))
    _bounds("mlp2_ce_b", check)


def mlp2_ce_d(loss, lossd, x, xd, lab, w1, w1d, b1, b1d, w2, w2d, b2, b2d, h1, h1d, z, zd, i_b, i_in, i_h, i_out, check=False):
    """Tangent of mlp2_ce (corpus/mlp2_ce_d.jl); returns nothing.  check as for mlp2_ce_b."""
    import torch
    B, I, H, O, s = _mlp_sizes(i_b, i_in, i_h, i_out)
    f = _f32()
    a = [_arr("loss", loss, f, 1), _arr("lossd", lossd, f, 1), _arr("x", x, f, s["x"]), _arr("xd", xd, f, s["x"]),
         _arr("lab", lab, torch.int64, B), _arr("w1", w1, f, s["w1"]), _arr("w1d", w1d, f, s["w1"]),
         _arr("b1", b1, f, H), _arr("b1d", b1d, f, H), _arr("w2", w2, f, s["w2"]), _arr("w2d", w2d, f, s["w2"]),
         _arr("b2", b2, f, O), _arr("b2d", b2d, f, O), _arr("h1", h1, f, s["h1"]), _arr("h1d", h1d, f, s["h1"]),
         _arr("z", z, f, s["z"]), _arr("zd", zd, f, s["z"]), B, I, H, O]
    _call("stade_hip_mlp2_ce_d", a, _stream_of(x))
    _bounds("mlp2_ce_d", check)


def mlp2_ce_hv(loss, lossb, x, xb, lab, w1, w1b, b1, b1b, w2, w2b, b2, b2b, h1, h1b, z, zb, i_b, i_in, i_h, i_out,
               lossd, lossbd, xd, xbd, w1d, w1bd, b1d, b1bd, w2d, w2bd, b2d, b2bd, h1d, h1bd, zd, zbd, check=False):
    """HVP of mlp2_ce (corpus/mlp2_ce_hv.jl); returns nothing.  check as for mlp2_ce_b."""
    import torch
    B, I, H, O, s = _mlp_sizes(i_b, i_in, i_h, i_out)
    f = _f32()
    a = [_arr("loss", loss, f, 1), _arr("lossb", lossb, f, 1), _arr("x", x, f, s["x"]), _arr("xb", xb, f, s["x"]),
         _arr("lab", lab, torch.int64, B), _arr("w1", w1, f, s["w1"]), _arr("w1b", w1b, f, s["w1"]),
         _arr("b1", b1, f, H), _arr("b1b", b1b, f, H), _arr("w2", w2, f, s["w2"]), _arr("w2b", w2b, f, s["w2"]),
         _arr("b2", b2, f, O), _arr("b2b", b2b, f, O), _arr("h1", h1, f, s["h1"]), _arr("h1b", h1b, f, s["h1"]),
         _arr("z", z, f, s["z"]), _arr("zb", zb, f, s["z"]), B, I, H, O,
         _arr("lossd", lossd, f, 1), _arr("lossbd", lossbd, f, 1), _arr("xd", xd, f, s["x"]), _arr("xbd", xbd, f, s["x"]),
         _arr("w1d", w1d, f, s["w1"]), _arr("w1bd", w1bd, f, s["w1"]), _arr("b1d", b1d, f, H), _arr("b1bd", b1bd, f, H),
         _arr("w2d", w2d, f, s["w2"]), _arr("w2bd", w2bd, f, s["w2"]), _arr("b2d", b2d, f, O), _arr("b2bd", b2bd, f, O),
         _arr("h1d", h1d, f, s["h1"]), _arr("h1bd", h1bd, f, s["h1"]), _arr("zd", zd, f, s["z"]), _arr("zbd", zbd, f, s["z"])]
    _call("stade_hip_mlp2_ce_hv", a, _stream_of(x))
    _bounds("mlp2_ce_hv", check)


# ------------------------------------------------------------------------------------------
# config 4: conv3x3(loss, xp, w, out, i_nb, i_c, i_k, i_h, i_w)   (Float32)
# ------------------------------------------------------------------------------------------

def _conv_sizes(i_nb, i_c, i_k, i_h, i_w):
    N, C, K, H, W = (_int(n, v) for n, v in (("i_nb", i_nb), ("i_c", i_c), ("i_k", i_k), ("i_h", i_h), ("i_w", i_w)))
    return N, C, K, H, W, dict(loss=1, xp=(W + 2) * (H + 2) * C * N, w=9 * C * K, out=W * H * K * N)


def _conv_args(names, arrays, s):
    """Validated pointers; a shadow (`<x>b`, `<x>d`, `<x>bd`) has the length of its primal `<x>`."""
    f = _f32()

    def primal(nm):
        for suffix in ("bd", "b", "d"):
            if nm.endswith(suffix) and nm[: -len(suffix)] in s:
                return nm[: -len(suffix)]
        return nm
    return [_arr(nm, v, f, s[primal(nm)]) for nm, v in zip(names, arrays)]


def conv3x3_b(loss, lossb, xp, xpb, w, wb, out, outb, i_nb, i_c, i_k, i_h, i_w):
    """Adjoint of conv3x3 (corpus/conv3x3_b.jl); returns nothing."""
    N, C, K, H, W, s = _conv_sizes(i_nb, i_c, i_k, i_h, i_w)
    a = _conv_args(("loss", "lossb", "xp", "xpb", "w", "wb", "out", "outb"), (loss, lossb, xp, xpb, w, wb, out, outb), s)
    _call("stade_hip_conv3x3_b", a + [N, C, K, H, W], _stream_of(xp))


def conv3x3_d(loss, lossd, xp, xpd, w, wd, out, outd, i_nb, i_c, i_k, i_h, i_w):
    """Tangent of conv3x3 (corpus/conv3x3_d.jl); returns nothing."""
    N, C, K, H, W, s = _conv_sizes(i_nb, i_c, i_k, i_h, i_w)
    a = _conv_args(("loss", "lossd", "xp", "xpd", "w", "wd", "out", "outd"), (loss, lossd, xp, xpd, w, wd, out, outd), s)
    _call("stade_hip_conv3x3_d", a + [N, C, K, H, W], _stream_of(xp))


def conv3x3_hv(loss, lossb, xp, xpb, w, wb, out, outb, i_nb, i_c, i_k, i_h, i_w,
               lossd, lossbd, xpd, xpbd, wd, wbd, outd, outbd):
    """HVP of conv3x3 (corpus/conv3x3_hv.jl); returns nothing."""
    N, C, K, H, W, s = _conv_sizes(i_nb, i_c, i_k, i_h, i_w)
    a = _conv_args(("loss", "lossb", "xp", "xpb", "w", "wb", "out", "outb"), (loss, lossb, xp, xpb, w, wb, out, outb), s)
    t = _conv_args(("lossd", "lossbd", "xpd", "xpbd", "wd", "wbd", "outd", "outbd"),
                   (lossd, lossbd, xpd, xpbd, wd, wbd, outd, outbd), s)
    _call("stade_hip_conv3x3_hv", a + [N, C, K, H, W] + t, _stream_of(xp))
