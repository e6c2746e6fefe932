"""The oracle's 80-bit truth mode, pinned.

Where the GPU and the fp64 oracle differ by more than the parity bar, the verdict follows the
reference's truth rule (`val_truth_verdict_lines` /root/reference/src/STADE.jl:18915-18932):
the GPU passes if its error against a high-precision truth is at most 20 times the oracle's
own error.  The reference's truth is the generated code rerun on BigFloat copies of the
inputs (`val_gpu_parity_script` 19045-19113).  Here it is the oracle's `f80` mode: the same
text transpiled to C with `long double` (x87 extended, 64-bit significand).  A truth that
silently keeps only double precision inflates both errors, and the 20x rule then admits a
wrong GPU result, so the mode is pinned three ways:

1. Unit texts whose 80-bit result is known in closed form and differs from the fp64 one:
   `1 + 2^-60` survives an array store and a returned scalar; a Float64 literal keeps its
   Float64 value, as the reference's rerun promotes it (`BigFloat * 0.1` multiplies by the
   Float64 0.1, not by a 64-bit rounding of 1/10); `Int / Int` is a Float64 quotient, as in
   Julia; `exp`, `tanh`, `log`, `sqrt` and `literal_pow` keep 64 bits (checked against 50-digit
   decimal values).
2. Planted mistakes, each of which must fail one of those answers: a dropped precision in the
   returned-value buffer, `-mlong-double-64`, literals rounded to 64 bits instead of kept at
   their Float64 value, `Int / Int` in extended precision, the double-precision libm, and the
   runner reading long doubles back through Python floats.
3. The config texts (and, where the reference is mounted, 15 of its generated kernels) at small
   sizes, against a second executor in 50-digit decimal arithmetic (`tests/xtruth.py`: the
   lowering's parser, Python evaluation, no C): the 80-bit results must be within 1e-17 of it
   and well inside the fp64 results' own error.

Deliberate difference from the reference's rerun: a `Vector{Float64}(undef, n)` allocated
inside a generated function (the HVP's `<stack>_d`) is held in extended precision here, while
the reference's rerun retypes `Float64` in `initstacks` only (19057).  That makes this truth
closer to the exact result, which part 3 measures.
"""
from __future__ import annotations

import ctypes
import re
import subprocess
from decimal import Decimal
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

import xtruth
from helpers import CORPUS, REF_CORPUS, make_args

UNIT = """
function t_add(a, b, n)
    for i = 1:n
        a[i] = a[i] + b[i]
    end
    return nothing
end

function t_ret(x, y)
    s = x + y
    return s
end

function t_ret2(a, x)
    s = a[1] + x
    t = s * 3.0
    return (s, t)
end

function t_lit(a)
    a[1] = a[1] * 0.1
    a[2] = 0.1 + a[2]
    return nothing
end

function t_intdiv(a, n, m)
    q = a[n] * (n / m)
    a[n] = q + 0.0 * a[m]
    return nothing
end

function t_libm(a)
    a[1] = exp(a[1])
    a[2] = tanh(a[2])
    a[3] = log(a[3])
    a[4] = sqrt(a[4])
    return nothing
end

function t_pow(a)
    a[1] = a[1] ^ 2
    a[2] = a[2] ^ 3
    a[3] = a[3] ^ -1
    return nothing
end
"""

LD = np.longdouble
TWO60 = LD(2) ** -60


def _exact_ld(fr: Fraction) -> LD:
    """The 64-bit-significand value nearest to a rational (numerator and denominator exact in
    long double, one IEEE division)."""
    return LD(fr.numerator) / LD(fr.denominator)


def _rel_ld(got: LD, want: Decimal) -> float:
    g = Fraction(*LD(got).as_integer_ratio())
    w = Fraction(want)
    return float(abs(g - w) / abs(w))


def unit_failures(lib) -> list[str]:
    """Every known answer of the unit texts that `lib` (an f80 oracle build) gets wrong."""
    bad = []
    a, b = np.ones(3, LD), np.full(3, TWO60, LD)
    lib.call("t_add", a, b, 3)
    if not np.all(a == LD(1) + TWO60):
        bad.append("t_add: 1 + 2^-60 lost in an array store")
    (s,) = lib.call("t_ret", 1.0, float(2.0 ** -60))
    if not (isinstance(s, LD) and s == LD(1) + TWO60):
        bad.append(f"t_ret: returned {s!r}, not 1 + 2^-60")
    s, t = lib.call("t_ret2", np.array([1.0], LD), float(2.0 ** -60))
    if not (s == LD(1) + TWO60 and t == (LD(1) + TWO60) * LD(3)):
        bad.append(f"t_ret2: returned {s!r}, {t!r}")
    a = np.array([1.0, 2.0 ** -60], LD)
    lib.call("t_lit", a)
    f64_01 = LD(np.float64(0.1))
    if a[0] != f64_01:
        bad.append(f"t_lit: 1 * 0.1 gave {a[0]!r}, not the Float64 value of 0.1 ({f64_01!r})")
    if a[1] != _exact_ld(Fraction(0.1) + Fraction(2) ** -60):
        bad.append(f"t_lit: 0.1 + 2^-60 gave {a[1]!r}")
    a = np.array([1.0, 0.0, 0.0], LD)
    lib.call("t_intdiv", a, 1, 3)
    if a[0] != LD(np.float64(1.0) / np.float64(3.0)):
        bad.append(f"t_intdiv: 1 / 3 gave {a[0]!r}, not the Float64 quotient")
    a = np.array([1.0, 0.5, 3.0, 2.0], LD)
    lib.call("t_libm", a)
    e2 = xtruth.CTX.exp(Decimal(1))
    want = [e2, xtruth._tanh(Decimal("0.5")), xtruth.CTX.ln(Decimal(3)), xtruth.CTX.sqrt(Decimal(2))]
    for k, (nm, w) in enumerate(zip(("exp(1)", "tanh(0.5)", "log(3)", "sqrt(2)"), want)):
        r = _rel_ld(a[k], w)
        if r > 2.5e-19:          # 64-bit significand: 1 ulp is 1.08e-19 relative at worst
            bad.append(f"t_libm: {nm} relative error {r:.2e}")
    x1, x2 = LD(1) + LD(2) ** -30, LD(1) + LD(2) ** -25
    a = np.array([x1, x2, 3.0], LD)
    lib.call("t_pow", a)
    if a[0] != _exact_ld(Fraction(1) + Fraction(2) ** -29 + Fraction(2) ** -60):
        bad.append("t_pow: (1 + 2^-30)^2 not exact")
    if a[1] != _exact_ld(Fraction(1) + 3 * Fraction(2) ** -25 + 3 * Fraction(2) ** -50):
        bad.append("t_pow: (1 + 2^-25)^3 not the twice-rounded product")
    if a[2] != LD(1) / LD(3):
        bad.append("t_pow: 3^-1 not inv(3) in 64 bits")
    return bad


def test_f80_unit_known_answers():
    from oracle import runner
    assert ctypes.sizeof(ctypes.c_longdouble) == np.dtype(LD).itemsize == 16
    assert np.finfo(LD).nmant == 63, "the oracle's truth mode needs the x87 80-bit long double"
    lib = runner.load(UNIT, precision="f80", tag="f80_unit")
    assert unit_failures(lib) == []


def test_f64_fails_the_f80_answers():
    """The answers distinguish the precisions: the fp64 build gets the extended ones wrong."""
    from oracle import runner

    class AsF80:
        """An fp64 build called with the f80 test's long double arrays (converted)."""

        def __init__(self, lib):
            self.lib = lib

        def call(self, name, *args):
            conv = [a.astype(np.float64) if isinstance(a, np.ndarray) and a.dtype == LD else a for a in args]
            r = self.lib.call(name, *conv)
            for a, c in zip(args, conv):
                if c is not a:
                    a[...] = c
            return tuple(LD(x) for x in r)
    assert len(unit_failures(AsF80(runner.load(UNIT, precision="f64", tag="f80_unit")))) >= 5


def _build_planted(tmp_path, edit_c=None, cflags=(), name="planted"):
    """The UNIT text transpiled in f80 mode, with `edit_c` applied to the C source and extra
    gcc flags, built into tmp_path and loaded as an oracle library."""
    from oracle import jl2c, runner
    c_src, infos = jl2c.transpile(UNIT, precision="f80", bounds_check=True)
    if edit_c is not None:
        new = edit_c(c_src)
        assert new != c_src, "the planted edit matched nothing"
        c_src = new
    c_path, so = tmp_path / f"{name}.c", tmp_path / f"{name}.so"
    c_path.write_text(c_src)
    subprocess.run(["gcc", *runner.CFLAGS, *cflags, "-o", str(so), str(c_path), "-lm"], check=True,
                   capture_output=True)
    return runner.OracleLib(so, infos, "f80")


PLANTS = {
    # the returned-value buffer written through a double
    "double_return": dict(edit_c=lambda s: s.replace("((long double *)__ret)[1] = (long double)",
                                                     "((long double *)__ret)[1] = (double)")
                          .replace("((long double *)__ret)[0] = (long double)", "((long double *)__ret)[0] = (double)")),
    # Float64 literals rounded to 64 bits (`0.1L`) instead of keeping their Float64 value
    "literal_L_suffix": dict(edit_c=lambda s: re.sub(r"\(\(long double\)(\d+\.\d+)\)", r"(\1L)", s)),
    # Int / Int in extended precision instead of a Float64 quotient
    "intdiv_extended": dict(edit_c=lambda s: re.sub(r"\(\(double\)(\w+) / \(double\)(\w+)\)",
                                                    r"((long double)\1 / (long double)\2)", s)),
    # the double-precision libm in the extended build
    "double_libm": dict(edit_c=lambda s: re.sub(r"\b(exp|tanh|log|sqrt)l\(", r"\1(", s)),
}


@pytest.mark.parametrize("plant", sorted(PLANTS))
def test_f80_planted_mistakes_fail(plant, tmp_path):
    lib = _build_planted(tmp_path, name=plant, **PLANTS[plant])
    assert unit_failures(lib), f"the planted mistake {plant} went unnoticed"


def test_f80_planted_long_double_64_fails(tmp_path):
    """`-mlong-double-64` makes `long double` a double: the library no longer holds 80-bit
    values, and the 16-byte array slots the runner passes are read as 8-byte doubles.  Called in
    a child process: a library built with another long double ABI may leave the x87 state of the
    process that called it unusable for the tests after it."""
    import json
    import sys
    lib = _build_planted(tmp_path, cflags=("-mlong-double-64",), name="ld64")
    code = (
        "import json, sys; sys.path[:0] = %r\n"
        "import test_oracle_f80 as t\n"
        "from oracle import runner, jl2c\n"
        "_, infos = jl2c.transpile(t.UNIT, precision='f80', bounds_check=True)\n"
        "lib = runner.OracleLib(%r, infos, 'f80')\n"
        "try:\n    bad = t.unit_failures(lib)\n"
        "except Exception as e:\n    bad = ['raised ' + type(e).__name__]\n"
        "print(json.dumps(bad))\n") % (sys.path[:6], str(lib.path))
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.strip(), r.stderr[-2000:]
    assert json.loads(r.stdout.strip().splitlines()[-1]), "-mlong-double-64 went unnoticed"


def test_f80_planted_runner_float_readback(tmp_path, monkeypatch):
    """The runner reading returned long doubles as Python floats (what indexing a ctypes
    c_longdouble array does) must fail the returned-scalar answers."""
    from oracle import runner
    lib = runner.load(UNIT, precision="f80", tag="f80_unit")
    monkeypatch.setattr(runner, "_ld_from_buffer", lambda buf, n: [LD(float(x)) for x in buf[:n]])
    bad = unit_failures(lib)
    assert any(b.startswith("t_ret") for b in bad), bad


# ---------------------------------------------------------------------------------------------
# part 3: whole texts against the 50-digit executor
# ---------------------------------------------------------------------------------------------

def _norm_err(got, want) -> float:
    """Normwise relative error of `got` (numbers) against exact decimals `want`."""
    if len(want) == 0:
        return 0.0
    w = [Fraction(x) for x in want]
    g = [Fraction(*LD(x).as_integer_ratio()) for x in got]
    scale = max(abs(x) for x in w)
    diff = max(abs(a - b) for a, b in zip(g, w))
    if scale == 0:
        return float(diff)
    return float(diff / scale)


def _compare_three(path_or_text, fname, args, stacks=()):
    """Run fname in f64 and f80 on the oracle and in decimal; returns (err80, err64, nouts),
    the worst normwise errors of every float output and returned float against the decimal."""
    from oracle import runner
    text = Path(path_or_text).read_text() if isinstance(path_or_text, Path) else path_or_text
    l64 = runner.load(path_or_text, precision="f64")
    l80 = runner.load(path_or_text, precision="f80")
    full = list(args) + list(stacks)
    a64 = [v.copy(order="K") if isinstance(v, np.ndarray) else v for v in full]
    a80 = [v.astype(LD if v.dtype != np.int64 else np.int64, order="K") if isinstance(v, np.ndarray) else v
           for v in full]
    r64 = l64.call(fname, *a64)
    r80 = l80.call(fname, *a80)
    arrs, rx = xtruth.run(text, fname, [v.copy(order="K") if isinstance(v, np.ndarray) else v for v in full])
    e80 = e64 = 0.0
    nouts = 0
    for v, x64, x80, xd in zip(full, a64, a80, arrs):
        if xd is None or (isinstance(v, np.ndarray) and v.dtype == np.int64):
            if xd is not None:
                assert list(np.ravel(x80, order="F")) == xd == list(np.ravel(x64, order="F"))
            continue
        keep = [k for k, q in enumerate(xd) if q is not None]
        want = [xd[k] for k in keep]
        f80 = np.ravel(x80, order="F")[keep]
        f64 = np.ravel(x64, order="F")[keep]
        e80 = max(e80, _norm_err(f80, want))
        e64 = max(e64, _norm_err(f64, want))
        nouts += 1
    assert len(r80) == len(rx) == len(r64)
    for q64, q80, qd in zip(r64, r80, rx):
        if isinstance(qd, Decimal):
            e80 = max(e80, _norm_err([q80], [qd]))
            e64 = max(e64, _norm_err([q64], [qd]))
            nouts += 1
        else:
            assert q80 == qd == q64
    return e80, e64, nouts


def _labels(B, O):
    from oracle import rng as jrng
    return np.array([1 + int(jrng.Xoshiro(17 + s).rand() * O) for s in range(B)], dtype=np.int64)


# name -> (Int64 arguments, base array shapes (shadows take their primal's), float scalars,
#          Int64 arrays, input scales)
CONFIG_CASES = {
    "affine_lsq": (dict(i_m=6, i_n=5), dict(loss=1, w=(6, 5), x=5, b=6, t=6, r=6), {}, None, {}),
    "diffusion2d": (dict(n=5), dict(loss=1, u=25, un=25), {}, None, {}),
    "burgers1d": (dict(n=9, nsteps=5), dict(loss=1, u=9, un=9), dict(nu=0.05, dt=0.1, dx=0.5, tend=100.0), None, {}),
    "mlp2_ce": (dict(i_b=3, i_in=4, i_h=5, i_out=3), dict(loss=1, x=12, w1=20, b1=5, w2=15, b2=3, h1=15, z=9), {},
                dict(lab=_labels(3, 3)), dict(w1=0.6, w1d=0.6, w2=0.6, w2d=0.6)),
    "conv3x3": (dict(i_nb=1, i_c=2, i_k=2, i_h=4, i_w=3), dict(loss=1, xp=6 * 5 * 2, w=9 * 2 * 2, out=4 * 3 * 2), {},
                None, dict(w=0.3, wd=0.3)),
}


def _config_args(name, mode):
    """Seeded small inputs for a config text, and the zeroed stacks its initstacks sizes."""
    from helpers import oracle_lib
    lib = oracle_lib(name, mode)
    fname = f"{name}_{mode}"
    ints, base, scalars, int_arrays, scales = CONFIG_CASES[name]
    info = lib.infos[fname]
    init = f"initstacks_{name}_b"
    stacks, stack_names = [], ()
    if init in lib.infos and mode != "d":
        sizing = [ints[a] if k == "i" else scalars[a] for a, k in lib.infos[init].args]
        st = lib.stacks(init, *sizing)
        if st:
            stack_names = tuple(a for a, _ in info.args[len(info.args) - len(st):])
        stacks = [np.zeros(len(s), np.int64) if s.dtype == np.int64 else np.zeros(len(s)) for s in st]
    shapes = {k + suf: v for k, v in base.items() for suf in ("", "b", "d", "bd")}
    shapes["__stacks__"] = stack_names
    args = make_args(lib, fname, shapes, ints, scalars, f"f80pin-{fname}", np.float64,
                     int_arrays=int_arrays, scales=scales)
    return [v for _, _, v in args], stacks


@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("name", sorted(CONFIG_CASES))
def test_f80_against_decimal_on_config_texts(name, mode):
    """The 80-bit oracle on each config text at a small size, against the 50-digit executor.
    Bars: 80-bit within 1e-17 (about 100 ulp of the format after a few hundred operations)
    and at least 16 times closer than the fp64 run, wherever fp64 is off by more than 1e-16."""
    vals, stacks = _config_args(name, mode)
    e80, e64, nouts = _compare_three(CORPUS / f"{name}_{mode}.jl", f"{name}_{mode}", vals, stacks)
    print(f"{name}_{mode}: {nouts} outputs, f80 {e80:.2e}, f64 {e64:.2e}")
    assert nouts > 0
    assert e80 <= 1e-17, f"{name}_{mode}: the 80-bit truth is {e80:.2e} from the 50-digit result"
    if e64 > 1e-16:
        assert e80 * 16 <= e64, f"{name}_{mode}: f80 {e80:.2e} is not clearly better than f64 {e64:.2e}"


def test_decimal_executor_catches_a_planted_index_mistake():
    """The comparison is not vacuous: a shifted neighbour in the text (a plausible index slip)
    moves the 50-digit result far from the oracle's."""
    text = (CORPUS / "diffusion2d_b.jl").read_text()
    bad = text.replace("ub[__icse_4 + ip] = ub[__icse_4 + ip] + __cse_3",
                       "ub[__icse_4 + im] = ub[__icse_4 + im] + __cse_3", 1)
    assert bad != text
    vals, stacks = _config_args("diffusion2d", "b")
    from oracle import runner
    l80 = runner.load(CORPUS / "diffusion2d_b.jl", precision="f80")
    a80 = [v.astype(LD) if isinstance(v, np.ndarray) else v for v in vals]
    l80.call("diffusion2d_b", *a80)
    arrs, _ = xtruth.run(bad, "diffusion2d_b", [v.copy() if isinstance(v, np.ndarray) else v for v in vals])
    assert _norm_err(a80[3], arrs[3]) > 1e-3


REF_KERNELS = ["affine_loss", "matvec_loss", "stencil_loss", "dotprod", "advection", "mlp1d", "fixed_sweeps",
               "bnd_branch", "selfrace_conv", "relu_field", "clamped_sumsq", "geomrecur", "sumsq_shifted",
               "two_field_loss", "bilinear"]


@pytest.mark.skipif(not REF_CORPUS.exists(), reason="reference corpus not mounted")
@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("name", REF_KERNELS)
def test_f80_against_decimal_on_reference_kernels(name, mode):
    """The reference's own generated code (its committed val-corpus snapshots), at the sizes
    tests/test_oracle_corpus.py uses: the same bars as the config texts."""
    from test_oracle_corpus import CASES
    from oracle import checks, runner, rng as jrng
    path = REF_CORPUS / f"{name}_{mode}.jl"
    ints, shapes = CASES[name]
    ld = runner.load(REF_CORPUS / f"{name}_d.jl")
    lib = runner.load(path)
    k = checks.kernel_from_lib(ld, name, ints, shapes)
    g = jrng.Xoshiro(jrng.val_stable_seed(f"f80pin-{name}-{mode}"))
    fname = f"{name}_{mode}"
    info = lib.infos[fname]
    init = f"initstacks_{name}_b"
    stacks = []
    if mode != "d" and init in lib.infos:
        sizing = [ints[a] for a, _ in lib.infos[init].args]
        stacks = [np.zeros(len(s), np.int64) if s.dtype == np.int64 else np.zeros(len(s))
                  for s in lib.stacks(init, *sizing)]
    nargs = len(info.args) - len(stacks)
    vals = []
    for a, kind in info.args[:nargs]:
        if kind == "i":
            vals.append(int(ints[a]))
        elif kind == "f":
            vals.append(float(jrng.val_normal(g)))
        elif kind == "Ai":
            raise AssertionError(f"{name}: unexpected Int64 array argument {a}")
        else:
            stem = a
            while stem not in k.shapes and stem[-1] in "bd":
                stem = stem[:-1]
            shp = k.shapes[stem]
            shp = shp if isinstance(shp, tuple) else (shp,)
            v = jrng.val_randn(g, int(np.prod(shp)))
            vals.append(np.asfortranarray(v.reshape(shp, order="F")) if len(shp) > 1 else v)
    e80, e64, nouts = _compare_three(path, fname, vals, stacks)
    print(f"{fname}: {nouts} outputs, f80 {e80:.2e}, f64 {e64:.2e}")
    assert e80 <= 1e-17, f"{fname}: the 80-bit truth is {e80:.2e} from the 50-digit result"
    if e64 > 1e-16:
        assert e80 * 16 <= e64
