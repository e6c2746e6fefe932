"""The oracle's Float32 mode: `precision="f32"` restates `cgen_convert_precision`
(/root/reference/src/STADE.jl:15351-15365): every float literal becomes `T(literal)` of the
parsed Float64 literal, the `Float64` element type of STADE's own stack allocations becomes
Float32, and Int64 (branch and tripcount stacks, indices) is untouched.  Arrays are the
caller's (Float32 here), and Julia's promotion rules still apply to what the conversion leaves
alone (`Int / Int` is a Float64, and Float32 op Float64 is Float64).

Pins, each chosen so that a plausible mistake in the mode fails it:
- closed-form unit texts whose Float32 result differs from the Float64 one in a known way
  (a literal left in Float64, a literal rounded once instead of twice, Int / Int evaluated
  in Float32, a Float64 stack, a converted Int64 stack);
- mistakes planted in the oracle (the transpiler's literal conversion switched off) that
  those texts catch;
- the Float32 oracle on the mlp2_ce and conv3x3 golden inputs against the torch float64
  fixtures (tests/golden/make_golden.py), at the fp32 parity bar.
"""
import numpy as np
import pytest

from helpers import CORPUS

F32_RTOL = 1e-5


def _load(text, precision="f32"):
    from oracle import runner
    return runner.load(text, precision=precision, bounds_check=True)


LIT_TEXT = """
function lit(y, x)
    y[1] = (x[1] + 1.0e-8) - x[1]
    y[2] = 1.0000000596046447753906250001 - 1.0
    y[3] = x[2] * (1 / 3)
    return nothing
end
"""

X = np.array([1.0, np.float32(1.0) / np.float32(7.0)])


def test_f32_literals_and_promotion():
    lib = _load(LIT_TEXT)
    y = np.zeros(3, dtype=np.float32)
    lib.call("lit", y, X.astype(np.float32))
    # (1) the literal is Float32: 1 + 1f-8 rounds to 1 in Float32 (a Float64 literal gives 1e-8)
    assert y[0] == 0.0
    # (2) T(literal) of the parsed Float64 literal: 1 + 2^-24 + tiny parses to 1 + 2^-24 in
    #     Float64, a tie that rounds to 1 in Float32 (a C float literal rounds once, to 1 + 2^-23)
    assert y[1] == 0.0
    # (3) Int / Int is a Float64, so x * (1 / 3) is a Float64 product rounded once into the
    #     Float32 array (all-Float32 arithmetic gives 0.047619052)
    x2 = np.float32(X[1])
    assert y[2] == np.float32(np.float64(x2) * (1 / 3))
    assert y[2] != x2 * np.float32(1 / 3)


def test_f64_mode_keeps_float64():
    lib = _load(LIT_TEXT, "f64")
    y = np.zeros(3)
    lib.call("lit", y, X.copy())
    assert y[0] == (1.0 + 1.0e-8) - 1.0 != 0.0
    assert y[1] == float("1.0000000596046447753906250001") - 1.0 != 0.0


STACK_TEXT = """
function initstacks_st_b(n)
    fs = Vector{Float64}(undef, max(0, div(n - 1, 1) + 1))
    bs = Vector{Int64}(undef, max(0, div(n - 1, 1) + 1))
    return (fs, bs)
end
function st_b(y, x, n, fs, bs)
    for i = 1:n
        fs[i] = x[i] + 1.0e-9
        bs[i] = 1099511627777 + i
    end
    for i = 1:n
        y[i] = fs[i] - x[i]
    end
    return nothing
end
"""


def test_f32_stacks():
    lib = _load(STACK_TEXT)
    fs, bs = lib.stacks("initstacks_st_b", 3)
    # the Float64 stack becomes Float32; the Int64 stack is untouched
    assert fs.dtype == np.float32 and bs.dtype == np.int64
    y = np.zeros(3, dtype=np.float32)
    lib.call("st_b", y, np.ones(3, dtype=np.float32), 3, fs, bs)
    assert np.all(y == 0.0)                        # 1 + 1e-9 stored in a Float32 slot is 1
    assert list(bs) == [2 ** 40 + 1 + i for i in (1, 2, 3)]   # 2^40 + k survives: not a float


def test_f64_stacks():
    lib = _load(STACK_TEXT, "f64")
    fs, bs = lib.stacks("initstacks_st_b", 3)
    assert fs.dtype == np.float64 and bs.dtype == np.int64
    y = np.zeros(3)
    lib.call("st_b", y, np.ones(3), 3, fs, bs)
    assert np.all(y == (1.0 + 1.0e-9) - 1.0)


def _planted(monkeypatch, mistake):
    """The transpiler with one mistake planted in its Float32 mode (CPU only)."""
    from oracle import jl2c
    orig = jl2c.CGen.ex

    def ex(self, e):
        r = orig(self, e)
        if self.f32 and e[0] == "num" and r[1] == "f":
            lit = e[1]
            txt = lit if ("." in lit or "e" in lit) else lit + ".0"
            if mistake == "literal_left_float64":
                return (txt, "f")
            if mistake == "literal_rounded_once":
                return (txt + "f", "f")
        return r
    monkeypatch.setattr(jl2c.CGen, "ex", ex)


@pytest.mark.parametrize("mistake,slot", [("literal_left_float64", 0), ("literal_rounded_once", 1)])
def test_planted_literal_mistakes_are_caught(monkeypatch, mistake, slot):
    _planted(monkeypatch, mistake)
    lib = _load(LIT_TEXT)
    y = np.zeros(3, dtype=np.float32)
    lib.call("lit", y, X.astype(np.float32))
    assert y[slot] != 0.0, f"the planted mistake {mistake} was not visible"


def test_planted_float32_division_is_caught(monkeypatch):
    """Int / Int evaluated in Float32 (a plausible shortcut in an all-Float32 mode) changes slot 2."""
    from oracle import jl2c
    orig = jl2c.CGen.binop

    def binop(self, e):
        r = orig(self, e)
        if self.f32 and e[1] == "/" and r[0].startswith("((double)"):
            return (r[0].replace("(double)", "(float)"), r[1])
        return r
    monkeypatch.setattr(jl2c.CGen, "binop", binop)
    lib = _load(LIT_TEXT)
    y = np.zeros(3, dtype=np.float32)
    lib.call("lit", y, X.astype(np.float32))
    x2 = np.float32(X[1])
    assert y[2] != np.float32(np.float64(x2) * (1 / 3))


@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("name", ["mlp2_ce", "conv3x3"])
def test_f32_oracle_matches_golden(name, mode):
    """The Float32 oracle on the golden inputs against torch's float64 autograd of the same
    primal, at the fp32 parity bar (the GPU is compared with this mode in every parity test
    of these two configs)."""
    import test_golden as tg
    fx = np.load(tg.GOLDEN / f"{name}.npz")
    args, sizes = tg._args(name, mode, fx, np.float32)
    from helpers import oracle_lib
    lib = oracle_lib(name, mode, "f32")
    ret = lib.call(f"{name}_{mode}", *[v for _, v in args])
    err = tg._check(name, mode, fx, {a: v for a, v in args}, ret, F32_RTOL)
    assert max(err.values()) > 0.0, "a Float32 evaluation that matches float64 exactly computes in float64"
