"""The lowering's contractions onto the matrix cores (stade_hip/lower/contract.py) on the CPU.

A rewritten function (matrix-product statements around the loops that remain) must compute
what the generated text computes: both run in the 50-digit decimal executor (tests/xtruth.py,
which runs a product statement by its definition, element by element through the offsets and
leading dimensions the rewrite chose), and every output agrees to 1e-40 relative (the
products reassociate the sums).  Cases: the MLP config's three texts, texts with the other
storage orders and with offsets, and texts the rewrite must leave alone.  A planted layout
mistake must be caught.
"""
from __future__ import annotations

from decimal import Decimal

import numpy as np
import pytest

import xtruth
from helpers import CORPUS, ROOT, make_args

TEXTS = ROOT / "tests" / "texts"


def _lower(text, fname, precision="f32", inbounds=True):
    from stade_hip.lower import hipgen
    return hipgen.lower_function(text, fname, precision=precision, inbounds=inbounds)


def _same(a0, r0, a1, r1, what):
    for k, (x0, x1) in enumerate(zip(a0, a1)):
        if x0 is None:
            continue
        for e, (p, q) in enumerate(zip(x0, x1)):
            if p is None or q is None:
                assert p is q, f"{what}: argument {k} element {e} set by one version only"
                continue
            assert p == q or abs(Decimal(p) - Decimal(q)) <= Decimal("1e-40") * (1 + abs(Decimal(p))), \
                f"{what}: argument {k} element {e}: {p} vs {q}"
    assert len(r0) == len(r1)
    for p, q in zip(r0, r1):
        assert abs(Decimal(p) - Decimal(q)) <= Decimal("1e-40") * (1 + abs(Decimal(p))), f"{what}: returned {p} vs {q}"


def _equivalent(text, fname, args, precision="f32"):
    from stade_hip.lower import syntax as S
    f0 = next(g for g in S.parse(text) if g.name == fname)
    fl = _lower(text, fname, precision)
    cp = lambda: [v.copy() if isinstance(v, np.ndarray) else v for v in args]
    a0, r0 = xtruth.run_func(f0, cp())
    a1, r1 = xtruth.run_func(fl.f, cp())
    _same(a0, r0, a1, r1, fname)
    return fl


# ---- the MLP config ------------------------------------------------------------------------------

MLP = dict(i_b=3, i_in=5, i_h=4, i_out=3)


@pytest.mark.parametrize("mode", ["b", "d", "hv"])
def test_mlp_texts_contract_and_agree(mode):
    from oracle import runner
    path = CORPUS / f"mlp2_ce_{mode}.jl"
    lib = runner.load(path)
    fname = f"mlp2_ce_{mode}"
    B, I, H, O = MLP["i_b"], MLP["i_in"], MLP["i_h"], MLP["i_out"]
    base = dict(loss=1, x=I * B, w1=H * I, b1=H, w2=O * H, b2=O, h1=H * B, z=O * B)
    shapes = {k + s: v for k, v in base.items() for s in ("", "b", "d", "bd")}
    args = make_args(lib, fname, shapes, MLP, {}, f"contract-{fname}", np.float64,
                     int_arrays=dict(lab=np.array([2, 3, 1], dtype=np.int64)))
    fl = _equivalent(path.read_text(), fname, [v for _, _, v in args])
    rec = fl.contract_rec
    # every dense-layer loop: the forward sums (twice in the adjoint: the backward recomputes
    # s1), and the two adjoint scatters
    assert rec["forward"] == {"b": 3, "d": 2, "hv": 3}[mode]
    assert rec["adjoint"] == {"b": 2, "d": 0, "hv": 2}[mode]
    # the backward loop's recomputed forward sums read the forward loop's products
    assert rec.get("reused", 0) == {"b": 1, "d": 0, "hv": 2}[mode]


CONV = dict(i_nb=2, i_c=2, i_k=3, i_h=3, i_w=4)


@pytest.mark.parametrize("mode", ["b", "d", "hv"])
def test_conv_texts_contract_by_tables_and_agree(mode):
    """The convolution's loops run over a four-digit flat index (x, y, output channel,
    sample) with a three-digit tap index: the table form, whose products gather both factors
    through offset tables and add into the input shadow atomically."""
    from oracle import runner
    path = CORPUS / f"conv3x3_{mode}.jl"
    lib = runner.load(path)
    fname = f"conv3x3_{mode}"
    N, C, K, H, W = (CONV[k] for k in ("i_nb", "i_c", "i_k", "i_h", "i_w"))
    base = dict(loss=1, xp=(W + 2) * (H + 2) * C * N, w=9 * C * K, out=W * H * K * N)
    shapes = {k + s: v for k, v in base.items() for s in ("", "b", "d", "bd")}
    args = make_args(lib, fname, shapes, CONV, {}, f"contract-{fname}", np.float64)
    fl = _equivalent(path.read_text(), fname, [v for _, _, v in args])
    rec = fl.contract_rec
    assert rec["forward"] == 1 and rec["adjoint"] == {"b": 1, "d": 0, "hv": 1}[mode]
    plan = fl_plan(fl)
    assert "offset tables" in plan and ("added atomically" in plan) == (mode != "d")


def fl_plan(fl) -> str:
    from stade_hip.lower import hipgen
    return " | ".join(hipgen.describe(fl.ops))


def test_f64_and_checked_texts_are_not_contracted():
    text = (CORPUS / "mlp2_ce_b.jl").read_text()
    assert not _lower(text, "mlp2_ce_b", "f64").contract_rec
    assert not _lower(text, "mlp2_ce_b", "f32", inbounds=False).contract_rec


# ---- other storage orders, offsets ---------------------------------------------------------------

# w row-major (k contiguous), an offset into x, the adjoint loop with index temporaries
ROWMAJOR = (TEXTS / "dense_rm_b.jl").read_text()

# the flat loop's fast coordinate is the batch: T(s, j) and the transposed scatters
BATCHFAST = (TEXTS / "dense_bf_b.jl").read_text()


def _dense_args(b=3, i=5, h=4, pad=2):
    r = np.random.default_rng(7)
    return [r.standard_normal(b * h), r.standard_normal(b * i + pad), np.zeros(b * i + pad),
            r.standard_normal(h * i), np.zeros(h * i), b, i, h]


@pytest.mark.parametrize("text", [ROWMAJOR, BATCHFAST], ids=["rowmajor", "batchfast"])
def test_other_layouts_contract_and_agree(text):
    fl = _equivalent(text, "dense_b", _dense_args())
    assert fl.contract_rec["forward"] == 1 and fl.contract_rec["adjoint"] == 1
    assert fl.contract_rec["gemms"] == 3


# ---- what must stay a loop ----------------------------------------------------------------------

@pytest.mark.parametrize("change", [
    # the accumulated array is read elsewhere in the loop
    ("        sb = y[(i_s - 1) * i_h + i_j] * 2.0\n", "        sb = y[(i_s - 1) * i_h + i_j] * 2.0 + xb[1]\n"),
    # a factor is written in the loop
    ("        y[idx] = s\n", "        y[idx] = s\n        w[idx] = 0.0\n"),
    # an offset that does not split into a part of the outer loop and a part of the inner one
    ("w[(i_j - 1) * i_in + i_k] * x", "w[(i_j - 1) * i_k + i_k] * x"),
])
def test_loops_that_are_not_contractions_stay(change):
    old, new = change
    text = ROWMAJOR.replace(old, new)
    assert text != ROWMAJOR
    fl = _lower(text, "dense_b")
    rec = fl.contract_rec or {"forward": 0, "adjoint": 0}
    assert rec["forward"] + rec["adjoint"] == 1, rec    # the other loop of the pair still is


def test_strides_other_than_one_take_the_table_form():
    """No unit stride in either direction: not the strided form, but the table form's gathers
    (the forward loop's products through offset tables), agreeing with the text."""
    text = ROWMAJOR.replace("w[(i_j - 1) * i_in + i_k] * x", "w[(i_j - 1) * i_in * 2 + i_k * 2 - 1] * x")
    b, i, h = 3, 5, 4
    args = _dense_args(b, i, h)
    args[3] = np.random.default_rng(3).standard_normal(2 * h * i)
    fl = _equivalent(text, "dense_b", args)
    assert fl.contract_rec["forward"] == 1 and "offset tables" in fl_plan(fl)


def test_planted_layout_mistake_is_caught(monkeypatch):
    """A rewrite that reads an operand in the other storage order (a plausible slip in
    choosing A_KM / B_KM) computes other sums: the decimal comparison fails."""
    from stade_hip.lower import contract
    real = contract._Rewriter.layout

    def flipped(a):
        km, ld = real(a)
        return (not km), ld
    monkeypatch.setattr(contract._Rewriter, "layout", staticmethod(flipped))
    with pytest.raises((AssertionError, IndexError, ValueError)):
        _equivalent(ROWMAJOR, "dense_b", _dense_args(b=3, i=5, h=5, pad=0))


def test_planted_table_mistake_is_caught(monkeypatch):
    """A table form that places a digit one step off (d P_d instead of (d - 1) P_d, a plausible
    slip in the mixed radix) reads or writes the wrong elements: the decimal comparison fails."""
    from stade_hip.lower import contract
    from oracle import runner
    real = contract._Tables.place

    def shifted(self, D):
        p = real(self, D)
        for d in D[:1]:
            for m, c in d.P.items():
                p[m] = p.get(m, 0) + c
        return {m: c for m, c in p.items() if c}
    monkeypatch.setattr(contract._Tables, "place", shifted)
    path = CORPUS / "conv3x3_b.jl"
    lib = runner.load(path)
    N, C, K, H, W = (CONV[k] for k in ("i_nb", "i_c", "i_k", "i_h", "i_w"))
    base = dict(loss=1, xp=(W + 2) * (H + 2) * C * N, w=9 * C * K, out=W * H * K * N)
    shapes = {k + s: v for k, v in base.items() for s in ("", "b", "d", "bd")}
    args = make_args(lib, "conv3x3_b", shapes, CONV, {}, "contract-planted", np.float64)
    with pytest.raises((AssertionError, IndexError, ValueError)):
        _equivalent(path.read_text(), "conv3x3_b", [v for _, _, v in args])


TWICE = """function twice_b(y, y2, x, w, i_b, i_in, i_h)
    for idx = 1:i_b * i_h
        i_s = div(idx - 1, i_h) + 1
        i_j = mod(idx - 1, i_h) + 1
        s = 0.0
        for i_k = 1:i_in
            s = s + w[(i_k - 1) * i_h + i_j] * x[(i_s - 1) * i_in + i_k]
        end
        y[idx] = s
    end
    BETWEEN
    for idx = 1:i_b * i_h
        i_s = div(idx - 1, i_h) + 1
        i_j = mod(idx - 1, i_h) + 1
        s = 1.0
        for i_k = 1:i_in
            s = s + w[(i_k - 1) * i_h + i_j] * x[(i_s - 1) * i_in + i_k]
        end
        y2[idx] = tanh(s)
    end
    return nothing
end
"""


@pytest.mark.parametrize("between,reused", [("", 1), ("w[1] = w[1] * 2.0", 0), ("y[1] = 0.0", 1)])
def test_a_repeated_product_is_reused_only_while_its_operands_stand(between, reused):
    text = TWICE.replace("BETWEEN", between)
    r = np.random.default_rng(5)
    b, i, h = 3, 5, 4
    args = [np.zeros(b * h), np.zeros(b * h), r.standard_normal(b * i), r.standard_normal(h * i), b, i, h]
    fl = _equivalent(text, "twice_b", args)
    assert fl.contract_rec.get("reused", 0) == reused
