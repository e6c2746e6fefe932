"""A CPU check of the general lowering's ownership decisions.

The lowering runs a loop one iteration per GPU thread when its analysis finds every plainly
written array element owned by one iteration (an index expression injective in the loop
variable), with accumulations at shared elements made atomic (`analysis.classify`).  Nothing
on the GPU checks that trust: a race shows up only when the hardware's order happens to break
it.  The reference checks its own emission the same way (/root/reference/test/
ownership_shim.jl:1-120): it runs every launch one logical thread at a time, records every array
access by thread, and reports an element as unsafe when two threads plainly write it, one
plainly writes it and another reads or atomically adds to it, or one reads it and another
atomically adds to it.

Here the function the planner planned (after the finishing, gather and fusion rewrites) runs
in the 50-digit executor (tests/xtruth.py), every iteration of every loop the plan runs in
parallel a logical thread.  Accumulations into arrays the plan makes atomic count as atomic
additions; every other access is a plain read or write.  The cases: the reference corpus's
generated functions at their fixture sizes, and the five configs' and the generic texts at small
sizes.  A planted analysis mistake must be caught.
"""
from __future__ import annotations

import json

import numpy as np
import pytest

import xtruth
from helpers import CORPUS, REF_CORPUS, ROOT, make_args


def plan_tracer(fl) -> xtruth.Tracer:
    """A tracer for the loops of a FuncLower's plan that run one iteration per thread."""
    from stade_hip.lower.hipgen import HostLoopOp, IfOp, ParOp
    par = {}

    def visit(ops):
        for op in ops:
            if isinstance(op, ParOp):
                par[id(op.pl.loop)] = {n: u.kind for n, u in op.pl.arrays.items()}
            elif isinstance(op, HostLoopOp):
                visit(op.ops)
            elif isinstance(op, IfOp):
                for b in op.branches:
                    visit(b)
    visit(fl.ops)
    return xtruth.Tracer(par)


def check_ownership(text: str, fname: str, args, precision: str = "f64") -> xtruth.Tracer:
    from stade_hip.lower import hipgen
    fl = hipgen.lower_function(text, fname, precision=precision)
    tr = plan_tracer(fl)
    xtruth.run_func(fl.f, [v.copy() if isinstance(v, np.ndarray) else v for v in args], tracer=tr)
    return tr


def _ref_cases():
    path = ROOT / "tests" / "golden" / "ref_corpus.json"
    return json.loads(path.read_text()) if path.exists() else []


@pytest.mark.skipif(not REF_CORPUS.exists(), reason="reference corpus not mounted")
def test_reference_corpus_plans_own_what_they_write():
    """Every reference generated function, at its smallest fixture case: no element that two
    iterations of a parallel loop plainly write, or that one writes and another reads or adds
    to, or that one reads and another adds to."""
    from helpers import seeded_inputs
    seen = {}
    for c in _ref_cases():
        seen.setdefault((c["name"], c["mode"]), c)
    z = np.load(ROOT / "tests" / "golden" / "ref_corpus.npz")
    bad, loops, funcs, skipped = [], 0, 0, []
    for (name, mode), case in sorted(seen.items()):
        text = (REF_CORPUS / f"{name}_{mode}.jl").read_text()
        ia = {a: z[f"{case['key']}/in/{a}"] for a, kind, _, _ in case["args"] if kind == "Ai"}
        args = seeded_inputs(case["args"], case["ints"], case["seed"], ia, zeros=case.get("zeros", ()),
                             scales=case.get("scales"))
        try:
            tr = check_ownership(text, f"{name}_{mode}", [v for _, _, v in args])
        except (NotImplementedError, ValueError, IndexError, TypeError) as e:
            skipped.append(f"{name}_{mode}: {type(e).__name__} {str(e)[:60]}")
            continue
        funcs += 1
        loops += tr.loops_checked
        bad += [(f"{name}_{mode}",) + v for v in tr.violations[:3]]
    print(f"{funcs} functions, {loops} parallel loop runs checked; skipped {len(skipped)}: {skipped[:4]}")
    assert not bad, bad[:10]
    assert funcs >= 400 and loops >= 1000


CONFIG_CASES = {
    "affine_lsq": (dict(i_m=6, i_n=5), dict(loss=1, w=(6, 5), x=5, b=6, t=6, r=6), {}, None),
    "diffusion2d": (dict(n=5), dict(loss=1, u=25, un=25), {}, None),
    "burgers1d": (dict(n=9, nsteps=4), dict(loss=1, u=9, un=9), dict(nu=0.05, dt=0.1, dx=0.5, tend=100.0), None),
    "mlp2_ce": (dict(i_b=3, i_in=4, i_h=5, i_out=3), dict(loss=1, x=12, w1=20, b1=5, w2=15, b2=3, h1=15, z=9), {},
                dict(lab=np.array([1, 3, 2], dtype=np.int64))),
    "conv3x3": (dict(i_nb=1, i_c=2, i_k=2, i_h=4, i_w=3), dict(loss=1, xp=60, w=36, out=24), {}, None),
    "generic/matvec_scatter": (dict(i_m=5, i_n=4), dict(loss=1, a=20, x=4, y=5), {}, None),
    "generic/flatmv": (dict(i_m=5, i_n=4), dict(loss=1, a=20, x=4, y=5), {}, None),
    "generic/window1d": (dict(i_n=11, i_k=4), dict(loss=1, inp=11, w=4, out=8), {}, None),
    "generic/binsum": (dict(i_n=13, i_b=4), dict(loss=1, v=13, c=4), {},
                       dict(bins=np.array([1, 2, 3, 4, 1, 2, 3, 4, 2, 2, 3, 1, 4], dtype=np.int64))),
}


@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("name", sorted(CONFIG_CASES))
def test_config_and_generic_plans_own_what_they_write(name, mode):
    from oracle import runner
    ints, base, scalars, ia = CONFIG_CASES[name]
    path = CORPUS / f"{name}_{mode}.jl"
    stem = name.split("/")[-1]
    lib = runner.load(path)
    fname = f"{stem}_{mode}"
    info = lib.infos[fname]
    init = f"initstacks_{stem}_b"
    stacks, names = [], ()
    if mode != "d" and init in lib.infos:
        st = lib.stacks(init, *[ints[a] if k == "i" else scalars[a] for a, k in lib.infos[init].args])
        stacks = [np.zeros(len(s), np.int64) if s.dtype == np.int64 else np.zeros(len(s)) for s in st]
        names = tuple(a for a, _ in info.args[len(info.args) - len(st):]) if st else ()
    shapes = {k + s: v for k, v in base.items() for s in ("", "b", "d", "bd")}
    shapes["__stacks__"] = names
    args = make_args(lib, fname, shapes, ints, scalars, f"own-{fname}", np.float64, int_arrays=ia)
    tr = check_ownership(path.read_text(), fname, [v for _, _, v in args] + stacks)
    assert tr.loops_checked > 0
    assert not tr.violations, tr.violations[:5]


@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("name", ["mlp2_ce", "conv3x3"])
def test_contracted_plans_own_what_they_write(name, mode):
    """The fp32 plans, whose dense-layer loops became matrix products (contract.py): the loops
    that remain (and the loops that fill the products' offset tables) write only what they own."""
    from oracle import runner
    ints, base, scalars, ia = CONFIG_CASES[name]
    path = CORPUS / f"{name}_{mode}.jl"
    lib = runner.load(path)
    fname = f"{name}_{mode}"
    shapes = {k + s: v for k, v in base.items() for s in ("", "b", "d", "bd")}
    args = make_args(lib, fname, shapes, ints, scalars, f"own32-{fname}", np.float64, int_arrays=ia)
    tr = check_ownership(path.read_text(), fname, [v for _, _, v in args], precision="f32")
    assert tr.loops_checked > 0
    assert not tr.violations, tr.violations[:5]


PLANTED = """function race_b(x, y, n)
    for i = 1:n
        k = div(i - 1, 2) + 1
        y[k] = x[i]
    end
    return nothing
end
"""


def test_planted_misclassification_is_caught(monkeypatch):
    """A plain write at a non-injective index: the real analysis keeps the loop in order (no
    parallel loop, nothing to check); an analysis that takes every index for injective (a
    plausible mistake in `linear_in`) runs it in parallel with y owned, and the check reports
    two iterations writing one element."""
    from stade_hip.lower import analysis
    x, y = np.arange(1.0, 9.0), np.zeros(4)
    tr = check_ownership(PLANTED, "race_b", [x, y, 8])
    assert tr.loops_checked == 0 and not tr.violations
    monkeypatch.setattr(analysis, "linear_in", lambda p, name: ({(): 1}, {}))
    tr = check_ownership(PLANTED, "race_b", [x, y, 8])
    assert tr.loops_checked == 1
    assert any(v[3] == "multi_writer" and v[1] == "y" for v in tr.violations), tr.violations


def test_planted_atomic_read_is_caught():
    """The checker itself: a read of an element another iteration adds to atomically."""
    from stade_hip.lower import syntax as S
    text = """function r_b(a, c, n)
    for i = 1:n
        a[1] = a[1] + c[i]
        c[i] = a[1]
    end
    return nothing
end
"""
    f = S.parse(text)[0]
    loop = f.body[0]
    tr = xtruth.Tracer({id(loop): {"a": "atomic", "c": "owned"}})
    xtruth.run_func(f, [np.zeros(1), np.ones(3), 3], tracer=tr)
    assert any(v[3] == "read_vs_atomic" and v[1] == "a" for v in tr.violations), tr.violations
