"""The lowering's kernel finishing passes (stade_hip/lower/finish.py) on the CPU.

Each pass follows a reference function:
- dead restores and the stack stores they leave unread: `cgen_dead_pops`
  /root/reference/src/STADE.jl:12356;
- merged accumulations: `cgen_merge_accum` 18144;
- dead scalars: `cgen_dead_scalars` 12369 over `cgen_dead_walk` 12151;
- unchecked accesses: `cgen_inbounds_wrap` 12376.

Two kinds of check:
- Unit texts, with planted cases each pass must leave alone: a value read after a `break`, an
  array between two accumulations, a restore that is read, a read that may raise.
- Equivalence: on every reference generated function the passes change (where the reference is
  mounted), the finished function gives the original's results in 50-digit decimal arithmetic
  (tests/xtruth.py), on seeded inputs.  A stack that lost stores is compared where the finished
  code still writes it.
"""
from __future__ import annotations

import json
import time
from decimal import Decimal

import numpy as np
import pytest

import xtruth
from helpers import REF_CORPUS, ROOT


def _fin(text, fname, stacks=(), inbounds=True):
    from stade_hip.lower import finish, syntax as S
    f = next(g for g in S.parse(text) if g.name == fname)
    return f, *finish.finish(f, set(stacks), inbounds=inbounds)


def _src(f) -> str:
    return repr(f.body)


# ---- merged accumulations ----------------------------------------------------------------

MERGE = """function m_b(a, x, y, n)
    for i = 1:n
        a[i] = a[i] + x[i]
        t = 2.0 * y[i]
        a[i] = a[i] + t
    end
    return nothing
end
"""


def test_merge_two_accumulations():
    f0, f, rec = _fin(MERGE, "m_b")
    assert rec["merged"] == 1
    from stade_hip.lower import syntax as S
    accs = [s for s in S.walk_stmts(f.body) if isinstance(s, S.Assign) and isinstance(s.lhs, S.Ref)]
    assert len(accs) == 1
    assert isinstance(accs[0].rhs, S.Bin) and isinstance(accs[0].rhs.b, S.Bin) and accs[0].rhs.b.op == "+"


@pytest.mark.parametrize("between", [
    "t = 2.0 * a[i]",          # reads the array between the two
    "x[i] = 1.0",              # not a scalar assignment
])
def test_no_merge_across(between):
    text = MERGE.replace("t = 2.0 * y[i]", between).replace("a[i] = a[i] + t", "a[i] = a[i] + y[i]")
    _, _, rec = _fin(text, "m_b")
    assert rec["merged"] == 0


def test_no_merge_when_the_first_value_changes():
    """`t` feeds the first addition and is reassigned between them: merging would add the new t."""
    text = """function m_b(a, x, y, n)
    for i = 1:n
        t = x[i]
        a[i] = a[i] + t
        t = 2.0 * y[i]
        a[i] = a[i] + t
    end
    return nothing
end
"""
    _, _, rec = _fin(text, "m_b")
    assert rec["merged"] == 0


# ---- dead scalars -------------------------------------------------------------------------

def test_dead_scalar_assignments_go():
    text = """function d_b(a, n)
    s = 0.0
    for i = 1:n
        u = a[i] * 2.0
        w = u + 1.0
        a[i] = u
    end
    s = 0.0
    return nothing
end
"""
    _, f, rec = _fin(text, "d_b")
    assert rec["dead_scalars"] == 3   # w, and both resets of s
    assert "'w'" not in _src(f) and "'s'" not in _src(f)


def test_lone_accumulation_in_a_loop_is_dead():
    """`s = s + x` alone in a loop, never read after it: dead in the least fixpoint."""
    text = """function d_b(a, n)
    s = 0.0
    for i = 1:n
        s = s + a[i]
    end
    return nothing
end
"""
    _, _, rec = _fin(text, "d_b")
    assert rec["dead_scalars"] == 2


def test_value_read_after_a_break_stays():
    """x = 1.0 reaches the read after the loop through the break."""
    text = """function d_b(a, n)
    r = 0.0
    for i = 1:n
        x = 1.0
        if a[i] > 0.0
            break
        end
        x = 2.0
    end
    a[1] = x
    return nothing
end
"""
    _, f, rec = _fin(text, "d_b")
    from stade_hip.lower import syntax as S
    xs = [s for s in S.walk_stmts(f.body) if isinstance(s, S.Assign) and isinstance(s.lhs, S.Var) and s.lhs.name == "x"]
    assert len(xs) == 2


def test_returned_scalar_stays():
    text = """function d_d(a, n, v)
    s = 0.0
    for i = 1:n
        s = s + a[i]
    end
    vd = 2.0 * s
    return vd
end
"""
    _, _, rec = _fin(text, "d_d")
    assert rec["dead_scalars"] == 0


def test_array_read_dead_only_when_inbounds():
    """A dead `u = a[k]` may raise an out-of-range error when accesses are checked."""
    text = """function d_b(a, k)
    u = a[k]
    return nothing
end
"""
    assert _fin(text, "d_b", inbounds=True)[2]["dead_scalars"] == 1
    assert _fin(text, "d_b", inbounds=False)[2]["dead_scalars"] == 0


# ---- dead pops ------------------------------------------------------------------------------

POPS = """function p_b(x, xb, n, s_stack)
    s = 0.0
    for i = 1:n
        s_stack[i] = s
        s = x[i]
    end
    for i = n:-1:1
        s = s_stack[i]
        s = 3.0
        xb[i] = xb[i] + s
    end
    return nothing
end
"""


def test_dead_restore_and_its_store_go():
    _, f, rec = _fin(POPS, "p_b", stacks={"s_stack"})
    assert rec["dead_restores"] == 1 and rec["dead_stacks"] == ["s_stack"]
    assert "s_stack" not in _src(f)


def test_live_restore_and_its_store_stay():
    text = POPS.replace("        s = 3.0\n", "")
    _, f, rec = _fin(text, "p_b", stacks={"s_stack"})
    assert rec["dead_restores"] == 0 and rec["dead_stacks"] == []
    assert _src(f).count("s_stack") == 2


def test_only_the_files_own_stacks():
    """A restore from an array that no initstacks allocates is not a pop."""
    _, _, rec = _fin(POPS, "p_b", stacks=set())
    assert rec["dead_restores"] == 0


# ---- inbounds ---------------------------------------------------------------------------------

def test_inbounds_drops_the_checks():
    from stade_hip.lower import hipgen
    text = (ROOT / "stade.jl_amd" / "corpus" / "generic" / "binsum_b.jl").read_text()
    checked, sc = hipgen.generate(text, "f64", inbounds=False)
    plain, sp = hipgen.generate(text, "f64", inbounds=True)
    # call sites of the checked accessors, and the accumulations' range tests
    uses = lambda src: (src.count("rd(a.A_"), src.count("wr(a.A_"), src.count("< (uint64_t)a.N_"))
    assert all(k > 0 for k in uses(checked)), uses(checked)
    assert uses(plain) == (0, 0, 0), uses(plain)
    assert sp["binsum_b"]["inbounds"] and not sc["binsum_b"]["inbounds"]


# ---- equivalence on the reference's generated code --------------------------------------------

def _ref_cases():
    path = ROOT / "tests" / "golden" / "ref_corpus.json"
    return json.loads(path.read_text()) if path.exists() else []


@pytest.mark.skipif(not REF_CORPUS.exists(), reason="reference corpus not mounted")
def test_finished_functions_equal_the_originals_in_decimal():
    """Every reference function that a pass changes, on its smallest fixture case: the finished
    syntax tree and the original give the same outputs and returns in 50-digit arithmetic
    (to 1e-40, the merges' reassociation), except the slots of stacks whose stores were deleted."""
    from helpers import seeded_inputs
    from stade_hip.lower import finish, hipgen, syntax as S
    cases = {}
    for c in _ref_cases():
        cases.setdefault((c["name"], c["mode"]), c)
    checked, skipped, t0 = 0, [], time.time()
    for (name, mode), case in sorted(cases.items()):
        text = (REF_CORPUS / f"{name}_{mode}.jl").read_text()
        fname = f"{name}_{mode}"
        funcs = {g.name: g for g in S.parse(text)}
        allocated = set()
        for g in funcs.values():
            if g.name.startswith("initstacks_"):
                allocated |= {s.lhs.name for s in S.walk_stmts(g.body)
                              if isinstance(s, S.Assign) and isinstance(s.lhs, S.Var) and isinstance(s.rhs, S.Alloc)}
        f = funcs[fname]
        g, rec = finish.finish(f, allocated)
        if not any(rec[k] for k in ("dead_restores", "merged", "dead_scalars")):
            continue
        ia = {a: np.array(case["ints"].get(a, 0)) for a in ()}
        z = np.load(ROOT / "tests" / "golden" / "ref_corpus.npz")
        ia = {a: z[f"{case['key']}/in/{a}"] for a, kind, _, _ in case["args"] if kind == "Ai"}
        args = seeded_inputs(case["args"], case["ints"], case["seed"], ia, zeros=case.get("zeros", ()),
                             scales=case.get("scales"))
        vals = [v for _, _, v in args]
        try:
            a0, r0 = xtruth.run_func(f, [v.copy() if isinstance(v, np.ndarray) else v for v in vals])
        except (NotImplementedError, ValueError, IndexError, TypeError) as e:
            skipped.append(f"{fname}: {type(e).__name__}")
            continue
        a1, r1 = xtruth.run_func(g, [v.copy() if isinstance(v, np.ndarray) else v for v in vals])
        dead = set(rec["dead_stacks"])
        for (an, kind, v), x0, x1 in zip(args, a0, a1):
            if x0 is None:
                continue
            if an in dead:
                before = list(np.ravel(v, order="F"))
                for k, (p, q) in enumerate(zip(x0, x1)):
                    if q is not None and q != before[k]:
                        assert p == q or abs(Decimal(p) - Decimal(q)) <= Decimal("1e-40") * (1 + abs(Decimal(p))), \
                            f"{fname}: stack {an}[{k + 1}] differs where the finished code writes it"
                continue
            for k, (p, q) in enumerate(zip(x0, x1)):
                if p is None or q is None:
                    assert p is q, f"{fname}: {an}[{k + 1}] written by one version only"
                    continue
                assert p == q or abs(Decimal(p) - Decimal(q)) <= Decimal("1e-40") * (1 + abs(Decimal(p))), \
                    f"{fname}: {an}[{k + 1}]: {p} vs {q}"
        assert len(r0) == len(r1)
        for p, q in zip(r0, r1):
            assert p == q or abs(Decimal(p) - Decimal(q)) <= Decimal("1e-40") * (1 + abs(Decimal(p))), f"{fname}: returned {p} vs {q}"
        checked += 1
    print(f"{checked} finished functions equal their originals ({len(skipped)} skipped: {skipped[:5]}), "
          f"{time.time() - t0:.1f} s")
    assert checked >= 150
