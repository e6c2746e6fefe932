"""The general lowering (stade_hip.lower) on the CPU: its parser's Julia semantics, type
inference, index analysis, loop plans, host-side initstacks, and the libraries it builds.
The GPU runs are tests/test_gpu_lowered.py."""
import os
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

from helpers import CORPUS, REF_CORPUS

GENERIC = CORPUS / "generic"


def _parse_expr(text):
    from stade_hip.lower import syntax
    f = syntax.parse(f"function f(y)\n    y[1] = {text}\nend\n")[0]
    return f.body[0].rhs


def test_julia_precedence():
    from stade_hip.lower.syntax import Bin, Num, Un, Var
    # juxtaposition binds tighter than / : 1/2x is 1/(2x)
    e = _parse_expr("1 / 2x")
    assert e == Bin("/", Num("1", True), Bin("*", Num("2", True), Var("x")))
    # ^ is right associative and binds tighter than unary minus
    assert _parse_expr("-x ^ 2") == Un("-", Bin("^", Var("x"), Num("2", True)))
    assert _parse_expr("a ^ b ^ c") == Bin("^", Var("a"), Bin("^", Var("b"), Var("c")))
    assert _parse_expr("x ^ -2") == Bin("^", Var("x"), Num("-2", True))
    # a binary operator at the end of a line continues the expression
    from stade_hip.lower import syntax
    f = syntax.parse("function f(y, a, b)\n    y[1] = a +\n        b\nend\n")[0]
    assert f.body[0].rhs == Bin("+", Var("a"), Var("b"))


def test_types_from_use():
    from stade_hip.lower import analysis, syntax
    f = syntax.parse((GENERIC / "binsum_b.jl").read_text())[1]
    T = analysis.infer_types(f)
    assert T.arrays["bins"] == "i" and T.arrays["v"] == "f" and T.arrays["cb"] == "f"
    assert T.scalars["__icse_0"] == "i" and T.scalars["i_n"] == "i"
    f = syntax.parse((CORPUS / "mlp2_ce_b.jl").read_text())[1]
    T = analysis.infer_types(f)
    assert T.arrays["lab"] == "i"          # i_l = lab[s] lands in an index
    assert T.scalars["se"] == "f" and T.scalars["i_l"] == "i"


def _poly(text, env_text=()):
    from stade_hip.lower import analysis, syntax
    body = "\n".join(f"    {l}" for l in env_text)
    f = syntax.parse(f"function f(y, idx, n, m)\n{body}\n    y[{text}] = 1.0\nend\n")[0]
    T = analysis.infer_types(f)
    for v in ("idx", "n", "m"):
        T.scalars[v] = "i"
    env = {s.lhs.name: s.rhs for s in f.body[:-1]}
    return analysis.to_poly(f.body[-1].lhs.idx[0], env, T), T


def test_divmod_fold_makes_the_flattened_index_injective():
    from stade_hip.lower import analysis
    p, _ = _poly("(i_s - 1) * n + i_j", ["i_s = div(idx - 1, n) + 1", "i_j = mod(idx - 1, n) + 1"])
    p, conds = analysis.fold_divmod(p)
    coef, rest = analysis.linear_in(p, "idx")
    assert coef == {(): 1} and rest == {}
    assert len(conds) == 1        # assumed: idx - 1 >= 0 and n > 0 (checked by the kernel)


def test_a_shared_index_is_not_injective():
    from stade_hip.lower import analysis
    p, _ = _poly("mod(idx - 1, n) + 1")
    p, _ = analysis.fold_divmod(p)
    assert analysis.linear_in(p, "idx") is None
    p, _ = _poly("div(idx - 1, n) + 1")
    assert analysis.linear_in(analysis.fold_divmod(p)[0], "idx") is None


PLANS = {
    # (text, function): (loop variable, array, kind) that the plan must contain
    # (the periodic scatter into ub taken as an owner-computes gather, the unb reset deferred;
    # the forward, loss and seed loops over the same cells fused into one)
    ("diffusion2d_b", "diffusion2d_b"): [("idx", "un", "owned"), ("idx", "ub", "owned"), ("idx", "unb", "read"),
                                         ("idx", "unb", "owned"), ("idx", "loss", "atomic")],
    # (the dense layers' sums and scatters as matrix products around the loops: contract.py)
    ("mlp2_ce_b", "mlp2_ce_b"): [("idx", "h1", "owned"), ("idx", "b1b", "atomic"), ("gemm", "w1b", "added"),
                                 ("gemm", "xb", "added"), ("gemm", "h1b", "added")],
    ("conv3x3_b", "conv3x3_b"): [("idx", "out", "owned"), ("gemm", "wb", "added atomically"),
                                 ("gemm", "xpb", "added atomically")],
    ("generic/binsum_b", "binsum_b"): [("i", "c", "atomic"), ("i", "vb", "owned")],
    ("generic/window1d_b", "window1d_b"): [("i", "wb", "atomic"), ("i", "inpb", "atomic"), ("i", "outb", "owned")],
    ("generic/matvec_scatter_b", "matvec_scatter_b"): [("idx", "y", "atomic"), ("idx", "ab", "owned"), ("idx", "xb", "atomic")],
}


@pytest.mark.parametrize("key", sorted(PLANS))
def test_plans(key):
    from stade_hip.lower import hipgen
    text, fname = key
    prec = "f32" if text.startswith(("mlp", "conv")) else "f64"
    _, sigs = hipgen.generate((CORPUS / f"{text}.jl").read_text(), prec)
    plan = " | ".join(sigs[fname]["plan"])
    for var, arr, kind in PLANS[key]:
        if var == "gemm":
            assert re.search(rf"matrix product into {arr} \({kind}", plan), (arr, kind, plan)
            continue
        assert re.search(rf"parallel over {var} \[[^\]]*\b{arr}:{kind}\b", plan), (var, arr, kind, plan)
    assert "loops in order" not in plan, plan       # every loop runs one iteration per thread


def test_burgers_time_loop_stays_on_the_host_with_a_device_guard():
    from stade_hip.lower import hipgen
    _, sigs = hipgen.generate((CORPUS / "burgers1d_b.jl").read_text())
    plan = sigs["burgers1d_b"]["plan"]
    assert plan.count("host loop over i_t") == 2 and "  device if" in plan
    assert sigs["burgers1d_b"]["args"][-2] == ("branch_stack", "Ai", 1)


@pytest.mark.parametrize("name, replayed", [("burgers1d_b", True), ("burgers1d_d", True), ("diffusion2d_b", False)])
def test_host_loops_replay_as_graphs(name, replayed):
    """A function with host loops runs its launch sequence through the graph cache (replayed
    when a frame repeats); one without issues its launches directly.  Either way the sequence
    sits in one function of the frame alone, and a reallocated local array drops the graphs."""
    from stade_hip.lower import hipgen
    src, _ = hipgen.generate((CORPUS / f"{name}.jl").read_text())
    body = src[src.index(f"extern \"C\" int32_t stade_hip_gen_{name}("):]
    body = body[:body.index("\n}\n")]
    assert ("g_graphs.run(a, stream, _launches)" in body) == replayed
    assert ("_launches(a, stream);" in body) == (not replayed)
    assert "<<<" not in body                     # every launch is in _launches
    assert "std::memset(&a, 0, sizeof a)" in body
    assert "g_graphs.clear();" in src


def test_block_sums_fold_and_commit():
    """The Burgers reverse loop sums into two scalars and leaves `ucb`'s last value: its blocks
    store their sums in slots (no atomic when the grid is large), and the one-block fold kernel
    adds them and also commits the last value, so that the one-thread commit kernel runs only
    when the fold does not."""
    from stade_hip.lower import hipgen
    src, _ = hipgen.generate((CORPUS / "burgers1d_b.jl").read_text())
    fold = src[src.index("void k12f("):]
    fold = fold[:fold.index("\n}\n")]
    assert "fold_load(g_p12_0" in fold and "fold_load(g_p12_1" in fold
    assert "fr.v_ucb = wb.v_ucb;" in fold
    assert fold.index("fr.v_ucb = wb.v_ucb;") < fold.index("return;\n    double _v0")  # before the guard's return
    assert "if (_g > 256) {" in src and "_cm12 = true;" in src and "if (!_cm12) {" in src
    k12 = src[src.index("void k12(const Args a)"):]
    k12 = k12[:k12.index("\n}\n")]
    assert "if (gridDim.x <= 256) {" in k12 and "block_part(g_p12_0" in k12


def test_initstacks_on_the_host_matches_the_oracle():
    from stade_hip.lower import initstacks
    from oracle import runner
    text = (CORPUS / "burgers1d_b.jl").read_text()
    lib = runner.load(CORPUS / "burgers1d_b.jl")
    for n, T in ((7, 3), (100, 0), (1, 9)):
        got = initstacks(text, "initstacks_burgers1d_b", n, T)
        want = lib.stacks("initstacks_burgers1d_b", n, T)
        assert [g[2] for g in got] == [len(w) for w in want]
        assert [g[1] for g in got] == ["Int64", "Float64"]


def test_built_libraries_export_their_entry_points():
    from stade_hip import lower
    for path in sorted(GENERIC.glob("*_*.jl")):
        lib = lower.lower(path, "f64")
        out = subprocess.run(["nm", "-D", "--defined-only", str(lib.path)], capture_output=True, text=True, check=True).stdout
        for fname in lib.sigs:
            assert f"stade_hip_gen_{fname}" in out, (path.name, fname)


def test_cpu_tensors_are_refused():
    import torch
    from stade_hip import lower
    lib = lower.lower(GENERIC / "binsum_b.jl", "f64")
    z = torch.zeros(3, dtype=torch.float64)
    with pytest.raises(ValueError, match="no CPU path"):
        lib.call("binsum_b", z[:1], z[:1], z, z, torch.ones(3, dtype=torch.int64), z, z, 3, 3)


@pytest.mark.skipif(not REF_CORPUS.exists(), reason="reference corpus not mounted")
def test_reference_corpus_breadth():
    """Every generated file of the reference's corpus (/root/reference/test/val-corpus) goes
    through the lowering's front end and planner; the count that lowers, and the causes of the
    refusals, are printed (HIP is generated but not compiled here: that is the test above)."""
    from stade_hip.lower import hipgen, LowerError
    files = sorted(p for p in REF_CORPUS.glob("*_*.jl") if re.search(r"_(b|d|hv)\.jl$", p.name))
    ok, causes = 0, {}
    for p in files:
        try:
            hipgen.generate(p.read_text())
            ok += 1
        except LowerError as e:
            c = re.sub(r"^[\w!]+: ", "", str(e)).split(" (")[0]
            causes[c] = causes.get(c, 0) + 1
    print(f"lowered {ok} of {len(files)} reference generated files; refusals: {causes}")
    assert ok >= 0.8 * len(files)


@pytest.mark.skipif(not REF_CORPUS.exists(), reason="reference corpus not mounted")
@pytest.mark.parametrize("name", ["transformer_b", "unet_hv", "advection_b"])
def test_reference_kernels_compile(name, tmp_path):
    """Three of the reference's generated kernels (attention with softmax, a U-Net HVP, an
    explicit time loop with an indexed tape) lower and compile for gfx950."""
    from stade_hip.lower import hipgen, runtime
    src, sigs = hipgen.generate((REF_CORPUS / f"{name}.jl").read_text())
    h = tmp_path / f"{name}.hip"
    h.write_text(src)
    r = subprocess.run([runtime.HIPCC, *runtime.FLAGS, "-o", str(h.with_suffix(".so")), str(h)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    assert name in sigs


GENERIC_CASES = {
    "matvec_scatter": (dict(i_m=5, i_n=4), dict(loss=1, a=20, x=4, y=5), {}),
    "flatmv": (dict(i_m=5, i_n=4), dict(loss=1, a=20, x=4, y=5), {}),
    "window1d": (dict(i_n=11, i_k=4), dict(loss=1, inp=11, w=4, out=8), {}),
    "binsum": (dict(i_n=13, i_b=4), dict(loss=1, v=13, c=4),
               dict(bins=np.array([1, 2, 3, 4, 1, 2, 3, 4, 2, 2, 3, 1, 4], dtype=np.int64))),
}


@pytest.mark.parametrize("name", sorted(GENERIC_CASES))
def test_generic_texts_pinned(name):
    """The derivative texts of corpus/generic (written by hand in STADE's generated form) by
    the reference's own oracles: the exact dot-product identity between tangent and adjoint
    (<= 1e-11, `val_validate_dotprod` /root/reference/src/STADE.jl:17108-17131), central
    differences of the adjoint and tangent (<= 1e-3, 16334-16351) and of the gradient for the
    HVP (17133-17153)."""
    from oracle import checks, runner, rng as jrng
    ints, shapes, ia = GENERIC_CASES[name]
    ld, lb, lh = (runner.load(GENERIC / f"{name}_{m}.jl") for m in ("d", "b", "hv"))
    k = checks.kernel_from_lib(ld, name, ints, shapes, int_arrays=ia)
    base = checks.random_values(k, jrng.Xoshiro(jrng.val_stable_seed(name)), base=True)
    s = jrng.val_stable_seed(name) + 1
    assert checks.dotprod(ld, lb, k, base, s) <= 1e-11
    assert checks.fd_adjoint(ld, lb, k, base, s) <= 1e-3
    assert checks.fd_tangent(ld, ld, k, base, s) <= 1e-3
    assert checks.fd_hvp(lb, lh, k, base, s) <= 1e-3


@pytest.mark.skipif(not REF_CORPUS.exists(), reason="reference corpus not mounted")
def test_ref_corpus_fixture_inputs_reproduce():
    """tests/test_gpu_ref_corpus.py draws its inputs again from the fixtures' seeds
    (helpers.seeded_inputs); they must be the inputs the fixtures' oracle run used
    (helpers.make_args on the generated text), and the stored oracle outputs must be what the
    oracle computes from them now."""
    import json
    from helpers import ParityCase, make_args, seeded_inputs
    from oracle import runner
    gold = Path(__file__).resolve().parent / "golden"
    meta = json.loads((gold / "ref_corpus.json").read_text())
    z = np.load(gold / "ref_corpus.npz")
    # every seventh case, and every case drawn at scaled inputs
    for case in [c for k, c in enumerate(meta) if k % 7 == 0 or c.get("scales")]:
        lib_o = runner.load(REF_CORPUS / f"{case['fname']}.jl")
        ia = {a: z[f"{case['key']}/in/{a}"] for a, kind, _, _ in case["args"] if kind == "Ai"}
        got = seeded_inputs(case["args"], case["ints"], case["seed"], ia, zeros=case.get("zeros", ()),
                            scales=case.get("scales"))
        shapes = {a: tuple(s) for a, kind, s, _ in case["args"] if kind == "Af"}
        shapes["__stacks__"] = tuple(s for s, _, _ in case["stacks"])
        want = make_args(lib_o, case["fname"], shapes, case["ints"], {}, case["seed"], np.float64, ia,
                         case.get("scales"))
        # the stacks initstacks returns are zero-filled
        want = [(a, k, np.zeros_like(v, order="F") if a in case.get("zeros", ()) else v) for a, k, v in want]
        assert [a for a, _, _ in got] == [a for a, _, _ in want]
        for (a, _, g), (_, _, w) in zip(got, want):
            assert np.array_equal(np.asarray(g), np.asarray(w)), f"{case['key']}: input {a} differs"
        pc = ParityCase(case["name"], case["mode"], want, [(s, (n, k)) for s, n, k in case["stacks"]], "f64").run_oracle(lib_o)
        for (a, _, v), h in zip(want, pc.host):
            k = f"{case['key']}/out/{a}"
            if k in z:
                assert np.array_equal(np.ravel(h, order="F"), z[k]), f"{case['key']}: oracle output {a} differs"


@pytest.mark.skipif(not REF_CORPUS.exists() or os.environ.get("STADE_FULL_CORPUS") != "1",
                    reason="compiles all 417 reference files (about 20 minutes on 8 cores): STADE_FULL_CORPUS=1")
def test_reference_corpus_compiles(tmp_path):
    """Every generated file of the reference's corpus lowers and compiles for gfx950."""
    import concurrent.futures as cf
    from stade_hip.lower import hipgen, runtime
    files = sorted(p for p in REF_CORPUS.glob("*_*.jl") if re.search(r"_(b|d|hv)\.jl$", p.name))

    def one(p):
        src, _ = hipgen.generate(p.read_text())
        h = tmp_path / f"{p.stem}.hip"
        h.write_text(src)
        r = subprocess.run([runtime.HIPCC, *runtime.FLAGS, "-o", str(h.with_suffix(".so")), str(h)],
                           capture_output=True, text=True)
        return None if r.returncode == 0 else (p.name, r.stderr[-300:])
    with cf.ThreadPoolExecutor(8) as ex:
        bad = [r for r in ex.map(one, files) if r]
    assert len(files) >= 400 and not bad, bad


@pytest.mark.skipif(not REF_CORPUS.exists(), reason="reference corpus not mounted")
@pytest.mark.parametrize("name, args", [
    ("advection", dict(i_nnode=8, i_nstep=3)),
    ("coarsen_retire", dict(levels=4, n=9)),
    ("windowed_relax_retire", dict(dx=0.25, num_passes=5, w0=6)),
    ("cascadic_mg_prolong", dict(h_coarse=0.5, nu=3, num_levels=4)),
])
def test_run_initstacks_matches_the_oracle(name, args):
    """lower.run_initstacks (initstacks_* run on the host with loops, branches, prefix index
    arrays and Int64 counts) against the same function transpiled by the oracle: every
    returned array's length and every returned count."""
    from oracle import runner
    from stade_hip import lower
    path = REF_CORPUS / f"{name}_b.jl"
    fn = f"initstacks_{name}_b"
    got = lower.run_initstacks(path.read_text(), fn, args)
    lib = runner.load(path)
    want = lib.call(fn, *(args[a] for a, _ in lib.infos[fn].args))
    assert len(got) == len(want) and len(got) > 0
    for (nm, v), w in zip(got, want):
        if isinstance(w, tuple):
            assert isinstance(v, np.ndarray) and v.size == w[0], (nm, v, w)
            assert (v.dtype == np.int64) == (w[1] == "Ai"), (nm, v.dtype, w)
        else:
            assert v == w, (nm, v, w)


def _gathered(text: str, fname: str) -> int:
    from stade_hip.lower import gather
    from stade_hip.lower.syntax import parse
    f = next(g for g in parse(text) if g.name == fname)
    n = [0]
    gather.transform(f.body, n)
    return n[0]


def test_periodic_scatter_becomes_a_gather():
    """The Burgers reverse loop's neighbour scatters into ub (periodic shifts of i_x) run as
    an owner-computes gather, its unb reset deferred to a loop of its own."""
    from stade_hip.lower import hipgen
    _, sigs = hipgen.generate((CORPUS / "burgers1d_b.jl").read_text())
    plan = " | ".join(sigs["burgers1d_b"]["plan"])
    assert re.search(r"parallel over i_x \[u:read, ub:owned, unb:read\] sums", plan), plan
    assert re.search(r"parallel over i_x \[unb:owned\]", plan), plan
    assert "ub:atomic" not in plan.split("host loop over i_t")[2], plan


def test_gathered_terms_merge_into_one_update():
    """The owner's four replayed neighbour terms and its own term add into ub[i_x]: merged
    into one update per iteration (four merges), one load and one store of the element."""
    from stade_hip.lower import hipgen
    src, sigs = hipgen.generate((CORPUS / "burgers1d_b.jl").read_text())
    assert sigs["burgers1d_b"]["finish"]["merged_gathered"] == 4
    fl = hipgen.lower_function((CORPUS / "burgers1d_b.jl").read_text(), "burgers1d_b")
    from stade_hip.lower.syntax import Assign, For, Ref, walk_stmts
    loops = [s for s in walk_stmts(fl.f.body) if isinstance(s, For) and s.var == "i_x"]
    rev = [L for L in loops if any(isinstance(t, Assign) and isinstance(t.lhs, Ref) and t.lhs.name == "ub"
                                   for t in L.body)]
    assert rev and all(sum(1 for t in L.body if isinstance(t, Assign) and isinstance(t.lhs, Ref) and t.lhs.name == "ub")
                       == 1 for L in rev), rev


_SCATTER = """function s_b(x, xb, y, yb, n)
    for i = 1:n
        ip = mod(i, n) + 1
        old = yb[i]
        yb[i] = 0.0
        xb[ip] = xb[ip] + WHAT
    end
    return nothing
end
"""


@pytest.mark.parametrize("what, expect", [
    ("2.0 * old", 1),                 # a periodic shift: rewritten
    ("old * x[ip]", 1),               # reads an array the loop never writes
    ("old * yb[ip]", 0),              # reads the array the loop resets, at a neighbour
])
def test_gather_only_where_exact(what, expect):
    assert _gathered(_SCATTER.replace("WHAT", what), "s_b") == expect


def test_no_gather_for_a_value_carried_from_the_previous_iteration():
    """c is assigned after the scatter that reads it, so the scatter adds the previous
    iteration's x (xb[t] gets x[t - 2]); a gather that recomputed c from the source iteration
    would add x[t - 1] instead.  The loop must be left as it is (and then runs in order)."""
    text = """function s_b(x, xb, n)
    c = 0.0
    for i = 1:n
        ip = mod(i, n) + 1
        xb[ip] = xb[ip] + c
        c = x[i]
    end
    return nothing
end
"""
    assert _gathered(text, "s_b") == 0
    # and with the carried value read by a statement of the value's slice
    text2 = text.replace("xb[ip] = xb[ip] + c", "d = 2.0 * c\n        xb[ip] = xb[ip] + d")
    assert _gathered(text2, "s_b") == 0


def test_no_gather_for_a_map_that_is_not_a_bijection():
    text = _SCATTER.replace("ip = mod(i, n) + 1", "ip = mod(i, 2) + 1").replace("WHAT", "old")
    assert _gathered(text, "s_b") == 0
    # a shift whose extent is not the loop's
    text = _SCATTER.replace("ip = mod(i, n) + 1", "ip = mod(i, n - 1) + 1").replace("WHAT", "old")
    assert _gathered(text, "s_b") == 0


def test_adjacent_loops_over_the_same_cells_fuse():
    """The diffusion adjoint's forward loop, loss loop (k = 1:n*n) and seed loop
    (k = n*n:-1:1) become one parallel loop: un written and read at the iteration's own index."""
    from stade_hip.lower import hipgen
    _, sigs = hipgen.generate((CORPUS / "diffusion2d_b.jl").read_text())
    par = [p for p in sigs["diffusion2d_b"]["plan"] if p.startswith("parallel")]
    assert len(par) == 3, par
    assert par[0].startswith("parallel over idx [loss:atomic, lossb:read, u:read, un:owned, unb:owned]"), par


_FUSE = """function f_b(x, y, z, s, n)
    for i = 1:n
        y[i] = 2.0 * x[i]
    end
    for k = n:-1:1
        BODY
    end
    return nothing
end
"""


@pytest.mark.parametrize("body, fused", [
    ("z[k] = y[k] + 1.0", True),             # reads what the first loop wrote, at its own index
    ("z[k] = y[mod(k, n) + 1]", False),       # reads another iteration's value
    ("s[1] = s[1] + y[k]", True),             # a sum of own-index values
])
def test_fusion_only_where_iterations_stay_independent(body, fused):
    from stade_hip.lower import hipgen
    _, sigs = hipgen.generate(_FUSE.replace("BODY", body))
    par = [p for p in sigs["f_b"]["plan"] if p.startswith("parallel")]
    assert (len(par) == 1) == fused, par



@pytest.mark.parametrize("mode, twins", [
    ("b", [("idx", "row", ["y"]), ("idx", "col", ["xb"])]),
    ("d", [("idx", "row", ["y", "yd"])]),
    ("hv", [("idx", "row", ["y", "yd"]), ("idx", "col", ["xb", "xbd"])]),
])
def test_flat_loops_get_their_twins(mode, twins):
    """The row-major flat mat-vec: the forward loop's y[i] (a row sum) takes the row-block twin,
    the adjoint loop's xb[j] (a column sum) the column-block twin (`cgen_rowblock_kernel`
    /root/reference/src/STADE.jl:18187, `cgen_colblock_kernel` 18371)."""
    from stade_hip.lower import hipgen
    _, sigs = hipgen.generate((GENERIC / f"flatmv_{mode}.jl").read_text())
    assert [tuple(t) for t in sigs[f"flatmv_{mode}"]["twins"]] == twins


@pytest.mark.parametrize("change", [
    "y[i] = y[i] + a[idx] * x[j]\n        y[j] = y[j] + 1.0",   # a second site at the column: mixed
    "y[i] = y[i] + a[idx] * x[j]\n        a[idx] = y[i]",       # the site is read in the loop
    "y[j + 1 - 1 + i - i] = y[j + 1 - 1 + i - i] + a[idx]",      # the index reads the column
])
def test_no_twin_unless_the_sites_agree(change):
    from stade_hip.lower import hipgen
    text = (GENERIC / "flatmv.jl").read_text().replace("y[i] = y[i] + a[idx] * x[j]", change)
    _, sigs = hipgen.generate(text)
    assert sigs["flatmv"]["twins"] == []


@pytest.mark.parametrize("name,expect", [("affine_lsq_b", ["i_i"]), ("affine_lsq_hv", ["i_i"]), ("affine_lsq_d", []),
                                         ("generic/window1d_b", []), ("generic/matvec_scatter_b", [])])
def test_lanes_over_rows_for_column_major_updates(name, expect):
    """The lanes-over-iterations form is chosen for a shared inner loop whose accumulations
    step along the outer loop with stride 1 and along their own index with a larger stride (the
    affine adjoint's wb[i, j]), not for loops that only read along the outer loop (the affine
    tangent's row sums) nor for updates along their own index (a window's taps)."""
    from stade_hip.lower import hipgen
    _, sigs = hipgen.generate((CORPUS / f"{name}.jl").read_text(), "f64")
    assert sigs[name.split("/")[-1]]["xsplit"] == expect
