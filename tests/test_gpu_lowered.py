"""The general lowering (stade_hip.lower) on the GPU against the oracle.

Every case lowers a generated text to HIP, runs the built library on the GPU through its C
entry point, and compares every output argument, stack and returned scalar with the oracle
(the same text transpiled to sequential C) on the same seeded inputs, to the parity bars
(fp64 1e-12, fp32 1e-5, integers exact) with the truth rule where a sum's order decides.

Texts: the three kernels of stade.jl_amd/corpus/generic (a flattened mat-vec with scatters
in the primal and the adjoint, an overlapping-window correlation, a binned sum over Int64
labels), and the five benchmark configs' own texts taken through the general path instead of
their hand-written kernels.  Sizes include ones whose accumulation targets are small enough,
with enough iterations, for the LDS-privatised atomics (binsum's bins, window1d's taps), and
ragged and empty ones."""
import numpy as np
import pytest

from helpers import CORPUS, ParityCase, make_args

pytestmark = pytest.mark.gpu

GENERIC = CORPUS / "generic"
FP32 = {"mlp2_ce", "conv3x3"}


def _lowered(path, precision):
    from stade_hip import lower
    return lower.lower(path, precision)


def _case(path, name, mode, shapes, ints, scalars=None, int_arrays=None, stacks=(), precision="f64", scales=None,
          label=None):
    from oracle import runner
    import torch
    lib_o = runner.load(path, precision=precision)
    fname = f"{name}_{mode}"
    shp = dict(shapes)
    shp["__stacks__"] = tuple(s for s, _ in stacks)
    fdt = np.float32 if precision == "f32" else np.float64
    args = make_args(lib_o, fname, shp, ints, scalars or {}, f"lowered-{fname}-{ints}", fdt, int_arrays, scales)
    low = _lowered(path, precision)
    dims = {a: v.shape for a, _, v in args if isinstance(v, np.ndarray) and v.ndim > 1}

    def run(dev, stack_d):
        return low.call(fname, *dev, *stack_d, shapes=dims)
    case = ParityCase(name, mode, args, stacks, precision, label=label or f"lowered {fname} {ints}", runner=run,
                      oracle_path=path)
    case.run_oracle(lib_o)
    return case, low


def _check(case, low, fname):
    print(f"{case.label}: plan {low.plan(fname)}", flush=True)
    case.run_gpu()
    print(f"{case.label}: worst {case.compare():.3e}", flush=True)


# ---- the three generic kernels ---------------------------------------------------------

@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("mn", [(1, 1), (5, 4), (300, 70), (2000, 513), (0, 3)])
def test_lowered_matvec_scatter(mode, mn):
    m, n = mn
    shapes = {k + s: v for k, v in dict(loss=1, a=m * n, x=n, y=m).items() for s in ("", "b", "d", "bd")}
    case, low = _case(GENERIC / f"matvec_scatter_{mode}.jl", "matvec_scatter", mode, shapes, dict(i_m=m, i_n=n))
    _check(case, low, f"matvec_scatter_{mode}")


@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("nk", [(1, 1), (9, 4), (1000, 7), (50000, 7), (3, 5)])
def test_lowered_window1d(mode, nk):
    n, k = nk
    nout = max(0, n - k + 1)
    shapes = {a + s: v for a, v in dict(loss=1, inp=n, w=k, out=nout).items() for s in ("", "b", "d", "bd")}
    case, low = _case(GENERIC / f"window1d_{mode}.jl", "window1d", mode, shapes, dict(i_n=n, i_k=k))
    _check(case, low, f"window1d_{mode}")


@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("nb", [(1, 1), (13, 4), (100000, 16), (20000, 3000), (0, 5)])
def test_lowered_binsum(mode, nb):
    from oracle import rng as jrng
    n, b = nb
    shapes = {a + s: v for a, v in dict(loss=1, v=n, c=b).items() for s in ("", "b", "d", "bd")}
    g = jrng.Xoshiro(41 + n)
    bins = np.array([1 + int(g.rand() * b) for _ in range(n)], dtype=np.int64)
    case, low = _case(GENERIC / f"binsum_{mode}.jl", "binsum", mode, shapes, dict(i_n=n, i_b=b), int_arrays=dict(bins=bins))
    _check(case, low, f"binsum_{mode}")


# ---- the benchmark configs' texts through the general path ------------------------------

@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("n", [1, 2, 3, 64, 257])
def test_lowered_diffusion2d(mode, n):
    shapes = {k: n * n for k in ("u", "ub", "un", "unb", "ud", "ubd", "und", "unbd")}
    shapes.update({k: 1 for k in ("loss", "lossb", "lossd", "lossbd")})
    case, low = _case(CORPUS / f"diffusion2d_{mode}.jl", "diffusion2d", mode, shapes, dict(n=n))
    _check(case, low, f"diffusion2d_{mode}")


@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("mn", [(1, 1), (65, 33), (256, 300)])
def test_lowered_affine_lsq(mode, mn):
    m, n = mn
    shapes = {k: (m, n) for k in ("w", "wb", "wd", "wbd")}
    shapes.update({k: n for k in ("x", "xb", "xd", "xbd")})
    shapes.update({k: m for k in ("b", "bb", "bd", "bbd", "t", "tb", "td", "tbd", "r", "rb", "rd", "rbd")})
    shapes.update({k: 1 for k in ("loss", "lossb", "lossd", "lossbd")})
    case, low = _case(CORPUS / f"affine_lsq_{mode}.jl", "affine_lsq", mode, shapes, dict(i_m=m, i_n=n))
    _check(case, low, f"affine_lsq_{mode}")


@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("case_", [(7, 6, 0.007), (100, 12, 10.0), (4097, 9, 10.0), (5, 0, 10.0), (2, 4, 10.0)])
def test_lowered_burgers1d(mode, case_):
    n, T, tend = case_
    shapes = {k: n for k in ("u", "ub", "un", "unb", "ud", "ubd", "und", "unbd")}
    shapes.update({k: 1 for k in ("loss", "lossb", "lossd", "lossbd")})
    scalars = dict(nu=0.05, dt=0.002, dx=0.5, tend=tend, nud=0.3, dtd=-0.2, dxd=0.1, tendd=0.7)
    stacks = () if mode == "d" else (("branch_stack", (T, "Ai")), ("u_stack", (T * n, "Af")))
    case, low = _case(CORPUS / f"burgers1d_{mode}.jl", "burgers1d", mode, shapes, dict(n=n, nsteps=T), scalars=scalars,
                      stacks=stacks)
    _check(case, low, f"burgers1d_{mode}")


@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("case_", [(300, 40, 10.0), (97, 25, 0.02)])
def test_lowered_graph_replay(mode, case_):
    """A function with a host time loop, called again with the same frame, replays its launch
    sequence as a captured HIP graph: three calls on the same device arrays (the inputs copied
    in before each), each against the oracle; the second call captures, the second and third
    launch the graph.  (0.02 stops the time loop early: the guard's branch flag.)"""
    import torch
    n, T, tend = case_
    shapes = {k: n for k in ("u", "ub", "un", "unb", "ud", "ubd", "und", "unbd")}
    shapes.update({k: 1 for k in ("loss", "lossb", "lossd", "lossbd")})
    scalars = dict(nu=0.05, dt=0.002, dx=0.5, tend=tend, nud=0.3, dtd=-0.2, dxd=0.1, tendd=0.7)
    stacks = () if mode == "d" else (("branch_stack", (T, "Ai")), ("u_stack", (T * n, "Af")))
    fname = f"burgers1d_{mode}"
    case, low = _case(CORPUS / f"{fname}.jl", "burgers1d", mode, shapes, dict(n=n, nsteps=T), scalars=scalars,
                      stacks=stacks, label=f"lowered {fname} graph replay {case_}")
    fixed = {}

    def run(dev, stack_d):
        # the same arrays every call: this call's inputs copied in, the outputs copied back
        if not fixed:
            fixed["a"] = [v.clone() if isinstance(v, torch.Tensor) else v for v in dev]
            fixed["s"] = [v.clone() for v in stack_d]
        for p, v in zip(fixed["a"] + fixed["s"], list(dev) + list(stack_d)):
            if isinstance(v, torch.Tensor):
                p.copy_(v)
        ret = low.call(fname, *fixed["a"], *fixed["s"], shapes={})
        for p, v in zip(fixed["a"] + fixed["s"], list(dev) + list(stack_d)):
            if isinstance(v, torch.Tensor):
                v.copy_(p)
        return ret
    case.runner = run
    c0 = low.graphs(fname)
    for _ in range(3):
        _check(case, low, fname)
    c1 = low.graphs(fname)
    print(f"{case.label}: graphs captured {c1[0] - c0[0]}, launched {c1[1] - c0[1]}", flush=True)
    assert (c1[0] - c0[0], c1[1] - c0[1]) == (1, 2), (c0, c1)


@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("size", [(8, 5, 7, 3), (33, 17, 40, 10)])
def test_lowered_mlp2_ce(mode, size):
    from oracle import rng as jrng
    B, I, H, O = size
    sz = dict(loss=1, x=I * B, w1=H * I, b1=H, w2=O * H, b2=O, h1=H * B, z=O * B)
    shapes = {k + s: v for k, v in sz.items() for s in ("", "b", "d", "bd")}
    lab = np.array([1 + int(jrng.Xoshiro(17 + s).rand() * O) for s in range(B)], dtype=np.int64)
    g1, g2 = np.sqrt(2.0 / (I + H)), np.sqrt(2.0 / (H + O))
    scales = {"w1": g1, "w1d": g1, "w2": g2, "w2d": g2, "b1": 0.1, "b2": 0.1}
    case, low = _case(CORPUS / f"mlp2_ce_{mode}.jl", "mlp2_ce", mode, shapes, dict(i_b=B, i_in=I, i_h=H, i_out=O),
                      int_arrays=dict(lab=lab), precision="f32", scales=scales)
    _check(case, low, f"mlp2_ce_{mode}")


@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("size", [(1, 1, 1, 1, 1), (2, 3, 5, 7, 9)])
def test_lowered_conv3x3(mode, size):
    N, C, K, H, W = size
    sz = dict(loss=1, xp=(W + 2) * (H + 2) * C * N, w=9 * C * K, out=W * H * K * N)
    shapes = {k + s: v for k, v in sz.items() for s in ("", "b", "d", "bd")}
    s = 1.0 / np.sqrt(9.0 * C)
    case, low = _case(CORPUS / f"conv3x3_{mode}.jl", "conv3x3", mode, shapes, dict(i_nb=N, i_c=C, i_k=K, i_h=H, i_w=W),
                      precision="f32", scales={"w": s, "wd": s})
    _check(case, low, f"conv3x3_{mode}")


# ---- narrow outputs: few iterations with long inner loops (a wave per iteration) ---------

@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("nk", [(20000, 19990), (60000, 59000), (3000, 2700)])
def test_lowered_window1d_narrow(mode, nk):
    """11, 1001 and 301 outputs of 19990-, 59000- and 2700-tap correlations: the lanes of a wave
    share each output's tap loop (the sum's order changes, within the fp64 bar)."""
    n, k = nk
    nout = n - k + 1
    shapes = {a + s: v for a, v in dict(loss=1, inp=n, w=k, out=nout).items() for s in ("", "b", "d", "bd")}
    case, low = _case(GENERIC / f"window1d_{mode}.jl", "window1d", mode, shapes, dict(i_n=n, i_k=k))
    _check(case, low, f"window1d_{mode}")


@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("mn", [(4, 200000), (16, 50000), (100, 5000)])
def test_lowered_affine_lsq_narrow(mode, mn):
    """Few rows and long rows: the row sums, and the adjoint's row loop with its accumulations
    into wb and xb, shared by the lanes of a wave."""
    m, n = mn
    shapes = {k: (m, n) for k in ("w", "wb", "wd", "wbd")}
    shapes.update({k: n for k in ("x", "xb", "xd", "xbd")})
    shapes.update({k: m for k in ("b", "bb", "bd", "bbd", "t", "tb", "td", "tbd", "r", "rb", "rd", "rbd")})
    shapes.update({k: 1 for k in ("loss", "lossb", "lossd", "lossbd")})
    case, low = _case(CORPUS / f"affine_lsq_{mode}.jl", "affine_lsq", mode, shapes, dict(i_m=m, i_n=n))
    _check(case, low, f"affine_lsq_{mode}")


# ---- which accumulation path ran: the kernels' path counters -------------------------------

def _paths(case, low, fname):
    """Run a case (checked against the oracle as above) with the lowered function's path
    counters on; returns them by name (`LoweredLib.set_stats`)."""
    import torch
    st = torch.zeros(8, dtype=torch.int64, device="cuda")
    low.set_stats(fname, st)
    try:
        _check(case, low, fname)
    finally:
        low.set_stats(fname, None)
    c = st.cpu().tolist()
    print(f"{case.label}: paths agg={c[0]} lane={c[1]} priv={c[2]} split={c[3]} block={c[4]} row={c[5]} col={c[6]}"
          f" xsplit={c[7]}", flush=True)
    return dict(agg=c[0], lane=c[1], priv=c[2], split=c[3], block=c[4], row=c[5], col=c[6], xsplit=c[7])


def _matvec_b(m, n):
    shapes = {k + s: v for k, v in dict(loss=1, a=m * n, x=n, y=m).items() for s in ("", "b", "d", "bd")}
    return _case(GENERIC / "matvec_scatter_b.jl", "matvec_scatter", "b", shapes, dict(i_m=m, i_n=n),
                 label=f"paths matvec_scatter_b m={m} n={n}")


def _binsum_b(n, b):
    from oracle import rng as jrng
    shapes = {a + s: v for a, v in dict(loss=1, v=n, c=b).items() for s in ("", "b", "d", "bd")}
    g = jrng.Xoshiro(41 + n)
    bins = np.array([1 + int(g.rand() * b) for _ in range(n)], dtype=np.int64)
    return _case(GENERIC / "binsum_b.jl", "binsum", "b", shapes, dict(i_n=n, i_b=b), int_arrays=dict(bins=bins),
                 label=f"paths binsum_b n={n} bins={b}")


def test_paths_every_lane_shares_the_target():
    """xb[j] at j = div(idx - 1, 128) + 1: the 64 lanes of every wave add into one element, and
    xb (8192 doubles, 64 KiB) is too large for the LDS copy, so every wave of the adjoint loop
    takes the aggregated branch: exactly 128 * 8192 / 64 single atomics, none per lane.  The
    forward loop's y (128 doubles, 8192 iterations per element) takes the LDS-privatised
    variant, and the loss sum one block total per block."""
    case, low = _matvec_b(128, 8192)
    p = _paths(case, low, "matvec_scatter_b")
    assert p["agg"] == 128 * 8192 // 64 and p["lane"] == 0
    assert p["priv"] > 0 and p["block"] > 0


def test_paths_no_lane_shares_the_target():
    """One row: every lane of a wave adds into its own xb[j] (70000 doubles, beyond the LDS
    copy), so the wave-aggregated branch never fires and every wave of the adjoint loop adds
    per lane (1093 full waves and a partial one).  The forward loop's y has one element and
    70000 iterations: its LDS-privatised variant runs."""
    case, low = _matvec_b(1, 70000)
    p = _paths(case, low, "matvec_scatter_b")
    assert p["agg"] == 0 and p["lane"] == -(-70000 // 64) and p["priv"] > 0


def test_paths_lds_privatised_bins():
    """16 bins and 100000 samples (6250 per bin): the LDS-privatised variant, and no global
    per-lane or per-wave atomics into the bins."""
    case, low = _binsum_b(100000, 16)
    p = _paths(case, low, "binsum_b")
    assert p["priv"] > 0 and p["lane"] == 0 and p["agg"] == 0


def test_paths_global_atomics_for_sparse_bins():
    """3000 bins and 20000 samples (under 32 per bin): no LDS copy; random bins, so waves add
    per lane."""
    case, low = _binsum_b(20000, 3000)
    p = _paths(case, low, "binsum_b")
    assert p["priv"] == 0 and p["lane"] > 0


def test_paths_narrow_output_form():
    """11 outputs of a 19990-tap correlation: the wave-per-iteration kernel runs."""
    n, k = 20000, 19990
    shapes = {a + s: v for a, v in dict(loss=1, inp=n, w=k, out=n - k + 1).items() for s in ("", "b", "d", "bd")}
    case, low = _case(GENERIC / "window1d_d.jl", "window1d", "d", shapes, dict(i_n=n, i_k=k),
                      label="paths window1d_d narrow")
    p = _paths(case, low, "window1d_d")
    assert p["split"] > 0



@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("mn", [(1000, 1024), (64, 257), (130, 700), (256, 300), (9000, 300), (16384, 260)])
def test_lowered_affine_lanes_over_rows(mode, mn):
    """A column-major matrix updated by rows (the affine adjoint's and HVP's row loops, whose
    inner loops accumulate into wb): the lanes take 16, 32 or 64 consecutive rows (fewer rows a
    block when the rows are few: 16 up to 8191 rows, 32 up to 16383, 64 at 16384) and the block's
    shares of each row's inner loop (64 / rows-a-block per wave, 16 waves) run it in parts,
    the rows' sums combined in a fixed order; rows past the range (1000, 130 and 9000 are not
    multiples of the block's rows) compute a row again and store nothing.  The row sums
    alone (the tangent's loop reads the matrix, updates nothing along it) keep the
    wave-per-row form.  Every output against the oracle; the forms' blocks ran."""
    m, n = mn
    shapes = {k: (m, n) for k in ("w", "wb", "wd", "wbd")}
    shapes.update({k: n for k in ("x", "xb", "xd", "xbd")})
    shapes.update({k: m for k in ("b", "bb", "bd", "bbd", "t", "tb", "td", "tbd", "r", "rb", "rd", "rbd")})
    shapes.update({k: 1 for k in ("loss", "lossb", "lossd", "lossbd")})
    case, low = _case(CORPUS / f"affine_lsq_{mode}.jl", "affine_lsq", mode, shapes, dict(i_m=m, i_n=n),
                      label=f"xsplit affine_lsq_{mode} {m}x{n}")
    p = _paths(case, low, f"affine_lsq_{mode}")
    assert p["split"] > 0
    assert (p["xsplit"] > 0) == (mode != "d")


# ---- flat loops: the row-block and column-block twins ------------------------------------

# (rows, columns): rows of 300, 256 and 513 columns (the last column block partial) take the
# row twin, and with at least 64 rows the column twin; a row of 255 columns, a single element and
# no rows take neither.  Few long rows split over several blocks each (10 x 100000: 49 chunks of
# 2041 iterations; 3 x 40000: 20 chunks).
FLAT_SIZES = [(100, 300), (64, 256), (2000, 513), (300, 5000), (63, 256), (64, 255), (1, 1), (0, 3),
              (10, 100000), (3, 40000)]


def _row_blocks(m, n):
    """Blocks of the row twin: `_tr * _ts` of the lowered host code."""
    ts = max(1, min(-(-n // 2048), -(-4096 // max(m, 1))))
    return m * ts


@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("mn", FLAT_SIZES)
def test_lowered_flat_twins(mode, mn):
    """The row-major flat mat-vec through the lowering against the oracle, with the path counters:
    the forward loop's row sums run as the row-block twin when the range is whole rows of at least
    256 (blocks of at least 2048 iterations of one row, about 4096 blocks), and the adjoint loop's
    column sums as the column-block twin when there are also at least 64 rows (32-column,
    128-row tiles)."""
    m, n = mn
    shapes = {k + s: v for k, v in dict(loss=1, a=m * n, x=n, y=m).items() for s in ("", "b", "d", "bd")}
    case, low = _case(GENERIC / f"flatmv_{mode}.jl", "flatmv", mode, shapes, dict(i_m=m, i_n=n),
                      label=f"flat twins flatmv_{mode} m={m} n={n}")
    p = _paths(case, low, f"flatmv_{mode}")
    assert p["row"] == (_row_blocks(m, n) if n >= 256 and m >= 1 else 0)
    col_blocks = (-(-n // 32)) * (-(-m // 128)) if n >= 256 and m >= 64 else 0
    assert p["col"] == (col_blocks if mode != "d" else 0)
