"""The Julia host code that `stade_hip_file` writes, run on the GPU against the oracle.

The emitted `<name>_hip` functions are executed by tests/jlhost.py (the image has no Julia):
each `ccall` goes through ctypes with the types the emitted text declares, and the results are
compared with the oracle like every other parity case (fp64 1e-12, fp32 1e-5, integers
exact).  Covered: the three generic kernels through the general lowering (b, d, hv), the
config kernels' hand-written entry points (a Burgers adjoint whose stacks come from the
emitted `initstacks_burgers1d_b_hip`, released by the garbage collector as Julia would, the
diffusion HVP, the affine adjoint with a matrix argument, the MLP adjoint with its labels),
and the two error paths: an out-of-range MLP label under `inbounds=false` and an
out-of-range bin in a lowered file, both throwing `BoundsError`, with the next call clean."""
import numpy as np
import pytest

from helpers import CORPUS, ParityCase, make_args
from jlhost import JlBoundsError, JlHost

pytestmark = pytest.mark.gpu

GENERIC = CORPUS / "generic"


def _host(tmp_path, src, **kw):
    from stade_hip import stade_hip_file
    from stade_hip.api import lib_path
    tmp_path.mkdir(parents=True, exist_ok=True)
    return JlHost(stade_hip_file(src, tmp_path / "host.jl", lib_path=str(lib_path()), **kw))


def _case(tmp_path, path, name, mode, shapes, ints, scalars=None, int_arrays=None, stacks=(), precision="f64",
          scales=None, initstacks=None, **kw):
    from oracle import runner
    print(f"emitted {name}_{mode} {ints}: oracle, emission", flush=True)
    lib_o = runner.load(path, precision=precision)
    fname = f"{name}_{mode}"
    shp = dict(shapes)
    shp["__stacks__"] = tuple(s for s, _ in stacks)
    fdt = np.float32 if precision == "f32" else np.float64
    args = make_args(lib_o, fname, shp, ints, scalars or {}, f"emitted-{fname}-{ints}", fdt, int_arrays, scales)
    host = _host(tmp_path, path, **kw)
    dims = {a: v.shape for a, _, v in args if isinstance(v, np.ndarray) and v.ndim > 1}

    def run(dev, stack_d):
        if initstacks is not None:
            # the stacks the emitted initstacks_<k>_b_hip allocates, copied out for the comparison
            own = host.call(f"initstacks_{name}_b_hip", *initstacks)
            own = own if isinstance(own, tuple) else (own,)
            assert [o.numel() for o in own] == [s.numel() for s in stack_d]
            for o, s in zip(own, stack_d):
                o.copy_(s)
            r = host.call(f"{fname}_hip", *dev, *own, dims=dims)
            for o, s in zip(own, stack_d):
                s.copy_(o)
            return r
        return host.call(f"{fname}_hip", *dev, *stack_d, dims=dims)
    case = ParityCase(name, mode, args, stacks, precision, label=f"emitted {fname} {ints}", runner=run,
                      oracle_path=path)
    case.run_oracle(lib_o)
    return case


def _check(case):
    case.run_gpu()
    print(f"{case.label}: worst {case.compare():.3e}", flush=True)


@pytest.mark.parametrize("mode", ["b", "d", "hv"])
def test_emitted_generic_matvec_scatter(tmp_path, mode):
    m, n = 300, 70
    shapes = {k + s: v for k, v in dict(loss=1, a=m * n, x=n, y=m).items() for s in ("", "b", "d", "bd")}
    _check(_case(tmp_path, GENERIC / f"matvec_scatter_{mode}.jl", "matvec_scatter", mode, shapes, dict(i_m=m, i_n=n)))


@pytest.mark.parametrize("mode", ["b", "d", "hv"])
def test_emitted_generic_window1d(tmp_path, mode):
    n, k = 1000, 7
    shapes = {a + s: v for a, v in dict(loss=1, inp=n, w=k, out=n - k + 1).items() for s in ("", "b", "d", "bd")}
    _check(_case(tmp_path, GENERIC / f"window1d_{mode}.jl", "window1d", mode, shapes, dict(i_n=n, i_k=k)))


def _bins(n, b, seed):
    from oracle import rng as jrng
    g = jrng.Xoshiro(seed)
    return np.array([1 + int(g.rand() * b) for _ in range(n)], dtype=np.int64)


@pytest.mark.parametrize("mode", ["b", "d", "hv"])
def test_emitted_generic_binsum(tmp_path, mode):
    n, b = 100000, 16
    shapes = {a + s: v for a, v in dict(loss=1, v=n, c=b).items() for s in ("", "b", "d", "bd")}
    _check(_case(tmp_path, GENERIC / f"binsum_{mode}.jl", "binsum", mode, shapes, dict(i_n=n, i_b=b),
                 int_arrays=dict(bins=_bins(n, b, 5))))


def test_emitted_burgers_adjoint_with_emitted_stacks(tmp_path):
    n, T = 100, 12
    shapes = {k: n for k in ("u", "ub", "un", "unb")}
    shapes.update(loss=1, lossb=1)
    scalars = dict(nu=0.05, dt=0.002, dx=0.5, tend=10.0)
    stacks = (("branch_stack", (T, "Ai")), ("u_stack", (T * n, "Af")))
    _check(_case(tmp_path, CORPUS / "burgers1d_b.jl", "burgers1d", "b", shapes, dict(n=n, nsteps=T), scalars=scalars,
                 stacks=stacks, initstacks=(n, T)))


def test_emitted_diffusion_hvp(tmp_path):
    n = 64
    shapes = {k: n * n for k in ("u", "ub", "un", "unb", "ud", "ubd", "und", "unbd")}
    shapes.update({k: 1 for k in ("loss", "lossb", "lossd", "lossbd")})
    _check(_case(tmp_path, CORPUS / "diffusion2d_hv.jl", "diffusion2d", "hv", shapes, dict(n=n)))


def test_emitted_affine_adjoint(tmp_path):
    m, n = 65, 33
    shapes = {k: (m, n) for k in ("w", "wb")}
    shapes.update({k: n for k in ("x", "xb")})
    shapes.update({k: m for k in ("b", "bb", "t", "tb", "r", "rb")})
    shapes.update(loss=1, lossb=1)
    _check(_case(tmp_path, CORPUS / "affine_lsq_b.jl", "affine_lsq", "b", shapes, dict(i_m=m, i_n=n)))


def _mlp_case(tmp_path, lab, **kw):
    B, I, H, O = 33, 17, 40, 10
    sz = dict(loss=1, x=I * B, w1=H * I, b1=H, w2=O * H, b2=O, h1=H * B, z=O * B)
    shapes = {k + s: v for k, v in sz.items() for s in ("", "b")}
    g1, g2 = np.sqrt(2.0 / (I + H)), np.sqrt(2.0 / (H + O))
    return _case(tmp_path, CORPUS / "mlp2_ce_b.jl", "mlp2_ce", "b", shapes, dict(i_b=B, i_in=I, i_h=H, i_out=O),
                 int_arrays=dict(lab=lab), precision="f32", scales={"w1": g1, "w2": g2, "b1": 0.1, "b2": 0.1}, **kw)


def test_emitted_mlp_adjoint_checked(tmp_path):
    lab = _bins(33, 10, 17)
    _check(_mlp_case(tmp_path, lab, inbounds=False))


@pytest.mark.parametrize("bad", [0, 11])
def test_emitted_mlp_label_out_of_range_throws(tmp_path, bad):
    lab = _bins(33, 10, 17)
    lab[5] = bad
    case = _mlp_case(tmp_path / "bad", lab, inbounds=False)
    with pytest.raises(JlBoundsError):
        case.run_gpu()
    # the flag is cleared: a good call afterwards passes
    _check(_mlp_case(tmp_path / "good", _bins(33, 10, 17), inbounds=False))


@pytest.mark.parametrize("bad", [0, 17])
def test_emitted_lowered_bin_out_of_range_throws(tmp_path, bad):
    """An index outside its array in a lowered file written with `inbounds=false`: every
    lowered access is checked, the kernel skips the access and flags it, the emitted host code
    throws BoundsError.  (With the default `inbounds=true`, as under Julia's @inbounds, such an
    index is undefined behaviour; no test gives one to an unchecked build.)"""
    import torch
    n, b = 5000, 16
    bins = _bins(n, b, 9)
    bins[1234] = bad
    host = _host(tmp_path, GENERIC / "binsum_b.jl", inbounds=False)
    dev = lambda k: torch.zeros(k, dtype=torch.float64, device="cuda")
    v = torch.randn(n, dtype=torch.float64, device="cuda")
    args = [dev(1), torch.ones(1, dtype=torch.float64, device="cuda"), v, dev(n),
            torch.from_numpy(bins).to("cuda"), dev(b), dev(b), n, b]
    with pytest.raises(JlBoundsError):
        host.call("binsum_b_hip", *args)
    torch.cuda.synchronize()
    # the next call, with good bins, runs clean and matches the oracle
    _check(_case(tmp_path / "good", GENERIC / "binsum_b.jl", "binsum", "b",
                 {a + s: v for a, v in dict(loss=1, v=n, c=b).items() for s in ("", "b")}, dict(i_n=n, i_b=b),
                 int_arrays=dict(bins=_bins(n, b, 9))))
