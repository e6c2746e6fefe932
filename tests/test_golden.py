"""The config kernels against the golden fixtures of tests/golden/ (torch CPU autograd in
float64 of the same primal, written by tests/golden/make_golden.py).

CPU tests: the oracle executing the derivative texts stade.jl_amd/corpus/<k>_{b,d,hv}.jl
(Float64) reproduces the fixture's gradient, directional derivative and Hessian-vector
product -- an AD independent of the texts, so a wrong term, sign or index in a hand-derived
text fails here.  GPU tests: libstade_hip, through the C ABI, reproduces the same fixtures
(Float32 configs on their float32-rounded inputs)."""
import numpy as np
import pytest

from helpers import ROOT, oracle_lib

GOLDEN = ROOT / "tests" / "golden"

# primal float inputs (with a fixture gradient), intermediates (outputs of the primal), Int args
CONFIGS = {
    "affine_lsq": dict(inputs=("w", "x", "b", "t"), scalars=(), inter=lambda s: {"r": s[0]}, ints=("i_m", "i_n"),
                       shapes={"w": lambda s: (s[0], s[1])}),
    "diffusion2d": dict(inputs=("u",), scalars=(), inter=lambda s: {"un": s[0] * s[0]}, ints=("n",)),
    "mlp2_ce": dict(inputs=("x", "w1", "b1", "w2", "b2"), scalars=(), inter=lambda s: {"h1": s[2] * s[0], "z": s[3] * s[0]},
                    ints=("i_b", "i_in", "i_h", "i_out")),
    "conv3x3": dict(inputs=("xp", "w"), scalars=(), inter=lambda s: {"out": s[0] * s[2] * s[3] * s[4]},
                    ints=("i_nb", "i_c", "i_k", "i_h", "i_w")),
    "burgers1d": dict(inputs=("u",), scalars=("nu", "dt", "dx", "tend"), inter=lambda s: {"un": s[0]}, ints=("n", "nsteps")),
}
FP32 = {"mlp2_ce", "conv3x3"}


def _base(name, known):
    for suf in ("bd", "b", "d"):
        if name.endswith(suf) and name[: -len(suf)] in known:
            return name[: -len(suf)], suf
    return name, ""


def _args(name, mode, fx, fdt):
    """Arguments of <name>_<mode> in the generated order, from the fixture: primal inputs,
    directions for their tangents, lossb = 1, zero shadows and intermediates."""
    cfg = CONFIGS[name]
    sizes = [int(v) for v in fx["sizes"]]
    inter = cfg["inter"](sizes)
    lib = oracle_lib(name, mode, "f64")
    info = lib.infos[f"{name}_{mode}"]
    known = set(cfg["inputs"]) | set(cfg["scalars"]) | set(inter) | {"loss"}
    out = []
    ints = dict(zip(cfg["ints"], sizes))
    for a, kind in info.args:
        if a in ("branch_stack", "u_stack"):
            continue
        base, suf = _base(a, known)
        if kind == "i":
            out.append((a, ints[a]))
        elif kind == "Ai":
            out.append((a, np.asarray(fx[a], dtype=np.int64).copy()))
        elif kind == "f":
            if suf == "":
                v = float(fx[a]) if a in fx.files else 0.0
            elif suf == "d" and f"{base}_dir" in fx.files:
                v = float(fx[f"{base}_dir"])
            else:
                v = 0.0
            out.append((a, v))
        else:
            if base == "loss":
                v = np.array([1.0 if suf == "b" else 0.0])
            elif base in cfg["inputs"]:
                if suf == "":
                    v = np.ravel(fx[base])
                elif suf == "d":
                    v = np.ravel(fx[f"{base}_dir"])
                else:
                    v = np.zeros(np.size(fx[base]))
            else:
                v = np.zeros(inter[base])
            v = np.asarray(v, dtype=fdt).copy()
            shp = cfg.get("shapes", {}).get(base)
            if shp is not None:  # a 2-D array of the text: Julia shape, column-major
                v = np.asfortranarray(v.reshape(shp(sizes), order="F"))
            out.append((a, v))
    return out, sizes


def _check(name, mode, fx, arrays, ret, rtol):
    cfg = CONFIGS[name]
    err = {}

    def rel(got, want):
        got, want = np.asarray(got, np.float64).ravel(order="F"), np.asarray(want, np.float64).ravel()
        scale = max(float(np.max(np.abs(want))), 1e-300)
        return float(np.max(np.abs(got - want))) / scale

    if mode in ("b", "hv"):
        err["loss"] = rel(arrays["loss"], fx["loss"])
        for k in cfg["inputs"]:
            err[f"{k}b"] = rel(arrays[f"{k}b"], fx[f"{k}_grad"])
            if mode == "hv":
                err[f"{k}bd"] = rel(arrays[f"{k}bd"], fx[f"{k}_hvp"])
        if cfg["scalars"]:
            sc = cfg["scalars"]
            if mode == "b":
                got = dict(zip(sc, ret))
                for k in sc:
                    want = fx[f"{k}_grad"] if f"{k}_grad" in fx.files else 0.0
                    err[f"{k}b"] = abs(got[k] - float(want)) / max(abs(float(want)), 1e-300) if float(want) else abs(got[k])
            else:
                for i, k in enumerate(sc):
                    for j, suf in enumerate(("grad", "hvp")):
                        want = float(fx[f"{k}_{suf}"]) if f"{k}_{suf}" in fx.files else 0.0
                        g = ret[2 * i + j]
                        err[f"{k}{'b' if j == 0 else 'bd'}"] = abs(g - want) / abs(want) if want else abs(g)
    if mode in ("d", "hv"):
        err["lossd"] = rel(arrays["lossd"], fx["lossd"])
    bad = {k: v for k, v in err.items() if not v <= rtol}
    assert not bad, f"{name}_{mode}: relative errors above {rtol:g}: {bad}"
    return err


@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("name", sorted(CONFIGS))
def test_oracle_matches_golden(name, mode):
    fx = np.load(GOLDEN / f"{name}.npz")
    args, sizes = _args(name, mode, fx, np.float64)
    lib = oracle_lib(name, mode, "f64")
    stacks = lib.stacks(f"initstacks_{name}_b", *sizes) if name == "burgers1d" and mode != "d" else ()
    ret = lib.call(f"{name}_{mode}", *[v for _, v in args], *stacks)
    _check(name, mode, fx, {a: v for a, v in args}, ret, 1e-10)


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("name", sorted(CONFIGS))
def test_gpu_matches_golden(name, mode):
    import torch
    import stade_hip
    print(f"golden {name}_{mode}", flush=True)
    fdt = np.float32 if name in FP32 else np.float64
    fx = np.load(GOLDEN / f"{name}.npz")
    args, sizes = _args(name, mode, fx, fdt)
    dev = [torch.from_numpy(np.ascontiguousarray(v.ravel(order="F"))).to("cuda") if isinstance(v, np.ndarray) else v
           for _, v in args]
    stacks = stade_hip.initstacks_burgers1d_b(*sizes) if name == "burgers1d" and mode != "d" else ()
    ret = getattr(stade_hip, f"{name}_{mode}")(*dev, *stacks)
    torch.cuda.synchronize()
    ret = () if ret is None else (ret if isinstance(ret, tuple) else (ret,))
    arrays = {a: (d.cpu().numpy() if isinstance(d, torch.Tensor) else d) for (a, _), d in zip(args, dev)}
    _check(name, mode, fx, arrays, ret, 1e-5 if fdt == np.float32 else 1e-10)
