"""The benchmark workloads themselves, at the shapes and with the inputs `bench.py` times.

Two kinds of check, both on the inputs `bench.py`'s workloads build (`Workload.host_inputs`:
the same seeds, scales, zero shadows and Burgers scalars):

1. Oracle parity at the benchmark's launch geometry.  Each case runs the generated text on
   the oracle and the entry point on the GPU and compares every output (the parity bars of
   `helpers.RTOL`, with the truth rule where they are exceeded):
   - mlp2_ce b/d/hv at the full 784 -> 1024 -> 10, batch 4096 (the GEMM split plan and
     the 4096-sample fp32 reductions the benchmark runs);
   - conv3x3 b/d/hv on one full 256 x 256 image, 64 -> 64 channels: the same 256-way
     weight-gradient split as the benchmark's 8 images;
   - burgers1d b/d/hv on 2^20 cells for 500 steps with nu = 1e-3, dx = 1/n,
     dt = 0.2 dx^2 / nu: 16 backward chunks, the 20-step tail chunk, the 4.2 GB tape.
   The oracle is sequential C and takes from seconds (conv, Burgers) to about two minutes
   (the MLP HVP) per case, so every case's oracle run starts in a worker thread when the
   module starts; each test then waits for its own.

2. Size-independent properties at the full benchmark size of every config (conv: all 8
   images), and for diffusion2d also at 8192 x 8192, on the GPU alone:
   - the adjoint's defining identity <yb, J xd> = <J^T yb, xd> between the `_d` and `_b`
     entry points over the whole in-place state, with random yb and xd
     (`val_validate_dotprod` /root/reference/src/STADE.jl:17108-17131, with its scale
     max(|lhs|, |rhs|, 1));
   - the symmetry of the Hessian of the loss, v^T (H w) = w^T (H v), from two `_hv` calls.
"""
from __future__ import annotations

import concurrent.futures as cf
import time

import numpy as np
import pytest

from helpers import ParityCase, oracle_lib

pytestmark = pytest.mark.gpu

# identity / symmetry bars: the reference's 1e-11 for fp64 code; fp32 code sums millions of
# rounded products, so its bar is 1e-4 (the measured values are printed)
PROP_RTOL = {"f64": 1e-11, "f32": 1e-4}


def _bench():
    import bench
    return bench


def _case(wl, label: str) -> ParityCase:
    """A ParityCase with every argument taken from the workload's host inputs by name."""
    prec = "f32" if wl.dtype == "f32" else "f64"
    lib = oracle_lib(wl.family, wl.mode, prec)
    h = wl.host_inputs()
    stacks = list(zip(("branch_stack", "u_stack"), wl.stack_lengths())) if wl.mode != "d" else []
    names = {s for s, _ in stacks}
    args = []
    for a, kind in lib.infos[wl.name].args:
        if a in names:
            continue
        v = h[a]
        if kind == "i":
            v = int(v)
        elif kind == "f":
            v = float(v)
        args.append((a, kind, v))
    return ParityCase(wl.family, wl.mode, args, stacks, prec, label=label)


class _Pool:
    """Oracle runs of the module's heavy cases, started together in worker threads."""

    def __init__(self):
        b = _bench()
        self.cases, self.futs = {}, {}
        specs = [("mlp2_ce", m, lambda m=m: b.Mlp(m)) for m in ("hv", "b", "d")]
        specs += [("conv3x3", m, lambda m=m: b.Conv(m, N=1)) for m in ("b", "d", "hv")]
        specs += [("burgers1d", m, lambda m=m: b.Burgers(m)) for m in ("d", "b", "hv")]
        self.ex = cf.ThreadPoolExecutor(max_workers=6)
        t0 = time.time()
        for fam, mode, mk in specs:
            key = (fam, mode)
            self.futs[key] = self.ex.submit(self._oracle, key, mk, t0)
        # the fp32 configs' truth (fp64 text) is cheap beside its oracle run: start it too, so a
        # case that needs the truth rule does not wait for it
        for fam in ("mlp2_ce", "conv3x3"):
            for mode in ("b", "d", "hv"):
                self.futs[(fam, mode, "truth")] = self.ex.submit(self._truth, (fam, mode), t0)

    def _oracle(self, key, mk, t0):
        wl = mk()
        case = _case(wl, f"{wl.name} benchmark workload")
        self.cases[key] = case
        case.run_oracle()
        print(f"[oracle {key[0]}_{key[1]} done at {time.time() - t0:.0f} s]", flush=True)
        return case

    def _truth(self, key, t0):
        case = self.futs[key].result()
        case.run_truth()
        print(f"[truth {key[0]}_{key[1]} done at {time.time() - t0:.0f} s]", flush=True)
        return case

    def get(self, fam, mode) -> ParityCase:
        print(f"waiting for the oracle of {fam}_{mode}", flush=True)
        return self.futs[(fam, mode)].result()

    def close(self):
        for f in self.futs.values():
            f.cancel()
        self.ex.shutdown(wait=True)


_POOL = None


@pytest.fixture(scope="module", autouse=True)
def oracle_pool():
    """Starts every heavy oracle run when the module starts (the property tests below run
    on the GPU meanwhile)."""
    global _POOL
    _POOL = _Pool()
    yield _POOL
    _POOL.close()
    _POOL = None


# ------------------------------------------------------------------------------------------
# properties at the full benchmark size
# ------------------------------------------------------------------------------------------

def _pairs(family: str, mode: str, suffix: str):
    """(primal, shadow, kind) of each float argument of the generated function: arrays
    ('A') and scalars ('F' with its 'R' or 'F' partner)."""
    from stade_hip.emit import KERNELS
    args = KERNELS[family].modes[mode].args
    out = []
    for (a, ka), (b, kb) in zip(args, args[1:]):
        if b == a + suffix and ka in ("A", "F"):
            out.append((a, b, ka))
    return out


def _dev_state(wl, dev="cuda"):
    import torch
    h = wl.host_inputs()
    return {k: (torch.from_numpy(np.ascontiguousarray(v.ravel(order="F"))).to(dev) if isinstance(v, np.ndarray) else v)
            for k, v in h.items()}


def _call(wl, mode, st: dict, stacks=()):
    import stade_hip
    b = _bench()
    names = b.arg_names(wl.family, mode)
    nst = len(stacks)
    return getattr(stade_hip, f"{wl.family}_{mode}")(*(st[a] for a in names[:len(names) - nst]), *stacks)


def _stacks(wl):
    import torch
    if wl.family != "burgers1d":
        return ()
    dt = torch.float64
    return tuple(torch.empty(k, dtype=torch.int64 if kind == "Ai" else dt, device="cuda") for k, kind in wl.stack_lengths())


def _rand_like(t, g):
    import torch
    return torch.randn(t.shape, generator=g, dtype=torch.float64, device=t.device).to(t.dtype)


def _dot(a, b):
    return float((a.double() * b.double()).sum().item())


def _scalar_dir(g, value: float) -> float:
    """A random direction for a float scalar argument, scaled by the scalar itself (a relative
    perturbation of order one), so that no scalar's term swamps the arrays' in a sum."""
    import torch
    return float(torch.randn(1, generator=g, device="cuda").item()) * (abs(value) or 1.0)


FULL = {
    "affine_lsq": lambda b: b.Affine("b"),
    "diffusion2d": lambda b: b.Diffusion("b"),
    "mlp2_ce": lambda b: b.Mlp("b"),
    "conv3x3": lambda b: b.Conv("b"),
    "burgers1d": lambda b: b.Burgers("b"),
    # a grid above the benchmark's: the 16-row chunks every mode takes at large n
    "diffusion2d_8192": lambda b: b.Diffusion("b", n=8192),
}


@pytest.mark.parametrize("family", list(FULL))
def test_dotprod_identity_full_size(family):
    """<yb, J xd> = <J^T yb, xd> over every float argument, between the tangent and the
    adjoint entry points, at the benchmark size and point."""
    import torch
    wl = FULL[family](_bench())
    print(f"dot-product identity {family} at the benchmark size", flush=True)
    base = _dev_state(wl)
    g = torch.Generator(device="cuda")
    g.manual_seed(20261202)
    bp = _pairs(wl.family, "b", "b")
    dp = _pairs(wl.family, "d", "d")
    assert [p for p, _, _ in bp] == [p for p, _, _ in dp]
    xd, yb = {}, {}
    for p, _, kind in bp:
        if kind == "A":
            xd[p] = _rand_like(base[p], g)
            yb[p] = _rand_like(base[p], g)
        else:
            xd[p] = _scalar_dir(g, base[p])
            yb[p] = float(torch.randn(1, generator=g, device="cuda").item())
    # tangent: tangents in = xd, out = J xd
    st = {k: (v.clone() if isinstance(v, torch.Tensor) else v) for k, v in base.items()}
    for p, s, _ in dp:
        st[s] = xd[p].clone() if isinstance(xd[p], torch.Tensor) else xd[p]
    _call(wl, "d", st)
    torch.cuda.synchronize()
    lhs = 0.0
    for p, s, kind in dp:
        lhs += _dot(yb[p], st[s]) if kind == "A" else yb[p] * xd[p]   # a scalar's tangent passes through
    # adjoint: shadows in = yb, out = J^T yb
    st = {k: (v.clone() if isinstance(v, torch.Tensor) else v) for k, v in base.items()}
    for p, s, _ in bp:
        st[s] = yb[p].clone() if isinstance(yb[p], torch.Tensor) else yb[p]
    ret = _call(wl, "b", st, _stacks(wl))
    torch.cuda.synchronize()
    ret = () if ret is None else (ret if isinstance(ret, tuple) else (ret,))
    scal = [p for p, _, kind in bp if kind == "F"]
    assert len(ret) == len(scal)
    rhs = 0.0
    for p, s, kind in bp:
        if kind == "A":
            rhs += _dot(st[s], xd[p])
    for p, v in zip(scal, ret):
        rhs += v * xd[p]
    scale = max(abs(lhs), abs(rhs), 1.0)
    err = abs(lhs - rhs) / scale
    print(f"dot-product identity {family}: lhs {lhs:.12e} rhs {rhs:.12e} rel {err:.3e}", flush=True)
    assert err <= PROP_RTOL[wl.dtype], f"{family}: <yb, J xd> - <J^T yb, xd> relative {err:.3e}"


@pytest.mark.parametrize("family", list(FULL))
def test_hessian_symmetry_full_size(family):
    """v^T (H w) = w^T (H v) for the Hessian of the loss, from two HVP calls at the
    benchmark point (lossb = 1, every other seed 0, as the benchmark runs)."""
    import torch
    b = _bench()
    wl = FULL[family](b)
    print(f"Hessian symmetry {family} at the benchmark size", flush=True)
    base = _dev_state(wl)
    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    # the HVP's argument list is the adjoint's, then (xd, xbd) per float argument
    bp = _pairs(wl.family, "b", "b")
    dirs = []
    for _ in range(2):
        v = {}
        for p, _, kind in bp:
            if kind == "A":
                v[p] = _rand_like(base[p], g)
            else:
                v[p] = _scalar_dir(g, base[p])
        dirs.append(v)
    hv_out = []
    for v in dirs:
        st = {k: (v_.clone() if isinstance(v_, torch.Tensor) else v_) for k, v_ in base.items()}
        for p, _, kind in bp:
            st[p + "d"] = v[p].clone() if kind == "A" else v[p]
            st[p + "bd"] = torch.zeros_like(base[p]) if kind == "A" else 0.0
        ret = _call(wl, "hv", st, _stacks(wl))
        torch.cuda.synchronize()
        ret = () if ret is None else (ret if isinstance(ret, tuple) else (ret,))
        scal = [p for p, _, kind in bp if kind == "F"]
        hw = {p: st[p + "bd"] for p, _, kind in bp if kind == "A"}
        for k, p in enumerate(scal):
            hw[p] = ret[2 * k + 1]          # the HVP returns (xb, xbd) pairs
        hv_out.append(hw)

    def inner(u, hw):
        tot = 0.0
        for p, _, kind in bp:
            tot += _dot(u[p], hw[p]) if kind == "A" else u[p] * hw[p]
        return tot
    lhs, rhs = inner(dirs[0], hv_out[1]), inner(dirs[1], hv_out[0])
    scale = max(abs(lhs), abs(rhs), 1.0)
    err = abs(lhs - rhs) / scale
    print(f"Hessian symmetry {family}: v'Hw {lhs:.12e} w'Hv {rhs:.12e} rel {err:.3e}", flush=True)
    assert err <= PROP_RTOL[wl.dtype], f"{family}: v'Hw - w'Hv relative {err:.3e}"


# ------------------------------------------------------------------------------------------
# oracle parity at the benchmark's launch geometry
# ------------------------------------------------------------------------------------------

@pytest.mark.parametrize("mode", ["b", "d", "hv"])
def test_conv3x3_benchmark_image(mode):
    """One full 256 x 256 image, 64 -> 64: the benchmark's 256-way weight-gradient split."""
    case = _POOL.get("conv3x3", mode)
    print(f"conv3x3_{mode} N=1 C=K=64 256x256 on the GPU", flush=True)
    case.run_gpu()
    print(f"conv3x3_{mode}: worst {case.compare():.3e}", flush=True)


@pytest.mark.parametrize("mode", ["d", "b", "hv"])
def test_burgers1d_benchmark_physics(mode):
    """2^20 cells, 500 steps, nu = 1e-3, dx = 1/n, dt = 0.2 dx^2 / nu (cdif = 0.2)."""
    case = _POOL.get("burgers1d", mode)
    print(f"burgers1d_{mode} n=2^20 nsteps=500 on the GPU", flush=True)
    case.run_gpu()
    print(f"burgers1d_{mode}: worst {case.compare():.3e}", flush=True)
    case.host = case.dev = case.stack_h = case.stack_d = None   # release the 4 GB tapes


@pytest.mark.parametrize("mode", ["d", "b", "hv"])
def test_mlp2_ce_benchmark_batch(mode):
    """784 -> 1024 -> 10 on the full batch of 4096."""
    case = _POOL.get("mlp2_ce", mode)
    print(f"mlp2_ce_{mode} B=4096 on the GPU", flush=True)
    case.run_gpu()
    print(f"mlp2_ce_{mode}: worst {case.compare():.3e}", flush=True)
