"""burgers1d under the checkpoint tape policy (stade_hip_burgers1d_b_ckpt / _hv_ckpt).

Against the oracle (the generated text, which stores every state): every output, the Int64
branch stack bit-exact and the returned scalars to the fp64 bar; the checkpoint rows equal the
oracle's u_stack rows k * every (the rows the policy does not keep are taken from the oracle,
so the stack comparison checks the kept ones).  Cases: segment lengths that divide the run,
do not, exceed it, equal 1 (the full tape), an early-stopping guard, a guard that runs no step,
and several 32-step chunks per segment.

At the benchmark size and physics (2^20 cells, 500 steps, nu = 1e-3, dt = 0.2 dx^2 / nu) the
policy is compared with the tape form on the GPU: the same kernels advance the same states, so
ub (+ ubd), un, loss and the branch stack are equal bit for bit; the scalar shadows are sums
chunked differently and agree to 1e-12."""
import numpy as np
import pytest

from helpers import ParityCase, make_args, oracle_lib

pytestmark = pytest.mark.gpu

CASES = [(7, 6, 10.0, 2), (7, 6, 0.007, 3), (7, 6, -1.0, 2), (7, 0, 10.0, 3), (2, 5, 10.0, 1), (100, 40, 10.0, 32),
         (100, 40, 10.0, 7), (100, 40, 10.0, 64), (4097, 70, 10.0, 32), (4097, 70, 10.0, 16), (8192, 33, 0.5, 5),
         (1 << 20, 40, 10.0, 32), (3000, 100, 10.0, 64)]


@pytest.mark.parametrize("mode", ["b", "hv"])
@pytest.mark.parametrize("case", CASES)
def test_burgers1d_ckpt_parity(mode, case):
    import torch
    import stade_hip
    n, T, tend, every = case
    print(f"burgers1d_{mode}_ckpt n={n} nsteps={T} tend={tend} every={every}", flush=True)
    shapes = {k: n for k in ("u", "ub", "un", "unb", "ud", "ubd", "und", "unbd")}
    shapes.update({k: 1 for k in ("loss", "lossb", "lossd", "lossbd")})
    scalars = dict(nu=0.05, dt=0.002, dx=0.5, tend=tend, nud=0.3, dtd=-0.2, dxd=0.1, tendd=0.7)
    stacks = (("branch_stack", (T, "Ai")), ("u_stack", (T * n, "Af")))
    lib = oracle_lib("burgers1d", mode)
    fname = f"burgers1d_{mode}"
    shp = dict(shapes)
    shp["__stacks__"] = ("branch_stack", "u_stack")
    args = make_args(lib, fname, shp, dict(n=n, nsteps=T), scalars, f"ckpt-{fname}-{n}-{T}")
    box = {}

    def run(dev, stack_d):
        _, lc = stade_hip.burgers1d_ckpt_lengths(n, T, every)
        ck = torch.full((lc,), float("nan"), dtype=torch.float64, device="cuda")
        fn = stade_hip.burgers1d_b_ckpt if mode == "b" else stade_hip.burgers1d_hv_ckpt
        r = fn(*dev, stack_d[0], ck, every)
        # the oracle's stack, with the rows the policy keeps replaced by the GPU's checkpoints
        full = torch.from_numpy(box["case"].stack_h[1].copy()).to("cuda")
        rows = (T + every - 1) // every
        for k in range(rows):
            if k * every < T:
                full[k * every * n:(k * every + 1) * n] = ck[k * n:(k + 1) * n]
        stack_d[1].copy_(full)
        return r

    case = ParityCase("burgers1d", mode, args, stacks, "f64", label=f"{fname}_ckpt n={n} T={T} every={every}", runner=run)
    box["case"] = case
    case.run_oracle(lib)
    case.run_gpu()
    print(f"{case.label}: worst {case.compare():.3e}", flush=True)


def _bench_args(mode):
    import bench
    import torch
    wl = bench.Burgers(mode)
    wl.setup(torch.device("cuda:0"))
    return wl


@pytest.mark.parametrize("mode", ["b", "hv"])
def test_burgers1d_ckpt_matches_tape_at_benchmark_size(mode):
    import torch
    import stade_hip
    every = 32
    print(f"burgers1d_{mode}: checkpoint policy (every {every}) against the tape form at 2^20 x 500", flush=True)
    wl = _bench_args(mode)
    n, T = wl.n, wl.T
    base = [a.clone() if isinstance(a, torch.Tensor) else a for a in wl.argv]
    tensors = lambda xs: [a for a in xs if isinstance(a, torch.Tensor)]
    # the tape form
    a1 = [a.clone() if isinstance(a, torch.Tensor) else a for a in base]
    r1 = getattr(stade_hip, f"burgers1d_{mode}")(*a1)
    torch.cuda.synchronize()
    # the checkpoint policy: the same arguments with u_stack replaced by the checkpoints
    a2 = [a.clone() if isinstance(a, torch.Tensor) else a for a in base]
    _, lc = stade_hip.burgers1d_ckpt_lengths(n, T, every)
    ck = torch.empty(lc, dtype=torch.float64, device="cuda")
    r2 = getattr(stade_hip, f"burgers1d_{mode}_ckpt")(*a2[:-1], ck, every)
    torch.cuda.synchronize()
    u_stack = a1[-1]
    for k, (x, y) in enumerate(zip(tensors(a1[:-1]), tensors(a2[:-1]))):
        assert torch.equal(x, y), f"argument {k} differs between the tape form and the checkpoint policy"
    rows = (T + every - 1) // every
    assert torch.equal(ck.view(rows, n), u_stack.view(T, n)[::every][:rows])
    for x, y in zip(r1, r2):
        assert abs(x - y) <= 1e-12 * max(abs(x), 1e-300), (r1, r2)
    print(f"burgers1d_{mode}: equal; scalar shadows {r1} / {r2}", flush=True)
