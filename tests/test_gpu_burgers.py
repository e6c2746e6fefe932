"""burgers1d on the GPU against the oracle (the transpiled generated code), fp64 to 1e-12;
the Int64 branch stack bit-exact, the tape written at the same slots with the same values.

Cases cover degenerate periodic grids (n = 1, 2), a guard that stops the loop early, a guard
that runs no step, no steps at all, several time chunks (more than 32 steps), several
blocks with a ragged last block, and the benchmark grid 2^20 on a few steps and on one full
32-step chunk plus a remainder."""
import pytest

from helpers import run_parity

pytestmark = pytest.mark.gpu

# (n, nsteps, tend) with dt = 0.002: tend = 0.007 runs 4 steps (0, .002, .004, .006 < .007); dt is
# small enough that the central scheme stays bounded over 70 steps (the oracle checks it)
CASES = [(1, 3, 10.0), (2, 5, 10.0), (7, 6, 0.007), (7, 6, -1.0), (7, 0, 10.0), (100, 40, 10.0),
         (4097, 70, 10.0), (8192, 33, 0.5), (1 << 20, 6, 10.0), (1 << 20, 40, 10.0)]


@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("case", CASES)
def test_burgers1d_parity(mode, case):
    n, T, tend = case
    shapes = {k: n for k in ("u", "ub", "un", "unb", "ud", "ubd", "und", "unbd")}
    shapes.update({k: 1 for k in ("loss", "lossb", "lossd", "lossbd")})
    scalars = dict(nu=0.05, dt=0.002, dx=0.5, tend=tend, nud=0.3, dtd=-0.2, dxd=0.1, tendd=0.7)
    stacks = () if mode == "d" else (("branch_stack", (T, "Ai")), ("u_stack", (T * n, "Af")))
    print(f"burgers1d_{mode} n={n} nsteps={T} tend={tend}", flush=True)
    run_parity("burgers1d", mode, shapes, dict(n=n, nsteps=T), scalars=scalars, stacks=stacks)
