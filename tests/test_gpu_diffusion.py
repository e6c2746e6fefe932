"""diffusion2d on the GPU against the oracle (the transpiled generated code), fp64 to 1e-12.

Sizes cover the degenerate periodic grids (n = 1, 2: coincident neighbours), grids smaller
than a tile, ragged tiles (the LDS row-streaming kernels), multiples of 128 (the 128-column
wave strips: one strip whose halo wraps onto itself at n = 128, three strips and a partly
empty block at 384; each chunk height the launch picks by n: adjoint and tangent 16 rows at
128, 384 and 4224, 32 at 2048 (the adjoint also at 1536), the adjoint 64 and the tangent 32 at
4096; the HVP as the tangent), multiples of 64 only (the 64-column wave
strips: one strip at n = 64, strip counts that leave a block partly empty at 192 and 320), and
the benchmark grid n = 4096."""
import numpy as np
import pytest

from helpers import run_parity

pytestmark = pytest.mark.gpu

SIZES = [1, 2, 3, 5, 35, 36, 64, 65, 100, 128, 129, 192, 257, 320, 384, 1536, 2048, 4096, 4224]


@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("n", SIZES)
def test_diffusion2d_parity(mode, n):
    c = n * n
    shapes = {k: c for k in ("u", "ub", "un", "unb", "ud", "und", "ubd", "unbd")}
    shapes.update({k: 1 for k in ("loss", "lossb", "lossd", "lossbd")})
    print(f"diffusion2d_{mode} n={n}", flush=True)
    run_parity("diffusion2d", mode, shapes, dict(n=n))


@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("n", [128, 384])
def test_diffusion2d_element_aligned_views(mode, n):
    """Arrays that are views one element into a larger allocation (8-byte aligned only): the
    128-column kernels move 16-byte pairs, so such arrays must take the 64-column kernels."""
    c = n * n
    shapes = {k: c for k in ("u", "ub", "un", "unb", "ud", "und", "ubd", "unbd")}
    shapes.update({k: 1 for k in ("loss", "lossb", "lossd", "lossbd")})
    print(f"diffusion2d_{mode} n={n} offset=1", flush=True)
    run_parity("diffusion2d", mode, shapes, dict(n=n), offset=1)
