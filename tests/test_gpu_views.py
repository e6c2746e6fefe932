"""Every entry point with arrays that are views one element into a larger allocation (so
8-byte aligned for fp64 and 4-byte aligned for fp32, never 16-byte aligned): the kernels'
16-byte vector paths must test alignment and fall back, with results unchanged.  One or two
cases per kernel, at sizes that reach the vector paths at full size (bench widths for the
MLP products, several tiles for the others); compared with the oracle as in the parity tests."""
import numpy as np
import pytest

from helpers import run_parity
from test_gpu_conv import conv_shapes

pytestmark = pytest.mark.gpu

MODES = ["b", "d", "hv"]


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("mn", [(65, 130), (1024, 1024)])
def test_affine_lsq_views(mode, mn):
    m, n = mn
    shapes = {k: (m, n) for k in ("w", "wb", "wd", "wbd")}
    shapes.update({k: n for k in ("x", "xb", "xd", "xbd")})
    shapes.update({k: m for k in ("b", "bb", "bd", "bbd", "t", "tb", "td", "tbd", "r", "rb", "rd", "rbd")})
    shapes.update({k: 1 for k in ("loss", "lossb", "lossd", "lossbd")})
    print(f"affine_lsq_{mode} m={m} n={n} offset=1", flush=True)
    run_parity("affine_lsq", mode, shapes, dict(i_m=m, i_n=n), offset=1)


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("size", [(130, 129, 131, 10), (256, 784, 1024, 10)])
def test_mlp2_ce_views(mode, size):
    from oracle import rng as jrng
    B, I, H, O = size
    sz = dict(loss=1, x=I * B, w1=H * I, b1=H, w2=O * H, b2=O, h1=H * B, z=O * B)
    shapes = {k + suf: v for k, v in sz.items() for suf in ("", "b", "d", "bd")}
    lab = np.array([1 + int(jrng.Xoshiro(17 + s).rand() * O) for s in range(B)], dtype=np.int64)
    g1, g2 = np.sqrt(2.0 / (I + H)), np.sqrt(2.0 / (H + O))
    scales = {"w1": g1, "w1d": g1, "w2": g2, "w2d": g2, "b1": 0.1, "b2": 0.1}
    print(f"mlp2_ce_{mode} B={B} I={I} H={H} O={O} offset=1", flush=True)
    run_parity("mlp2_ce", mode, shapes, dict(i_b=B, i_in=I, i_h=H, i_out=O), precision="f32",
               int_arrays=dict(lab=lab), scales=scales, offset=1)


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("size", [(2, 17, 33, 13, 70), (1, 64, 64, 40, 96)])
def test_conv3x3_views(mode, size):
    N, C, K, H, W = size
    s = 1.0 / np.sqrt(9.0 * C)
    print(f"conv3x3_{mode} N={N} C={C} K={K} H={H} W={W} offset=1", flush=True)
    run_parity("conv3x3", mode, conv_shapes(*size), dict(i_nb=N, i_c=C, i_k=K, i_h=H, i_w=W), precision="f32",
               scales={"w": s, "wd": s}, offset=1)


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("case", [(4097, 70, 10.0), (8192, 33, 0.5)])
def test_burgers1d_views(mode, case):
    n, T, tend = case
    shapes = {k: n for k in ("u", "ub", "un", "unb", "ud", "ubd", "und", "unbd")}
    shapes.update({k: 1 for k in ("loss", "lossb", "lossd", "lossbd")})
    scalars = dict(nu=0.05, dt=0.002, dx=0.5, tend=tend, nud=0.3, dtd=-0.2, dxd=0.1, tendd=0.7)
    stacks = () if mode == "d" else (("branch_stack", (T, "Ai")), ("u_stack", (T * n, "Af")))
    print(f"burgers1d_{mode} n={n} nsteps={T} tend={tend} offset=1", flush=True)
    run_parity("burgers1d", mode, shapes, dict(n=n, nsteps=T), scalars=scalars, stacks=stacks, offset=1)
