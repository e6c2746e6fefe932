"""conv3x3 on the GPU against the oracle (the transpiled generated code run in Float32, as
`stade_amdgpu_file(...; precision=Float32)` runs it), fp32 to 1e-5 relative (normwise), with
the truth rule (fp64 oracle) where the two differ by more.

Sizes cover a single pixel and channel, ragged image tiles (widths and heights that are not
multiples of the 64 x 4 and 32 x 2 pixel tiles), channel counts that are not multiples of the
staging chunk or of the 64-channel slabs (two slabs each way), and the benchmark's 64 -> 64
channels on a reduced image.  Every padded cell of xp holds a nonzero value, so the padded
frame of xpb (taps that land on the padding) is checked as well."""
import numpy as np
import pytest

from helpers import run_parity

pytestmark = pytest.mark.gpu

SIZES = [(1, 1, 1, 1, 1), (2, 3, 5, 7, 9), (2, 17, 33, 13, 70), (2, 70, 65, 6, 33), (1, 64, 64, 40, 96)]


def conv_shapes(N, C, K, H, W):
    sz = dict(loss=1, xp=(W + 2) * (H + 2) * C * N, w=9 * C * K, out=W * H * K * N)
    shapes = {}
    for k, v in sz.items():
        for suf in ("", "b", "d", "bd"):
            shapes[k + suf] = v
    return shapes


@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("size", SIZES)
def test_conv3x3_parity(mode, size):
    N, C, K, H, W = size
    s = 1.0 / np.sqrt(9.0 * C)
    print(f"conv3x3_{mode} N={N} C={C} K={K} H={H} W={W}", flush=True)
    run_parity("conv3x3", mode, conv_shapes(*size), dict(i_nb=N, i_c=C, i_k=K, i_h=H, i_w=W), precision="f32",
               scales={"w": s, "wd": s})


@pytest.mark.parametrize("size", [(1, 0, 3, 4, 5), (0, 2, 3, 4, 5), (1, 2, 0, 4, 5), (1, 2, 3, 0, 5)])
def test_conv3x3_empty(size):
    """Empty extents: nothing but the loss loops (empty) runs; shadows keep their values."""
    print(f"conv3x3_hv empty {size}", flush=True)
    N, C, K, H, W = size
    run_parity("conv3x3", "hv", conv_shapes(*size), dict(i_nb=N, i_c=C, i_k=K, i_h=H, i_w=W), precision="f32")
