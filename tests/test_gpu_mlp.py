"""mlp2_ce on the GPU against the oracle (the transpiled generated code run in Float32, as
`stade_amdgpu_file(...; precision=Float32)` runs it), fp32 to 1e-5 relative (normwise), with
the truth rule (fp64 oracle) where the two differ by more.

Sizes cover tiny and odd widths, widths that are not multiples of the 128 x 128 matrix-core
tile, an odd batch with the widest output layer (16) and a hidden width that is not a multiple
of 64, a hidden layer wider than 1024 (the per-sample head), and the benchmark widths 784 ->
1024 -> 10 on a reduced batch."""
import numpy as np
import pytest

from helpers import run_parity

pytestmark = pytest.mark.gpu

SIZES = [(8, 5, 7, 3), (64, 40, 48, 10), (130, 129, 131, 10), (33, 17, 300, 16), (16, 8, 1100, 4),
         (256, 784, 1024, 10), (8, 0, 7, 3), (0, 5, 7, 3)]


@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("size", SIZES)
def test_mlp2_ce_parity(mode, size):
    from oracle import rng as jrng
    B, I, H, O = size
    sz = dict(loss=1, x=I * B, w1=H * I, b1=H, w2=O * H, b2=O, h1=H * B, z=O * B)
    shapes = {}
    for k, v in sz.items():
        for suf in ("", "b", "d", "bd"):
            shapes[k + suf] = v
    lab = np.array([1 + int(jrng.Xoshiro(17 + s).rand() * O) for s in range(B)], dtype=np.int64)
    g1, g2 = np.sqrt(2.0 / (I + H)), np.sqrt(2.0 / (H + O))
    scales = {"w1": g1, "w1d": g1, "w2": g2, "w2d": g2, "b1": 0.1, "b2": 0.1}
    print(f"mlp2_ce_{mode} B={B} I={I} H={H} O={O}", flush=True)
    run_parity("mlp2_ce", mode, shapes, dict(i_b=B, i_in=I, i_h=H, i_out=O), precision="f32",
               int_arrays=dict(lab=lab), scales=scales)


@pytest.mark.parametrize("size", [(4, 3, 0, 2), (4, 3, 5, 0)])
def test_mlp2_ce_degenerate_widths_rejected(size):
    """An empty hidden or output layer with samples is refused with a named error before any
    launch (i_out = 0 leaves every label out of range, a BoundsError in the generated code)."""
    import torch
    import stade_hip
    B, I, H, O = size
    print(f"mlp2_ce_b degenerate B={B} I={I} H={H} O={O}", flush=True)
    f = lambda k: torch.zeros(k, dtype=torch.float32, device="cuda")
    lab = torch.ones(B, dtype=torch.int64, device="cuda")
    with pytest.raises(stade_hip.StadeHipError, match="i_h = 0|i_out = 0"):
        stade_hip.mlp2_ce_b(f(1), f(1), f(I * B), f(I * B), lab, f(H * I), f(H * I), f(H), f(H), f(O * H), f(O * H),
                            f(O), f(O), f(H * B), f(H * B), f(O * B), f(O * B), B, I, H, O)


@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("scale", [1e-4, 8.0, 30.0])
def test_mlp2_ce_tanh_regimes(mode, scale):
    """The forward epilogue's tanh (`tanh_f32` in csrc/mlp2_ce.hip: an odd polynomial below
    |s| = 0.625, 1 - 2/(exp(2|s|) + 1) above) against the oracle's libm tanhf with W1 and b1
    scaled so that one regime decides: 1e-4 keeps |s1| near 1e-3 (the polynomial alone), 8
    spreads |s1| over 0..20 (the exponential form and fp32 saturation at tanh = 1), 30 saturates
    most of the hidden layer, where 1 - h^2 and every W1/b1 sensitivity vanish."""
    from oracle import rng as jrng
    B, I, H, O = 64, 40, 96, 10
    sz = dict(loss=1, x=I * B, w1=H * I, b1=H, w2=O * H, b2=O, h1=H * B, z=O * B)
    shapes = {k + suf: v for k, v in sz.items() for suf in ("", "b", "d", "bd")}
    lab = np.array([1 + int(jrng.Xoshiro(23 + s).rand() * O) for s in range(B)], dtype=np.int64)
    g1, g2 = np.sqrt(2.0 / (I + H)) * scale, np.sqrt(2.0 / (H + O))
    bs = 0.1 * min(scale, 1.0)
    scales = {"w1": g1, "w1d": g1, "w2": g2, "w2d": g2, "b1": bs, "b2": 0.1}
    print(f"mlp2_ce_{mode} tanh regime: W1 scale {scale}", flush=True)
    run_parity("mlp2_ce", mode, shapes, dict(i_b=B, i_in=I, i_h=H, i_out=O), precision="f32",
               int_arrays=dict(lab=lab), scales=scales)
