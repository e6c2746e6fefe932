"""The general lowering's contractions (stade_hip/lower/contract.py) on the GPU against the oracle.

The fp32 texts whose dense-layer loops become matrix products on the matrix cores: the MLP
config's three texts at sizes that are not multiples of the product's 128 x 64 x 16 tiles,
with inner sums long enough for a K split, the conv config's three texts (the table form:
gathered factors, atomic scatters into the input shadow), and two test texts with the other
storage orders (row-major weights with an offset into the input; flat loops that run the
batch fastest).
Every output against the oracle (the text as written, transpiled to C) to the fp32 bar with
the truth rule, as for every lowered text; each plan must hold the products."""
import numpy as np
import pytest

from helpers import CORPUS, ROOT, ParityCase, make_args

pytestmark = pytest.mark.gpu

TEXTS = ROOT / "tests" / "texts"
BUILD = ROOT / "tests" / "_build" / "texts"


def _run(path, name, mode, shapes, ints, int_arrays=None, scales=None, out_dir=None):
    from oracle import runner
    from stade_hip import lower
    lib_o = runner.load(path, precision="f32")
    fname = f"{name}_{mode}"
    args = make_args(lib_o, fname, dict(shapes), ints, {}, f"contract-{fname}-{ints}", np.float32, int_arrays, scales)
    low = lower.lower(path, "f32", out_dir=out_dir)
    plan = low.plan(fname)
    label = f"contracted {fname} {ints}"
    print(f"{label}: plan {plan}", flush=True)
    assert any("matrix product" in line for line in plan), plan

    def run(dev, stack_d):
        return low.call(fname, *dev, *stack_d)
    case = ParityCase(name, mode, args, (), "f32", label=label, runner=run, oracle_path=path)
    case.run_oracle(lib_o)
    case.run_gpu()
    print(f"{label}: worst {case.compare():.3e}", flush=True)


@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("size", [(257, 131, 70, 10), (96, 784, 256, 12), (1, 1, 1, 1)])
def test_contracted_mlp2_ce(mode, size):
    from oracle import rng as jrng
    B, I, H, O = size
    sz = dict(loss=1, x=I * B, w1=H * I, b1=H, w2=O * H, b2=O, h1=H * B, z=O * B)
    shapes = {k + s: v for k, v in sz.items() for s in ("", "b", "d", "bd")}
    lab = np.array([1 + int(jrng.Xoshiro(29 + s).rand() * O) for s in range(B)], dtype=np.int64)
    g1, g2 = np.sqrt(2.0 / (I + H)), np.sqrt(2.0 / (H + O))
    scales = {"w1": g1, "w1d": g1, "w2": g2, "w2d": g2, "b1": 0.1, "b2": 0.1}
    _run(CORPUS / f"mlp2_ce_{mode}.jl", "mlp2_ce", mode, shapes, dict(i_b=B, i_in=I, i_h=H, i_out=O),
         int_arrays=dict(lab=lab), scales=scales)


@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("size", [(1, 1, 1, 1, 1), (2, 3, 5, 7, 9), (2, 16, 20, 33, 17), (1, 64, 64, 40, 70)])
def test_contracted_conv3x3(mode, size):
    """The table form: both factors gathered through offset tables, the input shadow added
    atomically (its elements take several taps' products)."""
    N, C, K, H, W = size
    sz = dict(loss=1, xp=(W + 2) * (H + 2) * C * N, w=9 * C * K, out=W * H * K * N)
    shapes = {k + s: v for k, v in sz.items() for s in ("", "b", "d", "bd")}
    s = 1.0 / np.sqrt(9.0 * C)
    _run(CORPUS / f"conv3x3_{mode}.jl", "conv3x3", mode, shapes, dict(i_nb=N, i_c=C, i_k=K, i_h=H, i_w=W),
         scales={"w": s, "wd": s})


@pytest.mark.parametrize("text", ["dense_rm", "dense_bf"])
@pytest.mark.parametrize("bih", [(3, 5, 4), (257, 131, 70), (64, 600, 130), (0, 5, 4)])
def test_contracted_dense_layouts(text, bih):
    b, i, h = bih
    shapes = dict(y=b * h, x=b * i + 2, xb=b * i + 2, w=h * i, wb=h * i)
    _run(TEXTS / f"{text}_b.jl", "dense", "b", shapes, dict(i_b=b, i_in=i, i_h=h), out_dir=BUILD)
