"""Why one fp32 output is judged by the truth rule: the conv tangent's `lossd` on the
(2, 70 -> 65, 6 x 33) parity case (`tests/test_gpu_conv.py`, the same seeded inputs).

`lossd = lossd0 + sum_q 0.5 * (2 out_q) * outd_q` is a sum of 25740 products whose signs
cancel: sum |terms| / |lossd| is above 3000 on these inputs. Each `out_q` and `outd_q` is
itself an fp32 sum over 630 taps, with a relative error of a few 1e-7 whatever the order, and
the cancellation multiplies that by the condition number. The tests below evaluate the text's
fp32 sums on the CPU in the text's own tap order (what the sequential oracle does: its error
against the fp64 value is 1.68e-6, as the GPU parity log records) and in other tap orders,
which any parallel evaluation uses (the GPU's matrix-core products take the taps in tiles):
the same arithmetic lands anywhere from 1e-7 to beyond 1e-5 from the fp64 value. The 1e-5
bar is therefore not a property of fp32 code for this output; the GPU's 1.17e-5 is judged
against the oracle's own error by the truth rule (`val_truth_verdict_lines`,
/root/reference/src/STADE.jl:18915-18932)."""
import numpy as np
import pytest

from helpers import make_args, oracle_lib

N, C, K, H, W = 2, 70, 65, 6, 33
f = np.float32


@pytest.fixture(scope="module")
def case():
    s = 1.0 / np.sqrt(9.0 * C)
    sz = dict(loss=1, xp=(W + 2) * (H + 2) * C * N, w=9 * C * K, out=W * H * K * N)
    shapes = {k + suf: v for k, v in sz.items() for suf in ("", "b", "d", "bd")}
    shapes["__stacks__"] = ()
    ints = dict(i_nb=N, i_c=C, i_k=K, i_h=H, i_w=W)
    lib = oracle_lib("conv3x3", "d", "f32")
    args = make_args(lib, "conv3x3_d", shapes, ints, {}, f"conv3x3_d-{ints}", np.float32, None, {"w": s, "wd": s})
    a = {name: v for name, _, v in args}

    # the taps t = 9 (ci - 1) + 3 (ky - 1) + kx of every output pixel, as the text indexes xp
    def taps(x):
        x = x.reshape(N, C, H + 2, W + 2)
        p = np.empty((N, C, 3, 3, H, W), np.float32)
        for ky in range(3):
            for kx in range(3):
                p[:, :, ky, kx] = x[:, :, ky:ky + H, kx:kx + W]
        return p.reshape(N, C * 9, H, W)

    px, pxd = taps(a["xp"]), taps(a["xpd"])
    wm, wdm = a["w"].reshape(K, C * 9), a["wd"].reshape(K, C * 9)
    d = np.float64
    out = np.einsum("kt,nthw->nkhw", wm.astype(d), px.astype(d))
    outd = np.einsum("kt,nthw->nkhw", wdm.astype(d), px.astype(d)) + np.einsum("kt,nthw->nkhw", wm.astype(d), pxd.astype(d))
    l0 = float(a["lossd"][0])
    return dict(px=px, pxd=pxd, wm=wm, wdm=wdm, out=out, outd=outd, l0=l0, truth=l0 + float(np.sum(out * outd)))


def fp32_taps(c, order, paired):
    """out and outd as fp32 sums over the taps in `order`: `paired` adds the text's
    (xp wd + w xpd) as one term, otherwise its two products are added one after the other (as
    two matrix-core products into one accumulator)."""
    s = np.zeros((N, K, H, W), f)
    sd = np.zeros((N, K, H, W), f)
    for t in order:
        x, xd = c["px"][:, t][:, None], c["pxd"][:, t][:, None]
        wt, wdt = c["wm"][:, t][None, :, None, None], c["wdm"][:, t][None, :, None, None]
        if paired:
            sd = f(sd + f(f(x * wdt) + f(wt * xd)))
        else:
            sd = f(f(sd + f(wt * xd)) + f(x * wdt))
        s = f(s + f(wt * x))
    return s, sd


def loss_seq(l0, out, outd):
    """The text's loss loop in fp32, in order."""
    acc = f(l0)
    for o, od in zip(out.ravel(), outd.ravel()):
        acc = f(acc + f(f(0.5) * f(f(2 * o) * od)))
    return float(acc)


def test_lossd_condition_number(case):
    terms = case["out"] * case["outd"]
    kappa = (abs(case["l0"]) + np.sum(np.abs(terms))) / abs(case["truth"])
    assert kappa > 3000, kappa


def test_text_order_reproduces_the_oracles_error(case):
    """The sequential evaluation (the oracle's) lands 1.68e-6 from the fp64 value, the figure
    the GPU parity log gives for the oracle on this case."""
    out, outd = fp32_taps(case, range(C * 9), paired=True)
    err = abs(loss_seq(case["l0"], out, outd) - case["truth"]) / abs(case["truth"])
    assert 1.5e-6 < err < 1.9e-6, err


def test_tap_order_alone_spans_the_bar(case):
    """Reordering the taps (and summing the products exactly afterwards, so that only the
    630-term sums differ) moves lossd from below 1e-6 to beyond 1e-5 of the fp64 value."""
    rng = np.random.default_rng(0)
    errs = []
    for _ in range(4):
        out, outd = fp32_taps(case, rng.permutation(C * 9), paired=False)
        lossd = case["l0"] + float(np.sum(out.astype(np.float64) * outd.astype(np.float64)))
        errs.append(abs(lossd - case["truth"]) / abs(case["truth"]))
    assert min(errs) < 1e-6 and max(errs) > 1e-5, errs
