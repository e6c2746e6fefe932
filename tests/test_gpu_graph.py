"""Entry points captured in a HIP graph (as bench.py issues the affine steps, and as a caller
running any of them in a loop would): every replay equals the eager call.

Each replay starts from the same inputs (restored by an eager copy between replays), runs
the captured calls, and is compared with the eager result; eager work and synchronisations
sit between the replays.  Kernels that sum in a fixed order are compared bit for bit; the
fp32 matrix-core paths, whose split products may add their K slices by atomics in the
hardware's order, within a normwise 1e-5 (a stale or skipped node would miss by far more)."""
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("mn", [(1024, 1024), (200, 77), (5000, 3)])
def test_affine_graph_replays_match_eager(mode, mn):
    import bench
    m, n = mn
    print(f"graph affine_lsq_{mode} {m}x{n}", flush=True)
    _replays_match_eager(bench.Affine(mode, m=m, n=n), exact=True)


# (family, workload constructor arguments, compared bit for bit)
OTHERS = [
    ("diffusion2d", dict(n=512), True),
    ("diffusion2d", dict(n=200), True),
    ("mlp2_ce", dict(B=512), False),
    ("conv3x3", dict(N=1, H=40, W=96), False),
]


@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("family,kw,exact", OTHERS, ids=[f"{f}-{'-'.join(map(str, k.values()))}" for f, k, _ in OTHERS])
def test_graph_replays_match_eager(family, kw, exact, mode):
    import bench
    cls = {"diffusion2d": bench.Diffusion, "mlp2_ce": bench.Mlp, "conv3x3": bench.Conv}[family]
    print(f"graph {family}_{mode} {kw}", flush=True)
    _replays_match_eager(cls(mode, **kw), exact=exact)


def _replays_match_eager(wl, exact: bool):
    import torch
    import stade_hip
    wl.setup(torch.device("cuda:0"))
    tensors = [a for a in wl.argv if isinstance(a, torch.Tensor)]
    saved = [t.clone() for t in tensors]

    def restore():
        for t, s in zip(tensors, saved):
            t.copy_(s)

    restore()
    wl.step()
    torch.cuda.synchronize()
    eager = [t.clone() for t in tensors]
    restore()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        wl.step()                      # warm-up off the capture (scratch sized here)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        wl.step()
    for rep in range(4):
        restore()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for k, (t, e) in enumerate(zip(tensors, eager)):
            if exact or not t.is_floating_point():
                assert torch.equal(t, e), f"replay {rep}: argument {k} differs from the eager call"
            else:
                err = (t.double() - e.double()).norm().item()
                assert err <= 1e-5 * max(e.double().norm().item(), 1e-30), \
                    f"replay {rep}: argument {k} differs from the eager call (normwise {err:.3e})"
        _ = torch.randn(1000, device="cuda").sum().item()   # eager work between replays
    assert stade_hip.device_error() == 0
