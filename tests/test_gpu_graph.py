"""The affine entry points captured in a HIP graph (as bench.py issues them, and as a caller
running them in a loop would): every replay equals the eager call bit for bit.

Each replay starts from the same inputs (restored by an eager copy between replays), runs
the captured calls, and is compared with the eager result; eager work and synchronisations
sit between the replays.  The kernels sum in a fixed order, so equality is exact."""
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("mn", [(1024, 1024), (200, 77), (5000, 3)])
def test_affine_graph_replays_match_eager(mode, mn):
    import torch
    import stade_hip
    import bench
    m, n = mn
    print(f"graph affine_lsq_{mode} {m}x{n}", flush=True)
    wl = bench.Affine(mode, m=m, n=n)
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
            assert torch.equal(t, e), f"replay {rep}: argument {k} differs from the eager call"
        _ = torch.randn(1000, device="cuda").sum().item()   # eager work between replays
    assert stade_hip.device_error() == 0
