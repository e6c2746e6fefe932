"""The library workspace under HIP graph capture.

A captured call keeps the addresses of the library's scratch buffer.  These tests check the
two rules that keep such a graph valid (`scratch()` in `stade.jl_amd/csrc/runtime.cpp`):
- a later, larger eager call retires the buffer a graph may hold instead of freeing it;
- a call that would have to grow the scratch while its stream is capturing is refused with
  STADE_HIP_ESTATE before it enqueues anything.

The scratch only grows within a process, and the full-size workloads of other test files grow
it to hundreds of megabytes.  This file's name sorts it before every other GPU test file, so
that its affine calls (scratch of 20 KB to a few MB) are the ones that grow it.  Run after
those files, the growth test is skipped, and says so."""
import pytest

pytestmark = pytest.mark.gpu


def affine_scratch_bytes(m: int, n: int) -> int:
    """The adjoint's scratch request in `stade_hip_affine_lsq_b` (`affine_lsq.hip`: 64 x 64
    tiles, at most 16 row-sum chunks per row): row partials, row sums and column partials."""
    ntiles, mtiles = -(-n // 64), -(-m // 64)
    tpc = -(-ntiles // 16)
    nchunks = -(-ntiles // tpc) if ntiles else 0
    return 8 * (nchunks * m + m + mtiles * n) + 256


def _capture(wl):
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        wl.step()                      # eager warm-up off the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        wl.step()
    return g


def test_graph_survives_a_later_scratch_growth():
    """Capture an affine adjoint at 300 x 200, grow the scratch with a larger eager adjoint,
    then replay: every replay equals the eager result, bit for bit (the adjoint's sums have a
    fixed order), and the workspace counts one retired buffer."""
    import torch
    import bench
    import stade_hip
    dev = torch.device("cuda:0")
    wl = bench.Affine("b", m=300, n=200)
    wl.setup(dev)
    tensors = [a for a in wl.argv if isinstance(a, torch.Tensor)]
    saved = [t.clone() for t in tensors]

    def restore():
        for t, s in zip(tensors, saved):
            t.copy_(s)
    wl.step()
    torch.cuda.synchronize()
    eager = [t.clone() for t in tensors]
    restore()
    g = _capture(wl)
    held0, retired0 = stade_hip.workspace_info()
    m = next((m for m in (1024, 2048, 4096, 8192) if affine_scratch_bytes(m, m) > held0), None)
    if m is None:
        pytest.skip(f"the workspace already holds {held0} bytes (grown by earlier tests); run this file first")
    big = bench.Affine("b", m=m, n=m)
    big.setup(dev)
    print(f"graph growth: eager affine_lsq_b {m}x{m} (scratch {held0} -> {affine_scratch_bytes(m, m)} bytes)", flush=True)
    big.step()
    torch.cuda.synchronize()
    held, retired = stade_hip.workspace_info()
    del big
    assert held >= affine_scratch_bytes(m, m) > held0
    assert retired == retired0 + 1, "the buffer the graph holds was not retired"
    for rep in range(3):
        restore()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for k, (t, e) in enumerate(zip(tensors, eager)):
            assert torch.equal(t, e), f"replay {rep} after the growth: argument {k} differs from the eager call"
        _ = torch.randn(1000, device="cuda").sum().item()   # eager work between replays
    assert stade_hip.device_error() == 0


def test_scratch_does_not_grow_under_capture():
    """An adjoint whose scratch exceeds what the workspace holds, captured without an eager
    call first: refused with the named error, and the workspace is unchanged."""
    import torch
    import bench
    import stade_hip
    dev = torch.device("cuda:0")
    held, _ = stade_hip.workspace_info()
    m = next((m for m in (512, 1024, 2048, 4096, 8192) if affine_scratch_bytes(m, m) > held), None)
    if m is None:
        pytest.skip(f"the workspace already holds {held} bytes (grown by earlier tests); run this file first")
    wl = bench.Affine("b", m=m, n=m)
    wl.setup(dev)
    torch.cuda.synchronize()
    print(f"capture refusal: affine_lsq_b {m}x{m} needs {affine_scratch_bytes(m, m)} bytes, {held} held", flush=True)
    g = torch.cuda.CUDAGraph()
    with pytest.raises(stade_hip.StadeHipError, match="cannot grow under graph capture"):
        with torch.cuda.graph(g):
            wl.step()
    torch.cuda.synchronize()
    assert stade_hip.workspace_info()[0] == held
    # and the same call made eagerly afterwards runs
    wl.step()
    torch.cuda.synchronize()
    assert stade_hip.device_error() == 0
