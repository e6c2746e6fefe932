"""stade_hip_diffusion2d_b_noalloc, the adjoint of diffusion2d without any allocation (its
reduction partials in a static device array), through the C ABI against
stade_hip_diffusion2d_b on the same inputs: two calls in a row, the second on a smaller grid,
and a third on another kernel path.  The two entry points share their kernels and their
summation order, so the results must be identical, bit for bit."""
import ctypes

import pytest

pytestmark = pytest.mark.gpu

P = ctypes.c_void_p


def _fn(name):
    import stade_hip
    f = getattr(stade_hip.lib(), name)
    f.restype = ctypes.c_int32
    f.argtypes = [P, P, P, P, P, P, ctypes.c_int64, P]
    return f


def _inputs(n, seed):
    import torch
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    r = lambda: torch.randn(n * n, generator=g, dtype=torch.float64, device="cuda")
    return dict(loss=torch.randn(1, generator=g, dtype=torch.float64, device="cuda"),
                lossb=torch.randn(1, generator=g, dtype=torch.float64, device="cuda"), u=r(), ub=r(), un=r(), unb=r())


def _run(fn, st, n):
    import stade_hip
    import torch
    args = [P(st[k].data_ptr()) for k in ("loss", "lossb", "u", "ub", "un", "unb")]
    rc = fn(*args, n, P(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, stade_hip.lib().stade_hip_last_error()


# 4096: the 128-column wave strips (2048 partials); 1000: the row-streaming kernel; 192: the
# 64-column wave strips
@pytest.mark.parametrize("sizes", [(4096, 1000, 192)])
def test_noalloc_matches_allocating_entry_point(sizes):
    import torch
    ref, new = _fn("stade_hip_diffusion2d_b"), _fn("stade_hip_diffusion2d_b_noalloc")
    for k, n in enumerate(sizes):
        print(f"diffusion2d_b_noalloc n={n} (call {k + 1})", flush=True)
        a = _inputs(n, 100 + k)
        b = {key: v.clone() for key, v in a.items()}
        _run(ref, a, n)
        _run(new, b, n)
        torch.cuda.synchronize()
        for key in ("loss", "ub", "un", "unb"):
            assert torch.equal(a[key], b[key]), f"n={n}: {key} differs between the two entry points"
        assert not torch.any(b["unb"]), "unb is reset"


def test_noalloc_calls_on_two_streams_are_ordered():
    """Two calls on two streams, issued back to back with no synchronisation between them,
    share the one static scratch array: the library orders the second after the first (the
    device's call lock and an event wait, as for every entry point), so each result equals the
    allocating entry point's on the same inputs, bit for bit."""
    import torch
    ref, new = _fn("stade_hip_diffusion2d_b"), _fn("stade_hip_diffusion2d_b_noalloc")
    n = 4096
    print(f"diffusion2d_b_noalloc n={n} on two streams", flush=True)
    ins = [_inputs(n, 200 + k) for k in range(2)]
    want = []
    for a in ins:
        w = {key: v.clone() for key, v in a.items()}
        _run(ref, w, n)
        want.append(w)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    for s, a in zip(streams, ins):
        with torch.cuda.stream(s):
            _run(new, a, n)
    torch.cuda.synchronize()
    for k, (a, w) in enumerate(zip(ins, want)):
        for key in ("loss", "ub", "un", "unb"):
            assert torch.equal(a[key], w[key]), f"call {k}: {key} differs from the allocating entry point"
