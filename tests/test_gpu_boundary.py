"""The boundary's own entry points on the GPU, through the C ABI: stacks allocated by
`stade_hip_initstacks_burgers1d_b` and released by `stade_hip_free`, the device error flag
for labels outside 1..i_out, and calls that share the workspace from two streams."""
import ctypes

import numpy as np
import pytest

from helpers import ParityCase, make_args, oracle_lib

pytestmark = pytest.mark.gpu


def test_initstacks_allocates_what_the_adjoint_fills():
    """initstacks_burgers1d_b's sizes through the C ABI (bit-exact lengths), the adjoint run
    on those library-allocated stacks against the oracle, then stade_hip_free."""
    import torch
    import stade_hip
    L = stade_hip.lib()
    n, T = 4097, 37
    L.stade_hip_initstacks_burgers1d_b.argtypes = [ctypes.c_int64, ctypes.c_int64,
                                                   ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_void_p)]
    L.stade_hip_initstacks_burgers1d_b.restype = ctypes.c_int32
    bs, us = ctypes.c_void_p(), ctypes.c_void_p()
    print(f"initstacks_burgers1d_b n={n} nsteps={T}", flush=True)
    assert L.stade_hip_initstacks_burgers1d_b(n, T, ctypes.byref(bs), ctypes.byref(us)) == 0
    assert bs.value and us.value
    lb, lu = stade_hip.burgers1d_stack_lengths(n, T)
    lib = oracle_lib("burgers1d", "b")
    ob, ou = lib.stacks("initstacks_burgers1d_b", n, T)
    assert (lb, lu) == (len(ob), len(ou)) == (T, T * n)
    shapes = {k: n for k in ("u", "ub", "un", "unb")}
    shapes.update(loss=1, lossb=1, __stacks__=("branch_stack", "u_stack"))
    args = make_args(lib, "burgers1d_b", shapes, dict(n=n, nsteps=T),
                     dict(nu=0.05, dt=0.002, dx=0.5, tend=10.0), "initstacks-abi")
    case = ParityCase("burgers1d", "b", args, (("branch_stack", (T, "Ai")), ("u_stack", (T * n, "Af"))), label="initstacks")
    case.run_oracle(lib)
    dev = {a: torch.from_numpy(np.ascontiguousarray(v)).to("cuda") for a, k, v in args if isinstance(v, np.ndarray)}
    F = ctypes.c_double
    sh = [F(v) for a, k, v in args if k == "f" and a.endswith("b")]
    argv, si = [], 0
    for a, k, v in args:
        if isinstance(v, np.ndarray):
            argv.append(ctypes.c_void_p(dev[a].data_ptr()))
        elif k == "i":
            argv.append(ctypes.c_int64(v))
        elif a.endswith("b"):
            argv.append(ctypes.byref(sh[si]))
            si += 1
        else:
            argv.append(F(v))
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert L.stade_hip_burgers1d_b(*argv, bs, us, stream) == 0, L.stade_hip_last_error()
    torch.cuda.synchronize()
    got_b = torch.empty(T, dtype=torch.int64, device="cuda")
    got_u = torch.empty(T * n, dtype=torch.float64, device="cuda")
    # copy out of the library's allocations through HIP (torch cannot wrap a raw pointer)
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    assert hip.hipMemcpy(got_b.data_ptr(), bs, 8 * T, 3) == 0
    assert hip.hipMemcpy(got_u.data_ptr(), us, 8 * T * n, 3) == 0
    for k, h in enumerate(case.ret_h):            # the returned scalar shadows
        assert abs(sh[k].value - h) <= 1e-12 * max(1.0, abs(h)), (k, sh[k].value, h)
    assert np.array_equal(got_b.cpu().numpy(), case.stack_h[0])
    e = np.max(np.abs(got_u.cpu().numpy() - case.stack_h[1])) / np.max(np.abs(case.stack_h[1]))
    assert e <= 1e-12, f"u_stack differs from the oracle by {e:.3e}"
    for (a, k, v), h in zip(args, case.host):
        if isinstance(v, np.ndarray) and np.any(h):
            g = dev[a].cpu().numpy()
            assert np.max(np.abs(g - h)) <= 1e-12 * np.max(np.abs(h)), a
    assert L.stade_hip_free(bs) == 0 and L.stade_hip_free(us) == 0
    assert L.stade_hip_free(None) == 0


@pytest.mark.parametrize("bad", [0, 4])
@pytest.mark.parametrize("mode", ["b", "d", "hv"])
def test_label_out_of_range_raises_with_check(mode, bad):
    """A label outside 1..i_out: check=True raises a BoundsError (the generated code's
    behaviour), the flag is then clear, and a valid call with check=True passes; without the
    check the call returns and the flag stays raised until read."""
    import torch
    import stade_hip
    B, I, H, O = 5, 4, 6, 3
    f = lambda k: torch.rand(k, dtype=torch.float32, device="cuda")
    lab = torch.tensor([1, 2, bad, 3, 1], dtype=torch.int64, device="cuda")
    good = torch.tensor([1, 2, 3, 3, 1], dtype=torch.int64, device="cuda")
    sz = dict(x=I * B, w1=H * I, b1=H, w2=O * H, b2=O, h1=H * B, z=O * B)

    def argv(labels):
        a = [f(1), f(1), f(sz["x"]), f(sz["x"]), labels]
        for k in ("w1", "b1", "w2", "b2", "h1", "z"):
            a += [f(sz[k]), f(sz[k])]
        a += [B, I, H, O]
        if mode == "hv":
            a += [f(1), f(1)] + [f(sz[k]) for k in ("x", "x", "w1", "w1", "b1", "b1", "w2", "w2", "b2", "b2", "h1", "h1", "z", "z")]
        return a
    fn = getattr(stade_hip, f"mlp2_ce_{mode}")
    print(f"mlp2_ce_{mode} label {bad} with check", flush=True)
    stade_hip.device_error()                       # start from a clear flag
    with pytest.raises(stade_hip.StadeHipBoundsError):
        fn(*argv(lab), check=True)
    assert not stade_hip.device_error()
    fn(*argv(good), check=True)
    fn(*argv(lab))                                 # inbounds: returns
    assert stade_hip.device_error()
    assert not stade_hip.device_error()


def test_calls_on_two_streams_are_ordered():
    """Two adjoints on two torch streams back to back share the library workspace (the loss
    partials); the second call's stream waits for the first's, so both losses are right."""
    import torch
    import stade_hip
    n = 2048
    g = torch.Generator(device="cuda")
    g.manual_seed(3)
    us = [torch.randn(n * n, generator=g, dtype=torch.float64, device="cuda") for _ in range(2)]
    want = []
    for u in us:
        un = u + 0.1 * (torch.roll(u.view(n, n), 1, 0) + torch.roll(u.view(n, n), -1, 0) + torch.roll(u.view(n, n), 1, 1)
                        + torch.roll(u.view(n, n), -1, 1) - 4 * u.view(n, n)).ravel()
        want.append(float((un * un).sum()))
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs = []
    torch.cuda.synchronize()
    print("diffusion2d_b on two streams", flush=True)
    for rep in range(3):
        res = []
        for u, s in zip(us, (s1, s2)):
            with torch.cuda.stream(s):
                z = lambda: torch.zeros(n * n, dtype=torch.float64, device="cuda")
                loss = torch.zeros(1, dtype=torch.float64, device="cuda")
                lossb = torch.ones(1, dtype=torch.float64, device="cuda")
                stade_hip.diffusion2d_b(loss, lossb, u, z(), z(), z(), n)
                res.append(loss)
        torch.cuda.synchronize()
        outs.append([float(r.item()) for r in res])
    for got in outs:
        for gv, wv in zip(got, want):
            assert abs(gv - wv) <= 1e-10 * abs(wv), (got, want)
