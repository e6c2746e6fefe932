"""bench.py's host side, on the CPU: every workload names arguments the generated text has,
and its CPU-baseline sample loads the oracle for a text that exists (a sample whose text is
missing would end the default benchmark run after the headline was measured)."""
from __future__ import annotations

import numpy as np
import pytest


def _bench():
    import bench
    return bench


@pytest.mark.parametrize("name", sorted(_bench().WORKLOADS))
def test_workload_cpu_sample_loads(name):
    b = _bench()
    wl = b.WORKLOADS[name]()
    run, desc, share = wl.cpu_sample()
    assert callable(run) and desc and 0.0 < share <= 1.0


@pytest.mark.parametrize("name", ["affine_lsq_b", "affine_lsq_d", "affine_lsq_hv"])
def test_affine_cpu_baseline_runs(name):
    """The affine samples are the full size and take milliseconds: run them end to end."""
    b = _bench()
    r = b.cpu_baseline(b.WORKLOADS[name](), budget_s=0.5, max_runs=3)
    assert r["value"] > 0 and r["cores"] == 1 and r["kind"] == "port"


@pytest.mark.parametrize("name", sorted(_bench().WORKLOADS))
def test_workload_inputs_cover_the_generated_arguments(name):
    b = _bench()
    wl = b.WORKLOADS[name]()
    if wl.family in ("burgers1d", "conv3x3", "mlp2_ce", "diffusion2d"):
        # the full-size inputs take seconds to draw; the argument names come from the text
        wl = {"burgers1d": lambda: type(wl)(wl.mode, n=64, nsteps=3),
              "conv3x3": lambda: b.Conv(wl.mode, N=1, C=4, K=4, H=8, W=8),
              "mlp2_ce": lambda: b.Mlp(wl.mode, B=8, I=6, H=5, O=3),
              "diffusion2d": lambda: b.Diffusion(wl.mode, n=8)}[wl.family]()
    h = wl.host_inputs()
    names = b.arg_names(wl.family, wl.mode)
    nst = len(wl.stack_lengths()) if wl.mode != "d" else 0
    for a in names[:len(names) - nst]:
        assert a in h, f"{name}: no input for argument {a}"
        assert isinstance(h[a], (np.ndarray, int, float)), f"{name}: {a} is {type(h[a])}"
