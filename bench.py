"""Gradient evaluations per second of STADE-generated derivative code on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--only NAME]
                    [--no-cpu-baseline]

A step is one evaluation of a generated function (`<k>_b`, `<k>_d` or `<k>_hv`) through the
C ABI of libstade_hip.so on synthetic inputs already resident in HBM.  The headline line is
the workload BASELINE.json quotes its metric on (configs[1], the diffusion adjoint on a
4096 x 4096 fp64 grid); every other implemented config is measured with the same protocol
and reported under "configs".

Timing: the K timed steps run with nothing added to the stream (value, ms_per_step); then the
same K steps run again with the library's profiler on (stade_hip_profile_*: a HIP event pair
recorded around every launch on the launch's own stream), and the dominant kernel's mean
launch duration comes from that pass.  Roofline achieved = algorithmic bytes (or flops) per
launch / that duration.  Algorithmic bytes
count each array element the generated function's contract reads once, each written once,
each read-modify-write twice; scalars and length-1 arrays are ignored.

CPU baseline: the same generated text run by the oracle (oracle/jl2c.py transpiled to C,
gcc -O2, one thread pinned to one core), on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "stade.jl_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3
FP64_PEAK_TFLOPS = 78.6


def _tensor(a, dev):
    import numpy as np
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


class Workload:
    name = ""
    kernel = ""           # dominant kernel (profiler name)
    bound = "hbm"
    dtype = "f64"

    def setup(self, dev):
        raise NotImplementedError

    def step(self):
        raise NotImplementedError

    def algo_bytes(self) -> float:          # per evaluation
        return 0.0

    def kernel_bytes(self) -> float:        # per launch of the dominant kernel
        return 0.0

    def kernel_flops(self) -> float:
        return 0.0

    def config(self) -> dict:
        return {}

    def cpu_sample(self):
        """(callable running one evaluation of the oracle, description); None if unavailable."""
        return None


class Diffusion(Workload):
    dtype = "f64"

    def __init__(self, mode="b", n=4096):
        self.mode, self.n = mode, n
        self.name = f"diffusion2d_{mode}"
        self.kernel = f"diffusion2d_{mode}"

    def setup(self, dev):
        import numpy as np
        import torch
        import stade_hip
        n = self.n
        c = n * n
        rng = stade_hip.api.Rng(stade_hip.stable_seed("diffusion2d"))
        u = stade_hip.rng_normal(rng, c)
        z = lambda: torch.zeros(c, dtype=torch.float64, device=dev)
        self.t = dict(loss=torch.zeros(1, dtype=torch.float64, device=dev),
                      lossb=torch.ones(1, dtype=torch.float64, device=dev),
                      lossd=torch.zeros(1, dtype=torch.float64, device=dev),
                      lossbd=torch.zeros(1, dtype=torch.float64, device=dev),
                      u=_tensor(u, dev), ub=z(), un=z(), unb=z(), und=z(), unbd=z(), ubd=z())
        if self.mode in ("d", "hv"):
            rng2 = stade_hip.api.Rng(stade_hip.stable_seed("diffusion2d") + 1)
            self.t["ud"] = _tensor(stade_hip.rng_normal(rng2, c), dev)
        self.host_u = u

    def step(self):
        import stade_hip
        t, n = self.t, self.n
        if self.mode == "b":
            stade_hip.diffusion2d_b(t["loss"], t["lossb"], t["u"], t["ub"], t["un"], t["unb"], n)
        elif self.mode == "d":
            stade_hip.diffusion2d_d(t["loss"], t["lossd"], t["u"], t["ud"], t["un"], t["und"], n)
        else:
            stade_hip.diffusion2d_hv(t["loss"], t["lossb"], t["u"], t["ub"], t["un"], t["unb"], n,
                                     t["lossd"], t["lossbd"], t["ud"], t["ubd"], t["und"], t["unbd"])

    def algo_bytes(self):
        per = {"b": 48, "d": 32, "hv": 96}[self.mode]
        return per * self.n * self.n

    def kernel_bytes(self):
        # pass 1 of the adjoint: u R, un W, unb R, ub R+W (unb's reset is pass 2)
        per = {"b": 40, "d": 32, "hv": 80}[self.mode]
        return per * self.n * self.n

    def config(self):
        return {"workload": f"diffusion2d_{self.mode} (STADE {'adjoint' if self.mode == 'b' else 'tangent' if self.mode == 'd' else 'HVP'}), "
                            f"periodic 5-point step + sum(un^2), {self.n}x{self.n} fp64, u ~ N(0,1) from val_stable_seed",
                "n": self.n, "cells": self.n * self.n}

    def cpu_sample(self):
        import numpy as np
        from oracle import runner
        lib = runner.load(ROOT / "stade.jl_amd" / "corpus" / f"diffusion2d_{self.mode}.jl", bounds_check=False)
        n, c = self.n, self.n * self.n
        u = self.host_u.copy()
        z = lambda: np.zeros(c)
        a = dict(ub=z(), un=z(), unb=z(), ud=np.ones(c), und=z(), ubd=z(), unbd=z())

        def run():
            if self.mode == "b":
                lib.call("diffusion2d_b", np.zeros(1), np.ones(1), u, a["ub"], a["un"], a["unb"], n)
            elif self.mode == "d":
                lib.call("diffusion2d_d", np.zeros(1), np.zeros(1), u, a["ud"], a["un"], a["und"], n)
            else:
                lib.call("diffusion2d_hv", np.zeros(1), np.ones(1), u, a["ub"], a["un"], a["unb"], n,
                         np.zeros(1), np.zeros(1), a["ud"], a["ubd"], a["und"], a["unbd"])
        return run, f"diffusion2d_{self.mode} at the full {n}x{n} grid"


class Affine(Workload):
    dtype = "f64"

    def __init__(self, mode="b", m=1024, n=1024):
        self.mode, self.m, self.n = mode, m, n
        self.name = f"affine_lsq_{mode}"
        self.kernel = "affine_cols" if mode != "d" else "affine_rows"

    def setup(self, dev):
        import torch
        import stade_hip
        m, n = self.m, self.n
        rng = stade_hip.api.Rng(stade_hip.stable_seed("affine_lsq"))
        w = stade_hip.rng_uniform(rng, m * n, -1.0, 1.0)
        x, b, t = (stade_hip.rng_normal(rng, k) for k in (n, m, m))
        rng2 = stade_hip.api.Rng(stade_hip.stable_seed("affine_lsq") + 1)
        wd, xd, bd, td = (stade_hip.rng_normal(rng2, k) for k in (m * n, n, m, m))
        f = lambda a: _tensor(a, dev)
        z = lambda k: torch.zeros(k, dtype=torch.float64, device=dev)
        self.t = dict(loss=z(1), lossb=f([1.0]), lossd=z(1), lossbd=z(1), w=f(w), wb=z(m * n), x=f(x), xb=z(n),
                      b=f(b), bb=z(m), t=f(t), tb=z(m), r=z(m), rb=z(m), wd=f(wd), wbd=z(m * n), xd=f(xd), xbd=z(n),
                      bd=f(bd), bbd=z(m), td=f(td), tbd=z(m), rd=z(m), rbd=z(m))

    def step(self):
        import stade_hip
        t, m, n = self.t, self.m, self.n
        base = [t[k] for k in ("loss",)]
        if self.mode == "b":
            stade_hip.affine_lsq_b(t["loss"], t["lossb"], t["w"], t["wb"], t["x"], t["xb"], t["b"], t["bb"], t["t"], t["tb"],
                                   t["r"], t["rb"], m, n)
        elif self.mode == "d":
            stade_hip.affine_lsq_d(t["loss"], t["lossd"], t["w"], t["wd"], t["x"], t["xd"], t["b"], t["bd"], t["t"], t["td"],
                                   t["r"], t["rd"], m, n)
        else:
            stade_hip.affine_lsq_hv(t["loss"], t["lossb"], t["w"], t["wb"], t["x"], t["xb"], t["b"], t["bb"], t["t"], t["tb"],
                                    t["r"], t["rb"], m, n, t["lossd"], t["lossbd"], t["wd"], t["wbd"], t["xd"], t["xbd"],
                                    t["bd"], t["bbd"], t["td"], t["tbd"], t["rd"], t["rbd"])
        del base

    def algo_bytes(self):
        mn, m, n = self.m * self.n, self.m, self.n
        if self.mode == "b":   # w R, wb RW, x R, xb RW, b R, bb RW, t R, tb RW, r W, rb RW
            return 8 * (3 * mn + 3 * n + 9 * m)
        if self.mode == "d":   # w, wd R; x, xd R; b, bd, t, td R; r, rd W
            return 8 * (2 * mn + 2 * n + 6 * m)
        return 8 * (6 * mn + 6 * n + 18 * m)

    def kernel_bytes(self):
        mn = self.m * self.n
        return 8 * {"b": 3 * mn, "d": 2 * mn, "hv": 6 * mn}[self.mode]

    def config(self):
        return {"workload": f"affine_lsq_{self.mode}, loss = 0.5*sum((W*x+b-t)^2), W {self.m}x{self.n} fp64 U[-1,1]",
                "m": self.m, "n": self.n}


class Burgers(Workload):
    """Config 5: 2^20 periodic cells, 500 guarded steps, nu = 1e-3, dx = 1/n, dt such that
    nu dt / dx^2 = 0.2; u0 = sin(2 pi x) + 0.1 N(0,1), x_i = (i - 1) / n; tend = 1 (every
    step runs)."""
    dtype = "f64"

    def __init__(self, mode="b", n=1 << 20, nsteps=500):
        self.mode, self.n, self.T = mode, n, nsteps
        self.name = f"burgers1d_{mode}"
        self.kernel = {"b": "burgers1d_bwd", "d": "burgers1d_fwd_hv", "hv": "burgers1d_bwd_hv"}[mode]
        self.nu = 1e-3
        self.dx = 1.0 / n
        self.dt = 0.2 * self.dx * self.dx / self.nu
        self.tend = 1.0

    def _u0(self):
        import numpy as np
        import stade_hip
        n = self.n
        x = np.arange(n, dtype=np.float64) / n
        rng = stade_hip.api.Rng(stade_hip.stable_seed("burgers1d"))
        return np.sin(2.0 * np.pi * x) + 0.1 * stade_hip.rng_normal(rng, n)

    def setup(self, dev):
        import torch
        import stade_hip
        n = self.n
        self.host_u = self._u0()
        rng2 = stade_hip.api.Rng(stade_hip.stable_seed("burgers1d") + 1)
        ud = stade_hip.rng_normal(rng2, n)
        z = lambda: torch.zeros(n, dtype=torch.float64, device=dev)
        self.t = dict(loss=torch.zeros(1, dtype=torch.float64, device=dev), lossb=torch.ones(1, dtype=torch.float64, device=dev),
                      lossd=torch.zeros(1, dtype=torch.float64, device=dev), lossbd=torch.zeros(1, dtype=torch.float64, device=dev),
                      u=_tensor(self.host_u, dev), ub=z(), un=z(), unb=z(), ud=_tensor(ud, dev), ubd=z(), und=z(), unbd=z())
        if self.mode != "d":
            self.stacks = stade_hip.initstacks_burgers1d_b(n, self.T, dev)

    def step(self):
        import stade_hip
        t, n, T = self.t, self.n, self.T
        if self.mode == "b":
            stade_hip.burgers1d_b(t["loss"], t["lossb"], t["u"], t["ub"], t["un"], t["unb"], self.nu, 0.0, self.dt, 0.0,
                                  self.dx, 0.0, self.tend, 0.0, n, T, *self.stacks)
        elif self.mode == "d":
            stade_hip.burgers1d_d(t["loss"], t["lossd"], t["u"], t["ud"], t["un"], t["und"], self.nu, 0.01, self.dt, 0.0,
                                  self.dx, 0.0, self.tend, 0.0, n, T)
        else:
            stade_hip.burgers1d_hv(t["loss"], t["lossb"], t["u"], t["ub"], t["un"], t["unb"], self.nu, 0.0, self.dt, 0.0,
                                   self.dx, 0.0, self.tend, 0.0, n, T, t["lossd"], t["lossbd"], t["ud"], t["ubd"], t["und"],
                                   t["unbd"], 0.01, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, *self.stacks)

    def _launches(self):
        return -(-self.T // 32)

    def algo_bytes(self):
        n, T = self.n, self.T
        if self.mode == "b":   # tape W + R, u R, un W, ub RW, unb RW
            return 8 * (2 * T * n + 6 * n)
        if self.mode == "d":   # u, ud R+W (advanced in place), un, und W
            return 8 * (6 * n)
        return 8 * (4 * T * n + 12 * n)

    def kernel_bytes(self):
        # per launch of the dominant kernel, averaged over the chunks: the tape rows it moves
        # plus one read and one write of its state vectors
        n, T, L = self.n, self.T, self._launches()
        if self.mode == "b":
            return 8 * (T * n + 2 * n * L) / L
        if self.mode == "d":
            return 8 * (4 * n * L) / L
        return 8 * (2 * T * n + 4 * n * L) / L

    def config(self):
        return {"workload": f"burgers1d_{self.mode}: 1-D viscous Burgers, {self.n} periodic cells fp64, {self.T} steps in a "
                            f"counted loop with a guard, nu=1e-3, u0=sin(2 pi x)+0.1 N(0,1), loss=sum(u_T^2)",
                "n": self.n, "nsteps": self.T, "tape_bytes": 8 * self.T * self.n}

    def cpu_sample(self):
        import numpy as np
        from oracle import runner
        Ts = 20
        lib = runner.load(ROOT / "stade.jl_amd" / "corpus" / f"burgers1d_{self.mode}.jl", bounds_check=False)
        n = self.n
        scale = Ts / self.T

        def run():
            u = self.host_u.copy()
            z = lambda: np.zeros(n)
            if self.mode == "d":
                lib.call("burgers1d_d", np.zeros(1), np.zeros(1), u, np.ones(n), z(), z(), self.nu, 0.01, self.dt, 0.0,
                         self.dx, 0.0, self.tend, 0.0, n, Ts)
            else:
                st = lib.stacks("initstacks_burgers1d_b", n, Ts, fill_nan=False)
                if self.mode == "b":
                    lib.call("burgers1d_b", np.zeros(1), np.ones(1), u, z(), z(), z(), self.nu, 0.0, self.dt, 0.0, self.dx, 0.0,
                             self.tend, 0.0, n, Ts, *st)
                else:
                    lib.call("burgers1d_hv", np.zeros(1), np.ones(1), u, z(), z(), z(), self.nu, 0.0, self.dt, 0.0, self.dx, 0.0,
                             self.tend, 0.0, n, Ts, np.zeros(1), np.zeros(1), np.ones(n), z(), z(), z(), 0.01, 0.0, 0.0, 0.0,
                             0.0, 0.0, 0.0, 0.0, *st)
        return run, f"burgers1d_{self.mode} on {n} cells for {Ts} of the {self.T} steps (time x {1/scale:.0f})", scale


class Mlp(Workload):
    """Config 3: x (784, 4096) ~ U[0,1], tanh hidden layer of 1024, 10-way softmax
    cross-entropy, Float32; W1, W2 Glorot-uniform U(+-sqrt(6 / (fan_in + fan_out))),
    b1 = b2 = 0, labels uniform in 1..10, HVP direction (xd, W1d, b1d, W2d, b2d) ~ N(0,1) --
    all from the seeded Xoshiro stream."""
    dtype = "f32"
    bound = "mfma"

    def __init__(self, mode="b", B=4096, I=784, H=1024, O=10):
        self.mode, self.B, self.I, self.H, self.O = mode, B, I, H, O
        self.name = f"mlp2_ce_{mode}"
        g = 2.0 * H * I * B
        # flops per launch of each matrix-core kernel: the tangent and HVP run each pair
        # (s1, s1d), (W1b, W1bd), (xb, xbd) as one dual launch of three products
        self.kernels = {"b": {"mlp_gemm_s1": g, "mlp_gemm_w1b": g, "mlp_gemm_xb": g},
                        "d": {"mlp_gemm_s1d": 3 * g},
                        "hv": {"mlp_gemm_s1d": 3 * g, "mlp_gemm_w1bd": 3 * g, "mlp_gemm_xbd": 3 * g}}[mode]
        self.kernel = next(iter(self.kernels))

    def _host(self, B):
        import numpy as np
        import stade_hip
        I, H, O = self.I, self.H, self.O
        rng = stade_hip.api.Rng(stade_hip.stable_seed("mlp2_ce"))
        x = stade_hip.rng_uniform(rng, I * B, 0.0, 1.0).astype(np.float32)
        a1, a2 = np.sqrt(6.0 / (I + H)), np.sqrt(6.0 / (H + O))
        w1 = stade_hip.rng_uniform(rng, H * I, -a1, a1).astype(np.float32)
        w2 = stade_hip.rng_uniform(rng, O * H, -a2, a2).astype(np.float32)
        b1, b2 = np.zeros(H, dtype=np.float32), np.zeros(O, dtype=np.float32)
        lab = stade_hip.rng_int_range(rng, B, 1, O)
        rng2 = stade_hip.api.Rng(stade_hip.stable_seed("mlp2_ce") + 1)
        d = {k: stade_hip.rng_normal(rng2, n).astype(np.float32)
             for k, n in (("xd", I * B), ("w1d", H * I), ("b1d", H), ("w2d", O * H), ("b2d", O))}
        return dict(x=x, w1=w1, b1=b1, w2=w2, b2=b2, lab=lab, **d)

    def setup(self, dev):
        import torch
        B, I, H, O = self.B, self.I, self.H, self.O
        h = self._host(B)
        f = lambda a: _tensor(a, dev)
        z = lambda k: torch.zeros(k, dtype=torch.float32, device=dev)
        t = {k: f(v) for k, v in h.items()}
        t.update(loss=z(1), lossb=f([1.0]).float(), lossd=z(1), lossbd=z(1))
        for k, n in (("x", I * B), ("w1", H * I), ("b1", H), ("w2", O * H), ("b2", O), ("h1", H * B), ("z", O * B)):
            for suf in ("b", "bd") if k not in ("h1", "z") else ("", "b", "d", "bd"):
                t.setdefault(k + suf, z(n))
        self.t = t

    def step(self):
        import stade_hip
        t = self.t
        sz = (self.B, self.I, self.H, self.O)
        if self.mode == "b":
            stade_hip.mlp2_ce_b(*(t[k] for k in ("loss", "lossb", "x", "xb", "lab", "w1", "w1b", "b1", "b1b", "w2", "w2b",
                                                "b2", "b2b", "h1", "h1b", "z", "zb")), *sz)
        elif self.mode == "d":
            stade_hip.mlp2_ce_d(*(t[k] for k in ("loss", "lossd", "x", "xd", "lab", "w1", "w1d", "b1", "b1d", "w2", "w2d",
                                                "b2", "b2d", "h1", "h1d", "z", "zd")), *sz)
        else:
            stade_hip.mlp2_ce_hv(*(t[k] for k in ("loss", "lossb", "x", "xb", "lab", "w1", "w1b", "b1", "b1b", "w2", "w2b",
                                                 "b2", "b2b", "h1", "h1b", "z", "zb")), *sz,
                                 *(t[k] for k in ("lossd", "lossbd", "xd", "xbd", "w1d", "w1bd", "b1d", "b1bd", "w2d", "w2bd",
                                                  "b2d", "b2bd", "h1d", "h1bd", "zd", "zbd")))

    def eval_flops(self):
        B, I, H, O = self.B, self.I, self.H, self.O
        return sum(self.kernels.values()) * 1.0 + {"b": 2, "d": 2, "hv": 4}[self.mode] * 2.0 * O * H * B

    def config(self):
        return {"workload": f"mlp2_ce_{self.mode}: x {self.I}x{self.B} fp32 U[0,1] -> tanh({self.H}) -> {self.O}-way softmax "
                            f"cross-entropy summed over the batch; Glorot-uniform weights, zero biases",
                "batch": self.B, "widths": [self.I, self.H, self.O]}

    def cpu_sample(self):
        import numpy as np
        from oracle import runner
        Bs = 128
        lib = runner.load(ROOT / "stade.jl_amd" / "corpus" / f"mlp2_ce_{self.mode}.jl", precision="f32", bounds_check=False)
        h = self._host(Bs)
        I, H, O = self.I, self.H, self.O
        z = lambda k: np.zeros(k, dtype=np.float32)
        one = np.ones(1, dtype=np.float32)

        def run():
            if self.mode == "b":
                lib.call("mlp2_ce_b", z(1), one, h["x"], z(I * Bs), h["lab"], h["w1"], z(H * I), h["b1"], z(H), h["w2"],
                         z(O * H), h["b2"], z(O), z(H * Bs), z(H * Bs), z(O * Bs), z(O * Bs), Bs, I, H, O)
            elif self.mode == "d":
                lib.call("mlp2_ce_d", z(1), z(1), h["x"], h["xd"], h["lab"], h["w1"], h["w1d"], h["b1"], h["b1d"], h["w2"],
                         h["w2d"], h["b2"], h["b2d"], z(H * Bs), z(H * Bs), z(O * Bs), z(O * Bs), Bs, I, H, O)
            else:
                lib.call("mlp2_ce_hv", z(1), one, h["x"], z(I * Bs), h["lab"], h["w1"], z(H * I), h["b1"], z(H), h["w2"],
                         z(O * H), h["b2"], z(O), z(H * Bs), z(H * Bs), z(O * Bs), z(O * Bs), Bs, I, H, O,
                         z(1), z(1), h["xd"], z(I * Bs), h["w1d"], z(H * I), h["b1d"], z(H), h["w2d"], z(O * H), h["b2d"], z(O),
                         z(H * Bs), z(H * Bs), z(O * Bs), z(O * Bs))
        return run, f"mlp2_ce_{self.mode} on {Bs} of the {self.B} samples (time x {self.B // Bs})", Bs / self.B


class Conv(Workload):
    """Config 4: 8 images of 256 x 256, 64 -> 64 channels, 3 x 3, zero border held in xp,
    Float32; xp interior ~ N(0,1), w He-normal N(0, 2 / (9 C)); tangent / HVP direction
    xpd (interior), wd the same laws -- from the seeded Xoshiro stream."""
    dtype = "f32"
    bound = "mfma"

    def __init__(self, mode="b", N=8, C=64, K=64, H=256, W=256):
        self.mode, self.N, self.C, self.K, self.H, self.W = mode, N, C, K, H, W
        self.name = f"conv3x3_{mode}"
        g = 2.0 * N * K * H * W * 9 * C
        self.kernels = {"b": {"conv_fwd": g, "conv_wgrad": g, "conv_dgrad": g},
                        "d": {"conv_fwd_d": 3 * g},
                        "hv": {"conv_fwd_hv": 3 * g, "conv_wgrad": g, "conv_wgrad2": 2 * g, "conv_dgrad_hv": 3 * g}}[mode]
        self.kernel = next(iter(self.kernels))

    def _host(self, N, H):
        import numpy as np
        import stade_hip
        C, K, W = self.C, self.K, self.W
        rng = stade_hip.api.Rng(stade_hip.stable_seed("conv3x3"))
        xp = np.zeros((N, C, H + 2, W + 2), dtype=np.float32)
        xp[:, :, 1:-1, 1:-1] = stade_hip.rng_normal(rng, N * C * H * W).reshape(N, C, H, W)
        w = (stade_hip.rng_normal(rng, 9 * C * K) * np.sqrt(2.0 / (9.0 * C))).astype(np.float32)
        rng2 = stade_hip.api.Rng(stade_hip.stable_seed("conv3x3") + 1)
        xpd = np.zeros_like(xp)
        xpd[:, :, 1:-1, 1:-1] = stade_hip.rng_normal(rng2, N * C * H * W).reshape(N, C, H, W)
        wd = (stade_hip.rng_normal(rng2, 9 * C * K) * np.sqrt(2.0 / (9.0 * C))).astype(np.float32)
        return dict(xp=xp.ravel(), w=w, xpd=xpd.ravel(), wd=wd)

    def setup(self, dev):
        import torch
        N, C, K, H, W = self.N, self.C, self.K, self.H, self.W
        h = self._host(N, H)
        f = lambda a: _tensor(a, dev)
        z = lambda k: torch.zeros(k, dtype=torch.float32, device=dev)
        nx, nw, no = N * C * (H + 2) * (W + 2), 9 * C * K, N * K * H * W
        self.t = {k: f(v) for k, v in h.items()}
        self.t.update(loss=z(1), lossb=f([1.0]).float(), lossd=z(1), lossbd=z(1), xpb=z(nx), xpbd=z(nx), wb=z(nw), wbd=z(nw),
                      out=z(no), outb=z(no), outd=z(no), outbd=z(no))

    def step(self):
        import stade_hip
        t = self.t
        sz = (self.N, self.C, self.K, self.H, self.W)
        if self.mode == "b":
            stade_hip.conv3x3_b(*(t[k] for k in ("loss", "lossb", "xp", "xpb", "w", "wb", "out", "outb")), *sz)
        elif self.mode == "d":
            stade_hip.conv3x3_d(*(t[k] for k in ("loss", "lossd", "xp", "xpd", "w", "wd", "out", "outd")), *sz)
        else:
            stade_hip.conv3x3_hv(*(t[k] for k in ("loss", "lossb", "xp", "xpb", "w", "wb", "out", "outb")), *sz,
                                 *(t[k] for k in ("lossd", "lossbd", "xpd", "xpbd", "wd", "wbd", "outd", "outbd")))

    def eval_flops(self):
        return sum(self.kernels.values()) * 1.0

    def config(self):
        return {"workload": f"conv3x3_{self.mode}: {self.N} x {self.C} x {self.H} x {self.W} fp32 input (zero border "
                            f"held in xp), 3x3 {self.C}->{self.K}, loss = 0.5 sum(out^2)",
                "batch": self.N, "channels": [self.C, self.K], "image": [self.H, self.W]}

    def cpu_sample(self):
        import numpy as np
        from oracle import runner
        Ns, Hs = 1, 32
        lib = runner.load(ROOT / "stade.jl_amd" / "corpus" / f"conv3x3_{self.mode}.jl", precision="f32", bounds_check=False)
        h = self._host(Ns, Hs)
        C, K, W = self.C, self.K, self.W
        nx, nw, no = Ns * C * (Hs + 2) * (W + 2), 9 * C * K, Ns * K * Hs * W
        z = lambda k: np.zeros(k, dtype=np.float32)
        one = np.ones(1, dtype=np.float32)
        sz = (Ns, C, K, Hs, W)

        def run():
            if self.mode == "b":
                lib.call("conv3x3_b", z(1), one, h["xp"], z(nx), h["w"], z(nw), z(no), z(no), *sz)
            elif self.mode == "d":
                lib.call("conv3x3_d", z(1), z(1), h["xp"], h["xpd"], h["w"], h["wd"], z(no), z(no), *sz)
            else:
                lib.call("conv3x3_hv", z(1), one, h["xp"], z(nx), h["w"], z(nw), z(no), z(no), *sz,
                         z(1), z(1), h["xpd"], z(nx), h["wd"], z(nw), z(no), z(no))
        share = (Ns * Hs) / (self.N * self.H)
        return run, (f"conv3x3_{self.mode} on {Ns} of the {self.N} images, {Hs} of the {self.H} rows "
                     f"(time x {1 / share:.0f})"), share


WORKLOADS = {
    "diffusion2d_b": lambda: Diffusion("b"),
    "diffusion2d_d": lambda: Diffusion("d"),
    "diffusion2d_hv": lambda: Diffusion("hv"),
    "affine_lsq_b": lambda: Affine("b"),
    "affine_lsq_d": lambda: Affine("d"),
    "affine_lsq_hv": lambda: Affine("hv"),
    "burgers1d_b": lambda: Burgers("b"),
    "burgers1d_d": lambda: Burgers("d"),
    "burgers1d_hv": lambda: Burgers("hv"),
    "mlp2_ce_b": lambda: Mlp("b"),
    "mlp2_ce_d": lambda: Mlp("d"),
    "mlp2_ce_hv": lambda: Mlp("hv"),
    "conv3x3_b": lambda: Conv("b"),
    "conv3x3_d": lambda: Conv("d"),
    "conv3x3_hv": lambda: Conv("hv"),
}
HEADLINE = "diffusion2d_b"


def _lib():
    import stade_hip
    L = stade_hip.lib()
    L.stade_hip_profile_read.argtypes = [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int64)]
    return L


def profiled_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from its committed counter summary
    (profiles/<kernel>_traffic.md: FETCH_SIZE and WRITE_SIZE per dispatch, each scaled by what
    the same counter reads for a 1 GiB copy), or None when there is none."""
    import re
    f = ROOT / "profiles" / f"{kernel}_traffic.md"
    if not f.exists():
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*(\d+)", f.read_text(), re.M)
    return int(m.group(1)) if m else None


def measure(wl: Workload, steps: int, warmup: int, dev) -> dict:
    import torch
    L = _lib()
    wl.setup(dev)
    for _ in range(warmup):
        wl.step()
    torch.cuda.synchronize()
    # pass 1, the timed region: K steps with nothing added to the stream
    t0 = time.perf_counter()
    for _ in range(steps):
        wl.step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    # pass 2: the same K steps with the library's profiler on (a HIP event pair around every
    # launch, on the launch's stream); only the per-launch kernel durations are taken from it,
    # since the event pairs themselves add ~14 us per diffusion step
    L.stade_hip_profile_start()
    for _ in range(steps):
        wl.step()
    torch.cuda.synchronize()
    tot, cnt = ctypes.c_double(0), ctypes.c_int64(0)
    per_kernel = {}
    if getattr(wl, "kernels", None):
        # the dominant kernel: the matrix-core launch with the largest total time
        best = None
        for k in wl.kernels:
            t_, c_ = ctypes.c_double(0), ctypes.c_int64(0)
            L.stade_hip_profile_read(k.encode(), ctypes.byref(t_), ctypes.byref(c_))
            if c_.value:
                per_kernel[k] = {"ms": t_.value / c_.value, "launches": c_.value,
                                 "tflops": wl.kernels[k] / (t_.value / c_.value * 1e-3) / 1e12}
                if best is None or t_.value > best[1]:
                    best = (k, t_.value, c_.value)
        if best:
            wl.kernel = best[0]
            tot.value, cnt.value = best[1], best[2]
    else:
        L.stade_hip_profile_read(wl.kernel.encode(), ctypes.byref(tot), ctypes.byref(cnt))
    L.stade_hip_profile_stop()
    ms_step = (t1 - t0) * 1e3 / steps
    out = {"evals_per_s": steps / (t1 - t0), "ms_per_step": ms_step, "steps": steps, "dtype": wl.dtype}
    if cnt.value:
        k_ms = tot.value / cnt.value
        out["kernel"] = wl.kernel
        out["kernel_ms"] = k_ms
        if wl.bound == "hbm":
            ach = wl.kernel_bytes() / (k_ms * 1e-3) / 1e9
            out["roofline"] = {"bound": "hbm", "achieved": ach, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                               "frac": ach / HBM_PEAK_GBS, "traffic": profiled_traffic(wl.kernel)}
        else:
            peak = FP32_PEAK_TFLOPS if wl.dtype == "f32" else FP64_PEAK_TFLOPS
            ach = wl.kernels[wl.kernel] / (k_ms * 1e-3) / 1e12
            out["roofline"] = {"bound": "mfma", "achieved": ach, "peak": peak, "unit": "TFLOP/s",
                               "frac": ach / peak, "traffic": None}
    if per_kernel:
        out["kernels"] = per_kernel
    if wl.bound == "mfma":
        out["eval_TFLOPs"] = wl.eval_flops() / (ms_step * 1e-3) / 1e12
        out["eval_mfma_frac"] = out["eval_TFLOPs"] / FP32_PEAK_TFLOPS
    if wl.bound == "hbm" and wl.algo_bytes():
        out["eval_GBps"] = wl.algo_bytes() / (ms_step * 1e-3) / 1e9
        out["eval_hbm_frac"] = out["eval_GBps"] / HBM_PEAK_GBS
    out["config"] = wl.config()
    return out


def cpu_baseline(wl: Workload, budget_s: float = 12.0, max_runs: int = 30) -> dict | None:
    sample = wl.cpu_sample()
    if sample is None:
        return None
    run, desc = sample[0], sample[1]
    scale = sample[2] if len(sample) > 2 else 1.0   # the sample's share of one evaluation
    try:
        cpus = sorted(os.sched_getaffinity(0))
        os.sched_setaffinity(0, {cpus[0]})
    except (AttributeError, OSError):
        cpus = None
    try:
        run()  # warm-up
        times = []
        t_start = time.perf_counter()
        while len(times) < max_runs and (time.perf_counter() - t_start) < budget_s:
            t0 = time.perf_counter()
            run()
            times.append(time.perf_counter() - t0)
    finally:
        if cpus:
            os.sched_setaffinity(0, set(cpus))
    times.sort()
    med = times[len(times) // 2]
    cpu_model = ""
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                cpu_model = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": scale / med, "unit": "evals/s", "cores": 1, "kind": "port",
            "sample": f"{desc}: median of {len(times)} runs of the oracle (generated Julia text transpiled to C, "
                      f"gcc -O2, 1 thread pinned to one core, {cpu_model})"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default=HEADLINE, choices=sorted(WORKLOADS))
    ap.add_argument("--only", action="store_true", help="measure the headline workload only")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a device-to-device copy of 1 GiB, 10 times (the reference kernel that scales "
                         "FETCH_SIZE / WRITE_SIZE counters to bytes)")
    ap.add_argument("--configs", default="", help="comma-separated workloads to measure besides the headline "
                                                  "(default: all)")
    ap.add_argument("--stream-ceiling", action="store_true",
                    help="run only torch's own elementwise kernels over the headline's bytes (4096^2 fp64: "
                         "un = u, ub += unb; 40 B per cell) and print their rate, a practical ceiling for "
                         "the adjoint pass's access mix")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build runs on one GPU; the multi-GPU design is described, not run "
              "(--gpus N > 1 is not supported)", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    if args.copy_calibration:
        n = 1 << 27
        src = torch.ones(n, dtype=torch.float64, device=dev)
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": 8 * n, "copy_bytes_written": 8 * n, "launches": 10}))
        return
    if args.stream_ceiling:
        n = 4096 * 4096
        u, unb, ub = (torch.randn(n, dtype=torch.float64, device=dev) for _ in range(3))
        un = torch.empty_like(u)

        def one():
            un.copy_(u)
            ub.add_(unb)

        for _ in range(5):
            one()
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 50
        t0.record()
        for _ in range(reps):
            one()
        t1.record()
        torch.cuda.synchronize()
        us = t0.elapsed_time(t1) * 1e3 / reps
        print(json.dumps({"stream_ceiling": "un = u (copy), ub += unb (add), torch kernels, 4096^2 fp64",
                          "bytes": 40 * n, "us": round(us, 1), "TBps": round(40 * n / us / 1e6, 3),
                          "frac_of_8TBps": round(40 * n / us / 1e6 / 8.0, 3)}))
        return
    head = WORKLOADS[args.workload]()
    res = measure(head, args.steps, args.warmup, dev)
    others = {}
    if not args.only:
        for nm, mk in WORKLOADS.items():
            if nm == args.workload or (args.configs and nm not in args.configs.split(",")):
                continue
            wl = mk()
            heavy = nm.startswith(("burgers1d", "conv3x3", "mlp2_ce"))
            others[nm] = measure(wl, 10 if heavy else max(5, args.steps // 2), 2 if heavy else max(2, args.warmup), dev)
            if not args.no_cpu_baseline:
                others[nm]["cpu_baseline"] = cpu_baseline(wl, budget_s=4.0, max_runs=5)
            del wl
            torch.cuda.empty_cache()
    cpu = None if args.no_cpu_baseline else cpu_baseline(head)
    line = {
        "metric": "gradient evals/sec per config",
        "value": res["evals_per_s"],
        "unit": "evals/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": res["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": head.dtype,
        "data": "synthetic (seeded Julia Xoshiro stream, val_stable_seed of the config name)",
        "config": res["config"],
        "roofline": res.get("roofline"),
        "cpu_baseline": cpu,
        "eval_hbm_frac": res.get("eval_hbm_frac"),
        "kernel_ms": res.get("kernel_ms"),
        "kernel_timing": "HIP event pair around each launch of the dominant kernel on its own stream, over a second "
                         "pass of the same K steps; value and ms_per_step come from the first, event-free pass",
        "configs": {k: {kk: vv for kk, vv in v.items() if kk != "config"} | {"workload": v["config"].get("workload")}
                    for k, v in others.items()},
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
