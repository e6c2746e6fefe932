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
    """A flat device copy of a host array; a matrix is flattened in Julia's column-major order."""
    import numpy as np
    import torch
    a = np.asarray(a)
    return torch.from_numpy(np.ascontiguousarray(a.ravel(order="F") if a.ndim > 1 else a)).to(dev)


def arg_names(family: str, mode: str) -> list[str]:
    """The generated function's argument names, in order, stacks included (the C ABI's and
    the Python mirror's order: `agen_signature_args` /root/reference/src/STADE.jl:3455-3464,
    `tgen_signature_args` 3306-3315, `hvp_emit` 6750-6756)."""
    from stade_hip.emit import KERNELS
    spec = KERNELS[family]
    names = [nm for nm, _ in spec.modes[mode].args]
    if mode != "d":
        names += [nm for nm, _, _ in spec.stacks]
    return names


class Workload:
    """One generated function of one config at the benchmark size.

    `host_inputs()` returns every argument of the config's three generated functions by its
    generated name (numpy arrays in Julia's column-major order, flattened; Python floats and
    ints), seeded as the benchmark seeds them; the GPU run, the CPU baseline and the
    full-size parity tests all take their inputs from it."""
    family = ""
    kernel = ""           # dominant kernel (profiler name)
    bound = "hbm"
    dtype = "f64"
    graph_steps = 0       # > 0: the timed steps are replays of a HIP graph of this many steps
    lowered = False       # True: the general lowering's library runs the generated text

    def __init__(self, mode: str):
        self.mode = mode
        self.name = f"{self.family}_{mode}"

    def host_inputs(self) -> dict:
        raise NotImplementedError

    def stack_lengths(self) -> list[tuple[int, str]]:
        """(length, 'Ai' | 'Af') of each stack argument (adjoint and HVP only)."""
        return []

    def setup(self, dev):
        import numpy as np
        import torch
        self.h = self.host_inputs()
        self.t = {k: _tensor(v, dev) if isinstance(v, np.ndarray) else v for k, v in self.h.items()}
        self.stacks = []
        if self.mode != "d":
            for length, kind in self.stack_lengths():
                dt = torch.int64 if kind == "Ai" else (torch.float64 if self.dtype == "f64" else torch.float32)
                self.stacks.append(torch.empty(length, dtype=dt, device=dev))
        names = arg_names(self.family, self.mode)
        self.argv = [self.t[a] for a in names[:len(names) - len(self.stacks)]] + self.stacks

    def step(self):
        if self.lowered:
            self._low.call(self.name, *self.argv, shapes=self._dims)
            return
        import stade_hip
        getattr(stade_hip, self.name)(*self.argv)

    def use_lowered(self):
        """Run the config's generated text through the general lowering (stade_hip.lower)
        instead of its hand-written entry point: the same inputs, the same outputs."""
        import numpy as np
        from stade_hip import lower
        self.lowered = True
        self.graph_steps = 0   # (a lowered call synchronises to check its error flag: no capture)
        path = ROOT / "stade.jl_amd" / "corpus" / f"{self.name}.jl"
        self._low = lower.lower(path, "f32" if self.dtype == "f32" else "f64")
        self._dims = {a: v.shape for a, v in self.host_inputs().items() if isinstance(v, np.ndarray) and v.ndim > 1}

    def algo_bytes(self) -> float:          # per evaluation
        return 0.0

    def kernel_bytes(self) -> float:        # per launch of the dominant kernel
        return 0.0

    def config(self) -> dict:
        return {}

    def sample(self):
        """A smaller workload of the same family for the CPU baseline, and the share of one
        full evaluation that it is (1.0: the full size)."""
        return self, 1.0

    def sample_desc(self) -> str:
        return f"{self.name} at the full size"

    def cpu_sample(self):
        """(callable running one evaluation of the oracle on `sample()`, description, share)."""
        import numpy as np
        from oracle import runner
        wl, share = self.sample()
        prec = "f32" if self.dtype == "f32" else "f64"
        # the sample runs the generated text of its own function (a policy variant such as the
        # checkpointed Burgers adjoint samples the tape form's text: the same CPU code)
        lib = runner.load(ROOT / "stade.jl_amd" / "corpus" / f"{wl.name}.jl", precision=prec, bounds_check=False)
        h = wl.host_inputs()
        names = arg_names(wl.family, wl.mode)
        nst = len(wl.stack_lengths()) if wl.mode != "d" else 0
        fdt = np.float64 if prec == "f64" else np.float32

        def run():
            argv = [h[a].copy(order="K") if isinstance(h[a], np.ndarray) else h[a] for a in names[:len(names) - nst]]
            if nst:
                argv += [np.empty(k, dtype=np.int64 if kind == "Ai" else fdt) for k, kind in wl.stack_lengths()]
            lib.call(wl.name, *argv)
        desc = wl.sample_desc()
        if share != 1.0:
            desc += f" ({1 / share:.0f}x less work than one benchmark evaluation; the rate is scaled by that share)"
        return run, desc, share


def _rng(name: str, salt: int = 0):
    import stade_hip
    return stade_hip.api.Rng(stade_hip.stable_seed(name) + salt)


class Diffusion(Workload):
    """Config 2: one periodic 5-point step on n x n fp64, u ~ N(0,1), loss = sum(un^2);
    tangent / HVP direction ud ~ N(0,1) from the next seed."""
    family = "diffusion2d"
    dtype = "f64"
    # the steps as replays of a captured HIP graph, as a caller looping over evaluations would
    # issue them: 2-5 % faster than eager launches (the evaluation is two or three launches)
    graph_steps = 10

    def __init__(self, mode="b", n=4096):
        super().__init__(mode)
        self.n = n
        self.kernel = f"diffusion2d_{mode}"

    def host_inputs(self):
        import numpy as np
        import stade_hip
        c = self.n * self.n
        z = lambda k: np.zeros(k)
        return dict(loss=z(1), lossb=np.ones(1), lossd=z(1), lossbd=z(1),
                    u=stade_hip.rng_normal(_rng("diffusion2d"), c), ub=z(c), un=z(c), unb=z(c),
                    ud=stade_hip.rng_normal(_rng("diffusion2d", 1), c), ubd=z(c), und=z(c), unbd=z(c), n=self.n)

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

    def sample_desc(self):
        return f"diffusion2d_{self.mode} at the full {self.n}x{self.n} grid"


class Affine(Workload):
    """Config 1: loss = 0.5 sum((W x + b - t)^2), W m x n fp64 U[-1,1], x, b, t N(0,1);
    direction (Wd, xd, bd, td) ~ N(0,1) from the next seed."""
    family = "affine_lsq"
    dtype = "f64"
    # launch-bound at 1024^2 (an evaluation is 2-3 dependent launches of a few microseconds):
    # the steps are issued as a captured HIP graph, as a caller running it in a loop would,
    # so that the host's per-launch cost is not what is measured
    graph_steps = 10

    def __init__(self, mode="b", m=1024, n=1024):
        super().__init__(mode)
        self.m, self.n = m, n
        self.kernel = "affine_cols" if mode != "d" else "affine_rows"

    def host_inputs(self):
        import numpy as np
        import stade_hip
        m, n = self.m, self.n
        rng = _rng("affine_lsq")
        w = stade_hip.rng_uniform(rng, m * n, -1.0, 1.0)
        x, b, t = (stade_hip.rng_normal(rng, k) for k in (n, m, m))
        rng2 = _rng("affine_lsq", 1)
        wd, xd, bd, td = (stade_hip.rng_normal(rng2, k) for k in (m * n, n, m, m))
        z = lambda k: np.zeros(k)
        mat = lambda a: np.asfortranarray(a.reshape((m, n), order="F"))   # w is an (i_m, i_n) Julia matrix
        return dict(loss=z(1), lossb=np.ones(1), lossd=z(1), lossbd=z(1), w=mat(w), wb=mat(z(m * n)), x=x, xb=z(n),
                    b=b, bb=z(m), t=t, tb=z(m), r=z(m), rb=z(m), wd=mat(wd), wbd=mat(z(m * n)), xd=xd, xbd=z(n),
                    bd=bd, bbd=z(m), td=td, tbd=z(m), rd=z(m), rbd=z(m), i_m=m, i_n=n)

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

    def sample_desc(self):
        return f"affine_lsq_{self.mode} at the full {self.m}x{self.n} size"


class Burgers(Workload):
    """Config 5: 2^20 periodic cells, 500 guarded steps, nu = 1e-3, dx = 1/n, dt such that
    nu dt / dx^2 = 0.2; u0 = sin(2 pi x) + 0.1 N(0,1), x_i = (i - 1) / n; tend = 1 (every
    step runs); tangent / HVP direction ud ~ N(0,1) from the next seed and nud = 0.01."""
    family = "burgers1d"
    dtype = "f64"

    def __init__(self, mode="b", n=1 << 20, nsteps=500, dx=None):
        super().__init__(mode)
        self.n, self.T = n, nsteps
        self.kernel = {"b": "burgers1d_bwd", "d": "burgers1d_fwd_tan", "hv": "burgers1d_bwd_hv"}[mode]
        if mode == "d":
            # no tape: the tangent is bound by its fp64 arithmetic (the state stays in LDS for 32
            # steps a launch).  Algorithmic flops: the text's 26 operations per cell and step
            # (__cse_1 1, __cse_2 3, und 17, un 5), averaged over the launches
            self.bound = "valu"
            self.kernels = {self.kernel: self.TAN_FLOPS * n * nsteps / max(1, self._launches())}
        self.nu = 1e-3
        self.dx = 1.0 / n if dx is None else dx
        self.dt = 0.2 * self.dx * self.dx / self.nu
        self.tend = 1.0

    def host_inputs(self):
        import numpy as np
        import stade_hip
        n = self.n
        x = np.arange(n, dtype=np.float64) / n
        u = np.sin(2.0 * np.pi * x) + 0.1 * stade_hip.rng_normal(_rng("burgers1d"), n)
        ud = stade_hip.rng_normal(_rng("burgers1d", 1), n)
        z = lambda k: np.zeros(k)
        return dict(loss=z(1), lossb=np.ones(1), lossd=z(1), lossbd=z(1), u=u, ub=z(n), un=z(n), unb=z(n),
                    ud=ud, ubd=z(n), und=z(n), unbd=z(n),
                    nu=self.nu, nub=0.0, dt=self.dt, dtb=0.0, dx=self.dx, dxb=0.0, tend=self.tend, tendb=0.0,
                    nud=0.01, nubd=0.0, dtd=0.0, dtbd=0.0, dxd=0.0, dxbd=0.0, tendd=0.0, tendbd=0.0,
                    n=n, nsteps=self.T)

    def stack_lengths(self):
        return [(self.T, "Ai"), (self.T * self.n, "Af")]

    TAN_FLOPS = 26   # fp64 operations per cell and step of burgers1d_d as written

    def _launches(self):
        return -(-self.T // 32)

    def eval_flops(self):
        return self.TAN_FLOPS * self.n * self.T

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

    def sample(self):
        Ts = 20
        return Burgers(self.mode, self.n, Ts), Ts / self.T

    def sample_desc(self):
        return f"burgers1d_{self.mode} on {self.n} cells for {self.T} steps"


class BurgersCkpt(Burgers):
    """Config 5 under the checkpoint tape policy (stade_hip_burgers1d_{b,hv}_ckpt): the state
    of every `every`-th step is kept and each segment is recomputed in the reverse sweep.
    Same inputs and outputs as Burgers; the tape the caller holds is 1/every of the full one."""

    def __init__(self, mode="b", n=1 << 20, nsteps=500, every=32):
        super().__init__(mode, n, nsteps)
        self.every = every
        self.name = f"burgers1d_{mode}_ckpt"

    def stack_lengths(self):
        return [(self.T, "Ai"), (-(-self.T // self.every) * self.n, "Af")]

    def step(self):
        import stade_hip
        getattr(stade_hip, f"burgers1d_{self.mode}_ckpt")(*self.argv, self.every)

    def config(self):
        c = super().config()
        c["workload"] = c["workload"].replace(f"burgers1d_{self.mode}:", f"burgers1d_{self.mode} (checkpoint policy, "
                                              f"every {self.every} steps):")
        c["tape_bytes"] = 8 * (-(-self.T // self.every)) * self.n
        c["every"] = self.every
        return c

    def sample(self):
        Ts = 20
        return Burgers(self.mode, self.n, Ts), Ts / self.T

    def sample_desc(self):
        return f"burgers1d_{self.mode} (tape form: the same CPU code) on {self.n} cells for 20 steps"


class Mlp(Workload):
    """Config 3: x (784, 4096) ~ U[0,1], tanh hidden layer of 1024, 10-way softmax
    cross-entropy, Float32; W1, W2 Glorot-uniform U(+-sqrt(6 / (fan_in + fan_out))),
    b1 = b2 = 0, labels uniform in 1..10, HVP direction (xd, W1d, b1d, W2d, b2d) ~ N(0,1) --
    all from the seeded Xoshiro stream."""
    family = "mlp2_ce"
    dtype = "f32"
    bound = "mfma"
    graph_steps = 10   # (replayed graphs, as for diffusion: 1-4 % faster than eager launches)

    def __init__(self, mode="b", B=4096, I=784, H=1024, O=10):
        super().__init__(mode)
        self.B, self.I, self.H, self.O = B, I, H, O
        g = 2.0 * H * I * B
        # flops per launch of each matrix-core kernel: the tangent and HVP run each pair
        # (s1, s1d), (W1b, W1bd), (xb, xbd) as one dual launch of three products, and the two
        # backward products (W1b and xb, or their dual forms) share one launch
        self.kernels = {"b": {"mlp_gemm_s1": g, "mlp_gemm_bwd": 2 * g},
                        "d": {"mlp_gemm_s1d": 3 * g},
                        "hv": {"mlp_gemm_s1d": 3 * g, "mlp_gemm_bwd2": 6 * g}}[mode]
        self.kernel = next(iter(self.kernels))

    def host_inputs(self):
        import numpy as np
        import stade_hip
        B, I, H, O = self.B, self.I, self.H, self.O
        f = lambda a: np.asarray(a, dtype=np.float32)
        rng = _rng("mlp2_ce")
        x = f(stade_hip.rng_uniform(rng, I * B, 0.0, 1.0))
        a1, a2 = np.sqrt(6.0 / (I + H)), np.sqrt(6.0 / (H + O))
        w1 = f(stade_hip.rng_uniform(rng, H * I, -a1, a1))
        w2 = f(stade_hip.rng_uniform(rng, O * H, -a2, a2))
        lab = stade_hip.rng_int_range(rng, B, 1, O)
        rng2 = _rng("mlp2_ce", 1)
        d = {k: f(stade_hip.rng_normal(rng2, n)) for k, n in (("xd", I * B), ("w1d", H * I), ("b1d", H), ("w2d", O * H), ("b2d", O))}
        z = lambda k: np.zeros(k, dtype=np.float32)
        h = dict(loss=z(1), lossb=np.ones(1, np.float32), lossd=z(1), lossbd=z(1), x=x, lab=lab, w1=w1, b1=z(H), w2=w2, b2=z(O),
                 i_b=B, i_in=I, i_h=H, i_out=O, **d)
        for k, n in (("x", I * B), ("w1", H * I), ("b1", H), ("w2", O * H), ("b2", O), ("h1", H * B), ("z", O * B)):
            for suf in ("b", "bd") if k not in ("h1", "z") else ("", "b", "d", "bd"):
                h.setdefault(k + suf, z(n))
        return h

    def eval_flops(self):
        B, I, H, O = self.B, self.I, self.H, self.O
        return sum(self.kernels.values()) * 1.0 + {"b": 2, "d": 2, "hv": 4}[self.mode] * 2.0 * O * H * B

    def config(self):
        return {"workload": f"mlp2_ce_{self.mode}: x {self.I}x{self.B} fp32 U[0,1] -> tanh({self.H}) -> {self.O}-way softmax "
                            f"cross-entropy summed over the batch; Glorot-uniform weights, zero biases",
                "batch": self.B, "widths": [self.I, self.H, self.O]}

    def sample(self):
        Bs = 128
        return Mlp(self.mode, Bs, self.I, self.H, self.O), Bs / self.B

    def sample_desc(self):
        return f"mlp2_ce_{self.mode} on a batch of {self.B}"


class Conv(Workload):
    """Config 4: 8 images of 256 x 256, 64 -> 64 channels, 3 x 3, zero border held in xp,
    Float32; xp interior ~ N(0,1), w He-normal N(0, 2 / (9 C)); tangent / HVP direction
    xpd (interior), wd the same laws -- from the seeded Xoshiro stream."""
    family = "conv3x3"
    dtype = "f32"
    bound = "mfma"
    graph_steps = 10   # (replayed graphs, as for diffusion: about 1 % faster than eager launches)

    def __init__(self, mode="b", N=8, C=64, K=64, H=256, W=256):
        super().__init__(mode)
        self.N, self.C, self.K, self.H, self.W = N, C, K, H, W
        g = 2.0 * N * K * H * W * 9 * C
        self.kernels = {"b": {"conv_fwd": g, "conv_wgrad": g, "conv_dgrad": g},
                        "d": {"conv_fwd_d": 3 * g},
                        "hv": {"conv_fwd_hv": 3 * g, "conv_wgrad": g, "conv_wgrad2": 2 * g, "conv_dgrad_hv": 3 * g}}[mode]
        self.kernel = next(iter(self.kernels))

    def host_inputs(self):
        import numpy as np
        import stade_hip
        N, C, K, H, W = self.N, self.C, self.K, self.H, self.W
        rng = _rng("conv3x3")
        xp = np.zeros((N, C, H + 2, W + 2), dtype=np.float32)
        xp[:, :, 1:-1, 1:-1] = stade_hip.rng_normal(rng, N * C * H * W).reshape(N, C, H, W)
        w = (stade_hip.rng_normal(rng, 9 * C * K) * np.sqrt(2.0 / (9.0 * C))).astype(np.float32)
        rng2 = _rng("conv3x3", 1)
        xpd = np.zeros_like(xp)
        xpd[:, :, 1:-1, 1:-1] = stade_hip.rng_normal(rng2, N * C * H * W).reshape(N, C, H, W)
        wd = (stade_hip.rng_normal(rng2, 9 * C * K) * np.sqrt(2.0 / (9.0 * C))).astype(np.float32)
        nx, nw, no = N * C * (H + 2) * (W + 2), 9 * C * K, N * K * H * W
        z = lambda k: np.zeros(k, dtype=np.float32)
        return dict(loss=z(1), lossb=np.ones(1, np.float32), lossd=z(1), lossbd=z(1), xp=xp.ravel(), xpb=z(nx), xpd=xpd.ravel(),
                    xpbd=z(nx), w=w, wb=z(nw), wd=wd, wbd=z(nw), out=z(no), outb=z(no), outd=z(no), outbd=z(no),
                    i_nb=N, i_c=C, i_k=K, i_h=H, i_w=W)

    def eval_flops(self):
        return sum(self.kernels.values()) * 1.0

    def config(self):
        return {"workload": f"conv3x3_{self.mode}: {self.N} x {self.C} x {self.H} x {self.W} fp32 input (zero border "
                            f"held in xp), 3x3 {self.C}->{self.K}, loss = 0.5 sum(out^2)",
                "batch": self.N, "channels": [self.C, self.K], "image": [self.H, self.W]}

    def sample(self):
        Ns, Hs = 1, 32
        return Conv(self.mode, Ns, self.C, self.K, Hs, self.W), (Ns * Hs) / (self.N * self.H)

    def sample_desc(self):
        return f"conv3x3_{self.mode} on {self.N} image(s) of {self.H} x {self.W}"


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
    "burgers1d_b_ckpt": lambda: BurgersCkpt("b"),
    "burgers1d_hv_ckpt": lambda: BurgersCkpt("hv"),
    "mlp2_ce_b": lambda: Mlp("b"),
    "mlp2_ce_d": lambda: Mlp("d"),
    "mlp2_ce_hv": lambda: Mlp("hv"),
    "conv3x3_b": lambda: Conv("b"),
    "conv3x3_d": lambda: Conv("d"),
    "conv3x3_hv": lambda: Conv("hv"),
}
HEADLINE = "diffusion2d_b"

# bench.py --sizes: (workload, label) around each benchmark size
SIZE_SWEEP = (
    [(lambda n=n, m=m: Diffusion(m, n=n), f"diffusion2d_{m} n={n}") for m in ("b", "d", "hv")
     for n in (512, 1024, 2048, 3072, 4096, 6144, 8192, 12288)]
    + [(lambda n=n, m=m: Affine(m, m=n, n=n), f"affine_lsq_{m} {n}x{n}") for m in ("b", "d", "hv")
       for n in (256, 1024, 2048, 4096, 8192)]
    + [(lambda n=n: Burgers("b", n=n), f"burgers1d_b n={n} T=500") for n in (1 << 16, 1 << 18, 1 << 20, 1 << 22)]
    + [(lambda b=b: Mlp("b", B=b), f"mlp2_ce_b batch={b}") for b in (512, 1024, 4096, 16384)]
    + [(lambda k=k: Conv("b", N=k), f"conv3x3_b {k} images") for k in (1, 2, 8, 16)]
)


def _lib():
    import stade_hip
    L = stade_hip.lib()
    L.stade_hip_profile_read.argtypes = [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int64)]
    return L


def profiled_traffic(workload: str):
    """HBM bytes per launch of the workload's dominant kernel from its committed counter
    summary (profiles/<workload>_traffic.md: FETCH_SIZE and WRITE_SIZE per dispatch, each
    scaled by what the same counter reads for a 1 GiB copy), or None when there is none.
    rocprofv3 counter passes cannot run inside the timed process, so the figure comes from
    the committed summary of a separate run of the same command."""
    import re
    f = ROOT / "profiles" / f"{workload}_traffic.md"
    if not f.exists():
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*(\d+)", f.read_text(), re.M)
    return int(m.group(1)) if m else None


def _graph_us(fn, per_graph: int = 20, replays: int = 25) -> float:
    """GPU time of one fn() in microseconds, with the host's launch cost taken out: per_graph
    calls captured in one HIP graph (torch.cuda.graph), the graph replayed `replays` times
    between two events."""
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(per_graph):
            fn()
    g.replay()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(replays):
        g.replay()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) * 1e3 / (replays * per_graph)


def launch_floor(dev) -> dict:
    """What an evaluation of the affine config (1024^2 fp64, 25.3 MB) must pay on this GPU,
    measured with graph replays so that the host's launch cost is out: torch's own kernels
    moving the matrix bytes in one launch and in three dependent launches, chains of one-element
    launches (the per-launch floor), and the library's affine evaluations themselves."""
    import torch
    n = 1024 * 1024
    w, wb = (torch.randn(n, dtype=torch.float64, device=dev) for _ in range(2))
    tiny = torch.zeros(1, dtype=torch.float64, device=dev)
    thirds = [(k * n // 3, (k + 1) * n // 3) for k in range(3)]
    cases = {
        "one launch, wb += w (24 MiB)": lambda: wb.add_(w),
        "three dependent launches, wb[k] += w[k] (8 MiB each)": lambda: [wb[a:b].add_(w[a:b]) for a, b in thirds],
        "one launch of one element": lambda: tiny.add_(1.0),
        "two dependent launches of one element": lambda: [tiny.add_(1.0) for _ in range(2)],
        "three dependent launches of one element": lambda: [tiny.add_(1.0) for _ in range(3)],
    }
    out = {name: round(_graph_us(fn), 2) for name, fn in cases.items()}
    for mode in ("b", "d", "hv"):
        wl = Affine(mode)
        wl.setup(dev)
        out[f"affine_lsq_{mode} evaluation (library, {2 if mode == 'd' else 3} launches)"] = round(_graph_us(wl.step), 2)
    return {"launch_floor_us": out, "graph_replayed": True,
            "affine_roofline_us": {m: round(Affine(m).algo_bytes() / 8e6, 2) for m in ("b", "d", "hv")}}


def measure(wl: Workload, steps: int, warmup: int, dev) -> dict:
    import torch
    L = _lib()
    wl.setup(dev)
    for _ in range(warmup):
        wl.step()
    torch.cuda.synchronize()
    run = lambda k: [wl.step() for _ in range(k)]
    if wl.graph_steps:
        # K steps as replays of captured graphs of graph_steps steps (and one of the remainder)
        graphs = {}
        for k in {min(wl.graph_steps, steps), steps % wl.graph_steps} - {0}:
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                wl.step()
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                run(k)
            g.replay()
            torch.cuda.synchronize()
            graphs[k] = g
        full, rest = divmod(steps, wl.graph_steps)

        def run(k):
            assert k == steps
            for _ in range(full):
                graphs[wl.graph_steps].replay()
            if rest:
                graphs[rest].replay()
    # pass 1, the timed region: K steps with nothing added to the stream
    t0 = time.perf_counter()
    run(steps)
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
                               "frac": ach / HBM_PEAK_GBS, "traffic": profiled_traffic(wl.name)}
        else:
            peak = FP32_PEAK_TFLOPS if wl.dtype == "f32" else FP64_PEAK_TFLOPS
            ach = wl.kernels[wl.kernel] / (k_ms * 1e-3) / 1e12
            out["roofline"] = {"bound": wl.bound, "achieved": ach, "peak": peak, "unit": "TFLOP/s",
                               "frac": ach / peak, "traffic": None}
    if per_kernel:
        out["kernels"] = per_kernel
    if wl.bound in ("mfma", "valu"):
        out["eval_TFLOPs"] = wl.eval_flops() / (ms_step * 1e-3) / 1e12
        out[f"eval_{wl.bound}_frac"] = out["eval_TFLOPs"] / (FP32_PEAK_TFLOPS if wl.dtype == "f32" else FP64_PEAK_TFLOPS)
    if wl.bound == "hbm" and wl.algo_bytes():
        out["eval_GBps"] = wl.algo_bytes() / (ms_step * 1e-3) / 1e9
        out["eval_hbm_frac"] = out["eval_GBps"] / HBM_PEAK_GBS
    out["config"] = wl.config()
    if wl.graph_steps:
        out["config"]["launch"] = f"HIP graph of {wl.graph_steps} steps, replayed (torch.cuda.graph)"
    if wl.lowered:
        out["config"]["path"] = "general lowering (stade_hip.lower) of the generated text"
    return out


def twins_bench(dev) -> None:
    """The flat twins of the general lowering against its ordinary form (the same text lowered
    with STADE_LOWER_TWINS=0): ms per call of flatmv_d and flatmv_b, fp64, seeded N(0,1) inputs,
    20 calls after 3 warm-ups."""
    import torch
    from stade_hip.lower import runtime
    gen = ROOT / "stade.jl_amd" / "corpus" / "generic"
    libs = {}
    for tw in ("1", "0"):
        os.environ["STADE_LOWER_TWINS"] = tw
        runtime._cache.clear()
        libs[tw] = {m: runtime.lower(gen / f"flatmv_{m}.jl", "f64") for m in ("b", "d")}
    os.environ.pop("STADE_LOWER_TWINS", None)
    g = torch.Generator(device=dev)
    g.manual_seed(7)

    def run(low, mode, m, n, reps=20):
        f = lambda k: torch.randn(k, dtype=torch.float64, device=dev, generator=g)
        z = lambda k: torch.zeros(k, dtype=torch.float64, device=dev)
        if mode == "b":
            args = [z(1), torch.ones(1, dtype=torch.float64, device=dev), f(m * n), z(m * n), f(n), z(n), z(m), z(m), m, n]
        else:
            args = [z(1), z(1), f(m * n), f(m * n), f(n), f(n), z(m), z(m), m, n]
        for _ in range(3):
            low.call(f"flatmv_{mode}", *args)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            low.call(f"flatmv_{mode}", *args)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / reps * 1e3

    for m, n, what in [(40960, 1024, "MLP head z = W2 h1 flattened: 40960 outputs of 1024 terms"),
                       (4096, 1024, "4096 rows of 1024"), (1024, 8192, "1024 rows of 8192"),
                       (10, 1 << 22, "10 outputs of 4194304 terms (the row twin's chunks)")]:
        for mode in ("d", "b"):
            t_on, t_off = run(libs["1"][mode], mode, m, n), run(libs["0"][mode], mode, m, n)
            nbytes = 8 * m * n * (2 if mode == "d" else 3)
            print(json.dumps({"shape": what, "m": m, "n": n, "function": f"flatmv_{mode}", "twins_ms": round(t_on, 4),
                              "ordinary_ms": round(t_off, 4), "speedup": round(t_off / t_on, 2),
                              "twins_GBps": round(nbytes / t_on / 1e6, 1)}), flush=True)


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
    ap.add_argument("--sizes", nargs="?", const="all", default=None, metavar="FAMILIES",
                    help="time each config's adjoint (and the headline's tangent and HVP) over a range of sizes around "
                         "the benchmark's and print one JSON line per size (evals/s and the roofline fraction); "
                         "optionally only the comma-separated families named")
    ap.add_argument("--lowered", action="store_true",
                    help="run every measured workload's generated text through the general lowering (stade_hip.lower) "
                         "instead of its hand-written kernels (the checkpointed Burgers forms have no text and are skipped)")
    ap.add_argument("--graph", type=int, default=None,
                    help="issue the measured workload's timed steps as replays of a captured HIP graph of this many "
                         "steps (0: eager launches; default: the workload's own choice)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a device-to-device copy of 1 GiB, 10 times (the reference kernel that scales "
                         "FETCH_SIZE / WRITE_SIZE counters to bytes)")
    ap.add_argument("--configs", default="", help="comma-separated workloads to measure besides the headline "
                                                  "(default: all)")
    ap.add_argument("--launch-floor", action="store_true",
                    help="time, with torch's own kernels, what any evaluation of the affine config must pay at "
                         "1024^2 fp64: one launch moving its 24 MiB matrix bytes (wb += w), the same bytes split "
                         "over three dependent launches, and chains of 1 and 3 launches of one element each")
    ap.add_argument("--twins", action="store_true",
                    help="time the general lowering's flat-loop twins (row-block, column-block) against the ordinary "
                         "form on the row-major flat mat-vec text (corpus/generic/flatmv_{b,d}.jl) at the MLP head's "
                         "shape and others, one JSON line per shape and function")
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
    if args.launch_floor:
        print(json.dumps(launch_floor(dev)))
        return
    if args.twins:
        twins_bench(dev)
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
    if args.sizes:
        keep = None if args.sizes == "all" else set(args.sizes.split(","))
        for mk, label in SIZE_SWEEP:
            if keep is not None and label.split(" ")[0].rsplit("_", 1)[0] not in keep:
                continue
            wl = mk()
            heavy = wl.family in ("burgers1d", "conv3x3", "mlp2_ce")
            r = measure(wl, 10 if heavy else 30, 2 if heavy else 5, dev)
            rf = r.get("roofline") or {}
            print(json.dumps({"size": label, "function": wl.name, "evals_per_s": r["evals_per_s"],
                              "ms_per_step": r["ms_per_step"], "kernel_ms": r.get("kernel_ms"),
                              "kernel_frac": rf.get("frac"), "bound": rf.get("bound"),
                              "eval_frac": r.get("eval_hbm_frac") or r.get("eval_mfma_frac") or r.get("eval_valu_frac")}),
                  flush=True)
            del wl
            torch.cuda.empty_cache()
        return
    head = WORKLOADS[args.workload]()
    if args.graph is not None:
        head.graph_steps = args.graph
    if args.lowered:
        head.use_lowered()
    res = measure(head, args.steps, args.warmup, dev)
    others = {}
    if not args.only:
        for nm, mk in WORKLOADS.items():
            if nm == args.workload or (args.configs and nm not in args.configs.split(",")):
                continue
            wl = mk()
            if args.lowered:
                if nm.endswith("_ckpt"):
                    continue
                wl.use_lowered()
            heavy = nm.startswith(("burgers1d", "conv3x3", "mlp2_ce"))
            others[nm] = measure(wl, 10 if heavy else max(5, args.steps // 2), 2 if heavy else max(2, args.warmup), dev)
            if not args.no_cpu_baseline:
                others[nm]["cpu_baseline"] = cpu_baseline(wl, budget_s=4.0, max_runs=5)
            # the full record of each function on a line of its own; the last line keeps a summary
            print(json.dumps({"detail": nm, **others[nm]}), flush=True)
            del wl
            torch.cuda.empty_cache()
    cpu = None if args.no_cpu_baseline else cpu_baseline(head)
    print(json.dumps({"detail": args.workload, **res, "cpu_baseline": cpu}), flush=True)
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
        "eval_mfma_frac": res.get("eval_mfma_frac"),
        "kernel": res.get("kernel"),
        "kernel_ms": res.get("kernel_ms"),
        "kernel_timing": "HIP event pair around each launch of the dominant kernel on its own stream, over a second "
                         "pass of the same K steps; value and ms_per_step come from the first, event-free pass",
        # per function: evals/s, ms per evaluation, the evaluation's fraction of its roofline
        # (HBM bytes, fp32 matrix-core or fp64 flops), the dominant kernel's fraction, the CPU
        # baseline's evals/s; each function's full record is on its own "detail" line above
        "configs": {k: _summary(v) for k, v in others.items()},
    }
    print(json.dumps(line))


def _sig(x, d=4):
    return None if x is None else float(f"{x:.{d}g}")


def _summary(r: dict) -> dict:
    frac = r.get("eval_hbm_frac") or r.get("eval_mfma_frac") or r.get("eval_valu_frac")
    return {"evals_per_s": _sig(r["evals_per_s"]), "ms": _sig(r["ms_per_step"]), "eval_frac": _sig(frac, 3),
            "kernel_frac": _sig((r.get("roofline") or {}).get("frac"), 3),
            "cpu_evals_per_s": _sig((r.get("cpu_baseline") or {}).get("value"), 3)}


if __name__ == "__main__":
    main()
