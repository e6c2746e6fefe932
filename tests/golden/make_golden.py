"""Write the golden fixtures of tests/golden/ with torch's CPU autograd in float64.

The five config kernels' derivative texts (stade.jl_amd/corpus/<k>_{b,d,hv}.jl) were written
by hand in the form STADE's generator emits, because the generator (Julia) cannot run here.
These fixtures pin their numbers against an independent AD: each primal of
stade.jl_amd/corpus/<k>.jl is restated in torch (float64, CPU, this container only), and
the fixture holds the inputs, the loss, the gradient of the loss with respect to every
float argument (what an adjoint with lossb = 1 accumulates from zero shadows), the
directional derivative along a seeded direction (what the tangent returns in lossd), and
the Hessian-vector product along it (what the HVP accumulates in the `bd` shadows).

Float32 configs (mlp2_ce, conv3x3): inputs are rounded to float32 first, then everything
is computed in float64 from those values.

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent
torch.set_default_dtype(torch.float64)


def _grad_jvp_hvp(f, args: dict, direction: dict):
    """loss, gradient, directional derivative and HVP of f(**args) along `direction`."""
    names = list(args)
    xs = [torch.tensor(args[k], dtype=torch.float64, requires_grad=True) for k in names]
    vs = [torch.tensor(direction[k], dtype=torch.float64) for k in names]
    loss = f(**dict(zip(names, xs)))
    grads = torch.autograd.grad(loss, xs, create_graph=True)
    dot = sum((g * v).sum() for g, v in zip(grads, vs))
    hv = torch.autograd.grad(dot, xs, allow_unused=True)
    out = {"loss": np.array([loss.item()]), "lossd": np.array([dot.item()])}
    for k, g, h in zip(names, grads, hv):
        out[f"{k}_grad"] = g.detach().numpy().copy()
        out[f"{k}_hvp"] = (h if h is not None else torch.zeros_like(g)).detach().numpy().copy()
    return out


def mlp(rng):
    B, I, H, O = 6, 5, 7, 3
    f32 = lambda a: np.asarray(a, dtype=np.float32).astype(np.float64)
    # Julia column-major (I, B), (H, I), (O, H) stored as C-order (B, I), (I, H), (H, O)
    a = {"x": f32(rng.uniform(0, 1, (B, I))), "w1": f32(rng.uniform(-0.7, 0.7, (I, H))), "b1": f32(0.1 * rng.standard_normal(H)),
         "w2": f32(rng.uniform(-0.7, 0.7, (H, O))), "b2": f32(0.1 * rng.standard_normal(O))}
    d = {k: f32(rng.standard_normal(v.shape)) for k, v in a.items()}
    lab = rng.integers(1, O + 1, size=B).astype(np.int64)
    lab_t = torch.tensor(lab - 1)

    def f(x, w1, b1, w2, b2):
        h1 = torch.tanh(b1 + x @ w1)
        z = b2 + h1 @ w2
        return (torch.log(torch.exp(z).sum(1)) - z[torch.arange(B), lab_t]).sum()
    out = _grad_jvp_hvp(f, a, d)
    return dict(sizes=np.array([B, I, H, O]), lab=lab, **{k: v for k, v in a.items()},
                **{k + "_dir": v for k, v in d.items()}, **out)


def conv(rng):
    N, C, K, H, W = 2, 3, 4, 5, 6
    f32 = lambda a: np.asarray(a, dtype=np.float32).astype(np.float64)
    # every padded cell nonzero, so the frame of the adjoint is pinned too
    a = {"xp": f32(rng.standard_normal((N, C, H + 2, W + 2))), "w": f32(rng.standard_normal((K, C, 3, 3)) / np.sqrt(9 * C))}
    d = {k: f32(rng.standard_normal(v.shape)) for k, v in a.items()}

    def f(xp, w):
        out = torch.nn.functional.conv2d(xp, w)
        return 0.5 * (out * out).sum()
    out = _grad_jvp_hvp(f, a, d)
    return dict(sizes=np.array([N, C, K, H, W]), **a, **{k + "_dir": v for k, v in d.items()}, **out)


def affine(rng):
    m, n = 9, 7
    # W Julia (m, n) column-major stored as C-order (n, m)
    a = {"w": rng.uniform(-1, 1, (n, m)), "x": rng.standard_normal(n), "b": rng.standard_normal(m), "t": rng.standard_normal(m)}
    d = {k: rng.standard_normal(v.shape) for k, v in a.items()}

    def f(w, x, b, t):
        r = (w * x[:, None]).sum(0) + b - t
        return 0.5 * (r * r).sum()
    out = _grad_jvp_hvp(f, a, d)
    return dict(sizes=np.array([m, n]), **a, **{k + "_dir": v for k, v in d.items()}, **out)


def diffusion(rng):
    n = 11
    # u Julia (n, n) column-major (i fastest) stored as C-order (j, i)
    a = {"u": rng.standard_normal((n, n))}
    d = {"u": rng.standard_normal((n, n))}

    def f(u):
        lap = torch.roll(u, 1, 1) + torch.roll(u, -1, 1) + torch.roll(u, 1, 0) + torch.roll(u, -1, 0) - 4.0 * u
        un = u + 0.1 * lap
        return (un * un).sum()
    out = _grad_jvp_hvp(f, a, d)
    return dict(sizes=np.array([n]), **a, **{k + "_dir": v for k, v in d.items()}, **out)


def burgers(rng):
    n, nsteps = 16, 7
    dx = 1.0 / n
    a = {"u": np.sin(2 * np.pi * np.arange(n) / n) + 0.1 * rng.standard_normal(n), "nu": np.array(0.05),
         "dt": np.array(0.2 * dx * dx / 0.05), "dx": np.array(dx)}
    # the guard stops the loop after 5 of the 7 steps
    tend = 4.5 * float(a["dt"])
    d = {"u": rng.standard_normal(n), "nu": np.array(0.3), "dt": np.array(-0.2), "dx": np.array(0.1)}
    d["dt"] = d["dt"] * float(a["dt"])
    d["dx"] = d["dx"] * dx

    def f(u, nu, dt, dx):
        cadv = 0.5 * dt / dx
        cdif = nu * dt / (dx * dx)
        tc = 0.0
        for _ in range(nsteps):
            if tc < tend:
                up, um = torch.roll(u, -1), torch.roll(u, 1)
                u = u - cadv * u * (up - um) + cdif * (up - 2.0 * u + um)
                tc = tc + float(dt.detach())
        return (u * u).sum()
    out = _grad_jvp_hvp(f, a, d)
    return dict(sizes=np.array([n, nsteps]), tend=np.array(tend), **a, **{k + "_dir": v for k, v in d.items()}, **out)


def main():
    for name, make, seed in (("mlp2_ce", mlp, 3), ("conv3x3", conv, 4), ("affine_lsq", affine, 1), ("diffusion2d", diffusion, 2),
                             ("burgers1d", burgers, 5)):
        rng = np.random.default_rng(seed)
        fx = make(rng)
        np.savez(OUT / f"{name}.npz", **fx)
        print(f"wrote {name}.npz ({len(fx)} arrays)")


if __name__ == "__main__":
    main()
