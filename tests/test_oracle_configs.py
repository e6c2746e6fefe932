"""The config kernel texts (stade.jl_amd/corpus) pinned by the reference's oracles and by
closed forms.

The generated `_b/_d/_hv` texts of the five configs were derived by hand from the primals
by STADE's rules (Julia is not available to run the generator).  Their text parity with
STADE is therefore unpinned; their numbers are pinned here:

* the reference's exact dot-product identity (1e-11) and central differences (1e-3) for
  the adjoint, tangent and HVP (`val_validate_*` /root/reference/src/STADE.jl:16334-17153);
* closed forms: affine (r = W x + b - t, Wb = r x' lossb, xb = W' r lossb, ...), diffusion
  (un = A u with the periodic 5-point matrix A built by brute force, ub = A' unb_total);
* the indexed tape: the u_stack index of the Burgers adjoint is a bijection of
  (step, cell) onto 1:nsteps*n with the cell loop as the fastest digit
  (/root/reference/test/validate_layout_bijection.jl), and the guard's branch stack is
  1 for the steps that ran and 0 after.
"""
import numpy as np
import pytest

from helpers import CORPUS, oracle_lib

CASES = {
    "affine_lsq": (dict(i_m=5, i_n=4), dict(loss=1, w=(5, 4), x=4, b=5, t=5, r=5), {}),
    "diffusion2d": (dict(n=5), dict(loss=1, u=25, un=25), {}),
    "burgers1d": (dict(n=7, nsteps=4), dict(loss=1, u=7, un=7), dict(nu=0.05, dt=0.1, dx=0.5, tend=100.0)),
}


def _setup(name):
    from oracle import checks, rng as jrng
    ints, shapes, sc = CASES[name]
    ld, lb, lh = oracle_lib(name, "d"), oracle_lib(name, "b"), oracle_lib(name, "hv")
    k = checks.kernel_from_lib(ld, name, ints, shapes, init_scalars=sc)
    base = checks.random_values(k, jrng.Xoshiro(jrng.val_stable_seed(name)), base=True)
    return checks, ld, lb, lh, k, base, jrng.val_stable_seed(name) + 1


@pytest.mark.parametrize("name", sorted(CASES))
def test_config_reference_oracles(name):
    checks, ld, lb, lh, k, base, s = _setup(name)
    assert checks.dotprod(ld, lb, k, base, s) <= 1e-11
    assert checks.fd_adjoint(ld, lb, k, base, s) <= 1e-3
    assert checks.fd_tangent(ld, ld, k, base, s) <= 1e-3
    assert checks.fd_hvp(lb, lh, k, base, s) <= 1e-3


@pytest.mark.parametrize("name", sorted(CASES))
def test_hvp_adjoint_part_equals_adjoint(name):
    """The xb half of the HVP is the adjoint itself (forward-over-reverse keeps the primal sweep)."""
    checks, ld, lb, lh, k, base, s = _setup(name)
    from oracle import rng as jrng
    g = jrng.Xoshiro(s)
    yb, xd, ybd = checks.random_values(k, g), checks.random_values(k, g), checks.random_values(k, g)
    xb = checks.call_adjoint(lb, k, base, yb)
    xb2, _ = checks.call_hvp(lh, k, base, yb, xd, ybd)
    np.testing.assert_allclose(xb2, xb, rtol=1e-13, atol=1e-13)


def test_affine_closed_form():
    from oracle import rng as jrng
    m, n = 6, 5
    g = jrng.Xoshiro(11)
    W = np.asfortranarray(jrng.rand_uniform(g, m * n, -1, 1).reshape((m, n), order="F"))
    x, b, t = (jrng.val_randn(g, k) for k in (n, m, m))
    lb = oracle_lib("affine_lsq", "b")
    Wb = np.asfortranarray(np.zeros((m, n)))
    xb, bb, tb, r, rb = np.zeros(n), np.zeros(m), np.zeros(m), np.zeros(m), np.zeros(m)
    loss, lossb = np.array([0.25]), np.array([1.5])
    lb.call("affine_lsq_b", loss, lossb, W.copy(order="F"), Wb, x.copy(), xb, b.copy(), bb, t.copy(), tb, r, rb, m, n)
    res = W @ x + b - t
    np.testing.assert_allclose(r, res, rtol=1e-14, atol=1e-14)
    np.testing.assert_allclose(loss[0], 0.25 + 0.5 * res @ res, rtol=1e-14)
    np.testing.assert_allclose(Wb, np.outer(res, x) * 1.5, rtol=1e-13, atol=1e-13)
    np.testing.assert_allclose(xb, W.T @ res * 1.5, rtol=1e-13, atol=1e-13)
    np.testing.assert_allclose(bb, res * 1.5, rtol=1e-14, atol=1e-14)
    np.testing.assert_allclose(tb, -res * 1.5, rtol=1e-14, atol=1e-14)
    assert np.all(rb == 0)
    # tangent: lossd = sum r * (Wd x + W xd + bd - td)
    ld = oracle_lib("affine_lsq", "d")
    Wd = np.asfortranarray(jrng.val_randn(g, m * n).reshape((m, n), order="F"))
    xd, bd, td = (jrng.val_randn(g, k) for k in (n, m, m))
    loss, lossd, r, rd = np.zeros(1), np.zeros(1), np.zeros(m), np.zeros(m)
    ld.call("affine_lsq_d", loss, lossd, W.copy(order="F"), Wd, x.copy(), xd, b.copy(), bd, t.copy(), td, r, rd, m, n)
    np.testing.assert_allclose(lossd[0], res @ (Wd @ x + W @ xd + bd - td), rtol=1e-13)


def _diffusion_matrix(n):
    """The periodic 5-point matrix A (un = A u), built entry by entry; A[c, k] accumulates so
    that coincident neighbours (n = 1, 2) count with their multiplicity."""
    N = n * n
    A = np.zeros((N, N))
    for j in range(n):
        for i in range(n):
            c = j * n + i
            A[c, c] += 1.0 - 0.4
            for (ii, jj) in (((i - 1) % n, j), ((i + 1) % n, j), (i, (j - 1) % n), (i, (j + 1) % n)):
                A[c, jj * n + ii] += 0.1
    return A


@pytest.mark.parametrize("n", [1, 2, 3, 4, 5, 7, 9])
def test_diffusion_brute_force(n):
    from oracle import rng as jrng
    g = jrng.Xoshiro(100 + n)
    u, ub0, unb0 = (jrng.val_randn(g, n * n) for _ in range(3))
    A = _diffusion_matrix(n)
    assert np.allclose(A, A.T)
    lb = oracle_lib("diffusion2d", "b")
    loss, lossb = np.array([0.5]), np.array([0.75])
    ub, un, unb = ub0.copy(), np.zeros(n * n), unb0.copy()
    lb.call("diffusion2d_b", loss, lossb, u.copy(), ub, un, unb, n)
    un_ref = A @ u
    np.testing.assert_allclose(un, un_ref, rtol=1e-13, atol=1e-13)
    np.testing.assert_allclose(loss[0], 0.5 + un_ref @ un_ref, rtol=1e-13)
    w = unb0 + 2 * un_ref * 0.75
    np.testing.assert_allclose(ub, ub0 + A.T @ w, rtol=1e-12, atol=1e-12)
    assert np.all(unb == 0)


def test_burgers_tape_layout_and_guard():
    from oracle import checks, rng as jrng
    lb = oracle_lib("burgers1d", "b")
    n, T = 7, 6
    k = checks.kernel_from_lib(lb, "burgers1d", dict(n=n, nsteps=T), dict(loss=1, u=n, un=n),
                               init_scalars=dict(nu=0.05, dt=0.1, dx=0.5, tend=0.35))
    base = checks.random_values(k, jrng.Xoshiro(3), base=True)
    yb = checks.random_values(k, jrng.Xoshiro(4))
    _, vals, ybs, (branch, tape) = checks.call_adjoint(lb, k, base, yb, return_state=True)
    # tc = 0, 0.1, 0.2, 0.30000000000000004 < 0.35: four steps ran
    assert list(branch) == [1, 1, 1, 1, 0, 0]
    t = tape.reshape(T, n)
    assert np.all(np.isfinite(t[:4])) and np.all(np.isnan(t[4:]))
    np.testing.assert_array_equal(t[0], base["u"])
    np.testing.assert_array_equal(vals["u"], base["u"])          # restored by the reverse sweep
    # the index formula ((i_x2 - 1) + (i_t - 1) * (div(n - 1, 1) + 1)) + 1 is a bijection, cell fastest
    idx = sorted(((ix - 1) + (it - 1) * ((n - 1) // 1 + 1)) + 1 for it in range(1, T + 1) for ix in range(1, n + 1))
    assert idx == list(range(1, T * n + 1))
    assert ((2 - 1) + (1 - 1) * n + 1) - ((1 - 1) + (1 - 1) * n + 1) == 1
