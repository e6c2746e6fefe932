"""The transpiled oracle against the reference's own generated code.

/root/reference/test/val-corpus holds STADE's committed `_b/_d/_hv.jl` snapshots (generated
with keep_push_pop = false, fuse_ii_loops = true, test/validate_corpus.jl:23).  Every one
must transpile and compile, and on a set of kernels chosen to cover the constructs of the
five configs (flattened nests, div/mod indices, scatter-accumulate, stencils, indexed
stacks, branch stacks, tanh, scalar returns) the generated adjoint, tangent and HVP must
pass the reference's own oracles (validate_corpus.jl:1-93): the exact dot-product identity
to 1e-11 and central differences to 1e-3.  A planted mistake in the oracle's input must
fail the identity.  Skipped where the reference is not mounted (the GPU box).
"""
import glob
import os

import numpy as np
import pytest

from helpers import REF_CORPUS

pytestmark = pytest.mark.skipif(not REF_CORPUS.exists(), reason="reference corpus not mounted")

CASES = {
    "affine_loss": (dict(i_n=7), dict(loss=1, u=7, a=7, b=7, v=7)),
    "matvec_loss": (dict(i_m=5, i_n=4), dict(loss=1, a=(5, 4), u=4, v=5)),
    "stencil_loss": (dict(i_n=9), dict(loss=1, u=9, w=9)),
    "dotprod": (dict(i_n=6), dict(loss=1, u=6, v=6)),
    "advection": (dict(i_nstep=3, i_nnode=8), dict(u=8, du=8)),
    "mlp1d": (dict(n_h=4), dict(loss=1, x=1, y=1, w1=4, b1=4, w2=16, b2=4, w3=4, b3=1, h1=4, h2=4, o=1)),
    "fixed_sweeps": (dict(i_n=5), dict(y=5, x=5)),
    "bnd_branch": (dict(i_n=6, i_m=4), dict(x=6, flag=6, out=6)),
    "selfrace_conv": (dict(i_n=6, i_nc=3), dict(x=9, w=3, z=6, loss=1)),
    "relu_field": (dict(i_n=8), dict(loss=1, u=8, v=8)),
    "clamped_sumsq": (dict(i_n=8), dict(loss=1, u=8)),
    "geomrecur": (dict(i_n=6), dict(loss=1, u=6)),
    "sumsq_shifted": (dict(i_n=5), dict(loss=1, u=5)),
    "two_field_loss": (dict(i_n=5), dict(loss=1, u=5, v=5, p=5, q=5)),
    "bilinear": (dict(i_m=4, i_n=3), dict(loss=1, x=4, a=(4, 3), y=3)),
}


def test_every_fixture_transpiles():
    from oracle import runner
    files = sorted(glob.glob(str(REF_CORPUS / "*_b.jl")) + glob.glob(str(REF_CORPUS / "*_d.jl")) + glob.glob(str(REF_CORPUS / "*_hv.jl")))
    assert len(files) >= 400
    import concurrent.futures as cf

    def one(p):
        try:
            runner.load(p)
            return None
        except Exception as e:  # noqa: BLE001
            return (os.path.basename(p), str(e)[:120])
    with cf.ThreadPoolExecutor(min(8, os.cpu_count() or 1)) as ex:
        bad = [r for r in ex.map(one, files) if r is not None]
    assert not bad, bad


def _setup(name):
    from oracle import checks, runner, rng as jrng
    ints, shapes = CASES[name]
    ld = runner.load(REF_CORPUS / f"{name}_d.jl")
    lb = runner.load(REF_CORPUS / f"{name}_b.jl")
    lh = runner.load(REF_CORPUS / f"{name}_hv.jl")
    k = checks.kernel_from_lib(ld, name, ints, shapes)
    base = checks.random_values(k, jrng.Xoshiro(jrng.val_stable_seed(name)), base=True)
    return checks, ld, lb, lh, k, base, jrng.val_stable_seed(name) + 1


@pytest.mark.parametrize("name", sorted(CASES))
def test_reference_oracles(name):
    checks, ld, lb, lh, k, base, s = _setup(name)
    assert checks.dotprod(ld, lb, k, base, s) <= 1e-11
    assert checks.fd_adjoint(ld, lb, k, base, s) <= 1e-3
    assert checks.fd_tangent(ld, ld, k, base, s) <= 1e-3
    assert checks.fd_hvp(lb, lh, k, base, s) <= 1e-3


def test_planted_mistake_fails_the_identity():
    """A dropped factor in the adjoint (2 v -> 3 v) must break <yb, J xd> = <J' yb, xd>."""
    from oracle import checks, runner, rng as jrng
    text = (REF_CORPUS / "affine_loss_b.jl").read_text()
    bad = text.replace("(2 * v[i_x2]) * lossb[1]", "(3 * v[i_x2]) * lossb[1]")
    assert bad != text
    ld = runner.load(REF_CORPUS / "affine_loss_d.jl")
    lb = runner.load(bad, tag="affine_loss_b_planted")
    ints, shapes = CASES["affine_loss"]
    k = checks.kernel_from_lib(ld, "affine_loss", ints, shapes)
    base = checks.random_values(k, jrng.Xoshiro(7), base=True)
    assert checks.dotprod(ld, lb, k, base, 8) > 1e-3
    # and a wrong index (a transposed operand) in the tangent
    t2 = (REF_CORPUS / "matvec_loss_d.jl").read_text().replace("ad[i_i, i_j]", "ad[i_j, i_i]")
    ld2 = runner.load(t2, tag="matvec_loss_d_planted")
    lb2 = runner.load(REF_CORPUS / "matvec_loss_b.jl")
    k2 = checks.kernel_from_lib(lb2, "matvec_loss", dict(i_m=4, i_n=4), dict(loss=1, a=(4, 4), u=4, v=4))
    base2 = checks.random_values(k2, jrng.Xoshiro(9), base=True)
    assert checks.dotprod(ld2, lb2, k2, base2, 10) > 1e-3


def test_julia_semantics_units():
    """Floored mod, truncated div, literal powers, juxtaposition, NaN max, empty ranges."""
    from oracle import runner
    src = '''
function sem(out, iout, a, b, x)
    iout[1] = mod(a, b)
    iout[2] = div(a, b)
    iout[3] = mod(-a, b)
    iout[4] = div(-a, b)
    out[1] = x ^ 2
    out[2] = 1 / 2x
    out[3] = -x ^ 2
    out[4] = max(x, 0.0 / 0.0)
    out[5] = 2 ^ 3
    s = 0.0
    for k = 5:4
        s = s + 1.0
    end
    out[6] = s
    for k = 3:-1:1
        s = s + k
    end
    out[7] = s
    out[8] = sign(0.0)
    return nothing
end
'''
    lib = runner.load(src, tag="semantics")
    out = np.zeros(8)
    iout = np.zeros(4, dtype=np.int64)
    lib.call("sem", out, iout, 7, 3, 3.0)
    assert list(iout) == [1, 2, 2, -2]
    assert out[0] == 9.0 and out[1] == 1.0 / 6.0 and out[2] == -9.0
    assert np.isnan(out[3]) and out[4] == 8.0 and out[5] == 0.0 and out[6] == 6.0 and out[7] == 0.0
