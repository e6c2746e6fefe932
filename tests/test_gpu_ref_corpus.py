"""The general lowering on the reference's own generated code, on the GPU.

The reference's committed generated files (/root/reference/test/val-corpus: adjoint, tangent
and HVP of every kernel: 417 files of 139 kernels) are
lowered by `build()` where the reference is mounted, into tests/_build/ref_corpus/ with an index
of their entry points.  The expected results are fixtures (tests/golden/make_ref_corpus.py):
the oracle's outputs on seeded inputs (two hand-chosen sizes for the kernels the oracle tests
size and for one whose recurrence needs scaled inputs, the size the reference's validator rule
finds for the others), and the 80-bit truth where it differs.  Each case draws the same inputs from the seed, runs the lowered library through its C
entry point, and compares every output argument, stack and returned scalar with the parity
bars (fp64 1e-12, integers exact) and the truth rule.  The reference's text is not read here."""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from helpers import ParityCase, seeded_inputs

pytestmark = pytest.mark.gpu

GOLD = Path(__file__).resolve().parent / "golden"
GEN = Path(__file__).resolve().parent / "_build" / "ref_corpus"
META = json.loads((GOLD / "ref_corpus.json").read_text())
_Z = {}


def _fixtures():
    if "z" not in _Z:
        _Z["z"] = np.load(GOLD / "ref_corpus.npz")
    return _Z["z"]


def _index():
    p = GEN / "ref_corpus_index.json"
    return json.loads(p.read_text()) if p.exists() else None


@pytest.mark.parametrize("case", META, ids=[m["key"] for m in META])
def test_lowered_reference_kernel(case):
    index = _index()
    if index is None or case["fname"] not in index or not (GEN / index[case["fname"]]["lib"]).exists():
        pytest.skip("the lowered reference kernels are built by build() where /root/reference is mounted")
    from stade_hip.lower.runtime import LoweredLib
    z = _fixtures()
    key, fname = case["key"], case["fname"]
    entry = index[fname]
    sig = dict(entry["sig"])
    sig["args"] = [tuple(x) for x in sig["args"]]
    low = LoweredLib(GEN / entry["lib"], {fname: sig}, "f64", None)
    ia = {a: z[f"{key}/in/{a}"] for a, kind, _, _ in case["args"] if kind == "Ai"}
    args = seeded_inputs(case["args"], case["ints"], case["seed"], ia, zeros=case.get("zeros", ()),
                         scales=case.get("scales"))
    stacks = [(s, (n, k)) for s, n, k in case["stacks"]]
    dims = {a: v.shape for a, _, v in args if isinstance(v, np.ndarray) and v.ndim > 1}
    print(f"reference {key}: {len(args)} arguments, plan {sig.get('plan')}", flush=True)
    pc = ParityCase(case["name"], case["mode"], args, stacks, "f64", label=f"reference {key}",
                    runner=lambda dev, sd: low.call(fname, *dev, *sd, shapes=dims),
                    partial=(sig.get("finish") or {}).get("dead_stacks", ()))
    # the oracle's results (an output left equal to its input is not stored) and the truth
    host, th = [], []
    for a, kind, v in args:
        if not isinstance(v, np.ndarray):
            host.append(v)
            th.append(v)
            continue
        out = z[f"{key}/out/{a}"] if f"{key}/out/{a}" in z else np.ravel(v, order="F")
        host.append(out)
        th.append(z[f"{key}/truth/{a}"] if f"{key}/truth/{a}" in z else out)
    pc.host = host
    pc.stack_h = [z[f"{key}/out/{s}"] for s, _ in stacks]
    pc.ret_h = tuple(case["ret"])
    pc._truth = dict(arrays=th, stacks=[z[f"{key}/truth/{s}"] if f"{key}/truth/{s}" in z else z[f"{key}/out/{s}"]
                                        for s, _ in stacks],
                     ret=tuple(np.longdouble(x) if isinstance(x, str) else x for x in case["ret_truth"]))
    pc.run_gpu()
    print(f"reference {key}: worst {pc.compare():.3e}", flush=True)
