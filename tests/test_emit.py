"""stade_hip_file: Julia host code for generated files, refusals with a named cause, and the
emitted `ccall`s checked argument by argument against the C prototypes of include/stade_hip.h."""
import re

import pytest

from helpers import CORPUS, REF_CORPUS, ROOT

NAMES = ["affine_lsq", "diffusion2d", "burgers1d", "mlp2_ce", "conv3x3"]


def _prototypes() -> dict[str, tuple[str, list[str]]]:
    """name -> (return type, [parameter types]) of every function the header declares."""
    text = (ROOT / "include" / "stade_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    out = {}
    for m in re.finditer(r"([A-Za-z_][\w ]*?\*?)\s*\b(stade_hip_\w+)\s*\(([^;{]*)\)\s*;", text, re.S):
        ret, name, params = m.group(1).strip(), m.group(2), m.group(3)
        types = []
        for prm in params.split(","):
            prm = " ".join(prm.split())
            if not prm or prm == "void":
                continue
            # drop the parameter name (and an array suffix such as `[2]`, a pointer in C)
            mm = re.match(r"(.*?)(\w+)(\[\d*\])?$", prm)
            t = mm.group(1).strip() + ("*" if mm.group(3) else "")
            types.append(t.replace(" *", "*").replace("const ", ""))
        out[name] = (ret.replace("const ", "").replace(" *", "*"), types)
    return out


# Julia ccall type -> C parameter type (const dropped), one to one
JL2C = {
    "Ptr{Float64}": "double*", "Ptr{Float32}": "float*", "Ref{Float64}": "double*", "Ptr{Int64}": "int64_t*",
    "Int64": "int64_t", "Float64": "double", "Ptr{Cvoid}": "hipStream_t", "Ref{Int32}": "int32_t*",
    "Int32": "int32_t", "Cstring": "char*",
}


def _split_top(s: str) -> list[str]:
    """Split at the commas outside any (), {} or []."""
    out, depth, cur = [], 0, ""
    for ch in s:
        if ch in "({[":
            depth += 1
        elif ch in ")}]":
            depth -= 1
        if ch == "," and depth == 0:
            out.append(cur.strip())
            cur = ""
        else:
            cur += ch
    if cur.strip():
        out.append(cur.strip())
    return out


def _ccalls(text: str):
    """(symbol, return type, [argument types], [argument values]) of every emitted ccall."""
    out = []
    for m in re.finditer(r"ccall\(", text):
        i, depth = m.end(), 1
        while depth:
            depth += {"(": 1, ")": -1}.get(text[i], 0)
            i += 1
        parts = _split_top(text[m.end():i - 1])
        sym = re.match(r"\(:(\w+), libstade_hip\)", parts[0]).group(1)
        types = parts[2].strip()
        assert types.startswith("(") and types.endswith(")"), types
        out.append((sym, parts[1], _split_top(types[1:-1]), parts[3:]))
    return out


@pytest.mark.parametrize("name", NAMES)
@pytest.mark.parametrize("mode", ["b", "d", "hv"])
def test_emit_generated_file(tmp_path, name, mode):
    from stade_hip import stade_hip_file
    out = tmp_path / f"{name}_{mode}_hip.jl"
    text = stade_hip_file(CORPUS / f"{name}_{mode}.jl", out)
    assert out.read_text() == text
    assert f"function {name}_{mode}_hip(" in text
    protos = _prototypes()
    syms = set(re.findall(r"ccall\(\(:(\w+), libstade_hip\)", text))
    assert f"stade_hip_{name}_{mode}" in syms
    assert syms <= set(protos), syms - set(protos)
    # the host function keeps the generated function's argument list
    gen = (CORPUS / f"{name}_{mode}.jl").read_text()
    m = re.search(rf"function {name}_{mode}\(([^)]*)\)", gen)
    h = re.search(rf"function {name}_{mode}_hip\(([^)]*)\)", text)
    assert m.group(1) == h.group(1)
    # one `end` at column 0 closes each top-level function
    lines = text.splitlines()
    assert sum(ln.startswith("function ") for ln in lines) == sum(ln == "end" for ln in lines)


@pytest.mark.parametrize("name", NAMES)
@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("inbounds", [True, False])
def test_emitted_ccall_types_match_header(tmp_path, name, mode, inbounds):
    """Each emitted ccall's return and argument types map one to one onto the prototype of
    the symbol in include/stade_hip.h (Ptr{Float64} <-> double*, Ptr{Float32} <-> float*,
    Ref{Float64} <-> a host double*, Int64 <-> int64_t, Ptr{Int64} <-> int64_t*, Ptr{Cvoid} <->
    hipStream_t), with as many values as types."""
    from stade_hip import stade_hip_file
    text = stade_hip_file(CORPUS / f"{name}_{mode}.jl", tmp_path / "o.jl", inbounds=inbounds)
    protos = _prototypes()
    calls = _ccalls(text)
    assert len(calls) == text.count("ccall(("), "a ccall the checker could not parse"
    seen = set()
    for sym, ret, jtypes, vals in calls:
        cret, ctypes_ = protos[sym]
        assert JL2C[ret] == cret.replace("const ", ""), f"{sym}: returns {cret}, ccall says {ret}"
        assert len(jtypes) == len(ctypes_), f"{sym}: {len(ctypes_)} parameters, ccall passes {len(jtypes)}"
        for k, (jt, ct) in enumerate(zip(jtypes, ctypes_)):
            assert JL2C[jt] == ct, f"{sym} parameter {k}: C {ct}, ccall {jt}"
        assert len(vals) == len(jtypes), f"{sym}: {len(jtypes)} types, {len(vals)} values"
        seen.add(sym)
    assert (("stade_hip_device_error" in seen) == (not inbounds and name == "mlp2_ce")), seen


def test_emitted_bounds_check_for_labels(tmp_path):
    from stade_hip import stade_hip_file
    text = stade_hip_file(CORPUS / "mlp2_ce_b.jl", tmp_path / "o.jl", inbounds=False)
    assert "throw(BoundsError(lab))" in text
    assert "stade_hip_device_error" not in stade_hip_file(CORPUS / "mlp2_ce_b.jl", tmp_path / "p.jl")


def test_refuses_unknown_kernel(tmp_path):
    from stade_hip import stade_hip_file
    from stade_hip.emit import StadeHipRefusal
    src = tmp_path / "other_b.jl"
    src.write_text((CORPUS / "diffusion2d_b.jl").read_text().replace("0.1 * (u[(j - 1) * n + im]", "0.2 * (u[(j - 1) * n + im]"))
    with pytest.raises(StadeHipRefusal, match="no kernel implemented"):
        stade_hip_file(src, tmp_path / "o.jl")


@pytest.mark.skipif(not REF_CORPUS.exists(), reason="reference corpus not mounted")
def test_refuses_reference_corpus_kernel(tmp_path):
    from stade_hip import stade_hip_file
    from stade_hip.emit import StadeHipRefusal
    with pytest.raises(StadeHipRefusal):
        stade_hip_file(REF_CORPUS / "affine_loss_b.jl", tmp_path / "o.jl")


def test_ccall_checker_catches_a_wrong_type(tmp_path, monkeypatch):
    """The check above fails on a planted mistake: the MLP's arrays emitted as Float64."""
    import dataclasses
    from stade_hip import emit
    monkeypatch.setitem(emit.KERNELS, "mlp2_ce", dataclasses.replace(emit.KERNELS["mlp2_ce"], eltype="Float64"))
    text = emit.stade_hip_file(CORPUS / "mlp2_ce_b.jl", tmp_path / "o.jl")
    protos = _prototypes()
    sym, ret, jtypes, vals = next(c for c in _ccalls(text) if c[0] == "stade_hip_mlp2_ce_b")
    assert any(JL2C[jt] != ct for jt, ct in zip(jtypes, protos[sym][1]))
