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
    "Int32": "int32_t", "Cstring": "char*", "Float32": "float", "Bool": "bool",
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
        sym = re.match(r"\(:(\w+), (libstade_hip|libstade_gen)\)", parts[0]).group(1)
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


def test_unknown_kernel_refused_without_the_general_path(tmp_path):
    from stade_hip import stade_hip_file
    from stade_hip.emit import StadeHipRefusal
    src = tmp_path / "other_b.jl"
    src.write_text((CORPUS / "diffusion2d_b.jl").read_text().replace("0.1 * (u[(j - 1) * n + im]", "0.2 * (u[(j - 1) * n + im]"))
    with pytest.raises(StadeHipRefusal, match="no kernel implemented"):
        stade_hip_file(src, tmp_path / "o.jl", general=False)


@pytest.mark.skipif(not REF_CORPUS.exists(), reason="reference corpus not mounted")
def test_reference_corpus_kernel_refused_without_the_general_path(tmp_path):
    from stade_hip import stade_hip_file
    from stade_hip.emit import StadeHipRefusal
    with pytest.raises(StadeHipRefusal):
        stade_hip_file(REF_CORPUS / "affine_loss_b.jl", tmp_path / "o.jl", general=False)


def test_lowering_refusal_names_the_cause(tmp_path):
    from stade_hip import stade_hip_file
    from stade_hip.emit import StadeHipRefusal
    src = tmp_path / "odd_b.jl"
    src.write_text("function odd_b(x, xb, n)\n    for i = 1:n\n        xb[i] = xb[i] + frobnicate(x[i])\n    end\n"
                   "    return nothing\nend\n")
    with pytest.raises(StadeHipRefusal, match="general lowering cannot take"):
        stade_hip_file(src, tmp_path / "o.jl")


def _gen_prototypes(text: str) -> dict[str, tuple[str, list[str]]]:
    """name -> (return type, [parameter types]) of the extern "C" functions in lowered HIP source."""
    from stade_hip.lower import hipgen
    src, _ = hipgen.generate(text)
    out = {}
    for m in re.finditer(r'extern "C" (?:const )?([\w*]+\*?)\s+(stade_hip_gen_\w+)\(([^)]*)\)', src):
        types = []
        for prm in m.group(3).split(","):
            prm = " ".join(prm.split())
            if not prm or prm == "void":
                continue
            types.append(re.match(r"(.*?)\s*\w+$", prm).group(1).replace("const ", "").replace(" *", "*"))
        out[m.group(2)] = (m.group(1), types)
    return out


GENERIC_FILES = [f"{k}_{m}" for k in ("matvec_scatter", "window1d", "binsum") for m in ("b", "d", "hv")]


def _check_lowered(text: str, gen_text: str) -> list[str]:
    protos = _gen_prototypes(gen_text)
    protos["stade_hip_gen_last_error"] = ("char*", [])
    bad = []
    for sym, ret, jtypes, vals in _ccalls(text):
        cret, ctys = protos[sym]
        if JL2C[ret] != cret:
            bad.append(f"{sym}: returns {cret}, ccall says {ret}")
        if len(jtypes) != len(ctys) or len(vals) != len(jtypes):
            bad.append(f"{sym}: {len(ctys)} parameters, ccall {len(jtypes)} types and {len(vals)} values")
            continue
        bad += [f"{sym} parameter {k}: C {ct}, ccall {jt}" for k, (jt, ct) in enumerate(zip(jtypes, ctys)) if JL2C[jt] != ct]
    return bad


@pytest.mark.parametrize("name", GENERIC_FILES)
def test_lowered_emission_ccall_types(tmp_path, name):
    """A file no hand-written kernel implements goes through the general lowering: one host
    function per generated function, keeping its argument list, whose ccall into the lowered
    library matches the generated C prototype type by type (arrays: pointer and Julia
    dimensions; Int64, Float64 by value; two host return buffers; the stream)."""
    from stade_hip import stade_hip_file
    src = CORPUS / "generic" / f"{name}.jl"
    text = stade_hip_file(src, tmp_path / "o.jl")
    assert "const libstade_gen = " in text
    gen = src.read_text()
    for fn, args in re.findall(r"^function (\w+)\(([^)]*)\)", gen, re.M):
        h = re.search(rf"^function {fn}_hip\(([^)]*)\)", text, re.M)
        assert h and h.group(1) == args, fn
    lines = text.splitlines()
    assert sum(ln.startswith("function ") for ln in lines) == sum(ln == "end" for ln in lines)
    calls = _ccalls(text)
    assert len(calls) == text.count("ccall(("), "a ccall the checker could not parse"
    assert _check_lowered(text, gen) == []


def test_lowered_ccall_checker_catches_a_wrong_type(tmp_path, monkeypatch):
    """The check above fails on a planted mistake: Float64 arrays emitted as Ptr{Float32}."""
    from stade_hip import emit, stade_hip_file
    real = emit._lowered_call
    monkeypatch.setattr(emit, "_lowered_call", lambda f, sig, c, et: real(f, sig, c, "Float32"))
    src = CORPUS / "generic" / "window1d_b.jl"
    text = stade_hip_file(src, tmp_path / "o.jl")
    assert any("Ptr{Float32}" in b for b in _check_lowered(text, src.read_text()))


def test_lowered_initstacks_allocate_on_the_device(tmp_path):
    from stade_hip.emit import _lowered_initstacks
    body = (CORPUS / "burgers1d_b.jl").read_text().split("\nend\n")[0] + "\nend"
    out = _lowered_initstacks("initstacks_burgers1d_b", body, "Float64")
    assert "function initstacks_burgers1d_b_hip(n, nsteps)" in out
    assert "branch_stack = ROCArray{Int64}(undef, max(0, div(nsteps - 1, 1) + 1))" in out
    assert "u_stack = ROCArray{Float64}(undef, " in out and "Vector{" not in out


@pytest.mark.skipif(not REF_CORPUS.exists(), reason="reference corpus not mounted")
def test_lowered_initstacks_fill_index_arrays_on_the_host():
    """An initstacks_* that fills index arrays element by element (indexed stacks: prefix
    offsets and saved loop values) keeps them host Vectors while it fills them and uploads them
    where it returns them; its stacks are allocated on the device; its counts pass through."""
    from stade_hip import emit
    text = (REF_CORPUS / "windowed_relax_retire_b.jl").read_text()
    _, body = emit._split_functions(text)["initstacks_windowed_relax_retire_b"]
    out = emit._lowered_initstacks("initstacks_windowed_relax_retire_b", body, "Float64")
    assert out.startswith("function initstacks_windowed_relax_retire_b_hip(dx, num_passes, w0)")
    for nm in ("prefix_branch_stack_1", "prefix_left_stack_1", "val_w_1"):
        assert re.search(rf"^\s*{nm} = Vector\{{Int(64)?\}}\(undef,", out, re.M), nm
        assert f"ROCArray({nm})" in out, nm
    for nm, t in (("branch_stack", "Int64"), ("left_stack", "Float64"), ("right_stack", "Float64")):
        assert re.search(rf"^\s*{nm} = ROCArray\{{{t}\}}\(undef,", out, re.M), nm
    ret = [ln for ln in out.splitlines() if ln.strip().startswith("return")][0]
    assert "__tot_branch_stack_1," in ret and "ROCArray(__tot" not in ret


def test_ccall_checker_catches_a_wrong_type(tmp_path, monkeypatch):
    """The check above fails on a planted mistake: the MLP's arrays emitted as Float64."""
    import dataclasses
    from stade_hip import emit
    monkeypatch.setitem(emit.KERNELS, "mlp2_ce", dataclasses.replace(emit.KERNELS["mlp2_ce"], eltype="Float64"))
    text = emit.stade_hip_file(CORPUS / "mlp2_ce_b.jl", tmp_path / "o.jl")
    protos = _prototypes()
    sym, ret, jtypes, vals = next(c for c in _ccalls(text) if c[0] == "stade_hip_mlp2_ce_b")
    assert any(JL2C[jt] != ct for jt, ct in zip(jtypes, protos[sym][1]))


@pytest.mark.parametrize("src", [f"{k}_{m}" for k in NAMES for m in ("b", "d", "hv")] + [f"generic/{g}" for g in GENERIC_FILES])
@pytest.mark.parametrize("inbounds", [True, False])
def test_emitted_lines_are_forms_the_gpu_tests_execute(tmp_path, src, inbounds):
    """Every statement of the emitted host functions is one of the forms tests/jlhost.py
    executes on the GPU, so those tests run the emitted text as written."""
    from jlhost import JlHost
    from stade_hip import stade_hip_file
    host = JlHost(stade_hip_file(CORPUS / f"{src}.jl", tmp_path / "o.jl", inbounds=inbounds))
    assert host.funcs
    assert host.unknown_lines() == []
