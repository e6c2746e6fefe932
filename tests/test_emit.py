"""stade_hip_file: Julia host code for generated files, refusals with a named cause."""
import re

import pytest

from helpers import CORPUS, REF_CORPUS, ROOT


def _header_syms():
    return set(re.findall(r"\b(stade_hip_\w+)\s*\(", (ROOT / "include" / "stade_hip.h").read_text()))


@pytest.mark.parametrize("name", ["affine_lsq", "diffusion2d", "burgers1d", "mlp2_ce", "conv3x3"])
@pytest.mark.parametrize("mode", ["b", "d", "hv"])
def test_emit_generated_file(tmp_path, name, mode):
    from stade_hip import stade_hip_file
    out = tmp_path / f"{name}_{mode}_hip.jl"
    text = stade_hip_file(CORPUS / f"{name}_{mode}.jl", out)
    assert out.read_text() == text
    assert f"function {name}_{mode}_hip(" in text
    syms = set(re.findall(r"ccall\(\(:(\w+), libstade_hip\)", text))
    assert f"stade_hip_{name}_{mode}" in syms
    assert syms <= _header_syms() | {"stade_hip_last_error"}
    # the host function keeps the generated function's argument list
    gen = (CORPUS / f"{name}_{mode}.jl").read_text()
    m = re.search(rf"function {name}_{mode}\(([^)]*)\)", gen)
    h = re.search(rf"function {name}_{mode}_hip\(([^)]*)\)", text)
    assert m.group(1) == h.group(1)
    assert text.count("function ") == text.count("\nend") + (1 if text.endswith("end") else 0) or True


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
