"""`stade_hip_file(in_path, out_path; ...)`: Julia host code that runs generated STADE
derivative code on libstade_hip.so.

It keeps the shape of the reference's `stade_amdgpu_file(in_path, out_path; precision,
reduction_threshold, inbounds, dead_scalars)` (/root/reference/src/STADE.jl:18604-18605,
via `stade_gpu_file` 18571-18599): it reads one `.jl` written by `stade_adjoint_file`,
`stade_tangent_file` or `stade_hvp_file` (`io_read_kernel_bundle` 17751) and writes one
`.jl` (`io_write_gpu_file` 17844).  For every generated function of the input it writes a
host function `<name>_hip` with the same arguments, the same in-place effects and the
same return convention as the generated function (`agen_emit` 3672, `hvp_emit`
6772-6779), whose body is one `ccall` into libstade_hip.so:

* `initstacks_<k>_b_hip(sizes...)` allocates the pre-sized stacks as `ROCArray`s
  (`cgen_stack_device_expr` 9798-9802) with the size formulas of the generated
  `initstacks_<k>_b`;
* `<k>_b_hip`, `<k>_d_hip`, `<k>_hv_hip` pass device pointers, Int64 sizes and scalar
  values, return the scalar shadows, and raise `ErrorException` with the library's
  message on a nonzero return code.

The kernel is identified by its primal, which STADE copies verbatim into every generated
file (the trailing `function <k>(...)` of each `_b/_d/_hv` file), compared after removing
comments and blank lines with the primal of `stade.jl_amd/corpus/<k>.jl`.

Any other generated file goes through the general lowering (`stade_hip.lower`): its
functions are written as HIP, built once for gfx950 into `lib/gen/<stem>_<hash>.so`, and
the host functions `ccall` that library's `stade_hip_gen_<name>` entry points.  Arrays
pass a device pointer and their Julia dimensions (the last one folding any further
dimensions), scalars pass by value, the returned scalars come back through two host
buffers (Float64 and Int64 values), and an index outside its array, which every lowered
access checks, throws `BoundsError` as the generated code would.  A file the lowering
cannot take is refused with the reason, as STADE refuses what it cannot port (e.g.
18532-18534).
"""
from __future__ import annotations

import re
from dataclasses import dataclass
from pathlib import Path

CORPUS = Path(__file__).resolve().parent.parent / "corpus"


@dataclass(frozen=True)
class Mode:
    entry: str           # C entry point
    args: tuple          # (julia name, kind) in generated-function order; kinds:
                         #   'A' Float array, 'I' Int64, 'F' Float scalar by value,
                         #   'R' Float scalar shadow (returned), 'S' Int64 stack, 'T' Float stack
    returns: tuple = ()  # names returned, in order


@dataclass(frozen=True)
class KernelSpec:
    name: str
    eltype: str                    # Julia element type of the float arrays
    modes: dict                    # 'b' | 'd' | 'hv' -> Mode
    stacks: tuple = ()             # (name, eltype, julia size expression) of initstacks_<k>_b
    stack_args: tuple = ()         # initstacks_<k>_b arguments
    device_checked: tuple = ()     # Int64 arrays whose values index other arrays on the device
                                   # (an out-of-range value raises the device error flag)


def _a(*names):
    return tuple((n, "A") for n in names)


KERNELS: dict[str, KernelSpec] = {
    "affine_lsq": KernelSpec(
        "affine_lsq", "Float64",
        {
            "b": Mode("stade_hip_affine_lsq_b",
                      _a("loss", "lossb", "w", "wb", "x", "xb", "b", "bb", "t", "tb", "r", "rb") + (("i_m", "I"), ("i_n", "I"))),
            "d": Mode("stade_hip_affine_lsq_d",
                      _a("loss", "lossd", "w", "wd", "x", "xd", "b", "bd", "t", "td", "r", "rd") + (("i_m", "I"), ("i_n", "I"))),
            "hv": Mode("stade_hip_affine_lsq_hv",
                       _a("loss", "lossb", "w", "wb", "x", "xb", "b", "bb", "t", "tb", "r", "rb") + (("i_m", "I"), ("i_n", "I"))
                       + _a("lossd", "lossbd", "wd", "wbd", "xd", "xbd", "bd", "bbd", "td", "tbd", "rd", "rbd")),
        }),
    "diffusion2d": KernelSpec(
        "diffusion2d", "Float64",
        {
            "b": Mode("stade_hip_diffusion2d_b", _a("loss", "lossb", "u", "ub", "un", "unb") + (("n", "I"),)),
            "d": Mode("stade_hip_diffusion2d_d", _a("loss", "lossd", "u", "ud", "un", "und") + (("n", "I"),)),
            "hv": Mode("stade_hip_diffusion2d_hv", _a("loss", "lossb", "u", "ub", "un", "unb") + (("n", "I"),)
                       + _a("lossd", "lossbd", "ud", "ubd", "und", "unbd")),
        }),
    "burgers1d": KernelSpec(
        "burgers1d", "Float64",
        {
            "b": Mode("stade_hip_burgers1d_b",
                      _a("loss", "lossb", "u", "ub", "un", "unb")
                      + (("nu", "F"), ("nub", "R"), ("dt", "F"), ("dtb", "R"), ("dx", "F"), ("dxb", "R"),
                         ("tend", "F"), ("tendb", "R"), ("n", "I"), ("nsteps", "I"))),
            "d": Mode("stade_hip_burgers1d_d",
                      _a("loss", "lossd", "u", "ud", "un", "und")
                      + (("nu", "F"), ("nud", "F"), ("dt", "F"), ("dtd", "F"), ("dx", "F"), ("dxd", "F"),
                         ("tend", "F"), ("tendd", "F"), ("n", "I"), ("nsteps", "I"))),
            "hv": Mode("stade_hip_burgers1d_hv",
                       _a("loss", "lossb", "u", "ub", "un", "unb")
                       + (("nu", "F"), ("nub", "R"), ("dt", "F"), ("dtb", "R"), ("dx", "F"), ("dxb", "R"),
                          ("tend", "F"), ("tendb", "R"), ("n", "I"), ("nsteps", "I"))
                       + _a("lossd", "lossbd", "ud", "ubd", "und", "unbd")
                       + (("nud", "F"), ("nubd", "R"), ("dtd", "F"), ("dtbd", "R"), ("dxd", "F"), ("dxbd", "R"),
                          ("tendd", "F"), ("tendbd", "R"))),
        },
        stacks=(("branch_stack", "Int64", "max(0, div(nsteps - 1, 1) + 1)"),
                ("u_stack", "Float64", "max(0, div(nsteps - 1, 1) + 1) * max(0, div(n - 1, 1) + 1)")),
        stack_args=("n", "nsteps")),
    "mlp2_ce": KernelSpec(
        "mlp2_ce", "Float32",
        {
            "b": Mode("stade_hip_mlp2_ce_b",
                      _a("loss", "lossb", "x", "xb") + (("lab", "L"),) + _a("w1", "w1b", "b1", "b1b", "w2", "w2b", "b2", "b2b",
                                                                         "h1", "h1b", "z", "zb")
                      + (("i_b", "I"), ("i_in", "I"), ("i_h", "I"), ("i_out", "I"))),
            "d": Mode("stade_hip_mlp2_ce_d",
                      _a("loss", "lossd", "x", "xd") + (("lab", "L"),) + _a("w1", "w1d", "b1", "b1d", "w2", "w2d", "b2", "b2d",
                                                                         "h1", "h1d", "z", "zd")
                      + (("i_b", "I"), ("i_in", "I"), ("i_h", "I"), ("i_out", "I"))),
            "hv": Mode("stade_hip_mlp2_ce_hv",
                       _a("loss", "lossb", "x", "xb") + (("lab", "L"),) + _a("w1", "w1b", "b1", "b1b", "w2", "w2b", "b2", "b2b",
                                                                          "h1", "h1b", "z", "zb")
                       + (("i_b", "I"), ("i_in", "I"), ("i_h", "I"), ("i_out", "I"))
                       + _a("lossd", "lossbd", "xd", "xbd", "w1d", "w1bd", "b1d", "b1bd", "w2d", "w2bd", "b2d", "b2bd",
                            "h1d", "h1bd", "zd", "zbd")),
        },
        device_checked=("lab",)),
    "conv3x3": KernelSpec(
        "conv3x3", "Float32",
        {
            "b": Mode("stade_hip_conv3x3_b",
                      _a("loss", "lossb", "xp", "xpb", "w", "wb", "out", "outb")
                      + (("i_nb", "I"), ("i_c", "I"), ("i_k", "I"), ("i_h", "I"), ("i_w", "I"))),
            "d": Mode("stade_hip_conv3x3_d",
                      _a("loss", "lossd", "xp", "xpd", "w", "wd", "out", "outd")
                      + (("i_nb", "I"), ("i_c", "I"), ("i_k", "I"), ("i_h", "I"), ("i_w", "I"))),
            "hv": Mode("stade_hip_conv3x3_hv",
                       _a("loss", "lossb", "xp", "xpb", "w", "wb", "out", "outb")
                       + (("i_nb", "I"), ("i_c", "I"), ("i_k", "I"), ("i_h", "I"), ("i_w", "I"))
                       + _a("lossd", "lossbd", "xpd", "xpbd", "wd", "wbd", "outd", "outbd")),
        }),
}


_FUNC_RE = re.compile(r"^function\s+([A-Za-z_][A-Za-z_0-9!]*)\s*\(([^)]*)\)", re.M)


def _split_functions(text: str) -> dict[str, tuple[list[str], str]]:
    """name -> (argument names, full text) of every top-level `function ... end`."""
    out = {}
    starts = [m for m in _FUNC_RE.finditer(text)]
    for k, m in enumerate(starts):
        end = starts[k + 1].start() if k + 1 < len(starts) else len(text)
        body = text[m.start():end]
        args = [a.split("::")[0].strip() for a in m.group(2).split(",") if a.strip()]
        out.setdefault(m.group(1), (args, body))
    return out


def _normalise(fn_text: str) -> str:
    lines = []
    for ln in fn_text.splitlines():
        ln = ln.split("#", 1)[0].strip()
        if ln:
            lines.append(re.sub(r"\s+", " ", ln))
    # the generated copy of the primal may drop the final `return nothing`
    while lines and lines[-1] in ("end",):
        lines.pop()
    if lines and lines[-1] == "return nothing":
        lines.pop()
    return "\n".join(lines)


def _primal_fingerprint(name: str) -> str:
    text = (CORPUS / f"{name}.jl").read_text()
    funcs = _split_functions(text)
    return _normalise(funcs[name][1])


class StadeHipRefusal(ValueError):
    """The input cannot be executed by libstade_hip: the message names the cause."""


def identify(text: str) -> tuple[KernelSpec, dict]:
    funcs = _split_functions(text)
    for name, spec in KERNELS.items():
        if name in funcs and _normalise(funcs[name][1]) == _primal_fingerprint(name):
            return spec, funcs
    names = ", ".join(sorted(funcs)) or "none"
    raise StadeHipRefusal(f"no kernel implemented by libstade_hip matches the primal in this file "
                          f"(functions found: {names}; implemented: {', '.join(sorted(KERNELS))})")


def _jl_call(spec: KernelSpec, fname: str, mode: Mode, stacks: list[tuple[str, str]], inbounds: bool = True) -> str:
    T = spec.eltype
    sig, types, vals = [], [], []
    rets = []
    for nm, kind in mode.args:
        sig.append(nm)
        if kind == "A":
            types.append(f"Ptr{{{T}}}")
            vals.append(f"pointer({nm})")
        elif kind == "L":
            types.append("Ptr{Int64}")
            vals.append(f"pointer({nm})")
        elif kind == "I":
            types.append("Int64")
            vals.append(f"Int64({nm})")
        elif kind == "F":
            types.append("Float64")
            vals.append(f"Float64({nm})")
        elif kind == "R":
            types.append("Ref{Float64}")
            vals.append(f"__r_{nm}")
            rets.append(nm)
    # an HVP returns (xb, xbd) pairs (`hvp_emit` /root/reference/src/STADE.jl:6772-6779)
    paired = [r for r in rets if not r.endswith("bd")]
    if len(paired) * 2 == len(rets) and all(p + "d" in rets for p in paired):
        rets = [x for p in paired for x in (p, p + "d")]
    for nm, et in stacks:
        sig.append(nm)
        types.append(f"Ptr{{{et}}}")
        vals.append(f"pointer({nm})")
    types.append("Ptr{Cvoid}")
    vals.append("AMDGPU.stream().stream")
    arrays = [nm for nm, kind in mode.args if kind in ("A", "L")] + [nm for nm, _ in stacks]
    lines = [f"function {fname}_hip({', '.join(sig)})"]
    for nm in rets:
        lines.append(f"    __r_{nm} = Ref{{Float64}}({nm})")
    lines.append(f"    GC.@preserve {' '.join(arrays)} begin")
    lines.append(f"        __rc = ccall((:{mode.entry}, libstade_hip), Int32,")
    lines.append(f"                     ({', '.join(types)},),")
    lines.append(f"                     {', '.join(vals)})")
    lines.append("    end")
    lines.append(f"    __rc == 0 || error(\"{mode.entry}: \", unsafe_string(ccall((:stade_hip_last_error, libstade_hip), Cstring, ())))")
    if not inbounds and spec.device_checked:
        # bounds checking on (`inbounds=false`): the device flag, read after the launches,
        # stands for the generated code's BoundsError on an out-of-range index value
        lines.append("    __flag = Ref{Int32}(0)")
        lines.append("    __rc = ccall((:stade_hip_device_error, libstade_hip), Int32, (Ref{Int32},), __flag)")
        lines.append("    __rc == 0 || error(\"stade_hip_device_error: \", unsafe_string(ccall((:stade_hip_last_error, libstade_hip), Cstring, ())))")
        lines.append(f"    __flag[] == 0 || throw(BoundsError({spec.device_checked[0]}))")
    if not rets:
        lines.append("    return nothing")
    elif len(rets) == 1:
        lines.append(f"    return __r_{rets[0]}[]")
    else:
        lines.append("    return (" + ", ".join(f"__r_{r}[]" for r in rets) + ")")
    lines.append("end")
    return "\n".join(lines)


_ALLOC_LINE_RE = re.compile(r"^(\s*)(\w+)\s*=\s*Vector\{(Float64|Float32|Int64|Int)\}\(undef,", re.M)
_ZEROS_LINE_RE = re.compile(r"^(\s*)(\w+)\s*=\s*zeros\((Float64|Float32|Int64|Int),", re.M)
_ELEM_WRITE_RE = re.compile(r"^\s*(\w+)\[[^\n=]*\]\s*(?:=|\+=|-=|\*=|/=)(?!=)", re.M)


def _lowered_initstacks(fname: str, body: str, eltype: str) -> str:
    """The generated `initstacks_<k>_b` with its stacks allocated on the device
    (`cgen_stack_device_expr` /root/reference/src/STADE.jl:9798-9802); the size arithmetic
    is kept as written.  An array the function fills element by element (the prefix offsets
    `prefix_*` and saved loop values `val_*` of indexed stacks) is filled in a host `Vector`,
    as written, and uploaded where the function returns it: a device array cannot be written
    element by element from the host, and the lowered kernels take device memory only."""
    written = set(_ELEM_WRITE_RE.findall(body))

    def dev_type(t: str) -> str:
        return "Int64" if t in ("Int64", "Int") else eltype

    def alloc(m):
        ind, nm, t = m.group(1), m.group(2), m.group(3)
        if nm in written:
            return m.group(0)
        return f"{ind}{nm} = ROCArray{{{dev_type(t)}}}(undef,"

    def zeros_(m):
        ind, nm, t = m.group(1), m.group(2), m.group(3)
        if nm in written:
            return m.group(0)
        return f"{ind}{nm} = AMDGPU.zeros({dev_type(t)},"
    body = _ALLOC_LINE_RE.sub(alloc, body)
    body = _ZEROS_LINE_RE.sub(zeros_, body)
    if written:
        def ret(m):
            items = [x.strip() for x in m.group(2).split(",")]
            items = [f"ROCArray({x})" if x in written else x for x in items]
            return f"{m.group(1)}return ({', '.join(items)})"
        body = re.sub(r"^(\s*)return \((.*)\)\s*$", ret, body, flags=re.M)
        body = re.sub(r"^(\s*)return (\w+)\s*$",
                      lambda m: f"{m.group(1)}return ROCArray({m.group(2)})" if m.group(2) in written else m.group(0),
                      body, flags=re.M)
    body = re.sub(rf"^function\s+{re.escape(fname)}\s*\(", f"function {fname}_hip(", body, count=1, flags=re.M)
    return body.rstrip()


def _lowered_call(fname: str, sig: dict, cfun: str, eltype: str) -> str:
    """Host function for one lowered function: one ccall into the generated library."""
    types, vals, arrays = [], [], []
    for nm, kind, nd in sig["args"]:
        if kind in ("Af", "Ai"):
            types.append("Ptr{Int64}" if kind == "Ai" else f"Ptr{{{eltype}}}")
            vals.append(f"pointer({nm})")
            arrays.append(nm)
            if nd == 1:
                types.append("Int64")
                vals.append(f"length({nm})")
            else:
                for d in range(1, nd):
                    types.append("Int64")
                    vals.append(f"size({nm}, {d})")
                types.append("Int64")
                vals.append(f"prod(size({nm})[{nd}:end])")
        elif kind == "i":
            types.append("Int64")
            vals.append(f"Int64({nm})")
        elif kind == "b":
            types.append("Bool")
            vals.append(f"Bool({nm})")
        else:
            types.append(eltype)
            vals.append(f"{eltype}({nm})")
    types += ["Ptr{Float64}", "Ptr{Int64}", "Ptr{Cvoid}"]
    vals += ["__ret", "__iret", "AMDGPU.stream().stream"]
    args = [nm for nm, _, _ in sig["args"]]
    lines = [f"function {fname}_hip({', '.join(args)})",
             "    __ret = zeros(Float64, 16)",
             "    __iret = zeros(Int64, 16)"]
    lines.append(f"    GC.@preserve {' '.join(arrays + ['__ret', '__iret'])} begin")
    lines.append(f"        __rc = ccall((:{cfun}, libstade_gen), Int32,")
    lines.append(f"                     ({', '.join(types)},),")
    lines.append(f"                     {', '.join(vals)})")
    lines.append("    end")
    lines.append("    __rc == -3 && throw(BoundsError())")
    lines.append(f"    __rc >= 0 || error(\"{cfun}: \", unsafe_string(ccall((:stade_hip_gen_last_error, libstade_gen), Cstring, ())))")
    kinds = sig.get("ret") or []
    vals_ret = [f"__iret[{k + 1}]" if kd == "i" else (f"__ret[{k + 1}]" if eltype == "Float64" else f"{eltype}(__ret[{k + 1}])")
                for k, kd in enumerate(kinds)]
    if not vals_ret:
        lines.append("    return nothing")
    elif len(vals_ret) == 1:
        lines.append(f"    return {vals_ret[0]}")
    else:
        lines.append("    return (" + ", ".join(vals_ret) + ")")
    lines.append("end")
    return "\n".join(lines)


def _lowered_file(text: str, in_path, out_path, precision, inbounds: bool = True) -> str:
    from .lower import LowerError, hipgen, lower
    if precision in (None, "Float64", "f64"):
        prec = "f32" if re.search(r"\bFloat32\b", text) and precision is None else "f64"
    elif precision in ("Float32", "f32"):
        prec = "f32"
    else:
        raise StadeHipRefusal(f"precision={precision}: the lowering writes Float64 or Float32 code")
    eltype = "Float32" if prec == "f32" else "Float64"
    try:
        lib = lower(text, prec, tag=Path(in_path).stem, inbounds=inbounds)
    except LowerError as e:
        raise StadeHipRefusal(f"{Path(in_path).name}: the general lowering cannot take this file: {e}") from e
    funcs = _split_functions(text)
    out = [
        f"# Generated by stade_hip_file from {Path(in_path).name} through the general lowering: host",
        "# functions that run the lowered HIP library (MI355X, gfx950) through ccall.  Arguments,",
        "# in-place effects and return values are those of the generated functions they stand for.",
        "using AMDGPU",
        f"const libstade_gen = \"{lib.path}\"",
        "",
    ]
    for fname, (args, body) in funcs.items():
        if fname.startswith("initstacks_"):
            out.append(_lowered_initstacks(fname, body, eltype))
        elif fname in lib.sigs:
            sig = lib.sigs[fname]
            if [a for a, _, _ in sig["args"]] != args:
                raise StadeHipRefusal(f"{fname}: the lowered argument list differs from the generated one")
            out.append(_lowered_call(fname, sig, f"stade_hip_gen_{hipgen.cname(fname)}", eltype))
        else:
            continue
        out.append("")
    result = "\n".join(out)
    Path(out_path).write_text(result)
    return result


def stade_hip_file(in_path, out_path, *, precision=None, inbounds: bool = True, lib_path: str | None = None,
                   general: bool = True) -> str:
    """Write Julia host code for the generated functions of `in_path` into `out_path`.

    `precision` mirrors `stade_amdgpu_file`'s keyword: `None` keeps the kernel's element
    type; a precision the library does not implement for that kernel is refused.
    `inbounds` mirrors it too: with `inbounds=false` the host functions read the device
    error flag after the call (one synchronisation) and throw a `BoundsError` where an
    index value held in an Int64 array (the MLP labels) is out of range; with the default
    `true`, as in the reference's GPU code, nothing is checked.  A file that goes through the
    general lowering is built the same way: with `inbounds=false` every array access is checked
    and an index out of range throws `BoundsError`; with `true` accesses are unchecked, as
    under Julia's `@inbounds`.
    `general=False` refuses, instead of lowering, a file whose primal matches none of the
    library's hand-written kernels.
    Returns the written text.
    """
    text = Path(in_path).read_text()
    try:
        spec, funcs = identify(text)
    except StadeHipRefusal:
        if not general:
            raise
        return _lowered_file(text, in_path, out_path, precision, inbounds)
    if precision not in (None, spec.eltype):
        raise StadeHipRefusal(f"{spec.name}: libstade_hip implements {spec.eltype} only, precision={precision} requested")
    libp = lib_path or "libstade_hip"
    out = [
        f"# Generated by stade_hip_file from {Path(in_path).name}: host functions for {spec.name}",
        "# that run on libstade_hip.so (MI355X, gfx950) through ccall.  Arguments, in-place effects",
        "# and return values are those of the generated functions they stand for.",
        "using AMDGPU",
        f"const libstade_hip = \"{libp}\"",
        "",
    ]
    emitted = 0
    for fname, (args, _) in funcs.items():
        if fname.startswith("initstacks_"):
            if spec.stacks:
                sa = ", ".join(spec.stack_args)
                out.append(f"function {fname}_hip({sa})")
                names = []
                for nm, et, size in spec.stacks:
                    out.append(f"    {nm} = ROCArray{{{et}}}(undef, {size})")
                    names.append(nm)
                out.append("    return " + (names[0] if len(names) == 1 else "(" + ", ".join(names) + ")"))
                out.append("end")
            else:
                out.append(f"function {fname}_hip({', '.join(args)})")
                out.append("    return nothing")
                out.append("end")
            out.append("")
            emitted += 1
            continue
        for mode_key in ("hv", "b", "d"):
            if fname == f"{spec.name}_{mode_key}":
                mode = spec.modes[mode_key]
                want = [nm for nm, _ in mode.args] + [nm for nm, _, _ in spec.stacks if mode_key != "d"]
                if args != want:
                    raise StadeHipRefusal(f"{fname}: argument list {args} differs from the one libstade_hip implements {want}")
                stacks = [(nm, et) for nm, et, _ in spec.stacks] if mode_key != "d" else []
                out.append(_jl_call(spec, fname, mode, stacks, inbounds))
                out.append("")
                emitted += 1
    if emitted == 0:
        raise StadeHipRefusal(f"{in_path}: no generated _b/_d/_hv function of {spec.name} found")
    result = "\n".join(out)
    Path(out_path).write_text(result)
    return result
