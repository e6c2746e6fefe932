"""General lowering of STADE-generated derivative code to HIP for MI355X (gfx950).

`stade_hip.lower.lower(path_or_text, precision)` reads any generated `.jl` (adjoint, tangent
or HVP text in the subset STADE's generators write), plans each function's loops for the GPU
(`analysis`), writes HIP (`hipgen`), builds it once with hipcc and returns a library whose
`call(name, *args)` runs the function on torch tensors in place (`runtime`).  It stands for
the reference's `cgen_body` / `cgen_device_assign` / `cgen_emit` pipeline
(/root/reference/src/STADE.jl:10409-12111), redesigned around one MI355X; the five benchmark
kernels keep their hand-written entry points in libstade_hip.so.
"""
from .runtime import LoweredLib, build_source, initstacks, initstacks_returns, lower, run_initstacks  # noqa: F401
from .syntax import LowerError  # noqa: F401
