"""CPU oracle for STADE-generated derivative code -- TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may
import this package, as the checker and as the reported CPU baseline.  The product
path (`stade.jl_amd/stade_hip`, `libstade_hip.so`, the Julia host text written by
`stade_hip_file`) never imports, links or runs anything here.

Contents
--------
jl2c     Julia-subset -> C transpiler: executes the reference's generated text
         (`/root/reference/test/val-corpus/*_{b,d,hv}.jl` and the config kernel texts
         in `stade.jl_amd/corpus/`) with Julia semantics.
runner   gcc build + ctypes calls on numpy arrays.
checks   the reference's own numerical oracles restated: dot-product identity
         (`val_validate_dotprod` /root/reference/src/STADE.jl:17108-17131), central
         finite differences (`val_finite_diff_check` 16334-16351, JVP 16376), HVP as a
         finite difference of the gradient (`val_validate_hvp` 17133-17153).
rng      Julia's `Random.Xoshiro(seed)` scalar stream, `val_stable_seed` (FNV-1a) and
         `val_normal` (Box-Muller, cosine branch), /root/reference/src/STADE.jl:16619-16637,
         pinned against /root/reference/test/validate_seed_stable.jl:37-56.

Parity status per function is stated in each module's header.
"""
