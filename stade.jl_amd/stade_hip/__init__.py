"""Python host mirror of the generated STADE functions, executed by libstade_hip.so.

Each function here has the name, argument order and argument meaning of the generated
Julia function it stands for (`<k>_b`, `<k>_d`, `<k>_hv` of stade.jl_amd/corpus/<k>.jl;
`agen_signature_args` /root/reference/src/STADE.jl:3455-3464, `tgen_signature_args`
3306-3315, `hvp_emit` 6750-6756) and calls the matching `stade_hip_*` C entry point:

* arrays are torch tensors on a ROCm device, flat and contiguous, holding the Julia
  array's column-major data; they are mutated in place as the generated code mutates
  them (outputs overwritten, shadows accumulated, resets applied, stacks written);
* Int64 arguments are Python ints; float scalar arguments are Python floats, and their
  shadows are returned the way the generated function returns them (the adjoint returns
  the scalar shadows, bare if one, a tuple otherwise; the HVP returns (xb, xbd) pairs);
* work is enqueued on torch's current stream of the tensors' device.

This is the product path: there is no CPU fallback.  If the library is missing, or a
tensor is not on a GPU, the call raises.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

from .api import (  # noqa: F401
    StadeHipError, StadeHipBoundsError, lib, lib_path, ENTRY_POINTS, device_error, workspace_info,
    affine_lsq_b, affine_lsq_d, affine_lsq_hv,
    diffusion2d_b, diffusion2d_d, diffusion2d_hv,
    burgers1d_b, burgers1d_d, burgers1d_hv, initstacks_burgers1d_b, burgers1d_stack_lengths,
    burgers1d_b_ckpt, burgers1d_hv_ckpt, burgers1d_ckpt_lengths,
    mlp2_ce_b, mlp2_ce_d, mlp2_ce_hv,
    conv3x3_b, conv3x3_d, conv3x3_hv,
    rng_normal, rng_uniform, rng_int_range, stable_seed,
)
from .emit import stade_hip_file  # noqa: F401
