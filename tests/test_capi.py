"""The C ABI: the library loads without a GPU, exports every symbol the header declares, and
rejects bad arguments with an error code and a message before any device work."""
import ctypes
import re
import subprocess

import pytest

from helpers import ROOT

HEADER = ROOT / "include" / "stade_hip.h"


def declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(stade_hip_\w+)\s*\(", text)))


def test_header_symbols_exported():
    import stade_hip
    path = stade_hip.lib_path()
    out = subprocess.run(["nm", "-D", "--defined-only", str(path)], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (stade_hip_\w+)", out))
    missing = [s for s in declared() if s not in exported]
    assert not missing, missing
    assert len(declared()) >= 15


def test_python_entry_table_matches_header():
    import stade_hip
    for nm in stade_hip.ENTRY_POINTS:
        assert nm in declared(), nm


def _lib():
    import stade_hip
    return stade_hip.lib()


def test_argument_errors_before_device_work():
    L = _lib()
    null = ctypes.c_void_p(0)
    rc = L.stade_hip_diffusion2d_b(null, null, null, null, null, null, -1, null)
    assert rc == -1 and b"negative" in L.stade_hip_last_error()
    rc = L.stade_hip_diffusion2d_d(null, null, null, null, null, null, 50000, null)
    assert rc == -3 and b"46340" in L.stade_hip_last_error()
    rc = L.stade_hip_affine_lsq_b(*([null] * 12), -2, 3, null)
    assert rc == -1 and b"negative" in L.stade_hip_last_error()
    # 65536 row tiles of 64 would exceed the grid's y dimension
    rc = L.stade_hip_affine_lsq_b(*([null] * 12), ctypes.c_int64(65536 * 64), ctypes.c_int64(1), null)
    assert rc == -3 and b"65535 row tiles" in L.stade_hip_last_error()
    rc = L.stade_hip_affine_lsq_b(*([null] * 12), ctypes.c_int64(1), ctypes.c_int64(65536 * 64), null)
    assert rc == -3 and b"65535 column tiles" in L.stade_hip_last_error()
    # the HVP's column kernel takes 32-column tiles: refused past 65535 of them, before any
    # device work (the pointers are never read)
    fake = ctypes.c_void_p(256)
    rc = L.stade_hip_affine_lsq_hv(*([fake] * 12), ctypes.c_int64(1), ctypes.c_int64(65535 * 32 + 1), *([fake] * 12), null)
    assert rc == -3 and b"65535 column tiles of 32" in L.stade_hip_last_error()
    # zero-trip: n = 0 runs no loop and needs no device
    assert L.stade_hip_diffusion2d_b(null, null, null, null, null, null, 0, null) == 0
    assert L.stade_hip_affine_lsq_d(*([null] * 12), 0, 5, null) == 0


def test_product_path_refuses_cpu_tensors():
    import numpy as np
    import torch
    import stade_hip
    t = torch.zeros(4, dtype=torch.float64)
    with pytest.raises(ValueError, match="not on a GPU"):
        stade_hip.diffusion2d_b(t[:1], t[:1], t, t, t, t, 2)
    with pytest.raises(TypeError, match="Int64"):
        stade_hip.diffusion2d_b(t[:1], t[:1], t, t, t, t, 2.0)


def test_noalloc_refuses_grids_beyond_its_scratch():
    """n = 46336 (a multiple of 128, 16-byte aligned arrays) needs 362 x 724 = 262088
    partial sums, above the static scratch's 131072: refused before any device work (the
    pointers are never dereferenced)."""
    L = _lib()
    f = L.stade_hip_diffusion2d_b_noalloc
    f.restype = ctypes.c_int32
    f.argtypes = [ctypes.c_void_p] * 6 + [ctypes.c_int64, ctypes.c_void_p]
    fake = ctypes.c_void_p(1 << 20)   # 16-byte aligned, never dereferenced
    rc = f(fake, fake, fake, fake, fake, fake, 46336, None)
    assert rc == -3 and b"262088 partial sums" in L.stade_hip_last_error()
    assert f(None, None, None, None, None, None, 0, None) == 0
