"""affine_lsq on the GPU against the oracle (the transpiled generated code), fp64 to 1e-12."""
import pytest

from helpers import run_parity

pytestmark = pytest.mark.gpu

# column tiles of 64 are grouped into at most 16 row-sum chunks: one tile a chunk up to n = 1024,
# then 2 (2048; 1088: 17 tiles in 9 chunks, the last a single tile), 3 (3000: 47 tiles, the
# last chunk short), 5 (5000: 79 tiles, a ragged last tile), 8 (4096^2: 64 tiles in 8 full
# chunks) and 9 tiles a chunk (8200: 129 tiles, the last chunk one tile short of 9).
SIZES = [(1, 1), (3, 5), (64, 64), (65, 130), (200, 77), (1, 300), (300, 1), (1024, 1024), (4, 0), (0, 3),
         (5000, 3), (5000, 0), (2048, 2048), (1000, 3000), (100, 1088), (70, 5000), (70, 8200), (4096, 4096),
         (3000, 5000)]


@pytest.mark.parametrize("mode", ["b", "d", "hv"])
@pytest.mark.parametrize("mn", SIZES)
def test_affine_lsq_parity(mode, mn):
    m, n = mn
    shapes = {}
    for k in ("w", "wb", "wd", "wbd"):
        shapes[k] = (m, n)
    for k in ("x", "xb", "xd", "xbd"):
        shapes[k] = n
    for k in ("b", "bb", "bd", "bbd", "t", "tb", "td", "tbd", "r", "rb", "rd", "rbd"):
        shapes[k] = m
    for k in ("loss", "lossb", "lossd", "lossbd"):
        shapes[k] = 1
    print(f"affine_lsq_{mode} m={m} n={n}", flush=True)
    run_parity("affine_lsq", mode, shapes, dict(i_m=m, i_n=n))

