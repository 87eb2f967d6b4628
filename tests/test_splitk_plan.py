"""The split-K plan the library reports (ic_gemm_splitk_bytes) for the small-M
shapes of the Flux text stream and the split-K tests, on a 256-CU device
(MI355X; the count the library assumes without a GPU).  Grouped launches pay
for the kernel that adds the slices, so the 512 x 3072 x 3072 grouped W4A8 runs
unsplit (its outputs are then the single fold chain's); the long-K grouped
shapes and the per-row ones keep splitting.  CPU only: the plan is host logic."""
from __future__ import annotations

import pytest


@pytest.mark.parametrize("M,N,K,G,int4,split", [
    (512, 3072, 3072, 24, 1, False),    # Flux text-stream proj, grouped: unsplit
    (512, 3072, 12288, 96, 1, True),    # Flux text-stream MLP-down, grouped
    (256, 3072, 3072, 24, 1, True),     # grouped, fewer tiles
    (64, 3072, 12288, 96, 1, True),     # the split-K tests' shapes
    (100, 1000, 3072, 24, 1, True),
    (512, 3072, 3072, 1, 0, True),      # W8A8 at the text-stream proj shape
    (512, 3072, 3072, 1, 1, True),      # per-row INT4
    (512, 9216, 3072, 24, 1, False),    # enough tiles: no split
    (4608, 3072, 12288, 96, 1, False),  # C3
    (16, 3072, 3072, 24, 1, False),     # the GEMV's rows
])
def test_splitk_plan(rt, M, N, K, G, int4, split):
    nb = rt.lib().ic_gemm_splitk_bytes(M, N, K, G, int4)
    assert (nb > 0) == split, nb
    if split:
        assert nb % (4 * M * N) == 0 and 2 <= nb // (4 * M * N) <= 16
