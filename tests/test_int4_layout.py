"""The K-interleaved INT4 order: the numpy restatement the GPU tests check
the repack kernel against, pinned here by the definition read nibble by
nibble, against the oracle's unpack of the checkpoint order."""
from __future__ import annotations

import numpy as np
import pytest

from _w4 import deinterleave_k, interleave_k


def _value(nib: int) -> int:
    return nib - 16 if nib >= 8 else nib


@pytest.mark.parametrize("N,K", [(1, 8), (3, 64), (5, 136)])
def test_interleave_matches_the_definition(oracle, N, K):
    rng = np.random.default_rng(N * 1000 + K)
    packed = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
    q = oracle.unpack_int4(packed, K)  # [N, K] int8, checkpoint order
    kil = interleave_k(packed)
    assert kil.shape == packed.shape and kil.dtype == np.uint8
    for n in range(N):
        for k in range(K):
            d, r = divmod(k, 8)
            byte = int(kil[n, 4 * d + (r % 4)])
            nib = byte & 15 if r < 4 else byte >> 4
            assert _value(nib) == q[n, k], (n, k)


def test_interleave_round_trip_and_is_not_identity():
    rng = np.random.default_rng(7)
    packed = rng.integers(0, 256, size=(64, 512), dtype=np.uint8)
    kil = interleave_k(packed)
    assert np.array_equal(deinterleave_k(kil), packed)
    assert not np.array_equal(kil, packed)
    # a word whose eight weights are k = 0..7 (nibbles 0..7): bytes 0x40 0x51 0x62 0x73
    word = np.array([[0x10, 0x32, 0x54, 0x76]], dtype=np.uint8)
    assert interleave_k(word).tolist() == [[0x40, 0x51, 0x62, 0x73]]
