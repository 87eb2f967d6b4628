"""The K-interleaved nibble order of packed INT4 rows (ic_int4_interleave_k),
restated with numpy for the tests: byte 4d + j of a row holds weight
k = 8d + j in its low nibble and k = 8d + 4 + j in its high nibble; the
checkpoint order holds k = 2b low and 2b + 1 high in byte b."""
from __future__ import annotations

import numpy as np


def _nibbles(packed: np.ndarray) -> np.ndarray:
    """uint8 [N, K/2] -> nibble values [N, K] in byte order (low first)."""
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    out = np.empty((p.shape[0], 2 * p.shape[1]), dtype=np.uint8)
    out[:, 0::2] = p & 15
    out[:, 1::2] = p >> 4
    return out


def _pack(nib: np.ndarray) -> np.ndarray:
    return (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)


def interleave_k(packed: np.ndarray) -> np.ndarray:
    """Checkpoint order -> K-interleaved order (K a multiple of 8)."""
    nib = _nibbles(packed)  # nibble i of a row is weight k = i
    N, K = nib.shape
    assert K % 8 == 0
    w = nib.reshape(N, K // 8, 2, 4)  # [word, half (k < 4 or not), j]
    out = np.empty((N, K // 8, 4, 2), dtype=np.uint8)  # [word, byte j, low/high]
    out[..., 0] = w[:, :, 0, :]
    out[..., 1] = w[:, :, 1, :]
    return _pack(out.reshape(N, K))


def deinterleave_k(kil: np.ndarray) -> np.ndarray:
    """K-interleaved order -> checkpoint order."""
    nib = _nibbles(kil)
    N, K = nib.shape
    v = nib.reshape(N, K // 8, 4, 2)  # [word, byte j, low/high]
    out = np.empty((N, K // 8, 2, 4), dtype=np.uint8)
    out[:, :, 0, :] = v[..., 0]
    out[:, :, 1, :] = v[..., 1]
    return _pack(out.reshape(N, K))
