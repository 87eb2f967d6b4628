"""Decoders of the e3m2 operand formats of ic_gemm_w4a8_f6 (test
infrastructure), written from the format definition:

* e3m2: sign bit 5, exponent bits 4..2 with bias 3, mantissa bits 1..0;
  value = (-1)^s 2^(e-3) (1 + m/4) for e > 0, (-1)^s 2^-2 (m/4) for e = 0.
* 32 codes pack into 24 bytes, code i at bits 6i .. 6i+5 (little-endian).
* A6: per 16-row block and 128-K stage, 3072 bytes: three parts u of 16 rows
  x 64 bytes; row r of part u holds bytes 16u .. 16u+15 of the row's four
  48-byte records; record c = 24 bytes of h codes then 24 bytes of l codes
  of the K values 128 s + 32 c .. +31.
* W6: per 16-column block and stage, 1536 bytes: heads (16 x 64 bytes,
  bytes 0..15 of chunks 0..3) then tails (16 x 32 bytes, bytes 16..23).
"""
from __future__ import annotations

import numpy as np


def e3m2_value(code: int) -> float:
    s = -1.0 if code & 32 else 1.0
    e, m = (code >> 2) & 7, code & 3
    return s * (2.0 ** (e - 3) * (1 + m / 4) if e else 2.0 ** -2 * (m / 4))


E3M2 = np.array([e3m2_value(c) for c in range(64)])


def unpack6(b: np.ndarray) -> np.ndarray:
    """[..., 24] uint8 -> [..., 32] codes (code i at bits 6i of the little-endian run)."""
    bits = np.unpackbits(b.astype(np.uint8), axis=-1, bitorder="little")  # [..., 192]
    bits = bits.reshape(*b.shape[:-1], 32, 6)
    return (bits * (1 << np.arange(6))).sum(-1)


def decode_a6(buf: np.ndarray, M: int, K: int):
    """-> (h, l) float arrays [M, K] of the values the codes encode."""
    S = K // 128
    rb = (M + 15) // 16
    x = buf[: rb * S * 3072].reshape(rb, S, 3, 16, 4, 16)     # block, stage, part, row, record, byte
    rec = x.transpose(0, 3, 1, 4, 2, 5).reshape(rb * 16, S, 4, 48)[:M]  # row, stage, record, 48 bytes
    h = E3M2[unpack6(rec[..., :24])].reshape(M, K)
    l = E3M2[unpack6(rec[..., 24:])].reshape(M, K)
    return h, l


def decode_w6(buf: np.ndarray, N: int, K: int) -> np.ndarray:
    """-> float array [N, K] of the weight values."""
    S = K // 128
    cb = (N + 15) // 16
    x = buf[: cb * S * 1536].reshape(cb, S, 1536)
    heads = x[:, :, :1024].reshape(cb, S, 16, 4, 16)
    tails = x[:, :, 1024:].reshape(cb, S, 16, 4, 8)
    chunk = np.concatenate([heads, tails], axis=-1)            # block, stage, col, chunk, 24
    chunk = chunk.transpose(0, 2, 1, 3, 4).reshape(cb * 16, S, 4, 24)[:N]
    return E3M2[unpack6(chunk)].reshape(N, K)
