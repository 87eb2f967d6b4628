"""CPU checks of the e3m2 operand format of ic_gemm_w4a8_f6: the encoder's
code table (csrc/gemm_f6.h) against the e3m2 definition, and the 6-bit
packing of the test decoder against an independent packer."""
from __future__ import annotations

import os
import re

import numpy as np

import _f6

HDR = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "comfyui-int-crush_amd", "csrc",
                   "gemm_f6.h")


def test_encoder_table_matches_e3m2_definition():
    text = open(HDR).read()
    expr = re.search(r"kE3M2Mag\s*=\s*([^;]+);", text).group(1)
    mags = {int(sh) // 6: int(v) for v, sh in re.findall(r"\((\d+)ull\s*<<\s*(\d+)\)", expr)}
    mags.setdefault(0, 0)
    assert sorted(mags) == list(range(9))
    for a, code in mags.items():
        assert code < 32 and _f6.E3M2[code] == a          # |v| = a encodes exactly
        assert _f6.E3M2[code | 32] == -a                   # the sign bit negates
    # every integer in [-8, 8] has exactly one nonnegative-zero code, and the
    # x = 16 h + l split of every int8 code stays inside that range
    x = np.arange(-128, 128)
    h = (x + 8) >> 4
    l = x - 16 * h
    assert h.min() == -8 and h.max() == 8 and l.min() == -8 and l.max() == 7


def test_unpack6_against_independent_packer():
    rng = np.random.default_rng(0)
    codes = rng.integers(0, 64, size=(5, 32))
    packed = np.zeros((5, 24), np.uint8)
    for r in range(5):
        v = 0
        for i, c in enumerate(codes[r]):
            v |= int(c) << (6 * i)
        packed[r] = np.frombuffer(v.to_bytes(24, "little"), np.uint8)
    assert np.array_equal(_f6.unpack6(packed), codes)
