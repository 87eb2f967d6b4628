"""CPU checks of the numeric shortcuts the gfx950 kernels rely on.

These emulate the kernel formulas with numpy's IEEE f32/f64 arithmetic (which
is what the GPU executes, RN-even, no contraction) and compare them with exact
rational rounding.  INTCRUSH_EXHAUSTIVE=1 widens the samples to every pair.
"""
from __future__ import annotations

import os
import shutil
import subprocess
from fractions import Fraction

import numpy as np
import pytest

EXHAUSTIVE = os.environ.get("INTCRUSH_EXHAUSTIVE") == "1"


def _all_finite(dt):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    if dt == "f16":
        v = bits.view(np.float16).astype(np.float32)
    else:
        v = (bits.astype(np.uint32) << 16).view(np.float32)
    return v[np.isfinite(v)]


def _round_dt(v64, dt, oracle):
    return oracle.round_dtype(v64, 0 if dt == "f16" else 1)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_smoothrot_divide_fast_path(oracle, dt):
    """div_round_dt: RN_dt(RN32(x * RN32(1/f))) with an IEEE-divide slow path
    below the normal range equals the exactly rounded quotient RN_dt(x/f)."""
    xs = _all_finite(dt)
    fs = xs[xs != 0]
    rng = np.random.default_rng(0)
    if not EXHAUSTIVE:
        extra = _round_dt(np.array([3.0, 7.0, 0.1, 1e-3]), dt, oracle).astype(np.float32)
        fs = np.concatenate([rng.choice(fs, 48, replace=False), fs[np.abs(fs) < 1e-4][:8], extra])
        xs = np.concatenate([rng.choice(xs, 4096, replace=False), xs[np.abs(xs) < 1e-4][:512]])
    tiny = np.float32(2.0 ** -14 if dt == "f16" else 2.0 ** -126)
    for f in fs:
        rcp = np.float32(1.0) / np.float32(f)
        with np.errstate(all="ignore"):
            p = xs * rcp
            slow = ~((np.abs(p) >= tiny) & np.isfinite(p)) & (p != 0)
            got = _round_dt(p.astype(np.float64), dt, oracle)
            got[slow] = _round_dt((xs[slow] / np.float32(f)).astype(np.float64), dt, oracle)
        # RN_dt(RN64(x/f)) is the exact rounding for quotients of <= 11-bit values
        want = _round_dt(xs.astype(np.float64) / np.float64(f), dt, oracle)
        ok = (got == want) | (np.isnan(got) & np.isnan(want))
        assert ok.all(), (f, xs[~ok][:4])
        # the fast path as compiled for fp16: one rounding of the exact
        # product (v_fma_mix), taken when |RN_dt(x * rcp)| > min normal
        with np.errstate(all="ignore"):
            h = _round_dt(xs.astype(np.float64) * np.float64(rcp), dt, oracle)
        fast = (np.abs(h) > tiny) & np.isfinite(h)
        assert np.array_equal(h[fast], want[fast]), (f, xs[fast][h[fast] != want[fast]][:4])


def test_double_rounding_of_quotients_is_exact(oracle):
    """RN16(RN64(x/f)) == RN16(x/f) on tie-prone subnormal quotients (rationals)."""
    xs = np.array([2.0 ** -24 * k for k in (1, 3, 5, 91, 1023)] + [1.0, 3.0, 65504.0], np.float64)
    fs = np.array([2.0, 14.0, 3.0, 6.0, 0.5, 7.0], np.float64)
    for x in xs:
        for f in fs:
            want = oracle._round_fraction(Fraction(x) / Fraction(f), 0)
            assert oracle.round_dtype(np.array([x / f]), 0)[0] == want


def _rto24(y):
    b = np.asarray(y, np.float64).view(np.uint64)
    lo = b & np.uint64(0xFFFFFFFF)
    sticky = (lo & np.uint64(0x1FFFFFFF)) != 0
    b = (b & ~np.uint64(0x1FFFFFFF)) | (sticky.astype(np.uint64) << np.uint64(29))
    return b.view(np.float64).astype(np.float32)


@pytest.mark.parametrize("dt", [0, 1])
def test_round_to_odd_then_rn16(oracle, dt):
    """round_f64_to_dt: RN_dt(rto24(y)) == RN_dt(y), including values a hair
    away from 16-bit midpoints where RN32 would double-round."""
    rng = np.random.default_rng(1)
    base = rng.standard_normal(20000) * np.exp2(rng.integers(-20, 12, 20000))
    mids = oracle.round_dtype(base, dt).astype(np.float64)
    ulp = np.abs(mids) * (2.0 ** (-11 if dt == 0 else -8))
    near = np.concatenate([mids + ulp / 2 + ulp * 2.0 ** -30, mids + ulp / 2 - ulp * 2.0 ** -30,
                           mids + ulp / 2, base])
    got = oracle.round_dtype(_rto24(near).astype(np.float64), dt)
    want = oracle.round_dtype(near, dt)
    assert np.array_equal(got, want)
    # plain RN32 first would be wrong on some of these
    bad = oracle.round_dtype(near.astype(np.float32).astype(np.float64), dt)
    assert not np.array_equal(bad, want)


def test_quant_divide_via_fp64_reciprocal():
    """quant_code: RN32(v * RN64(1/s)) == RN32(v/s) for 16-bit-exact v, normal s."""
    rng = np.random.default_rng(2)
    v = rng.standard_normal(200000).astype(np.float16).astype(np.float32)
    s = (np.abs(rng.standard_normal(200000)) * np.exp2(rng.integers(-30, 10, 200000))).astype(np.float32)
    s = np.maximum(s, np.float32(1e-8) / np.float32(127.0))
    got = (v.astype(np.float64) * (1.0 / s.astype(np.float64))).astype(np.float32)
    want = v / s
    assert np.array_equal(got, want)


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
@pytest.mark.parametrize("dt", [0, 1])
def test_quant_markstein_exhaustive(tmp_path, dt):
    """quant_code_mk: q0 = RN32(v r), e = fma(-q0, s, v), q = fma(e, r, q0),
    code = trunc(RN32(q +- 0.5)), r = RN32(1/s), equals the reference code for
    every (v, m) of the 16-bit type with |v| <= m (both signs), while the
    single-rounding shortcut does not (so the checker detects a wrong formula)."""
    src = os.path.join(os.path.dirname(os.path.abspath(__file__)), "numerics_quant_check.c")
    exe = str(tmp_path / "qcheck")
    subprocess.check_call(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", src, "-o", exe, "-lm"])
    out = subprocess.run([exe, str(dt)], capture_output=True, text=True, timeout=300, check=True).stdout.split()
    fields = dict(zip(out[0::2], (int(v) for v in out[1::2])))
    assert fields["pairs"] > 10**9
    assert fields["mismatches"] == 0
    assert fields["shortcut_mismatches"] > 0
