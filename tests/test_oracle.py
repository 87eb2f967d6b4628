"""Pins the CPU oracle against the reference's own known answers and against
closed forms / exact arithmetic (no GPU).

Each check is chosen so that a plausible slip in the oracle (wrong sign in H4,
transposed digit order, wrong rounding rule, dropped pad, wrong group index)
fails it.
"""
from __future__ import annotations

import math
from fractions import Fraction

import numpy as np
import pytest
import torch


# ---------------------------------------------------------------- INT4 pack / unpack
# Known answers of the reference tests/test_quant_utils.py:65-99 and test_w4a8_gemm.py:49-57.
def test_pack_unpack_known_answers(oracle):
    v = np.array([-8, -1, 0, 1, 7, -3, 5, 0], np.int8)
    packed = oracle.pack_int4(v)
    # low nibble = even index, two's complement: -8 -> 0x8, -1 -> 0xF, 0, 1, 7, -3 -> 0xD, 5, 0
    assert packed.tolist() == [0xF8, 0x10, 0xD7, 0x05]
    assert oracle.unpack_int4(packed[None], 8)[0].tolist() == v.tolist()
    odd = np.array([-8, 0, 7], np.int8)
    assert oracle.unpack_int4(oracle.pack_int4(odd)[None], 3)[0].tolist() == odd.tolist()
    for fill in (-8, 7):
        vals = np.full((2, 16), fill, np.int8)
        assert np.array_equal(oracle.unpack_int4(oracle.pack_int4(vals), 16), vals)
    assert oracle.pack_int4(np.zeros((4, 33), np.int8)).shape == (4, 17)
    with pytest.raises(ValueError):
        oracle.pack_int4(np.array([8], np.int8))


def test_unpack_brute_force_all_bytes(oracle):
    packed = np.arange(256, dtype=np.uint8)[None]
    out = oracle.unpack_int4(packed, 512)[0]
    for b in range(256):
        lo, hi = b & 15, b >> 4
        assert out[2 * b] == (lo - 16 if lo >= 8 else lo)
        assert out[2 * b + 1] == (hi - 16 if hi >= 8 else hi)


def test_pack_unpack_roundtrip(oracle):
    rng = np.random.default_rng(0)
    v = rng.integers(-8, 8, size=(7, 130)).astype(np.int8)
    assert np.array_equal(oracle.unpack_int4(oracle.pack_int4(v), 130), v)


# ---------------------------------------------------------------- Hadamard
def _kron_h(R):
    """_quant_utils.py:81-93 construction, independently: kron of H4/2."""
    h4 = np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], np.float64) / 2
    H = h4
    while H.shape[0] < R:
        H = np.kron(H, h4)
    return H


@pytest.mark.parametrize("R", [4, 16, 64, 256])
def test_hadamard_properties(R):
    H = _kron_h(R)
    assert np.allclose(np.abs(H), 1 / math.sqrt(R))
    assert np.array_equal(H @ H.T, np.eye(R))  # exact: entries are powers of two
    assert np.array_equal(H, H.T)
    assert np.array_equal(H @ H, np.eye(R))    # symmetric + orthogonal -> involution


@pytest.mark.parametrize("R", [16, 64, 256])
@pytest.mark.parametrize("dtype", [0, 1])
def test_prepare_rotation_matches_kron_matmul(oracle, R, dtype):
    torch_dt = torch.float16 if dtype == 0 else torch.bfloat16
    x = torch.randn(5, 3 * R, generator=torch.Generator().manual_seed(R)).to(torch_dt)
    xv = x.float().numpy().astype(np.float64)
    H = _kron_h(R)
    # x @ H^T per block in float64 is exact for 16-bit inputs; then one rounding
    ref = (xv.reshape(5, 3, R) @ H.T).reshape(5, 3 * R)
    ref = oracle.round_dtype(ref, dtype)
    for fast in (False, True):
        got = oracle.prepare(x, dtype, rot_size=R, fast=fast)
        assert np.array_equal(got, ref)


def test_prepare_rotation_pad_and_perm(oracle):
    R, K_in, K_w = 64, 100, 192  # rotation pad 100 -> 128, then w_in pad to 192
    x = torch.randn(3, K_in, generator=torch.Generator().manual_seed(1)).to(torch.float16)
    perm = torch.randperm(K_w, generator=torch.Generator().manual_seed(2))
    xp = np.zeros((3, 128))
    xp[:, :K_in] = x.float().numpy()
    H = _kron_h(R)
    rot = oracle.round_dtype((xp.reshape(3, 2, R) @ H.T).reshape(3, 128), 0)
    full = np.zeros((3, K_w), np.float32)
    full[:, :128] = rot
    got = oracle.prepare(x, 0, rot_size=R, w_in=K_w, perm=perm)
    assert np.array_equal(got, full[:, perm.numpy()])


def test_prepare_inverse_perm_roundtrip(oracle):
    K = 256
    x = torch.randn(2, K, generator=torch.Generator().manual_seed(3)).to(torch.float16)
    perm = torch.randperm(K, generator=torch.Generator().manual_seed(4))
    inv = torch.argsort(perm)
    y = oracle.prepare(x, 0, perm=perm)
    assert np.array_equal(y[:, inv.numpy()], x.float().numpy())


def test_prepare_smoothrot_divide_exact(oracle):
    """x / RN16(f) rounded once (torch half division), checked with rationals."""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 64, generator=g).to(torch.float16)
    x[0, :8] = torch.tensor([6e-8, -6e-8, 1e-5, 65504, -65504, 0.0, 3.0, 1.0], dtype=torch.float16)
    f = torch.exp(torch.randn(64, generator=g)) * 3
    f[:8] = torch.tensor([3.0, 7.0, 11.0, 0.5, 2.0, 5.0, 1e-3, 1e4])
    got = oracle.prepare(x, 0, smoothrot=f)
    fd = f.to(torch.float16).double().numpy()
    for i in range(2):
        for j in range(64):
            q = Fraction(float(x[i, j])) / Fraction(float(fd[j]))
            assert got[i, j] == oracle._round_fraction(q, 0), (i, j)


def _exact_rot(vals, R):
    """Exact rationals of H x for one block (no rounding)."""
    H = _kron_h(R)
    xv = [Fraction(float(v)) for v in vals]
    return [sum((Fraction(H[i, j]) * xv[j] for j in range(R)), Fraction(0)) for i in range(R)]


def _flush_rational(vals, R):
    """The bf16 flush restated independently: zero every input below
    2^(floor(log2 max|x|) - (43 - 2k)), R = 4^k."""
    k = {16: 2, 64: 3, 256: 4, 1024: 5, 4096: 6}[R]
    mx = max(abs(Fraction(float(v))) for v in vals)
    e = mx.numerator.bit_length() - mx.denominator.bit_length()
    if Fraction(2) ** e > mx:
        e -= 1
    thr = Fraction(2) ** (e - (43 - 2 * k))
    return [v if abs(Fraction(float(v))) >= thr else 0.0 for v in vals]


def test_bf16_wide_block_flush_then_exact(oracle):
    """A bf16 block spanning 2^-100..2^10: inputs below 2^(10 - 39) are
    flushed (R = 16, k = 2) and the rest rotated exactly; equal to the exact
    rational Hadamard of the kept inputs, rounded once."""
    R = 16
    vals = torch.tensor([[2.0 ** 10, 2.0 ** -100, -3.0, 2.0 ** -90] + [1.0] * 11 + [2.0 ** -29]],
                        dtype=torch.bfloat16)
    got = oracle.prepare(vals, 1, rot_size=R)
    kept = _flush_rational(vals[0].float().tolist(), R)
    assert kept[1] == 0.0 and kept[3] == 0.0 and kept[2] == -3.0 and kept[15] == 2.0 ** -29
    for i, q in enumerate(_exact_rot(kept, R)):
        assert got[0, i] == oracle._round_fraction(q, 1)


def test_bf16_midpoint_plus_tiny_term(oracle):
    """(1 + 2^-8) / 4 is a bf16 rounding midpoint.  A tiny term inside the
    exact span breaks the tie upwards exactly; one beyond the span is flushed
    and the tie goes to even (0.25), as the reference's fp32-accumulating
    matmul would also lose it."""
    R = 16
    for tiny, up in ((2.0 ** -30, True), (2.0 ** -100, False)):
        vals = torch.tensor([[1.0, 2.0 ** -8, tiny] + [0.0] * 13], dtype=torch.bfloat16)
        got = oracle.prepare(vals, 1, rot_size=R)
        assert got[0, 0] == (0.25 + 2.0 ** -9 if up else 0.25), tiny


@pytest.mark.parametrize("R", [16, 64, 256, 1024])
def test_bf16_flush_only_moves_ties_and_near_ties(oracle, R):
    """Random wide-span bf16 blocks (GELU-like tails down to 1e-37): the
    flushed result equals the kept inputs' exact rotation (rounded once), is
    within one bf16 ulp of the exact unflushed rotation, and differs from it
    only where a rounding boundary lies between the two exact values."""
    g = torch.Generator().manual_seed(R)
    x = torch.randn(2, R, generator=g) * 3
    tiny = torch.rand(2, R, generator=g) < 0.1
    x[tiny] = torch.randn(int(tiny.sum()), generator=g) * torch.pow(10.0, -torch.randint(10, 37, (int(tiny.sum()),), generator=g).float())
    xb = x.to(torch.bfloat16)
    got = oracle.prepare(xb, 1, rot_size=R)
    for m in range(2):
        full = _exact_rot(xb[m].float().tolist(), R)
        kept = _exact_rot(_flush_rational(xb[m].float().tolist(), R), R)
        for i in range(R):
            z = got[m, i]
            assert z == oracle._round_fraction(kept[i], 1)
            zf = oracle._round_fraction(full[i], 1)
            if z != zf:
                lo, hi = sorted((kept[i], full[i]))
                assert abs(z - zf) <= 2.0 ** (np.floor(np.log2(max(abs(z), abs(zf)))) - 7)
                # a midpoint between the two candidates lies in [lo, hi]
                mid = Fraction(float(z) + float(zf)) / 2
                assert lo <= mid <= hi


def test_bf16_flushed_blocks_are_exact_in_double(oracle):
    """After the flush, the C oracle's double butterflies never report an
    inexact block on bf16 rows, whatever the input range."""
    import ctypes

    L = oracle.lib()
    g = torch.Generator().manual_seed(9)
    for R in (16, 64, 256, 1024, 4096):
        x = torch.randn(3, 4096, generator=g) * torch.pow(2.0, torch.randint(-120, 100, (3, 4096), generator=g).float())
        xv = np.ascontiguousarray(x.to(torch.bfloat16).float().numpy())
        out = np.zeros((3, 4096), np.float32)
        n = ctypes.c_int64(-1)
        rc = L.oc_prepare(oracle._p(xv), 1, 3, 4096, None, R, 4096, None, None, oracle._p(out), ctypes.byref(n), 1)
        assert rc == 0 and n.value == 0, (R, n.value)


# ---------------------------------------------------------------- quantization
@pytest.mark.parametrize("M,K", [(1, 64), (4, 256), (16, 1024), (256, 4096)])
def test_quantize_reference_cpu_vectors(oracle, M, K):
    """tests/test_w8a8_fused_kernels.py:479-492 of the reference: seed 0 inputs,
    torch.round reference.  The GPU rule (round half away from zero) agrees
    everywhere except where the f32 quotient is exactly k + 1/2, and there it
    is one code further from zero."""
    torch.manual_seed(0)
    x = torch.randn(M, K)
    ref_s = x.float().abs().amax(dim=1).clamp(min=1e-8) / 127.0
    quot = x.float() / ref_s.unsqueeze(1)
    ref_q = quot.round().clamp(-128, 127).to(torch.int8)
    q_rne, s_rne = oracle.quantize(x.numpy(), rule="rne")
    q_gpu, s_gpu = oracle.quantize(x.numpy(), rule="gpu")
    assert np.array_equal(q_rne, ref_q.numpy())
    assert np.array_equal(s_rne, ref_s.numpy())
    assert np.array_equal(s_gpu, ref_s.numpy())
    diff = q_gpu.astype(int) - ref_q.numpy().astype(int)
    qn = quot.numpy()
    ties = (np.abs(qn) - np.floor(np.abs(qn))) == 0.5
    assert np.array_equal(diff != 0, ties & (np.floor(np.abs(qn)) % 2 == 0))
    assert np.array_equal(np.sign(diff[diff != 0]), np.sign(qn[diff != 0]).astype(int))


def test_quantize_rounding_rules_on_ties(oracle):
    x = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -2.5, 0.49999997, 0.0]], np.float32)
    q_gpu, s = oracle.quantize(x, rule="gpu")
    q_rne, _ = oracle.quantize(x, rule="rne")
    assert s[0] == np.float32(1.0)
    assert q_gpu[0].tolist() == [127, 1, 2, 3, -1, -3, 1, 0]  # half away from zero (+ f32 quirk)
    assert q_rne[0].tolist() == [127, 0, 2, 2, 0, -2, 0, 0]   # half to even


def test_quantize_zero_row_and_floor(oracle):
    q, s = oracle.quantize(np.zeros((1, 8), np.float32))
    assert s[0] == np.float32(np.float32(1e-8) / np.float32(127.0))
    assert not q.any()


# ---------------------------------------------------------------- GEMM pieces
def test_gemm_acc_exact_and_groups(oracle):
    rng = np.random.default_rng(1)
    a = rng.integers(-128, 128, (9, 384)).astype(np.int8)
    w = rng.integers(-8, 8, (11, 384)).astype(np.int8)
    full = a.astype(np.int64) @ w.astype(np.int64).T
    assert np.array_equal(oracle.gemm_acc(a, w), full)
    g = oracle.gemm_acc(a, w, 3)
    assert np.array_equal(g.sum(0), full)
    assert np.array_equal(g[1], a[:, 128:256].astype(np.int64) @ w[:, 128:256].astype(np.int64).T)


def test_epilogue_matches_fp32_fallback(oracle):
    """The restated integer+epilogue path agrees with the independent fp32
    dequant -> F.linear fallback on the same integer inputs."""
    rng = np.random.default_rng(2)
    M, N, K, G = 16, 24, 512, 4
    a = rng.integers(-128, 128, (M, K)).astype(np.int8)
    q = rng.integers(-8, 8, (N, K)).astype(np.int8)
    packed = oracle.pack_int4(q)
    s_a = (rng.random(M) * 0.01 + 1e-3).astype(np.float32)
    s_w = (rng.random((N, G)) * 0.02 + 1e-3).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    acc = oracle.gemm_acc(a, oracle.unpack_int4(packed, K), G)
    out = oracle.epilogue(acc, s_a, s_w, bias, out_dtype=2)
    ref = oracle.linear_fallback_fp32(a.astype(np.float32) * s_a[:, None], packed, s_w, K, True, bias)
    assert np.allclose(out, ref, rtol=1e-5, atol=1e-4)


def test_dequant_w4a16_exact(oracle):
    rng = np.random.default_rng(3)
    q = rng.integers(-8, 8, (6, 256)).astype(np.int8)
    s = (rng.random((6, 2)) * 0.02 + 1e-3).astype(np.float16).astype(np.float32)
    w = oracle.dequant_w4a16(oracle.pack_int4(q), s, 256, 0)
    exact = q.astype(np.float64) * np.repeat(s.astype(np.float64), 128, axis=1)
    assert np.array_equal(w, exact.astype(np.float16).astype(np.float32))


@pytest.mark.parametrize("int4", [True, False])
def test_reference_fallback_forward_matches_integer_chain(oracle, int4):
    """The fp32 fallback forward (SmoothRot divide, Hadamard by matmul, pad,
    perm, fp32 dequant, F.linear) and the integer chain (prepare -> per-token
    INT8 quantization -> exact accumulators -> epilogue) are independent
    codings of the same layer; they agree within the activation-quantization
    error.  A transposed operand, a wrong group layout or a misapplied perm
    in either one breaks the agreement."""
    g = torch.Generator().manual_seed(7)
    M, K_in, K_w, N, R = 12, 1000, 1280, 40, 256  # rotation pad 1000 -> 1024, then w_in pad to 1280
    x = torch.randn(M, K_in, generator=g).to(torch.float16)
    sr = torch.exp(torch.randn(K_in, generator=g) * 0.5)
    perm = torch.randperm(K_w, generator=g)
    if int4:
        q = torch.randint(-8, 8, (N, K_w), generator=g, dtype=torch.int8).numpy()
        w = oracle.pack_int4(q)
        s_w = (torch.rand(N, K_w // 128, generator=g) * 2e-2 + 1e-3).numpy().astype(np.float32)
    else:
        q = torch.randint(-127, 128, (N, K_w), generator=g, dtype=torch.int8).numpy()
        w = q
        s_w = (torch.rand(N, 1, generator=g) * 2e-3 + 1e-4).numpy().astype(np.float32)
    fb = oracle.reference_fallback_forward(x, w, s_w, K_w, int4=int4, smoothrot=sr, rot_size=R, perm=perm).numpy()
    y = oracle.prepare(x, oracle.DT_F16, smoothrot=sr, rot_size=R, w_in=K_w, perm=perm)
    qa, s_a = oracle.quantize(y)
    G = s_w.shape[1]
    acc = oracle.gemm_acc(qa, q, G)
    chain = oracle.epilogue(acc, s_a, s_w, None, out_dtype=oracle.DT_F32)
    cos = float((fb * chain).sum() / np.sqrt((fb * fb).sum() * (chain * chain).sum()))
    assert cos > 0.9999
    assert np.abs(fb - chain).max() < 0.02 * np.abs(fb).max()
