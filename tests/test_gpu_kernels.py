"""GPU parity of the gfx950 kernels against the CPU oracle.

Integer stages (INT8 activation codes, unpacked weights, int32 accumulators)
and the restated fp32 epilogue formula must be bit-exact; fp16/bf16 linear
outputs must also sit within rtol 1e-2 / cosine >= 0.9999 of the reference
fp32 dequant -> F.linear fallback.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DT = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _acts(M, K, dtype, seed, outliers=0.0, student_t=False):
    g = _gen(seed)
    if student_t:
        torch.manual_seed(seed)  # torch.distributions samples from the global generator
        x = torch.distributions.StudentT(4.0).sample((M, K))
    else:
        x = torch.randn(M, K, generator=g)
    if outliers:
        idx = torch.randperm(K, generator=g)[: max(1, int(K * outliers))]
        x[:, idx] *= 20.0
    return x.to(dtype)


# ------------------------------------------------------------------ unpack
def test_unpack_int4_known_answers(rt, oracle, dev):
    # tests/test_quant_utils.py:65-99 of the reference
    cases = [
        np.array([[-8, -1, 0, 1, 7, -3, 5, 0]], np.int8),
        np.array([[-8, 0, 7]], np.int8),
        np.full((2, 16), -8, np.int8),
        np.full((2, 16), 7, np.int8),
    ]
    for v in cases:
        packed = oracle.pack_int4(v)
        got = rt.unpack_int4_to_int8(torch.from_numpy(packed).to(dev), v.shape[1]).cpu().numpy()
        assert np.array_equal(got, v)


def test_unpack_int4_all_bytes(rt, oracle, dev):
    packed = np.arange(256, dtype=np.uint8).reshape(4, 64)
    got = rt.unpack_int4_to_int8(torch.from_numpy(packed).to(dev), 128).cpu().numpy()
    assert np.array_equal(got, oracle.unpack_int4(packed, 128))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("G", [1, 4])
def test_unpack_int4_to_float(rt, oracle, dev, dtype, G):
    g = _gen(1)
    N, K = 64, 512
    packed = torch.randint(0, 256, (N, K // 2), generator=g, dtype=torch.uint8)
    s = (torch.rand(N, G, generator=g) * 2e-2 + 1e-3).to(torch.float16).float()
    got = rt.unpack_int4_to_float(packed.to(dev), s.to(dev), K, dtype).float().cpu().numpy()
    ref = oracle.dequant_w4a16(packed.numpy(), s.numpy(), K, DT[dtype])
    assert np.array_equal(got, ref)


# ------------------------------------------------------------------ quantize
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("K", [64, 1000, 4096, 6144, 12288, 20480])
def test_dynamic_quantize(rt, oracle, dev, dtype, K):
    if dtype == torch.float32 and K > 8192 and K < 16384:
        K = 8192
    x = _acts(24, K, dtype, seed=K)
    x[3] = 0  # all-zero row: s = 1e-8/127, codes 0
    q, s = rt.dynamic_quantize_activation(x.to(dev))
    q_ref, s_ref = oracle.quantize(oracle.to_dtype_values(x, DT[dtype]))
    assert np.array_equal(s.cpu().numpy(), s_ref)
    assert np.array_equal(q.cpu().numpy(), q_ref)


def test_dynamic_quantize_3d_and_prealloc(rt, dev):
    x = torch.randn(2, 8, 128, device=dev, dtype=torch.float16)
    q, s = rt.dynamic_quantize_activation(x)
    assert q.shape == (2, 8, 128) and s.shape == (2, 8)
    s_buf = torch.empty(16, device=dev)
    q_buf = torch.empty(16, 128, dtype=torch.int8, device=dev)
    q2, s2 = rt.dynamic_quantize_activation(x.reshape(16, 128), s_a_out=s_buf, x_int8_out=q_buf)
    assert q2.data_ptr() == q_buf.data_ptr() and s2.data_ptr() == s_buf.data_ptr()
    assert torch.equal(q2, q.reshape(16, 128)) and torch.equal(s2, s.reshape(16))


def test_quantize_round_half_away_quirk(rt, dev):
    # q = 0.49999997 + 0.5 rounds to 1.0 in f32, so trunc gives 1 (triton_quantize.py:142-145)
    s = np.float32(127.0) / np.float32(127.0)  # row max 127 -> s = 1
    row = torch.tensor([[127.0, 0.49999997, -0.49999997, 2.5, -2.5, 0.5]], dtype=torch.float32)
    q, sc = rt.dynamic_quantize_activation(row.to(dev))
    assert float(sc[0]) == float(s)
    assert q.cpu().tolist() == [[127, 1, -1, 3, -3, 1]]


# ------------------------------------------------------------------ fused prep
ROT_CASES = [
    # (K_in, R, w_in, smoothrot, perm, smooth)
    (512, 16, None, False, False, False),
    (512, 64, None, True, False, False),
    (768, 256, None, True, True, False),
    (3072, 256, None, True, True, False),
    (2048, 1024, None, False, True, False),
    (4096, 4096, None, False, False, False),
    (8192, 4096, None, True, True, False),
    (1000, 256, None, False, False, False),     # rotation pad 1000 -> 1024
    (1000, 0, 1024, True, True, False),         # w_in pad, no rotation
    (1536, 1024, 2304, False, True, False),     # rotation pad 1536 -> 2048, then w_in pad
    (640, 64, None, False, True, True),         # old SmoothQuant after the gather
    (13824, 1024, 14336, False, False, False),  # Wan FFN-down pad path
    (12288, 256, None, True, True, False),      # Flux MLP down-proj (C3 prep)
    (5120, 256, None, False, False, False),     # three-wave workgroups, two tiles (Wan qkv/proj width)
    (5120, 64, None, True, True, False),
    (6144, 256, None, False, True, False),
    (3072, 16, None, True, False, False),       # three-wave workgroups, one full tile
    (5120, 1024, None, True, True, False),      # five one-block waves, one tile (Wan qkv/proj/FFN-up prep)
    (4200, 1024, None, False, True, False),     # the same, rotation pad 4200 -> 5120
    (2500, 1024, None, True, False, False),     # three one-block waves, pad 2500 -> 3072
    (6000, 1024, 6400, True, True, False),      # three-wave workgroups, two tiles, then w_in pad
    (2048, 64, None, False, False, False),      # no perm: rows kept in the waves' exchange slices, one tile
    (6144, 64, None, False, False, False),      # the same with two three-wave tiles
    (9216, 256, None, True, True, False),       # one twelve-wave tile, 3072 positions of it padding
    (10000, 1024, 11008, False, True, False),   # the same tile with one-block waves, pads to 10240 and 11008
    (15360, 256, None, True, True, False),      # two eight-wave tiles (Flux single-block output projection)
    (16384, 1024, None, True, True, False),     # two eight-wave tiles, one-block waves (RC = 3 layout)
    (15360, 64, None, False, True, False),      # two eight-wave tiles, 64-blocks
]


def _prep_inputs(K_in, R, w_in, use_sr, use_perm, use_sm, seed):
    g = _gen(seed)
    K_r = ((K_in + R - 1) // R) * R if R else K_in
    K_w = max(w_in or K_r, K_r)
    sr = torch.exp(torch.randn(K_in, generator=g) * 0.5) if use_sr else None
    perm = torch.randperm(K_w, generator=g) if use_perm else None
    sm = torch.exp(torch.randn(K_w, generator=g) * 0.3) if use_sm else None
    return K_w, sr, perm, sm


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("case", ROT_CASES)
def test_rotate_quantize_bit_exact(rt, oracle, dev, dtype, case):
    K_in, R, w_in, use_sr, use_perm, use_sm = case
    K_w, sr, perm, sm = _prep_inputs(K_in, R, w_in, use_sr, use_perm, use_sm, seed=K_in + R)
    x = _acts(6, K_in, dtype, seed=R + 7, outliers=0.01)
    x[2] = 0
    srp = rt.prepare_factors(sr.to(dev), dtype) if sr is not None else None
    smp = rt.prepare_factors(sm.to(dev), dtype) if sm is not None else None
    pp = rt.prepare_perm(perm.to(dev), K_w) if perm is not None else None
    q, s = rt.rotate_quantize(x.to(dev), rot_size=R, w_in=K_w, smoothrot=srp, perm=pp, smooth=smp)
    y = rt.prepare_activation(x.to(dev), rot_size=R, w_in=K_w, smoothrot=srp, perm=pp, smooth=smp)
    y_ref = oracle.prepare(x, DT[dtype], smoothrot=sr, rot_size=R, w_in=K_w, perm=perm, smooth=sm)
    q_ref, s_ref = oracle.quantize(y_ref)
    assert np.array_equal(y.float().cpu().numpy(), y_ref)
    assert np.array_equal(s.cpu().numpy(), s_ref)
    assert np.array_equal(q.cpu().numpy(), q_ref)


def _bf16_wide_rows(M, K, R, seed):
    """bf16 rows whose Hadamard blocks span far beyond double's exact range:
    GELU-tanh of N(0, 16) (tails down to ~1e-37 next to values of ~20), and a
    first row of crafted blocks [1, 2^-8, t, 0, ...]: their outputs
    2^-k (1 +- 2^-8) sit on bf16 rounding midpoints, and the tiny term t is
    either inside the exact span (2^-30, breaks the tie upwards) or beyond it
    (2^-100, flushed, tie to even)."""
    g = _gen(seed)
    x = torch.nn.functional.gelu(torch.randn(M, K, generator=g) * 4.0, approximate="tanh")
    x[0] = 0.0
    for b, b0 in enumerate(range(0, K, R)):
        x[0, b0] = 1.0
        x[0, b0 + 1] = 2.0 ** -8
        x[0, b0 + 2] = 2.0 ** -30 if b % 2 else 2.0 ** -100
    return x.to(torch.bfloat16)


@pytest.mark.parametrize("R", [16, 64, 256, 1024, 4096])
@pytest.mark.parametrize("path", ["fast", "general"])
def test_bf16_wide_span_rows_match_oracle(rt, oracle, dev, R, path):
    """Rows with ~1e-37 tails (post-GELU activations): the kernels flush
    inputs beyond each block's exact span exactly as the oracle does and
    rotate the rest exactly -- prepared values, codes and scales bit-exact.
    "fast" runs the single-pass kernel (SmoothRot + perm, aligned rows);
    "general" the one-workgroup-per-row kernel (an odd row stride)."""
    M, K = 6, 8192
    x = _bf16_wide_rows(M, K, R, seed=R)
    K_w, sr, perm, _ = _prep_inputs(K, R, None, True, True, False, seed=R + 1)
    srp = rt.prepare_factors(sr.to(dev), torch.bfloat16)
    pp = rt.prepare_perm(perm.to(dev), K_w)
    xd = x.to(dev)
    if path == "general":
        xd = torch.zeros(M, K + 3, dtype=torch.bfloat16, device=dev)[:, :K]
        xd.copy_(x.to(dev))
    q, s = rt.rotate_quantize(xd, rot_size=R, w_in=K_w, smoothrot=srp, perm=pp)
    y = rt.prepare_activation(xd, rot_size=R, w_in=K_w, smoothrot=srp, perm=pp)
    y_ref = oracle.prepare(x, 1, smoothrot=sr, rot_size=R, w_in=K_w, perm=perm)
    q_ref, s_ref = oracle.quantize(y_ref)
    assert np.array_equal(y.float().cpu().numpy(), y_ref)
    assert np.array_equal(s.cpu().numpy(), s_ref)
    assert np.array_equal(q.cpu().numpy(), q_ref)
    # the crafted row: no SmoothRot / perm, outputs of block 0 / 1 on known values
    y0 = rt.prepare_activation(x[:1].to(dev), rot_size=R).float().cpu()
    k = {16: 2, 64: 3, 256: 4, 1024: 5, 4096: 6}[R]
    u = 2.0 ** -k
    assert float(y0[0, 0]) == u  # block 0: 2^-100 flushed, 2^-k (1 + 2^-8) ties to even
    assert float(y0[0, R]) == u * (1 + 2.0 ** -7)  # block 1: 2^-30 kept, the tie breaks upwards


def test_rotate_quantize_f32(rt, oracle, dev):
    x = _acts(4, 2048, torch.float32, seed=3)
    fac = torch.exp(torch.randn(2048, generator=_gen(4)) * 0.5)
    srp = rt.prepare_factors(fac.to(dev), torch.float32)
    q, s = rt.rotate_quantize(x.to(dev), rot_size=256, smoothrot=srp)
    q_ref, s_ref = oracle.rotate_quantize(x, 2, smoothrot=fac, rot_size=256)
    # f32 rows are exact whenever the oracle reports every block sum exact;
    # allow +-1 code where a block is not (documented fp64 limitation)
    assert np.array_equal(s.cpu().numpy(), s_ref) or np.allclose(s.cpu().numpy(), s_ref, rtol=1e-6)
    assert np.abs(q.cpu().numpy().astype(int) - q_ref.astype(int)).max() <= 1


def test_rotate_quantize_determinism(rt, dev):
    x = torch.randn(64, 3072, device=dev, dtype=torch.float16)
    a = rt.rotate_quantize(x, rot_size=256)
    b = rt.rotate_quantize(x, rot_size=256)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


# ------------------------------------------------------------------ GEMMs
GEMM_SHAPES = [(256, 256, 256), (300, 200, 192), (512, 384, 1024), (16, 1024, 512), (1, 96, 128)]


def _int8(shape, seed, lo=-128, hi=128):
    return torch.randint(lo, hi, shape, generator=_gen(seed), dtype=torch.int8)


@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
def test_w8a8_accumulators(rt, oracle, dev, M, N, K):
    a = _int8((M, K), 1)
    w = _int8((N, K), 2)
    acc = rt.gemm_acc_i32(a.to(dev), w.to(dev)).cpu().numpy()
    assert np.array_equal(acc, oracle.gemm_acc(a.numpy(), w.numpy()))


@pytest.mark.parametrize("M,N,K", [(4096, 4096, 256), (4096, 3072, 256), (4000, 3000, 384)])
def test_w8a8_accumulators_full_grid(rt, dev, M, N, K):
    """Shapes that fill the CUs with 256 x 256 tiles (4096^2) or 256 x 192
    tiles (4096 x 3072, and ragged edges): int32 accumulators equal the exact
    integer matmul, computed in float64 on the CPU (|acc| < 2^53)."""
    a = _int8((M, K), 21)
    w = _int8((N, K), 22)
    acc = rt.gemm_acc_i32(a.to(dev), w.to(dev)).cpu()
    ref = (a.double() @ w.double().T).to(torch.int64)
    assert torch.equal(acc.to(torch.int64), ref)


@pytest.mark.parametrize("M,N,K", [(4096, 3072, 256), (4000, 3000, 384)])
@pytest.mark.parametrize("grouped", [False, True])
def test_w4a8_accumulators_full_grid(rt, oracle, dev, M, N, K, grouped):
    """Shapes large enough for 256 x 128 tiles (small ones take 128 x 128):
    int32 accumulators (per 128-group when grouped) equal the exact integer
    matmul of the unpacked weights, computed in float64 on the CPU."""
    G = K // 128 if grouped else 1
    a = _int8((M, K), 23)
    packed = torch.randint(0, 256, (N, K // 2), generator=_gen(24), dtype=torch.uint8)
    s_w = torch.rand(N, G, generator=_gen(25)) * 1e-2 + 1e-3
    acc = rt.gemm_acc_i32(a.to(dev), packed.to(dev), int4=True, s_w=s_w.to(dev)).cpu().to(torch.int64)
    w = torch.from_numpy(oracle.unpack_int4(packed.numpy(), K)).double()
    ad = a.double()
    if G == 1:
        ref = (ad @ w.T).to(torch.int64)
    else:
        ref = torch.stack([(ad[:, 128 * g:128 * g + 128] @ w[:, 128 * g:128 * g + 128].T) for g in range(G)]).to(torch.int64)
    assert torch.equal(acc, ref)


@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
@pytest.mark.parametrize("G", [1, "g128"])
def test_w4a8_accumulators(rt, oracle, dev, M, N, K, G):
    G = K // 128 if G == "g128" and K % 128 == 0 else 1
    a = _int8((M, K), 3)
    packed = torch.randint(0, 256, (N, K // 2), generator=_gen(4), dtype=torch.uint8)
    s_w = torch.rand(N, G, generator=_gen(5)) * 1e-2 + 1e-3
    acc = rt.gemm_acc_i32(a.to(dev), packed.to(dev), int4=True, s_w=s_w.to(dev)).cpu().numpy()
    ref = oracle.gemm_acc(a.numpy(), oracle.unpack_int4(packed.numpy(), K), G)
    assert np.array_equal(acc, ref)


@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("with_bias", [False, True])
@pytest.mark.parametrize("M,N,K", [(256, 256, 512), (130, 320, 192)])
def test_w8a8_output_formula(rt, oracle, dev, out_dtype, with_bias, M, N, K):
    a = _int8((M, K), 6)
    w = _int8((N, K), 7, -127, 128)
    s_a = torch.rand(M, generator=_gen(8)) * 0.05 + 1e-3
    s_w = (torch.rand(N, generator=_gen(9)) * 2e-3 + 1e-4).to(torch.float16).float()
    bias = (torch.randn(N, generator=_gen(10))).to(out_dtype) if with_bias else None
    out = rt.fused_int8_gemm_dequant(a.to(dev), w.to(dev), s_w.to(dev), s_a.to(dev),
                                     bias=None if bias is None else bias.to(dev), out_dtype=out_dtype)
    acc = oracle.gemm_acc(a.numpy(), w.numpy())
    ref = oracle.epilogue(acc, s_a.numpy(), s_w.numpy(), None if bias is None else bias.float().numpy(),
                          DT[out_dtype])
    assert np.array_equal(out.float().cpu().numpy(), ref)


@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("grouped", [False, True])
@pytest.mark.parametrize("M,N,K", [(256, 256, 512), (260, 136, 384), (4608, 3072, 1024)])
def test_w4a8_output_formula(rt, oracle, dev, out_dtype, grouped, M, N, K):
    G = K // 128 if grouped else 1
    a = _int8((M, K), 11)
    packed = torch.randint(0, 256, (N, K // 2), generator=_gen(12), dtype=torch.uint8)
    s_a = torch.rand(M, generator=_gen(13)) * 0.05 + 1e-3
    s_w = (torch.rand(N, G, generator=_gen(14)) * 2e-2 + 1e-3).to(torch.float16).float()
    bias = torch.randn(N, generator=_gen(15)).to(out_dtype)
    out = rt.gemm_w4a8(a.to(dev), packed.to(dev), s_w.to(dev), s_a.to(dev), bias=bias.to(dev),
                       out_dtype=out_dtype)
    acc = oracle.gemm_acc(a.numpy(), oracle.unpack_int4(packed.numpy(), K), G)
    ref = oracle.epilogue(acc, s_a.numpy(), s_w.numpy(), bias.float().numpy(), DT[out_dtype])
    assert np.array_equal(out.float().cpu().numpy(), ref)


SPLITK_SHAPES = [(64, 3072, 12288), (512, 3072, 12288), (100, 1000, 3072)]


@pytest.mark.parametrize("M,N,K", SPLITK_SHAPES)
@pytest.mark.parametrize("fmt", ["int8", "int4"])
def test_splitk_per_row_bit_exact(rt, oracle, dev, M, N, K, fmt):
    """Small M: the library splits K over workgroups (the size query says
    so); with per-row scales the int32 partials add exactly, so the output
    equals the oracle's unsplit epilogue formula bit for bit."""
    int4 = fmt == "int4"
    assert rt.lib().ic_gemm_splitk_bytes(M, N, K, 1, int(int4)) > 0
    a = _int8((M, K), 51, -127, 128)
    s_a = torch.rand(M, generator=_gen(52)) * 0.05 + 1e-3
    s_w = (torch.rand(N, generator=_gen(53)) * 2e-3 + 1e-4).to(torch.float16).float()
    bias = torch.randn(N, generator=_gen(54)).to(torch.bfloat16)
    if int4:
        w = torch.randint(0, 256, (N, K // 2), generator=_gen(55), dtype=torch.uint8)
        out = rt.gemm_w4a8(a.to(dev), w.to(dev), s_w.to(dev), s_a.to(dev), bias=bias.to(dev), out_dtype=torch.bfloat16)
        wq = oracle.unpack_int4(w.numpy(), K)
    else:
        w = _int8((N, K), 55, -127, 128)
        out = rt.fused_int8_gemm_dequant(a.to(dev), w.to(dev), s_w.to(dev), s_a.to(dev), bias=bias.to(dev),
                                         out_dtype=torch.bfloat16)
        wq = w.numpy()
    ref = oracle.epilogue(oracle.gemm_acc(a.numpy(), wq), s_a.numpy(), s_w.numpy(), bias.float().numpy(),
                          DT[torch.bfloat16])
    assert np.array_equal(out.float().cpu().numpy(), ref)


@pytest.mark.parametrize("M,N,K", SPLITK_SHAPES)
def test_splitk_grouped_w4a8(rt, oracle, dev, M, N, K):
    """Grouped scales with split K: each slice folds its groups in order and
    the slices' fp32 partials are added in slice order, so outputs may differ
    from the single fold chain by fp32 rounding only.  Both sums are within
    G * 2^-24 * T of the exact value (T = sum of the absolute group terms), so
    they differ by at most G * 2^-23 * T, plus one fp16 ulp where the final
    rounding falls differently; and both sit within the fp32 dequant ->
    F.linear tolerance."""
    G = K // 128
    assert rt.lib().ic_gemm_splitk_bytes(M, N, K, G, 1) > 0
    a = _int8((M, K), 56, -127, 128)
    w = torch.randint(0, 256, (N, K // 2), generator=_gen(57), dtype=torch.uint8)
    s_a = torch.rand(M, generator=_gen(58)) * 0.05 + 1e-3
    s_w = (torch.rand(N, G, generator=_gen(59)) * 2e-2 + 1e-3).to(torch.float16).float()
    out = rt.gemm_w4a8(a.to(dev), w.to(dev), s_w.to(dev), s_a.to(dev), out_dtype=torch.float16).float().cpu()
    wq = oracle.unpack_int4(w.numpy(), K)
    acc = oracle.gemm_acc(a.numpy(), wq, G)  # [G, M, N]
    ref = torch.from_numpy(oracle.epilogue(acc, s_a.numpy(), s_w.numpy(), None, DT[torch.float16]))
    terms = (np.abs(acc).astype(np.float64) * s_w.numpy().T.astype(np.float64)[:, None, :]).sum(0)
    T = torch.from_numpy(terms * s_a.numpy().astype(np.float64)[:, None])
    big = torch.maximum(out.abs(), ref.abs()).clamp_min(2.0 ** -14)
    ulp = torch.pow(2.0, torch.floor(torch.log2(big))) * 2.0 ** -10
    assert ((out - ref).abs().double() <= G * 2.0 ** -23 * T + ulp.double()).all()
    exact = (a.double() @ (torch.from_numpy(wq).double().reshape(N, G, 128)
                           * s_w.double().reshape(N, G, 1)).reshape(N, K).T) * s_a.double().reshape(M, 1)
    assert torch.allclose(out.double(), exact, rtol=1e-2, atol=1e-2 * exact.abs().max().item() * 1e-2)
    assert _cos(out, exact.float()) >= 0.9999


C5_ROWS = [0, 1, 255, 256, 12345, 32511, 32512, 32759]  # tile edges and the last, partial tile


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_c5_full_size_prep_sampled_rows(rt, oracle, dev, dtype):
    """Wan FFN-down activation prep at full size: 32760 rows of 13824 (1% of
    channels x20), rotated in 1024-blocks and padded to 14336.  Rows are
    independent, so sampled rows (first, last, tile edges) must equal the
    oracle's prep and quantization bit for bit.  (Heavy-tailed Student-t rows
    are the accuracy gate's input, test_c5_accuracy_gate_student_t.)"""
    M, K_in, K_w = 32760, 13824, 14336
    x = _acts(M, K_in, dtype, seed=41, outliers=0.01)
    q, s = rt.rotate_quantize(x.to(dev), rot_size=1024, w_in=K_w)
    rows = torch.tensor(C5_ROWS)
    y_ref = oracle.prepare(x[rows], DT[dtype], smoothrot=None, rot_size=1024, w_in=K_w, perm=None, smooth=None)
    q_ref, s_ref = oracle.quantize(y_ref)
    assert np.array_equal(s[rows.to(dev)].cpu().numpy(), s_ref)
    assert np.array_equal(q[rows.to(dev)].cpu().numpy(), q_ref)


# (M, K_in, R, w_in, SmoothRot + perm): the persistent row loop of the wide
# prep tiles (each workgroup walks rows r, r + grid, ...; the next row's
# activations are loaded while the current one is rotated).  Sampled rows: the
# first ones (first row of a workgroup), the first rows of a workgroup's second
# and later iterations, and the last rows.
FULL_PREP = [
    (4608, 12288, 256, None, True),    # C3: one twelve-wave tile
    (4608, 15360, 256, None, True),    # Flux single-block projection: two eight-wave tiles
    (2048, 16384, 1024, None, True),   # two eight-wave tiles, one-block waves
    (2048, 15360, 64, None, False),
]
FULL_PREP_ROWS = [0, 1, 255, 256, 257, 511, 512, 1023, 1024, 1500, 2047]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,K_in,R,w_in,srp", FULL_PREP)
def test_wide_prep_persistent_rows(rt, oracle, dev, dtype, M, K_in, R, w_in, srp):
    K_w, sr, perm, _ = _prep_inputs(K_in, R, w_in, srp, srp, False, seed=K_in + 3)
    x = _acts(M, K_in, dtype, seed=K_in + 5, outliers=0.01)
    srf = rt.prepare_factors(sr.to(dev), dtype) if sr is not None else None
    pp = rt.prepare_perm(perm.to(dev), K_w) if perm is not None else None
    q, s = rt.rotate_quantize(x.to(dev), rot_size=R, w_in=K_w, smoothrot=srf, perm=pp)
    rows = torch.tensor([r for r in FULL_PREP_ROWS if r < M] + [M - 2, M - 1])
    q_ref, s_ref = oracle.rotate_quantize(x[rows], DT[dtype], smoothrot=sr, rot_size=R, w_in=K_w, perm=perm)
    assert np.array_equal(s[rows.to(dev)].cpu().numpy(), s_ref)
    assert np.array_equal(q[rows.to(dev)].cpu().numpy(), q_ref)


@pytest.mark.parametrize("fmt", ["int4_g128", "int8"])
def test_c5_full_size_gemm_sampled_rows(rt, oracle, dev, fmt):
    """Wan FFN-down at its full size (M=32760, K_w=14336, N=5120; G=112 for
    INT4): one launch of the production kernel, and the output rows at tile
    edges and in the last partial M-tile equal the oracle's accumulators and
    epilogue formula bit for bit."""
    M, K, N = 32760, 14336, 5120
    a = _int8((M, K), 31, -127, 128)
    s_a = torch.rand(M, generator=_gen(32)) * 0.05 + 1e-3
    if fmt == "int8":
        w = _int8((N, K), 33, -127, 128)
        s_w = (torch.rand(N, generator=_gen(34)) * 2e-3 + 1e-4).to(torch.float16).float()
        out = rt.fused_int8_gemm_dequant(a.to(dev), w.to(dev), s_w.to(dev), s_a.to(dev),
                                         out_dtype=torch.float16)
        w_q, G = w.numpy(), 1
    else:
        G = K // 128
        w = torch.randint(0, 256, (N, K // 2), generator=_gen(35), dtype=torch.uint8)
        s_w = (torch.rand(N, G, generator=_gen(36)) * 2e-2 + 1e-3).to(torch.float16).float()
        out = rt.gemm_w4a8(a.to(dev), w.to(dev), s_w.to(dev), s_a.to(dev), out_dtype=torch.float16)
        w_q = oracle.unpack_int4(w.numpy(), K)
    rows = torch.tensor(C5_ROWS)
    acc = oracle.gemm_acc(a[rows].numpy(), w_q, G)
    ref = oracle.epilogue(acc, s_a[rows].numpy(), s_w.numpy(), None, DT[torch.float16])
    assert np.array_equal(out[rows.to(dev)].float().cpu().numpy(), ref)


def test_w8a8_generic_kernel_matches(rt, dev):
    M, N, K = 64, 96, 200  # K not a multiple of 64 -> generic kernel
    a = _int8((M, K), 16).to(dev)
    w = _int8((N, K), 17).to(dev)
    s_a = torch.rand(M, device=dev) * 0.01 + 1e-3
    s_w = torch.rand(N, device=dev) * 0.01 + 1e-3
    out = rt.fused_int8_gemm_dequant(a, w, s_w, s_a, out_dtype=torch.float32)
    ref = (a.float() @ w.float().t()) * (s_a[:, None] * s_w[None, :])
    assert torch.allclose(out, ref, rtol=1e-6, atol=1e-6)


def _cos(a, b):
    a = a.reshape(-1).double()
    b = b.reshape(-1).double()
    return float((a @ b) / (a.norm() * b.norm()))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("G", [1, 24])
def test_w4a16_vs_fp32(rt, oracle, dev, dtype, G):
    M, N, K = 300, 512, 3072
    x = _acts(M, K, dtype, seed=20)
    packed = torch.randint(0, 256, (N, K // 2), generator=_gen(21), dtype=torch.uint8)
    s_w = (torch.rand(N, G, generator=_gen(22)) * 2e-2 + 1e-3).to(torch.float16).float()
    bias = torch.randn(N, generator=_gen(23)).to(dtype)
    out = rt.gemm_w4a16(x.to(dev), packed.to(dev), s_w.to(dev), bias=bias.to(dev)).float().cpu()
    w = torch.from_numpy(oracle.dequant_w4a16(packed.numpy(), s_w.numpy(), K, DT[dtype]))
    ref = x.float() @ w.t() + bias.float()
    # fp32 accumulation order differs from the CPU; the output is one rounding of it
    tol = 1e-2 if dtype == torch.float16 else 2e-2
    assert torch.allclose(out, ref, rtol=tol, atol=tol * ref.abs().max().item() * 1e-2)
    assert _cos(out, ref) >= 0.9999


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("grouped", [False, True])
@pytest.mark.parametrize("M,N", [(512, 300), (512, 264), (100, 264)])
def test_w4a16_dequant_bit_exact_one_hot(rt, oracle, dev, dtype, grouped, M, N):
    """x = one-hot rows (row m selects k = m): each output is a single product
    1 * w[n, m] accumulated in fp32 and rounded to the activation type, so the
    GEMM output equals the kernel's in-LDS dequantized weight, which must be
    RN_dt(q * RN_dt(s)) bit for bit.  N = 300 takes the direct epilogue, N = 264
    the LDS-staged one; M = 100 the 128-row tile."""
    K = 512
    G = K // 128 if grouped else 1
    x = torch.zeros(M, K, dtype=dtype)
    x[torch.arange(M), torch.arange(M) % K] = 1
    packed = torch.randint(0, 256, (N, K // 2), generator=_gen(24), dtype=torch.uint8)
    s_w = (torch.rand(N, G, generator=_gen(25)) * 2e-2 + 1e-3).to(torch.float16).float()
    out = rt.gemm_w4a16(x.to(dev), packed.to(dev), s_w.to(dev)).float().cpu().numpy()
    w = oracle.dequant_w4a16(packed.numpy(), s_w.numpy(), K, DT[dtype])  # [N, K]
    assert np.array_equal(out, w[:, np.arange(M) % K].T)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_w4a16_full_size_c2_sampled_rows(rt, oracle, dev, dtype):
    """C2 at full size (M=4608, K=3072, N=12288, g128): one launch; sampled
    rows (tile edges, last tile) within fp32-accumulation tolerance of the
    dequantized-weight product computed on the CPU."""
    M, K, N, G = 4608, 3072, 12288, 24
    x = _acts(M, K, dtype, seed=26)
    packed = torch.randint(0, 256, (N, K // 2), generator=_gen(27), dtype=torch.uint8)
    s_w = (torch.rand(N, G, generator=_gen(28)) * 2e-2 + 1e-3).to(torch.float16).float()
    out = rt.gemm_w4a16(x.to(dev), packed.to(dev), s_w.to(dev))
    rows = torch.tensor([0, 1, 255, 256, 2000, 4351, 4352, 4607])
    w = torch.from_numpy(oracle.dequant_w4a16(packed.numpy(), s_w.numpy(), K, DT[dtype]))
    ref = x[rows].float() @ w.t()
    got = out[rows.to(dev)].float().cpu()
    tol = 1e-2 if dtype == torch.float16 else 2e-2
    assert torch.allclose(got, ref, rtol=tol, atol=tol * ref.abs().max().item() * 1e-2)
    assert _cos(got, ref) >= 0.9999


# ------------------------------------------------------------------ linear accuracy gate
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_w4a8_linear_vs_fp32_fallback(rt, oracle, dev, dtype):
    """C3-style layer at reduced M: fused prep + W4A8 vs the fp32 dequant->F.linear fallback."""
    M, K, N, R = 128, 12288, 512, 256
    g = _gen(30)
    x = _acts(M, K, dtype, seed=31, outliers=0.01)
    sr = torch.exp(torch.randn(K, generator=g) * 0.5)
    perm = torch.randperm(K, generator=g)
    W = torch.randn(N, K, generator=g)
    # converter-side group quantization (_quant_utils.py:237-270) in permuted space
    Wg = W.reshape(N, K // 128, 128)
    s_w = (Wg.abs().amax(-1) / 7.0).clamp(min=1e-8).to(torch.float16).float()
    qw = (Wg / s_w[..., None]).round().clamp(-8, 7).to(torch.int8).reshape(N, K)
    packed = torch.from_numpy(oracle.pack_int4(qw.numpy()))
    bias = torch.randn(N, generator=g).to(dtype)
    srp = rt.prepare_factors(sr.to(dev), dtype)
    q, s = rt.rotate_quantize(x.to(dev), rot_size=R, w_in=K, smoothrot=srp, perm=rt.prepare_perm(perm.to(dev), K))
    out = rt.gemm_w4a8(q, packed.to(dev), s_w.to(dev), s, bias=bias.to(dev), out_dtype=dtype).float().cpu()
    x_prep = oracle.prepare(x, DT[dtype], smoothrot=sr, rot_size=R, w_in=K, perm=perm)
    ref = torch.from_numpy(oracle.linear_fallback_fp32(x_prep, packed.numpy(), s_w.numpy(), K, True,
                                                        bias.float().numpy()))
    rel = (out - ref).norm() / ref.norm()
    assert _cos(out, ref) >= 0.9999, f"cosine {_cos(out, ref)} rel {rel}"


@pytest.mark.parametrize("fmt", ["w4a8_g128", "w8a8"])
def test_c5_accuracy_gate_student_t(rt, oracle, dev, fmt):
    """The C5 accuracy gate on its heavy-tailed input: Wan FFN-down
    (13824 -> 14336 with the R=1024 pad, N=5120) at full K and N on 256
    Student-t (nu = 4) fp16 rows.  Weights are a random layer of the padded
    space quantized by the converter's rule (_quant_utils.py:237-270: INT4
    with fp16 scales per 128-group, or INT8 per output row).  The fused prep +
    GEMM output must reach cosine >= 0.9999 against the reference fp32
    fallback (fp32 prep, W = q * s, F.linear), the north-star bar."""
    M, K_in, K, N, R = 256, 13824, 14336, 5120, 1024
    x = _acts(M, K_in, torch.float16, seed=61, student_t=True)
    W = torch.randn(N, K, generator=_gen(62)) * 0.02
    if fmt == "w8a8":
        s_w = (W.abs().amax(1) / 127.0).clamp(min=1e-8).to(torch.float16).float()
        wq = (W / s_w[:, None]).round().clamp(-128, 127).to(torch.int8)
        wt = wq
    else:
        Wg = W.reshape(N, K // 128, 128)
        s_w = (Wg.abs().amax(-1) / 7.0).clamp(min=1e-8).to(torch.float16).float()
        wq = (Wg / s_w[..., None]).round().clamp(-8, 7).to(torch.int8).reshape(N, K)
        wt = torch.from_numpy(oracle.pack_int4(wq.numpy()))
    q, s = rt.rotate_quantize(x.to(dev), rot_size=R, w_in=K)
    if fmt == "w8a8":
        out = rt.fused_int8_gemm_dequant(q, wt.to(dev), s_w.to(dev), s, out_dtype=torch.float16)
    else:
        out = rt.gemm_w4a8(q, wt.to(dev), s_w.to(dev), s, out_dtype=torch.float16)
    out = out.float().cpu()
    ref = oracle.reference_fallback_forward(x, wt.numpy(), s_w.numpy(), K, int4=fmt != "w8a8", rot_size=R)
    c = _cos(out, ref)
    rel = float((out - ref).norm() / ref.norm())
    print(f"[c5 gate {fmt}] cosine {c:.7f}, relative error {rel:.4g}", flush=True)  # the margin, with -s
    assert torch.isfinite(out).all()
    assert c >= 0.9999, f"cosine {c:.7f}, relative error {rel:.4g}"


def test_w8a8_linear_vs_fp32_fallback(rt, oracle, dev):
    """C1-style layer at reduced M (rot_size 0, per-channel scales)."""
    M, K, N = 256, 3072, 768
    g = _gen(40)
    x = torch.randn(M, K, generator=g).to(torch.float16)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    s_w = (torch.rand(N, generator=g) * (2e-3 - 1e-4) + 1e-4).to(torch.float16).float()
    q, s = rt.dynamic_quantize_activation(x.to(dev))
    out = rt.fused_int8_gemm_dequant(q, w.to(dev), s_w.to(dev), s, out_dtype=torch.float16).float().cpu()
    ref = torch.from_numpy(oracle.linear_fallback_fp32(x.float().numpy(), w.numpy(), s_w.numpy(), K, False))
    assert _cos(out, ref) >= 0.9999


# ------------------------------------------------------------------ rows wider than one workgroup
@pytest.mark.parametrize("dtype,K_in,R,w_in", [
    (torch.bfloat16, 20480, 256, None),
    (torch.float16, 24576, 1024, 25600),      # rotation and w_in pads on top of the chunking
    (torch.bfloat16, 17000, 64, None),        # pad 17000 -> 17024 inside the last chunk
])
def test_wide_rows_prep_bit_exact(rt, oracle, dev, dtype, K_in, R, w_in):
    """Rows wider than the single-pass kernels hold (16384 16-bit values): the
    rotation runs on column chunks of whole Hadamard blocks, then the pad,
    perm gather and quantization in a second pass -- the same values, codes
    and scales as the oracle's one-shot prep."""
    M = 5
    K_w, sr, perm, _ = _prep_inputs(K_in, R, w_in, True, True, False, seed=K_in)
    x = _acts(M, K_in, dtype, seed=K_in + 1, outliers=0.01)
    srp = rt.prepare_factors(sr.to(dev), dtype)
    pp = rt.prepare_perm(perm.to(dev), K_w)
    q, s = rt.rotate_quantize(x.to(dev), rot_size=R, w_in=K_w, smoothrot=srp, perm=pp)
    y = rt.prepare_activation(x.to(dev), rot_size=R, w_in=K_w, smoothrot=srp, perm=pp)
    y_ref = oracle.prepare(x, DT[dtype], smoothrot=sr, rot_size=R, w_in=K_w, perm=perm)
    q_ref, s_ref = oracle.quantize(y_ref)
    assert np.array_equal(y.float().cpu().numpy(), y_ref)
    assert np.array_equal(s.cpu().numpy(), s_ref)
    assert np.array_equal(q.cpu().numpy(), q_ref)


def test_wide_rows_prep_f32_and_old_smooth(rt, oracle, dev):
    """f32 rows wider than 8192 (the f32 single-pass limit) with the
    old-SmoothQuant divide after the gather: values within the documented
    f32 bound (blocks whose double sums are inexact: +-1 code)."""
    M, K = 4, 12288
    K_w, _, perm, sm = _prep_inputs(K, 256, None, False, True, True, seed=5)
    x = _acts(M, K, torch.float32, seed=6)
    smp = rt.prepare_factors(sm.to(dev), torch.float32)
    q, s = rt.rotate_quantize(x.to(dev), rot_size=256, w_in=K_w, perm=rt.prepare_perm(perm.to(dev), K_w), smooth=smp)
    q_ref, s_ref = oracle.rotate_quantize(x, 2, rot_size=256, w_in=K_w, perm=perm, smooth=sm)
    assert np.allclose(s.cpu().numpy(), s_ref, rtol=1e-6)
    assert np.abs(q.cpu().numpy().astype(int) - q_ref.astype(int)).max() <= 1


# ------------------------------------------------------------------ 288 x 192 grouped INT4 tiles
# Shapes whose 256 x 128 tiling ends in a partly filled round of workgroups
# on 256 CUs and whose 288 x 192 (or 256 x 192) tiling takes fewer rounds: the
# library runs them on gemm_i8_big_kernel (16-bit outputs).  C3 itself, a
# shape partial in both M and N with 128- and 256-column groups, and shapes
# that take the 256-row (4096 rows) and 320-row (5120 rows) variants, with
# 128- and 64-column groups.
BIG_TILE_CASES = [(4608, 3072, 12288, 128), (4600, 3064, 1024, 128), (4600, 3064, 1024, 256),
                  (4096, 3072, 1024, 128), (4000, 3064, 1024, 64),
                  (5120, 3072, 1024, 128), (5100, 3064, 1024, 64)]  # 320-row variant


@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,N,K,gs", BIG_TILE_CASES)
def test_w4a8_big_tile_sampled_rows(rt, oracle, dev, out_dtype, M, N, K, gs):
    """Grouped W4A8 on the 288 x 192 tiles: every column of sampled rows
    (first and last rows of tiles, the partial last tile row) bit-exact
    against the oracle's accumulators and epilogue."""
    G = K // gs
    a = _int8((M, K), 91, -127, 128)
    w = torch.randint(0, 256, (N, K // 2), generator=_gen(92), dtype=torch.uint8)
    s_a = torch.rand(M, generator=_gen(93)) * 0.05 + 1e-3
    s_w = (torch.rand(N, G, generator=_gen(94)) * 2e-2 + 1e-3).to(torch.float16).float()
    bias = torch.randn(N, generator=_gen(95)).to(out_dtype)
    assert rt.lib().ic_gemm_splitk_bytes(M, N, K, G, 1) == 0
    out = rt.gemm_w4a8(a.to(dev), w.to(dev), s_w.to(dev), s_a.to(dev), bias=bias.to(dev), out_dtype=out_dtype)
    out = out.float().cpu()
    rows = torch.tensor(sorted({0, 1, 127, 128, 143, 144, 159, 160, 255, 256, 287, 288, 319, 320, 2 * 288 + 77,
                                M // 2, (M - 1) // 288 * 288, (M - 1) // 256 * 256, (M - 1) // 320 * 320,
                                M - 2, M - 1}))
    fb = math.gcd(gs, 128)
    acc = oracle.gemm_acc(a[rows].numpy(), oracle.unpack_int4(w.numpy(), K), K // fb)
    sw = np.repeat(s_w.numpy(), gs // fb, axis=1)
    ref = torch.from_numpy(oracle.epilogue(acc, s_a[rows].numpy(), sw, bias.float().numpy(), DT[out_dtype]))
    assert torch.equal(out[rows], ref)


# 256-, 288- and 320-row tiles (4096, 4608, 5120 rows), ragged in M and N; one
# and nine 128-K stages (the int8-weight loop alternates two fragment sets by
# stage and finishes the last stage's deferred block row after the loop)
ROW_BIG_CASES = [(4096, 3072, 1024), (4608, 3072, 1024), (5120, 3072, 1024), (4600, 3064, 1024),
                 (5100, 3064, 1024), (4608, 3072, 128), (4096, 3072, 1152)]


@pytest.mark.parametrize("int4", [False, True])
@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,N,K", ROW_BIG_CASES)
def test_per_row_big_tile_sampled_rows(rt, oracle, dev, out_dtype, M, N, K, int4):
    """Per-row W8A8 and per-row W4A8 on the big tiles (int32 sums over all of
    K, one scale per column): every column of sampled rows (first and last
    rows of tiles and wave rows, the partial last tile row) bit-exact against
    the oracle's accumulators and epilogue."""
    a = _int8((M, K), 71, -127, 128)
    if int4:
        w = torch.randint(0, 256, (N, K // 2), generator=_gen(72), dtype=torch.uint8)
        wq = oracle.unpack_int4(w.numpy(), K)
        s_w = (torch.rand(N, 1, generator=_gen(74)) * 2e-2 + 1e-3).to(torch.float16).float()
    else:
        w = _int8((N, K), 72, -127, 128)
        wq = w.numpy()
        s_w = (torch.rand(N, generator=_gen(74)) * 2e-3 + 1e-4).to(torch.float16).float()
    s_a = torch.rand(M, generator=_gen(73)) * 0.05 + 1e-3
    bias = torch.randn(N, generator=_gen(75)).to(out_dtype)
    assert rt.lib().ic_gemm_splitk_bytes(M, N, K, 1, int(int4)) == 0
    if int4:
        out = rt.gemm_w4a8(a.to(dev), w.to(dev), s_w.to(dev), s_a.to(dev), bias=bias.to(dev), out_dtype=out_dtype)
    else:
        out = rt.fused_int8_gemm_dequant(a.to(dev), w.to(dev), s_w.to(dev), s_a.to(dev), bias=bias.to(dev),
                                         out_dtype=out_dtype)
    out = out.float().cpu()
    rows = torch.tensor(sorted({0, 1, 127, 128, 143, 144, 159, 160, 255, 256, 287, 288, 319, 320, 2 * 288 + 77,
                                M // 2, (M - 1) // 288 * 288, (M - 1) // 256 * 256, (M - 1) // 320 * 320,
                                M - 2, M - 1}))
    acc = oracle.gemm_acc(a[rows].numpy(), wq)
    ref = torch.from_numpy(oracle.epilogue(acc, s_a[rows].numpy(), s_w.numpy(), bias.float().numpy(),
                                           DT[out_dtype]))
    assert torch.equal(out[rows], ref)


# ------------------------------------------------------------------ group sizes other than 128
@pytest.mark.parametrize("gs", [256, 512, 64, 192, 32, 96])
@pytest.mark.parametrize("M,N,K", [(300, 384, 2048), (64, 3072, 4096), (4608, 3072, 1024), (600, 1000, 1536),
                                   (5, 1000, 1536)])
def test_w4a8_group_sizes(rt, oracle, dev, gs, M, N, K):
    """Group sizes other than 128 run the MFMA kernels: multiples of 128
    (tiled and split-K) fold each 128-column stage, odd multiples of 64 (the
    288 x 192 kernel's 64-block mode) each 64-K step, odd multiples of 32
    (its 32-column mode) each 32-column half step, with the scale of the
    step's group.  Bit-exact against the oracle's epilogue over accumulators
    of gcd(group, 128) columns with the scales repeated."""
    if K % gs:
        pytest.skip("K not a multiple of the group size")
    G = K // gs
    fb = math.gcd(gs, 128)
    a = _int8((M, K), 81, -127, 128)
    w = torch.randint(0, 256, (N, K // 2), generator=_gen(82), dtype=torch.uint8)
    s_a = torch.rand(M, generator=_gen(83)) * 0.05 + 1e-3
    s_w = (torch.rand(N, G, generator=_gen(84)) * 2e-2 + 1e-3).to(torch.float16).float()
    bias = torch.randn(N, generator=_gen(85)).to(torch.bfloat16)
    out = rt.gemm_w4a8(a.to(dev), w.to(dev), s_w.to(dev), s_a.to(dev), bias=bias.to(dev), out_dtype=torch.bfloat16)
    out = out.float().cpu()
    wq = oracle.unpack_int4(w.numpy(), K)
    rows = torch.tensor(sorted({0, 1, M // 2, M - 1}))
    acc = oracle.gemm_acc(a[rows].numpy(), wq, K // fb)
    sw = np.repeat(s_w.numpy(), gs // fb, axis=1)
    ref = torch.from_numpy(oracle.epilogue(acc, s_a[rows].numpy(), sw, bias.float().numpy(), 1))
    split = rt.lib().ic_gemm_splitk_bytes(M, N, K, G, 1) > 0
    if not split:
        assert torch.equal(out[rows], ref)
    else:  # slices of the fold added in slice order (bounded in test_splitk_grouped_w4a8)
        assert _cos(out[rows], ref) >= 0.99999
        assert torch.allclose(out[rows], ref, rtol=1e-2, atol=1e-2 * ref.abs().max().item())


def test_w4a8_huge_row_stride(rt, oracle, dev):
    """An activation view whose row stride times the tile's 320 rows passes
    2^31 bytes runs the scalar kernel (the tile kernels form row offsets in
    32 bits): correct outputs, no out-of-range DMA."""
    M, N, K, ld = 400, 64, 256, 6_800_000
    big = torch.randint(-127, 128, (M, ld), dtype=torch.int8, device=dev)
    xa = big[:, :K]
    assert xa.stride(0) * 320 >= 2 ** 31
    w = torch.randint(0, 256, (N, K // 2), generator=_gen(97), dtype=torch.uint8)
    s_a = torch.rand(M, generator=_gen(98)) * 0.05 + 1e-3
    s_w = (torch.rand(N, 2, generator=_gen(99)) * 2e-2 + 1e-3).to(torch.float16).float()
    out = rt.gemm_w4a8(xa, w.to(dev), s_w.to(dev), s_a.to(dev), out_dtype=torch.bfloat16).float().cpu()
    rows = [0, 1, 200, 319, 320, 399]
    a = xa[rows].cpu().numpy()
    del big, xa
    acc = oracle.gemm_acc(a, oracle.unpack_int4(w.numpy(), K), 2)
    ref = oracle.epilogue(acc, s_a[rows].numpy(), s_w.numpy(), None, 1)
    assert np.array_equal(out[rows].numpy(), ref)


@pytest.mark.parametrize("gs", [256, 64, 96])
def test_w4a8_scalar_kernel_fold_blocks(rt, oracle, dev, gs):
    """Operands the MFMA tiles cannot take (a 1-byte offset activation view)
    run the scalar kernel, which folds per gcd(group, 128) columns like the
    MFMA kernels: bit-exact against the oracle's blocked epilogue."""
    M, N, K = 40, 200, 768
    G = K // gs
    fb = math.gcd(gs, 128)
    base = _int8((M, K + 1), 86, -127, 128)
    a = base[:, 1:]
    w = torch.randint(0, 256, (N, K // 2), generator=_gen(87), dtype=torch.uint8)
    s_a = torch.rand(M, generator=_gen(88)) * 0.05 + 1e-3
    s_w = (torch.rand(N, G, generator=_gen(89)) * 2e-2 + 1e-3).to(torch.float16).float()
    xa = base.to(dev)[:, 1:]
    assert xa.data_ptr() % 16 != 0
    out = rt.gemm_w4a8(xa, w.to(dev), s_w.to(dev), s_a.to(dev), out_dtype=torch.float32).cpu()
    acc = oracle.gemm_acc(np.ascontiguousarray(a.numpy()), oracle.unpack_int4(w.numpy(), K), K // fb)
    ref = oracle.epilogue(acc, s_a.numpy(), np.repeat(s_w.numpy(), gs // fb, axis=1), None, 2)
    assert np.array_equal(out.numpy(), ref)


@pytest.mark.parametrize("G", [48, 12, 96, 32])  # group sizes 64, 256, 32 and 96 at K = 3072
@pytest.mark.parametrize("M", [200, 100])  # 256 x 256 and 128 x 256 tiles
def test_w4a16_group_sizes(rt, oracle, dev, G, M):
    N, K = 256, 3072
    x = _acts(M, K, torch.bfloat16, seed=86)
    packed = torch.randint(0, 256, (N, K // 2), generator=_gen(87), dtype=torch.uint8)
    s_w = (torch.rand(N, G, generator=_gen(88)) * 2e-2 + 1e-3).to(torch.float16).float()
    out = rt.gemm_w4a16(x.to(dev), packed.to(dev), s_w.to(dev)).float().cpu()
    w = torch.from_numpy(oracle.dequant_w4a16(packed.numpy(), s_w.numpy(), K, 1))
    ref = x.float() @ w.t()
    assert torch.allclose(out, ref, rtol=2e-2, atol=2e-2 * ref.abs().max().item() * 1e-2)
    assert _cos(out, ref) >= 0.9999


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("K,G", [(8192, 64), (8256, 129), (12288, 96)])  # 128, 129 and 192 stages of 64 K
def test_w4a16_long_k_three_slot_ring(rt, oracle, dev, dtype, K, G):
    """Long K on the big-tile W4A16 modes: K = 8192 with one DMA stage in
    flight, K > 8192 with two (per-wave vmcnt counts at each stage top, an odd
    and an even stage count): within fp32-accumulation tolerance of the
    dequantized-weight product, and one-hot rows return the dequantized
    weights bit for bit."""
    print(f"[w4a16 long K] K={K} G={G} {dtype}", flush=True)
    M, N = 300, 200
    x = _acts(M, K, dtype, seed=130)
    packed = torch.randint(0, 256, (N, K // 2), generator=_gen(131), dtype=torch.uint8)
    s_w = (torch.rand(N, G, generator=_gen(132)) * 2e-2 + 1e-3).to(torch.float16).float()
    bias = torch.randn(N, generator=_gen(133)).to(dtype)
    out = rt.gemm_w4a16(x.to(dev), packed.to(dev), s_w.to(dev), bias=bias.to(dev)).float().cpu()
    w = torch.from_numpy(oracle.dequant_w4a16(packed.numpy(), s_w.numpy(), K, DT[dtype]))
    ref = x.float() @ w.t() + bias.float()
    tol = 1e-2 if dtype == torch.float16 else 2e-2
    assert torch.allclose(out, ref, rtol=tol, atol=tol * ref.abs().max().item() * 1e-2)
    assert _cos(out, ref) >= 0.9999
    hot = torch.zeros(M, K, dtype=dtype)
    cols = (torch.arange(M) * 27) % K  # spread over the stages
    hot[torch.arange(M), cols] = 1
    out1 = rt.gemm_w4a16(hot.to(dev), packed.to(dev), s_w.to(dev)).float().cpu().numpy()
    assert np.array_equal(out1, w.numpy()[:, cols.numpy()].T)


@pytest.mark.parametrize("K,G", [(64, 1), (128, 2), (192, 3)])  # one, two and three 64-K stages
def test_w4a16_big_tiles_short_k(rt, oracle, dev, K, G):
    """The big-tile W4A16 mode with one to three stages (prologue, first and
    last stage at once): within fp32-accumulation tolerance of the
    dequantized-weight product."""
    M, N = 200, 64
    x = _acts(M, K, torch.float16, seed=140 + K)
    packed = torch.randint(0, 256, (N, K // 2), generator=_gen(141), dtype=torch.uint8)
    s_w = (torch.rand(N, G, generator=_gen(142)) * 2e-2 + 1e-3).to(torch.float16).float()
    out = rt.gemm_w4a16(x.to(dev), packed.to(dev), s_w.to(dev)).float().cpu()
    w = torch.from_numpy(oracle.dequant_w4a16(packed.numpy(), s_w.numpy(), K, DT[torch.float16]))
    ref = x.float() @ w.t()
    assert torch.allclose(out, ref, rtol=1e-2, atol=1e-2 * ref.abs().max().item() * 1e-2)
    assert _cos(out, ref) >= 0.9999


@pytest.mark.parametrize("M,N,K,G,dtype,bias", [
    (300, 200, 512, 4, torch.float16, True),        # ragged M and N, two row tiles
    (1000, 1048, 1024, 8, torch.bfloat16, False),   # N past a 192-column tile
    (260, 64, 8256, 129, torch.float16, True),      # K > 8192: the three-slot ring; 64-column groups
    (4096, 384, 576, 1, torch.bfloat16, True),      # per-row scales, 256-row tiles
])
def test_w4a16_staged_equals_plain(rt, dev, M, N, K, G, dtype, bias):
    """The staged operand layout (w4a16_stage_layout + gemm_w4a16_staged): the
    copy is the stated permutation of the packed weights and scales, and the
    GEMM's outputs equal gemm_w4a16's bit for bit (the same big-tile kernel
    and summation order, other DMA addresses)."""
    print(f"[w4a16 staged] M={M} N={N} K={K} G={G} {dtype} bias={bias}", flush=True)
    assert rt.w4a16_staged_pays(M, N, K, G)
    x = _acts(M, K, dtype, seed=150).to(dev)
    packed = torch.randint(0, 256, (N, K // 2), generator=_gen(151), dtype=torch.uint8).to(dev)
    s_w = (torch.rand(N, G, generator=_gen(152)) * 2e-2 + 1e-3).to(dev)
    b = torch.randn(N, generator=_gen(153)).to(dtype).to(dev) if bias else None
    ws, ss = rt.w4a16_stage_layout(packed, s_w)
    assert ws.shape == (K // 64, N, 32) and ss.shape == (G, N)
    assert torch.equal(ws.permute(1, 0, 2).reshape(N, K // 2), packed)
    assert torch.equal(ss, s_w.t())
    ref = rt.gemm_w4a16(x, packed, s_w, bias=b)
    out = rt.gemm_w4a16_staged(x, ws, ss, bias=b)
    assert torch.equal(out, ref)


@pytest.mark.parametrize("K,G", [(128, 1), (192, 3), (8320, 65)])  # two-slot ring; three-slot past K = 8192
def test_w4a16_wide_tiles_one_hot(rt, oracle, dev, K, G):
    """The 256-column W4A16 tiles, which the host picks at C2's row and column
    counts (3 rounds of 288 x 256 against 4 of 288 x 192), on both rings and
    both operand layouts: one-hot activation rows return the dequantized
    weights bit for bit at every one of the 4608 x 12288 outputs."""
    M, N = 4608, 12288
    print(f"[w4a16 wide] M={M} N={N} K={K} G={G}", flush=True)
    cols = ((torch.arange(M) * 27 + 5) % K).numpy()
    hot = torch.zeros(M, K, dtype=torch.float16)
    hot[torch.arange(M), torch.from_numpy(cols)] = 1
    packed = torch.randint(0, 256, (N, K // 2), generator=_gen(160), dtype=torch.uint8)
    s_w = (torch.rand(N, G, generator=_gen(161)) * 2e-2 + 1e-3).to(torch.float16).float()
    # expected out[m, n] = dequant(w[n, cols[m]]): the selected nibbles packed
    # as a K = M matrix with one scale per column, through the oracle
    nib = (packed.numpy()[:, cols // 2] >> (4 * (cols & 1)).astype(np.uint8)) & 0xF
    sub = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    s_sub = np.ascontiguousarray(s_w.numpy()[:, cols // (K // G)])
    want = oracle.dequant_w4a16(sub, s_sub, M, DT[torch.float16]).T
    out = rt.gemm_w4a16(hot.to(dev), packed.to(dev), s_w.to(dev))
    assert np.array_equal(out.float().cpu().numpy(), want)
    ws, ss = rt.w4a16_stage_layout(packed.to(dev), s_w.to(dev))
    assert torch.equal(rt.gemm_w4a16_staged(hot.to(dev), ws, ss), out)


def test_w4a16_staged_rule_and_rejection(rt, dev):
    """w4a16_staged_pays admits the big-tile shapes only, and the entry point
    rejects the rest with an error instead of running another kernel."""
    assert rt.w4a16_staged_pays(4608, 12288, 3072, 24)
    assert not rt.w4a16_staged_pays(128, 12288, 3072, 24)   # the GEMV / small-tile range
    assert not rt.w4a16_staged_pays(4608, 12288, 3040, 95)  # K not a multiple of 64
    assert not rt.w4a16_staged_pays(4608, 12288, 3072, 96)  # 32-column groups
    assert not rt.w4a16_staged_pays(4608, 12284, 3072, 24)  # N not a multiple of 8
    packed = torch.randint(0, 256, (64, 64), dtype=torch.uint8, device=dev)
    ws, ss = rt.w4a16_stage_layout(packed, torch.ones(64, 1, device=dev))
    with pytest.raises(RuntimeError):
        rt.gemm_w4a16_staged(torch.zeros(100, 128, dtype=torch.float16, device=dev), ws, ss)


def test_w4a16_row_stride_past_the_384_row_tile(rt, oracle, dev):
    """An activation row stride whose 384-row tile offsets pass 2^31 bytes
    (while 256 rows stay below) runs the scalar W4A16 kernel: correct
    outputs, no out-of-range DMA."""
    M, N, K, ld = 400, 64, 256, 3_500_000  # 7.0 MB rows: 256 * 7.0 MB < 2^31 <= 384 * 7.0 MB
    assert 256 * ld * 2 < 2 ** 31 <= 384 * ld * 2
    big = torch.zeros(M, ld, dtype=torch.bfloat16, device=dev)
    x = _acts(M, K, torch.bfloat16, seed=101)
    big[:, :K] = x.to(dev)
    xa = big[:, :K]
    packed = torch.randint(0, 256, (N, K // 2), generator=_gen(102), dtype=torch.uint8)
    s_w = (torch.rand(N, 2, generator=_gen(103)) * 2e-2 + 1e-3).to(torch.float16).float()
    out = rt.gemm_w4a16(xa, packed.to(dev), s_w.to(dev)).float().cpu()
    del big, xa
    w = torch.from_numpy(oracle.dequant_w4a16(packed.numpy(), s_w.numpy(), K, 1))
    ref = x.float() @ w.t()
    assert _cos(out, ref) >= 0.9999
    assert torch.allclose(out, ref, rtol=2e-2, atol=2e-2 * ref.abs().max().item() * 1e-2)
