"""GPU parity of the small-batch (M <= 16) GEMV kernels.

W8A8 / W4A8 outputs must be bit-identical to the oracle's epilogue formula
(exact int32 block sums, per-group fold in group order), both through the
explicit ic_gemv_* entry points and through the GEMM entry points, which
route M <= 16 to them.  W4A16 is checked against the fp32 dequant -> F.linear
reference (rtol 1e-2, cosine >= 0.9999).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DT = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _int8(shape, seed, lo=-128, hi=128):
    return torch.randint(lo, hi, shape, generator=_gen(seed), dtype=torch.int8)


def _cos(a, b):
    a = a.reshape(-1).double()
    b = b.reshape(-1).double()
    return float((a @ b) / (a.norm() * b.norm()))


@pytest.mark.parametrize("M", [1, 2, 5, 16])
@pytest.mark.parametrize("N,K", [(18432 // 8, 3072), (200, 1024), (33, 128)])
@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("via", ["gemv", "gemm"])
def test_gemv_w8a8_bit_exact(rt, oracle, dev, M, N, K, out_dtype, via):
    a = _int8((M, K), 1 + M)
    w = _int8((N, K), 2, -127, 128)
    s_a = torch.rand(M, generator=_gen(3)) * 0.05 + 1e-3
    s_w = (torch.rand(N, generator=_gen(4)) * 2e-3 + 1e-4).to(torch.float16).float()
    bias = torch.randn(N, generator=_gen(5)).to(out_dtype) if M % 2 else None
    args = (a.to(dev), w.to(dev), s_w.to(dev), s_a.to(dev))
    b_dev = None if bias is None else bias.to(dev)
    if via == "gemv":
        out = rt.gemv(args[0], args[1], args[2], args[3], bias=b_dev, out_dtype=out_dtype, kind="w8a8")
    else:
        out = rt.fused_int8_gemm_dequant(*args, bias=b_dev, out_dtype=out_dtype)
    acc = oracle.gemm_acc(a.numpy(), w.numpy())
    ref = oracle.epilogue(acc, s_a.numpy(), s_w.numpy(), None if bias is None else bias.float().numpy(),
                          DT[out_dtype])
    assert np.array_equal(out.float().cpu().numpy(), ref)


@pytest.mark.parametrize("M", [1, 2, 7, 16])
@pytest.mark.parametrize("N,K", [(18432 // 8, 3072), (136, 1536), (20, 256)])
@pytest.mark.parametrize("grouped", [False, True])
@pytest.mark.parametrize("via", ["gemv", "gemm"])
def test_gemv_w4a8_bit_exact(rt, oracle, dev, M, N, K, grouped, via):
    G = K // 128 if grouped else 1
    out_dtype = torch.bfloat16 if grouped else torch.float16
    a = _int8((M, K), 11 + M)
    packed = torch.randint(0, 256, (N, K // 2), generator=_gen(12), dtype=torch.uint8)
    s_a = torch.rand(M, generator=_gen(13)) * 0.05 + 1e-3
    s_w = (torch.rand(N, G, generator=_gen(14)) * 2e-2 + 1e-3).to(torch.float16).float()
    bias = torch.randn(N, generator=_gen(15)).to(out_dtype)
    args = (a.to(dev), packed.to(dev), s_w.to(dev), s_a.to(dev))
    if via == "gemv":
        out = rt.gemv(*args, bias=bias.to(dev), out_dtype=out_dtype, kind="w4a8")
    else:
        out = rt.gemm_w4a8(*args, bias=bias.to(dev), out_dtype=out_dtype)
    acc = oracle.gemm_acc(a.numpy(), oracle.unpack_int4(packed.numpy(), K), G)
    ref = oracle.epilogue(acc, s_a.numpy(), s_w.numpy(), bias.float().numpy(), DT[out_dtype])
    assert np.array_equal(out.float().cpu().numpy(), ref)


@pytest.mark.parametrize("gs", [32, 64, 96, 256, 384])
@pytest.mark.parametrize("M", [1, 5, 16])
@pytest.mark.parametrize("via", ["gemv", "gemm"])
def test_gemv_w4a8_group_sizes(rt, oracle, dev, gs, M, via):
    """Groups other than 128 columns: the GEMV folds per gcd(group, 128)
    columns in K order with each block's group scale, as the GEMM kernels
    do.  Bit-exact against the oracle's blocked epilogue."""
    import math
    N, K = 264, 3072 if gs != 256 else 2048
    G, fb = K // gs, math.gcd(gs, 128)
    a = _int8((M, K), 41 + M)
    packed = torch.randint(0, 256, (N, K // 2), generator=_gen(42), dtype=torch.uint8)
    s_a = torch.rand(M, generator=_gen(43)) * 0.05 + 1e-3
    s_w = (torch.rand(N, G, generator=_gen(44)) * 2e-2 + 1e-3).to(torch.float16).float()
    bias = torch.randn(N, generator=_gen(45)).to(torch.bfloat16)
    args = (a.to(dev), packed.to(dev), s_w.to(dev), s_a.to(dev))
    if via == "gemv":
        out = rt.gemv(*args, bias=bias.to(dev), out_dtype=torch.bfloat16, kind="w4a8")
    else:
        out = rt.gemm_w4a8(*args, bias=bias.to(dev), out_dtype=torch.bfloat16)
    acc = oracle.gemm_acc(a.numpy(), oracle.unpack_int4(packed.numpy(), K), K // fb)
    sw = np.repeat(s_w.numpy(), gs // fb, axis=1)
    ref = oracle.epilogue(acc, s_a.numpy(), sw, bias.float().numpy(), DT[torch.bfloat16])
    assert np.array_equal(out.float().cpu().numpy(), ref)


def test_gemv_group_sums_past_the_lds_take_the_gemm(rt, oracle, dev):
    """M = 16, K = 8192 in groups of 32: the fold sums (256 KB) exceed the
    GEMV's LDS, so the GEMM entry point runs the tiled kernel -- same
    numbers -- and the explicit GEMV refuses."""
    M, N, K, gs = 16, 200, 8192, 32
    G = K // gs
    a = _int8((M, K), 51)
    packed = torch.randint(0, 256, (N, K // 2), generator=_gen(52), dtype=torch.uint8)
    s_a = torch.rand(M, generator=_gen(53)) * 0.05 + 1e-3
    s_w = (torch.rand(N, G, generator=_gen(54)) * 2e-2 + 1e-3).to(torch.float16).float()
    args = (a.to(dev), packed.to(dev), s_w.to(dev), s_a.to(dev))
    with pytest.raises(RuntimeError, match="fit 128 KB"):
        rt.gemv(*args, out_dtype=torch.bfloat16, kind="w4a8")
    out = rt.gemm_w4a8(*args, out_dtype=torch.bfloat16)
    acc = oracle.gemm_acc(a.numpy(), oracle.unpack_int4(packed.numpy(), K), K // gs)
    ref = oracle.epilogue(acc, s_a.numpy(), s_w.numpy(), None, DT[torch.bfloat16])
    assert np.array_equal(out.float().cpu().numpy(), ref)


def test_gemv_matches_tiled_gemm_rows(rt, dev):
    """The same rows computed at M = 16 (GEMV) and inside an M = 300 GEMM agree
    bit for bit.  N = 6144 gives the GEMM enough tiles that it does not split
    K (a grouped split-K sums its slices in another fp32 order)."""
    K, N = 3072, 6144
    assert rt.lib().ic_gemm_splitk_bytes(300, N, K, K // 128, 1) == 0
    a = _int8((300, K), 21).to(dev)
    packed = torch.randint(0, 256, (N, K // 2), generator=_gen(22), dtype=torch.uint8).to(dev)
    s_a = (torch.rand(300, generator=_gen(23)) * 0.05 + 1e-3).to(dev)
    s_w = (torch.rand(N, K // 128, generator=_gen(24)) * 2e-2 + 1e-3).to(torch.float16).float().to(dev)
    big = rt.gemm_w4a8(a, packed, s_w, s_a, out_dtype=torch.float16)
    small = rt.gemm_w4a8(a[:16].contiguous(), packed, s_w, s_a[:16].contiguous(), out_dtype=torch.float16)
    assert torch.equal(big[:16], small)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M", [1, 3, 16])
@pytest.mark.parametrize("G", [1, 24])
def test_gemv_w4a16_vs_fp32(rt, oracle, dev, dtype, M, G):
    N, K = 2304, 3072
    x = torch.randn(M, K, generator=_gen(30 + M)).to(dtype)
    packed = torch.randint(0, 256, (N, K // 2), generator=_gen(31), dtype=torch.uint8)
    s_w = (torch.rand(N, G, generator=_gen(32)) * 2e-2 + 1e-3).to(torch.float16).float()
    bias = torch.randn(N, generator=_gen(33)).to(dtype)
    out_v = rt.gemv(x.to(dev), packed.to(dev), s_w.to(dev), bias=bias.to(dev), kind="w4a16").float().cpu()
    out_g = rt.gemm_w4a16(x.to(dev), packed.to(dev), s_w.to(dev), bias=bias.to(dev)).float().cpu()
    w = torch.from_numpy(oracle.dequant_w4a16(packed.numpy(), s_w.numpy(), K, DT[dtype]))
    ref = x.float() @ w.t() + bias.float()
    tol = 1e-2 if dtype == torch.float16 else 2e-2
    for out in (out_v, out_g):
        assert torch.allclose(out, ref, rtol=tol, atol=tol * ref.abs().max().item() * 1e-2)
        assert _cos(out, ref) >= 0.9999


def test_gemv_argument_errors(rt, dev):
    a = torch.zeros(17, 256, dtype=torch.int8, device=dev)
    w = torch.zeros(32, 256, dtype=torch.int8, device=dev)
    s = torch.ones(32, device=dev)
    with pytest.raises(RuntimeError, match="M=17"):
        rt.gemv(a, w, s, torch.ones(17, device=dev), kind="w8a8")
    with pytest.raises(RuntimeError, match="multiple of 128"):
        rt.gemv(a[:4, :200].contiguous(), w[:, :200].contiguous(), s, torch.ones(4, device=dev), kind="w8a8")
