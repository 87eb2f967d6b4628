"""Chained MLP epilogue: ic_gemm_w8a8_chain / ic_gemm_w4a8_chain through
_hip_runtime.gemm_chain.

The chained GEMM finishes each output as the plain GEMM does with the same
activation (fused_int8_gemm_dequant / gemm_w4a8), then divides its tile by the
next linear's SmoothRot factors and rotates it in R-blocks, the first half of
_prep_activation (_ops.py:337-365).  Everything here is integer or exactly
rounded arithmetic, so the checks are bit-exact:
  * y equals the plain GEMM's output h passed through prepare_activation
    (the prep kernel, itself bit-exact against the oracle in
    test_gpu_kernels.py), at every routing of the tile (partial M and N
    tiles, R = 16 / 64 / 256, with and without factors, fp16 and bf16, W8A8,
    per-row and grouped W4A8);
  * sampled rows of y equal oracle.prepare of the same rows of h;
  * the down-projection's codes and scales from rotate_quantize(y, rot_size
    0, w_in, perm) equal rotate_quantize(h, R, w_in, factors, perm);
  * at the Flux MLP-up shape (M 4608, K 3072, N 12288, W4A8 g128, R 256,
    bf16, GELU-tanh), the whole output against the two-kernel path.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

DT = {torch.float16: 0, torch.bfloat16: 1}
ACT_GELU_TANH = 3


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _operands(kind, M, K, N, seed, act_scale=1.0):
    g = _gen(seed)
    xq = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    s_a = (torch.rand(M, generator=g) * 0.02 + 0.005) * act_scale
    bias = torch.randn(N, generator=g) * 0.1
    if kind == "w8a8":
        w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
        s_w = torch.rand(N, generator=g) * 2e-3 + 1e-4
    else:
        w = torch.randint(0, 256, (N, K // 2), generator=g, dtype=torch.uint8)
        G = K // 128 if kind == "w4a8_g128" else 1
        s_w = torch.rand(N, G, generator=g) * 0.02 + 1e-3
    return xq, w, s_w, s_a, bias


def _plain(rt, kind, xq, w, s_w, s_a, bias, dtype, act):
    if kind == "w8a8":
        return rt.fused_int8_gemm_dequant(xq, w, s_w, s_a, bias=bias, out_dtype=dtype, activation=act)
    return rt.gemm_w4a8(xq, w, s_w, s_a, bias=bias, out_dtype=dtype, activation=act)


def _bits(t):
    return t.view(torch.int16).cpu()


CASES = [  # (kind, M, K, N, R, smoothrot)
    ("w4a8_g128", 300, 384, 768, 256, True),
    ("w4a8_g128", 300, 384, 768, 64, True),
    ("w4a8_g128", 130, 256, 320, 64, True),   # last N tile holds one 64-block
    ("w4a8_g128", 64, 512, 512, 16, False),
    ("w4a8_row", 200, 384, 768, 256, True),
    ("w4a8_row", 129, 256, 272, 16, True),    # last N tile holds one 16-block
    ("w8a8", 300, 384, 768, 256, True),
    ("w8a8", 77, 256, 512, 64, False),
    ("w8a8", 256, 128, 256, 16, True),
]


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("case", CASES)
def test_chain_equals_gemm_then_prep(rt, oracle, dev, dtype, case):
    kind, M, K, N, R, use_sr = case
    xq, w, s_w, s_a, bias = _operands(kind, M, K, N, seed=M + N + R)
    g = _gen(N + 1)
    sr = torch.exp(torch.randn(N, generator=g) * 0.5) if use_sr else None
    srf = rt.prepare_factors(sr.to(dev), dtype) if use_sr else None
    args = [t.to(dev) for t in (xq, w, s_w, s_a, bias)]
    h = _plain(rt, kind, *args, dtype, ACT_GELU_TANH)
    y_ref = rt.prepare_activation(h, rot_size=R, smoothrot=srf)
    y = rt.gemm_chain(*args[:4], rot_size=R, smoothrot=srf, bias=args[4], out_dtype=dtype,
                      activation=ACT_GELU_TANH)
    torch.cuda.synchronize()
    print(f"chain {kind} {dtype} M={M} K={K} N={N} R={R} sr={use_sr}", flush=True)
    assert y.shape == (M, N) and y.dtype == dtype
    assert torch.equal(_bits(y), _bits(y_ref))
    rows = sorted({0, 1, M // 2, 127 % M, 128 % M, M - 1})
    y_or = oracle.prepare(h[rows].float().cpu().numpy(), DT[dtype], smoothrot=sr, rot_size=R)
    assert np.array_equal(y[rows].float().cpu().numpy(), y_or)
    # the down-projection's codes: pad to K_w, perm, whole-row scale
    K_w = N + 64
    perm = rt.prepare_perm(torch.randperm(K_w, generator=g).to(dev), K_w)
    q_ref, s_ref = rt.rotate_quantize(h, rot_size=R, w_in=K_w, smoothrot=srf, perm=perm)
    q, s = rt.rotate_quantize(y, rot_size=0, w_in=K_w, perm=perm)
    assert torch.equal(s.cpu(), s_ref.cpu())
    assert torch.equal(q.cpu(), q_ref.cpu())


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["w4a8_g128", "w8a8"])
def test_chain_no_activation_and_wide_bf16_blocks(rt, oracle, dev, kind):
    """activation 0 (the plain dequant, bit-exact against the oracle's
    epilogue), and bf16 rows whose GELU outputs span far more binades than
    the exact fp64 rotation allows (the flush rule of the prep kernels)."""
    M, K, N, R = 160, 256, 512, 256
    xq, w, s_w, s_a, bias = _operands(kind, M, K, N, seed=11)
    args = [t.to(dev) for t in (xq, w, s_w, s_a, bias)]
    h = _plain(rt, kind, *args, torch.bfloat16, 0)
    y = rt.gemm_chain(*args[:4], rot_size=R, bias=args[4], out_dtype=torch.bfloat16, activation=0)
    assert torch.equal(_bits(y), _bits(rt.prepare_activation(h, rot_size=R)))
    # pre-activations of several hundred: GELU-tanh leaves values down to the
    # f32 subnormals beside values of several hundred in the same block
    xq, w, s_w, s_a, bias = _operands(kind, M, K, N, seed=12, act_scale=40.0)
    args = [t.to(dev) for t in (xq, w, s_w, s_a, bias)]
    h = _plain(rt, kind, *args, torch.bfloat16, ACT_GELU_TANH)
    hf = h.float().abs()
    assert (hf[hf > 0].min() < 1e-30) and hf.max() > 10.0
    y = rt.gemm_chain(*args[:4], rot_size=R, bias=args[4], out_dtype=torch.bfloat16, activation=ACT_GELU_TANH)
    assert torch.equal(_bits(y), _bits(rt.prepare_activation(h, rot_size=R)))
    rows = [0, 5, M - 1]
    y_or = oracle.prepare(h[rows].float().cpu().numpy(), DT[torch.bfloat16], rot_size=R)
    assert np.array_equal(y[rows].float().cpu().numpy(), y_or)


@pytest.mark.gpu
def test_chain_flux_mlp_up_full_size(rt, dev):
    """Flux MLP up-projection (3072 -> 12288, M 4608, W4A8 g128, bf16,
    GELU-tanh) chained into the down-projection's R = 256 SmoothRot prep: the
    whole output and the down-projection's codes against the two-kernel path."""
    M, K, N, R = 4608, 3072, 12288, 256
    xq, w, s_w, s_a, bias = _operands("w4a8_g128", M, K, N, seed=5)
    g = _gen(6)
    srf = rt.prepare_factors(torch.exp(torch.randn(N, generator=g) * 0.5).to(dev), torch.bfloat16)
    args = [t.to(dev) for t in (xq, w, s_w, s_a, bias)]
    h = _plain(rt, "w4a8_g128", *args, torch.bfloat16, ACT_GELU_TANH)
    y = rt.gemm_chain(*args[:4], rot_size=R, smoothrot=srf, bias=args[4], out_dtype=torch.bfloat16,
                      activation=ACT_GELU_TANH)
    y_ref = rt.prepare_activation(h, rot_size=R, smoothrot=srf)
    assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16))
    perm = rt.prepare_perm(torch.randperm(N, generator=g).to(dev), N)
    q_ref, s_ref = rt.rotate_quantize(h, rot_size=R, w_in=N, smoothrot=srf, perm=perm)
    q, s = rt.rotate_quantize(y, rot_size=0, w_in=N, perm=perm)
    assert torch.equal(s, s_ref) and torch.equal(q, q_ref)


def test_chain_rejects_before_launch(rt):
    """Argument errors are reported before anything touches a GPU."""
    with pytest.raises(ValueError):
        rt.gemm_chain(torch.zeros(4, 128, dtype=torch.int8), torch.zeros(256, 128, dtype=torch.int8),
                      torch.ones(256), torch.ones(4), rot_size=256)  # CPU tensors
    lib = rt.lib()
    fake = 0x1000
    # rot_size outside 16 / 64 / 256
    assert lib.ic_gemm_w8a8_chain(fake, 1, 128, 128, fake, 1024, 128, fake, fake, None, 0, 0, None, None,
                                  1024, fake, 0, 1024, None) == 2
    # f32 output
    assert lib.ic_gemm_w8a8_chain(fake, 1, 128, 128, fake, 256, 128, fake, fake, None, 0, 0, None, None,
                                  256, fake, 2, 256, None) == 1
    # N not a multiple of rot_size
    assert lib.ic_gemm_w4a8_chain(fake, 1, 128, 128, fake, 100, 64, fake, 1, fake, None, 0, 0, None, None,
                                  64, fake, 0, 128, None) == 1
    # factors without their reciprocals
    assert lib.ic_gemm_w4a8_chain(fake, 1, 128, 128, fake, 256, 64, fake, 1, fake, None, 0, 0, None, fake,
                                  256, fake, 0, 256, None) == 1
    # group size 64
    assert lib.ic_gemm_w4a8_chain(fake, 1, 128, 128, fake, 256, 64, fake, 2, fake, None, 0, 0, None, None,
                                  256, fake, 0, 256, None) == 2
