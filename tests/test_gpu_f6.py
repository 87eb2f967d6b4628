"""GPU parity of the grouped W4A8 GEMM on e3m2 operands (ic_gemm_w4a8_f6).

* The format conversions, decoded on the CPU from the format definition
  (tests/_f6.py): every activation code x equals 16 h + l with h in [-8, 8],
  l in [-8, 7]; every weight equals the two's-complement nibble.
* The GEMM's outputs equal the oracle's epilogue formula over exact int32
  group sums and, where ic_gemm_w4a8 runs unsplit (its split-K launches add
  slice partials in a different order), its outputs bit for bit, including
  operands at the extremes, where each 128-column group sum reaches
  128 * 128 * 8 = 2^17 and the f8f6f4 MFMA must still sum exactly.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import _f6

pytestmark = pytest.mark.gpu


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def test_f6_formats_decode(rt, oracle, dev):
    M, K, N = 37, 384, 45
    x = torch.randint(-128, 128, (M, K), generator=_gen(1), dtype=torch.int8)
    x[0, :256] = torch.arange(-128, 128, dtype=torch.int16).to(torch.int8)  # every code
    w = torch.randint(0, 256, (N, K // 2), generator=_gen(2), dtype=torch.uint8)
    w[0, :128] = torch.arange(0, 256, 2, dtype=torch.int16).to(torch.uint8)
    a6 = rt.f6_split_activations(x.to(dev)).cpu().numpy()
    w6 = rt.f6_repack_weights(w.to(dev), K).cpu().numpy()
    h, l = _f6.decode_a6(a6, M, K)
    assert np.array_equal(16 * h + l, x.numpy().astype(np.float64))
    assert h.min() >= -8 and h.max() <= 8 and l.min() >= -8 and l.max() <= 7
    assert np.array_equal(_f6.decode_w6(w6, N, K), oracle.unpack_int4(w.numpy(), K).astype(np.float64))


SHAPES = [
    (4608, 3072, 12288, 96),   # C3 (288-row tiles)
    (4096, 3072, 3072, 24),    # Flux image stream (256-row tiles)
    (640, 384, 1024, 4),       # groups of 256 columns
    (300, 200, 1024, 8),       # partial row and column tiles
    (33, 104, 256, 2),
]


@pytest.mark.parametrize("M,N,K,G", SHAPES)
@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16])
def test_f6_gemm_matches_int8_kernel(rt, oracle, dev, M, N, K, G, out_dtype):
    x = torch.randint(-128, 128, (M, K), generator=_gen(M + K), dtype=torch.int8)
    w = torch.randint(0, 256, (N, K // 2), generator=_gen(N), dtype=torch.uint8)
    s_w = (torch.rand(N, G, generator=_gen(3)) * 1.9e-2 + 1e-3).to(torch.float16).float()
    s_a = torch.rand(M, generator=_gen(4)) * 0.05 + 1e-3
    bias = torch.randn(N, generator=_gen(5)).to(out_dtype) if M % 2 == 0 else None
    xd, wd, swd, sad = x.to(dev), w.to(dev), s_w.to(dev), s_a.to(dev)
    bd = None if bias is None else bias.to(dev)
    ref = rt.gemm_w4a8(xd, wd, swd, sad, bias=bd, out_dtype=out_dtype)
    out = rt.gemm_w4a8_f6(rt.f6_split_activations(xd), M, K, rt.f6_repack_weights(wd, K), N, swd, sad, bias=bd,
                          out_dtype=out_dtype)
    if rt.lib().ic_gemm_splitk_bytes(M, N, K, G, 1) == 0:
        # the int8 route without a K split folds in the same order
        assert torch.equal(out, ref)
    if M * N * K <= 1 << 28:
        acc = oracle.gemm_acc(x.numpy(), oracle.unpack_int4(w.numpy(), K), K // 128)
        sw128 = np.repeat(s_w.numpy(), (K // G) // 128, axis=1)
        exp = oracle.epilogue(acc, s_a.numpy(), sw128, None if bias is None else bias.float().numpy(),
                              0 if out_dtype == torch.float16 else 1)
        assert np.array_equal(out.float().cpu().numpy(), exp)


@pytest.mark.parametrize("xv,nib", [(-128, 8), (127, 8), (-128, 7), (127, 7)])
def test_f6_gemm_extreme_group_sums(rt, oracle, dev, xv, nib):
    M, N, K = 64, 64, 512
    x = torch.full((M, K), xv, dtype=torch.int8)
    x[1::2, 1::3] = -x[1::2, 1::3] if xv != -128 else 127  # cancellation in alternate rows
    w = torch.full((N, K // 2), nib | (nib << 4), dtype=torch.uint8)
    s_w = torch.full((N, K // 128), 2.0 ** -20)
    s_a = torch.ones(M)
    out = rt.gemm_w4a8_f6(rt.f6_split_activations(x.to(dev)), M, K, rt.f6_repack_weights(w.to(dev), K), N,
                          s_w.to(dev), s_a.to(dev), out_dtype=torch.float16)
    acc = oracle.gemm_acc(x.numpy(), oracle.unpack_int4(w.numpy(), K), K // 128)
    if (xv, nib) == (-128, 8):
        assert np.abs(acc).max() == 128 * 128 * 8
    exp = oracle.epilogue(acc, s_a.numpy(), s_w.numpy(), None, 0)
    assert np.array_equal(out.float().cpu().numpy(), exp)


def test_f6_rejects_unsupported(rt, dev):
    x = torch.zeros(16, 192, dtype=torch.int8, device=dev)
    with pytest.raises(ValueError):
        rt.f6_split_activations(x)
    a6 = torch.zeros(rt.lib().ic_f6_activation_bytes(16, 256), dtype=torch.uint8, device=dev)
    w6 = torch.zeros(rt.lib().ic_f6_weight_bytes(16, 256), dtype=torch.uint8, device=dev)
    with pytest.raises(RuntimeError):  # one group: the per-row formula is ic_gemm_w4a8's
        rt.gemm_w4a8_f6(a6, 16, 256, w6, 16, torch.ones(16, 1, device=dev), torch.ones(16, device=dev))
