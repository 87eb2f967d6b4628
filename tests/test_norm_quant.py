"""Norm / softmax fused with per-token INT8 quantization: fused_layernorm_quantize,
fused_rmsnorm_quantize and fused_softmax_quantize (kernels/triton_quantize.py:201-567).

CPU tests pin the oracle's restatement (oracle.normalize_rows / norm_quantize)
against the reference tests' own PyTorch formulas at their own bar (codes within
+-1, tests/test_w8a8_fused_kernels.py:31-57, :73-77 of the reference), against
closed forms, and show a planted mistake fails; they also check the mirror's CPU
branch is the reference CPU branch bit for bit.  GPU tests compare the
ic_norm_quantize kernel with the oracle.  The block-input fusion
ic_norm_rotate_quantize (normalise, round to the dtype, rotate_quantize) is
checked against the oracle's composition of the same steps.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

KINDS = ("layer", "rms", "softmax")
DT = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}
REF_SHAPES = [(1, 64), (4, 256), (16, 1024), (64, 4096)]  # the reference tests' shapes


def _torch_reference(x: torch.Tensor, kind, gamma=None, beta=None, eps=1e-5):
    """f32 PyTorch normalisation + round-half-even quantization, the formula the
    reference tests judge their kernels against."""
    xf = x.float()
    K = xf.shape[-1]
    if kind == "layer":
        y = F.layer_norm(xf, (K,), gamma.float(), beta.float() if beta is not None else None, eps)
    elif kind == "rms":
        y = xf / torch.sqrt(torch.mean(xf * xf, dim=-1, keepdim=True) + eps) * gamma.float()
    else:
        y = F.softmax(xf, dim=-1)
    s = y.abs().amax(dim=-1).clamp(min=1e-8) / 127.0
    q = (y / s.unsqueeze(-1)).round().clamp(-128, 127).to(torch.int8)
    return q, s


def _inputs(M, K, seed, dtype=torch.float32, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(M, K, generator=g) * scale).to(dtype)
    gamma = torch.randn(K, generator=g)
    beta = torch.randn(K, generator=g)
    return x, gamma, beta


def _eps(kind):
    return 1e-5 if kind == "layer" else 1e-6


# ---------------------------------------------------------------- oracle pins (CPU)
@pytest.mark.parametrize("M,K", REF_SHAPES)
@pytest.mark.parametrize("kind", KINDS)
def test_oracle_matches_reference_formula(oracle, M, K, kind):
    x, gamma, beta = _inputs(M, K, 100 + M + K)
    q, s = oracle.norm_quantize(x.numpy(), kind, gamma.numpy(), beta.numpy() if kind == "layer" else None,
                                _eps(kind))
    rq, rs = _torch_reference(x, kind, gamma, beta if kind == "layer" else None, _eps(kind))
    assert np.abs(q.astype(np.int32) - rq.numpy().astype(np.int32)).max() <= 1
    assert np.allclose(s, rs.numpy(), rtol=1e-5, atol=0)


@pytest.mark.parametrize("kind", ("layer", "rms"))
def test_oracle_no_beta_and_unit_gamma_closed_forms(oracle, kind):
    """gamma = 1, beta = None: LayerNorm rows have mean 0 and variance 1 (up to
    eps), RMSNorm rows have mean square 1."""
    x, _, _ = _inputs(8, 2048, 7)
    y = oracle.normalize_rows(x.numpy(), kind, np.ones(2048, np.float32), None, _eps(kind)).astype(np.float64)
    if kind == "layer":
        assert np.abs(y.mean(axis=1)).max() < 1e-5
        assert np.abs(y.var(axis=1) - 1.0).max() < 1e-4
    else:
        assert np.abs((y * y).mean(axis=1) - 1.0).max() < 1e-4


def test_oracle_constant_rows(oracle):
    """Constant rows: LayerNorm gives 0 (scale floor 1e-8/127, codes 0); softmax
    is uniform (every code 127, s = (1/K)/127); RMSNorm gives sign(c) * c/|c|
    up to eps, every code +-127."""
    K = 96
    x = np.full((3, K), 0.75, np.float32)
    x[1] = -2.5
    x[2] = 0.0
    ones = np.ones(K, np.float32)
    q, s = oracle.norm_quantize(x, "layer", ones, None, 1e-5)
    assert (q == 0).all() and np.all(s == np.float32(1e-8) / np.float32(127.0))
    q, s = oracle.norm_quantize(x, "softmax")
    assert (q == 127).all()
    assert np.allclose(s, (1.0 / K) / 127.0, rtol=1e-6)
    q, s = oracle.norm_quantize(x[:2], "rms", ones, None, 1e-6)
    assert (q[0] == 127).all() and (q[1] == -127).all()


def test_oracle_softmax_properties(oracle):
    """Softmax codes are >= 0, the row maximum codes to 127, dequantized rows
    sum to 1 within the quantization step, and shifting every logit by an
    exactly representable constant changes nothing."""
    x, _, _ = _inputs(32, 1000, 11, scale=3.0)
    xv = x.numpy()
    q, s = oracle.norm_quantize(xv, "softmax")
    assert (q >= 0).all()
    assert (q.max(axis=1) == 127).all()
    assert np.all(np.abs((q.astype(np.float64) * s[:, None]).sum(axis=1) - 1.0) <= 1000 * s / 2 + 1e-6)
    q2, s2 = oracle.norm_quantize(xv + np.float32(0.5), "softmax")
    exact = np.array_equal((xv + np.float32(0.5)) - np.float32(0.5), xv)
    if exact:
        assert np.array_equal(q, q2) and np.array_equal(s, s2)


def test_oracle_planted_mistake_is_caught(oracle):
    """A LayerNorm without its mean subtraction (RMS statistics) fails the
    reference-formula check on rows with a nonzero mean."""
    x, gamma, beta = _inputs(16, 1024, 5)
    x = x + 1.0
    rq, _ = _torch_reference(x, "layer", gamma, beta, 1e-5)
    wrong = oracle.normalize_rows(x.numpy(), "rms", gamma.numpy(), None, 1e-5) + beta.numpy()
    q, _ = oracle.quantize(wrong)
    assert np.abs(q.astype(np.int32) - rq.numpy().astype(np.int32)).max() > 1


# ---------------------------------------------------------------- mirror: CPU branch + ABI
@pytest.mark.parametrize("M,K", REF_SHAPES)
def test_cpu_branch_is_reference_cpu_semantics(rt, M, K):
    """CPU tensors follow the reference's CPU branches exactly (their tests
    assert torch.equal against the f32 PyTorch formula)."""
    x, gamma, beta = _inputs(M, K, 3)
    for kind, out in (("layer", rt.fused_layernorm_quantize(x, gamma, beta)),
                      ("rms", rt.fused_rmsnorm_quantize(x, gamma)),
                      ("softmax", rt.fused_softmax_quantize(x))):
        rq, rs = _torch_reference(x, kind, gamma, beta if kind == "layer" else None, _eps(kind))
        assert torch.equal(out[0], rq), kind
        assert torch.allclose(out[1], rs, atol=1e-6), kind


def test_cpu_branch_shapes_and_extremes(rt):
    x = torch.randn(2, 8, 128)
    for q, s in (rt.fused_layernorm_quantize(x, torch.ones(128)), rt.fused_rmsnorm_quantize(x, torch.ones(128)),
                 rt.fused_softmax_quantize(x)):
        assert q.shape == (2, 8, 128) and s.shape == (2, 8) and q.dtype == torch.int8 and s.dtype == torch.float32
    q, s = rt.fused_softmax_quantize(torch.tensor([[1000.0, -1000.0, 0.0, 500.0]]))
    assert not torch.isnan(s).any()
    q, s = rt.fused_layernorm_quantize(torch.zeros(2, 64), torch.ones(64), torch.zeros(64))
    assert torch.isfinite(s).all()


@pytest.mark.parametrize("args", [
    # bad kind
    (None, 0, 1, 64, 64, 9, None, None, 0.0, None, 64, None, None),
    # softmax with gamma
    (None, 0, 1, 64, 64, 3, 1, None, 0.0, None, 64, None, None),
    # LayerNorm without gamma
    (None, 0, 1, 64, 64, 1, None, None, 1e-5, None, 64, None, None),
    # RMSNorm with beta
    (None, 0, 1, 64, 64, 2, 1, 1, 1e-6, None, 64, None, None),
    # K = 0, ld too small
    (None, 0, 1, 0, 64, 3, None, None, 0.0, None, 64, None, None),
    (None, 0, 1, 64, 32, 3, None, None, 0.0, None, 64, None, None),
])
def test_norm_quantize_argument_validation(rt, args):
    lib = rt.lib()
    assert lib.ic_norm_quantize(*args) == 1
    assert lib.ic_last_error().decode().startswith("ic_norm_quantize")


def test_norm_quantize_empty_batch(rt):
    assert rt.lib().ic_norm_quantize(None, 0, 0, 64, 64, 3, None, None, 0.0, None, 64, None, None) == 0


# ---------------------------------------------------------------- GPU parity
GPU_SHAPES = [(1, 64), (16, 1024), (64, 4096), (4608, 3072), (300, 16384), (37, 100), (9, 1000), (5, 20000)]
DTYPES = [torch.float16, torch.bfloat16, torch.float32]


def _check_codes(q, rq, s, rs, kind):
    d = np.abs(q.astype(np.int32) - rq.astype(np.int32))
    assert d.max() <= 1, kind
    assert (d == 0).mean() >= 0.9999, kind
    assert np.allclose(s, rs, rtol=2e-7 if kind != "softmax" else 1e-6, atol=0), kind


@pytest.mark.gpu
@pytest.mark.parametrize("M,K", GPU_SHAPES)
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("kind", KINDS)
def test_norm_quantize_matches_oracle(rt, oracle, dev, M, K, dtype, kind):
    """ic_norm_quantize against the oracle on the same inputs: codes equal
    (+-1 where an f32 result sits on a rounding edge, which the fp64 sum order
    or the device expf can move), scales equal to an ulp or two.  Shapes cover
    the reference tests' sizes, Flux hidden rows, the register-resident limit
    (16384) and the generic path (K not a multiple of 8, K > 16384)."""
    x, gamma, beta = _inputs(M, K, 200 + K, dtype, scale=2.0 if kind == "softmax" else 1.0)
    b = beta if kind == "layer" else None
    xd = x.to(dev)
    if kind == "layer":
        q, s = rt.fused_layernorm_quantize(xd, gamma.to(dev), b.to(dev), eps=1e-5)
    elif kind == "rms":
        q, s = rt.fused_rmsnorm_quantize(xd, gamma.to(dev), eps=1e-6)
    else:
        q, s = rt.fused_softmax_quantize(xd)
    xv = x.float().numpy()
    rq, rs = oracle.norm_quantize(xv, kind, gamma.numpy() if kind != "softmax" else None,
                                  b.numpy() if b is not None else None, _eps(kind))
    _check_codes(q.cpu().numpy(), rq, s.cpu().numpy(), rs, kind)
    if kind != "softmax" or dtype != torch.float32:
        # the reference tests' own bar against the f32 PyTorch formula
        tq, _ = _torch_reference(x.float(), kind, gamma, b, _eps(kind))
        assert (q.cpu().int() - tq.int()).abs().max() <= 1


@pytest.mark.gpu
def test_norm_quantize_buffers_shapes_and_edge_rows(rt, dev):
    """Pre-allocated outputs are filled in place; 3-D inputs keep their leading
    dims; zero rows, constant rows and extreme logits stay finite."""
    M, K = 8, 256
    x = torch.randn(M, K, dtype=torch.float16, device=dev)
    g = torch.randn(K, device=dev)
    s_buf = torch.empty(M, dtype=torch.float32, device=dev)
    q_buf = torch.empty(M, K, dtype=torch.int8, device=dev)
    q, s = rt.fused_layernorm_quantize(x, g, None, s_a_out=s_buf, x_int8_out=q_buf)
    assert q is q_buf and s is s_buf
    q, s = rt.fused_rmsnorm_quantize(torch.randn(2, 8, 128, device=dev), torch.ones(128, device=dev))
    assert q.shape == (2, 8, 128) and s.shape == (2, 8)
    q, s = rt.fused_layernorm_quantize(torch.zeros(2, 64, device=dev), torch.ones(64, device=dev),
                                       torch.zeros(64, device=dev))
    assert (q == 0).all().item() and torch.isfinite(s).all().item()
    q, s = rt.fused_softmax_quantize(torch.tensor([[1000.0, -1000.0, 0.0, 500.0]] * 8, device=dev))
    assert not torch.isnan(s).any().item() and (q >= 0).all().item()
    assert q[:, 0].eq(127).all().item()


# ---------------------------------------------------------------- norm + rotate + quantize
def test_oracle_norm_rotate_is_the_composition(oracle):
    """The oracle contract of ic_norm_rotate_quantize is its definition:
    normalise (fp64 statistics, f32 arithmetic), round once to the activation
    dtype, then the pinned rotate_quantize.  Cross-check the first half against
    F.layer_norm in f32 (rounded to bf16): the prepared codes agree within one
    code, the reference tests' own bar for a fused norm quantizer."""
    K = 3072
    x, _, _ = _inputs(64, K, 41, dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(42)
    scale = torch.randn(K, generator=g) * 0.1
    shift = torch.randn(K, generator=g) * 0.1
    sr = torch.exp(torch.randn(K, generator=g) * 0.5)
    perm = torch.randperm(K, generator=g)
    kw = dict(smoothrot=sr.numpy(), rot_size=256, perm=perm.numpy())
    q, s = oracle.norm_rotate_quantize(x, oracle.DT_BF16, "layer", (1 + scale).numpy(), shift.numpy(), 1e-6, **kw)
    y = (F.layer_norm(x.float(), (K,), eps=1e-6) * (1 + scale) + shift).to(torch.bfloat16)
    rq, rs = oracle.rotate_quantize(y, oracle.DT_BF16, **kw)
    assert np.abs(q.astype(np.int32) - rq.astype(np.int32)).max() <= 1
    assert np.allclose(s, rs, rtol=1e-2)


NRQ_CASES = [  # (M, K_in, w_in, rot_size, smoothrot+perm, affine)
    (4608, 3072, 3072, 256, True, True),     # Flux pre-qkv / pre-MLP rows
    (512, 3072, 3072, 256, True, False),
    (300, 5120, 5120, 1024, True, True),     # Wan hidden rows, five one-block waves
    (64, 13824, 14336, 1024, False, True),   # Wan FFN-down width, seven one-block waves, zero pad
    (48, 12288, 12288, 256, True, True),     # one twelve-wave tile
    (33, 9008, 9216, 64, True, False),       # the same tile, rotation pad 9008 -> 9024, then w_in pad
    (24, 15360, 16384, 16, True, True),      # two eight-wave tiles, w_in pad
    (40, 2048, 2048, 16, True, True),
    (40, 4096, 4096, 0, True, True),         # no rotation: norm + divide + perm + quantize
    (17, 1024, 1024, 64, False, False),
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", NRQ_CASES)
@pytest.mark.parametrize("norm", ["layer", "rms"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_norm_rotate_quantize_matches_oracle(rt, oracle, dev, case, norm, dtype):
    """ic_norm_rotate_quantize against the oracle's composition, bit for bit:
    the normalised values are rounded once to the dtype, after which every step
    is the exactly defined rotate_quantize."""
    M, K, K_w, R, with_prep, affine = case
    g = torch.Generator().manual_seed(M + K + R)
    x = (torch.randn(M, K, generator=g) * 3 + 0.5).to(dtype)
    w = (1 + 0.2 * torch.randn(K, generator=g)) if affine else None
    b = 0.1 * torch.randn(K, generator=g) if affine else None
    sr = torch.exp(torch.randn(K, generator=g) * 0.5) if with_prep else None
    perm = torch.randperm(K_w, generator=g) if with_prep else None
    q, s = rt.norm_rotate_quantize(
        x.to(dev), norm=norm, weight=w.to(dev) if w is not None else None,
        bias=b.to(dev) if b is not None else None, eps=1e-6, rot_size=R, w_in=K_w,
        smoothrot=rt.prepare_factors(sr.to(dev), dtype) if sr is not None else None,
        perm=rt.prepare_perm(perm.to(dev), K_w) if perm is not None else None)
    rq, rs = oracle.norm_rotate_quantize(
        x, DT[dtype], norm, w.numpy() if w is not None else None, b.numpy() if b is not None else None, 1e-6,
        smoothrot=sr.numpy() if sr is not None else None, rot_size=R, w_in=K_w,
        perm=perm.numpy() if perm is not None else None)
    assert np.array_equal(s.cpu().numpy(), rs)
    assert np.array_equal(q.cpu().numpy(), rq)


@pytest.mark.gpu
def test_norm_rotate_quantize_rejects_unsupported(rt, dev):
    x = torch.randn(4, 100, dtype=torch.float16, device=dev)  # K not a multiple of 16
    with pytest.raises(RuntimeError, match="ic_norm_rotate_quantize"):
        rt.norm_rotate_quantize(x, norm="layer", rot_size=0)
    with pytest.raises(ValueError):
        rt.norm_rotate_quantize(torch.randn(4, 64, dtype=torch.float16, device=dev), norm="batch")
