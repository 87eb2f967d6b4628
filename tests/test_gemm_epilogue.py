"""The activation / residual epilogue of the INT8 and W4A8 GEMMs
(kernels/triton_int8_gemm.py:119-130 and its arguments :142-143).

CPU: the oracle's activations against torch's own SiLU / GELU / GELU-tanh in
float64, the reduction of the extended epilogue to the plain one, and the
host-side argument checks.  GPU: every routing of the GEMM (GEMV at M <= 16,
split K at small M, the MFMA tiles with the LDS-staged 16-bit epilogue, the
direct epilogue for ragged N or an odd residual stride, the shape-generic
kernel) for each activation and residual dtype.  With activation 0 the
residual add is one f32 addition, so those outputs are bit-exact; with an
activation the GPU's f32 evaluation (hardware exp2 and reciprocal, the
Abramowitz & Stegun erf) may differ from the float64 oracle by a few f32 ulp
before the final rounding, so outputs are held to 2^-20 (|v| + |act(v)| +
|residual|) plus one ulp of the output dtype.  The f32 outputs are the ones
that tell GELU from GELU-tanh (their difference is far above that bound and
may hide under a bf16 ulp).  Also int8_gemm_int8out (the GEMM re-quantized to
INT8 with whole-row scales), bit-exact against the oracle.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

DT = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}
MANT = {torch.float16: 10, torch.bfloat16: 7}


def _gen(seed):
    return torch.Generator().manual_seed(seed)


# ------------------------------------------------------------------ CPU
def _grid():
    v = np.linspace(-30.0, 30.0, 6001)
    return np.concatenate([v, [0.0, -0.0, 1e-30, -1e-30, 1e-3, -1e-3, 88.0, -88.0, 200.0, -200.0]])


def test_oracle_silu_is_torch_silu(oracle):
    v = _grid()
    ref = F.silu(torch.from_numpy(v)).numpy()
    assert np.allclose(oracle.activate(v, 1), ref, rtol=1e-13, atol=1e-300)


@pytest.mark.parametrize("act,approx", [(2, "none"), (3, "tanh")])
def test_oracle_gelu_is_torch_gelu(oracle, act, approx):
    v = _grid()
    ref = F.gelu(torch.from_numpy(v), approximate=approx).numpy()
    assert np.allclose(oracle.activate(v, act), ref, rtol=1e-12, atol=1e-15)


def test_oracle_activation_special_values(oracle):
    for act in (1, 2, 3):
        assert oracle.activate(np.array([0.0]), act)[0] == 0.0
        big = oracle.activate(np.array([50.0, -50.0]), act)
        assert big[0] == 50.0 and abs(big[1]) < 1e-15
    # the two GELUs differ by far more than the f32 tolerance of the GPU tests
    v = np.linspace(-4, 4, 801)
    assert np.abs(oracle.activate(v, 2) - oracle.activate(v, 3)).max() > 1e-4
    with pytest.raises(ValueError):
        oracle.activate(v, 4)


def _f32_gelu_as(v, rcp_ulp=0, exp_ulp=0):
    """The kernel's f32 GELU (Abramowitz & Stegun 7.1.26 erf) in numpy f32,
    with its reciprocal and exp2 results moved by rcp_ulp / exp_ulp ulp (the
    hardware instructions are within 1 ulp)."""
    f = np.float32
    a = np.abs(v) * f(0.70710678118654752)
    t = f(1) / (f(1) + f(0.3275911) * a)
    if rcp_ulp:
        t = np.nextafter(t, f(rcp_ulp * np.inf))
    p = t * (f(0.254829592) + t * (f(-0.284496736) + t * (f(1.421413741) + t * (f(-1.453152027)
                                                                                + t * f(1.061405429)))))
    e = np.exp2(((a * a) * f(-1.44269504088896341)).astype(np.float64)).astype(np.float32)
    if exp_ulp:
        e = np.nextafter(e, f(exp_ulp * np.inf))
    q = p * e
    return (v * f(0.5)) * np.where(v >= 0, f(2) - q, q)


def test_gelu_erf_approximation_bound(oracle):
    """The published 1.5e-7 bound of the erf approximation plus f32 rounding
    keeps the kernel's GELU within 2^-21 (|v| + |GELU(v)|) of float64 GELU:
    inside the 2^-20 the GPU tests allow, on both sides of every branch."""
    v = np.concatenate([np.linspace(-12, 12, 240001), np.geomspace(1e-6, 12, 20001),
                        -np.geomspace(1e-6, 12, 20001), [0.0]]).astype(np.float32)
    ref = oracle.activate(v.astype(np.float64), 2)
    for ru in (-1, 0, 1):
        for eu in (-1, 0, 1):
            err = np.abs(_f32_gelu_as(v, ru, eu).astype(np.float64) - ref)
            assert (err <= 2.0 ** -21 * (np.abs(v) + np.abs(ref))).all(), (ru, eu)


def test_epilogue_ex_reduces_to_epilogue(oracle):
    g = np.random.default_rng(3)
    acc = g.integers(-2 ** 20, 2 ** 20, (7, 9)).astype(np.int32)
    s_a = (g.random(7) * 1e-3).astype(np.float32)
    s_w = (g.random(9) * 1e-2).astype(np.float32)
    b = g.standard_normal(9).astype(np.float32)
    for dt in (0, 1, 2):
        assert np.array_equal(oracle.epilogue_ex(acc, s_a, s_w, b, dt), oracle.epilogue(acc, s_a, s_w, b, dt))
    # residual on unit scales: the integers themselves plus the residual
    acc = np.arange(-6, 6, dtype=np.int32).reshape(3, 4)
    r = np.full((3, 4), 0.5, np.float32)
    out = oracle.epilogue_ex(acc, np.ones(3, np.float32), np.ones(4, np.float32), None, 2, 0, r)
    assert np.array_equal(out, acc.astype(np.float32) + 0.5)
    silu = oracle.epilogue_ex(acc, np.ones(3, np.float32), np.ones(4, np.float32), None, 2, 1, None)
    assert silu[1, 2] == 0.0 and silu[0, 0] < 0 and silu[2, 3] > 4.9


def test_epilogue_args_checks(rt):
    with pytest.raises(ValueError, match="activation"):
        rt._epilogue_args(4, None, 2, 2)
    with pytest.raises(ValueError, match="activation"):
        rt._epilogue_args(-1, None, 2, 2)
    with pytest.raises(ValueError, match="residual shape"):
        rt._epilogue_args(0, torch.zeros(3, 4), 3, 5)
    wide = torch.zeros(3, 12, dtype=torch.float16)
    act, ptr, dt, ldr, keep = rt._epilogue_args(1, wide[:, :5], 3, 5)
    assert (act, dt, ldr) == (1, 0, 12) and ptr.value == wide.data_ptr()
    # a transposed view is made contiguous; a 3-D residual is flattened to rows
    _, _, _, ldr, keep = rt._epilogue_args(0, torch.zeros(5, 3).t(), 3, 5)
    assert ldr == 5 and keep.is_contiguous()
    _, _, dt, ldr, _ = rt._epilogue_args(0, torch.zeros(1, 3, 5, dtype=torch.bfloat16), 3, 5)
    assert (dt, ldr) == (1, 5)
    with pytest.raises(TypeError):
        rt._epilogue_args(0, torch.zeros(3, 5, dtype=torch.float64), 3, 5)


# ------------------------------------------------------------------ GPU
# (M, N, K, route); the route is asserted where the library exposes it
SHAPES = [
    (5, 384, 512, "gemv"),
    (100, 1000, 3072, "splitk"),
    (384, 512, 512, "tiles"),
    (260, 250, 384, "ragged"),
    (1400, 5752, 256, "big"),  # 16-bit out: 256 x 192 tiles, partial in M and N (every format)
]
FMTS = ["int8", "int4", "int4g"]


def _ulp(ref: np.ndarray, dtype) -> np.ndarray:
    if dtype == torch.float32:
        return np.zeros_like(ref, dtype=np.float64)
    mant = MANT[dtype]
    emin = -14 if dtype == torch.float16 else -126
    e = np.floor(np.log2(np.maximum(np.abs(ref).astype(np.float64), 2.0 ** emin)))
    return 2.0 ** (e - mant)


def _problem(M, N, K, fmt, seed, oracle):
    a = torch.randint(-127, 128, (M, K), generator=_gen(seed), dtype=torch.int8)
    s_a = torch.rand(M, generator=_gen(seed + 1)) * 0.02 + 1e-3
    G = K // 128 if fmt == "int4g" else 1
    if fmt == "int8":
        w = torch.randint(-127, 128, (N, K), generator=_gen(seed + 2), dtype=torch.int8)
        wq = w.numpy()
        s_w = (torch.rand(N, generator=_gen(seed + 3)) * 2e-3 + 1e-4).to(torch.float16).float()
    else:
        w = torch.randint(0, 256, (N, K // 2), generator=_gen(seed + 2), dtype=torch.uint8)
        wq = oracle.unpack_int4(w.numpy(), K)
        s_w = (torch.rand(N, G, generator=_gen(seed + 3)) * 3e-2 + 1e-3).to(torch.float16).float()
    bias = torch.randn(N, generator=_gen(seed + 4)).to(torch.bfloat16)
    acc = oracle.gemm_acc(a.numpy(), wq, G)
    return a, w, s_a, s_w, bias, acc


def _run(rt, fmt, a, w, s_a, s_w, bias, out_dtype, act, res, dev):
    kw = dict(bias=bias.to(dev), out_dtype=out_dtype, activation=act, residual=res)
    if fmt == "int8":
        return rt.fused_int8_gemm_dequant(a.to(dev), w.to(dev), s_w.to(dev), s_a.to(dev), **kw)
    return rt.gemm_w4a8(a.to(dev), w.to(dev), s_w.to(dev), s_a.to(dev), **kw)


def _residuals(M, N, out_dtype, seed, dev):
    """None, a contiguous one in the output's 16-bit dtype (bf16 for f32
    outputs), an f32 one, and an f16 view with an odd row stride."""
    g = _gen(seed)
    r16 = torch.randn(M, N, generator=g).to(out_dtype if out_dtype != torch.float32 else torch.bfloat16)
    r32 = torch.randn(M, N, generator=g) * 3.0
    odd = torch.randn(M, N + 3, generator=g).to(torch.float16)
    return [("none", None), ("r16", r16.to(dev)), ("r32", r32.to(dev)), ("odd", odd.to(dev)[:, :N])]


@pytest.mark.gpu
@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("M,N,K,route", SHAPES)
def test_gemm_epilogue_matches_oracle(rt, oracle, dev, M, N, K, route, fmt, out_dtype):
    if fmt == "int4g" and K % 128:
        pytest.skip("grouped scales need K % 128 == 0")
    if route == "big" and out_dtype == torch.float32:
        pytest.skip("the big tiles write 16-bit outputs only")
    G = K // 128 if fmt == "int4g" else 1
    if route == "splitk":
        assert rt.lib().ic_gemm_splitk_bytes(M, N, K, G, int(fmt != "int8")) > 0
    elif route != "gemv":
        assert rt.lib().ic_gemm_splitk_bytes(M, N, K, G, int(fmt != "int8")) == 0
    a, w, s_a, s_w, bias, acc = _problem(M, N, K, fmt, 900 + M, oracle)
    v32 = _run(rt, fmt, a, w, s_a, s_w, bias, torch.float32, 0, None, dev).cpu().numpy()
    if not (route == "splitk" and fmt == "int4g"):
        # (grouped split-K sums its slices in another order: test_gpu_kernels
        # bounds that; the options below act on whatever value the GEMM made)
        assert np.array_equal(v32, oracle.epilogue(acc, s_a.numpy(), s_w.numpy(), bias.float().numpy(), 2))
    v = v32.astype(np.float64)
    for rname, res in _residuals(M, N, out_dtype, 77, dev):
        r = None if res is None else res.float().cpu().numpy()
        for act in (0, 1, 2, 3):
            out = _run(rt, fmt, a, w, s_a, s_w, bias, out_dtype, act, res, dev).float().cpu().numpy()
            tag = f"{route} {fmt} {out_dtype} act={act} res={rname}"
            if act == 0:
                # one f32 addition, then the rounding: bit-exact
                s = v32 if r is None else (v32 + r.astype(np.float32))
                ref = oracle.round_dtype(s.astype(np.float64), DT[out_dtype])
                assert np.array_equal(out, ref), tag
                continue
            act_v = oracle.activate(v, act)
            ref = oracle.round_dtype(act_v if r is None else act_v + r, DT[out_dtype])
            av = np.abs(act_v)
            bound = 2.0 ** -20 * (np.abs(v) + av + (0 if r is None else np.abs(r))) + _ulp(ref, out_dtype)
            err = np.abs(out.astype(np.float64) - ref)
            bad = err > bound
            assert not bad.any(), f"{tag}: {bad.sum()} outside, worst {err.max():.3g}"
            # the outputs are not trivially equal to the unactivated ones
            assert np.abs(ref - oracle.round_dtype(v if r is None else v + r, DT[out_dtype])).max() > 1e-2


@pytest.mark.gpu
def test_gemm_epilogue_generic_kernel(rt, oracle, dev):
    """K not a multiple of the MFMA step: the shape-generic kernel applies the
    same epilogue."""
    M, N, K = 70, 96, 200
    a, w, s_a, s_w, bias, acc = _problem(M, N, K, "int8", 31, oracle)
    r = torch.randn(M, N, generator=_gen(32)).to(torch.float16)
    v32 = oracle.epilogue(acc, s_a.numpy(), s_w.numpy(), bias.float().numpy(), DT[torch.float32])
    out = _run(rt, "int8", a, w, s_a, s_w, bias, torch.float32, 0, r.to(dev), dev).cpu().numpy()
    assert np.array_equal(out, v32 + r.float().numpy())
    out = _run(rt, "int8", a, w, s_a, s_w, bias, torch.float32, 1, r.to(dev), dev).cpu().numpy()
    ref = oracle.epilogue_ex(acc, s_a.numpy(), s_w.numpy(), bias.float().numpy(), 2, 1, r.float().numpy())
    assert np.allclose(out, ref, rtol=2e-6, atol=1e-6)


@pytest.mark.gpu
def test_gemm_epilogue_rejects_bad_arguments(rt, dev):
    a = torch.zeros(32, 128, dtype=torch.int8, device=dev)
    w = torch.zeros(64, 128, dtype=torch.int8, device=dev)
    s = torch.ones(64, device=dev)
    sa = torch.ones(32, device=dev)
    with pytest.raises(ValueError, match="activation"):
        rt.fused_int8_gemm_dequant(a, w, s, sa, activation=5)
    with pytest.raises(ValueError, match="residual shape"):
        rt.fused_int8_gemm_dequant(a, w, s, sa, residual=torch.zeros(32, 63, device=dev))
    with pytest.raises(ValueError):
        rt.fused_int8_gemm_dequant(a, w, s, sa, residual=torch.zeros(32, 64))  # host residual
    # the C entry point checks its own arguments too
    P = rt._ptr
    out = torch.empty(32, 64, dtype=torch.bfloat16, device=dev)
    rc = rt.lib().ic_gemm_w8a8_ex(P(a), 32, 128, 128, P(w), 64, 128, P(sa), P(s), None, 0, 7, None, 0, 0,
                                  P(out), 1, 64, None, 0, None)
    assert rc != 0 and b"activation" in rt.lib().ic_last_error()
    r = torch.zeros(32, 64, device=dev)
    rc = rt.lib().ic_gemm_w8a8_ex(P(a), 32, 128, 128, P(w), 64, 128, P(sa), P(s), None, 0, 1, P(r), 2, 10,
                                  P(out), 1, 64, None, 0, None)
    assert rc != 0 and b"stride" in rt.lib().ic_last_error()


@pytest.mark.gpu
def test_gemm_epilogue_default_is_plain_gemm(rt, dev):
    """activation 0 and no residual run the plain kernels: identical bits."""
    g = _gen(5)
    a = torch.randint(-127, 128, (512, 1024), generator=g, dtype=torch.int8).to(dev)
    w = torch.randint(0, 256, (768, 512), generator=g, dtype=torch.uint8).to(dev)
    s_w = (torch.rand(768, 8, generator=g) * 1e-2 + 1e-3).to(dev)
    s_a = (torch.rand(512, generator=g) * 1e-2).to(dev)
    x = rt.gemm_w4a8(a, w, s_w, s_a, out_dtype=torch.bfloat16)
    y = rt.gemm_w4a8(a, w, s_w, s_a, out_dtype=torch.bfloat16, activation=0, residual=None)
    assert torch.equal(x, y)


# ------------------------------------------------------------------ int8_gemm_int8out
@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K", [(300, 1000, 512), (5, 384, 256), (512, 3072, 1024)])
def test_int8_gemm_int8out_matches_oracle(rt, oracle, dev, M, N, K):
    """INT8 codes and per-row scales of the re-quantized GEMM output equal the
    oracle's quantizer applied to the oracle's f32 dequant, bit for bit; the
    scale is the whole row's: a row whose abs-max sits in its last N-tile
    scales every tile by it (the reference kernel's per-tile scale would not)."""
    a, w, s_a, s_w, _bias, acc = _problem(M, N, K, "int8", 41, oracle)
    # plant the row abs-max of row 0 in its last column
    w[-1, :] = 127
    a[0, :] = 127
    s_w[-1] = s_w.max()
    acc = oracle.gemm_acc(a.numpy(), w.numpy())
    c, s_c = rt.int8_gemm_int8out(a.to(dev), w.to(dev), s_w.to(dev), s_a.to(dev))
    v = oracle.epilogue(acc, s_a.numpy(), s_w.numpy(), None, 2)
    q_ref, s_ref = oracle.quantize(v)
    assert np.array_equal(s_c.cpu().numpy(), s_ref)
    assert np.array_equal(c.cpu().numpy(), q_ref)
    assert abs(v[0]).argmax() == N - 1 and c[0, -1].item() == 127
    # pre-allocated outputs are filled in place
    c2 = torch.empty(M, N, dtype=torch.int8, device=dev)
    s2 = torch.empty(M, dtype=torch.float32, device=dev)
    r = rt.int8_gemm_int8out(a.to(dev), w.to(dev), s_w.to(dev), s_a.to(dev), c_out=c2, s_c_out=s2)
    assert r[0].data_ptr() == c2.data_ptr() and r[1].data_ptr() == s2.data_ptr()
    assert torch.equal(c2.cpu(), c.cpu()) and torch.equal(s2.cpu(), s_c.cpu())
    with pytest.raises(AssertionError):
        rt.int8_gemm_int8out(a.to(dev), w.to(dev), s_w.to(dev), s_a.to(dev), c_out=c2[:, :-1])
