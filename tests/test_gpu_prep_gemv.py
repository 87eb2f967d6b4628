"""GPU parity of the single-launch prep + GEMV (ic_prep_gemv_w4a8 / _w8a8).

Each call must give, bit for bit, what rotate_quantize followed by the GEMM
entry point gives (they route M <= 16 to the GEMV), and that must equal the
oracle: prepare -> quantize -> exact int32 accumulators -> the epilogue.  The
cases cover every rotation size, both tile counts (K <= 4096, K <= 8192),
the pad paths (K_in below the rotated width, w_in above it), SmoothRot,
PermuQuant and old-SmoothQuant factors, both 16-bit activation types, the
three weight modes, the epilogue options, unaligned activation rows, the
Flux modulation shape, the bf16 flush rule and graph replay.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DT = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _layer(rt, dev, K_in, K_w, N, fmt, seed, *, sr=True, perm=True, smooth=False, dtype=torch.bfloat16):
    g = _gen(seed)
    fac = torch.exp(torch.randn(K_in, generator=g) * 0.5) if sr else None
    pm = torch.randperm(K_w, generator=g) if perm else None
    smf = torch.exp(torch.randn(K_w, generator=g) * 0.3) if smooth else None
    if fmt == "int8":
        w = torch.randint(-127, 128, (N, K_w), generator=g, dtype=torch.int8)
        s_w = (torch.rand(N, generator=g) * 2e-3 + 1e-4).to(torch.float16).float()
    else:
        G = K_w // 128 if fmt == "int4_g128" else 1
        w = torch.randint(0, 256, (N, K_w // 2), generator=g, dtype=torch.uint8)
        s_w = (torch.rand(N, G, generator=g) * 2e-2 + 1e-3).to(torch.float16).float()
    return dict(
        fac=fac, pm=pm, smf=smf, w=w, s_w=s_w,
        srp=rt.prepare_factors(fac.to(dev), dtype) if sr else None,
        pmd=rt.prepare_perm(pm.to(dev), K_w) if perm else None,
        smp=rt.prepare_factors(smf.to(dev), dtype) if smooth else None,
        wd=w.to(dev), swd=s_w.to(dev))


def _two_launches(rt, x, L, fmt, R, K_w, **epi):
    q, s_a = rt.rotate_quantize(x, rot_size=R, w_in=K_w, smoothrot=L["srp"], perm=L["pmd"], smooth=L["smp"])
    if fmt == "int8":
        return rt.fused_int8_gemm_dequant(q, L["wd"], L["swd"], s_a, **epi)
    return rt.gemm_w4a8(q, L["wd"], L["swd"], s_a, **epi)


def _fused(rt, x, L, fmt, R, K_w, **epi):
    return rt.prep_gemv(x, L["wd"], L["swd"], int4=fmt != "int8", rot_size=R, w_in=K_w, smoothrot=L["srp"],
                        perm=L["pmd"], smooth=L["smp"], **epi)


def _oracle(oracle, x, dtype, L, fmt, R, K_w, bias=None, out_dtype=torch.bfloat16, activation=0, residual=None):
    q, s = oracle.rotate_quantize(x.float(), DT[dtype], smoothrot=L["fac"], rot_size=R, w_in=K_w,
                                  perm=None if L["pm"] is None else L["pm"].numpy(), smooth=L["smf"])
    if fmt == "int8":
        acc, G = oracle.gemm_acc(q, L["w"].numpy()), 1
    else:
        G = L["s_w"].shape[1]
        acc = oracle.gemm_acc(q, oracle.unpack_int4(L["w"].numpy(), K_w), G)
    b = None if bias is None else bias.float().numpy()
    if activation == 0 and residual is None:
        return oracle.epilogue(acc, s, L["s_w"].numpy(), b, DT[out_dtype])
    return None  # the activation is checked against the two-launch path only (f32 vs float64 evaluation)


# (K_in, w_in, rot_size): plain, pad to the rotated width, pad past it, two tiles
SHAPES = [(3072, 3072, 256), (2880, 3072, 256), (1008, 1152, 64), (8192, 8192, 1024), (2048, 2048, 0),
          (4096, 4096, 4096), (512, 512, 16), (4608, 6144, 1024)]


# every M of 1, 2, 5, 16 whose codes fit the single launch's LDS (M * K_w <= 16384)
CASES = [(K_in, K_w, R, M) for (K_in, K_w, R) in SHAPES for M in (1, 2, 5, 16) if M * K_w <= 16384]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("fmt", ["int4_g128", "int4_row", "int8"])
@pytest.mark.parametrize("K_in,K_w,R,M", CASES)
def test_prep_gemv_matches_two_launches_and_oracle(rt, oracle, dev, dtype, fmt, K_in, K_w, R, M):
    assert M * K_w <= rt.PREP_GEMV_MAX_CODES
    N = 200 if K_w > 4096 else 136
    L = _layer(rt, dev, K_in, K_w, N, fmt, 7 + K_in + M, smooth=fmt == "int8" and M == 2, dtype=dtype)
    x = (torch.randn(M, K_in, generator=_gen(M)) * 2).to(dtype)
    x[:, :: max(1, K_in // 30)] *= 20  # outlier channels
    bias = torch.randn(N, generator=_gen(3)).to(dtype) if M % 2 else None
    xd = x.to(dev)
    epi = dict(bias=None if bias is None else bias.to(dev), out_dtype=dtype)
    got = _fused(rt, xd, L, fmt, R, K_w, **epi)
    ref2 = _two_launches(rt, xd, L, fmt, R, K_w, **epi)
    torch.cuda.synchronize()
    assert torch.equal(got, ref2)
    ref = _oracle(oracle, x, dtype, L, fmt, R, K_w, bias=bias, out_dtype=dtype)
    assert np.array_equal(got.float().cpu().numpy(), ref)


def test_flux_modulation_shape(rt, oracle, dev):
    """img_mod / txt_mod of a Flux double block: M = 1, 3072 -> 18432, bf16,
    R = 256, SmoothRot + PermuQuant, INT4 g128, bf16 bias."""
    K, N = 3072, 18432
    L = _layer(rt, dev, K, K, N, "int4_g128", 99)
    x = torch.randn(1, K, generator=_gen(98)).to(torch.bfloat16)
    bias = torch.randn(N, generator=_gen(97)).to(torch.bfloat16)
    epi = dict(bias=bias.to(dev), out_dtype=torch.bfloat16)
    got = _fused(rt, x.to(dev), L, "int4_g128", 256, K, **epi)
    assert torch.equal(got, _two_launches(rt, x.to(dev), L, "int4_g128", 256, K, **epi))
    ref = _oracle(oracle, x, torch.bfloat16, L, "int4_g128", 256, K, bias=bias)
    assert np.array_equal(got.float().cpu().numpy(), ref)


@pytest.mark.parametrize("fmt", ["int4_g128", "int8"])
@pytest.mark.parametrize("act", [1, 3])
def test_epilogue_options(rt, dev, fmt, act):
    M, K, N = 3, 2048, 264
    L = _layer(rt, dev, K, K, N, fmt, 41, dtype=torch.float16)
    x = torch.randn(M, K, generator=_gen(42)).to(torch.float16).to(dev)
    res = torch.randn(M, N, generator=_gen(43)).to(torch.float16).to(dev)
    bias = torch.randn(N, generator=_gen(44)).to(torch.float16).to(dev)
    for out_dtype in (torch.float16, torch.float32):
        epi = dict(bias=bias, out_dtype=out_dtype, activation=act, residual=res)
        assert torch.equal(_fused(rt, x, L, fmt, 256, K, **epi), _two_launches(rt, x, L, fmt, 256, K, **epi))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_row_stride_and_unaligned_rows(rt, dev, dtype):
    """Rows with a stride > K_in (a multiple of 8) run in one launch; rows at
    an odd element offset or with K_in not a multiple of 16 are outside the
    single launch (prep_gemv_ok says so, the C entry point refuses them)."""
    M, K, N = 4, 1536, 72
    L = _layer(rt, dev, K, K, N, "int4_g128", 51, dtype=dtype)
    base = torch.randn(M, K + 8, generator=_gen(52)).to(dtype).to(dev)
    x = base[:, :K]
    assert x.stride(0) == K + 8 and rt.prep_gemv_ok(x, K, L["wd"], K // 128)
    got = rt.prep_gemv(x, L["wd"], L["swd"], int4=True, rot_size=64, smoothrot=L["srp"], perm=L["pmd"],
                       out_dtype=dtype)
    assert torch.equal(got, _two_launches(rt, x, L, "int4_g128", 64, K, out_dtype=dtype))
    odd = base[:, 1:K + 1]
    assert not rt.prep_gemv_ok(odd, K, L["wd"], K // 128)
    with pytest.raises(ValueError, match="single-launch limits"):
        rt.prep_gemv(odd, L["wd"], L["swd"], int4=True, rot_size=64, smoothrot=L["srp"], perm=L["pmd"])
    lib = rt.lib()
    rc = lib.ic_prep_gemv_w4a8(odd.data_ptr(), rt._dt(dtype, "x"), M, K, K + 8, None, None, 64, None, None, None,
                               L["wd"].data_ptr(), N, K, K // 2, L["swd"].data_ptr(), K // 128, None, 0, 0, None, 0,
                               0, got.data_ptr(), rt._dt(dtype, "out"), N, None)
    assert rc != 0 and b"16-byte" in lib.ic_last_error()


@pytest.mark.parametrize("R", [256, 4096])
def test_bf16_flush_rows(rt, oracle, dev, R):
    """bf16 rows whose blocks span more binades than the fp64 butterflies hold
    exactly: values far below the block maximum are flushed first (with
    R = 4096 the block spans the four waves)."""
    M, K, N = 2, 4096, 96
    x = torch.randn(M, K, generator=_gen(61))
    x[0, 7] = 1e-30
    x[0, 2000:2010] = 3e-36
    x[1, ::331] = 1e25
    x = x.to(torch.bfloat16)
    L = _layer(rt, dev, K, K, N, "int4_g128", 62)
    got = _fused(rt, x.to(dev), L, "int4_g128", R, K, out_dtype=torch.bfloat16)
    assert torch.equal(got, _two_launches(rt, x.to(dev), L, "int4_g128", R, K, out_dtype=torch.bfloat16))
    ref = _oracle(oracle, x, torch.bfloat16, L, "int4_g128", R, K)
    assert np.array_equal(got.float().cpu().numpy(), ref)


def test_graph_replay(rt, dev):
    """Captured into a hipGraph and replayed with new inputs, with eager work
    between the replays: every replay equals the eager call."""
    M, K, N = 1, 3072, 2304
    L = _layer(rt, dev, K, K, N, "int4_g128", 71)
    static_x = torch.zeros(M, K, dtype=torch.bfloat16, device=dev)
    static_out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    _fused(rt, static_x, L, "int4_g128", 256, K, out=static_out)  # warm-up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _fused(rt, static_x, L, "int4_g128", 256, K, out=static_out)
    for i in range(4):
        x = torch.randn(M, K, generator=_gen(72 + i)).to(torch.bfloat16).to(dev)
        static_x.copy_(x)
        graph.replay()
        eager = _fused(rt, x, L, "int4_g128", 256, K)
        torch.cuda.synchronize()
        assert torch.equal(static_out, eager), f"replay {i}"


def test_argument_errors(rt, dev):
    L = _layer(rt, dev, 1024, 1024, 64, "int4_g128", 81)
    x = torch.randn(2, 1024, device=dev).to(torch.bfloat16)
    call = lambda xx, **kw: rt.prep_gemv(xx, L["wd"], L["swd"], int4=True, rot_size=256, **kw)  # noqa: E731
    with pytest.raises(ValueError, match="single-launch limits"):
        call(x.float())  # f32 rows
    with pytest.raises(ValueError, match="single-launch limits"):
        call(torch.zeros(17, 1024, device=dev, dtype=torch.bfloat16))  # M = 17
    big = _layer(rt, dev, 8192, 8192, 64, "int4_g128", 82)
    with pytest.raises(ValueError, match="single-launch limits"):  # M * K beyond the codes in LDS
        rt.prep_gemv(torch.zeros(3, 8192, device=dev, dtype=torch.bfloat16), big["wd"], big["swd"], int4=True)
    # the C entry point checks by itself
    lib = rt.lib()
    rc = lib.ic_prep_gemv_w4a8(None, 2, 1, 1024, 1024, None, None, 0, None, None, None, None, 64, 1024, 512, None,
                               1, None, 0, 0, None, 0, 0, None, 1, 64, None)
    assert rc != 0 and b"f16/bf16" in lib.ic_last_error()
    rc = lib.ic_prep_gemv_w4a8(None, 1, 0, 1024, 1024, None, None, 256, None, None, None, None, 64, 1024, 512, None,
                               3, None, 0, 0, None, 0, 0, None, 1, 64, None)
    assert rc != 0 and b"num_groups" in lib.ic_last_error()
    rc = lib.ic_prep_gemv_w4a8(None, 1, 1, 1024, 1024, None, None, 256, None, None, None, None, 64, 1024, 512, None,
                               8, None, 0, 0, None, 0, 0, None, 1, 64, None)
    assert rc != 0 and b"null pointer" in lib.ic_last_error()
    rc = lib.ic_prep_gemv_w8a8(None, 1, 0, 1024, 1024, None, None, 48, None, None, None, None, 64, 1024, 1024, None,
                               None, 0, 0, None, 0, 0, None, 1, 64, None)
    assert rc != 0 and b"rot_size 48" in lib.ic_last_error()
