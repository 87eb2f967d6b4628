"""ic_gemm_w4a8_noalloc: the split-K W4A8 GEMM with the library's static
scratch instead of a caller workspace.  Called through the C ABI and compared
bit-exactly with ic_gemm_w4a8_ws (same kernels, workspace from torch) on two
calls in a row, the second smaller, so the second call reuses scratch the
first one left behind."""
from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

SCRATCH = 32 << 20  # IC_NOALLOC_SCRATCH_BYTES


def _operands(M, N, K, seed, dev):
    g = torch.Generator().manual_seed(seed)
    xq = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    packed = torch.randint(0, 256, (N, K // 2), generator=g, dtype=torch.uint8)
    s_w = (torch.rand(N, K // 128, generator=g) * 1e-2 + 1e-3).to(torch.float16).float()
    s_a = torch.rand(M, generator=g) * 1e-2 + 1e-4
    bias = torch.randn(N, generator=g).to(torch.float16)
    return [t.to(dev) for t in (xq, packed, s_w, s_a, bias)]


def _run(rt, entry, M, N, K, ops, ws=None):
    xq, packed, s_w, s_a, bias = ops
    out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=xq.device)
    L = rt.lib()
    args = [rt._ptr(xq), M, K, K, rt._ptr(packed), N, K // 2, rt._ptr(s_w), K // 128, rt._ptr(s_a),
            rt._ptr(bias), rt.IC_DTYPE_F16, rt._ptr(out), rt.IC_DTYPE_BF16, N]
    if entry == "ic_gemm_w4a8_ws":
        args += [rt._ptr(ws), ws.numel() if ws is not None else 0]
    rc = getattr(L, entry)(*args, rt._stream(xq))
    assert rc == 0, L.ic_last_error().decode()
    return out


@pytest.mark.parametrize("shapes", [
    ((64, 3072, 12288), (24, 1024, 4096)),   # both split K
    ((128, 3072, 3072), (40, 512, 2048)),
])
def test_noalloc_matches_workspace_entry(rt, dev, shapes):
    L = rt.lib()
    for i, (M, N, K) in enumerate(shapes):
        need = L.ic_gemm_splitk_bytes(M, N, K, K // 128, 1)
        assert 0 < need <= SCRATCH, (M, N, K, need)
        ops = _operands(M, N, K, 100 + i, dev)
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        ref = _run(rt, "ic_gemm_w4a8_ws", M, N, K, ops, ws)
        got = _run(rt, "ic_gemm_w4a8_noalloc", M, N, K, ops)
        torch.cuda.synchronize()
        assert not torch.isnan(ref.float()).any()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"call {i}: {M}x{N}x{K}"


def test_noalloc_unsplit_and_gemv_shapes(rt, dev):
    # no split-K (scratch untouched) and the M <= 16 GEMV route
    for M, N, K in ((2048, 3072, 1024), (4, 2048, 3072)):
        assert rt.lib().ic_gemm_splitk_bytes(M, N, K, K // 128, 1) == 0
        ops = _operands(M, N, K, 7, dev)
        ref = _run(rt, "ic_gemm_w4a8_ws", M, N, K, ops)
        got = _run(rt, "ic_gemm_w4a8_noalloc", M, N, K, ops)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


def test_noalloc_rejects_plans_beyond_the_scratch(rt, dev):
    L = rt.lib()
    # 8 K slices of a 512 x 3072 output: 48 MiB of partials on 256 CUs
    M, N, K = 512, 3072, 65536
    need = L.ic_gemm_splitk_bytes(M, N, K, K // 128, 1)
    assert need > SCRATCH, need
    # the size check runs before any launch: nothing is read, so null operands are fine
    rc = L.ic_gemm_w4a8_noalloc(None, M, K, K, None, N, K // 2, None, K // 128, None, None, 0, None,
                                rt.IC_DTYPE_BF16, N, None)
    assert rc == 2
    assert "static" in L.ic_last_error().decode()


def test_noalloc_captured_in_a_graph(rt, dev):
    """ic_init_device resolves the scratch outside the capture; the captured
    no-alloc GEMM, replayed three times with eager work and synchronizations
    between the replays, matches ic_gemm_w4a8_ws every time."""
    M, N, K = 64, 3072, 12288
    need = rt.lib().ic_gemm_splitk_bytes(M, N, K, K // 128, 1)
    assert 0 < need <= SCRATCH
    ops = _operands(M, N, K, 300, dev)
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    ref = _run(rt, "ic_gemm_w4a8_ws", M, N, K, ops, ws)
    rt.init_device(dev)
    xq, packed, s_w, s_a, bias = ops
    out = torch.zeros(M, N, dtype=torch.bfloat16, device=dev)
    L = rt.lib()
    args = [rt._ptr(xq), M, K, K, rt._ptr(packed), N, K // 2, rt._ptr(s_w), K // 128, rt._ptr(s_a),
            rt._ptr(bias), rt.IC_DTYPE_F16, rt._ptr(out), rt.IC_DTYPE_BF16, N]
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            rc = L.ic_gemm_w4a8_noalloc(*args, ctypes.c_void_p(s.cuda_stream))
    assert rc == 0, L.ic_last_error().decode()
    torch.cuda.current_stream().wait_stream(s)
    for i in range(3):
        out.fill_(float("nan"))
        other = _run(rt, "ic_gemm_w4a8_noalloc", 24, 1024, 4096, _operands(24, 1024, 4096, 301 + i, dev))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"replay {i}"
        assert not torch.isnan(other.float()).any()
