"""GPU parity of the K-interleaved INT4 order (ic_int4_interleave_k,
ic_gemm_w4a8_kil_ex): the repack kernel equals the numpy restatement in
tests/_w4.py, and W4A8 on interleaved weights equals W4A8 on the checkpoint
order bit for bit on every route -- the 288 x 192 kernel in each fold mode,
the 256 x 128 / split-K tiles, the GEMV, the scalar kernel -- with and without
the activation / residual epilogue, and through the drop-in Linear."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import __graft_entry__
from _layers import int4_layer, load_linear
from _w4 import interleave_k

pytestmark = pytest.mark.gpu


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _packed(N, K, seed):
    return torch.randint(0, 256, (N, K // 2), generator=_gen(seed), dtype=torch.uint8)


@pytest.mark.parametrize("N,K", [(7, 8), (384, 1024), (3072, 12288)])
def test_interleave_kernel_matches_numpy(rt, dev, N, K):
    w = _packed(N, K, N + K)
    ref = interleave_k(w.numpy())
    out = rt.int4_interleave_k(w.to(dev))
    assert np.array_equal(out.cpu().numpy(), ref)
    wd = w.to(dev)
    assert rt.int4_interleave_k(wd, out=wd) is wd  # in place
    assert np.array_equal(wd.cpu().numpy(), ref)
    wide = torch.zeros(N, K // 2 + 48, dtype=torch.uint8)  # rows with a longer stride
    wide[:, :K // 2] = w
    o2 = rt.int4_interleave_k(wide.to(dev)[:, :K // 2])
    assert np.array_equal(o2.cpu().numpy(), ref)


# (M, N, K, G, out dtype): the route each takes is named after it
ROUTES = [
    (600, 384, 1024, 8, torch.bfloat16),    # 288 x 192, fold per 128 columns
    (600, 384, 1024, 16, torch.float16),    # 288 x 192, fold per 64
    (600, 384, 1024, 32, torch.bfloat16),   # 288 x 192, fold per 32
    (600, 384, 1024, 1, torch.bfloat16),    # per-row INT4
    (200, 256, 1024, 8, torch.float32),     # 256 x 128 (f32 output)
    (64, 3072, 3072, 24, torch.bfloat16),   # split-K
    (1, 2304, 3072, 1, torch.bfloat16),     # GEMV
    (5, 512, 1024, 32, torch.float16),      # GEMV, fold per 32
    (16, 256, 3072, 24, torch.float32),     # GEMV, fold per 128
    (37, 96, 520, 1, torch.float16),        # scalar kernel (K not a multiple of 128)
    (37, 96, 520, 65, torch.bfloat16),      # scalar kernel, groups of 8
    (4608, 3072, 12288, 96, torch.bfloat16),  # C3
]


@pytest.mark.parametrize("M,N,K,G,out_dtype", ROUTES)
@pytest.mark.parametrize("epi", [False, True])
def test_kil_gemm_equals_plain(rt, dev, M, N, K, G, out_dtype, epi):
    print(f"[kil] M={M} N={N} K={K} G={G} out={out_dtype} epi={epi}", flush=True)
    g = _gen(M * 7 + N + K + G)
    q = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8).to(dev)
    w = _packed(N, K, 3 + K).to(dev)
    sw = (torch.rand(N, G, generator=g) * 0.02 + 1e-3).to(dev)
    sa = (torch.rand(M, generator=g) * 0.05 + 1e-3).to(dev)
    bias = torch.randn(N, generator=g).to(torch.float16).to(dev)
    kw = {}
    if epi:
        kw = dict(activation=rt.ACT_GELU, residual=torch.randn(M, N, generator=g).to(torch.bfloat16).to(dev))
    plain = rt.gemm_w4a8(q, w, sw, sa, bias=bias, out_dtype=out_dtype, **kw)
    kil = rt.gemm_w4a8(q, rt.int4_interleave_k(w), sw, sa, bias=bias, out_dtype=out_dtype, kil=True, **kw)
    assert torch.equal(plain, kil)
    assert torch.isfinite(plain.float()).all()


def test_dropin_linear_uses_the_interleaved_copy(dev, monkeypatch):
    """W4A8 layers keep one interleaved copy of their weights per device; the
    outputs equal those of the checkpoint order (INTCRUSH_W4_INTERLEAVE=0)."""
    ops_mod = __graft_entry__._submodule("_ops")
    from test_gpu_ops import _to_dev, _x

    K, N = 1024, 192
    ops = ops_mod.make_intcrush_ops("int4_crush", 256)
    sd = int4_layer(N, K, G=8, seed=140)
    lin = _to_dev(load_linear(ops, "double_blocks.0.img_mlp.2", sd, K, N), dev)
    x = _x(300, K, torch.bfloat16, 141).to(dev)
    monkeypatch.setenv("INTCRUSH_W4_INTERLEAVE", "0")
    ref = lin(x).clone()
    assert lin._intcrush_state(x)._wpad is None
    monkeypatch.setenv("INTCRUSH_W4_INTERLEAVE", "1")
    out = lin(x)
    st = lin._intcrush_state(x)
    assert st._wpad is not None and st._wpad[0][2] is True
    assert st._wpad[1].data_ptr() != lin.weight._qdata.data_ptr()
    assert torch.equal(out, ref)


@pytest.mark.parametrize("K,G", [(1024, 8), (64, 2)])
def test_cast_weights_are_not_cached(dev, monkeypatch, K, G):
    """Weights that reach forward as a per-call cast copy (ComfyUI's offload or
    weight-patch path) are not cached by address -- a later copy may reuse the
    address with other contents: W4A8 runs them in the checkpoint order, and a
    narrow layer's zero-padded operands are built for that call.  Outputs equal
    the resident weights', and the resident cache is left as it was."""
    import comfy.quant_ops as qo

    ops_mod = __graft_entry__._submodule("_ops")
    from test_gpu_ops import _to_dev, _x

    N = 192
    ops = ops_mod.make_intcrush_ops("int4_crush", 64)
    sd = int4_layer(N, K, G=G, seed=150 + K)
    lin = _to_dev(load_linear(ops, "double_blocks.0.img_mlp.2", sd, K, N), dev)
    x = _x(300, K, torch.bfloat16, 151).to(dev)
    ref = lin(x).clone()
    st = lin._intcrush_state(x)
    cached = st._wpad
    assert cached is not None and cached[0][2] is True

    def cast_copy(s, input=None, dtype=None, device=None, bias_dtype=None, offloadable=False):
        w = s.weight
        w2 = qo.QuantizedTensor(w._qdata.clone(), w._layout_type, w._params)
        return (w2, s.bias, None) if offloadable else (w2, s.bias)

    monkeypatch.setattr(ops_mod, "_cast_fns", (cast_copy, lambda *a: None))
    monkeypatch.setattr(lin, "comfy_cast_weights", True, raising=False)
    for _ in range(2):
        out = lin(x)
        assert torch.equal(out, ref)
    assert lin._intcrush_state(x)._wpad is cached
