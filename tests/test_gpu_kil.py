"""GPU parity of the derived INT4 weight forms: the K-interleaved order
(ic_int4_interleave_k, ic_gemm_w4a8_kil_ex) and the weights unpacked to int8
(ic_unpack_int4_to_int8, ic_gemm_w4a8_unpacked_ex).  The repack kernel equals
the numpy restatement in tests/_w4.py, and W4A8 on either form equals W4A8 on
the checkpoint order bit for bit on every route -- the 288 x 192 kernel in
each fold mode, the 256 x 128 / split-K tiles, the GEMV, the scalar kernel --
with and without the activation / residual epilogue, and through the drop-in
Linear."""
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


@pytest.mark.parametrize("M,N,K,G,out_dtype", ROUTES)
@pytest.mark.parametrize("epi", [False, True])
def test_unpacked_gemm_equals_plain(rt, dev, M, N, K, G, out_dtype, epi):
    """The unpacked form takes the int8-weight kernels: the 288 x 192 kernel's
    grouped int8 mode, per-row W8A8, the int8 256 x 128 and split-K tiles, the
    scalar kernel (the tile kernels also at M <= 16); every one folds in the
    same order as the packed routes."""
    print(f"[unpacked] M={M} N={N} K={K} G={G} out={out_dtype} epi={epi}", flush=True)
    g = _gen(M * 5 + N + K + G)
    q = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8).to(dev)
    w = _packed(N, K, 5 + K).to(dev)
    sw = (torch.rand(N, G, generator=g) * 0.02 + 1e-3).to(dev)
    sa = (torch.rand(M, generator=g) * 0.05 + 1e-3).to(dev)
    bias = torch.randn(N, generator=g).to(torch.bfloat16).to(dev)
    kw = {}
    if epi:
        kw = dict(activation=rt.ACT_GELU_TANH, residual=torch.randn(M, N, generator=g).to(torch.float16).to(dev))
    plain = rt.gemm_w4a8(q, w, sw, sa, bias=bias, out_dtype=out_dtype, **kw)
    w8 = rt.unpack_int4_to_int8(w, K)
    un = rt.gemm_w4a8_unpacked(q, w8, sw, sa, bias=bias, out_dtype=out_dtype, **kw)
    assert torch.equal(plain, un)
    assert torch.isfinite(plain.float()).all()


def test_unpacked_rule(rt, dev):
    """Unpacked weights for launches whose 288 x 192 tiles fill at most half
    the CUs and whose groups are whole 128-column blocks; never for the GEMV."""
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    assert rt.w4a8_unpacked_pays(512, 3072, 3072, 24, device=dev)
    assert not rt.w4a8_unpacked_pays(16, 3072, 3072, 24, device=dev)
    assert not rt.w4a8_unpacked_pays(512, 3072, 3072, 48, device=dev)  # groups of 64
    assert rt.w4a8_unpacked_pays(512, 3072, 3072, 1, device=dev)
    tiles_half = cus // 2  # 288-row tiles x 192-column tiles
    assert rt.w4a8_unpacked_pays(288, 192 * tiles_half, 3072, 24, device=dev)
    assert not rt.w4a8_unpacked_pays(288, 192 * (tiles_half + 1), 3072, 24, device=dev)
    assert not rt.w4a8_unpacked_pays(4608, 3072, 12288, 96, device=dev)


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
    monkeypatch.setenv("INTCRUSH_W4_UNPACKED", "0")  # this small launch would take the unpacked copy
    monkeypatch.setenv("INTCRUSH_W4_INTERLEAVE", "0")
    ref = lin(x).clone()
    assert "kil" not in lin._intcrush_state(x)._wcache
    monkeypatch.setenv("INTCRUSH_W4_INTERLEAVE", "1")
    out = lin(x)
    st = lin._intcrush_state(x)
    assert "kil" in st._wcache
    assert st._wcache["kil"][1].data_ptr() != lin.weight._qdata.data_ptr()
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
    monkeypatch.setenv("INTCRUSH_W4_UNPACKED", "0")
    ref = lin(x).clone()
    st = lin._intcrush_state(x)
    cached = dict(st._wcache)
    assert "kil" in cached

    def cast_copy(s, input=None, dtype=None, device=None, bias_dtype=None, offloadable=False):
        w = s.weight
        w2 = qo.QuantizedTensor(w._qdata.clone(), w._layout_type, w._params)
        return (w2, s.bias, None) if offloadable else (w2, s.bias)

    monkeypatch.setattr(ops_mod, "_cast_fns", (cast_copy, lambda *a: None))
    monkeypatch.setattr(lin, "comfy_cast_weights", True, raising=False)
    for _ in range(2):
        out = lin(x)
        assert torch.equal(out, ref)
    now = lin._intcrush_state(x)._wcache
    assert now.keys() == cached.keys() and all(now[k] is cached[k] for k in cached)


def test_dropin_linear_uses_the_unpacked_copy(dev, monkeypatch):
    """A W4A8 layer called with few rows runs its unpacked int8 copy (kept per
    device next to the interleaved one, which larger launches use); outputs
    equal the packed route's bit for bit, with and without a K pad."""
    ops_mod = __graft_entry__._submodule("_ops")
    from test_gpu_ops import _to_dev, _x

    for K, N, G, seed in ((1024, 192, 8, 160), (1000, 192, 1, 161)):
        ops = ops_mod.make_intcrush_ops("int4_crush", 0 if K % 8 else 256)
        sd = int4_layer(N, K, G=G, seed=seed)
        lin = _to_dev(load_linear(ops, "double_blocks.0.txt_mlp.2", sd, K, N), dev)
        x = _x(300, K, torch.bfloat16, seed + 1).to(dev)
        monkeypatch.setenv("INTCRUSH_W4_UNPACKED", "0")
        ref = lin(x).clone()
        st = lin._intcrush_state(x)
        assert "unpacked" not in st._wcache
        monkeypatch.setenv("INTCRUSH_W4_UNPACKED", "1")
        out = lin(x)
        assert "unpacked" in st._wcache
        w8 = st._wcache["unpacked"][1]
        assert w8.dtype == torch.int8 and w8.shape == (N, st.k_gemm)
        assert torch.equal(out, ref)
        assert lin(x) is not None and st._wcache["unpacked"][1] is w8  # built once


def test_dropin_w4a16_uses_the_staged_copy(dev, monkeypatch):
    """A W4A16 layer (unrotated INT4) called with more than 128 rows runs its
    staged copy (stage-major weights, group-major scales, kept per device; for
    K = 1000 built from the weights padded to the prepared width 1024);
    outputs equal the row-major route's bit for bit.  Calls of at most 128
    rows keep the row-major route and build no staged copy."""
    ops_mod = __graft_entry__._submodule("_ops")
    from test_gpu_ops import _to_dev, _x

    for K, N, G, dtype, seed in ((1024, 192, 8, torch.bfloat16, 170), (768, 136, 6, torch.float16, 171),
                                 (1000, 192, 1, torch.float16, 172)):
        ops = ops_mod.make_intcrush_ops("int4_crush", 256)
        sd = int4_layer(N, K, G=G, seed=seed)
        lin = _to_dev(load_linear(ops, "single_blocks.0.modulation.lin", sd, K, N), dev)
        assert not lin._intcrush_rot_need
        small = _x(100, K, dtype, seed + 2).to(dev)
        lin(small)
        st = lin._intcrush_state(small)
        assert "staged" not in st._wcache
        x = _x(300, K, dtype, seed + 1).to(dev)
        monkeypatch.setenv("INTCRUSH_W4A16_STAGED", "0")
        ref = lin(x).clone()
        assert "staged" not in st._wcache
        monkeypatch.setenv("INTCRUSH_W4A16_STAGED", "1")
        out = lin(x)
        assert torch.equal(out, ref)
        assert st.k_gemm % 64 == 0
        ws = st._wcache["staged"][1]
        assert ws.dtype == torch.uint8 and ws.shape == (st.k_gemm // 64, N, 32)
        assert lin(x) is not None and st._wcache["staged"][1] is ws  # built once
