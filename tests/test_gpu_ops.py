"""The drop-in Linear on the GPU: every forward path runs the gfx950 kernels
and matches the CPU oracle (bit-exact where the path is integer up to the
fp32 epilogue, tolerance where the reference itself is a float GEMM)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import __graft_entry__
from _layers import int4_layer, int8_layer, load_linear

pytestmark = pytest.mark.gpu

ops_mod = __graft_entry__._submodule("_ops")
DT = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}


def _cos(a, b):
    a = a.reshape(-1).double()
    b = b.reshape(-1).double()
    return float((a @ b) / (a.norm() * b.norm()))


def _x(M, K, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    idx = torch.randperm(K, generator=g)[: max(1, K // 100)]
    x[:, idx] *= 20
    return x.to(dtype)


def _to_dev(lin, dev):
    """Move a loaded Linear's tensors to the GPU (as ComfyUI's model
    management does for the weights)."""
    import comfy.quant_ops as qo

    w = lin.weight
    lin.weight = torch.nn.Parameter(w.to(dev), requires_grad=False) if not hasattr(w, "_qdata") else \
        torch.nn.Parameter(qo.QuantizedTensor(w._qdata.to(dev), w._layout_type, type(w._params)(
            scale=w._params.scale.to(dev), orig_dtype=w._params.orig_dtype, orig_shape=w._params.orig_shape,
            rot_need=w._params.rot_need, rot_size=w._params.rot_size,
            perm=None if w._params.perm is None else w._params.perm.to(dev),
            zp=None if w._params.zp is None else w._params.zp.to(dev))), requires_grad=False)
    if lin.bias is not None:
        lin.bias = torch.nn.Parameter(lin.bias.to(dev), requires_grad=False)
    for name in ("_intcrush_perm", "_intcrush_smooth", "_intcrush_smoothrot_factors", "_intcrush_L1",
                 "_intcrush_L2"):
        t = getattr(lin, name)
        if t is not None:
            setattr(lin, name, t.to(dev))
    lin._intcrush_invalidate()
    return lin


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("G", [1, 4])
def test_w4a8_layer_bit_exact(oracle, dev, dtype, G):
    """Rotated INT4 layer: fused prep+quant + W4A8 GEMM == oracle integer
    pipeline + fp32 epilogue, bit for bit."""
    M, K, N, R = 37, 512, 96, 64
    ops = ops_mod.make_intcrush_ops("int4_crush", R)
    sd = int4_layer(N, K, G=G, seed=1)
    lin = _to_dev(load_linear(ops, "double_blocks.0.img_mlp.2", sd, K, N), dev)
    x = _x(M, K, dtype, 2)
    out = lin(x.to(dev).reshape(1, M, K)).reshape(M, N).float().cpu().numpy()
    y = oracle.prepare(x, DT[dtype], smoothrot=sd["weight_smoothrot_factors"], rot_size=R, w_in=K,
                       perm=sd["weight_perm"])
    q, s = oracle.quantize(y)
    acc = oracle.gemm_acc(q, oracle.unpack_int4(sd["weight"].numpy(), K), G)
    ref = oracle.epilogue(acc, s, sd["weight_scale"].float().numpy(), sd["bias"].float().numpy(), DT[dtype])
    assert np.array_equal(out, ref)


def test_w4a16_layer_non_rotated(oracle, dev):
    """`modulation` layers are not rotated -> W4A16; bias ignored as in the
    reference (_ops.py:474)."""
    M, K, N = 5, 768, 64
    ops = ops_mod.make_intcrush_ops("int4_crush", 256)
    sd = int4_layer(N, K, G=6, seed=3, perm=True, smoothrot=True)
    lin = _to_dev(load_linear(ops, "single_blocks.0.modulation.lin", sd, K, N), dev)
    assert not lin._intcrush_rot_need
    x = _x(M, K, torch.float16, 4)
    out = lin(x.to(dev)).float().cpu()
    y = oracle.prepare(x, 0, smoothrot=sd["weight_smoothrot_factors"], rot_size=0, w_in=K, perm=sd["weight_perm"])
    w = oracle.dequant_w4a16(sd["weight"].numpy(), sd["weight_scale"].float().numpy(), K, 0)
    ref = torch.from_numpy(y) @ torch.from_numpy(w).t()
    assert _cos(out, ref) >= 0.99999
    assert torch.allclose(out, ref, rtol=1e-2, atol=1e-2 * float(ref.abs().max()))


def test_int8_graph_replays_match_eager(oracle, dev):
    """INT8 layers replay a hipGraph of prep+quantize+GEMM.  Every replay,
    with eager GPU work and synchronisation in between, equals the eager
    result; the LRU keeps four shapes; a new bias object re-captures."""
    K, N, R = 512, 128, 256
    ops = ops_mod.make_intcrush_ops("int8_crush", R)
    sd = int8_layer(N, K, seed=5, perm=True, smoothrot=True)
    lin = _to_dev(load_linear(ops, "double_blocks.0.img_attn.qkv", sd, K, N), dev)
    rt = __graft_entry__._submodule("_hip_runtime")
    assert rt.USE_CUDA_GRAPHS
    xs = [_x(64, K, torch.float16, 10 + i).to(dev) for i in range(4)]
    eager = []
    for x in xs:  # first call of a shape runs eagerly and captures
        eager.append(lin(x).clone())
    runner = lin._graph_runner
    assert runner is not None and len(runner.cached_keys()) == 1
    for rep in range(3):
        for x, e in zip(xs, eager):
            y = lin(x)
            torch.cuda.synchronize()
            assert torch.equal(y, e), f"replay {rep} differs from eager"
            _ = torch.randn(1000, device=dev) * 2  # unrelated eager work between replays
    # reference for the eager result
    y_ref = oracle.prepare(xs[0].cpu(), 0, smoothrot=sd["weight_smoothrot_factors"], rot_size=R, w_in=K,
                           perm=sd["weight_perm"])
    q, s = oracle.quantize(y_ref)
    ref = oracle.epilogue(oracle.gemm_acc(q, sd["weight"].numpy()), s, sd["weight_scale"].float().numpy(),
                          sd["bias"].float().numpy(), 0)
    assert np.array_equal(eager[0].float().cpu().numpy(), ref)
    for M in (16, 32, 48, 80, 96):
        lin(_x(M, K, torch.float16, M).to(dev))
    assert len(runner.cached_keys()) == 4
    lin.bias = torch.nn.Parameter(lin.bias.clone(), requires_grad=False)
    y = lin(xs[1])
    assert torch.equal(y, eager[1])


def test_int8_zero_point_eager(dev):
    K, N = 256, 64
    ops = ops_mod.make_intcrush_ops("int8_crush", 0)
    sd = int8_layer(N, K, seed=6, zp=True)
    lin_cpu = load_linear(ops, "blk.fc", sd, K, N)
    lin = _to_dev(load_linear(ops, "blk.fc", sd, K, N), dev)
    # no rotation here, so use outlier-free N(0,1) activations (the C1 setting):
    # per-token INT8 of rows with x20 outliers is the error the rotation removes
    x = torch.randn(33, K, generator=torch.Generator().manual_seed(7)).to(torch.float16)
    out = lin(x.to(dev)).float().cpu()
    assert lin._graph_runner is None
    W = (sd["weight"].float() - sd["weight_zp"].reshape(-1, 1)) * sd["weight_scale"].float().reshape(-1, 1)
    ref = x.float() @ W.t() + sd["bias"].float()  # fp32 dequant -> linear
    assert _cos(out, ref) >= 0.9999
    del lin_cpu


def test_svd_residual_and_zero_point_w4a8(dev):
    M, K, N, R = 24, 512, 64, 64
    ops = ops_mod.make_intcrush_ops("int4_crush", R)
    sd = int4_layer(N, K, G=4, seed=8, zp=True, svd_rank=8)
    lin_cpu = load_linear(ops, "blk.fc", sd, K, N)
    lin = _to_dev(load_linear(ops, "blk.fc", sd, K, N), dev)
    x = _x(M, K, torch.float16, 9)
    out = lin(x.to(dev)).float().cpu()
    ref = lin_cpu(x.float())
    ref = ref + 0  # fp32 reference fallback incl. residuals, drops bias on this path
    ref = ref + sd["bias"].float()  # the W4A8 path keeps the bias (_ops.py:455-457)
    assert _cos(out, ref) >= 0.9999


def _lora(N, K, rank, seed):
    """A standard LoRA adapter as ComfyUI hands it over (name, weights
    (up [N, r], down [r, K], alpha))."""
    import types

    g = torch.Generator().manual_seed(seed)
    up = torch.randn(N, rank, generator=g) * 0.05
    down = torch.randn(rank, K, generator=g) * 0.05
    return types.SimpleNamespace(name="lora", weights=(up, down, float(rank) / 2))


def _attach(lin, adapter, strength):
    lin._intcrush_adapter = adapter
    lin._intcrush_lora_strength = strength
    lin._intcrush_adapter_ready = False


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_folded_residuals_w4a8(dev, dtype):
    """Zero point, SVD branch and a standard LoRA reach the W4A8 GEMM as one
    residual: the output is round(f32 GEMM + residual) bit for bit, stays
    within two output ulps of the reference's one-addmm_-per-term order, and
    matches the fp32 fallback with the same corrections."""
    rt = __graft_entry__._submodule("_hip_runtime")
    M, K, N, R = 40, 512, 96, 64
    ops = ops_mod.make_intcrush_ops("int4_crush", R)
    sd = int4_layer(N, K, G=4, seed=21, zp=True, svd_rank=8)
    lin_cpu = load_linear(ops, "blk.fc", sd, K, N)
    lin = _to_dev(load_linear(ops, "blk.fc", sd, K, N), dev)
    _attach(lin, _lora(N, K, 16, 22), 0.8)
    _attach(lin_cpu, _lora(N, K, 16, 22), 0.8)
    x = _x(M, K, dtype, 23).to(dev)
    out = lin(x)
    # the same pieces by hand: GEMM in f32, the folded residual, one rounding
    params = lin.weight._params
    st = lin._intcrush_state(x)
    kw = dict(rot_size=R, w_in=lin._intcrush_w_in, smoothrot=st.smoothrot, perm=st.perm)
    x_prep = rt.prepare_activation(x, **kw)
    q, s_a = rt.rotate_quantize(x, **kw)
    res, lora = lin._fold_linear_residuals(x, x_prep, params, dtype, x_prep)
    assert lora and res.dtype == dtype and tuple(res.shape) == (M, N)
    v = rt.gemm_w4a8(q, lin.weight._qdata, params.scale, s_a, bias=lin.bias, out_dtype=torch.float32)
    assert torch.equal(out, (v + res.float()).to(dtype))
    # the reference's order: GEMM rounded, then each correction by its own addmm_
    # (four roundings to the dtype where the fold has two): against the exact
    # float64 sum the fold is no less accurate
    plain = rt.gemm_w4a8(q, lin.weight._qdata, params.scale, s_a, bias=lin.bias, out_dtype=dtype)
    lin._zp_correction(plain, x_prep, params.scale, params.zp)
    plain = lin._apply_residuals(x, plain, x_prep=x_prep)
    xd, xpd = x.double(), x_prep.double()
    G = params.scale.reshape(N, -1).shape[1]
    zt = xpd.reshape(M, G, -1).sum(-1) @ (params.scale.reshape(N, G).double() * params.zp.double().reshape(-1, 1)).t()
    L1, L2 = lin._intcrush_L1.double(), lin._intcrush_L2.double()
    up, down, alpha = (t.double() if torch.is_tensor(t) else t for t in lin._intcrush_adapter.weights)
    exact = v.double() - zt + (xpd @ L2.t()) @ L1.t() + (alpha / 16 * 0.8) * ((xd @ down.t()) @ up.t())
    e_fold = (out.double() - exact).abs()
    e_plain = (plain.double() - exact).abs()
    assert e_fold.mean() <= 1.05 * e_plain.mean(), (e_fold.mean().item(), e_plain.mean().item())
    ref = lin_cpu(x.float().cpu()) + sd["bias"].float()  # fp32 fallback (it drops the bias)
    assert _cos(out.float().cpu(), ref) >= 0.9999


def test_folded_residuals_int8_eager(dev):
    """INT8 with a zero point runs eagerly; the zero-point term and a LoRA
    go through the GEMM's residual epilogue, the SVD branch on the raw input
    as the reference's INT8 path has it."""
    rt = __graft_entry__._submodule("_hip_runtime")
    M, K, N = 33, 256, 64
    ops = ops_mod.make_intcrush_ops("int8_crush", 0)
    sd = int8_layer(N, K, seed=24, zp=True)
    lin = _to_dev(load_linear(ops, "blk.fc", sd, K, N), dev)
    _attach(lin, _lora(N, K, 8, 25), 1.0)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(26)).to(torch.float16)
    out = lin(x.to(dev))
    assert lin._graph_runner is None
    params = lin.weight._params
    st = lin._intcrush_state(x.to(dev))
    x2 = x.to(dev)
    x_prep = rt.prepare_activation(x2, rot_size=0, w_in=lin._intcrush_w_in, smoothrot=st.smoothrot, perm=st.perm,
                                   smooth=st.smooth)
    q, s_a = rt.rotate_quantize(x2, rot_size=0, w_in=lin._intcrush_w_in, smoothrot=st.smoothrot, perm=st.perm,
                                smooth=st.smooth)
    res, lora = lin._fold_linear_residuals(x2, x_prep, params, torch.float16, x2)
    assert lora
    v = rt.fused_int8_gemm_dequant(q, lin.weight._qdata, params.scale, s_a, bias=lin.bias, out_dtype=torch.float32)
    assert torch.equal(out, (v + res.float()).to(torch.float16))
    up, down, alpha = _lora(N, K, 8, 25).weights
    W = (sd["weight"].float() - sd["weight_zp"].reshape(-1, 1)) * sd["weight_scale"].float().reshape(-1, 1)
    ref = x.float() @ W.t() + sd["bias"].float() + (alpha / 8) * ((x.float() @ down.t()) @ up.t())
    assert _cos(out.float().cpu(), ref) >= 0.9999


def test_gpu_forward_refuses_silent_fallback(dev, monkeypatch):
    ops = ops_mod.make_intcrush_ops("int4_crush", 64)
    lin = _to_dev(load_linear(ops, "blk.fc", int4_layer(16, 256, seed=11), 256, 16), dev)
    rt = __graft_entry__._submodule("_hip_runtime")
    monkeypatch.setattr(rt, "KERNELS_AVAILABLE", False)
    monkeypatch.delenv("INTCRUSH_ALLOW_TORCH_FALLBACK", raising=False)
    with pytest.raises(RuntimeError, match="refusing a silent PyTorch"):
        lin(torch.randn(2, 256, device=dev, dtype=torch.float16))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fused_quant_int8_gemm_dequant(rt, oracle, dev, dtype):
    """fused_quant_int8_gemm_dequant (kernels/triton_int8_gemm.py:331-389):
    per-token quantization of x then the W8A8 GEMM; equals the oracle's
    quantize -> accumulators -> epilogue bit for bit."""
    M, K, N = 300, 1024, 384
    g = torch.Generator().manual_seed(70)
    x = (torch.randn(M, K, generator=g) * 3).to(dtype)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    s_w = (torch.rand(N, generator=g) * 2e-3 + 1e-4).to(torch.float16).float()
    bias = torch.randn(N, generator=g).to(dtype)
    out = rt.fused_quant_int8_gemm_dequant(x.to(dev), w.to(dev), s_w.to(dev), bias=bias.to(dev), out_dtype=dtype)
    q, s = oracle.quantize(oracle.to_dtype_values(x, DT[dtype]))
    ref = oracle.epilogue(oracle.gemm_acc(q, w.numpy()), s, s_w.numpy(), bias.float().numpy(), DT[dtype])
    assert np.array_equal(out.float().cpu().numpy(), ref)


@pytest.mark.parametrize("zp", [False, True])
def test_int8_layer_use_fused_w8a8(oracle, dev, monkeypatch, zp):
    """The USE_FUSED_W8A8 branch of the INT8 forward (_ops.py:546-558): the
    prepared activation goes through fused_quant_int8_gemm_dequant, then the
    zero-point term when present.  Graphs are off so the eager branch runs."""
    rt = __graft_entry__._submodule("_hip_runtime")
    monkeypatch.setattr(rt, "USE_FUSED_W8A8", True)
    monkeypatch.setattr(rt, "USE_CUDA_GRAPHS", False)
    M, K, N, R = 48, 512, 160, 256
    ops = ops_mod.make_intcrush_ops("int8_crush", R)
    sd = int8_layer(N, K, seed=71, perm=True, smoothrot=True, zp=zp)
    lin = _to_dev(load_linear(ops, "double_blocks.1.img_attn.qkv", sd, K, N), dev)
    x = _x(M, K, torch.bfloat16, 72)
    out = lin(x.to(dev)).float().cpu()
    y = oracle.prepare(x, DT[torch.bfloat16], smoothrot=sd["weight_smoothrot_factors"], rot_size=R, w_in=K,
                       perm=sd["weight_perm"])
    q, s = oracle.quantize(y)
    s_w = sd["weight_scale"].float().numpy()
    ref = oracle.epilogue(oracle.gemm_acc(q, sd["weight"].numpy()), s, s_w, sd["bias"].float().numpy(),
                          DT[torch.bfloat16])
    if not zp:
        assert lin._graph_runner is None
        assert np.array_equal(out.numpy(), ref)
        return
    # zero point: out -= (sum_k x_prep) * (s * zp), one rounding of the bf16 output
    corr = y.astype(np.float64).sum(1)[:, None] * (s_w.reshape(-1) * sd["weight_zp"].numpy())[None, :]
    exact = ref.astype(np.float64) - corr
    assert _cos(out, torch.from_numpy(exact)) >= 0.9999
    assert np.allclose(out.numpy(), exact, rtol=2e-2, atol=2e-2 * np.abs(exact).max() * 1e-2)


@pytest.mark.parametrize("dtype,K", [(torch.bfloat16, 20480), (torch.float32, 12288)])
def test_w4a8_layer_wider_than_one_workgroup(oracle, dev, dtype, K):
    """Rotated INT4 layers whose rows are wider than the single-pass prep
    holds (20480 bf16 values, 12288 f32 values) through the ops Linear:
    the chunked rotation + second pass, then the W4A8 GEMM.  bf16: bit-exact
    against the oracle chain; f32: within the fp32 fallback's tolerance."""
    M, N, R = 24, 256, 256
    ops = ops_mod.make_intcrush_ops("int4_crush", R)
    sd = int4_layer(N, K, seed=90)
    lin = _to_dev(load_linear(ops, "single_blocks.0.linear2", sd, K, N), dev)
    x = _x(M, K, dtype, 91)
    out = lin(x.to(dev)).float().cpu()
    y = oracle.prepare(x, DT[dtype], smoothrot=sd["weight_smoothrot_factors"], rot_size=R, w_in=K,
                       perm=sd["weight_perm"])
    q, s = oracle.quantize(y)
    ref = oracle.epilogue(oracle.gemm_acc(q, oracle.unpack_int4(sd["weight"].numpy(), K), K // 128), s,
                          sd["weight_scale"].float().numpy(), sd["bias"].float().numpy(), DT[dtype])
    if dtype == torch.bfloat16:
        assert np.array_equal(out.numpy(), ref)
    else:
        assert _cos(out, torch.from_numpy(ref)) >= 0.9999


# ------------------------------------------------------------------ K not a multiple of 128
@pytest.mark.parametrize("K,G,R", [(64, 1, 64), (96, 3, 16), (320, 10, 64), (64, 2, 0)])
def test_narrow_layers_take_the_mfma_kernels(oracle, dev, K, G, R):
    """Layers whose prepared width is not a multiple of 128 (e.g. a 64-wide
    patch embedding) run the MFMA kernels at the next multiple of
    lcm(128, group size): zero weights, zero codes and scale-1 groups in the
    extra columns.  Bit-exact against the oracle over the real columns, and no
    scalar-kernel warning is logged."""
    rt = __graft_entry__._submodule("_hip_runtime")
    M, N = 40, 96
    ops = ops_mod.make_intcrush_ops("int4_crush", R if R else 256)
    sd = int4_layer(N, K, G=G, seed=120 + K)
    name = "double_blocks.0.img_mlp.2" if R else "double_blocks.0.img_mod.modulation"
    lin = _to_dev(load_linear(ops, name, sd, K, N), dev)
    assert lin._intcrush_rot_need == bool(R)
    x = _x(M, K, torch.bfloat16, 121)
    before = set(rt._SCALAR_WARNED)
    out = lin(x.to(dev)).float().cpu().numpy()
    st = lin._intcrush_state(x.to(dev))
    assert st.k_gemm % 128 == 0 and st.k_gemm > K
    assert set(rt._SCALAR_WARNED) == before
    if R:  # W4A8
        y = oracle.prepare(x, 1, smoothrot=sd["weight_smoothrot_factors"], rot_size=R, w_in=K,
                           perm=sd["weight_perm"])
        q, s = oracle.quantize(y)
        acc = oracle.gemm_acc(q, oracle.unpack_int4(sd["weight"].numpy(), K), G)
        ref = oracle.epilogue(acc, s, sd["weight_scale"].float().numpy(), sd["bias"].float().numpy(), 1)
        assert np.array_equal(out, ref)
    else:  # W4A16 (unrotated INT4)
        y = oracle.prepare(x, 1, smoothrot=sd["weight_smoothrot_factors"], rot_size=0, w_in=K,
                           perm=sd["weight_perm"])
        w = oracle.dequant_w4a16(sd["weight"].numpy(), sd["weight_scale"].float().numpy(), K, 1)
        ref = torch.from_numpy(y) @ torch.from_numpy(w).t()
        assert _cos(torch.from_numpy(out), ref) >= 0.9999


def test_narrow_int8_layer_graph_replays(oracle, dev):
    """A 64-wide INT8 layer: the hipGraph runner runs prep + GEMM at 128
    columns; every replay equals the oracle."""
    rt = __graft_entry__._submodule("_hip_runtime")
    K, N = 64, 128
    ops = ops_mod.make_intcrush_ops("int8_crush", 64)
    sd = int8_layer(N, K, seed=130, perm=True, smoothrot=True)
    lin = _to_dev(load_linear(ops, "double_blocks.0.img_attn.qkv", sd, K, N), dev)
    x = _x(48, K, torch.float16, 131).to(dev)
    before = set(rt._SCALAR_WARNED)
    first = lin(x).clone()
    for _ in range(3):
        y = lin(x)
        torch.cuda.synchronize()
        assert torch.equal(y, first)
    assert set(rt._SCALAR_WARNED) == before
    yp = oracle.prepare(x.cpu(), 0, smoothrot=sd["weight_smoothrot_factors"], rot_size=64, w_in=K,
                        perm=sd["weight_perm"])
    q, s = oracle.quantize(yp)
    ref = oracle.epilogue(oracle.gemm_acc(q, sd["weight"].numpy()), s, sd["weight_scale"].float().numpy(),
                          sd["bias"].float().numpy(), 0)
    assert np.array_equal(first.float().cpu().numpy(), ref)
