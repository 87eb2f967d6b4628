"""Config C4 (the Flux-dev denoise step, bench_flux.FluxStep) at reduced depth:
one double-stream and one single-stream block at the step's full token counts
(4096 image + 512 text tokens, bf16), with the step's fusions -- the adaptive
LayerNorm in the qkv / MLP-up prep, the GELU-tanh epilogue of MLP-up, the
single block's proj + MLP-down residual epilogue -- and its M = 1
modulation GEMVs (W4A8 for the double block, W4A16 for the single block).

  * every quantized linear call of the eager forward: INT8 codes and scales
    bit-exact against the oracle's prep (with the normalisation where fused),
    outputs bit-exact against the oracle's accumulators and epilogue formula
    (activation outputs within the f32-evaluation bound of the epilogue tests;
    grouped split-K launches within the slice-order bound), on sampled rows;
  * each block's output against the same model whose quantized linears are
    the fp32 dequant -> F.linear fallback (fp32 prep, fp32 weights q * s):
    cosine >= 0.9999;
  * the step captured into a hipGraph: every replay equals the eager output.

Reference: the ops-layer linear forward _ops.py:817-862 (W4A8 :443-464,
W4A16 :466-481), the fallback _ops.py:483-491 with the group layout of
_quant_utils.py:237-270.
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import bench_flux as bf

pytestmark = pytest.mark.gpu

BF16 = 1
ROWS = {1: [0], bf.TXT_TOKENS: [0, 1, 255, 256, 511],
        bf.IMG_TOKENS: [0, 1, 255, 256, 2047, 3840, 4095],
        bf.IMG_TOKENS + bf.TXT_TOKENS: [0, 511, 512, 2048, 4095, 4096, 4352, 4607]}


@pytest.fixture(scope="module")
def flux(rt, dev):
    torch.backends.cuda.matmul.allow_tf32 = False
    return bf.FluxStep(rt, dev, seed=0, n_double=1, n_single=1)


def _cos(a, b):
    a = a.reshape(-1).double()
    b = b.reshape(-1).double()
    return float((a @ b) / (a.norm() * b.norm()))


def _ulp_bf16(ref):
    e = np.floor(np.log2(np.maximum(np.abs(ref).astype(np.float64), 2.0 ** -126)))
    return 2.0 ** (e - 7)


def _record(monkeypatch):
    """Wrap the step's linear entry points so that every call's inputs and
    outputs are kept (cloned; the forward runs eagerly)."""
    calls = []
    oq, onq, og, o16 = bf.QLinear.quantize, bf.QLinear.norm_quantize, bf.QLinear.gemm, bf.W4A16Linear.__call__

    def quantize(self, rt, x, q_out=None, s_out=None):
        q, s = oq(self, rt, x, q_out, s_out)
        calls.append(dict(kind="prep", layer=self, x=x.clone(), q=q.clone(), s=s.clone()))
        return q, s

    def norm_quantize(self, rt, x, weight, bias, q_out=None, s_out=None):
        q, s = onq(self, rt, x, weight, bias, q_out, s_out)
        calls.append(dict(kind="norm_prep", layer=self, x=x.clone(), w=weight.clone(), b=bias.clone(),
                          q=q.clone(), s=s.clone()))
        return q, s

    def gemm(self, rt, q, s_a, act, out=None, activation=0, residual=None):
        o = og(self, rt, q, s_a, act, out=out, activation=activation, residual=residual)
        calls.append(dict(kind="gemm", layer=self, q=q.clone(), s=s_a.clone(), out=o.clone(), act=activation,
                          res=None if residual is None else residual.clone()))
        return o

    def w4a16(self, rt, x):
        o = o16(self, rt, x)
        calls.append(dict(kind="w4a16", layer=self, x=x.clone(), out=o.clone()))
        return o

    monkeypatch.setattr(bf.QLinear, "quantize", quantize)
    monkeypatch.setattr(bf.QLinear, "norm_quantize", norm_quantize)
    monkeypatch.setattr(bf.QLinear, "gemm", gemm)
    monkeypatch.setattr(bf.W4A16Linear, "__call__", w4a16)
    return calls


def _prep_kw(layer):
    return dict(smoothrot=layer.sr.fdt.cpu(), rot_size=bf.ROT_SIZE, w_in=layer.K, perm=layer.perm.cpu().long())


def test_flux_step_linears_match_oracle(rt, oracle, flux, monkeypatch):
    calls = _record(monkeypatch)
    with torch.no_grad():
        flux.forward()
    torch.cuda.synchronize()
    monkeypatch.undo()
    kinds = [c["kind"] for c in calls]
    # 1 double block: 2 modulation GEMVs + 2 streams x 4 linears; 1 single block: 4 linears + 1 W4A16 GEMV
    assert kinds.count("gemm") == 14 and kinds.count("w4a16") == 1
    assert kinds.count("norm_prep") == 6 and kinds.count("prep") == 8
    seen_act = seen_res = 0
    for c in calls:
        L = c["layer"]
        if c["kind"] in ("prep", "norm_prep"):
            M = c["x"].shape[0]
            rows = torch.tensor(ROWS[M])
            x = c["x"][rows.to(c["x"].device)].cpu()
            if c["kind"] == "prep":
                q_ref, s_ref = oracle.rotate_quantize(x, BF16, **_prep_kw(L))
            else:
                q_ref, s_ref = oracle.norm_rotate_quantize(x, BF16, "layer", weight=c["w"].cpu().numpy(),
                                                           bias=c["b"].cpu().numpy(), eps=1e-6, **_prep_kw(L))
            tag = f"{c['kind']} M={M} K={L.K}"
            assert np.array_equal(c["s"][rows.to(c["s"].device)].cpu().numpy(), s_ref), tag
            assert np.array_equal(c["q"][rows.to(c["q"].device)].cpu().numpy(), q_ref), tag
        elif c["kind"] == "gemm":
            M, K, N = c["q"].shape[0], L.K, L.N
            G = K // bf.GROUP
            rows = torch.tensor(ROWS[M])
            dr = rows.to(c["q"].device)
            acc = oracle.gemm_acc(c["q"][dr].cpu().numpy(), oracle.unpack_int4(L.w.cpu().numpy(), K), G)
            s_a = c["s"][dr].cpu().numpy()
            s_w = L.s_w.cpu().numpy()
            v32 = oracle.epilogue(acc, s_a, s_w, L.b.float().cpu().numpy(), 2)
            r = None if c["res"] is None else c["res"][dr].float().cpu().numpy()
            out = c["out"][dr].float().cpu().numpy()
            tag = f"gemm M={M} K={K} N={N} act={c['act']} res={r is not None}"
            split = rt.lib().ic_gemm_splitk_bytes(M, N, K, G, 1) > 0
            if c["act"] == 0 and not split:
                s = v32 if r is None else v32 + r.astype(np.float32)
                assert np.array_equal(out, oracle.round_dtype(s.astype(np.float64), BF16)), tag
                seen_res += r is not None
                continue
            v = v32.astype(np.float64)
            act_v = oracle.activate(v, c["act"])
            ref = oracle.round_dtype(act_v if r is None else act_v + r, BF16)
            bound = 2.0 ** -20 * (np.abs(v) + np.abs(act_v) + (0 if r is None else np.abs(r))) + _ulp_bf16(ref)
            if split:
                # slices of the group fold added in slice order: within G * 2^-23 of
                # the sum of the absolute group terms (as the split-K tests bound it)
                T = (np.abs(acc).astype(np.float64) * s_w.T.astype(np.float64)[:, None, :]).sum(0)
                bound = bound + G * 2.0 ** -23 * T * s_a.astype(np.float64)[:, None] * (1 + 2.0 ** -8)
            err = np.abs(out.astype(np.float64) - ref)
            assert (err <= bound).all(), f"{tag}: {int((err > bound).sum())} outside, worst {err.max():.3g}"
            seen_act += c["act"] != 0
        else:  # W4A16 modulation GEMV (M = 1): fp32 accumulation in another order
            w = torch.from_numpy(oracle.dequant_w4a16(L.w.cpu().numpy(), L.s_w.cpu().numpy(), L.K, BF16))
            ref = c["x"].float().cpu() @ w.t() + L.b.float().cpu()
            got = c["out"].float().cpu()
            assert torch.allclose(got, ref, rtol=2e-2, atol=2e-2 * ref.abs().max().item() * 1e-2)
            assert _cos(got, ref) >= 0.9999
    assert seen_act == 3 and seen_res == 1  # three MLP-up GELU epilogues, the single block's residual


# ---------------------------------------------------------------- fp32 fallback model
def _hadamard(R, dev):
    h4 = torch.tensor([[1., 1., 1., -1.], [1., 1., -1., 1.], [1., -1., 1., 1.], [-1., 1., 1., 1.]]) / 2
    H = h4
    while H.shape[0] < R:
        H = torch.kron(H, h4)
    return H.to(dev)


def _fallback_linear(oracle, cache):
    """The reference's PyTorch fallback for one layer, in fp32 on the GPU:
    W = q * s[n, k // 128], x -> x / f -> block Hadamard -> perm -> F.linear."""

    def weight(layer):
        if id(layer) not in cache:
            q = torch.from_numpy(oracle.unpack_int4(layer.w.cpu().numpy(), layer.K)).float()
            s = layer.s_w.cpu().repeat_interleave(bf.GROUP, dim=1)
            cache[id(layer)] = (q * s).to(layer.w.device)
        return cache[id(layer)]

    def prep(layer, x):
        x2 = x.float()
        if layer.rotated:
            x2 = x2 / layer.sr.fdt
            M = x2.shape[0]
            Ht = _hadamard(bf.ROT_SIZE, x2.device).t().contiguous()
            x2 = (x2.reshape(M, -1, bf.ROT_SIZE) @ Ht).reshape(M, -1)
            x2 = x2[:, layer.perm.long()]
        return x2

    def linear(layer, x, activation=0, residual=None):
        y = F.linear(prep(layer, x), weight(layer), layer.b.float())
        if activation == bf.GELU_TANH:
            y = F.gelu(y, approximate="tanh")
        if residual is not None:
            y = y + residual.float()
        return y.to(x.dtype)

    return linear


def test_flux_step_blocks_vs_fp32_fallback(rt, oracle, flux, monkeypatch):
    with torch.no_grad():
        got = []
        out = flux.forward(collect=got)
        linear = _fallback_linear(oracle, {})

        def norm_call(self, rt_, x, weight, bias, activation=0):
            y = (F.layer_norm(x.float(), (x.shape[-1],), eps=1e-6) * weight + bias).to(x.dtype)
            return linear(self, y, activation)

        monkeypatch.setattr(bf.QLinear, "norm_call", norm_call)
        monkeypatch.setattr(bf.QLinear, "__call__", lambda self, rt_, x, residual=None: linear(self, x, 0, residual))
        monkeypatch.setattr(bf.W4A16Linear, "__call__", lambda self, rt_, x: linear(self, x))
        monkeypatch.setattr(bf.FluxStep, "_mod_w4a8", lambda self, layer, v: linear(layer, v).chunk(6, dim=-1))
        ref = []
        ref_out = flux.forward(collect=ref)
    torch.cuda.synchronize()
    pairs = [("double img", got[0][0], ref[0][0]), ("double txt", got[0][1], ref[0][1]),
             ("single", got[1], ref[1]), ("final", out, ref_out)]
    for name, a, b in pairs:
        assert torch.isfinite(a).all(), name
        c = _cos(a, b)
        assert c >= 0.9999, f"{name}: cosine {c:.6f} against the fp32 fallback model"


def test_flux_step_graph_replay_equals_eager(flux):
    with torch.no_grad():
        flux.forward()
        torch.cuda.synchronize()
        eager = flux.forward().clone()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = flux.forward()
        for i in range(3):
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), f"replay {i}"
            flux.forward()  # eager work between replays
            torch.cuda.synchronize()
        assert torch.isfinite(eager).all()


def test_dropin_ops_step_matches_fused_step(rt, flux):
    """The C4 step through the drop-in ops layer (IntCrushOps.Linear for every
    quantized linear, torch adaLN / GELU / residuals between them) computes
    the same function as the fused step: each block's output within cosine
    0.9999 (the fused prep rounds the normalised activations once, the
    unfused path twice; the fused GELU is evaluated in f32, torch's in bf16),
    and its hipGraph replays equal its eager output."""
    dropin = bf.DropInFluxStep(rt, flux.dev, seed=0, n_double=1, n_single=1)
    with torch.no_grad():
        got, ref = [], []
        out = dropin.forward(collect=got)
        ref_out = flux.forward(collect=ref)
        torch.cuda.synchronize()
        for name, a, b in (("double img", got[0][0], ref[0][0]), ("double txt", got[0][1], ref[0][1]),
                           ("single", got[1], ref[1]), ("final", out, ref_out)):
            assert torch.isfinite(a).all(), name
            assert _cos(a, b) >= 0.9999, f"{name}: cosine {_cos(a, b):.6f}"
        eager = dropin.forward().clone()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            o = dropin.forward()
        for _ in range(2):
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(o, eager)
    # the W4A16-bias switch the drop-in step needs is scoped to its forward
    assert "INTCRUSH_W4A16_BIAS" not in os.environ
