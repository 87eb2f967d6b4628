"""One denoise step of a random-init Flux-dev-style DiT on one MI355X, the
workload behind `bench.py --config c4step`.

Model (batch 1, bf16, 4096 image + 512 text tokens, hidden 3072, 24 heads of
128, MLP 12288): embedders, 19 double-stream blocks, 38 single-stream blocks
and the final layer, run as one forward.  Every block linear (qkv
3072->9216, proj 3072->3072, MLP 3072->12288->3072; each stream of a double
block has its own) is an INT4 W4A8 linear through the library, the way the
INT4 ops layer runs it when a rotation is configured (_ops.py:443-461): the
fused rotate+quantize kernel (SmoothRot divide, Hadamard R=256, PermuQuant
gather, per-token INT8 codes) and then the W4A8 GEMM with group-128 scales
and the bias in its epilogue.  The M = 1 modulation linears 3072->18432 run
the GEMV kernels: double-block img_mod/txt_mod as rotated W4A8, single-block
modulation as W4A16 (the naming rule of _ops.py:30-32 and :699-706 leaves
a layer whose name contains "modulation" unrotated, and :843-851 sends an
unrotated INT4 layer to W4A16).  Attention is torch's SDPA on its flash or
memory-efficient backend.  The adaptive LayerNorm in front of qkv and MLP-up
(LayerNorm without affine, then (1 + scale) * . + shift from the modulation)
is fused into those linears' prep: one norm_rotate_quantize launch per linear
reads the block input and writes its INT8 codes.  The MLP's GELU (tanh form)
is the MLP-up GEMM's epilogue activation, and the single block's
proj(attn) + down(h) sum is the MLP-down GEMM's residual epilogue.  QK
RMSNorm, RoPE, residual gates, the embedders and the final layer are torch
ops in bf16 (the embedders and final layer are unquantized bf16 linears).

The single-stream block's fused linear1/linear2 are the config's separate
qkv + MLP-up and proj + MLP-down linears; proj(attn) + down(gelu(up)) equals
linear2 applied to the concatenation.  Weights are random: INT4 codes
uniform over all 256 byte values, fp16-representable group scales
U(1e-3, 2e-2), SmoothRot factors exp(N(0, 0.5)) and a random permutation per
layer, small biases.

The whole step is captured once into a hipGraph and replayed; every layer
holds its own weights, so they stream from HBM as in a real step (about
4.3 GB of INT4 codes per step).
"""
from __future__ import annotations

import math
import os

HID, HEADS, HEAD_DIM, MLP = 3072, 24, 128, 12288
N_DOUBLE, N_SINGLE = 19, 38
IMG_TOKENS, TXT_TOKENS = 4096, 512
IN_CH, CTX_DIM, VEC_DIM, TIME_DIM = 64, 4096, 768, 256
ROPE_AXES, ROPE_THETA = (16, 56, 56), 10000
ROT_SIZE, GROUP = 256, 128
GELU_TANH = 3  # GEMM epilogue activation code (GELU, tanh approximation)
MOD_N = 6 * HID  # 18432
# (name, K, N) of the quantized linears of one block and stream
BLOCK_LINEARS = (("qkv", HID, 3 * HID), ("proj", HID, HID), ("mlp_up", HID, MLP), ("mlp_down", MLP, HID))


class QLinear:
    """One INT4 W4A8 linear: packed codes [N, K/2] (w, the checkpoint's nibble
    order, and wk, the K-interleaved copy the GEMM reads, as the drop-in
    Linear keeps it; w8, the codes unpacked to int8, made at the first launch
    that fills at most half the CUs, which reads it instead -- the text
    stream's 512 rows; INTCRUSH_W4_UNPACKED=0 keeps wk), fp32 group scales [N, K/128], bf16 bias, prepared
    SmoothRot factors and permutation."""

    def __init__(self, rt, K, N, gen, dev, act, rotated=True):
        import torch

        self.K, self.N = K, N
        self.w = torch.randint(0, 256, (N, K // 2), generator=gen, device=dev, dtype=torch.uint8)
        self.wk = rt.int4_interleave_k(self.w) if rotated else None
        self.w8 = None
        s = torch.rand(N, K // GROUP, generator=gen, device=dev) * (2e-2 - 1e-3) + 1e-3
        self.s_w = s.to(torch.float16).float().contiguous()
        self.b = (torch.randn(N, generator=gen, device=dev) * 0.02).to(act)
        self.rotated = rotated
        if rotated:
            self.sr = rt.prepare_factors(torch.exp(torch.randn(K, generator=gen, device=dev) * 0.5), act)
            self.perm = rt.prepare_perm(torch.randperm(K, generator=gen, device=dev), K)

    def quantize(self, rt, x, q_out=None, s_out=None):
        return rt.rotate_quantize(x, rot_size=ROT_SIZE, w_in=self.K, smoothrot=self.sr, perm=self.perm,
                                  s_a_out=s_out, x_int8_out=q_out)

    def norm_quantize(self, rt, x, weight, bias, q_out=None, s_out=None):
        """Adaptive LayerNorm (weight = 1 + scale, bias = shift) fused into the prep."""
        return rt.norm_rotate_quantize(x, norm="layer", weight=weight, bias=bias, eps=1e-6, rot_size=ROT_SIZE,
                                       w_in=self.K, smoothrot=self.sr, perm=self.perm, s_a_out=s_out,
                                       x_int8_out=q_out)

    def norm_call(self, rt, x, weight, bias, activation=0):
        q, s_a = self.norm_quantize(rt, x, weight, bias)
        return self.gemm(rt, q, s_a, x.dtype, activation=activation)

    def gemm(self, rt, q, s_a, act, out=None, activation=0, residual=None):
        if (os.environ.get("INTCRUSH_W4_UNPACKED", "1") != "0"
                and rt.w4a8_unpacked_pays(q.shape[0], self.N, self.K, self.s_w.shape[1], device=q.device)):
            if self.w8 is None:
                self.w8 = rt.unpack_int4_to_int8(self.w, self.K)
            return rt.gemm_w4a8_unpacked(q, self.w8, self.s_w, s_a, bias=self.b, out_dtype=act, out=out,
                                         activation=activation, residual=residual)
        return rt.gemm_w4a8(q, self.wk, self.s_w, s_a, bias=self.b, out_dtype=act, out=out, kil=True,
                            activation=activation, residual=residual)

    def __call__(self, rt, x, residual=None):
        q, s_a = self.quantize(rt, x)
        return self.gemm(rt, q, s_a, x.dtype, residual=residual)


class W4A16Linear(QLinear):
    """Unrotated INT4 linear on the W4A16 path (single-block modulation)."""

    def __init__(self, rt, K, N, gen, dev, act):
        super().__init__(rt, K, N, gen, dev, act, rotated=False)

    def __call__(self, rt, x):
        return rt.gemm_w4a16(x, self.w, self.s_w, bias=self.b)


class DenseLinear:
    """Unquantized bf16 linear (embedders, final layer)."""

    def __init__(self, K, N, gen, dev, act):
        import torch

        self.w = (torch.randn(N, K, generator=gen, device=dev) / math.sqrt(K)).to(act)
        self.b = (torch.randn(N, generator=gen, device=dev) * 0.02).to(act)

    def __call__(self, x):
        import torch.nn.functional as F

        return F.linear(x, self.w, self.b)


class FluxStep:
    """The step's model.  n_double / n_single shorten the block stacks (the
    tests run one block of each kind at the step's full token counts)."""

    def __init__(self, rt, dev, seed=0, n_double=N_DOUBLE, n_single=N_SINGLE):
        import torch

        self.rt, self.dev, self.act = rt, dev, torch.bfloat16
        act = self.act
        g = torch.Generator(device=dev).manual_seed(seed)

        def q(K, N):
            return QLinear(rt, K, N, g, dev, act)

        self.img_in = DenseLinear(IN_CH, HID, g, dev, act)
        self.txt_in = DenseLinear(CTX_DIM, HID, g, dev, act)
        self.time_in = (DenseLinear(TIME_DIM, HID, g, dev, act), DenseLinear(HID, HID, g, dev, act))
        self.guid_in = (DenseLinear(TIME_DIM, HID, g, dev, act), DenseLinear(HID, HID, g, dev, act))
        self.vec_in = (DenseLinear(VEC_DIM, HID, g, dev, act), DenseLinear(HID, HID, g, dev, act))
        ones = torch.ones(HEAD_DIM, device=dev, dtype=act)
        self.double = []
        for _ in range(n_double):
            blk = {"img_mod": q(HID, MOD_N), "txt_mod": q(HID, MOD_N), "qk_scale": ones}
            for stream in ("img", "txt"):
                for name, K, N in BLOCK_LINEARS:
                    blk[f"{stream}_{name}"] = q(K, N)
            self.double.append(blk)
        self.single = []
        for _ in range(n_single):
            blk = {"mod": W4A16Linear(rt, HID, MOD_N, g, dev, act), "qk_scale": ones}
            for name, K, N in BLOCK_LINEARS:
                blk[name] = q(K, N)
            self.single.append(blk)
        self.final_mod = DenseLinear(HID, 2 * HID, g, dev, act)
        self.final = DenseLinear(HID, IN_CH, g, dev, act)
        # step inputs: packed latent tokens, T5 context, CLIP pooled vector
        self.img = torch.randn(IMG_TOKENS, IN_CH, generator=g, device=dev).to(act)
        self.txt = torch.randn(TXT_TOKENS, CTX_DIM, generator=g, device=dev).to(act)
        self.y = torch.randn(1, VEC_DIM, generator=g, device=dev).to(act)
        self.t = torch.full((1,), 0.5, device=dev)
        self.guidance = torch.full((1,), 3.5, device=dev)
        side = int(math.isqrt(IMG_TOKENS))
        ids = torch.zeros(TXT_TOKENS + IMG_TOKENS, 3, device=dev)
        r = torch.arange(IMG_TOKENS, device=dev)
        ids[TXT_TOKENS:, 1] = (r // side).float()
        ids[TXT_TOKENS:, 2] = (r % side).float()
        self.ids = ids

    # ── layer inventories (for op counts and the per-part timings) ──
    def quantized_linears(self):
        """(M, layer) for every block linear of the step."""
        out = []
        for blk in self.double:
            for stream, M in (("img", IMG_TOKENS), ("txt", TXT_TOKENS)):
                for name, _, _ in BLOCK_LINEARS:
                    out.append((M, blk[f"{stream}_{name}"]))
        for blk in self.single:
            for name, _, _ in BLOCK_LINEARS:
                out.append((IMG_TOKENS + TXT_TOKENS, blk[name]))
        return out

    def modulation_linears(self):
        return [blk[k] for blk in self.double for k in ("img_mod", "txt_mod")] + [blk["mod"] for blk in self.single]

    # ── pieces of the forward ──
    @staticmethod
    def _timestep_embedding(t, dim, time_factor=1000.0):
        import torch

        half = dim // 2
        freqs = torch.exp(-math.log(10000.0) * torch.arange(half, device=t.device, dtype=torch.float32) / half)
        args = (t * time_factor)[:, None].float() * freqs[None]
        return torch.cat([torch.cos(args), torch.sin(args)], dim=-1)

    def _rope_tables(self):
        """Rotation matrices [tokens, 64, 2, 2] (fp32) of the three-axis rotary
        embedding: [[cos, -sin], [sin, cos]] per frequency pair."""
        import torch

        angles = []
        for axis, dim in enumerate(ROPE_AXES):
            omega = 1.0 / ROPE_THETA ** (torch.arange(0, dim, 2, device=self.dev, dtype=torch.float64) / dim)
            angles.append(self.ids[:, axis].double()[:, None] * omega[None])
        a = torch.cat(angles, dim=-1)
        c, s = torch.cos(a), torch.sin(a)
        return torch.stack((c, -s, s, c), dim=-1).reshape(*a.shape, 2, 2).float()

    @staticmethod
    def _apply_rope(x, freqs):
        """x [H, S, D]: rotate each (even, odd) pair by its angle, in fp32."""
        xf = x.float().reshape(*x.shape[:-1], -1, 1, 2)
        out = freqs[..., 0] * xf[..., 0] + freqs[..., 1] * xf[..., 1]
        return out.reshape(x.shape).to(x.dtype)

    @staticmethod
    def _rms_norm(x, scale):
        import torch.nn.functional as F

        return F.rms_norm(x, (HEAD_DIM,), weight=scale, eps=1e-6)

    @staticmethod
    def _modulate(x, shift, scale):
        import torch
        import torch.nn.functional as F

        return torch.addcmul(shift, F.layer_norm(x, (HID,), eps=1e-6), 1 + scale)

    def _split_heads(self, qkv, scale):
        """qkv [S, 9216] -> q, k (RMS-normed), v as [H, S, D]."""
        q, k, v = qkv.view(-1, 3, HEADS, HEAD_DIM).permute(1, 2, 0, 3)
        return self._rms_norm(q, scale), self._rms_norm(k, scale), v

    def attention(self, q, k, v, freqs):
        """Joint attention over [H, S, D] inputs; returns [S, H*D]."""
        import torch.nn.functional as F
        from torch.nn.attention import SDPBackend, sdpa_kernel

        q = self._apply_rope(q, freqs)
        k = self._apply_rope(k, freqs)
        # the math backend is excluded: its batched products in bf16 are
        # not used on this GPU
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            o = F.scaled_dot_product_attention(q[None], k[None], v.contiguous()[None])
        return o[0].transpose(0, 1).reshape(-1, HEADS * HEAD_DIM)

    def _mod_w4a8(self, layer, vec_silu):
        q, s_a = layer.quantize(self.rt, vec_silu)
        return layer.gemm(self.rt, q, s_a, self.act).chunk(6, dim=-1)

    @staticmethod
    def _ada(shift, scale):
        """(weight, bias) of the fused adaptive LayerNorm: 1 + scale and shift, f32."""
        return (1.0 + scale.float()).reshape(-1), shift.float().reshape(-1)

    def _double_block(self, blk, img, txt, vec_silu, freqs):
        import torch

        rt = self.rt
        im = self._mod_w4a8(blk["img_mod"], vec_silu)
        tm = self._mod_w4a8(blk["txt_mod"], vec_silu)
        iq, ik, iv = self._split_heads(blk["img_qkv"].norm_call(rt, img, *self._ada(im[0], im[1])), blk["qk_scale"])
        tq, tk, tv = self._split_heads(blk["txt_qkv"].norm_call(rt, txt, *self._ada(tm[0], tm[1])), blk["qk_scale"])
        attn = self.attention(torch.cat((tq, iq), 1), torch.cat((tk, ik), 1), torch.cat((tv, iv), 1), freqs)
        t_a, i_a = attn[:TXT_TOKENS], attn[TXT_TOKENS:]
        img = torch.addcmul(img, im[2], blk["img_proj"](rt, i_a))
        h = blk["img_mlp_up"].norm_call(rt, img, *self._ada(im[3], im[4]), activation=GELU_TANH)
        img = torch.addcmul(img, im[5], blk["img_mlp_down"](rt, h))
        txt = torch.addcmul(txt, tm[2], blk["txt_proj"](rt, t_a))
        h = blk["txt_mlp_up"].norm_call(rt, txt, *self._ada(tm[3], tm[4]), activation=GELU_TANH)
        txt = torch.addcmul(txt, tm[5], blk["txt_mlp_down"](rt, h))
        return img, txt

    def _single_block(self, blk, x, vec_silu, freqs):
        import torch

        rt = self.rt
        shift, scale, gate = blk["mod"](rt, vec_silu).chunk(6, dim=-1)[:3]
        ada = self._ada(shift, scale)
        q, k, v = self._split_heads(blk["qkv"].norm_call(rt, x, *ada), blk["qk_scale"])
        h = blk["mlp_up"].norm_call(rt, x, *ada, activation=GELU_TANH)
        out = blk["proj"](rt, self.attention(q, k, v, freqs))
        out = blk["mlp_down"](rt, h, residual=out)  # proj(attn) + down(h) in the epilogue
        return torch.addcmul(x, gate, out)

    def forward(self, collect=None):
        """One denoise step; returns the predicted latent tokens [4096, 64].
        collect: optional list that receives each block's outputs ((img, txt)
        after a double block, x after a single block)."""
        import torch
        import torch.nn.functional as F

        def mlp(pair, x):
            return pair[1](F.silu(pair[0](x)))

        img = self.img_in(self.img)
        txt = self.txt_in(self.txt)
        vec = (mlp(self.time_in, self._timestep_embedding(self.t, TIME_DIM).to(self.act))
               + mlp(self.guid_in, self._timestep_embedding(self.guidance, TIME_DIM).to(self.act))
               + mlp(self.vec_in, self.y))
        vec_silu = F.silu(vec)
        freqs = self._rope_tables()
        for blk in self.double:
            img, txt = self._double_block(blk, img, txt, vec_silu, freqs)
            if collect is not None:
                collect.append((img, txt))
        x = torch.cat((txt, img), 0)
        for blk in self.single:
            x = self._single_block(blk, x, vec_silu, freqs)
            if collect is not None:
                collect.append(x)
        img = x[TXT_TOKENS:]
        shift, scale = self.final_mod(vec_silu).chunk(2, dim=-1)
        return self.final(self._modulate(img, shift, scale))

    # ── parts timed on their own (static inputs) ──
    def parts(self):
        """Callables running one kind of work of the step on static buffers:
        the W4A8 GEMMs, the rotate+quantize launches, the modulation GEMVs
        and the 57 attention calls, each with the step's shapes and layers."""
        import torch

        rt, dev, act = self.rt, self.dev, self.act
        g = torch.Generator(device=dev).manual_seed(1)
        lin = self.quantized_linears()
        shapes = sorted({(M, l.K) for M, l in lin})
        x = {s: torch.randn(*s, generator=g, device=dev).to(act) for s in shapes}
        q = {s: torch.empty(*s, dtype=torch.int8, device=dev) for s in shapes}
        s_a = {M: torch.empty(M, dtype=torch.float32, device=dev) for M, _ in shapes}
        out = {(M, l.N): torch.empty(M, l.N, dtype=act, device=dev) for M, l in lin}
        for M, l in lin:  # valid codes and scales for the GEMM-only part
            l.quantize(rt, x[(M, l.K)], q[(M, l.K)], s_a[M])
        ada_w = 1.0 + 0.1 * torch.randn(HID, generator=g, device=dev)
        ada_b = 0.1 * torch.randn(HID, generator=g, device=dev)
        normed = {id(l) for name in ("qkv", "mlp_up") for l in self._kind_layers(name)}
        vec_silu = torch.randn(1, HID, generator=g, device=dev).to(act)
        S = IMG_TOKENS + TXT_TOKENS
        qkv = [torch.randn(HEADS, S, HEAD_DIM, generator=g, device=dev).to(act) for _ in range(3)]
        freqs = self._rope_tables()

        gelu = {id(l) for l in self._kind_layers("mlp_up")}

        def gemm():
            for M, l in lin:
                l.gemm(rt, q[(M, l.K)], s_a[M], act, out=out[(M, l.N)],
                       activation=GELU_TANH if id(l) in gelu else 0)

        def prep():
            for M, l in lin:
                if id(l) in normed:
                    l.norm_quantize(rt, x[(M, l.K)], ada_w, ada_b, q[(M, l.K)], s_a[M])
                else:
                    l.quantize(rt, x[(M, l.K)], q[(M, l.K)], s_a[M])

        def modulation():
            for blk in self.double:
                self._mod_w4a8(blk["img_mod"], vec_silu)
                self._mod_w4a8(blk["txt_mod"], vec_silu)
            for blk in self.single:
                blk["mod"](rt, vec_silu)

        def attention():
            for _ in range(len(self.double) + len(self.single)):
                self.attention(*qkv, freqs)

        def gemm_kind(name):
            sel = [(M, l) for M, l in lin if l in self._kind_layers(name)]

            def fn():
                for M, l in sel:
                    l.gemm(rt, q[(M, l.K)], s_a[M], act, out=out[(M, l.N)],
                           activation=GELU_TANH if id(l) in gelu else 0)
            return fn

        return {"gemm_w4a8": gemm, "rotate_quantize": prep, "modulation_gemvs": modulation,
                "attention_sdpa": attention}, {name: gemm_kind(name) for name, _, _ in BLOCK_LINEARS}

    def _kind_layers(self, name):
        ids = []
        for blk in self.double:
            ids += [blk[f"img_{name}"], blk[f"txt_{name}"]]
        ids += [blk[name] for blk in self.single]
        return ids

    def op_counts(self):
        lin_ops = sum(2.0 * M * l.K * l.N for M, l in self.quantized_linears())
        mod_ops = sum(2.0 * l.K * l.N for l in self.modulation_linears())
        S = IMG_TOKENS + TXT_TOKENS
        attn_flops = (len(self.double) + len(self.single)) * 4.0 * HEADS * S * S * HEAD_DIM
        wbytes = sum(l.w.numel() + 4 * l.s_w.numel() for _, l in self.quantized_linears())
        return dict(lin_ops=lin_ops, mod_ops=mod_ops, attn_flops=attn_flops, weight_bytes=wbytes,
                    n_layers=len(self.quantized_linears()), n_mods=len(self.modulation_linears()))


# ── the same step through the drop-in ops layer ─────────────────────────────
def _ensure_comfy():
    """ComfyUI is not installed in this image: put the minimal stand-in of
    the modules the ops layer imports (tests/fake_comfy) on the path."""
    import importlib.util
    import os
    import sys

    if importlib.util.find_spec("comfy") is None:
        sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "tests", "fake_comfy"))


class DropInFluxStep(FluxStep):
    """FluxStep with every quantized linear an IntCrushOps.Linear from
    make_intcrush_ops("int4_crush", 256), loaded through
    _load_from_state_dict with the same packed weights, fp16 group scales,
    SmoothRot factors, PermuQuant indices and biases: the path a ComfyUI user
    of the drop-in gets (reference _ops.py:817-862).  Each linear runs its own
    prep + GEMM; the adaptive LayerNorm, GELU-tanh and residual sums are torch
    ops between them, as in a DiT's own forward, so none of the hand fusions
    of FluxStep apply.  Names follow ComfyUI's Flux so the rotation rule
    (_ops.py:30-32) sends img_mod / txt_mod to rotated W4A8 GEMVs and the
    single block's modulation to W4A16.  The W4A16 bias is kept
    (INTCRUSH_W4A16_BIAS=1, set only while forward runs) so the two steps
    compute the same function."""

    def __init__(self, rt, dev, seed=0, n_double=N_DOUBLE, n_single=N_SINGLE):
        super().__init__(rt, dev, seed, n_double, n_single)
        _ensure_comfy()
        import __graft_entry__

        # registers the INT-Crush layouts with comfy.quant_ops (a no-op if the
        # package was imported after comfy and already did)
        __graft_entry__._submodule("quant_layout").register_intcrush_layouts()
        ops = __graft_entry__._submodule("_ops").make_intcrush_ops("int4_crush", ROT_SIZE)
        self.lin = {}
        for i, blk in enumerate(self.double):
            for s in ("img", "txt"):
                self._wrap(ops, blk[f"{s}_mod"], f"double_blocks.{i}.{s}_mod.lin")
                for name, path in (("qkv", "attn.qkv"), ("proj", "attn.proj"), ("mlp_up", "mlp.0"),
                                   ("mlp_down", "mlp.2")):
                    self._wrap(ops, blk[f"{s}_{name}"], f"double_blocks.{i}.{s}_{path}")
        for i, blk in enumerate(self.single):
            self._wrap(ops, blk["mod"], f"single_blocks.{i}.modulation.lin")
            for name in ("qkv", "proj", "mlp_up", "mlp_down"):
                self._wrap(ops, blk[name], f"single_blocks.{i}.{name}")

    def forward(self, *args, **kwargs):
        import os

        prev = os.environ.get("INTCRUSH_W4A16_BIAS")
        os.environ["INTCRUSH_W4A16_BIAS"] = "1"
        try:
            return super().forward(*args, **kwargs)
        finally:
            if prev is None:
                del os.environ["INTCRUSH_W4A16_BIAS"]
            else:
                os.environ["INTCRUSH_W4A16_BIAS"] = prev

    def _wrap(self, ops, layer, prefix):
        import torch

        sd = {"weight": layer.w, "weight_scale": layer.s_w.to(torch.float16), "bias": layer.b}
        if layer.rotated:
            sd["weight_smoothrot_factors"] = layer.sr.fdt
            sd["weight_perm"] = layer.perm.long()
        lin = ops.Linear(layer.K, layer.N, bias=True, device=layer.w.device, dtype=torch.bfloat16)
        full = {f"{prefix}.{k}": v for k, v in sd.items()}
        missing, unexpected, errors = [], [], []
        lin._load_from_state_dict(full, prefix + ".", {}, True, missing, unexpected, errors)
        if errors:
            raise RuntimeError(f"loading {prefix}: {errors}")
        if lin._intcrush_rot_need != layer.rotated:
            raise RuntimeError(f"{prefix}: rotation rule gave {lin._intcrush_rot_need}")
        self.lin[id(layer)] = lin

    def _call(self, layer, x):
        return self.lin[id(layer)](x)

    def _mod_w4a8(self, layer, vec_silu):
        return self._call(layer, vec_silu).chunk(6, dim=-1)

    def _double_block(self, blk, img, txt, vec_silu, freqs):
        import torch
        import torch.nn.functional as F

        im = self._mod_w4a8(blk["img_mod"], vec_silu)
        tm = self._mod_w4a8(blk["txt_mod"], vec_silu)
        iq, ik, iv = self._split_heads(self._call(blk["img_qkv"], self._modulate(img, im[0], im[1])), blk["qk_scale"])
        tq, tk, tv = self._split_heads(self._call(blk["txt_qkv"], self._modulate(txt, tm[0], tm[1])), blk["qk_scale"])
        attn = self.attention(torch.cat((tq, iq), 1), torch.cat((tk, ik), 1), torch.cat((tv, iv), 1), freqs)
        t_a, i_a = attn[:TXT_TOKENS], attn[TXT_TOKENS:]
        img = torch.addcmul(img, im[2], self._call(blk["img_proj"], i_a))
        h = F.gelu(self._call(blk["img_mlp_up"], self._modulate(img, im[3], im[4])), approximate="tanh")
        img = torch.addcmul(img, im[5], self._call(blk["img_mlp_down"], h))
        txt = torch.addcmul(txt, tm[2], self._call(blk["txt_proj"], t_a))
        h = F.gelu(self._call(blk["txt_mlp_up"], self._modulate(txt, tm[3], tm[4])), approximate="tanh")
        txt = torch.addcmul(txt, tm[5], self._call(blk["txt_mlp_down"], h))
        return img, txt

    def _single_block(self, blk, x, vec_silu, freqs):
        import torch
        import torch.nn.functional as F

        shift, scale, gate = self._call(blk["mod"], vec_silu).chunk(6, dim=-1)[:3]
        xm = self._modulate(x, shift, scale)
        q, k, v = self._split_heads(self._call(blk["qkv"], xm), blk["qk_scale"])
        h = F.gelu(self._call(blk["mlp_up"], xm), approximate="tanh")
        out = self._call(blk["proj"], self.attention(q, k, v, freqs)) + self._call(blk["mlp_down"], h)
        return torch.addcmul(x, gate, out)
