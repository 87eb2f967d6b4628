"""INT-Crush ops factory: the ComfyUI `custom_operations` class whose Linear
runs the gfx950 kernels.

Drop-in counterpart of the reference's _ops.py:146-883.  `make_intcrush_ops`
keeps its signature and memoisation, the returned class derives from
ComfyUI's `manual_cast`, and its Linear keeps every `_intcrush_*` attribute
that LoRA attach (`_lora.py`), graph replay (`_cuda_graph.py`) and the
loaders read.  The weight format, state-dict keys and per-layer rotation
rule are unchanged, so existing INT-Crush .safetensors files load as before.

Forward dispatch (reference _ops.py:817-862):
  INT4, rotated layer        -> W4A8: one fused prep+quantize kernel
                                (SmoothRot divide, Hadamard, pad, PermuQuant
                                gather, per-token INT8) + INT4xINT8 MFMA GEMM
                                with the nibble unpack and the per-row or
                                per-group dequant fused in
  INT4, not rotated / use_w4a16 -> W4A16: fused prep kernel + INT4->fp16/bf16
                                MFMA GEMM
  INT4, use_pytorch          -> fp32 dequant -> F.linear (reference fallback)
  INT8                       -> hipGraph replay of prep+quantize+GEMM, or the
                                same kernels eagerly (zero-point, casting hooks)
  M <= 16 tokens             -> the bandwidth-bound GEMV kernels

Device tensors never fall back to PyTorch silently: if the HIP library is
missing the forward raises, unless INTCRUSH_ALLOW_TORCH_FALLBACK=1 (or
use_pytorch=True) asks for the PyTorch path explicitly.  CPU tensors use the
PyTorch path, as the reference does without kernels.

Reference behaviours kept on purpose (documented quirks):
  * the W4A16 and PyTorch INT4 paths ignore the bias (_ops.py:474, :488);
    INTCRUSH_W4A16_BIAS=1 adds it;
  * the INT8 paths feed the raw (unrotated) input to the SVD low-rank
    residual (_ops.py:567, :577).
"""
from __future__ import annotations

import logging
import math
import os
from typing import Any, Callable

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _hip_runtime as _rt
from ._cuda_graph import CudaGraphRunner
from ._quant_utils import expand_group_scales, rotate_activations
from .quant_layout import IntCrushInt4Layout, IntCrushInt8Layout

_log = logging.getLogger(__name__)

# Layer-name substrings that disable rotation (_ops.py:30-32).
_NO_ROTATION_NAME_SUBSTRINGS: tuple[str, ...] = (
    "embed", "norm", "modulation", "output", "lm_head", "proj_out",
)

# State-dict key suffixes (_ops.py:36-45).
_SD_KEY_WEIGHT = "weight"
_SD_KEY_SCALE = "weight_scale"
_SD_KEY_ZP = "weight_zp"
_SD_KEY_PERM = "weight_perm"
_SD_KEY_SMOOTH = "weight_smooth"
_SD_KEY_SMOOTHROT = "weight_smoothrot_factors"
_SD_KEY_L1 = "weight_L1"
_SD_KEY_L2 = "weight_L2"
_SD_KEY_QUANT = "comfy_quant"
_SD_KEY_BIAS = "bias"
_KNOWN_SUFFIXES = (_SD_KEY_WEIGHT, _SD_KEY_SCALE, _SD_KEY_ZP, _SD_KEY_PERM, _SD_KEY_SMOOTH,
                   _SD_KEY_SMOOTHROT, _SD_KEY_L1, _SD_KEY_L2, _SD_KEY_BIAS, _SD_KEY_QUANT)
_VALID_SCALE_DTYPES = (torch.float16, torch.float32)


def _env_flag(name: str, default: str = "0") -> bool:
    return os.environ.get(name, default) == "1"


# ── lazy ComfyUI imports (_ops.py:53-72) ──────────────────────────────────
_QuantizedTensor = None
_cast_fns = None


def _get_qt():
    global _QuantizedTensor
    if _QuantizedTensor is None:
        from comfy.quant_ops import QuantizedTensor

        _QuantizedTensor = QuantizedTensor
    return _QuantizedTensor


def _get_cast():
    global _cast_fns
    if _cast_fns is None:
        from comfy.ops import cast_bias_weight, uncast_bias_weight

        _cast_fns = (cast_bias_weight, uncast_bias_weight)
    return _cast_fns


def _move_adapter_weights(adapter: Any, device: torch.device, dtype: torch.dtype) -> None:
    moved = [w.to(device=device, dtype=dtype) if isinstance(w, torch.Tensor) else w for w in adapter.weights]
    adapter.weights = type(adapter.weights)(moved)


def _hip_ready(x: torch.Tensor) -> bool:
    """Whether the gfx950 kernels serve this input; raises for device tensors
    when the library is missing and no PyTorch fallback was requested."""
    if not x.is_cuda:
        return False
    if _rt.KERNELS_AVAILABLE:
        return True
    if _env_flag("INTCRUSH_ALLOW_TORCH_FALLBACK"):
        return False
    raise RuntimeError(
        f"INT-Crush gfx950 kernels are not loaded ({_rt.LOAD_ERROR}); refusing a silent PyTorch "
        "fallback on the GPU (set INTCRUSH_ALLOW_TORCH_FALLBACK=1 to allow it)")


def _gemm_width(layer) -> int:
    """Width the GEMM kernels run a layer at: its prepared width K_w, or, when
    K_w is not a multiple of 128 (the MFMA kernels' K step; e.g. a 64-wide
    patch embedding), the next multiple of lcm(128, group size).  The extra
    columns hold zero weights and zero codes: their products add nothing to
    the exact int32 sums, and their fold blocks add fma(0, s, f) = f, so the
    outputs are those of the unpadded product.  Layers with a zero point or an
    SVD residual, whose corrections are formed over the prepared activation,
    keep K_w (and the scalar kernel)."""
    K_w = layer._intcrush_w_in
    w = layer.weight
    params = getattr(w, "_params", None)
    if (K_w is None or K_w % 128 == 0 or params is None or getattr(params, "zp", None) is not None
            or layer._intcrush_L1 is not None):
        return K_w
    sc = params.scale
    G = sc.shape[1] if sc.dim() > 1 else 1
    if G > 1 and (K_w % G or (K_w // G) % 32):
        return K_w  # groups the MFMA kernels do not take at any width
    step = 128 if G <= 1 else 128 * (K_w // G) // math.gcd(128, K_w // G)
    return -(-K_w // step) * step


class _DeviceState:
    """Per (device, activation dtype) kernel-side copies of a layer's
    preparation tensors: rounded SmoothRot / SmoothQuant factors with their
    reciprocals, and the int32 PermuQuant indices; and the operands of the
    GEMM at its width (_gemm_width): the prepared width k_gemm, the perm and
    old-SmoothQuant factors extended over the extra columns (identity, 1), and
    the weights and scales padded once (zero weights; scale 1 for the extra
    groups), for W4A8 layers rewritten once in the K-interleaved nibble order
    that the W4A8 kernels expand with fewer instructions (a second copy of
    the packed weights on the device, N x K/2 bytes per layer;
    INTCRUSH_W4_INTERLEAVE=0 keeps the checkpoint order), and unpacked once
    to int8 for the W4A8 launches that fill at most half the CUs (N x K bytes
    per layer that meets such a launch; INTCRUSH_W4_UNPACKED=0 turns it off),
    and for W4A16 layers copied once to the staged layout of the big-tile
    kernel (stage-major weights, group-major scales: N x K/2 + 4 N G bytes
    per layer with a launch of more than 128 rows; INTCRUSH_W4A16_STAGED=0
    turns it off)."""

    __slots__ = ("smoothrot", "smooth", "perm", "k_w", "k_gemm", "perm_gemm", "smooth_gemm", "_wcache")

    def __init__(self, layer, device: torch.device, dtype: torch.dtype):
        f = layer._intcrush_smoothrot_factors
        self.smoothrot = _rt.prepare_factors(f.to(device), dtype) if f is not None else None
        sm = layer._intcrush_smooth if f is None else None  # old SmoothQuant only without SmoothRot
        self.smooth = _rt.prepare_factors(sm.to(device), dtype) if sm is not None else None
        p = layer._intcrush_perm
        K_w = layer._intcrush_w_in
        self.perm = _rt.prepare_perm(p.to(device), K_w) if p is not None else None
        self.k_w = K_w
        self.k_gemm = _gemm_width(layer)
        self.perm_gemm, self.smooth_gemm, self._wcache = self.perm, self.smooth, {}
        if self.k_gemm != K_w:
            if p is not None:
                ext = torch.arange(K_w, self.k_gemm, device=device, dtype=p.dtype)
                self.perm_gemm = _rt.prepare_perm(torch.cat([p.to(device), ext]), self.k_gemm)
            if sm is not None:
                ones = torch.ones(self.k_gemm - K_w, device=device, dtype=sm.dtype)
                self.smooth_gemm = _rt.prepare_factors(torch.cat([sm.to(device), ones]), dtype)

    def gemm_weights(self, qdata: torch.Tensor, scale: torch.Tensor, kil: bool = False,
                     cache: bool = True, unpack: bool = False,
                     staged: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
        """(weights, scales) at k_gemm columns; the layer's own when no pad
        is needed.  kil (packed INT4, k_gemm a multiple of 8): the weights in
        the K-interleaved nibble order, for gemm_w4a8(..., kil=True).  unpack
        (packed INT4): the weights unpacked to int8 [N, k_gemm], for
        gemm_w4a8_unpacked.  staged (packed INT4, k_gemm a multiple of 64):
        weights [k_gemm/64, N, 32] and scales [G, N] for gemm_w4a16_staged.
        cache: keep the derived copy for the next call
        (one per form), keyed by the tensors' addresses -- only for the
        layer's resident weights; a per-call cast copy (offloaded or patched
        weights) may reuse an address with other contents, so its derived
        copy is built for that call alone."""
        int4 = qdata.dtype == torch.uint8
        staged = staged and int4 and self.k_gemm % 64 == 0
        unpack = unpack and int4 and not staged
        kil = kil and self.k_gemm % 8 == 0 and not unpack and not staged
        if self.k_gemm == self.k_w and not kil and not unpack and not staged:
            return qdata, scale
        N = qdata.shape[0]
        form = "staged" if staged else ("unpacked" if unpack else ("kil" if kil else "padded"))
        key = (qdata.data_ptr(), scale.data_ptr())
        hit = self._wcache.get(form) if cache else None
        if hit is None or hit[0] != key:
            wq, sc = qdata, scale
            if self.k_gemm != self.k_w:
                cols = (self.k_gemm // 2 if int4 else self.k_gemm) - qdata.shape[1]
                wq = torch.cat([qdata, qdata.new_zeros(N, cols)], dim=1)
                sc = scale.reshape(N, -1)
                if sc.shape[1] > 1:
                    extra = self.k_gemm // (self.k_w // sc.shape[1]) - sc.shape[1]
                    sc = torch.cat([sc, sc.new_ones(N, extra)], dim=1)
                sc = sc.reshape(N) if scale.dim() == 1 else sc
            # new tensors: the layer's weights stay as loaded
            if kil:
                wq = _rt.int4_interleave_k(wq)
            elif unpack:
                wq = _rt.unpack_int4_to_int8(wq, self.k_gemm)
            elif staged:
                wq, sc = _rt.w4a16_stage_layout(wq, sc)
            if not cache:
                return wq, sc
            hit = (key, wq, sc)
            self._wcache[form] = hit
        return hit[1], hit[2]


# ── ops factory ───────────────────────────────────────────────────────────
_ops_cache: dict[tuple, type] = {}


def make_intcrush_ops(quant_format: str, rot_size: int, use_pytorch: bool = False,
                      use_w4a16: bool = False) -> type:
    """Build (once per argument tuple) the manual_cast ops class with the
    INT-Crush Linear (_ops.py:146-163).

    quant_format: "int4_crush" or "int8_crush"; rot_size: Hadamard block
    size (0, 16, 64, 256, 1024, 4096); use_pytorch: force the PyTorch
    dequant path; use_w4a16: never take the W4A8 path for INT4 layers."""
    key = (quant_format, rot_size, use_pytorch, use_w4a16)
    cls = _ops_cache.get(key)
    if cls is not None:
        return cls
    from comfy.ops import manual_cast

    class IntCrushOps(manual_cast):

        class Linear(manual_cast.Linear):
            """INT-Crush Linear: QuantizedTensor storage, gfx950 forward."""

            def __init__(self, *args: Any, **kwargs: Any) -> None:
                super().__init__(*args, **kwargs)
                self._intcrush_is_quantized = False
                self._intcrush_rot_need = True
                self._intcrush_rot_size = rot_size
                self._intcrush_perm = None
                self._intcrush_smooth = None
                self._intcrush_smoothrot_factors = None
                self._intcrush_L1 = None
                self._intcrush_L2 = None
                self._intcrush_use_pytorch = use_pytorch
                self._intcrush_use_w4a16 = use_w4a16
                self._intcrush_w_in = None
                self.quant_format = None
                self.layout_type = None
                self._intcrush_adapter = None
                self._intcrush_lora_strength = None
                self._intcrush_adapter_ready = False
                self._intcrush_adapter_device = None
                self._intcrush_dev_states = {}
                self._graph_runner = None

            # ── preparation state ─────────────────────────────────────
            def _intcrush_state(self, x: torch.Tensor) -> _DeviceState:
                key = (x.device, x.dtype)
                st = self._intcrush_dev_states.get(key)
                if st is None:
                    if len(self._intcrush_dev_states) >= 4:
                        self._intcrush_dev_states.clear()
                    st = _DeviceState(self, x.device, x.dtype)
                    self._intcrush_dev_states[key] = st
                return st

            def _intcrush_invalidate(self) -> None:
                self._intcrush_dev_states = {}
                self._graph_runner = None

            def _kernel_rot(self) -> int:
                return self._intcrush_rot_size if self._intcrush_rot_need else 0

            # ── residuals (PyTorch, as in the reference) ──────────────
            def _apply_adapter(self, x_raw: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
                """LoRA-family residual on the raw input (_ops.py:195-271).

                Standard LoRA uses one [M, rank] intermediate and an in-place
                addmm_; every other adapter type uses its own h() / g().
                The graph runner is not invalidated here: the captured graph
                covers only prep + quantize + GEMM, which an adapter does not
                change (the reference drops the graph on every call, F12)."""
                adapter = self._intcrush_adapter
                if adapter is None:
                    return out
                if not self._intcrush_adapter_ready or self._intcrush_adapter_device != x_raw.device:
                    _move_adapter_weights(adapter, x_raw.device, x_raw.dtype)
                    self._intcrush_adapter_ready = True
                    self._intcrush_adapter_device = x_raw.device
                strength = self._intcrush_lora_strength
                if adapter.name == "lora":
                    up, down, alpha = adapter.weights[0], adapter.weights[1], adapter.weights[2]
                    rank = down.shape[0]
                    scale = (float(alpha) / rank if alpha else 1.0) * strength
                    mid = F.linear(x_raw, down)
                    out.addmm_(mid.to(out.dtype), up.t().to(out.dtype), beta=1, alpha=scale)
                    return out
                adapter.multiplier = strength
                out.add_(adapter.h(x_raw, out).to(out.dtype))
                return adapter.g(out)

            def _svd_factors(self, x: torch.Tensor):
                """L1 [N, r] and L2 [r, K] on x's device and dtype, cached on the
                module (_ops.py:372-381); (None, None) without an SVD branch."""
                L1, L2 = self._intcrush_L1, self._intcrush_L2
                if L1 is None or L2 is None:
                    return None, None
                if L1.device != x.device or L1.dtype != x.dtype:
                    L1 = self._intcrush_L1 = L1.to(device=x.device, dtype=x.dtype)
                if L2.device != x.device or L2.dtype != x.dtype:
                    L2 = self._intcrush_L2 = L2.to(device=x.device, dtype=x.dtype)
                return L1, L2

            def _apply_residuals(self, x: torch.Tensor, out: torch.Tensor,
                                 x_prep: torch.Tensor | None = None, folded: bool = False,
                                 lora_folded: bool = False) -> torch.Tensor:
                """SVD low-rank residual, then the adapter (_ops.py:367-387).
                folded / lora_folded: the SVD branch / standard LoRA were already
                added by the GEMM's residual epilogue (_fold_linear_residuals)."""
                L1, L2 = self._svd_factors(x)
                if L1 is not None and not folded:
                    src = x_prep if x_prep is not None else x.reshape(-1, x.shape[-1])
                    mid = src.to(L1.dtype) @ L2.t()
                    out.addmm_(mid.to(out.dtype), L1.t().to(out.dtype), beta=1, alpha=1)
                if not lora_folded:
                    self._apply_adapter(x.reshape(-1, x.shape[-1]), out)  # in place, as :386
                return out

            def _fold_linear_residuals(self, x: torch.Tensor, x_prep: torch.Tensor | None, params,
                                       out_dtype: torch.dtype, svd_src: torch.Tensor | None):
                """The corrections the reference adds to the GEMM output one
                addmm_ at a time -- the zero-point term (_ops.py:459-461, here
                group-aware), the SVD low-rank branch (:370-384) and a standard
                LoRA (:236-244) -- as one [M, N] tensor in the output dtype, for
                the GEMM's residual epilogue: one small GEMM over the
                concatenated factors [sum_g x_prep | svd_src L2^T | c x down^T]
                times [-(s zp) | L1 | up]^T, each factor in the dtype the
                reference multiplies it in.  svd_src is what the path's SVD
                branch reads (the prepared activation on the INT4 paths, the raw
                input on the INT8 path).  Returns (residual or None, standard
                LoRA folded)."""
                x2 = x.reshape(-1, x.shape[-1])
                M = x2.shape[0]
                A, B = [], []
                if params.zp is not None:
                    N = params.zp.numel()
                    s = params.scale.reshape(N, -1).float()
                    G = s.shape[1]
                    A.append(x_prep.float().reshape(M, G, -1).sum(-1))
                    B.append(-(s * params.zp.reshape(-1, 1).float()))
                L1, L2 = self._svd_factors(x)
                if L1 is not None:
                    A.append(svd_src.to(L1.dtype) @ L2.t())
                    B.append(L1)
                lora = False
                adapter = self._intcrush_adapter
                if adapter is not None and adapter.name == "lora":
                    if not self._intcrush_adapter_ready or self._intcrush_adapter_device != x2.device:
                        _move_adapter_weights(adapter, x2.device, x2.dtype)
                        self._intcrush_adapter_ready = True
                        self._intcrush_adapter_device = x2.device
                    up, down, alpha = adapter.weights[0], adapter.weights[1], adapter.weights[2]
                    rank = down.shape[0]
                    c = (float(alpha) / rank if alpha else 1.0) * self._intcrush_lora_strength
                    A.append(F.linear(x2, down) * c)
                    B.append(up)
                    lora = True
                if not A:
                    return None, False
                a = torch.cat([t.to(out_dtype) for t in A], 1)
                bt = torch.cat([t.to(out_dtype) for t in B], 1).t().contiguous()  # [k, N], no transposed view
                return a @ bt, lora

            def _finish_forward(self, out: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
                return out.to(x.dtype).reshape(*x.shape[:-1], -1)

            # ── activation preparation ───────────────────────────────
            def _prep_activation(self, x: torch.Tensor, pad_to_w_in: bool = True,
                                 apply_perm: bool = True) -> torch.Tensor:
                """reshape -> SmoothRot divide -> Hadamard -> pad -> perm
                (_ops.py:337-365).  Device tensors run the fused prep kernel;
                CPU tensors the PyTorch ops of the reference."""
                x2 = x.reshape(-1, x.shape[-1])
                if _hip_ready(x2):
                    st = self._intcrush_state(x2)
                    R = self._kernel_rot()
                    K_r = -(-x2.shape[-1] // R) * R if R else x2.shape[-1]
                    w_in = max(self._intcrush_w_in, K_r) if pad_to_w_in else K_r
                    perm = st.perm if (apply_perm and pad_to_w_in) else None
                    if apply_perm and not pad_to_w_in and self._intcrush_perm is not None:
                        return self._prep_activation_torch(x2, pad_to_w_in, apply_perm)
                    return _rt.prepare_activation(x2, rot_size=R, w_in=w_in, smoothrot=st.smoothrot, perm=perm)
                return self._prep_activation_torch(x2, pad_to_w_in, apply_perm)

            def _prep_activation_torch(self, x2: torch.Tensor, pad_to_w_in: bool, apply_perm: bool):
                f = self._intcrush_smoothrot_factors
                if f is not None:
                    x2 = x2 / f.to(device=x2.device, dtype=x2.dtype)
                if self._intcrush_rot_need:
                    x2 = rotate_activations(x2, self._intcrush_rot_size)
                if pad_to_w_in and x2.shape[-1] < self._intcrush_w_in:
                    x2 = F.pad(x2, (0, self._intcrush_w_in - x2.shape[-1]))
                if apply_perm and self._intcrush_perm is not None:
                    x2 = x2[..., self._intcrush_perm.to(x2.device)]
                return x2

            def _prep_int8_torch(self, x2: torch.Tensor) -> torch.Tensor:
                """INT8 prep on CPU: _prep_activation then the old SmoothQuant
                divide after the gather (_ops.py:529-533)."""
                xp = self._prep_activation_torch(x2, True, True)
                if self._intcrush_smoothrot_factors is None and self._intcrush_smooth is not None:
                    xp = xp / self._intcrush_smooth.to(device=xp.device, dtype=xp.dtype)
                return xp

            # ── ComfyUI casting (VBAR / low-VRAM), _ops.py:401-433 ────
            def _setup_casting(self, x: torch.Tensor):
                QT = _get_qt()
                need_cast = (
                    self.comfy_cast_weights or self.weight_function or self.bias_function
                    or getattr(self, "weight_lowvram_function", None) is not None
                    or getattr(self, "bias_lowvram_function", None) is not None
                )
                if not need_cast:
                    return self.weight, self.bias, None, QT
                weight_dtype = self.weight._params.orig_dtype if isinstance(self.weight, QT) else x.dtype
                cast, uncast_fn = _get_cast()
                weight, bias, offload_stream = cast(self, input=None, dtype=weight_dtype, device=x.device,
                                                    bias_dtype=x.dtype, offloadable=True)
                return weight, bias, (lambda: uncast_fn(self, weight, bias, offload_stream)), QT

            def _casting_hooks(self) -> bool:
                return bool(self.comfy_cast_weights or self.weight_function or self.bias_function
                            or getattr(self, "weight_lowvram_function", None)
                            or getattr(self, "bias_lowvram_function", None))

            # ── forward paths ────────────────────────────────────────
            def _forward_predequant(self, weight, bias, x):
                """Weight already dequantized by a wrapper (_ops.py:435-441)."""
                x2 = self._prep_activation(x, pad_to_w_in=False, apply_perm=False)
                out = F.linear(x2, weight.to(x2.dtype), None if bias is None else bias.to(x2.dtype))
                out = self._apply_residuals(x, out, x_prep=x2)
                return self._finish_forward(out, x)

            @staticmethod
            def _zp_correction(out, x_prep, scale, zp):
                """out -= sum_k x_prep[m,k] * zp[n] * s[n, g(k)]: the zero-point
                term of W = (q - zp) * s (_ops.py:449-461, group-aware)."""
                N = out.shape[1]
                s = scale.reshape(N, -1).float()
                G = s.shape[1]
                M, K = x_prep.shape
                xs = x_prep.float().reshape(M, G, K // G).sum(-1)  # [M, G]
                corr = xs @ (s * zp.reshape(-1, 1).float()).t()  # [M, N]
                out.sub_(corr.to(out.dtype))

            def _forward_int4_w4a8(self, qdata, weight, bias, x):
                """W4A8 (_ops.py:443-464): fused prep+quantize, fused INT4 GEMM."""
                x2 = x.reshape(-1, x.shape[-1])
                st = self._intcrush_state(x2)
                params = weight._params
                R = self._intcrush_rot_size
                need_prep = params.zp is not None or (self._intcrush_L1 is not None and self._intcrush_L2 is not None)
                x_prep = (_rt.prepare_activation(x2, rot_size=R, w_in=self._intcrush_w_in, smoothrot=st.smoothrot,
                                                 perm=st.perm) if need_prep else None)
                q, s_a = _rt.rotate_quantize(x2, rot_size=R, w_in=st.k_gemm, smoothrot=st.smoothrot,
                                             perm=st.perm_gemm)
                res, lora = self._fold_linear_residuals(x, x_prep, params, x.dtype, x_prep)
                # resident weights: a cached derived copy -- unpacked to int8 for launches that fill
                # at most half the CUs, else K-interleaved; a per-call cast copy: the checkpoint order
                own = weight is self.weight
                N = qdata.shape[0]
                G = params.scale.reshape(N, -1).shape[1]
                if G > 1:
                    G = st.k_gemm // (st.k_w // G)  # groups at the GEMM's (padded) width
                if (own and _env_flag("INTCRUSH_W4_UNPACKED", "1")
                        and _rt.w4a8_unpacked_pays(q.shape[0], N, st.k_gemm, G, device=q.device)):
                    wq, ws = st.gemm_weights(qdata, params.scale, unpack=True)
                    out = _rt.gemm_w4a8_unpacked(q, wq, ws, s_a, bias=bias, out_dtype=x.dtype, residual=res)
                else:
                    kil = own and _env_flag("INTCRUSH_W4_INTERLEAVE", "1") and st.k_gemm % 8 == 0
                    wq, ws = st.gemm_weights(qdata, params.scale, kil=kil, cache=own)
                    out = _rt.gemm_w4a8(q, wq, ws, s_a, bias=bias, out_dtype=x.dtype, residual=res, kil=kil)
                out = self._apply_residuals(x, out, x_prep=x_prep, folded=True, lora_folded=lora)
                return self._finish_forward(out, x)

            def _forward_int4_w4a16(self, qdata, weight, bias, x):
                """W4A16 (_ops.py:466-481): fused prep, INT4->fp16/bf16 MFMA GEMM."""
                x2 = x.reshape(-1, x.shape[-1])
                st = self._intcrush_state(x2)
                params = weight._params
                x_prep = _rt.prepare_activation(x2, rot_size=self._kernel_rot(), w_in=st.k_gemm,
                                                smoothrot=st.smoothrot, perm=st.perm_gemm)
                b = bias if _env_flag("INTCRUSH_W4A16_BIAS") else None
                own = weight is self.weight
                N = qdata.shape[0]
                G = params.scale.reshape(N, -1).shape[1]
                if G > 1:
                    G = st.k_gemm // (st.k_w // G)  # groups at the GEMM's (padded) width
                if (own and _env_flag("INTCRUSH_W4A16_STAGED", "1")
                        and _rt.w4a16_staged_pays(x_prep.shape[0], N, st.k_gemm, G)):
                    # the layer's weights in the staged layout, built once and kept
                    wq, ws = st.gemm_weights(qdata, params.scale, staged=True)
                    out = _rt.gemm_w4a16_staged(x_prep, wq, ws, bias=b)
                else:
                    wq, ws = st.gemm_weights(qdata, params.scale, cache=own)
                    out = _rt.gemm_w4a16(x_prep, wq, ws, bias=b)
                if params.zp is not None:
                    self._zp_correction(out, x_prep, params.scale, params.zp)
                out = self._apply_residuals(x, out, x_prep=x_prep)
                return self._finish_forward(out, x)

            def _forward_int4_pytorch(self, qdata, weight, x):
                """fp32 dequant -> F.linear (_ops.py:483-491)."""
                w = IntCrushInt4Layout.dequantize(qdata, weight._params).to(x.device, x.dtype)
                x2 = self._prep_activation_torch(x.reshape(-1, x.shape[-1]), True, True)
                out = F.linear(x2, w)
                out = self._apply_residuals(x, out, x_prep=x2)
                return self._finish_forward(out, x)

            def _forward_int8(self, qdata, weight, bias, x):
                """INT8 (_ops.py:493-579): graph replay or eager kernels."""
                params = weight._params
                zp = params.zp
                compute_dtype = x.dtype if x.dtype in (torch.float16, torch.bfloat16) else torch.bfloat16
                x2 = x.reshape(-1, x.shape[-1])
                if not _hip_ready(x2):
                    # dequantize in compute_dtype, as the reference does (_ops.py:538-545)
                    xp = self._prep_int8_torch(x2).to(compute_dtype)
                    s = expand_group_scales(params.scale, qdata.shape[0], qdata.shape[1]).to(xp.device)
                    s = s.to(compute_dtype)
                    w = qdata.to(device=xp.device, dtype=compute_dtype) * s
                    if zp is not None:
                        w = w - zp.reshape(-1, 1).to(device=xp.device, dtype=compute_dtype) * s
                    out = F.linear(xp, w, None if bias is None else bias.to(compute_dtype))
                    out = self._apply_residuals(x, out)
                    return self._finish_forward(out, x)
                if zp is None and not self._casting_hooks() and _rt.USE_CUDA_GRAPHS:
                    if self._graph_runner is None:
                        self._graph_runner = CudaGraphRunner(self, safe_no_clone=True)
                    out = self._graph_runner.run(x, bias, compute_dtype)
                    out = self._apply_residuals(x, out)
                    return self._finish_forward(out, x)
                st = self._intcrush_state(x2)
                R = self._kernel_rot()
                fused = _rt.USE_FUSED_W8A8 and x2.dtype in (torch.float16, torch.bfloat16)
                x_prep = None
                if zp is not None or fused:
                    x_prep = _rt.prepare_activation(x2, rot_size=R, w_in=st.k_gemm, smoothrot=st.smoothrot,
                                                    perm=st.perm_gemm, smooth=st.smooth_gemm)
                wq, ws = st.gemm_weights(qdata, params.scale, cache=weight is self.weight)
                if fused:
                    out = _rt.fused_quant_int8_gemm_dequant(x_prep, wq, ws, bias=bias, out_dtype=compute_dtype)
                    if zp is not None:
                        self._zp_correction(out, x_prep, params.scale, zp)
                    out = self._apply_residuals(x, out)
                    return self._finish_forward(out, x)
                q, s_a = _rt.rotate_quantize(x2, rot_size=R, w_in=st.k_gemm, smoothrot=st.smoothrot,
                                             perm=st.perm_gemm, smooth=st.smooth_gemm)
                # the INT8 path's SVD branch reads the raw input (_ops.py:578)
                res, lora = self._fold_linear_residuals(x, x_prep, params, compute_dtype, x2)
                out = _rt.fused_int8_gemm_dequant(q, wq, ws, s_a, bias=bias, out_dtype=compute_dtype, residual=res)
                out = self._apply_residuals(x, out, folded=True, lora_folded=lora)
                return self._finish_forward(out, x)

            # ── state-dict loading (_ops.py:583-761) ─────────────────
            @staticmethod
            def _detect_weight_format(weight, scale):
                if weight is None or scale is None or scale.dtype not in _VALID_SCALE_DTYPES:
                    return None
                if weight.dtype == torch.uint8:
                    return "int4_crush"
                if weight.dtype == torch.int8:
                    return "int8_crush"
                return None

            def _pop_intcrush_tensors(self, state_dict: dict, prefix: str) -> dict:
                t = {
                    "weight": state_dict.pop(prefix + _SD_KEY_WEIGHT),
                    "scale": state_dict.pop(prefix + _SD_KEY_SCALE),
                    "zp": state_dict.pop(prefix + _SD_KEY_ZP, None),
                    "perm": state_dict.pop(prefix + _SD_KEY_PERM, None),
                    "smooth": state_dict.pop(prefix + _SD_KEY_SMOOTH, None),
                    "smoothrot_factors": state_dict.pop(prefix + _SD_KEY_SMOOTHROT, None),
                    "L1": state_dict.pop(prefix + _SD_KEY_L1, None),
                    "L2": state_dict.pop(prefix + _SD_KEY_L2, None),
                    "bias": state_dict.pop(prefix + _SD_KEY_BIAS, None),
                }
                state_dict.pop(prefix + _SD_KEY_QUANT, None)
                return t

            def _store_intcrush_attrs(self, tensors: dict, params, device) -> None:
                self._intcrush_perm = params.perm
                self._intcrush_w_in = self.in_features
                self._intcrush_smooth = (tensors["smooth"].float().to(device)
                                         if tensors["smooth"] is not None else None)
                self._intcrush_smoothrot_factors = (tensors["smoothrot_factors"].float().to(device)
                                                    if tensors["smoothrot_factors"] is not None else None)
                self._intcrush_L1 = (tensors["L1"].to(device=device, dtype=torch.float16)
                                     if tensors["L1"] is not None else None)
                self._intcrush_L2 = (tensors["L2"].to(device=device, dtype=torch.float16)
                                     if tensors["L2"] is not None else None)
                self._intcrush_invalidate()

            @staticmethod
            def _clear_known_missing_keys(missing_keys: list, prefix: str) -> None:
                for suffix in _KNOWN_SUFFIXES:
                    if prefix + suffix in missing_keys:
                        missing_keys.remove(prefix + suffix)

            def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys,
                                      unexpected_keys, error_msgs):
                from comfy.quant_ops import QUANT_ALGOS, QuantizedTensor, get_layout_class

                fmt = self._detect_weight_format(state_dict.get(prefix + _SD_KEY_WEIGHT),
                                                 state_dict.get(prefix + _SD_KEY_SCALE))
                if fmt is None:
                    super()._load_from_state_dict(state_dict, prefix, local_metadata, strict, missing_keys,
                                                  unexpected_keys, error_msgs)
                    return
                qconfig = QUANT_ALGOS[fmt]
                layout_type = qconfig["comfy_tensor_layout"]
                layout_cls = get_layout_class(layout_type)
                tensors = self._pop_intcrush_tensors(state_dict, prefix)
                w0 = getattr(self, "weight", None)
                device = w0.device if w0 is not None else torch.device("cpu")
                name = prefix.lower()
                rot_need = rot_size > 0 and not any(s in name for s in _NO_ROTATION_NAME_SUBSTRINGS)
                self._intcrush_rot_need = rot_need
                self._intcrush_rot_size = rot_size
                self._intcrush_is_quantized = True
                perm, zp = tensors["perm"], tensors["zp"]
                scale = tensors["scale"].float()
                if fmt == "int8_crush":
                    scale = scale.reshape(-1)
                params = layout_cls.Params(
                    scale=scale.to(device=device), orig_dtype=torch.float16,
                    orig_shape=(self.out_features, self.in_features), rot_need=rot_need, rot_size=rot_size,
                    perm=perm.to(device=device) if perm is not None else None,
                    zp=zp.to(device=device) if zp is not None else None,
                )
                self._store_intcrush_attrs(tensors, params, device)
                self.weight = nn.Parameter(
                    QuantizedTensor(tensors["weight"].to(device=device, dtype=qconfig["storage_t"]),
                                    layout_type, params),
                    requires_grad=False)
                self.quant_format = fmt
                self.layout_type = layout_type
                b = tensors["bias"]
                self.bias = nn.Parameter(b.to(device=device), requires_grad=False) if b is not None else None
                if perm is not None:
                    self.register_parameter("weight_perm", nn.Parameter(perm.to(device=device), requires_grad=False))
                if zp is not None:
                    self.register_parameter("weight_zp", nn.Parameter(zp.to(device=device), requires_grad=False))
                self._clear_known_missing_keys(missing_keys, prefix)

            def convert_weight(self, weight, inplace: bool = False):
                """Keep QuantizedTensor weights as they are (_ops.py:763-768)."""
                QT = _get_qt()
                if self._intcrush_is_quantized and isinstance(weight, QT):
                    return weight
                return super().convert_weight(weight, inplace)

            def set_weight(self, out_weight, inplace_update=False, seed=0, return_weight=False, **kwargs):
                """Requantize patched float weights, keeping rotation and
                permutation (_ops.py:770-807)."""
                import dataclasses

                self._intcrush_invalidate()
                if not self._intcrush_is_quantized:
                    w = out_weight.to(self.weight.dtype)
                    if return_weight:
                        return w
                    self.weight = nn.Parameter(w, requires_grad=False)
                    return None
                from comfy.quant_ops import QuantizedTensor, get_layout_class

                if isinstance(out_weight, QuantizedTensor):
                    if return_weight:
                        return out_weight
                    self.weight = nn.Parameter(out_weight, requires_grad=False)
                    return None
                layout_cls = get_layout_class(self.layout_type)
                packed, params = layout_cls.quantize(out_weight.float(), scale="recalculate",
                                                     stochastic_rounding=seed)
                params = dataclasses.replace(params, rot_need=self._intcrush_rot_need,
                                             rot_size=self._intcrush_rot_size, perm=self._intcrush_perm)
                qt = QuantizedTensor(packed, self.layout_type, params)
                if return_weight:
                    return qt
                self.weight = nn.Parameter(qt, requires_grad=False)
                return None

            def set_bias(self, out_bias, inplace_update=False, seed=0, return_weight=False, **kwargs):
                if out_bias is None:
                    return None
                if return_weight:
                    return out_bias
                self._graph_runner = None
                self.bias = nn.Parameter(out_bias, requires_grad=False)
                return None

            # ── forward (_ops.py:817-862) ────────────────────────────
            @torch.no_grad()
            def forward(self, x: torch.Tensor) -> torch.Tensor:
                if not self._intcrush_is_quantized:
                    return super().forward(x)
                weight, bias, uncast, QT = self._setup_casting(x)
                try:
                    if not isinstance(weight, QT):
                        return self._forward_predequant(weight, bias, x)
                    qdata = weight._qdata
                    if isinstance(weight._params, IntCrushInt4Layout.Params):
                        if self._intcrush_use_pytorch or not _hip_ready(x):
                            return self._forward_int4_pytorch(qdata, weight, x)
                        if (not self._intcrush_use_w4a16 and self._intcrush_rot_need
                                and _rt.HIP_W4A8_GEMM and _rt.HIP_ROTATE_QUANT):
                            return self._forward_int4_w4a8(qdata, weight, bias, x)
                        if x.dtype in (torch.float16, torch.bfloat16) and _rt.HIP_W4A16_GEMM:
                            return self._forward_int4_w4a16(qdata, weight, bias, x)
                        return self._forward_int4_pytorch(qdata, weight, x)
                    if isinstance(weight._params, IntCrushInt8Layout.Params):
                        return self._forward_int8(qdata, weight, bias, x)
                    return super().forward(x)
                finally:
                    if uncast is not None:
                        uncast()

        class GroupNorm(manual_cast.GroupNorm):
            pass

        class LayerNorm(manual_cast.LayerNorm):
            pass

        class Conv2d(manual_cast.Conv2d):
            pass

        class Conv3d(manual_cast.Conv3d):
            pass

        class ConvTranspose2d(manual_cast.ConvTranspose2d):
            pass

        class Embedding(manual_cast.Embedding):
            pass

    _ops_cache[key] = IntCrushOps
    return IntCrushOps


__all__ = ["make_intcrush_ops"]
