"""QuantizedTensor layout classes of the INT-Crush INT4 / INT8 formats.

Same public surface as the reference's quant_layout.py:44-234, so that
ComfyUI's QuantizedTensor machinery (VBAR paging, offload, LoRA patching)
handles INT-Crush weights exactly as before:

  IntCrushInt4Layout / IntCrushInt8Layout
      .Params               frozen dataclass: scale, orig_dtype, orig_shape,
                            rot_need, rot_size, perm, zp
      .state_dict_tensors() safetensors key layout
      .dequantize()         full dequantization to fp32
      .quantize()           float -> packed (ComfyUI's requantization hook)
      .supports_fast_matmul()
  register_intcrush_layouts()

Difference from the reference: dequantize() understands group scales
[N, G] (column k uses group k // (K / G), the layout written by the
converter, _quant_utils.py:237-270).  The reference reshapes the scale to
[N*G, 1] and fails for G > 1 (quant_layout.py:83-87).
"""
from __future__ import annotations

import logging
from dataclasses import dataclass

import torch

from ._quant_utils import (INT4_MAX, INT4_MIN, INT4_SCALE_DIVISOR, INT8_MAX, INT8_MIN,
                           INT8_SCALE_DIVISOR, expand_group_scales, pack_int4, unpack_int4)

__all__ = ["IntCrushInt4Layout", "IntCrushInt8Layout", "register_intcrush_layouts"]

try:  # the real base class when comfy_kitchen is installed (quant_layout.py:24-41)
    from comfy_kitchen.tensor.base import BaseLayoutParams
except ImportError:
    @dataclass(frozen=True)
    class BaseLayoutParams:
        scale: torch.Tensor
        orig_dtype: torch.dtype
        orig_shape: tuple

        def __post_init__(self):
            pass


def _fields_of(params) -> list[str]:
    out = ["scale"]
    if params.perm is not None:
        out.append("perm")
    if params.zp is not None:
        out.append("zp")
    return out


def _scale_to_f32(params) -> None:
    if isinstance(params.scale, torch.Tensor):
        object.__setattr__(params, "scale", params.scale.to(dtype=torch.float32, non_blocking=True))


def _state_dict(qdata, params) -> dict:
    out = {"": qdata, "weight_scale": params.scale}
    if params.perm is not None:
        out["weight_perm"] = params.perm
    if params.zp is not None:
        out["weight_zp"] = params.zp
    return out


def _dequant(q: torch.Tensor, params) -> torch.Tensor:
    N, K = q.shape
    s = expand_group_scales(params.scale, N, K)
    w = q.float()
    if params.zp is not None:
        w = w - params.zp.reshape(-1, 1).float()
    return w * s


def _kernels_ready() -> bool:
    from . import _hip_runtime as rt

    return bool(rt.KERNELS_AVAILABLE)


class IntCrushInt4Layout:
    """Packed INT4 (uint8, two values per byte, low nibble = even column) with
    fp16 scales [out, 1] (per row) or [out, groups]."""

    @dataclass(frozen=True)
    class Params(BaseLayoutParams):
        rot_need: bool = True
        rot_size: int = 256
        perm: torch.Tensor | None = None
        zp: torch.Tensor | None = None

        def _tensor_fields(self) -> list[str]:
            return _fields_of(self)

        def _validate_tensor_fields(self):
            _scale_to_f32(self)

    @classmethod
    def state_dict_tensors(cls, qdata, params):
        return _state_dict(qdata, params)

    @classmethod
    def dequantize(cls, qdata, params):
        """W = (q - zp) * s in fp32 (quant_layout.py:80-87, group-aware)."""
        return _dequant(unpack_int4(qdata, params.orig_shape[1]), params)

    @classmethod
    def supports_fast_matmul(cls):
        return _kernels_ready()

    @classmethod
    def quantize(cls, tensor, scale=None, stochastic_rounding=0, inplace_ops=False):
        """Per-row INT4 quantization of an already rotated/permuted weight
        (quant_layout.py:95-129): s = max|W| / 7 in fp16, q = round(W / s)."""
        if scale is None or (isinstance(scale, str) and scale == "recalculate"):
            s = (tensor.abs().amax(dim=1, keepdim=True) / INT4_SCALE_DIVISOR).clamp(min=1e-8).to(torch.float16)
        elif isinstance(scale, torch.Tensor):
            s = scale.to(torch.float16).reshape(-1, 1)
        else:
            s = torch.tensor([[scale]], dtype=torch.float16, device=tensor.device)
        q = (tensor / s.to(tensor.dtype)).round().clamp(INT4_MIN, INT4_MAX).to(torch.int8)
        params = cls.Params(scale=s.reshape(-1), orig_dtype=tensor.dtype, orig_shape=tuple(tensor.shape))
        return pack_int4(q), params


class IntCrushInt8Layout:
    """Plain int8 weights with per-row scales [out] (fp32 after loading)."""

    @dataclass(frozen=True)
    class Params(BaseLayoutParams):
        rot_need: bool = True
        rot_size: int = 256
        perm: torch.Tensor | None = None
        zp: torch.Tensor | None = None

        def _tensor_fields(self) -> list[str]:
            return _fields_of(self)

        def _validate_tensor_fields(self):
            _scale_to_f32(self)

    @classmethod
    def state_dict_tensors(cls, qdata, params):
        return _state_dict(qdata, params)

    @classmethod
    def dequantize(cls, qdata, params):
        """W = (q - zp) * s in fp32 (quant_layout.py:163-168)."""
        return _dequant(qdata, params)

    @classmethod
    def supports_fast_matmul(cls):
        return _kernels_ready()

    @classmethod
    def quantize(cls, tensor, scale=None, stochastic_rounding=0, inplace_ops=False):
        """Per-row INT8 quantization (quant_layout.py:171-202): s = max|W| / 127 in fp32."""
        if scale is None or (isinstance(scale, str) and scale == "recalculate"):
            s = (tensor.abs().amax(dim=1, keepdim=True) / INT8_SCALE_DIVISOR).clamp(min=1e-8).to(torch.float32)
        elif isinstance(scale, torch.Tensor):
            s = scale.to(torch.float32).reshape(-1, 1)
        else:
            s = torch.tensor([[scale]], dtype=torch.float32, device=tensor.device)
        q = (tensor / s.to(tensor.dtype)).round().clamp(INT8_MIN, INT8_MAX).to(torch.int8)
        params = cls.Params(scale=s.reshape(-1), orig_dtype=tensor.dtype, orig_shape=tuple(tensor.shape))
        return q, params


def register_intcrush_layouts() -> None:
    """Register both layouts and the "int4_crush" / "int8_crush" algorithms with
    ComfyUI (quant_layout.py:205-234).  Idempotent; a no-op without ComfyUI."""
    log = logging.getLogger(__name__)
    try:
        from comfy.quant_ops import QUANT_ALGOS, register_layout_class
    except ImportError:
        log.debug("INT-Crush: comfy.quant_ops not available; layout registration skipped")
        return
    try:
        register_layout_class("IntCrushInt4Layout", IntCrushInt4Layout)
        register_layout_class("IntCrushInt8Layout", IntCrushInt8Layout)
    except Exception:
        log.warning("INT-Crush: layout class registration failed", exc_info=True)
    QUANT_ALGOS.setdefault("int4_crush", {
        "storage_t": torch.uint8,
        "parameters": {"weight_scale", "weight_zp", "weight_perm"},
        "comfy_tensor_layout": "IntCrushInt4Layout",
    })
    QUANT_ALGOS.setdefault("int8_crush", {
        "storage_t": torch.int8,
        "parameters": {"weight_scale", "weight_perm", "weight_zp"},
        "comfy_tensor_layout": "IntCrushInt8Layout",
    })
