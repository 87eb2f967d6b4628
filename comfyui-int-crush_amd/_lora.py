"""LoRA-family adapters as residuals on INT-Crush Linear modules.

Counterpart of the reference's _lora.py:22-87.  The adapter objects parsed
by ComfyUI (LoRA, LoKr, LoHa, OFT, BOFT, GLoRA) are stored on the module and
applied on the raw, unrotated input by the Linear's forward, so the
quantized weight and its fast kernels stay untouched.
"""
from __future__ import annotations

import logging
from typing import Any

__all__ = ["clear_intcrush_lora", "attach_lora_as_buffers"]

_log = logging.getLogger(__name__)

_ADAPTER_ATTRS = {
    "_intcrush_adapter": None,
    "_intcrush_lora_strength": None,
    "_intcrush_adapter_ready": False,
    "_intcrush_adapter_device": None,
}


def clear_intcrush_lora(model: Any) -> int:
    """Detach adapters from every INT-Crush Linear; returns the module count
    (_lora.py:22-35)."""
    n = 0
    for module in model.model.modules():
        if hasattr(module, "_intcrush_adapter"):
            for name, value in _ADAPTER_ATTRS.items():
                setattr(module, name, value)
            n += 1
    return n


def attach_lora_as_buffers(model: Any, lora_sd: dict, strength: float) -> tuple[int, int]:
    """Parse a LoRA state dict with ComfyUI and store each adapter on its
    INT-Crush Linear (_lora.py:38-87).  Returns (attached, parsed patches)."""
    import comfy.lora
    import comfy.lora_convert
    import comfy.weight_adapter

    lora_sd = comfy.lora_convert.convert_lora(lora_sd)
    key_map = comfy.lora.model_lora_keys_unet(model.model, {})
    patches = comfy.lora.load_lora(lora_sd, key_map)
    if not patches:
        return 0, 0
    clear_intcrush_lora(model)
    by_weight_key = {f"{name}.weight": m for name, m in model.model.named_modules()
                     if hasattr(m, "_intcrush_adapter")}
    attached = 0
    for weight_key, patch in patches.items():
        module = by_weight_key.get(weight_key)
        if module is None or not isinstance(patch, comfy.weight_adapter.WeightAdapterBase):
            continue
        module._intcrush_adapter = patch
        module._intcrush_lora_strength = strength
        module._intcrush_adapter_ready = False
        attached += 1
    if attached == 0:
        _log.debug("[INT-Crush LoRA] no INT-Crush layer among the %d patch targets", len(patches))
    return attached, len(patches)
