"""Minimal stand-in for the parts of ComfyUI the INT-Crush plugin touches.

Test infrastructure: ComfyUI is not installed here or on the GPU box.  Each
module mirrors only the names the plugin imports (comfy.ops, comfy.quant_ops,
comfy.sd, comfy.utils, comfy.lora, comfy.lora_convert, comfy.weight_adapter)
with the behaviour the plugin relies on.
"""
