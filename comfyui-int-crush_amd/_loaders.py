"""ComfyUI loader nodes of INT-Crush (same node names, inputs and outputs as
the reference's _loaders.py:72-318):

  SimpleINT4UNetLoader(unet_name, rot_size)  -> (MODEL,)
  SimpleINT8UNetLoader(unet_name, rot_size)  -> (MODEL,)
  IntCrushLoRALoader(model, lora_name, strength) -> (MODEL,)
  IntCrushLoRAUnloader(model)                -> (MODEL,)

The loaders read the safetensors metadata (int_crush.format_version,
int_crush.rot_size, int_crush.padded_layers), build the ops class with
make_intcrush_ops and hand it to ComfyUI's load_diffusion_model, so a model
file written for the reference loads unchanged and runs on the gfx950 kernels.
"""
from __future__ import annotations

import logging

import torch

from ._checkpoint import parse_padded_layers
from ._lora import attach_lora_as_buffers, clear_intcrush_lora
from ._ops import make_intcrush_ops
from ._quant_utils import VALID_ROT_SIZES

log = logging.getLogger(__name__)

_INT4_FORMAT_VERSIONS: tuple[str, ...] = ("2", "3")
_INT8_FORMAT_VERSIONS: tuple[str, ...] = ("1",)


def _filenames(kind: str) -> list[str]:
    try:
        import folder_paths

        return folder_paths.get_filename_list(kind)
    except Exception:
        return []


def _detect_rot_size(metadata: dict | None, default_rot_size: int, format_versions: tuple[str, ...]) -> int:
    """rot_size from the file's metadata when it is an INT-Crush file of the
    expected format, else the node input (_loaders.py:46-67)."""
    if not metadata or metadata.get("int_crush.format_version") not in format_versions:
        return default_rot_size
    raw = metadata.get("int_crush.rot_size")
    if raw is not None:
        try:
            value = int(raw)
        except (TypeError, ValueError):
            value = None
        if value in VALID_ROT_SIZES:
            log.info("[INT-Crush] checkpoint metadata sets the Hadamard block size: rot_size %d", value)
            return value
    log.warning("[INT-Crush] the checkpoint is an INT-Crush one but names no valid rot_size; the node's "
                "rot_size %d is used, and outputs are wrong if the weights were quantized with another",
                default_rot_size)
    return default_rot_size


def _read_metadata(path: str) -> dict:
    import comfy.utils

    try:
        _, metadata = comfy.utils.load_torch_file(path, return_metadata=True)
    except Exception:
        metadata = {}
    return metadata or {}


def _resolve(unet_name: str) -> str:
    import folder_paths

    path = folder_paths.get_full_path("diffusion_models", unet_name)
    if path is None:
        raise FileNotFoundError(f"Model not found: {unet_name}")
    return path


class SimpleINT4UNetLoader:
    """Loads an INT-Crush model with packed INT4 weights (_loaders.py:72-114)."""

    @classmethod
    def INPUT_TYPES(cls):
        return {"required": {
            "unet_name": (_filenames("diffusion_models"),),
            "rot_size": (list(VALID_ROT_SIZES), {"default": 256}),
        }}

    RETURN_TYPES = ("MODEL",)
    FUNCTION = "load"
    CATEGORY = "loaders/INT-Crush"

    def load(self, unet_name: str, rot_size: int):
        from comfy.sd import load_diffusion_model

        path = _resolve(unet_name)
        rot_size = _detect_rot_size(_read_metadata(path), rot_size, _INT4_FORMAT_VERSIONS)
        use_w4a16 = rot_size == 0
        if use_w4a16:
            log.info("[INT-Crush] rot_size 0: INT4 layers run W4A16 (W4A8 needs rotated activations)")
        ops_cls = make_intcrush_ops("int4_crush", rot_size, use_w4a16=use_w4a16)
        if torch.cuda.is_available():
            torch.cuda.empty_cache()
        return (load_diffusion_model(path, model_options={"custom_operations": ops_cls}),)


class SimpleINT8UNetLoader:
    """Loads an INT-Crush model with int8 weights (_loaders.py:117-161)."""

    @classmethod
    def INPUT_TYPES(cls):
        return {"required": {
            "unet_name": (_filenames("diffusion_models"),),
            "rot_size": (list(VALID_ROT_SIZES), {"default": 256}),
        }}

    RETURN_TYPES = ("MODEL",)
    FUNCTION = "load"
    CATEGORY = "loaders/INT-Crush"

    def load(self, unet_name: str, rot_size: int):
        from comfy.sd import load_diffusion_model

        path = _resolve(unet_name)
        metadata = _read_metadata(path)
        rot_size = _detect_rot_size(metadata, rot_size, _INT8_FORMAT_VERSIONS)
        ops_cls = make_intcrush_ops("int8_crush", rot_size)
        if torch.cuda.is_available():
            torch.cuda.empty_cache()
        model = load_diffusion_model(path, model_options={"custom_operations": ops_cls})
        padded = metadata.get("int_crush.padded_layers", "")
        if padded:
            _apply_padded_layer_fixes(model, padded)
        return (model,)


def _apply_padded_layer_fixes(model, padded_str: str) -> None:
    """Trim weight columns of layers whose in_features were padded by the
    converter and fix the patch-embedding channel count (_loaders.py:164-226).
    `padded_str` is "key=orig_in_features;..." from int_crush.padded_layers."""
    import comfy.utils

    m = model.model
    for layer_key, orig_in in parse_padded_layers(padded_str).items():
        module_path = layer_key.rsplit(".weight", 1)[0]
        try:
            module = comfy.utils.get_attr(m, module_path)
        except AttributeError:
            continue
        weight = getattr(module, "weight", None)
        if weight is not None:
            if hasattr(weight, "_qdata"):
                q, params = weight._qdata, weight._params
                padded_in = q.shape[1] if q.dim() > 1 else q.shape[0]
                if padded_in > orig_in:
                    from comfy.quant_ops import QuantizedTensor

                    extra = {k: getattr(params, k) for k in ("rot_need", "rot_size", "perm", "zp")
                             if getattr(params, k, None) is not None}
                    new_params = type(params)(scale=params.scale, orig_dtype=params.orig_dtype,
                                              orig_shape=(params.orig_shape[0], orig_in), **extra)
                    module.weight = torch.nn.Parameter(
                        QuantizedTensor(q[:, :orig_in].contiguous(), weight._layout_type, new_params),
                        requires_grad=False)
                    log.info("[INT-Crush] INT8 layer %s: padded width %d trimmed to %d inputs", layer_key,
                             padded_in, orig_in)
            elif weight.shape[1] > orig_in:
                padded_in = weight.shape[1]
                module.weight = torch.nn.Parameter(weight[:, :orig_in].contiguous(), requires_grad=False)
                log.info("[INT-Crush] INT8 layer %s: padded width %d trimmed to %d inputs", layer_key, padded_in,
                         orig_in)
        if module_path == "img_in" and hasattr(m, "in_channels"):
            ps = getattr(m, "patch_size", 1)
            m.in_channels = orig_in // (ps * ps) if ps else orig_in


class IntCrushLoRALoader:
    """Attaches a LoRA as a residual on the raw input (_loaders.py:231-281)."""

    @classmethod
    def INPUT_TYPES(cls):
        return {"required": {
            "model": ("MODEL",),
            "lora_name": (_filenames("loras"), {"tooltip": "The name of the LoRA."}),
            "strength": ("FLOAT", {"default": 1.0, "min": -10.0, "max": 10.0, "step": 0.01}),
        }}

    RETURN_TYPES = ("MODEL",)
    FUNCTION = "load"
    CATEGORY = "loaders/INT-Crush"

    def load(self, model, lora_name: str, strength: float):
        import comfy.utils
        import folder_paths

        path = folder_paths.get_full_path_or_raise("loras", lora_name)
        lora_sd, _meta = comfy.utils.load_torch_file(path, safe_load=True, return_metadata=True)
        if not lora_sd:
            raise ValueError(f"INT-Crush LoRA: empty file '{lora_name}'")
        attached, total = attach_lora_as_buffers(model, lora_sd, strength)
        if attached == 0:
            log.warning("[INT-Crush LoRA] none of the %d LoRA patches belongs to an INT-Crush layer", total)
        else:
            log.info("[INT-Crush LoRA] LoRA applied to %d INT-Crush layer(s)", attached)
        return (model,)


class IntCrushLoRAUnloader:
    """Removes the LoRA residuals (_loaders.py:284-301)."""

    @classmethod
    def INPUT_TYPES(cls):
        return {"required": {"model": ("MODEL",)}}

    RETURN_TYPES = ("MODEL",)
    FUNCTION = "unload"
    CATEGORY = "loaders/INT-Crush"

    def unload(self, model):
        n = clear_intcrush_lora(model)
        log.info("[INT-Crush LoRA] LoRA removed from %d layer(s)", n)
        return (model,)


NODE_CLASS_MAPPINGS = {
    "SimpleINT4UNetLoader": SimpleINT4UNetLoader,
    "SimpleINT8UNetLoader": SimpleINT8UNetLoader,
    "IntCrushLoRALoader": IntCrushLoRALoader,
    "IntCrushLoRAUnloader": IntCrushLoRAUnloader,
}

NODE_DISPLAY_NAME_MAPPINGS = {
    "SimpleINT4UNetLoader": "INT4 UNet Loader (INT-Crush)",
    "SimpleINT8UNetLoader": "INT8 UNet Loader (INT-Crush)",
    "IntCrushLoRALoader": "LoRA Loader (INT-Crush)",
    "IntCrushLoRAUnloader": "LoRA Unloader (INT-Crush)",
}

__all__ = ["SimpleINT4UNetLoader", "SimpleINT8UNetLoader", "IntCrushLoRALoader", "IntCrushLoRAUnloader",
           "NODE_CLASS_MAPPINGS", "NODE_DISPLAY_NAME_MAPPINGS"]
