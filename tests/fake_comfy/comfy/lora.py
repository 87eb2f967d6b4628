"""comfy.lora stand-in: maps "<module>.lora_up/.lora_down/.alpha" keys."""
from .weight_adapter import LoRAAdapter


def model_lora_keys_unet(model, key_map=None):
    key_map = dict(key_map or {})
    for name, _ in model.named_modules():
        if name:
            key_map[name] = f"{name}.weight"
    return key_map


def load_lora(lora_sd, key_map):
    patches = {}
    for lora_key, weight_key in key_map.items():
        up = lora_sd.get(f"{lora_key}.lora_up.weight")
        down = lora_sd.get(f"{lora_key}.lora_down.weight")
        if up is None or down is None:
            continue
        alpha = lora_sd.get(f"{lora_key}.alpha")
        patches[weight_key] = LoRAAdapter((up, down, float(alpha) if alpha is not None else None, None, None, None))
    return patches
