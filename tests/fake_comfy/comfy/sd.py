"""comfy.sd stand-in: builds a small Flux-style DiT from a state dict with the
given custom_operations and loads the weights through the ops' Linear."""
import torch

from . import utils

LAST_MODEL = {}


class ModelPatcher:
    def __init__(self, model):
        self.model = model


class _Block(torch.nn.Module):
    pass


def _ensure(parent, path):
    node = parent
    for part in path:
        if not hasattr(node, part):
            node.add_module(part, _Block())
        node = getattr(node, part)
    return node


def load_diffusion_model(unet_path, model_options=None):
    """Every `<path>.weight` key becomes a Linear of the custom ops class; the
    module tree mirrors the key paths."""
    ops = (model_options or {})["custom_operations"]
    sd = utils.load_torch_file(unet_path)
    root = torch.nn.Module()
    for key, t in sorted(sd.items()):
        if not key.endswith(".weight") or key.startswith("__in__."):
            continue
        path = key[: -len(".weight")].split(".")
        out_f = t.shape[0]
        scale = sd.get(key[: -len("weight")] + "weight_scale")
        if t.dtype == torch.uint8:
            in_f = sd.get("__in__." + key, None)
            in_f = int(in_f.item()) if in_f is not None else t.shape[1] * 2
        else:
            in_f = t.shape[1]
        bias = (key[: -len("weight")] + "bias") in sd
        parent = _ensure(root, path[:-1])
        parent.add_module(path[-1], ops.Linear(in_f, out_f, bias=bias, device=None))
    sd = {k: v for k, v in sd.items() if not k.startswith("__in__.")}
    missing, unexpected = root.load_state_dict(sd, strict=False)
    LAST_MODEL["missing"] = missing
    LAST_MODEL["unexpected"] = unexpected
    return ModelPatcher(root)
