"""comfy.utils stand-in: safetensors loading and attribute lookup."""
import safetensors
import torch


def load_torch_file(ckpt, safe_load=False, device=None, return_metadata=False):
    with safetensors.safe_open(ckpt, framework="pt", device="cpu") as f:
        sd = {k: f.get_tensor(k) for k in f.keys()}
        metadata = f.metadata() or {}
    return (sd, metadata) if return_metadata else sd


def get_attr(obj, attr):
    for name in attr.split("."):
        obj = getattr(obj, name)
    return obj
