"""Reading and writing INT-Crush .safetensors checkpoints with their metadata.

The loaders take three metadata keys from a model file (reference
_loaders.py:21-67, :156-226): ``int_crush.format_version`` ("2"/"3" for
INT4 files, "1" for INT8), ``int_crush.rot_size`` (one of the valid
rotation sizes) and ``int_crush.padded_layers`` ("key=orig_in_features;..."
for layers whose input width the converter padded, e.g. Wan's FFN
13824 -> 14336, which the INT8 loader trims back).  The reference writes
them only from its offline converter; these helpers write and read the same
keys so that a checkpoint edited or re-saved in Python (a re-padded layer, a
changed rot size, an added zero point) loads through the nodes unchanged.
"""
from __future__ import annotations

import os
from dataclasses import dataclass, field
from typing import Mapping

import torch

from ._quant_utils import VALID_ROT_SIZES

__all__ = ["FORMAT_VERSIONS", "CheckpointInfo", "checkpoint_metadata", "format_padded_layers",
           "parse_padded_layers", "save_checkpoint", "load_checkpoint"]

# format_version written for each weight format, and the versions read as it
FORMAT_VERSIONS: dict[str, tuple[str, ...]] = {"int4_crush": ("3", "2"), "int8_crush": ("1",)}

_KEY_VERSION = "int_crush.format_version"
_KEY_ROT = "int_crush.rot_size"
_KEY_PADDED = "int_crush.padded_layers"


def parse_padded_layers(padded: str) -> dict[str, int]:
    """"key=orig_in;key=orig_in" -> {key: orig_in} (entries without '=' are
    skipped, as the loader skips them)."""
    out: dict[str, int] = {}
    for entry in (padded or "").split(";"):
        if "=" in entry:
            k, v = entry.split("=", 1)
            out[k.strip()] = int(v.strip())
    return out


def format_padded_layers(padded: Mapping[str, int]) -> str:
    """Inverse of parse_padded_layers; keys must name a ``.weight`` tensor."""
    parts = []
    for key, orig_in in padded.items():
        if not key.endswith(".weight") or any(c in key for c in ";="):
            raise ValueError(f"padded-layer key must be a '<module>.weight' name without ';' or '=': {key!r}")
        if int(orig_in) <= 0:
            raise ValueError(f"padded-layer width must be positive: {key}={orig_in}")
        parts.append(f"{key}={int(orig_in)}")
    return ";".join(parts)


def checkpoint_metadata(fmt: str, rot_size: int, padded_layers: Mapping[str, int] | None = None,
                        extra: Mapping[str, str] | None = None) -> dict[str, str]:
    """The metadata dict the loaders read, for weight format `fmt`
    ("int4_crush" / "int8_crush")."""
    if fmt not in FORMAT_VERSIONS:
        raise ValueError(f"unknown weight format {fmt!r} (expected one of {sorted(FORMAT_VERSIONS)})")
    if int(rot_size) not in VALID_ROT_SIZES:
        raise ValueError(f"rot_size {rot_size} is not one of {VALID_ROT_SIZES}")
    meta = {str(k): str(v) for k, v in (extra or {}).items()}
    meta[_KEY_VERSION] = FORMAT_VERSIONS[fmt][0]
    meta[_KEY_ROT] = str(int(rot_size))
    if padded_layers:
        meta[_KEY_PADDED] = format_padded_layers(padded_layers)
    return meta


def _weight_format(state_dict: Mapping[str, torch.Tensor]) -> str | None:
    """int4_crush when the quantized weights are packed uint8, int8_crush when
    they are int8 (the rule of _ops.py:583-597); None without either."""
    kinds = {t.dtype for k, t in state_dict.items() if k.endswith(".weight") and
             (k[: -len(".weight")] + ".weight_scale") in state_dict}
    if torch.uint8 in kinds and torch.int8 not in kinds:
        return "int4_crush"
    if torch.int8 in kinds and torch.uint8 not in kinds:
        return "int8_crush"
    return None


def save_checkpoint(path: str, state_dict: Mapping[str, torch.Tensor], *, rot_size: int,
                    fmt: str | None = None, padded_layers: Mapping[str, int] | None = None,
                    extra_metadata: Mapping[str, str] | None = None) -> dict[str, str]:
    """Write `state_dict` as a .safetensors file carrying the INT-Crush
    metadata; returns the metadata written.

    fmt defaults to the format of the quantized weights in the dict (packed
    uint8 -> int4_crush, int8 -> int8_crush).  Every padded layer must be a
    quantized weight in the dict; for INT8 its stored width must exceed the
    original one, as the loader trims columns [orig_in, stored).
    """
    from safetensors.torch import save_file

    fmt = fmt or _weight_format(state_dict)
    if fmt is None:
        raise ValueError("cannot tell the weight format (no packed-uint8 or int8 '.weight' with a '.weight_scale'); "
                         "pass fmt=")
    for key, orig_in in (padded_layers or {}).items():
        if key not in state_dict:
            raise KeyError(f"padded layer {key!r} is not in the state dict")
        w = state_dict[key]
        stored = w.shape[1] * (2 if w.dtype == torch.uint8 else 1) if w.dim() > 1 else w.shape[0]
        if fmt == "int8_crush" and not 0 < int(orig_in) < stored:
            raise ValueError(f"padded layer {key}: original width {orig_in} must be below the stored {stored}")
        if int(orig_in) > stored:
            raise ValueError(f"padded layer {key}: original width {orig_in} exceeds the stored {stored}")
    meta = checkpoint_metadata(fmt, rot_size, padded_layers, extra_metadata)
    tensors = {k: v.detach().to("cpu").contiguous() for k, v in state_dict.items()}
    d = os.path.dirname(os.path.abspath(path))
    os.makedirs(d, exist_ok=True)
    save_file(tensors, path, metadata=meta)
    return meta


@dataclass
class CheckpointInfo:
    """What the loaders will take from a file's metadata."""
    fmt: str | None                 # int4_crush / int8_crush from format_version; None if not INT-Crush
    format_version: str | None
    rot_size: int | None            # None when absent or not a valid size
    padded_layers: dict[str, int] = field(default_factory=dict)
    metadata: dict[str, str] = field(default_factory=dict)


def load_checkpoint(path: str, device: str = "cpu") -> tuple[dict[str, torch.Tensor], CheckpointInfo]:
    """Read a .safetensors checkpoint and its INT-Crush metadata (safetensors'
    loader executes nothing from the file)."""
    from safetensors import safe_open
    from safetensors.torch import load_file

    with safe_open(path, framework="pt") as f:
        meta = dict(f.metadata() or {})
    sd = load_file(path, device=device)
    ver = meta.get(_KEY_VERSION)
    fmt = next((k for k, v in FORMAT_VERSIONS.items() if ver in v), None)
    try:
        rot = int(meta.get(_KEY_ROT, ""))
    except ValueError:
        rot = None
    if rot not in VALID_ROT_SIZES:
        rot = None
    return sd, CheckpointInfo(fmt=fmt, format_version=ver, rot_size=rot,
                              padded_layers=parse_padded_layers(meta.get(_KEY_PADDED, "")), metadata=meta)
