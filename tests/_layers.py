"""Synthetic INT-Crush layers and model files for the ops/loader tests.

Writes state dicts with the reference key set (_ops.py:36-45): packed INT4
`weight` [N, ceil(K/2)] uint8 or int8 [N, K], `weight_scale` fp16 [N, G] or
[N, 1], optional `weight_perm`, `weight_smoothrot_factors`, `weight_smooth`,
`weight_zp`, `weight_L1`/`weight_L2` and `bias`.
"""
from __future__ import annotations

import os

import torch

import __graft_entry__

qu = __graft_entry__._submodule("_quant_utils")


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def int4_layer(N: int, K: int, *, G: int | None = None, seed: int = 0, perm: bool = True,
               smoothrot: bool = True, bias: bool = True, zp: bool = False, svd_rank: int = 0) -> dict:
    """State dict (no prefix) of one INT4 layer with group-size K/G scales."""
    g = gen(seed)
    G = G if G is not None else max(1, K // 128)
    q = torch.randint(-8, 8, (N, K), generator=g, dtype=torch.int8)
    sd = {
        "weight": qu.pack_int4(q),
        "weight_scale": (torch.rand(N, G, generator=g) * 2e-2 + 1e-3).to(torch.float16),
    }
    if perm:
        sd["weight_perm"] = torch.randperm(K, generator=g)
    if smoothrot:
        sd["weight_smoothrot_factors"] = torch.exp(torch.randn(K, generator=g) * 0.5)
    if bias:
        sd["bias"] = torch.randn(N, generator=g).to(torch.float16)
    if zp:
        sd["weight_zp"] = torch.randint(-2, 3, (N,), generator=g).to(torch.float32)
    if svd_rank:
        sd["weight_L1"] = (torch.randn(N, svd_rank, generator=g) * 0.05).to(torch.float16)
        sd["weight_L2"] = (torch.randn(svd_rank, K, generator=g) * 0.05).to(torch.float16)
    return sd


def int8_layer(N: int, K: int, *, seed: int = 0, perm: bool = False, smoothrot: bool = False,
               smooth: bool = False, bias: bool = True, zp: bool = False) -> dict:
    g = gen(seed)
    sd = {
        "weight": torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8),
        "weight_scale": (torch.rand(N, 1, generator=g) * (2e-3 - 1e-4) + 1e-4).to(torch.float16),
    }
    if perm:
        sd["weight_perm"] = torch.randperm(K, generator=g)
    if smoothrot:
        sd["weight_smoothrot_factors"] = torch.exp(torch.randn(K, generator=g) * 0.5)
    if smooth:
        sd["weight_smooth"] = torch.exp(torch.randn(K, generator=g) * 0.3)
    if bias:
        sd["bias"] = torch.randn(N, generator=g).to(torch.float16)
    if zp:
        sd["weight_zp"] = torch.randint(-2, 3, (N,), generator=g).to(torch.float32)
    return sd


def prefixed(prefix: str, sd: dict) -> dict:
    return {f"{prefix}.{k}": v for k, v in sd.items()}


def load_linear(ops, prefix: str, sd: dict, in_features: int, out_features: int, device="cpu"):
    """Build ops.Linear and load a prefixed state dict through
    _load_from_state_dict, as ComfyUI's model loading does."""
    lin = ops.Linear(in_features, out_features, bias="bias" in sd, device=device)
    full = prefixed(prefix, sd)
    missing, unexpected, errors = [], [], []
    lin._load_from_state_dict(full, prefix + ".", {}, True, missing, unexpected, errors)
    assert not errors, errors
    return lin


def write_model(path: str, layers: dict, metadata: dict) -> None:
    """layers: {module_path: (state dict, in_features)} -> safetensors file."""
    from safetensors.torch import save_file

    flat = {}
    for name, (sd, in_f) in layers.items():
        flat.update(prefixed(name, sd))
        if sd["weight"].dtype == torch.uint8:
            flat[f"__in__.{name}.weight"] = torch.tensor([in_f])
    os.makedirs(os.path.dirname(path), exist_ok=True)
    save_file({k: v.contiguous() for k, v in flat.items()}, path, metadata=metadata)
