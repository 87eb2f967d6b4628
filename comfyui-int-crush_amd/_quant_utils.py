"""Host-side quantization helpers of the INT-Crush format.

Counterpart of the reference's _quant_utils.py (file:line below).  These are
plain PyTorch routines used by the layout classes (dequantize / quantize),
by the PyTorch path of the ops layer (`use_pytorch=True` or CPU tensors) and
by the loaders; the GPU forward never calls them.

Format facts restated here (reference citations):
  * regular Hadamard H = (H4 / 2)^{(x)k}, R = 4^k, H4 = [[1,1,1,-1],
    [1,1,-1,1],[1,-1,1,1],[-1,1,1,1]]                 (_quant_utils.py:67-93)
  * block rotation y_blk = x_blk @ H^T after zero-padding K to a multiple of R
                                                      (_quant_utils.py:117-147)
  * INT4 packing: two's complement nibbles, low nibble = even k
                                                      (_quant_utils.py:170-197)
  * group scales: s[n, g] = max|W[n, g*gs:(g+1)*gs]| / 7 (INT4) or / 127
    (INT8), clamped at 1e-8 and stored as fp16       (_quant_utils.py:237-270)
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

INT4_MIN, INT4_MAX = -8, 7
INT4_SCALE_DIVISOR = 7.0
INT4_TWOS_COMPLEMENT_BIAS = 16
INT8_MIN, INT8_MAX = -128, 127
INT8_SCALE_DIVISOR = 127.0
DEFAULT_GROUP_SIZE = 128
VALID_ROT_SIZES = (0, 16, 64, 256, 1024, 4096)

_H4 = ((1.0, 1.0, 1.0, -1.0), (1.0, 1.0, -1.0, 1.0), (1.0, -1.0, 1.0, 1.0), (-1.0, 1.0, 1.0, 1.0))
_hadamard_cache: dict[tuple, torch.Tensor] = {}


def is_power_of_two(n: int) -> bool:
    return n > 0 and (n & (n - 1)) == 0


def is_power_of_four(n: int) -> bool:
    return n >= 4 and is_power_of_two(n) and (n.bit_length() - 1) % 2 == 0


def make_hadamard_regular(n: int, dtype: torch.dtype = torch.float16, device="cpu") -> torch.Tensor:
    """Normalised regular Hadamard matrix of size n = 4^k (_quant_utils.py:67-93).

    Its entries are +-2^-k, exact in every float type, and it is symmetric and
    orthogonal (H @ H = I)."""
    if not is_power_of_four(n):
        raise ValueError(f"Regular Hadamard requires a power of 4, got {n}")
    key = (n, dtype, str(device))
    H = _hadamard_cache.get(key)
    if H is None:
        base = torch.tensor(_H4, dtype=torch.float64) * 0.5
        H = base
        while H.shape[0] < n:
            H = torch.kron(H, base)
        H = H.to(dtype=dtype, device=device)
        _hadamard_cache[key] = H
    return H


def rotate_activations(x: torch.Tensor, rot_size: int) -> torch.Tensor:
    """Block Hadamard rotation of the last dimension (_quant_utils.py:117-147).

    K is zero-padded to a multiple of rot_size, then each block is multiplied
    by H^T in x's dtype, as the reference does."""
    if rot_size <= 0:
        return x
    if not is_power_of_four(rot_size):
        raise ValueError(f"rot_size must be one of {VALID_ROT_SIZES[1:]}, got {rot_size}")
    K = x.shape[-1]
    pad = (-K) % rot_size
    if pad:
        x = F.pad(x, (0, pad))
    lead = x.shape[:-1]
    H = make_hadamard_regular(rot_size, x.dtype, x.device)
    y = torch.matmul(x.reshape(*lead, -1, rot_size), H.t())
    return y.reshape(*lead, K + pad)


def pack_int4(values: torch.Tensor) -> torch.Tensor:
    """[.., K] integers in [-8, 7] -> [.., ceil(K/2)] uint8 (_quant_utils.py:170-182)."""
    v = values.to(torch.int16)
    if v.numel() and (int(v.min()) < INT4_MIN or int(v.max()) > INT4_MAX):
        raise ValueError(f"Values must be in [{INT4_MIN}, {INT4_MAX}]")
    if v.shape[-1] % 2:
        v = F.pad(v, (0, 1))
    nib = (v & 0xF).to(torch.uint8)
    return nib[..., 0::2] | (nib[..., 1::2] << 4)


def unpack_int4(packed: torch.Tensor, K: int) -> torch.Tensor:
    """[.., Kp] uint8 -> [.., K] int8 (_quant_utils.py:185-197)."""
    p = packed.to(torch.int16)
    lo = p & 0xF
    hi = (p >> 4) & 0xF
    both = torch.stack((lo, hi), dim=-1).reshape(*p.shape[:-1], -1)[..., :K]
    return torch.where(both >= 8, both - 16, both).to(torch.int8)


def group_scales(W: torch.Tensor, divisor: float, group_size: int = DEFAULT_GROUP_SIZE) -> torch.Tensor:
    """Per-group symmetric scales [N, G] in fp16 (_quant_utils.py:237-252)."""
    N, K = W.shape
    pad = (-K) % group_size
    Wp = F.pad(W, (0, pad)) if pad else W
    m = Wp.reshape(N, -1, group_size).abs().amax(dim=2)
    return (m / divisor).clamp(min=1e-8).to(torch.float16)


def quantize_weights_grouped(W: torch.Tensor, scales: torch.Tensor, qmin: int, qmax: int,
                             group_size: int = DEFAULT_GROUP_SIZE) -> torch.Tensor:
    """round(W / s[n, k // gs]) clamped to [qmin, qmax] (_quant_utils.py:255-270)."""
    N, K = W.shape
    pad = (-K) % group_size
    Wp = F.pad(W, (0, pad)) if pad else W
    q = (Wp.reshape(N, -1, group_size) / scales.unsqueeze(2).to(W.dtype)).round().clamp(qmin, qmax)
    return q.reshape(N, -1).to(torch.int8)


def expand_group_scales(scale: torch.Tensor, N: int, K: int) -> torch.Tensor:
    """Scale [N], [N, 1] or [N, G] -> per-element [N, K] (group layout of
    _quant_utils.py:237-270: column k uses group k // (K / G))."""
    s = scale.reshape(N, -1).float()
    G = s.shape[1]
    if G == 1:
        return s.expand(N, K)
    if K % G:
        raise ValueError(f"K={K} is not a multiple of the {G} scale groups")
    return s.repeat_interleave(K // G, dim=1)


__all__ = [
    "INT4_MIN", "INT4_MAX", "INT4_SCALE_DIVISOR", "INT4_TWOS_COMPLEMENT_BIAS", "INT8_MIN", "INT8_MAX",
    "INT8_SCALE_DIVISOR", "DEFAULT_GROUP_SIZE", "VALID_ROT_SIZES", "is_power_of_two", "is_power_of_four",
    "make_hadamard_regular", "rotate_activations", "pack_int4", "unpack_int4", "group_scales",
    "quantize_weights_grouped", "expand_group_scales",
]
