"""HIP kernel runtime for INT-Crush on MI355X (gfx950).

Counterpart of the reference's _triton_runtime.py:1-130: it loads the
hand-written gfx950 kernels (libintcrush_gfx950.so, C ABI in include/intcrush.h)
through ctypes, exposes one Python callable per kernel with the reference's
signatures, and publishes availability flags plus the USE_FUSED_W8A8 /
USE_CUDA_GRAPHS toggles and the INTCRUSH_NO_CUDA_GRAPHS environment switch.

Differences from the reference runtime:
  * there is no silent degradation for device tensors: every callable raises
    RuntimeError when the library is missing or a kernel reports an error;
  * the only CPU branch is the one the reference itself documents for
    dynamic_quantize_activation on CPU tensors (kernels/triton_quantize.py:176-179);
  * the flags keep the reference names (TRITON_*) as aliases of the HIP ones so
    that code written against the reference runtime keeps working.

Every kernel is enqueued on torch's current stream of the tensor's device, with
no host synchronisation, so all callables may be captured into a hipGraph
(torch.cuda.CUDAGraph) provided the caller pre-allocates the outputs.
"""
from __future__ import annotations

import ctypes
import logging
import os

import torch

log = logging.getLogger(__name__)

LIB_NAME = "libintcrush_gfx950.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

IC_DTYPE_F16, IC_DTYPE_BF16, IC_DTYPE_F32 = 0, 1, 2
_DT_CODE = {torch.float16: IC_DTYPE_F16, torch.bfloat16: IC_DTYPE_BF16, torch.float32: IC_DTYPE_F32}
VALID_ROT_SIZES = (0, 16, 64, 256, 1024, 4096)

# ── Availability flags (reference names below) ──────────────────────────────
KERNELS_AVAILABLE = False
HIP_DYNQUANT = False
HIP_ROTATE_QUANT = False
HIP_INT8_GEMM = False
HIP_W4A8_GEMM = False
HIP_W4A16_GEMM = False
HIP_INT4_UNPACK = False
HIP_INT4_INT8_UNPACK = False
HIP_FUSED_QGD = False
LOAD_ERROR: str | None = None

# ── User toggles (same meaning as _triton_runtime.py:24-32, :60-61) ─────────
USE_FUSED_W8A8: bool = False
USE_CUDA_GRAPHS: bool = True
if os.environ.get("INTCRUSH_NO_CUDA_GRAPHS", "0") == "1":
    USE_CUDA_GRAPHS = False

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
# name -> (argtypes, restype); kept in the order of include/intcrush.h
SIGNATURES: dict[str, tuple[list, object]] = {
    "ic_version": ([], ctypes.c_char_p),
    "ic_last_error": ([], ctypes.c_char_p),
    "ic_max_fused_row": ([], _L),
    "ic_smoothrot_prepare": ([_P, _L, _I, _P, _P, _P], _I),
    "ic_rotate_quantize": ([_P, _I, _L, _L, _L, _P, _P, _I, _L, _P, _P, _P, _P, _L, _P, _P], _I),
    "ic_prepare_activation": ([_P, _I, _L, _L, _L, _P, _P, _I, _L, _P, _P, _P, _P, _L, _P], _I),
    "ic_permute_quantize": ([_P, _I, _L, _L, _L, _L, _P, _P, _P, _P, _L, _P, _P, _L, _P], _I),
    "ic_dynamic_quantize": ([_P, _I, _L, _L, _L, _P, _L, _P, _P], _I),
    "ic_norm_quantize": ([_P, _I, _L, _L, _L, _I, _P, _P, ctypes.c_float, _P, _L, _P, _P], _I),
    "ic_norm_rotate_quantize": ([_P, _I, _L, _L, _L, _I, _P, _P, ctypes.c_float, _P, _P, _I, _L, _P, _P, _L,
                                 _P, _P], _I),
    "ic_gemm_w8a8": ([_P, _L, _L, _L, _P, _L, _L, _P, _P, _P, _I, _P, _I, _L, _P], _I),
    "ic_gemm_w4a8": ([_P, _L, _L, _L, _P, _L, _L, _P, _L, _P, _P, _I, _P, _I, _L, _P], _I),
    "ic_gemm_splitk_bytes": ([_L, _L, _L, _L, _I], _L),
    "ic_gemm_w8a8_ws": ([_P, _L, _L, _L, _P, _L, _L, _P, _P, _P, _I, _P, _I, _L, _P, _L, _P], _I),
    "ic_gemm_w4a8_ws": ([_P, _L, _L, _L, _P, _L, _L, _P, _L, _P, _P, _I, _P, _I, _L, _P, _L, _P], _I),
    "ic_init_device": ([], _I),
    "ic_gemm_w4a8_noalloc": ([_P, _L, _L, _L, _P, _L, _L, _P, _L, _P, _P, _I, _P, _I, _L, _P], _I),
    "ic_gemm_w8a8_ex": ([_P, _L, _L, _L, _P, _L, _L, _P, _P, _P, _I, _I, _P, _I, _L, _P, _I, _L, _P, _L, _P], _I),
    "ic_gemm_w4a8_ex": ([_P, _L, _L, _L, _P, _L, _L, _P, _L, _P, _P, _I, _I, _P, _I, _L, _P, _I, _L, _P, _L,
                         _P], _I),
    "ic_int4_interleave_k": ([_P, _L, _L, _L, _P, _L, _P], _I),
    "ic_gemm_w4a8_kil_ex": ([_P, _L, _L, _L, _P, _L, _L, _P, _L, _P, _P, _I, _I, _P, _I, _L, _P, _I, _L, _P, _L,
                             _P], _I),
    "ic_gemm_w4a8_unpacked_ex": ([_P, _L, _L, _L, _P, _L, _L, _P, _L, _P, _P, _I, _I, _P, _I, _L, _P, _I, _L, _P,
                                  _L, _P], _I),
    "ic_gemm_w8a8_chain": ([_P, _L, _L, _L, _P, _L, _L, _P, _P, _P, _I, _I, _P, _P, _I, _P, _I, _L, _P], _I),
    "ic_gemm_w4a8_chain": ([_P, _L, _L, _L, _P, _L, _L, _P, _L, _P, _P, _I, _I, _P, _P, _I, _P, _I, _L, _P], _I),
    "ic_gemm_w4a16": ([_P, _I, _L, _L, _L, _P, _L, _L, _P, _L, _P, _I, _P, _L, _P], _I),
    "ic_w4a16_stage_layout": ([_P, _L, _L, _L, _P, _L, _P, _P, _P], _I),
    "ic_gemm_w4a16_staged": ([_P, _I, _L, _L, _L, _P, _L, _P, _L, _P, _I, _P, _L, _P], _I),
    "ic_unpack_int4_to_int8": ([_P, _L, _L, _L, _P, _L, _P], _I),
    "ic_unpack_int4_to_float": ([_P, _P, _L, _L, _L, _L, _P, _I, _L, _P], _I),
    "ic_f6_activation_bytes": ([_L, _L], _L),
    "ic_f6_weight_bytes": ([_L, _L], _L),
    "ic_f6_split_activations": ([_P, _L, _L, _L, _P, _P], _I),
    "ic_f6_repack_weights": ([_P, _L, _L, _L, _P, _P], _I),
    "ic_gemm_w4a8_f6": ([_P, _L, _L, _P, _L, _P, _L, _P, _P, _I, _P, _I, _L, _P], _I),
    "ic_gemm_w8a8_acc_i32": ([_P, _L, _L, _L, _P, _L, _L, _P, _I, _P], _I),
    "ic_gemm_w4a8_acc_i32": ([_P, _L, _L, _L, _P, _L, _L, _P, _L, _P, _I, _P], _I),
    "ic_gemm_w8a8_generic": ([_P, _L, _L, _L, _P, _L, _L, _P, _P, _P, _I, _P, _I, _L, _P], _I),
    "ic_gemv_w8a8": ([_P, _L, _L, _L, _P, _L, _L, _P, _P, _P, _I, _P, _I, _L, _P], _I),
    "ic_gemv_w4a8": ([_P, _L, _L, _L, _P, _L, _L, _P, _L, _P, _P, _I, _P, _I, _L, _P], _I),
    "ic_gemv_w4a16": ([_P, _I, _L, _L, _L, _P, _L, _L, _P, _L, _P, _I, _P, _L, _P], _I),
    "ic_prep_gemv_w4a8": ([_P, _I, _L, _L, _L, _P, _P, _I, _P, _P, _P, _P, _L, _L, _L, _P, _L, _P, _I, _I, _P, _I,
                           _L, _P, _I, _L, _P], _I),
    "ic_prep_gemv_w8a8": ([_P, _I, _L, _L, _L, _P, _P, _I, _P, _P, _P, _P, _L, _L, _L, _P, _P, _I, _I, _P, _I, _L,
                           _P, _I, _L, _P], _I),
}

_lib = None


def _load():
    lib = ctypes.CDLL(LIB_PATH)
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    return lib


def load_library(reload: bool = False):
    """(Re)load the shared library and refresh the availability flags."""
    global _lib, LOAD_ERROR
    if _lib is not None and not reload:
        return _lib
    try:
        _lib = _load()
        LOAD_ERROR = None
        log.info("[INT-Crush] HIP kernels loaded: %s", _lib.ic_version().decode())
    except (OSError, AttributeError) as exc:
        _lib = None
        LOAD_ERROR = f"{type(exc).__name__}: {exc}"
        log.debug("[INT-Crush] HIP kernels not available: %s", LOAD_ERROR)
    _set_flags(_lib is not None)
    return _lib


def _set_flags(ok: bool) -> None:
    g = globals()
    for name in ("KERNELS_AVAILABLE", "HIP_DYNQUANT", "HIP_ROTATE_QUANT", "HIP_INT8_GEMM",
                 "HIP_W4A8_GEMM", "HIP_W4A16_GEMM", "HIP_INT4_UNPACK", "HIP_INT4_INT8_UNPACK",
                 "HIP_FUSED_QGD"):
        g[name] = ok
    # reference flag names (_triton_runtime.py:16-22, :74-81)
    g["TRITON_AVAILABLE"] = ok
    g["TRITON_INT4_UNPACK"] = ok
    g["TRITON_INT8_GEMM"] = ok
    g["TRITON_INT4_INT8_UNPACK"] = ok
    g["TRITON_DYNQUANT"] = ok
    g["TRITON_W4A8_GEMM"] = ok
    g["TRITON_FUSED_QGD"] = ok


TRITON_AVAILABLE = TRITON_INT4_UNPACK = TRITON_INT8_GEMM = TRITON_INT4_INT8_UNPACK = False
TRITON_DYNQUANT = TRITON_W4A8_GEMM = TRITON_FUSED_QGD = False
load_library()


# ── helpers ─────────────────────────────────────────────────────────────────
def lib():
    if _lib is None:
        raise RuntimeError(
            f"INT-Crush gfx950 kernels are not loaded ({LOAD_ERROR}); build them with "
            "__graft_entry__.build() or comfyui-int-crush_amd/_build_lib.py")
    return _lib


def _ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _call(name: str, *args) -> None:
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        raise RuntimeError(f"[INT-Crush] {name} failed ({rc}): {lib().ic_last_error().decode()}")


def _dt(t: torch.dtype, who: str) -> int:
    if t not in _DT_CODE:
        raise TypeError(f"{who}: unsupported dtype {t} (expected float16, bfloat16 or float32)")
    return _DT_CODE[t]


def _need_cuda(*tensors: torch.Tensor | None) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("INT-Crush HIP kernels need device tensors; got a CPU tensor")


def _rows(t: torch.Tensor) -> torch.Tensor:
    """2-D view with unit column stride (copy only when required)."""
    t2 = t.reshape(-1, t.shape[-1])
    if t2.stride(-1) != 1 or (t2.shape[0] > 1 and t2.stride(0) < t2.shape[1]):
        t2 = t2.contiguous()
    return t2


def _alloc_or_reuse(shape, dtype, device, existing):
    """kernels/triton_quantize.py:57-66: reuse a matching pre-allocated buffer."""
    if existing is not None and tuple(existing.shape) == tuple(shape) and existing.dtype == dtype:
        return existing
    return torch.empty(shape, dtype=dtype, device=device)


# ── SmoothRot / SmoothQuant factors ─────────────────────────────────────────
class PreparedFactors:
    """Per-channel divide factors rounded to the activation dtype plus their
    reciprocals (ic_smoothrot_prepare); built once per layer and dtype."""

    __slots__ = ("fdt", "rcp", "dtype", "K")

    def __init__(self, factors: torch.Tensor, dtype: torch.dtype):
        _need_cuda(factors)
        f = factors.detach().reshape(-1).to(torch.float32).contiguous()
        self.K = f.numel()
        self.dtype = dtype
        self.fdt = torch.empty_like(f)
        self.rcp = torch.empty_like(f)
        with torch.cuda.device(f.device):
            _call("ic_smoothrot_prepare", _ptr(f), self.K, _dt(dtype, "prepare_factors"),
                  _ptr(self.fdt), _ptr(self.rcp), _stream(f))


def prepare_factors(factors: torch.Tensor | None, dtype: torch.dtype) -> PreparedFactors | None:
    return None if factors is None else PreparedFactors(factors, dtype)


def prepare_perm(perm: torch.Tensor | None, width: int | None = None) -> torch.Tensor | None:
    """PermuQuant indices as a contiguous int32 device tensor, range-checked once."""
    if perm is None:
        return None
    p = perm.detach().reshape(-1)
    if width is not None and p.numel() != width:
        raise ValueError(f"perm has {p.numel()} entries, expected {width}")
    if p.numel() and (int(p.min()) < 0 or int(p.max()) >= p.numel()):
        raise ValueError("perm entries must lie in [0, len(perm))")
    return p.to(torch.int32).contiguous()


# ── fused prep + quantization ───────────────────────────────────────────────
def _prep_shape(x2: torch.Tensor, rot_size: int, w_in: int | None, smoothrot: PreparedFactors | None,
                perm: torch.Tensor | None, smooth: PreparedFactors | None, who: str) -> tuple[int, int, int]:
    """Checks of the preparation arguments; returns (rot_size, K_w, dtype code)."""
    K_in = x2.shape[1]
    R = int(rot_size)
    if R not in VALID_ROT_SIZES:
        raise ValueError(f"rot_size must be one of {VALID_ROT_SIZES}, got {R}")
    K_r = ((K_in + R - 1) // R) * R if R else K_in
    K_w = max(int(w_in) if w_in is not None else K_r, K_r)
    dt = _dt(x2.dtype, who)
    for f in (smoothrot, smooth):
        if f is not None and f.dtype != x2.dtype:
            raise ValueError("prepared factors were built for another activation dtype")
    if smoothrot is not None and smoothrot.K != K_in:
        raise ValueError(f"SmoothRot factors have {smoothrot.K} entries, expected {K_in}")
    if smooth is not None and smooth.K != K_w:
        raise ValueError(f"smooth factors have {smooth.K} entries, expected {K_w}")
    if perm is not None and (perm.dtype != torch.int32 or perm.numel() != K_w or not perm.is_cuda):
        raise ValueError("perm must be an int32 device tensor of length w_in (see prepare_perm)")
    return R, K_w, dt


def rotate_quantize(x: torch.Tensor, *, rot_size: int = 0, w_in: int | None = None,
                    smoothrot: PreparedFactors | None = None, perm: torch.Tensor | None = None,
                    smooth: PreparedFactors | None = None, s_a_out: torch.Tensor | None = None,
                    x_int8_out: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """SmoothRot divide -> Hadamard(rot_size) -> pad to w_in -> perm gather ->
    old-smooth divide -> per-token INT8 quant, one kernel (one HBM pass).

    Semantics of _ops.py:337-365 + :529-533 followed by
    dynamic_quantize_activation (kernels/triton_quantize.py:151-198).
    Returns (x_int8 [M, w_in], s_a [M] float32).
    """
    _need_cuda(x)
    x2 = _rows(x)
    M, K_in = x2.shape
    R, K_w, dt = _prep_shape(x2, rot_size, w_in, smoothrot, perm, smooth, "rotate_quantize")
    s_a = _alloc_or_reuse((M,), torch.float32, x2.device, s_a_out)
    q = _alloc_or_reuse((M, K_w), torch.int8, x2.device, x_int8_out)
    with torch.cuda.device(x2.device):
        if K_w <= _fused_limit(dt):
            _call("ic_rotate_quantize", _ptr(x2), dt, M, K_in, x2.stride(0),
                  _ptr(smoothrot.rcp) if smoothrot else None, _ptr(smoothrot.fdt) if smoothrot else None,
                  R, K_w, _ptr(perm), _ptr(smooth.rcp) if smooth else None,
                  _ptr(smooth.fdt) if smooth else None, _ptr(q), q.stride(0), _ptr(s_a), _stream(x2))
        else:
            y = _rotate_wide(x2, R, smoothrot, dt)
            _call("ic_permute_quantize", _ptr(y), dt, M, y.shape[1], y.stride(0), K_w, _ptr(perm),
                  _ptr(smooth.rcp) if smooth else None, _ptr(smooth.fdt) if smooth else None,
                  _ptr(q), q.stride(0), _ptr(s_a), None, 0, _stream(y))
    return q, s_a


def _fused_limit(dt: int) -> int:
    """Widest row the single-pass prep kernels hold."""
    return lib().ic_max_fused_row() // (2 if dt == IC_DTYPE_F32 else 1)


def _rotate_wide(x2: torch.Tensor, R: int, smoothrot: PreparedFactors | None, dt: int) -> torch.Tensor:
    """SmoothRot divide + block Hadamard of rows wider than the single-pass
    kernels hold, into [M, K_r] in x's dtype: the rotation is block-diagonal,
    so ic_prepare_activation runs on column chunks of whole blocks.  The pad,
    perm gather and old-SmoothQuant divide follow in ic_permute_quantize."""
    M, K_in = x2.shape
    K_r = ((K_in + R - 1) // R) * R if R else K_in
    lim = _fused_limit(dt)
    step = (lim // R) * R if R else lim
    y = torch.empty(M, K_r, dtype=x2.dtype, device=x2.device)
    for c0 in range(0, K_r, step):
        kin = min(step, K_in - c0)
        kw = min(step, K_r - c0)
        _call("ic_prepare_activation", _ptr(x2[:, c0:]), dt, M, kin, x2.stride(0),
              _ptr(smoothrot.rcp[c0:]) if smoothrot else None, _ptr(smoothrot.fdt[c0:]) if smoothrot else None,
              R, kw, None, None, None, _ptr(y[:, c0:]), y.stride(0), _stream(x2))
    return y


def prepare_activation(x: torch.Tensor, *, rot_size: int = 0, w_in: int | None = None,
                       smoothrot: PreparedFactors | None = None, perm: torch.Tensor | None = None,
                       smooth: PreparedFactors | None = None,
                       out: torch.Tensor | None = None) -> torch.Tensor:
    """_prep_activation (_ops.py:337-365) on the GPU, result in x.dtype [M, w_in]."""
    _need_cuda(x)
    x2 = _rows(x)
    M, K_in = x2.shape
    R = int(rot_size)
    if R not in VALID_ROT_SIZES:
        raise ValueError(f"rot_size must be one of {VALID_ROT_SIZES}, got {R}")
    K_r = ((K_in + R - 1) // R) * R if R else K_in
    K_w = max(int(w_in) if w_in is not None else K_r, K_r)
    dt = _dt(x2.dtype, "prepare_activation")
    if perm is not None and (perm.dtype != torch.int32 or perm.numel() != K_w):
        raise ValueError("perm must be an int32 device tensor of length w_in (see prepare_perm)")
    y = _alloc_or_reuse((M, K_w), x2.dtype, x2.device, out)
    with torch.cuda.device(x2.device):
        if K_w <= _fused_limit(dt):
            _call("ic_prepare_activation", _ptr(x2), dt, M, K_in, x2.stride(0),
                  _ptr(smoothrot.rcp) if smoothrot else None, _ptr(smoothrot.fdt) if smoothrot else None,
                  R, K_w, _ptr(perm), _ptr(smooth.rcp) if smooth else None,
                  _ptr(smooth.fdt) if smooth else None, _ptr(y), y.stride(0), _stream(x2))
        else:
            yr = _rotate_wide(x2, R, smoothrot, dt)
            _call("ic_permute_quantize", _ptr(yr), dt, M, yr.shape[1], yr.stride(0), K_w, _ptr(perm),
                  _ptr(smooth.rcp) if smooth else None, _ptr(smooth.fdt) if smooth else None,
                  None, 0, None, _ptr(y), y.stride(0), _stream(yr))
    return y


def _cpu_per_row_int8_quant(x: torch.Tensor):
    """Reference CPU semantics, kernels/triton_quantize.py:43-54 (torch.round)."""
    s_a = x.abs().amax(dim=1).clamp(min=1e-8) / 127.0
    x_int8 = (x / s_a.unsqueeze(1)).round().clamp(-128, 127).to(torch.int8)
    return x_int8, s_a


def dynamic_quantize_activation(x: torch.Tensor, s_a_out: torch.Tensor | None = None,
                                x_int8_out: torch.Tensor | None = None):
    """kernels/triton_quantize.py:151-198: per-token symmetric INT8, s = max|x|/127.

    Device tensors run the gfx950 kernel (rounding q = trunc(x/s +- 0.5), the
    reference GPU rule); CPU tensors follow the reference CPU branch.
    """
    orig_shape = x.shape
    x2 = x.reshape(-1, x.shape[-1])
    M, K = x2.shape
    if not x2.is_cuda:
        q, s = _cpu_per_row_int8_quant(x2.to(torch.float32))
    else:
        x2 = _rows(x2)
        s = _alloc_or_reuse((M,), torch.float32, x2.device, s_a_out)
        q = _alloc_or_reuse((M, K), torch.int8, x2.device, x_int8_out)
        with torch.cuda.device(x2.device):
            _call("ic_dynamic_quantize", _ptr(x2), _dt(x2.dtype, "dynamic_quantize_activation"), M, K,
                  x2.stride(0), _ptr(q), q.stride(0), _ptr(s), _stream(x2))
    if orig_shape != x2.shape:
        q = q.reshape(orig_shape)
        s = s.reshape(*orig_shape[:-1])
    return q, s


# ── normalisation fused with quantization (kernels/triton_quantize.py:201-567) ──
IC_NORM_LAYER, IC_NORM_RMS, IC_SOFTMAX = 1, 2, 3


def _f32_vec(t: torch.Tensor | None, K: int, who: str, device) -> torch.Tensor | None:
    if t is None:
        return None
    v = t.detach().reshape(-1)
    if v.numel() != K:
        raise ValueError(f"{who} has {v.numel()} entries, expected {K}")
    return v.to(device=device, dtype=torch.float32).contiguous()


def _norm_quantize(x: torch.Tensor, kind: int, gamma, beta, eps: float, s_a_out, x_int8_out, who: str):
    orig_shape = x.shape
    x2 = _rows(x)
    M, K = x2.shape
    s = _alloc_or_reuse((M,), torch.float32, x2.device, s_a_out)
    q = _alloc_or_reuse((M, K), torch.int8, x2.device, x_int8_out)
    g = _f32_vec(gamma, K, "gamma", x2.device)
    b = _f32_vec(beta, K, "beta", x2.device)
    with torch.cuda.device(x2.device):
        _call("ic_norm_quantize", _ptr(x2), _dt(x2.dtype, who), M, K, x2.stride(0), kind, _ptr(g), _ptr(b),
              float(eps), _ptr(q), q.stride(0), _ptr(s), _stream(x2))
    if orig_shape != x2.shape:
        q = q.reshape(orig_shape)
        s = s.reshape(*orig_shape[:-1])
    return q, s


def norm_rotate_quantize(x: torch.Tensor, *, norm: str = "layer", weight: torch.Tensor | None = None,
                         bias: torch.Tensor | None = None, eps: float = 1e-6, rot_size: int = 0,
                         w_in: int | None = None, smoothrot: PreparedFactors | None = None,
                         perm: torch.Tensor | None = None, s_a_out: torch.Tensor | None = None,
                         x_int8_out: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """LayerNorm ("layer") or RMSNorm ("rms") of each row, optional affine
    (adaptive LayerNorm passes weight = 1 + scale, bias = shift), rounded once to
    x.dtype, then rotate_quantize on the result -- one kernel, one HBM pass.

    Equals rotate_quantize(RN_dtype(norm(x) * weight + bias), ...) with the row
    statistics in fp64; the block-input fusion in front of the prep of
    _ops.py:337-365 (no reference entry point fuses the two).  f16/bf16 rows,
    K and w_in multiples of 16.  Returns (x_int8 [M, w_in], s_a [M] float32)."""
    _need_cuda(x)
    kind = {"layer": IC_NORM_LAYER, "rms": IC_NORM_RMS}.get(norm)
    if kind is None:
        raise ValueError(f"norm must be 'layer' or 'rms', got {norm!r}")
    x2 = _rows(x)
    M, K_in = x2.shape
    R = int(rot_size)
    if R not in VALID_ROT_SIZES:
        raise ValueError(f"rot_size must be one of {VALID_ROT_SIZES}, got {R}")
    K_r = ((K_in + R - 1) // R) * R if R else K_in
    K_w = max(int(w_in) if w_in is not None else K_r, K_r)
    dt = _dt(x2.dtype, "norm_rotate_quantize")
    if smoothrot is not None and (smoothrot.dtype != x2.dtype or smoothrot.K != K_in):
        raise ValueError("SmoothRot factors were prepared for another dtype or width")
    if perm is not None and (perm.dtype != torch.int32 or perm.numel() != K_w or not perm.is_cuda):
        raise ValueError("perm must be an int32 device tensor of length w_in (see prepare_perm)")
    w = _f32_vec(weight, K_in, "weight", x2.device)
    b = _f32_vec(bias, K_in, "bias", x2.device)
    s_a = _alloc_or_reuse((M,), torch.float32, x2.device, s_a_out)
    q = _alloc_or_reuse((M, K_w), torch.int8, x2.device, x_int8_out)
    with torch.cuda.device(x2.device):
        _call("ic_norm_rotate_quantize", _ptr(x2), dt, M, K_in, x2.stride(0), kind, _ptr(w), _ptr(b), float(eps),
              _ptr(smoothrot.rcp) if smoothrot else None, _ptr(smoothrot.fdt) if smoothrot else None, R, K_w,
              _ptr(perm), _ptr(q), q.stride(0), _ptr(s_a), _stream(x2))
    return q, s_a


def _cpu_quant_reshaped(y: torch.Tensor, orig_shape):
    q, s = _cpu_per_row_int8_quant(y.reshape(-1, y.shape[-1]).float())
    return q.reshape(orig_shape), s.reshape(*orig_shape[:-1])


def fused_layernorm_quantize(x: torch.Tensor, gamma: torch.Tensor, beta: torch.Tensor | None = None,
                             eps: float = 1e-5, s_a_out: torch.Tensor | None = None,
                             x_int8_out: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """LayerNorm over the last dim fused with per-row INT8 quantization
    (kernels/triton_quantize.py:277-345).  Device tensors run ic_norm_quantize
    (statistics in fp64, y in f32, quantized without rounding y to x's dtype,
    as the reference GPU kernel does); CPU tensors follow the reference CPU
    branch (F.layer_norm in f32, rounded to x's dtype, then torch.round)."""
    if not x.is_cuda:
        K = x.shape[-1]
        y = torch.nn.functional.layer_norm(x.to(torch.float32), (K,), gamma.to(torch.float32),
                                           beta.to(torch.float32) if beta is not None else None, eps)
        return _cpu_quant_reshaped(y.to(x.dtype), x.shape)
    return _norm_quantize(x, IC_NORM_LAYER, gamma, beta, eps, s_a_out, x_int8_out, "fused_layernorm_quantize")


def fused_rmsnorm_quantize(x: torch.Tensor, gamma: torch.Tensor, eps: float = 1e-6,
                           s_a_out: torch.Tensor | None = None,
                           x_int8_out: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """RMSNorm x / sqrt(mean(x^2) + eps) * gamma fused with per-row INT8
    quantization (kernels/triton_quantize.py:397-459); CPU tensors follow the
    reference CPU branch."""
    if not x.is_cuda:
        xf = x.to(torch.float32)
        rms = torch.sqrt(torch.mean(xf * xf, dim=-1, keepdim=True) + eps)
        return _cpu_quant_reshaped((xf / rms * gamma.to(torch.float32)).to(x.dtype), x.shape)
    return _norm_quantize(x, IC_NORM_RMS, gamma, None, eps, s_a_out, x_int8_out, "fused_rmsnorm_quantize")


def fused_softmax_quantize(x: torch.Tensor, s_a_out: torch.Tensor | None = None,
                           x_int8_out: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Softmax over the last dim fused with per-row INT8 quantization
    (kernels/triton_quantize.py:518-567); CPU tensors follow the reference
    CPU branch (f32 softmax, then torch.round)."""
    if not x.is_cuda:
        return _cpu_quant_reshaped(torch.softmax(x.to(torch.float32), dim=-1), x.shape)
    return _norm_quantize(x, IC_SOFTMAX, None, None, 0.0, s_a_out, x_int8_out, "fused_softmax_quantize")


# ── GEMMs ───────────────────────────────────────────────────────────────────
def _bias_args(bias: torch.Tensor | None, N: int):
    if bias is None:
        return None, 0, None
    b = bias.detach().reshape(-1)
    if b.numel() != N:
        raise ValueError(f"bias has {b.numel()} entries, expected {N}")
    b = b.contiguous()
    return _ptr(b), _dt(b.dtype, "bias"), b


def _out_buffer(out, M, N, out_dtype, device):
    if out is not None:
        assert tuple(out.shape) == (M, N), f"out shape mismatch: {tuple(out.shape)} vs ({M}, {N})"
        assert out.stride(-1) == 1, "out must have unit column stride"
        return out
    return torch.empty((M, N), dtype=out_dtype, device=device)


def _splitk_workspace(M: int, N: int, K: int, G: int, int4: bool, device) -> tuple[torch.Tensor | None, int]:
    """Workspace for the split-K form of the GEMM when the library plans one
    (small M: too few output tiles to occupy the GPU); (None, 0) otherwise.
    Allocated from torch's caching allocator, so it is graph-capture safe."""
    nb = int(lib().ic_gemm_splitk_bytes(M, N, K, G, 1 if int4 else 0))
    if nb <= 0:
        return None, 0
    return torch.empty(nb, dtype=torch.uint8, device=device), nb


# Epilogue activation codes (kernels/triton_int8_gemm.py:24-27 for 0-2).
ACT_NONE, ACT_SILU, ACT_GELU, ACT_GELU_TANH = 0, 1, 2, 3


def _epilogue_args(activation: int, residual: torch.Tensor | None, M: int, N: int):
    """Checked activation code and residual (pointer, dtype code, row stride,
    tensor kept alive) for the ic_gemm_*_ex entry points."""
    act = int(activation)
    if act not in (ACT_NONE, ACT_SILU, ACT_GELU, ACT_GELU_TANH):
        raise ValueError(f"activation must be 0 (none), 1 (SiLU), 2 (GELU) or 3 (GELU tanh), got {activation}")
    if residual is None:
        return act, None, 0, 0, None
    r = residual.detach()
    if r.dim() != 2:
        r = r.reshape(-1, r.shape[-1])
    if tuple(r.shape) != (M, N):
        raise ValueError(f"residual shape {tuple(residual.shape)} does not match the output ({M}, {N})")
    if r.stride(-1) != 1 or r.stride(0) < N:
        r = r.contiguous()
    return act, _ptr(r), _dt(r.dtype, "residual"), r.stride(0), r


def fused_int8_gemm_dequant(x_int8: torch.Tensor, w_int8: torch.Tensor, s_w: torch.Tensor,
                            s_a: torch.Tensor, bias: torch.Tensor | None = None,
                            out_dtype: torch.dtype = torch.bfloat16, activation: int = 0,
                            residual: torch.Tensor | None = None,
                            out: torch.Tensor | None = None) -> torch.Tensor:
    """W8A8: f32(x_int8 @ w_int8^T) * (s_a[m] * s_w[n]) + bias, then the
    optional activation and residual add in f32, cast to out_dtype.

    Signature of kernels/triton_int8_gemm.py:135-205, epilogue :119-130:
    activation 0 none, 1 SiLU, 2 GELU (erf); 3 adds GELU with the tanh
    approximation.  residual [M, N] f16/bf16/f32 is added after the activation.
    """
    assert x_int8.dtype == torch.int8, f"x_int8 must be int8, got {x_int8.dtype}"
    assert w_int8.dtype == torch.int8, f"w_int8 must be int8, got {w_int8.dtype}"
    _need_cuda(x_int8, w_int8, s_w, s_a, bias, residual)
    M, K = x_int8.shape
    N, K_w = w_int8.shape
    assert K == K_w, f"K mismatch: {K} vs {K_w}"
    xq = _rows(x_int8)
    w = _rows(w_int8)
    sw = s_w.detach().reshape(-1).to(torch.float32).contiguous()
    if sw.numel() != N:
        raise ValueError(f"s_w must hold one scale per output channel ({N}), got {sw.numel()}")
    sa = s_a.detach().reshape(-1).to(torch.float32).contiguous()
    bp, bdt, _keep = _bias_args(bias, N)
    act, rp, rdt, ldr, _rkeep = _epilogue_args(activation, residual, M, N)
    c = _out_buffer(out, M, N, out_dtype, x_int8.device)
    _warn_if_scalar_gemm("fused_int8_gemm_dequant", K, 1, xq, w)
    with torch.cuda.device(xq.device):
        ws, nb = _splitk_workspace(M, N, K, 1, False, xq.device)
        _call("ic_gemm_w8a8_ex", _ptr(xq), M, K, xq.stride(0), _ptr(w), N, w.stride(0), _ptr(sa),
              _ptr(sw), bp, bdt, act, rp, rdt, ldr, _ptr(c), _dt(c.dtype, "out"), c.stride(0), _ptr(ws), nb,
              _stream(xq))
    return c


def int8_gemm_int8out(x_int8: torch.Tensor, w_int8: torch.Tensor, s_w: torch.Tensor, s_a: torch.Tensor,
                      c_out: torch.Tensor | None = None,
                      s_c_out: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """W8A8 GEMM re-quantized to INT8 with a per-row scale, for chained GEMMs
    (kernels/triton_int8_gemm.py:392-536; the returned s_c is the next GEMM's s_a).

    The reference documents it as fused_int8_gemm_dequant followed by
    dynamic_quantize_activation; its kernel computes the row abs-max inside
    each N-tile and every tile writes s_c, so the last tile's scale wins and
    the other tiles' codes use their own.  Here the scale is the abs-max of
    the whole row, exactly that documented equivalence: the W8A8 GEMM writes
    the f32 dequantized values (no bias) into a temporary, then the per-token
    quantizer (q = trunc(v / s +- 0.5), s = max(|v|, 1e-8) / 127) runs on it.
    """
    assert x_int8.dtype == torch.int8, f"x_int8 must be int8, got {x_int8.dtype}"
    assert w_int8.dtype == torch.int8, f"w_int8 must be int8, got {w_int8.dtype}"
    M, K = x_int8.shape
    N, K_w = w_int8.shape
    assert K == K_w, f"K mismatch: {K} vs {K_w}"
    if c_out is not None:
        assert tuple(c_out.shape) == (M, N), f"c_out shape mismatch: {tuple(c_out.shape)} vs ({M}, {N})"
        assert c_out.dtype == torch.int8, f"c_out must be int8, got {c_out.dtype}"
    if s_c_out is not None:
        assert tuple(s_c_out.shape) == (M,), f"s_c_out shape mismatch: {tuple(s_c_out.shape)} vs ({M},)"
        assert s_c_out.dtype == torch.float32, f"s_c_out must be float32, got {s_c_out.dtype}"
    v = fused_int8_gemm_dequant(x_int8, w_int8, s_w, s_a, out_dtype=torch.float32)
    return dynamic_quantize_activation(v, s_a_out=s_c_out, x_int8_out=c_out)


def fused_w4a8_gemm_dequant(x_int8, w_int8, s_w, s_a, bias=None, out_dtype=torch.bfloat16, out=None,
                            activation: int = 0, residual: torch.Tensor | None = None):
    """kernels/triton_w4a8_gemm.py:111-169: the INT8 GEMM on already unpacked
    INT4 weights ([N, K] int8, per-row s_w).  gemm_w4a8 is the fused path."""
    return fused_int8_gemm_dequant(x_int8, w_int8, s_w, s_a, bias=bias, out_dtype=out_dtype,
                                   activation=activation, residual=residual, out=out)


_SCALAR_WARNED: set = set()


def _warn_if_scalar_gemm(who: str, K: int, G: int, *tensors: torch.Tensor, out64: bool = False) -> None:
    """The INT8 / W4A8 GEMMs run MFMA tiles only for K a multiple of 128,
    group sizes that are multiples of 128 (W4A8 also odd multiples of 64 or
    of 32 when out64: a 16-bit output whose rows and residual suit the
    288 x 192 tile's staged stores) and 16-byte aligned operands and row
    strides; anything else takes the scalar kernel (one thread per output,
    ~100x slower).  Log that once per shape instead of running it silently."""
    gs = K // G
    ok = K % 128 == 0 and (G == 1 or gs % 128 == 0 or (out64 and gs % 32 == 0))
    for t in tensors:
        ok = ok and t.data_ptr() % 16 == 0 and (t.dim() < 2 or (t.stride(0) * t.element_size()) % 16 == 0)
    key = (who, K, G)
    if not ok and key not in _SCALAR_WARNED:
        _SCALAR_WARNED.add(key)
        log.warning("[INT-Crush] %s: K=%d, group size %d or operand alignment has no MFMA tiling; "
                    "running the scalar fallback kernel (about 100x slower)", who, K, gs)


def int4_interleave_k(w_packed: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """Packed INT4 rows [N, K/2] (checkpoint nibble order) -> the same weights
    in the K-interleaved order gemm_w4a8(..., kil=True) takes
    (ic_int4_interleave_k): byte 4d + j holds k = 8d + j low and 8d + 4 + j
    high.  out may be w_packed itself."""
    assert w_packed.dtype == torch.uint8 and w_packed.dim() == 2, "w_packed must be uint8 [N, K/2]"
    _need_cuda(w_packed)
    N, half = w_packed.shape
    if (2 * half) % 8:
        raise ValueError(f"int4_interleave_k: K={2 * half} must be a multiple of 8")
    w = w_packed if w_packed.stride(1) == 1 else w_packed.contiguous()
    o = out if out is not None else torch.empty_like(w, memory_format=torch.contiguous_format)
    assert o.shape == w.shape and o.dtype == torch.uint8 and o.stride(1) == 1, "out must be uint8 [N, K/2]"
    with torch.cuda.device(w.device):
        _call("ic_int4_interleave_k", _ptr(w), N, 2 * half, w.stride(0), _ptr(o), o.stride(0), _stream(w))
    return o


def gemm_w4a8(x_int8: torch.Tensor, w_packed: torch.Tensor, s_w: torch.Tensor, s_a: torch.Tensor,
              bias: torch.Tensor | None = None, out_dtype: torch.dtype = torch.bfloat16,
              out: torch.Tensor | None = None, activation: int = 0,
              residual: torch.Tensor | None = None, kil: bool = False) -> torch.Tensor:
    """W4A8 with the INT4 unpack fused into the GEMM.

    w_packed [N, K/2] uint8; s_w [N, G] (or [N]) float scales, group size K/G.
    out = (sum_g f32(acc_g) * s_w[n,g]) * s_a[m] + bias  (G > 1)
    out = f32(acc) * (s_a[m] * s_w[n]) + bias           (G == 1)
    then the activation and residual of fused_int8_gemm_dequant, in f32.
    kil: w_packed is in the K-interleaved nibble order (int4_interleave_k),
    which the kernels expand with fewer instructions; same outputs.
    """
    assert x_int8.dtype == torch.int8, f"x_int8 must be int8, got {x_int8.dtype}"
    assert w_packed.dtype == torch.uint8, f"w_packed must be uint8, got {w_packed.dtype}"
    _need_cuda(x_int8, w_packed, s_w, s_a, bias, residual)
    xq = _rows(x_int8)
    M, K = xq.shape
    N = w_packed.shape[0]
    assert w_packed.shape[1] * 2 >= K, f"packed weight too narrow for K={K}"
    w = _rows(w_packed)
    sw = s_w.detach().reshape(N, -1).to(torch.float32).contiguous()
    G = sw.shape[1]
    if K % G:
        raise ValueError(f"K={K} is not a multiple of the {G} scale groups")
    sa = s_a.detach().reshape(-1).to(torch.float32).contiguous()
    bp, bdt, _keep = _bias_args(bias, N)
    act, rp, rdt, ldr, _rkeep = _epilogue_args(activation, residual, M, N)
    c = _out_buffer(out, M, N, out_dtype, xq.device)
    out64 = (c.dtype != torch.float32 and N % 8 == 0 and c.data_ptr() % 16 == 0 and c.stride(0) % 8 == 0
             and (rp is None or (rdt != 2 and (rp.value or 0) % 16 == 0 and ldr % 8 == 0)))
    _warn_if_scalar_gemm("gemm_w4a8", K, G, xq, w, out64=out64)
    with torch.cuda.device(xq.device):
        ws, nb = _splitk_workspace(M, N, K, G, True, xq.device)
        _call("ic_gemm_w4a8_kil_ex" if kil else "ic_gemm_w4a8_ex", _ptr(xq), M, K, xq.stride(0), _ptr(w), N,
              w.stride(0), _ptr(sw), G, _ptr(sa), bp, bdt, act, rp, rdt, ldr, _ptr(c), _dt(c.dtype, "out"),
              c.stride(0), _ptr(ws), nb, _stream(xq))
    return c

def w4a8_unpacked_pays(M: int, N: int, K: int, G: int, device=None) -> bool:
    """Whether a W4A8 launch of M x N outputs over K runs faster on weights
    unpacked to one byte each (gemm_w4a8_unpacked) than on packed INT4: when
    its 288 x 192 tiles fill at most half the CUs (and the groups are whole
    128-column blocks, which the unpacked kernels need for their MFMA tiles).  There the L2 serves the doubled
    weight bytes without contention and the dropped in-loop INT4 expansion
    shows (measured on MI355X: 512 x 3072 x 3072 23.9 -> 19.2 us, 1024 x 3072
    x 12288 85 -> 67 us); on a full launch the two are level (C3 175 us each)
    or the packed form leads (the Wan FFN-down, 2 %)."""
    if M <= 16 or K % 128 or K % G or (G > 1 and (K // G) % 128):
        return False  # the GEMV reads the packed weights; other groups have their own fold modes
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    return ((M + 287) // 288) * ((N + 191) // 192) * 2 <= cus


def gemm_w4a8_unpacked(x_int8: torch.Tensor, w_int8: torch.Tensor, s_w: torch.Tensor, s_a: torch.Tensor,
                       bias: torch.Tensor | None = None, out_dtype: torch.dtype = torch.bfloat16,
                       out: torch.Tensor | None = None, activation: int = 0,
                       residual: torch.Tensor | None = None) -> torch.Tensor:
    """gemm_w4a8 on the INT4 weights unpacked to int8 [N, K] (unpack_int4_to_int8;
    ic_gemm_w4a8_unpacked_ex): the same outputs bit for bit, without the
    in-loop INT4 expansion and at twice the weight bytes (see
    w4a8_unpacked_pays).  s_w [N, G] group scales or [N] per-row scales."""
    assert x_int8.dtype == torch.int8, f"x_int8 must be int8, got {x_int8.dtype}"
    assert w_int8.dtype == torch.int8, f"w_int8 must be int8, got {w_int8.dtype}"
    _need_cuda(x_int8, w_int8, s_w, s_a, bias, residual)
    xq = _rows(x_int8)
    M, K = xq.shape
    N = w_int8.shape[0]
    assert w_int8.shape[1] >= K, f"unpacked weight too narrow for K={K}"
    w = _rows(w_int8)
    sw = s_w.detach().reshape(N, -1).to(torch.float32).contiguous()
    G = sw.shape[1]
    if K % G:
        raise ValueError(f"K={K} is not a multiple of the {G} scale groups")
    sa = s_a.detach().reshape(-1).to(torch.float32).contiguous()
    bp, bdt, _keep = _bias_args(bias, N)
    act, rp, rdt, ldr, _rkeep = _epilogue_args(activation, residual, M, N)
    c = _out_buffer(out, M, N, out_dtype, xq.device)
    _warn_if_scalar_gemm("gemm_w4a8_unpacked", K, G, xq, w)
    with torch.cuda.device(xq.device):
        ws, nb = _splitk_workspace(M, N, K, G, False, xq.device)
        _call("ic_gemm_w4a8_unpacked_ex", _ptr(xq), M, K, xq.stride(0), _ptr(w), N, w.stride(0), _ptr(sw), G,
              _ptr(sa), bp, bdt, act, rp, rdt, ldr, _ptr(c), _dt(c.dtype, "out"), c.stride(0), _ptr(ws), nb,
              _stream(xq))
    return c


def init_device(device=None) -> None:
    """Per-device set-up (ic_init_device) for `device` (default: the current
    one): resolves the no-alloc scratch address, so that code capturing
    ic_gemm_w4a8_noalloc into a graph does no lookup inside the capture."""
    with torch.cuda.device(device if device is not None else torch.cuda.current_device()):
        _call("ic_init_device")


def f6_split_activations(x_int8: torch.Tensor) -> torch.Tensor:
    """int8 codes [M, K] -> the e3m2 activation buffer of gemm_w4a8_f6
    (x = 16 h + l per code, blocked by 16 rows; ic_f6_split_activations)."""
    assert x_int8.dtype == torch.int8, f"x_int8 must be int8, got {x_int8.dtype}"
    _need_cuda(x_int8)
    xq = _rows(x_int8)
    M, K = xq.shape
    nb = lib().ic_f6_activation_bytes(M, K)
    if nb <= 0:
        raise ValueError(f"f6_split_activations: K={K} must be a positive multiple of 128")
    a6 = torch.empty(nb, dtype=torch.uint8, device=xq.device)
    with torch.cuda.device(xq.device):
        _call("ic_f6_split_activations", _ptr(xq), M, K, xq.stride(0), _ptr(a6), _stream(xq))
    return a6


def f6_repack_weights(w_packed: torch.Tensor, K: int) -> torch.Tensor:
    """Packed INT4 [N, K/2] -> the e3m2 weight buffer of gemm_w4a8_f6
    (blocked by 16 columns; ic_f6_repack_weights).  Once per layer."""
    assert w_packed.dtype == torch.uint8, f"w_packed must be uint8, got {w_packed.dtype}"
    _need_cuda(w_packed)
    w = _rows(w_packed)
    N = w.shape[0]
    nb = lib().ic_f6_weight_bytes(N, K)
    if nb <= 0:
        raise ValueError(f"f6_repack_weights: K={K} must be a positive multiple of 128")
    w6 = torch.zeros(nb, dtype=torch.uint8, device=w.device)
    with torch.cuda.device(w.device):
        _call("ic_f6_repack_weights", _ptr(w), N, K, w.stride(0), _ptr(w6), _stream(w))
    return w6


def gemm_w4a8_f6(a6: torch.Tensor, M: int, K: int, w6: torch.Tensor, N: int, s_w: torch.Tensor,
                 s_a: torch.Tensor, bias: torch.Tensor | None = None, out_dtype: torch.dtype = torch.bfloat16,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """Grouped W4A8 on e3m2 operands (ic_gemm_w4a8_f6): the outputs of
    gemm_w4a8 for the same codes, weights and group scales, bit for bit."""
    _need_cuda(a6, w6, s_w, s_a, bias)
    if a6.numel() < lib().ic_f6_activation_bytes(M, K) or w6.numel() < lib().ic_f6_weight_bytes(N, K):
        raise ValueError("gemm_w4a8_f6: operand buffers smaller than the M x K / N x K formats")
    sw = s_w.detach().reshape(N, -1).to(torch.float32).contiguous()
    sa = s_a.detach().reshape(-1).to(torch.float32).contiguous()
    bp, bdt, _keep = _bias_args(bias, N)
    c = _out_buffer(out, M, N, out_dtype, a6.device)
    with torch.cuda.device(a6.device):
        _call("ic_gemm_w4a8_f6", _ptr(a6), M, K, _ptr(w6), N, _ptr(sw), sw.shape[1], _ptr(sa), bp, bdt, _ptr(c),
              _dt(c.dtype, "out"), c.stride(0), _stream(a6))
    return c


CHAIN_ROT_SIZES = (16, 64, 256)


def gemm_chain(x_int8: torch.Tensor, w: torch.Tensor, s_w: torch.Tensor, s_a: torch.Tensor, *,
               rot_size: int, smoothrot: PreparedFactors | None = None, bias: torch.Tensor | None = None,
               out_dtype: torch.dtype = torch.bfloat16, activation: int = 0,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """Chained MLP epilogue (ic_gemm_w8a8_chain / ic_gemm_w4a8_chain): the
    up-projection GEMM whose output rows leave already prepared as the next
    linear's activation.

    w int8 [N, K] (W8A8, s_w [N]) or packed uint8 [N, K/2] (W4A8, s_w [N, G]).
    Each output h = RN_dt(act(dequant + bias)) as in fused_int8_gemm_dequant /
    gemm_w4a8 with `activation`, then divided by the next linear's SmoothRot
    factors (prepared for out_dtype; None: no divide) and rotated in blocks of
    rot_size (16, 64 or 256) columns, each step rounded to out_dtype: the
    first half of _prep_activation (_ops.py:337-365).  Returns y [M, N]; the
    down-projection's codes are then rotate_quantize(y, rot_size=0,
    w_in=K_w, perm=perm), which pads, gathers and takes the whole row's scale.
    """
    assert x_int8.dtype == torch.int8, f"x_int8 must be int8, got {x_int8.dtype}"
    _need_cuda(x_int8, w, s_w, s_a, bias)
    if out_dtype not in (torch.float16, torch.bfloat16):
        raise TypeError("gemm_chain writes the next linear's activation: float16 or bfloat16")
    R = int(rot_size)
    if R not in CHAIN_ROT_SIZES:
        raise ValueError(f"gemm_chain rotates blocks of {CHAIN_ROT_SIZES} columns, got rot_size={R}")
    if smoothrot is not None and smoothrot.dtype != out_dtype:
        raise ValueError("prepared SmoothRot factors were built for another activation dtype")
    xq = _rows(x_int8)
    M, K = xq.shape
    wr = _rows(w)
    N = wr.shape[0]
    if smoothrot is not None and smoothrot.K != N:
        raise ValueError(f"SmoothRot factors have {smoothrot.K} entries, expected N={N}")
    sa = s_a.detach().reshape(-1).to(torch.float32).contiguous()
    bp, bdt, _keep = _bias_args(bias, N)
    c = _out_buffer(out, M, N, out_dtype, xq.device)
    rp = _ptr(smoothrot.rcp) if smoothrot is not None else None
    fp = _ptr(smoothrot.fdt) if smoothrot is not None else None
    with torch.cuda.device(xq.device):
        if wr.dtype == torch.int8:
            assert wr.shape[1] == K, f"K mismatch: {K} vs {wr.shape[1]}"
            sw = s_w.detach().reshape(-1).to(torch.float32).contiguous()
            if sw.numel() != N:
                raise ValueError(f"s_w must hold one scale per output channel ({N}), got {sw.numel()}")
            _call("ic_gemm_w8a8_chain", _ptr(xq), M, K, xq.stride(0), _ptr(wr), N, wr.stride(0), _ptr(sa),
                  _ptr(sw), bp, bdt, int(activation), rp, fp, R, _ptr(c), _dt(c.dtype, "out"), c.stride(0),
                  _stream(xq))
        elif wr.dtype == torch.uint8:
            assert wr.shape[1] * 2 >= K, f"packed weight too narrow for K={K}"
            sw = s_w.detach().reshape(N, -1).to(torch.float32).contiguous()
            G = sw.shape[1]
            if K % G:
                raise ValueError(f"K={K} is not a multiple of the {G} scale groups")
            _call("ic_gemm_w4a8_chain", _ptr(xq), M, K, xq.stride(0), _ptr(wr), N, wr.stride(0), _ptr(sw), G,
                  _ptr(sa), bp, bdt, int(activation), rp, fp, R, _ptr(c), _dt(c.dtype, "out"), c.stride(0),
                  _stream(xq))
        else:
            raise TypeError(f"gemm_chain weights must be int8 or packed uint8, got {wr.dtype}")
    return c


def gemm_w4a16(x: torch.Tensor, w_packed: torch.Tensor, s_w: torch.Tensor,
               bias: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """W4A16: x @ RN_dt(q * RN_dt(s))^T (+ bias) in x.dtype (fp16/bf16)."""
    assert w_packed.dtype == torch.uint8, f"w_packed must be uint8, got {w_packed.dtype}"
    _need_cuda(x, w_packed, s_w, bias)
    x2 = _rows(x)
    M, K = x2.shape
    N = w_packed.shape[0]
    assert w_packed.shape[1] * 2 >= K, f"packed weight too narrow for K={K}"
    w = _rows(w_packed)
    sw = s_w.detach().reshape(N, -1).to(torch.float32).contiguous()
    G = sw.shape[1]
    if K % G:
        raise ValueError(f"K={K} is not a multiple of the {G} scale groups")
    dt = _dt(x2.dtype, "gemm_w4a16")
    if dt == IC_DTYPE_F32:
        raise TypeError("gemm_w4a16 needs float16 or bfloat16 activations")
    bp, bdt, _keep = _bias_args(bias, N)
    c = _out_buffer(out, M, N, x2.dtype, x2.device)
    with torch.cuda.device(x2.device):
        _call("ic_gemm_w4a16", _ptr(x2), dt, M, K, x2.stride(0), _ptr(w), N, w.stride(0), _ptr(sw), G,
              bp, bdt, _ptr(c), c.stride(0), _stream(x2))
    return c


def w4a16_staged_pays(M: int, N: int, K: int, G: int) -> bool:
    """Whether a W4A16 launch of M x N outputs over K takes the big-tile
    kernel that reads the staged operand layout (w4a16_stage_layout;
    ic_gemm_w4a16_staged): M above the GEMV and small-tile range, K and the
    group size multiples of 64, N a multiple of 8.  There it gives the same
    outputs bit for bit as gemm_w4a16, in fewer DMA cache-line requests per
    stage (measured on MI355X: C2 4608 x 12288 x 3072 f16 324 -> 314 us,
    4096 x 5120 x 5120 bf16 228 -> 211 us)."""
    return M > 128 and K % 64 == 0 and K % G == 0 and (G == 1 or (K // G) % 64 == 0) and N % 8 == 0


def w4a16_stage_layout(w_packed: torch.Tensor, s_w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Packed INT4 weights [N, K/2] and scales [N, G] -> the staged operand
    layout of gemm_w4a16_staged (ic_w4a16_stage_layout): weights stage-major
    [K/64, N, 32] (the 32 packed bytes of each row and 64-K stage), scales
    group-major [G, N].  A one-time copy, as the K-interleaved W4A8 form."""
    assert w_packed.dtype == torch.uint8, f"w_packed must be uint8, got {w_packed.dtype}"
    _need_cuda(w_packed, s_w)
    w = _rows(w_packed)
    N = w.shape[0]
    K = 2 * w.shape[1]
    sw = s_w.detach().reshape(N, -1).to(torch.float32).contiguous()
    G = sw.shape[1]
    ws = torch.empty(K // 64, N, 32, dtype=torch.uint8, device=w.device)
    ss = torch.empty(G, N, dtype=torch.float32, device=w.device)
    with torch.cuda.device(w.device):
        _call("ic_w4a16_stage_layout", _ptr(w), N, K, w.stride(0), _ptr(sw), G, _ptr(ws), _ptr(ss), _stream(w))
    return ws, ss


def gemm_w4a16_staged(x: torch.Tensor, w_staged: torch.Tensor, s_staged: torch.Tensor,
                      bias: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """gemm_w4a16 on the staged operand layout of w4a16_stage_layout
    (ic_gemm_w4a16_staged): the same outputs bit for bit, for the shapes
    w4a16_staged_pays admits (the entry point rejects the others)."""
    assert w_staged.dtype == torch.uint8 and w_staged.dim() == 3, "w_staged must be uint8 [K/64, N, 32]"
    _need_cuda(x, w_staged, s_staged, bias)
    x2 = _rows(x)
    M, K = x2.shape
    S, N, _ = w_staged.shape
    if 64 * S != K:
        raise ValueError(f"staged weights cover K={64 * S}, activations K={K}")
    ss = s_staged.detach().to(torch.float32).contiguous()
    G = ss.shape[0]
    dt = _dt(x2.dtype, "gemm_w4a16_staged")
    if dt == IC_DTYPE_F32:
        raise TypeError("gemm_w4a16_staged needs float16 or bfloat16 activations")
    bp, bdt, _keep = _bias_args(bias, N)
    c = _out_buffer(out, M, N, x2.dtype, x2.device)
    with torch.cuda.device(x2.device):
        _call("ic_gemm_w4a16_staged", _ptr(x2), dt, M, K, x2.stride(0), _ptr(w_staged.contiguous()), N, _ptr(ss), G,
              bp, bdt, _ptr(c), c.stride(0), _stream(x2))
    return c


# ── small-batch GEMV (M <= 16; the GEMM callables route there by themselves) ──
GEMV_MAX_M = 16


def gemv(x: torch.Tensor, w: torch.Tensor, s_w: torch.Tensor, s_a: torch.Tensor | None = None,
         bias: torch.Tensor | None = None, out_dtype: torch.dtype | None = None, *,
         kind: str) -> torch.Tensor:
    """Explicit GEMV entry points (ic_gemv_w8a8 / ic_gemv_w4a8 / ic_gemv_w4a16).

    kind "w8a8": x int8 codes [M, K], w int8 [N, K], s_w [N], s_a [M].
    kind "w4a8": x int8 codes, w packed uint8 [N, K/2], s_w [N, G] (G = 1 or K/128), s_a [M].
    kind "w4a16": x fp16/bf16 [M, K], w packed uint8, s_w [N, G]; out in x.dtype.
    """
    _need_cuda(x, w, s_w, s_a, bias)
    x2 = _rows(x)
    M, K = x2.shape
    wr = _rows(w)
    N = wr.shape[0]
    bp, bdt, _keep = _bias_args(bias, N)
    with torch.cuda.device(x2.device):
        if kind == "w4a16":
            sw = s_w.detach().reshape(N, -1).to(torch.float32).contiguous()
            c = torch.empty((M, N), dtype=x2.dtype, device=x2.device)
            _call("ic_gemv_w4a16", _ptr(x2), _dt(x2.dtype, "gemv"), M, K, x2.stride(0), _ptr(wr), N,
                  wr.stride(0), _ptr(sw), sw.shape[1], bp, bdt, _ptr(c), c.stride(0), _stream(x2))
            return c
        sa = s_a.detach().reshape(-1).to(torch.float32).contiguous()
        c = torch.empty((M, N), dtype=out_dtype or torch.bfloat16, device=x2.device)
        if kind == "w8a8":
            sw = s_w.detach().reshape(-1).to(torch.float32).contiguous()
            _call("ic_gemv_w8a8", _ptr(x2), M, K, x2.stride(0), _ptr(wr), N, wr.stride(0), _ptr(sa),
                  _ptr(sw), bp, bdt, _ptr(c), _dt(c.dtype, "out"), c.stride(0), _stream(x2))
        elif kind == "w4a8":
            sw = s_w.detach().reshape(N, -1).to(torch.float32).contiguous()
            _call("ic_gemv_w4a8", _ptr(x2), M, K, x2.stride(0), _ptr(wr), N, wr.stride(0), _ptr(sw),
                  sw.shape[1], _ptr(sa), bp, bdt, _ptr(c), _dt(c.dtype, "out"), c.stride(0), _stream(x2))
        else:
            raise ValueError(f"unknown GEMV kind {kind!r}")
    return c


# ── single-launch prep + GEMV (M <= 16) ─────────────────────────────────────
PREP_GEMV_MAX_K = 8192
PREP_GEMV_MAX_CODES = 16384


def prep_gemv_ok(x: torch.Tensor, K_w: int, w: torch.Tensor, num_groups: int = 1) -> bool:
    """Whether prep_gemv takes a call with activations x, prepared width K_w
    and weights w (otherwise rotate_quantize and the GEMM entry points do):
    f16/bf16 rows, K_in a multiple of 16, 16-byte aligned rows and weights."""
    if x.dim() < 1 or x.shape[-1] == 0:
        return False
    M, K_in = x.numel() // x.shape[-1], x.shape[-1]
    ldx = x.stride(-2) if x.dim() > 1 else K_in
    return (x.dtype in (torch.float16, torch.bfloat16) and 1 <= M <= GEMV_MAX_M and K_w % 128 == 0
            and K_w <= PREP_GEMV_MAX_K and M * K_w <= PREP_GEMV_MAX_CODES and K_in % 16 == 0
            and x.stride(-1) == 1 and x.data_ptr() % 16 == 0 and ldx % 8 == 0 and w.dim() == 2
            and w.stride(-1) == 1 and w.data_ptr() % 16 == 0 and (w.stride(0) * w.element_size()) % 16 == 0
            and num_groups in (1, K_w // 128))


def prep_gemv(x: torch.Tensor, w: torch.Tensor, s_w: torch.Tensor, *, int4: bool, rot_size: int = 0,
              w_in: int | None = None, smoothrot: PreparedFactors | None = None,
              perm: torch.Tensor | None = None, smooth: PreparedFactors | None = None,
              bias: torch.Tensor | None = None, out_dtype: torch.dtype = torch.bfloat16,
              out: torch.Tensor | None = None, activation: int = 0,
              residual: torch.Tensor | None = None) -> torch.Tensor:
    """One launch for M <= 16 tokens (ic_prep_gemv_w4a8 / ic_prep_gemv_w8a8):
    rotate_quantize(x, rot_size, w_in, smoothrot, perm, smooth) followed by
    gemm_w4a8 (int4: w packed uint8 [N, K/2], s_w [N, G] with G = 1 or K/128)
    or fused_int8_gemm_dequant (w int8 [N, K], s_w [N]) with their epilogue
    (bias, activation, residual).  Bit-identical to the two calls; the small-M
    form of fused_quant_int8_gemm_dequant (kernels/triton_int8_gemm.py:243-389).
    Calls outside prep_gemv_ok raise."""
    _need_cuda(x, w, s_w, bias, residual)
    x2 = _rows(x)
    M, K_in = x2.shape
    R, K_w, dt = _prep_shape(x2, rot_size, w_in, smoothrot, perm, smooth, "prep_gemv")
    wr = _rows(w)
    N = wr.shape[0]
    if int4:
        assert wr.dtype == torch.uint8 and wr.shape[1] * 2 >= K_w, "w must be packed uint8 [N, >= K/2]"
        sw = s_w.detach().reshape(N, -1).to(torch.float32).contiguous()
    else:
        assert wr.dtype == torch.int8 and wr.shape[1] >= K_w, "w must be int8 [N, >= K]"
        sw = s_w.detach().reshape(-1).to(torch.float32).contiguous()
        if sw.numel() != N:
            raise ValueError(f"s_w must hold one scale per output channel ({N}), got {sw.numel()}")
    G = sw.shape[1] if int4 else 1
    if not prep_gemv_ok(x2, K_w, wr, G):
        raise ValueError(f"prep_gemv: M={M}, K={K_w}, dtype {x2.dtype}, {G} groups or the weight layout is "
                         f"outside the single-launch limits (use rotate_quantize and the GEMM)")
    bp, bdt, _keep = _bias_args(bias, N)
    act, rp, rdt, ldr, _rkeep = _epilogue_args(activation, residual, M, N)
    c = _out_buffer(out, M, N, out_dtype, x2.device)
    sr = (_ptr(smoothrot.rcp), _ptr(smoothrot.fdt)) if smoothrot else (None, None)
    sm = (_ptr(smooth.rcp), _ptr(smooth.fdt)) if smooth else (None, None)
    with torch.cuda.device(x2.device):
        head = (_ptr(x2), dt, M, K_in, x2.stride(0), sr[0], sr[1], R, _ptr(perm), sm[0], sm[1], _ptr(wr), N, K_w,
                wr.stride(0), _ptr(sw))
        tail = (bp, bdt, act, rp, rdt, ldr, _ptr(c), _dt(c.dtype, "out"), c.stride(0), _stream(x2))
        if int4:
            _call("ic_prep_gemv_w4a8", *head, G, *tail)
        else:
            _call("ic_prep_gemv_w8a8", *head, *tail)
    return c


def fused_quant_int8_gemm_dequant(x: torch.Tensor, w_int8: torch.Tensor, s_w: torch.Tensor,
                                  bias: torch.Tensor | None = None,
                                  out_dtype: torch.dtype = torch.bfloat16,
                                  out: torch.Tensor | None = None) -> torch.Tensor:
    """kernels/triton_int8_gemm.py:331-389: quantize fp16/bf16 x per token, then
    the W8A8 GEMM (two launches, same numbers as the reference single kernel)."""
    assert x.dtype in (torch.float16, torch.bfloat16), f"x must be fp16/bf16, got {x.dtype}"
    assert w_int8.dtype == torch.int8, f"w_int8 must be int8, got {w_int8.dtype}"
    M, K = x.shape
    N, K_w = w_int8.shape
    assert K == K_w, f"K mismatch: {K} vs {K_w}"
    q, s = dynamic_quantize_activation(x)
    if out is not None and tuple(out.shape) != (M, N):
        out = None
    return fused_int8_gemm_dequant(q, w_int8, s_w, s, bias=bias, out_dtype=out_dtype, out=out)


# ── unpack ──────────────────────────────────────────────────────────────────
def unpack_int4_to_int8(packed: torch.Tensor, K: int) -> torch.Tensor:
    """kernels/triton_int4_to_int8_unpack.py:55-81: [N, K/2] uint8 -> [N, K] int8."""
    _need_cuda(packed)
    p = _rows(packed)
    N = p.shape[0]
    out = torch.empty(N, K, dtype=torch.int8, device=p.device)
    with torch.cuda.device(p.device):
        _call("ic_unpack_int4_to_int8", _ptr(p), N, K, p.stride(0), _ptr(out), out.stride(0), _stream(p))
    return out


def unpack_int4_to_float(packed: torch.Tensor, scale: torch.Tensor, K: int,
                         dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """INT4 -> fp16/bf16 with per-row or per-group scale, w = RN_dt(q * RN_dt(s))."""
    _need_cuda(packed, scale)
    p = _rows(packed)
    N = p.shape[0]
    sw = scale.detach().reshape(N, -1).to(torch.float32).contiguous()
    G = sw.shape[1]
    if K % G:
        raise ValueError(f"K={K} is not a multiple of the {G} scale groups")
    out = torch.empty(N, K, dtype=dtype, device=p.device)
    with torch.cuda.device(p.device):
        _call("ic_unpack_int4_to_float", _ptr(p), _ptr(sw), G, N, K, p.stride(0), _ptr(out),
              _dt(dtype, "unpack_int4_to_float"), out.stride(0), _stream(p))
    return out


def unpack_int4_to_float16(packed: torch.Tensor, scale: torch.Tensor, K: int) -> torch.Tensor:
    """kernels/triton_int4_unpack.py:62-88 (scale [N] or [N, G])."""
    return unpack_int4_to_float(packed, scale, K, torch.float16)


# ── debug: raw accumulators ─────────────────────────────────────────────────
def gemm_acc_i32(x_int8: torch.Tensor, w: torch.Tensor, *, int4: bool = False,
                 s_w: torch.Tensor | None = None, generic: bool = False) -> torch.Tensor:
    """int32 accumulators of the production GEMM: [M, N], or [G, M, N] for
    grouped INT4 weights (s_w [N, G] selects the grouping)."""
    _need_cuda(x_int8, w, s_w)
    xq = _rows(x_int8)
    M, K = xq.shape
    wr = _rows(w)
    N = wr.shape[0]
    with torch.cuda.device(xq.device):
        if int4:
            sw = (s_w if s_w is not None else torch.ones(N, 1, device=xq.device)).detach()
            sw = sw.reshape(N, -1).to(torch.float32).contiguous()
            G = sw.shape[1]
            acc = torch.empty((G, M, N) if G > 1 else (M, N), dtype=torch.int32, device=xq.device)
            _call("ic_gemm_w4a8_acc_i32", _ptr(xq), M, K, xq.stride(0), _ptr(wr), N, wr.stride(0),
                  _ptr(sw), G, _ptr(acc), 1 if generic else 0, _stream(xq))
        else:
            acc = torch.empty((M, N), dtype=torch.int32, device=xq.device)
            _call("ic_gemm_w8a8_acc_i32", _ptr(xq), M, K, xq.stride(0), _ptr(wr), N, wr.stride(0),
                  _ptr(acc), 1 if generic else 0, _stream(xq))
    return acc


__all__ = [
    "KERNELS_AVAILABLE", "TRITON_AVAILABLE", "TRITON_INT4_UNPACK", "TRITON_INT8_GEMM",
    "TRITON_INT4_INT8_UNPACK", "TRITON_DYNQUANT", "TRITON_W4A8_GEMM", "TRITON_FUSED_QGD",
    "USE_FUSED_W8A8", "USE_CUDA_GRAPHS", "dynamic_quantize_activation", "fused_int8_gemm_dequant",
    "fused_quant_int8_gemm_dequant", "fused_w4a8_gemm_dequant", "unpack_int4_to_int8",
    "unpack_int4_to_float16", "rotate_quantize", "prepare_activation", "gemm_w4a8", "int4_interleave_k",
    "gemm_w4a8_unpacked", "w4a8_unpacked_pays", "gemm_w4a16", "w4a16_staged_pays", "w4a16_stage_layout",
    "gemm_w4a16_staged", "unpack_int4_to_float", "prepare_factors", "prepare_perm", "PreparedFactors", "gemm_acc_i32",
    "gemv", "GEMV_MAX_M", "fused_layernorm_quantize", "fused_rmsnorm_quantize", "fused_softmax_quantize",
    "norm_rotate_quantize", "ACT_NONE", "ACT_SILU", "ACT_GELU", "ACT_GELU_TANH", "int8_gemm_int8out",
    "gemm_chain", "CHAIN_ROT_SIZES", "prep_gemv", "prep_gemv_ok", "PREP_GEMV_MAX_K", "PREP_GEMV_MAX_CODES",
    "load_library",
]
