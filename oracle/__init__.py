"""CPU oracle for the INT-Crush quantized-linear forward.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py as the checker.  The product package never
imports anything from here.

The heavy lifting is the C restatement in intcrush_oracle.c (built by
oracle/Makefile into liboracle_intcrush.so); this module wraps it with numpy,
adds an exact big-integer fallback for Hadamard blocks whose double sum is not
provably exact (wide-range bf16/f32 rows), and provides the reference PyTorch
fallback (fp32 dequant -> F.linear) that the fp16/bf16 outputs are judged
against.

Reference citations are file:line in ThunderFun/ComfyUI-INT-Crush.

How each function is pinned (tests/test_oracle.py, tests/test_numerics_proofs.py,
tests/test_norm_quant.py, tests/test_gemm_epilogue.py); none is left unpinned:
  unpack_int4 / pack_int4   the reference's known answers (tests/test_quant_utils.py:65-99
                            of the reference), all 256 byte values, round trips
  prepare (Hadamard)        orthogonality and involution of H, closed-form entries
                            against a Kronecker-product matmul, exact rational
                            recomputation for wide-range blocks
  prepare (divide/pad/perm) torch fp16/bf16 division, perm followed by its inverse,
                            zero pads
  quantize                  the reference CPU quantizer's vectors at its test shapes,
                            hand-built ties and the 0.49999997 quirk, zero rows
  gemm_acc                  int64 matmul; group sums add to the ungrouped sum
  epilogue                  against linear_fallback_fp32 on the same integers
  activate / epilogue_ex    torch's F.silu / F.gelu (erf and tanh forms) in float64 over a dense
                            grid and saturation values; reduces to epilogue without options
  dequant_w4a16             single correctly rounded fp16 product (numpy fp16)
  reference_fallback_forward against the integer chain (prepare -> quantize ->
                            gemm_acc -> epilogue) within quantization error; a
                            reversed perm or transposed group scales fail it
  normalize_rows /          the reference tests' PyTorch formulas (codes within +-1,
  norm_quantize             their own bar); closed forms (constant rows, uniform
                            softmax, unit-variance LayerNorm); a LayerNorm without
                            its mean subtraction fails them
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from fractions import Fraction

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_intcrush.so")
_lib = None

DT_F16, DT_BF16, DT_F32 = 0, 1, 2


def build(force: bool = False) -> str:
    """Compile the C oracle with gcc (oracle/Makefile)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.check_call(["make", "-s", "-B" if force else "all"], cwd=_HERE)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        i64 = ctypes.c_int64
        L.oc_round.argtypes = [ctypes.c_double, ctypes.c_int]
        L.oc_round.restype = ctypes.c_double
        L.oc_prepare.argtypes = [P, ctypes.c_int, i64, i64, P, ctypes.c_int, i64, P, P, P,
                                 ctypes.POINTER(i64), ctypes.c_int]
        L.oc_prepare.restype = ctypes.c_int
        L.oc_quantize.argtypes = [P, i64, i64, P, P]
        L.oc_quantize.restype = None
        L.oc_quantize_rne.argtypes = [P, i64, i64, P, P]
        L.oc_quantize_rne.restype = None
        L.oc_unpack_int4.argtypes = [P, i64, i64, i64, P]
        L.oc_pack_int4.argtypes = [P, i64, i64, P]
        L.oc_dequant_w4a16.argtypes = [P, P, i64, i64, i64, i64, ctypes.c_int, P]
        L.oc_gemm_acc.argtypes = [P, i64, i64, P, i64, i64, P]
        L.oc_gemm_acc.restype = i64
        L.oc_epilogue.argtypes = [P, i64, i64, i64, P, P, P, ctypes.c_int, P]
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return None if a is None else np.ascontiguousarray(a, dtype=dtype)


# ---------------------------------------------------------------- rounding
def round_dtype(values, dtype: int) -> np.ndarray:
    """RN-even of float64 values to fp16/bf16/f32, returned as float32 values."""
    v = np.asarray(values, dtype=np.float64)
    if dtype == DT_F16:
        return v.astype(np.float16).astype(np.float32)  # numpy's cast is RN-even
    if dtype == DT_F32:
        return v.astype(np.float32)
    L = lib()
    flat = v.reshape(-1)
    out = np.array([L.oc_round(float(d), DT_BF16) for d in flat], dtype=np.float32)
    return out.reshape(v.shape)


def to_dtype_values(x, dtype: int) -> np.ndarray:
    """Exact values of a torch/numpy array of the given dtype as float32."""
    try:
        import torch

        if isinstance(x, torch.Tensor):
            return x.detach().to("cpu", torch.float32).numpy()
    except ImportError:  # pragma: no cover
        pass
    return np.asarray(x, dtype=np.float32)


# ---------------------------------------------------------------- prep
def _exact_hadamard_block(vals: np.ndarray, k: int) -> list[Fraction]:
    """y = H x with Python rationals (no rounding at all)."""
    R = len(vals)
    ys: list[Fraction] = [Fraction(float(v)) for v in vals]
    for d in range(k):
        st = 1 << (2 * d)
        for base in range(R):
            if (base >> (2 * d)) & 3:
                continue
            a, b, c, e = (ys[base + i * st] for i in range(4))
            s = (a + b + c + e) / 2
            ys[base], ys[base + st], ys[base + 2 * st], ys[base + 3 * st] = s - e, s - c, s - b, s - a
    return ys


def _round_fraction(q: Fraction, dtype: int) -> float:
    """Exact RN-even of a rational to fp16/bf16/f32."""
    if q == 0:
        return 0.0
    p, emin, maxv = {DT_F16: (11, -14, 65504.0), DT_BF16: (8, -126, 3.3895313892515355e38),
                     DT_F32: (24, -126, 3.4028234663852886e38)}[dtype]
    sign = -1 if q < 0 else 1
    a = abs(q)
    E = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** E > a:
        E -= 1
    E = max(E, emin)
    quantum = Fraction(2) ** (E - (p - 1))
    n = a / quantum
    fl = n.numerator // n.denominator
    rem = n - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    r = float(fl * quantum)
    if r > maxv:
        r = float("inf")
    return sign * r


def prepare(x, dtype: int, *, smoothrot=None, rot_size: int = 0, w_in: int | None = None,
            perm=None, smooth=None, fast: bool = True) -> np.ndarray:
    """Reference _prep_activation (+ old SmoothQuant divide) of a 2-D row block.

    x: [M, K_in] values of `dtype` (float32 array or tensor).  smoothrot /
    smooth: raw fp32 factors (rounded to dtype here, as `.to(x.dtype)` does,
    _ops.py:350, :533).  Returns float32 [M, K_w] holding exact dtype values.
    """
    L = lib()
    xv = np.ascontiguousarray(to_dtype_values(x, dtype), dtype=np.float32)
    M, K_in = xv.shape
    R = int(rot_size)
    K_r = ((K_in + R - 1) // R) * R if R else K_in
    K_w = int(w_in) if w_in is not None else K_r
    K_w = max(K_w, K_r)
    srf = None if smoothrot is None else round_dtype(np.asarray(to_dtype_values(smoothrot, DT_F32), np.float64), dtype)
    smf = None if smooth is None else round_dtype(np.asarray(to_dtype_values(smooth, DT_F32), np.float64), dtype)
    pm = None if perm is None else np.ascontiguousarray(np.asarray(perm).astype(np.int32))
    out = np.zeros((M, K_w), np.float32)
    n_inexact = ctypes.c_int64(0)
    rc = L.oc_prepare(_p(xv), dtype, M, K_in, _p(srf), R, K_w, _p(pm), _p(smf), _p(out),
                      ctypes.byref(n_inexact), 1 if fast else 0)
    if rc != 0:
        raise ValueError(f"oc_prepare rejected arguments (rot_size={R}, K_in={K_in}, w_in={K_w})")
    if n_inexact.value:
        out = _prepare_exact_rows(xv, dtype, srf, R, K_w, pm, smf, out)
    return out


def flush_small_bf16(blk: np.ndarray, k: int) -> np.ndarray:
    """bf16 rows only: inputs more than 43 - 2k binades below the largest
    finite magnitude of their Hadamard block (R = 4^k) become zero before the
    rotation (the rule intcrush_oracle.c's flush_small_bf16 applies)."""
    blk = np.array(blk, dtype=np.float64)
    fin = np.abs(blk[np.isfinite(blk)])
    mx = fin.max() if fin.size else 0.0
    if mx == 0.0:
        return blk
    thr = 2.0 ** (int(np.frexp(mx)[1]) - 1 - (43 - 2 * k))
    blk[np.abs(blk) < thr] = 0.0
    return blk


def inexact_block_rows(x, dtype: int, *, smoothrot=None, rot_size: int = 0) -> np.ndarray:
    """Rows of `prepare`'s input whose Hadamard blocks include one whose double
    sum is not provably exact (after the SmoothRot divide and, for bf16, the
    flush rule): the rows _prepare_exact_rows recomputes.  Boolean [M]; all
    False for fp16 inputs and without rotation."""
    L = lib()
    R = int(rot_size)
    xv = np.ascontiguousarray(to_dtype_values(x, dtype), dtype=np.float32)
    M, K_in = xv.shape
    flags = np.zeros(M, bool)
    if R <= 1:
        return flags
    k = (R.bit_length() - 1) // 2
    K_r = ((K_in + R - 1) // R) * R
    p = {DT_F16: 11, DT_BF16: 8, DT_F32: 24}[dtype]
    srf = None if smoothrot is None else round_dtype(np.asarray(to_dtype_values(smoothrot, DT_F32), np.float64), dtype)
    for m in range(M):
        a = np.zeros(K_r, np.float64)
        a[:K_in] = xv[m]
        if srf is not None:
            a[:K_in] = [L.oc_round(float(v) / float(f), dtype) for v, f in zip(xv[m], srf)]
        for b0 in range(0, K_r, R):
            blk = a[b0:b0 + R]
            if dtype == DT_BF16:
                blk = flush_small_bf16(blk, k)
            nz = blk[blk != 0]
            if nz.size:
                emax = int(np.max(np.frexp(np.abs(nz))[1])) - 1
                qmin = int(np.min(np.frexp(np.abs(nz))[1])) - p
                if (emax + 1 + 2 * k) - qmin > 53:
                    flags[m] = True
                    break
    return flags


def _prepare_exact_rows(xv, dtype, srf, R, K_w, pm, smf, out):
    """Recompute rows containing a block whose double sum is not provably exact."""
    L = lib()
    k = (R.bit_length() - 1) // 2
    M, K_in = xv.shape
    K_r = ((K_in + R - 1) // R) * R
    p = {DT_F16: 11, DT_BF16: 8, DT_F32: 24}[dtype]
    for m in range(M):
        a = np.zeros(K_r, np.float64)
        a[:K_in] = xv[m]
        if srf is not None:
            a[:K_in] = [L.oc_round(float(v) / float(f), dtype) for v, f in zip(xv[m], srf)]
        y = np.zeros(K_w, np.float64)
        redo = False
        for b0 in range(0, K_r, R):
            blk = a[b0:b0 + R]
            if dtype == DT_BF16:
                blk = flush_small_bf16(blk, k)
            nz = blk[blk != 0]
            if nz.size:
                emax = int(np.max(np.frexp(np.abs(nz))[1])) - 1
                qmin = int(np.min(np.frexp(np.abs(nz))[1])) - p
                if (emax + 1 + 2 * k) - qmin > 53:
                    redo = True
            ys = _exact_hadamard_block(blk, k)
            y[b0:b0 + R] = [_round_fraction(v, dtype) for v in ys]
        if not redo:
            continue
        row = y[pm] if pm is not None else y
        if smf is not None:
            row = np.array([L.oc_round(float(v) / float(f), dtype) for v, f in zip(row, smf)])
        out[m] = row.astype(np.float32)
    return out


def quantize(v, *, rule: str = "gpu"):
    """Per-token dynamic INT8 quantization (kernels/triton_quantize.py:109-146).

    rule="gpu": q = trunc(f32(v/s) +- 0.5) (the Triton kernel rule, the canonical one);
    rule="rne": torch.round half-to-even (the reference CPU fallback, :43-54).
    Returns (int8 [M, K], float32 [M]).
    """
    L = lib()
    xv = np.ascontiguousarray(v, dtype=np.float32)
    M, K = xv.shape
    q = np.zeros((M, K), np.int8)
    s = np.zeros(M, np.float32)
    (L.oc_quantize if rule == "gpu" else L.oc_quantize_rne)(_p(xv), M, K, _p(q), _p(s))
    return q, s


def rotate_quantize(x, dtype: int, **kw):
    """prepare() followed by quantize(): the fused kernel's full contract."""
    return quantize(prepare(x, dtype, **kw))


# ---------------------------------------------------------------- norm + quantize
def normalize_rows(x, kind: str, gamma=None, beta=None, eps: float = 1e-5) -> np.ndarray:
    """Row normalisation of the fused norm / softmax quantizers
    (kernels/triton_quantize.py:209-274 LayerNorm, :348-394 RMSNorm, :462-515
    softmax), as the canonical arithmetic of this build: row statistics in
    fp64, eps taken as an f32 value, y formed in f32 with one rounding per
    operation:
      layer    mean = f32(S1/K), rstd = f32(1/sqrt(max(S2/K - (S1/K)^2, 0) + eps)),
               S1 = sum x, S2 = sum x^2 (one pass; exact in fp64 for realistic rows),
               y = f32(f32(x - mean) * rstd) * gamma (+ beta)
      rms      rstd = f32(1/sqrt(sum x^2 / K + eps)), y = f32(x * rstd) * gamma
      softmax  m = max x, e = f32(exp(f32(x - m))), inv = f32(1 / sum e), y = e * inv
    The reference sums in f32 in Triton's order; its own tests bound the codes
    to +-1 of an f32 PyTorch computation, which pins this restatement."""
    xv = np.ascontiguousarray(x, dtype=np.float32)
    M, K = xv.shape
    e = float(np.float32(eps))
    x64 = xv.astype(np.float64)
    if kind == "layer":
        mean64 = x64.sum(axis=1) / K
        var = np.maximum((x64 * x64).sum(axis=1) / K - mean64 * mean64, 0.0)
        mean = mean64.astype(np.float32)
        rstd = (1.0 / np.sqrt(var + e)).astype(np.float32)
        y = (xv - mean[:, None]) * rstd[:, None]
    elif kind == "rms":
        rstd = (1.0 / np.sqrt((x64 * x64).sum(axis=1) / K + e)).astype(np.float32)
        y = xv * rstd[:, None]
    if kind in ("layer", "rms"):
        if gamma is not None:
            y = y * np.asarray(gamma, np.float32)[None, :]
        if beta is not None:
            y = y + np.asarray(beta, np.float32)[None, :]
        return y.astype(np.float32)
    if kind == "softmax":
        m = xv.max(axis=1)
        ex = np.exp((xv - m[:, None]).astype(np.float64)).astype(np.float32)
        inv = (1.0 / ex.astype(np.float64).sum(axis=1)).astype(np.float32)
        return (ex * inv[:, None]).astype(np.float32)
    raise ValueError(f"unknown normalisation {kind!r}")


def norm_quantize(x, kind: str, gamma=None, beta=None, eps: float = 1e-5):
    """normalize_rows() then the GPU quantization rule: the full contract of
    ic_norm_quantize.  Returns (int8 [M, K], float32 [M])."""
    return quantize(normalize_rows(x, kind, gamma, beta, eps))


def norm_rotate_quantize(x, dtype: int, kind: str, weight=None, bias=None, eps: float = 1e-6, **prep_kw):
    """The contract of ic_norm_rotate_quantize: normalize_rows() (optional
    affine), rounded once to the activation dtype, then rotate_quantize()."""
    y = normalize_rows(to_dtype_values(x, dtype), kind, weight, bias, eps)
    return rotate_quantize(round_dtype(y, dtype), dtype, **prep_kw)


# ---------------------------------------------------------------- weights
def unpack_int4(packed, K: int) -> np.ndarray:
    """_quant_utils.py:185-197."""
    L = lib()
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    N, Kp = p.shape
    out = np.zeros((N, K), np.int8)
    L.oc_unpack_int4(_p(p), N, K, Kp, _p(out))
    return out


def pack_int4(vals) -> np.ndarray:
    """_quant_utils.py:170-182."""
    L = lib()
    v = np.ascontiguousarray(vals, dtype=np.int8)
    if v.ndim == 1:
        return pack_int4(v[None])[0]
    if v.size and (v.min() < -8 or v.max() > 7):
        raise ValueError("Values must be in [-8, 7]")
    N, K = v.shape
    out = np.zeros((N, (K + 1) // 2), np.uint8)
    L.oc_pack_int4(_p(v), N, K, _p(out))
    return out


def dequant_w4a16(packed, s_w, K: int, dtype: int) -> np.ndarray:
    """W4A16 weight RN_dt(q * RN_dt(s)) (triton_int4_unpack.py:49-56, group scales)."""
    L = lib()
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    s = np.ascontiguousarray(np.asarray(s_w, np.float32).reshape(p.shape[0], -1))
    N, G = s.shape
    out = np.zeros((N, K), np.float32)
    L.oc_dequant_w4a16(_p(p), _p(s), G, N, K, p.shape[1], dtype, _p(out))
    return out


# ---------------------------------------------------------------- GEMM
def gemm_acc(a_q, w_q, num_groups: int = 1) -> np.ndarray:
    """Exact int32 accumulators [G, M, N] (G=1 -> [M, N])."""
    L = lib()
    A = np.ascontiguousarray(a_q, dtype=np.int8)
    W = np.ascontiguousarray(w_q, dtype=np.int8)
    M, K = A.shape
    N = W.shape[0]
    acc = np.zeros((num_groups, M, N), np.int32)
    ovf = L.oc_gemm_acc(_p(A), M, K, _p(W), N, num_groups, _p(acc))
    if ovf:
        raise OverflowError(f"{ovf} accumulators exceed int32")
    return acc[0] if num_groups == 1 else acc


def epilogue(acc, s_a, s_w, bias=None, out_dtype: int = DT_F16) -> np.ndarray:
    """Dequant epilogue (triton_int8_gemm.py:105-117 and the group layout)."""
    L = lib()
    acc = np.ascontiguousarray(acc, dtype=np.int32)
    G = 1 if acc.ndim == 2 else acc.shape[0]
    M, N = acc.shape[-2:]
    sa = np.ascontiguousarray(s_a, dtype=np.float32)
    sw = np.ascontiguousarray(np.asarray(s_w, np.float32).reshape(N, -1))
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    out = np.zeros((M, N), np.float32)
    L.oc_epilogue(_p(acc), M, N, G, _p(sa), _p(sw), _p(b), out_dtype, _p(out))
    return out


def activate(v, act: int) -> np.ndarray:
    """Epilogue activations of triton_int8_gemm.py:119-124 in float64:
    1 SiLU v * sigmoid(v), 2 GELU 0.5 v (1 + erf(v / sqrt 2)); 3 is GELU with
    the tanh approximation 0.5 v (1 + tanh(sqrt(2/pi) (v + 0.044715 v^3))),
    which the reference kernel does not have (its Flux-style MLPs use it)."""
    from scipy.special import erf

    v = np.asarray(v, np.float64)
    if act == 0:
        return v.copy()
    if act == 1:
        with np.errstate(over="ignore"):
            return v / (1.0 + np.exp(-v))
    if act == 2:
        return 0.5 * v * (1.0 + erf(v / np.sqrt(2.0)))
    if act == 3:
        return 0.5 * v * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (v + 0.044715 * v ** 3)))
    raise ValueError(f"unknown activation {act}")


def epilogue_ex(acc, s_a, s_w, bias=None, out_dtype: int = DT_F16, activation: int = 0, residual=None):
    """The GEMM epilogue with the options of triton_int8_gemm.py:119-130: the
    f32 dequant (+ bias) value of epilogue(), the activation in float64, plus
    the residual, then one rounding to out_dtype.  The GPU evaluates the
    activation and the add in f32, so it matches to a few f32 ulp before the
    final rounding (within one ulp of out_dtype after it)."""
    v = epilogue(acc, s_a, s_w, bias, DT_F32).astype(np.float64)
    v = activate(v, activation)
    if residual is not None:
        v = v + np.asarray(residual, np.float64)
    return round_dtype(v, out_dtype)


# ---------------------------------------------------------------- fp32 fallback
def dequant_weight_fp32(w, s_w, K: int, int4: bool):
    """IntCrushInt{4,8}Layout.dequantize (quant_layout.py:80-87, :163-168) with
    the [N, G] group layout of _quant_utils.py:237-270: W = q * s[n, k // gs]."""
    import torch

    q = torch.as_tensor(unpack_int4(w, K) if int4 else np.asarray(w), dtype=torch.float32)
    s = torch.as_tensor(np.asarray(s_w, np.float32)).reshape(q.shape[0], -1)
    G = s.shape[1]
    return q * s.repeat_interleave(K // G, dim=1)


def linear_fallback_fp32(x_prep, w, s_w, K: int, int4: bool, bias=None):
    """Reference PyTorch fallback (_ops.py:483-491, :538-545) in fp32:
    F.linear(x_prep, dequant(W), bias)."""
    import torch
    import torch.nn.functional as F

    W = dequant_weight_fp32(w, s_w, K, int4)
    xp = torch.as_tensor(np.asarray(x_prep, np.float32))
    b = None if bias is None else torch.as_tensor(np.asarray(bias, np.float32))
    return F.linear(xp, W, b).numpy()


def reference_fallback_forward(x, w, s_w, K: int, *, int4: bool, smoothrot=None, rot_size: int = 0,
                               perm=None, bias=None):
    """CPU restatement of the reference PyTorch fallback forward in fp32
    (_forward_int4_pytorch _ops.py:483-491 / no-kernel INT8 path :538-545):
    dequantize W = q * s (group layout), prep the activation (SmoothRot divide,
    block Hadamard via matmul, pad, perm; _ops.py:337-365) and F.linear.
    Used as the timed CPU baseline; runs on whatever torch threads are set."""
    import torch
    import torch.nn.functional as F

    W = dequant_weight_fp32(w, s_w, K, int4)
    x2 = x.reshape(-1, x.shape[-1]).to(torch.float32)
    if smoothrot is not None:
        x2 = x2 / smoothrot.to(torch.float32)
    if rot_size:
        R = int(rot_size)
        pad = (-x2.shape[-1]) % R
        if pad:
            x2 = F.pad(x2, (0, pad))
        h4 = torch.tensor([[1., 1., 1., -1.], [1., 1., -1., 1.], [1., -1., 1., 1.], [-1., 1., 1., 1.]]) / 2
        H = h4
        while H.shape[0] < R:
            H = torch.kron(H, h4)
        x2 = torch.matmul(x2.reshape(x2.shape[0], -1, R), H.T).reshape(x2.shape[0], -1)
    if x2.shape[-1] < K:
        x2 = F.pad(x2, (0, K - x2.shape[-1]))
    if perm is not None:
        x2 = x2[..., perm]
    b = None if bias is None else bias.to(torch.float32)
    return F.linear(x2, W, b)
