"""The C ABI library loads and exports every entry point include/intcrush.h
declares; argument validation fails cleanly without touching a GPU."""
from __future__ import annotations

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "intcrush.h")


def declared_functions() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"\b(ic_[a-z0-9_]+)\s*\(", text)


def test_header_declares_entry_points():
    names = declared_functions()
    for must in ("ic_rotate_quantize", "ic_gemm_w8a8", "ic_gemm_w4a8", "ic_gemm_w4a16",
                 "ic_unpack_int4_to_int8", "ic_dynamic_quantize"):
        assert must in names


def test_library_exports_every_declared_symbol(rt):
    assert rt.KERNELS_AVAILABLE, rt.LOAD_ERROR
    lib = ctypes.CDLL(rt.LIB_PATH)
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} not exported"
        assert name in rt.SIGNATURES, f"{name} has no ctypes signature in _hip_runtime"
    assert set(rt.SIGNATURES) == set(declared_functions())


def test_version_and_limits(rt):
    lib = rt.lib()
    assert lib.ic_version().decode().startswith("intcrush-gfx950")
    assert lib.ic_max_fused_row() == 16384


@pytest.mark.parametrize("call", [
    # bad dtype
    lambda L: L.ic_rotate_quantize(None, 7, 1, 16, 16, None, None, 0, 16, None, None, None, None, 16, None, None),
    # rot_size not a regular Hadamard size
    lambda L: L.ic_rotate_quantize(None, 0, 1, 32, 32, None, None, 32, 32, None, None, None, None, 32, None, None),
    # K_w smaller than the rotated width
    lambda L: L.ic_rotate_quantize(None, 0, 1, 100, 100, None, None, 64, 100, None, None, None, None, 128, None, None),
    # fused row limit
    lambda L: L.ic_prepare_activation(None, 0, 1, 20000, 20000, None, None, 0, 20000, None, None, None, None, 20000, None),
    # K not divisible by groups
    lambda L: L.ic_gemm_w4a8(None, 1, 100, 100, None, 4, 50, None, 3, None, None, 0, None, 0, 4, None),
    # w4a16 with f32 activations
    lambda L: L.ic_gemm_w4a16(None, 2, 1, 64, 64, None, 4, 32, None, 1, None, 0, None, 4, None),
    # K-interleaved INT4: K not a multiple of 8
    lambda L: L.ic_int4_interleave_k(None, 4, 12, 6, None, 6, None),
    lambda L: L.ic_gemm_w4a8_kil_ex(None, 1, 100, 100, None, 4, 50, None, 1, None, None, 0, 0, None, 0, 0, None, 0,
                                    4, None, 0, None),
    # unpacked INT4: K not divisible by groups; weight rows shorter than K
    lambda L: L.ic_gemm_w4a8_unpacked_ex(None, 1, 100, 100, None, 4, 100, None, 3, None, None, 0, 0, None, 0, 0, None,
                                         0, 4, None, 0, None),
    lambda L: L.ic_gemm_w4a8_unpacked_ex(None, 1, 100, 100, None, 4, 50, None, 1, None, None, 0, 0, None, 0, 0, None,
                                         0, 4, None, 0, None),
    # staged W4A16: K not a multiple of 64; f32 activations; M in the GEMV /
    # small-tile range (addresses that are never dereferenced: the checks
    # run before any launch)
    lambda L: L.ic_w4a16_stage_layout(None, 4, 96, 48, None, 1, None, None, None),
    lambda L: L.ic_gemm_w4a16_staged(None, 2, 256, 128, 128, None, 64, None, 1, None, 0, None, 64, None),
    lambda L: L.ic_gemm_w4a16_staged(4096, 0, 64, 128, 128, 4096, 64, 4096, 1, None, 0, 4096, 64, None),
])
def test_argument_validation(rt, call):
    lib = rt.lib()
    rc = call(lib)
    assert rc in (1, 2)
    assert lib.ic_last_error().decode()


def test_empty_batch_is_a_no_op(rt):
    lib = rt.lib()
    assert lib.ic_dynamic_quantize(None, 0, 0, 64, 64, None, 64, None, None) == 0
    assert lib.ic_gemm_w8a8(None, 0, 64, 64, None, 8, 64, None, None, None, 0, None, 0, 8, None) == 0


def test_cpu_tensors_are_rejected(rt):
    import torch

    with pytest.raises(ValueError):
        rt.rotate_quantize(torch.zeros(2, 64, dtype=torch.float16))
    with pytest.raises(ValueError):
        rt.unpack_int4_to_int8(torch.zeros(2, 8, dtype=torch.uint8), 16)


def test_dynamic_quantize_cpu_branch_is_reference_semantics(rt):
    import torch

    torch.manual_seed(0)
    x = torch.randn(4, 256)
    q, s = rt.dynamic_quantize_activation(x)
    ref_s = x.abs().amax(dim=1).clamp(min=1e-8) / 127.0
    assert torch.equal(s, ref_s)
    assert torch.equal(q, (x / ref_s[:, None]).round().clamp(-128, 127).to(torch.int8))
