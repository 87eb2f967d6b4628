"""CPU AddressSanitizer / UndefinedBehaviorSanitizer runs of the host code:

* the C oracle (oracle/intcrush_oracle.c) driven over every entry point,
  odd shapes, pads, perms and dtypes (tests/san_oracle_driver.c);
* the C ABI's argument validation and host planning (tests/san_abi_driver.cpp)
  against the library built with both sanitizers on its host code (the
  gfx950 device code is compiled as for the product; no call launches).

Both drivers exit non-zero on a failed check; a sanitizer report aborts them.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "comfyui-int-crush_amd", "csrc")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer"]


def _run(cmd, env=None, timeout=300):
    res = subprocess.run(cmd, capture_output=True, text=True, env=env, timeout=timeout)
    assert res.returncode == 0, f"{' '.join(map(str, cmd))}\n{res.stdout[-3000:]}\n{res.stderr[-3000:]}"
    return res


def _hipcc():
    for c in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if c and os.path.exists(c):
            return c
    pytest.skip("hipcc not available")


def test_oracle_under_asan_ubsan(tmp_path):
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    exe = tmp_path / "oracle_san"
    _run(["gcc", "-std=c11", "-O1", "-g", "-ffp-contract=off", *SAN, os.path.join(ROOT, "tests", "san_oracle_driver.c"),
          os.path.join(ROOT, "oracle", "intcrush_oracle.c"), "-lm", "-o", str(exe)])
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1", UBSAN_OPTIONS="print_stacktrace=1")
    res = _run([str(exe)], env=env)
    assert "clean" in res.stdout


def test_abi_validation_under_asan_ubsan(tmp_path):
    hipcc = _hipcc()
    srcs = sorted(f for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")))
    host_san = [x for f in SAN for x in ("-Xarch_host", f)]

    def compile_one(f):
        obj = tmp_path / (f + ".o")
        _run([hipcc, "--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off",
              "-fhip-fp32-correctly-rounded-divide-sqrt", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
              "-mllvm", "-amdgpu-mfma-vgpr-form=1", "-Wno-inline-asm", "-Wno-unused-command-line-argument",
              "-Xarch_host", "-g", *host_san, "-c", os.path.join(CSRC, f), "-o", str(obj)])
        return str(obj)

    with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 2)) as ex:
        objs = list(ex.map(compile_one, srcs))
    drv = tmp_path / "san_abi_driver.o"
    _run([hipcc, "-x", "c++", "-O1", "-g", "-std=c++17", *SAN, "-c", os.path.join(ROOT, "tests", "san_abi_driver.cpp"),
          "-o", str(drv)])
    exe = tmp_path / "abi_san"
    _run([hipcc, "-O1", "-g", *host_san, str(drv), *objs, "-o", str(exe)])
    # the HIP runtime keeps allocations until exit: no leak check
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1", UBSAN_OPTIONS="print_stacktrace=1")
    res = _run([str(exe)], env=env)
    assert "clean" in res.stdout
