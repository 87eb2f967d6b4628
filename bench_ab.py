"""Side-by-side timing of the fused prep in two builds of the library.

Loads two copies of libintcrush_gfx950.so into one process (`--base`, e.g.
one built from an earlier commit in a `git worktree` with that tree's
`__graft_entry__.build()`, and `--new`, by default the in-tree build), runs
`ic_rotate_quantize` / `ic_norm_rotate_quantize` of both on the same inputs,
checks that their codes and scales are identical, and then times each build
with alternating hipGraph replays (20 launches per replay, over three input
copies so that every launch reads its row block from HBM).  One line per
case: the sorted per-launch times of each build, in microseconds.

The cases are the prep shapes of the Flux and Wan configs (the prep in
front of the reference's quantized linear, _ops.py:337-365, and
kernels/triton_quantize.py:109-146); `--case` selects some of them.

    python bench_ab.py --base /path/to/old/libintcrush_gfx950.so [--case flux3072_f16 ...]
"""
from __future__ import annotations

import argparse
import ctypes
import os
import sys

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

# name: (M, K_in, K_w, R, smoothrot, perm, dtype, norm)
CASES = {
    "c3_f16": (4608, 12288, 12288, 256, True, True, torch.float16, None),
    "c3_bf16": (4608, 12288, 12288, 256, True, True, torch.bfloat16, None),
    "flux3072_f16": (4608, 3072, 3072, 256, True, True, torch.float16, None),
    "flux3072_bf16": (4096, 3072, 3072, 256, True, True, torch.bfloat16, None),
    "flux3072_m512": (512, 3072, 3072, 256, True, True, torch.bfloat16, None),
    "flux3072_r64": (4608, 3072, 3072, 64, True, True, torch.float16, None),
    "w4096": (4096, 4096, 4096, 256, True, True, torch.float16, None),
    "c3_noperm_r64": (4608, 12288, 12288, 64, False, True, torch.float16, None),
    "c3_plain_bf16": (4608, 12288, 12288, 256, False, False, torch.bfloat16, None),
    "flux15360_f16": (4608, 15360, 15360, 256, True, True, torch.float16, None),
    "flux15360_bf16": (4608, 15360, 15360, 256, True, True, torch.bfloat16, None),
    "wan_down": (32760, 13824, 14336, 1024, False, False, torch.float16, None),
    "wan5120": (32760, 5120, 5120, 1024, False, False, torch.float16, None),
    "norm3072_bf16": (4608, 3072, 3072, 256, True, True, torch.bfloat16, "layer"),
    "norm3072_r64": (4096, 3072, 3072, 64, True, True, torch.float16, "layer"),
}


def _graph_us(fn, launches=20):
    g = torch.cuda.CUDAGraph()
    fn(0)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        for i in range(launches):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    g.replay()
    b.record()
    b.synchronize()
    return a.elapsed_time(b) / launches * 1000.0


def run_case(name, libs, rt, rounds):
    M, K_in, K_w, R, smr, pm, dt, norm = CASES[name]
    dev = torch.device("cuda:0")
    P = ctypes.c_void_p
    copies = 3
    xs = [torch.randn(M, K_in, device=dev).to(dt) for _ in range(copies)]
    sr = rt.prepare_factors(torch.exp(torch.randn(K_in, device=dev) * 0.5), dt) if smr else None
    perm = rt.prepare_perm(torch.randperm(K_w, device=dev), K_w) if pm else None
    nw = (1 + 0.1 * torch.randn(K_in, device=dev)).float()
    nb = (0.1 * torch.randn(K_in, device=dev)).float()
    outs = {k: (torch.empty(M, K_w, dtype=torch.int8, device=dev), torch.empty(M, dtype=torch.float32, device=dev))
            for k in libs}
    dtc = 0 if dt == torch.float16 else 1

    def call(lib, x, q, s):
        stream = P(torch.cuda.current_stream().cuda_stream)  # the capture stream while a graph records
        if norm is None:
            rc = lib.ic_rotate_quantize(P(x.data_ptr()), dtc, M, K_in, K_in,
                                        P(sr.rcp.data_ptr()) if sr is not None else None,
                                        P(sr.fdt.data_ptr()) if sr is not None else None, R, K_w,
                                        P(perm.data_ptr()) if perm is not None else None, None, None,
                                        P(q.data_ptr()), K_w, P(s.data_ptr()), stream)
        else:
            rc = lib.ic_norm_rotate_quantize(P(x.data_ptr()), dtc, M, K_in, K_in, rt.IC_NORM_LAYER,
                                             P(nw.data_ptr()), P(nb.data_ptr()), ctypes.c_float(1e-6),
                                             P(sr.rcp.data_ptr()) if sr is not None else None,
                                             P(sr.fdt.data_ptr()) if sr is not None else None, R, K_w,
                                             P(perm.data_ptr()) if perm is not None else None,
                                             P(q.data_ptr()), K_w, P(s.data_ptr()), stream)
        if rc != 0:
            raise RuntimeError(f"{name}: entry point returned {rc}")

    for k, lib in libs.items():
        call(lib, xs[0], *outs[k])
    torch.cuda.synchronize()
    (qa, sa), (qb, sb) = outs["base"], outs["new"]
    same = torch.equal(qa, qb) and torch.equal(sa, sb)
    times = {k: [] for k in libs}
    for _ in range(rounds):
        for k, lib in libs.items():
            q, s = outs[k]
            times[k].append(_graph_us(lambda i, lib=lib, q=q, s=s: call(lib, xs[i % copies], q, s)))
    del xs
    fmt = lambda v: "[" + ", ".join(f"{t:.1f}" for t in sorted(v)) + "]"
    print(f"{name}: M={M} K_in={K_in} K_w={K_w} R={R} smoothrot={smr} perm={pm} {str(dt)[6:]} norm={norm}: "
          f"base {fmt(times['base'])} new {fmt(times['new'])} us; outputs {'identical' if same else 'DIFFER'}",
          flush=True)
    return same


def main():
    import __graft_entry__

    rt = __graft_entry__._submodule("_hip_runtime")
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--base", required=True, help="path of the library build to compare against")
    ap.add_argument("--new", default=rt.LIB_PATH, help="path of the library build under test (default: in-tree)")
    ap.add_argument("--case", action="append", choices=sorted(CASES), help="cases to run (default: all)")
    ap.add_argument("--rounds", type=int, default=4, help="alternating timed replays per build")
    args = ap.parse_args()
    if not torch.cuda.is_available():
        sys.exit("bench_ab.py needs a GPU")
    libs = {}
    for key, path in (("base", args.base), ("new", args.new)):
        lib = ctypes.CDLL(os.path.abspath(path))
        for fn in ("ic_rotate_quantize", "ic_norm_rotate_quantize"):
            getattr(lib, fn).argtypes, getattr(lib, fn).restype = rt.SIGNATURES[fn]
        libs[key] = lib
    ok = True
    for name in args.case or list(CASES):
        ok = run_case(name, libs, rt, args.rounds) and ok
        torch.cuda.empty_cache()
    sys.exit(0 if ok else 1)


if __name__ == "__main__":
    main()
