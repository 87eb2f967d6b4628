#!/usr/bin/env python3
"""Benchmark of the INT-Crush quantized-linear forward on one MI355X.

Default workload (the headline metric, "W4A8 linear TOPS ... at Flux shapes"):
BASELINE config 3, the Flux MLP down-projection as an INT4 W4A8 linear:
  x [4608, 12288] fp16 (N(0,1), 1% of channels x20), SmoothRot factors
  lognormal(0, 0.5), PermuQuant perm, rot_size 256, INT4 weights [3072, 12288]
  packed with fp16 group-128 scales.
One step = fused prep+quantize kernel + W4A8 GEMM (one linear forward).
Other --config values are the remaining BASELINE shapes (C1 W8A8, C2 W4A16)
and the M = 1 modulation linears of the Flux step (C4), which run the
bandwidth-bound GEMV kernels.

Timing: inputs are resident in HBM before the timed region; weights and
activations rotate over enough copies that the 256 MB Infinity Cache cannot
serve repeats.  `value` is whole-step throughput from HIP events around K
steps; the dominant kernel is also timed alone (back-to-back launches between
two events on the launch stream) for the roofline entry.

Prints ONE JSON line with the driver's contract fields plus "roofline" and
"cpu_baseline" (the reference fp32 PyTorch fallback, restated under oracle/,
timed on this host's cores).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "W4A8 linear TOPS & % INT8-MFMA peak at Flux shapes; denoise step ms"
PEAK_INT8_TOPS = 5000.0       # MI355X dense INT8 MFMA, published
PEAK_FP16_TFLOPS = 2500.0     # MI355X dense FP16/BF16 MFMA, published
PEAK_HBM_GBPS = 8000.0        # MI355X HBM3E, published
PEAK_SCLK_MHZ = 2400.0        # MI355X peak engine clock the published MFMA peaks assume


def cpu_model():
    """The host CPU's model name from /proc/cpuinfo (what `lscpu` prints as
    "Model name"), followed by its CPUID family / model / stepping, which name
    the part where a virtualised host reports only a generic brand string
    ("AMD EPYC").  None where /proc/cpuinfo is absent."""
    fields = {}
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if not ln.strip():
                    break  # first processor's block only
                k, _, v = ln.partition(":")
                fields.setdefault(k.strip(), v.strip())
    except OSError:
        return None
    name = fields.get("model name")
    if name is None:
        return None
    ids = [f"{k.split()[-1]} {fields[k]}" for k in ("cpu family", "model", "stepping") if k in fields]
    return f"{name} ({', '.join(ids)})" if ids else name

CONFIGS = {
    "c1": dict(name="C1 W8A8 linear 3072->3072, M=4096, rot 0", fmt="int8", M=4096, K=3072, N=3072,
               rot=0, smoothrot=False, perm=False, G=1, act="fp16"),
    "c2": dict(name="C2 W4A16 linear 3072->12288, M=4608, g128", fmt="w4a16", M=4608, K=3072, N=12288,
               rot=0, smoothrot=False, perm=False, G=24, act="fp16"),
    "c3": dict(name="C3 W4A8 linear 12288->3072 (Flux MLP down-proj), M=4608, g128, R=256",
               fmt="int4", M=4608, K=12288, N=3072, rot=256, smoothrot=True, perm=True, G=96, act="fp16"),
    "c4mod_w4a8": dict(name="C4 modulation GEMV W4A8 3072->18432, M=1, g128, R=256 (double-block img_mod/txt_mod)",
                       fmt="int4", M=1, K=3072, N=18432, rot=256, smoothrot=True, perm=True, G=24, act="bf16"),
    "c4mod_w4a16": dict(name="C4 modulation GEMV W4A16 3072->18432, M=1, g128 (single-block modulation)",
                        fmt="w4a16", M=1, K=3072, N=18432, rot=0, smoothrot=False, perm=False, G=24, act="bf16"),
    "c4mod_w8a8": dict(name="C4 modulation GEMV W8A8 3072->18432, M=1 (INT8 checkpoint)",
                       fmt="int8", M=1, K=3072, N=18432, rot=0, smoothrot=False, perm=False, G=1, act="bf16"),
    # C5, Wan2.1-14B FFN down-projection: K 13824 rotated in 1024-blocks and
    # padded to 14336 (the weights were quantized in the padded space)
    "c5down_w4a8": dict(name="C5 Wan FFN-down W4A8 13824(->14336)->5120, M=32760, g128, R=1024",
                        fmt="int4", M=32760, K_in=13824, K=14336, N=5120, rot=1024, smoothrot=False,
                        perm=False, G=112, act="fp16", dist="student_t", cpu_rows=2048),
    "c5down_w8a8": dict(name="C5 Wan FFN-down W8A8 13824(->14336)->5120, M=32760, R=1024",
                        fmt="int8", M=32760, K_in=13824, K=14336, N=5120, rot=1024, smoothrot=False,
                        perm=False, G=1, act="fp16", dist="student_t", cpu_rows=2048),
}
# The rest of the Wan2.1-14B block's linears, for the C5 set
for _fmt, _tag in (("int4", "w4a8"), ("int8", "w8a8")):
    for _lin, _K, _N in (("qkv", 5120, 15360), ("proj", 5120, 5120), ("up", 5120, 13824)):
        CONFIGS[f"c5{_lin}_{_tag}"] = dict(
            name=f"C5 Wan {_lin} {_tag.upper()} {_K}->{_N}, M=32760, R=1024", fmt=_fmt, M=32760, K=_K, N=_N,
            rot=1024, smoothrot=False, perm=False, G=_K // 128 if _fmt == "int4" else 1, act="fp16",
            dist="student_t", cpu_rows=2048)
# C5 set: the four linears of one Wan2.1-14B block, timed one after another
SETS = {f"c5set_{t}": dict(name=f"C5 Wan2.1-14B block linear set {t.upper()} (qkv, proj, FFN-up, FFN-down), "
                                f"M=32760, R=1024" + (", g128" if t == "w4a8" else ""),
                           members=[f"c5{m}_{t}" for m in ("qkv", "proj", "up", "down")])
        for t in ("w4a8", "w8a8")}


def _parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="c3", choices=sorted(CONFIGS) + sorted(SETS) + [STEP_CONFIG, MLP_CONFIG, F6_CONFIG])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--calib-copy", action="store_true",
                    help="also run a plain 256 MiB device copy (PMC calibration)")
    ap.add_argument("--no-vendor", action="store_true",
                    help="skip the hipBLASLt reference GEMM on the same shape")
    ap.add_argument("--eager", action="store_true",
                    help="launch eagerly instead of replaying a captured graph (for counter collection)")
    ap.add_argument("--no-step", action="store_true",
                    help="skip the denoise-step times the default (c3) line carries")
    ap.add_argument("--w4-order", default="kil", choices=["kil", "plain", "unpacked"],
                    help="INT4 weight form the W4A8 GEMMs read: packed in the K-interleaved order (rewritten "
                         "once per weight, as the drop-in Linear does), packed in the checkpoint's order, or "
                         "unpacked to int8 (what the drop-in Linear uses for launches that fill at most half "
                         "the CUs)")
    ap.add_argument("--w16-layout", default="staged", choices=["staged", "plain"],
                    help="operand layout the W4A16 GEMMs read: the staged copy (stage-major weights, "
                         "group-major scales; what the drop-in Linear keeps for launches of more than 128 "
                         "rows) or the checkpoint's row-major packed weights and [N, G] scales")
    ap.add_argument("--rows", type=int, default=None,
                    help="override the config's M (GEMM configs; the line then names the override and "
                         "carries no committed traffic figure)")
    return ap.parse_args()


def make_inputs(cfg, seed=0):
    """Seeded synthetic inputs of BASELINE.json's config (host tensors)."""
    import torch

    g = torch.Generator().manual_seed(seed)
    M, K, N, G = cfg["M"], cfg["K"], cfg["N"], cfg["G"]
    K_in = cfg.get("K_in", K)
    act = torch.float16 if cfg["act"] == "fp16" else torch.bfloat16
    if cfg.get("dist") == "student_t":
        torch.manual_seed(seed)  # torch.distributions draws from the global generator
        x = torch.distributions.StudentT(4.0).sample((M, K_in))
    else:
        x = torch.randn(M, K_in, generator=g)
    if cfg["fmt"] == "int4" and cfg["name"].startswith("C3"):
        idx = torch.randperm(K, generator=g)[: K // 100]
        x[:, idx] *= 20.0
    x = x.to(act)
    inp = {"x": x}
    if cfg["fmt"] == "int8":
        inp["w"] = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
        inp["s_w"] = (torch.rand(N, 1, generator=g) * (2e-3 - 1e-4) + 1e-4).to(torch.float16).float()
    else:
        inp["w"] = torch.randint(0, 256, (N, K // 2), generator=g, dtype=torch.uint8)
        inp["s_w"] = (torch.rand(N, G, generator=g) * (2e-2 - 1e-3) + 1e-3).to(torch.float16).float()
    inp["smoothrot"] = torch.exp(torch.randn(K_in, generator=g) * 0.5) if cfg["smoothrot"] else None
    inp["perm"] = torch.randperm(K, generator=g) if cfg["perm"] else None
    return inp


def algorithmic(cfg):
    """(ops per GEMM launch, HBM bytes per GEMV launch, bytes per prep launch)."""
    M, K, N, G = cfg["M"], cfg["K"], cfg["N"], cfg["G"]
    K_in = cfg.get("K_in", K)
    ops = 2.0 * M * N * K  # K = padded weight K (pad columns carry rotated data)
    wbytes = N * K if cfg["fmt"] == "int8" else N * K // 2
    gemv_bytes = wbytes + 2 * N * G + 2 * M * K_in + 2 * M * N  # fp16 scales, 16-bit x and out
    prep_bytes = M * K_in * 2 + M * K + 4 * M
    return ops, gemv_bytes, prep_bytes


EAGER = False


def _time_loop(fn, n):
    """Average ms of n calls, captured once into a hipGraph (torch.cuda.CUDAGraph)
    and replayed between two events, so host launch latency does not hide the
    kernels (the reference replays CUDA graphs too, _cuda_graph.py:252-297).
    The kernels never allocate, synchronise or clear memory, so the graph holds
    kernel nodes only; outputs are checked against eager runs in the tests."""
    import torch

    if EAGER:
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record()
        for i in range(n):
            fn(i)
        e.record()
        e.synchronize()
        return s.elapsed_time(e) / n
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(n):
            fn(i)
    g.replay()  # warm-up replay
    torch.cuda.synchronize()
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    s.record()
    g.replay()
    e.record()
    e.synchronize()
    return s.elapsed_time(e) / n


def gpu_bench(cfg, inp, steps, warmup, rt, w4_order="kil", w16_layout="staged"):
    import torch

    dev = torch.device("cuda:0")
    M, K, N = cfg["M"], cfg["K"], cfg["N"]
    K_in = cfg.get("K_in", K)
    act = inp["x"].dtype
    # enough copies that weights + activations exceed the 256 MB Infinity Cache
    per_copy = inp["x"].numel() * inp["x"].element_size() + inp["w"].numel() * inp["w"].element_size()
    copies = max(2, min(64, math.ceil(640e6 / per_copy)))
    xs = [inp["x"].to(dev) for _ in range(copies)]
    ws = [inp["w"].to(dev) for _ in range(copies)]
    kil = cfg["fmt"] == "int4" and w4_order == "kil"
    unpacked = cfg["fmt"] == "int4" and w4_order == "unpacked"
    if kil:  # the per-layer rewrite the drop-in Linear does once, outside the timed steps
        ws = [rt.int4_interleave_k(w) for w in ws]
    elif unpacked:
        ws = [rt.unpack_int4_to_int8(w, K) for w in ws]
    s_w = inp["s_w"].to(dev)
    # W4A16: the staged operand layout the drop-in Linear keeps per layer, built
    # once outside the timed steps (big-tile shapes only)
    staged = (cfg["fmt"] == "w4a16" and w16_layout == "staged"
              and rt.w4a16_staged_pays(M, N, K, s_w.reshape(N, -1).shape[1]))
    if staged:
        ws = [rt.w4a16_stage_layout(w, s_w) for w in ws]
    sr = rt.prepare_factors(inp["smoothrot"].to(dev), act) if inp["smoothrot"] is not None else None
    perm = rt.prepare_perm(inp["perm"].to(dev), K) if inp["perm"] is not None else None
    q = torch.empty(M, K, dtype=torch.int8, device=dev)
    s_a = torch.empty(M, dtype=torch.float32, device=dev)
    out = torch.empty(M, N, dtype=act, device=dev)

    def prep(i):
        rt.rotate_quantize(xs[i % copies], rot_size=cfg["rot"], w_in=K, smoothrot=sr, perm=perm,
                           s_a_out=s_a, x_int8_out=q)

    def gemm(i):
        w = ws[i % copies]
        if staged:
            rt.gemm_w4a16_staged(xs[i % copies], w[0], w[1], out=out)
        elif cfg["fmt"] == "w4a16":
            rt.gemm_w4a16(xs[i % copies], w, s_w, out=out)
        elif cfg["fmt"] == "int8":
            rt.fused_int8_gemm_dequant(q, w, s_w, s_a, out_dtype=act, out=out)
        elif unpacked:
            rt.gemm_w4a8_unpacked(q, w, s_w, s_a, out_dtype=act, out=out)
        else:
            rt.gemm_w4a8(q, w, s_w, s_a, out_dtype=act, out=out, kil=kil)

    def step(i):
        if cfg["fmt"] != "w4a16":
            prep(i)
        gemm(i)

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    step_ms = _time_loop(step, steps)
    wall = time.perf_counter() - t0
    # kernels alone: a GEMV lasts ~10 us, so one replay's fixed launch cost is
    # spread over more launches there (the per-dispatch kernel-trace average
    # and this figure then agree)
    reps = steps if M > rt.GEMV_MAX_M else max(steps, 400)
    gemm_ms = _time_loop(gemm, reps)
    prep_ms = _time_loop(prep, reps) if cfg["fmt"] != "w4a16" else None
    return step_ms, wall, gemm_ms, prep_ms, copies


def cpu_baseline(cfg, inp):
    """Reference fp32 fallback (oracle restatement) timed on this host."""
    import torch

    import oracle

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    M, K, N = cfg["M"], cfg["K"], cfg["N"]
    rows = min(M, cfg.get("cpu_rows", M))  # bounded sample: the first `rows` tokens
    x = inp["x"][:rows]
    kw = dict(int4=cfg["fmt"] != "int8", smoothrot=inp["smoothrot"], rot_size=cfg["rot"], perm=inp["perm"])
    w = inp["w"].numpy()
    s_w = inp["s_w"].numpy()
    oracle.reference_fallback_forward(x, w, s_w, K, **kw)  # warm-up
    ts = []
    for _ in range(3):
        t0 = time.perf_counter()
        oracle.reference_fallback_forward(x, w, s_w, K, **kw)
        ts.append(time.perf_counter() - t0)
    t = statistics.median(ts)
    shape = "full shape" if rows == M else f"first {rows} of {M} tokens (throughput of the slice)"
    return {"value": round(2.0 * rows * N * K / t / 1e12, 5), "unit": "TOPS", "cores": cores,
            "cpu": cpu_model(), "kind": "port", "seconds_per_call": round(t, 5),
            "sample": f"{rows}x{cfg.get('K_in', K)} -> {N}, {shape}, fp32 dequant + prep + F.linear per call "
                      f"(the reference fallback re-dequantizes every forward), median of 3 after 1 warm-up"}


# ---------------------------------------------------------------- C4: Flux step
# One denoise step of a Flux-dev-style DiT: the model is
# in bench_flux.py (quantized block linears through this library, attention
# in torch's SDPA, glue in torch).  The step is captured once into a hipGraph
# and replayed; its parts are also timed alone on static inputs.
STEP_CONFIG = "c4step"
FLUX_LINEARS = (("qkv", 3072, 9216), ("proj", 3072, 3072), ("mlp_up", 3072, 12288), ("mlp_down", 12288, 3072))


def _time_graph(fn, reps):
    """Average ms of fn() captured once into a hipGraph and replayed reps
    times (launched eagerly instead under --eager).  Returns (ms, output of
    the captured call)."""
    import torch

    fn()
    torch.cuda.synchronize()
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    if EAGER:
        s.record()
        for _ in range(reps):
            out = fn()
        e.record()
        e.synchronize()
        return s.elapsed_time(e) / reps, out
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    g.replay()
    torch.cuda.synchronize()
    s.record()
    for _ in range(reps):
        g.replay()
    e.record()
    e.synchronize()
    return s.elapsed_time(e) / reps, out


def flux_step_bench(args, rt):
    import torch

    import bench_flux

    model = bench_flux.FluxStep(rt, torch.device("cuda:0"))
    reps = max(1, args.steps)
    for _ in range(max(0, args.warmup)):
        model.forward()
    torch.cuda.synchronize()
    eager = model.forward()
    torch.cuda.synchronize()
    eager = eager.clone()
    step_ms, out = _time_graph(model.forward, reps)
    torch.cuda.synchronize()
    replay_equal = bool(torch.equal(out, eager))
    finite = bool(torch.isfinite(out).all())
    parts, kinds = model.parts()
    part_ms = {name: _time_graph(fn, reps)[0] for name, fn in parts.items()}
    per_kind = {name: round(_time_graph(fn, reps)[0], 4) for name, fn in kinds.items()}
    r = dict(step_ms=step_ms, part_ms=part_ms, per_kind=per_kind, replay_equal=replay_equal, finite=finite)
    r.update(model.op_counts())
    # the same step through the drop-in ops layer (IntCrushOps.Linear per linear)
    del parts, kinds
    dropin = bench_flux.DropInFluxStep(rt, torch.device("cuda:0"))
    for _ in range(max(1, args.warmup)):
        dropin.forward()
    torch.cuda.synchronize()
    d_eager = dropin.forward().clone()
    torch.cuda.synchronize()
    d_eager_ms, d_eager_wall = _time_eager(dropin.forward, reps)
    d_ms, d_out = _time_graph(dropin.forward, reps)
    torch.cuda.synchronize()
    a, b = d_out.double().reshape(-1), eager.double().reshape(-1)
    r.update(dropin_step_ms=d_ms, dropin_eager_ms=d_eager_ms, dropin_eager_wall_ms=d_eager_wall,
             dropin_replay_equal=bool(torch.equal(d_out, d_eager)),
             dropin_cos_vs_fused=float((a @ b) / (a.norm() * b.norm())))
    return r


def _time_eager(fn, reps):
    """Average ms (HIP events) and host wall ms of reps eager calls of fn."""
    import torch

    torch.cuda.synchronize()
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    e.synchronize()
    return s.elapsed_time(e) / reps, (time.perf_counter() - t0) * 1e3 / reps


def denoise_step_times(rt, reps=5, warmup=2):
    """The C4 denoise step three ways: the fused model
    (FluxStep: hand-fused norms and epilogues) replayed as one hipGraph; the
    drop-in model (DropInFluxStep: every quantized linear an
    IntCrushOps.Linear, torch glue between them) replayed as one hipGraph; and
    the drop-in model launched eagerly, layer by layer, the way ComfyUI calls
    IntCrushOps.Linear.forward (reference _ops.py:817-862)."""
    import torch

    import bench_flux

    dev = torch.device("cuda:0")
    fused = bench_flux.FluxStep(rt, dev)
    for _ in range(warmup):
        fused.forward()
    fused_ms, _ = _time_graph(fused.forward, reps)
    del fused
    torch.cuda.empty_cache()
    dropin = bench_flux.DropInFluxStep(rt, dev)
    for _ in range(warmup):
        dropin.forward()
    eager_ms, eager_wall = _time_eager(dropin.forward, reps)
    graph_ms, _ = _time_graph(dropin.forward, reps)
    del dropin
    torch.cuda.empty_cache()
    return {"fused_graph_ms": round(fused_ms, 3), "dropin_graph_ms": round(graph_ms, 3),
            "dropin_eager_ms": round(eager_ms, 3), "dropin_eager_host_wall_ms": round(eager_wall, 3),
            "dropin_eager_over_graph": round(eager_ms / graph_ms, 4), "reps": reps,
            "workload": "C4 Flux-dev denoise step, batch 1, bf16, random init: 19 double + 38 single blocks, "
                        "4096 image + 512 text tokens, W4A8 R=256 g128 block linears, M=1 modulation GEMVs, "
                        "attention in torch SDPA",
            "note": "fused: FluxStep (adaLN fused into the preps, GELU-tanh and residual in GEMM epilogues), one "
                    "hipGraph; dropin: every quantized linear an IntCrushOps.Linear (make_intcrush_ops("
                    "'int4_crush', 256), ComfyUI stand-in from tests/fake_comfy), torch glue between them, "
                    "as one hipGraph and eagerly (per-layer forward calls, no whole-step capture)"}


def flux_step_cpu_baseline(rows=512):
    """Reference fp32 fallback (oracle restatement) on one layer of each Flux
    linear shape at `rows` tokens; the step estimate scales that throughput to
    the step's operations (labelled as extrapolated)."""
    import torch

    import oracle

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    gen = torch.Generator().manual_seed(0)
    ops, secs = 0.0, 0.0
    for _, k, n in FLUX_LINEARS:
        x = torch.randn(rows, k, generator=gen).to(torch.bfloat16)
        w = torch.randint(0, 256, (n, k // 2), generator=gen, dtype=torch.uint8).numpy()
        sw = (torch.rand(n, k // 128, generator=gen) * (2e-2 - 1e-3) + 1e-3).to(torch.float16).float().numpy()
        kw = dict(int4=True, smoothrot=torch.exp(torch.randn(k, generator=gen) * 0.5), rot_size=256,
                  perm=torch.randperm(k, generator=gen))
        oracle.reference_fallback_forward(x, w, sw, k, **kw)  # warm-up
        ts = []
        for _ in range(3):
            t0 = time.perf_counter()
            oracle.reference_fallback_forward(x, w, sw, k, **kw)
            ts.append(time.perf_counter() - t0)
        secs += statistics.median(ts)
        ops += 2.0 * rows * k * n
    return ops / secs, cores


def flux_step_main(args, rt):
    r = flux_step_bench(args, rt)
    pm = r["part_ms"]
    total_ops = r["lin_ops"] + r["mod_ops"]
    gemm_tops = r["lin_ops"] / (pm["gemm_w4a8"] * 1e-3) / 1e12
    breakdown = {"step": round(r["step_ms"], 4)}
    breakdown.update({k: round(v, 4) for k, v in pm.items()})
    breakdown["other_torch_ops"] = round(r["step_ms"] - sum(pm.values()), 4)
    breakdown["gemm_by_layer"] = r["per_kind"]
    line = {
        "metric": METRIC, "value": round(total_ops / (r["step_ms"] * 1e-3) / 1e12, 3), "unit": "TOPS",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(r["step_ms"], 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "C4 Flux-dev denoise step, batch 1, bf16, random init: embedders, "
                               "19 double blocks (img 4096 + txt 512 tokens) + 38 single blocks (4608 tokens), "
                               "final layer; block linears W4A8 R=256 g128 SmoothRot+perm with bias, "
                               "76 M=1 modulation GEMVs, attention in torch SDPA (flash), whole step in one hipGraph",
                   "quantized_linears": r["n_layers"], "modulation_gemvs": r["n_mods"],
                   "int4_weight_bytes": r["weight_bytes"], "attention_flops": r["attn_flops"],
                   "parallelism": "single GPU"},
        "value_note": "quantized linear + modulation ops of the step divided by the whole step time "
                      "(attention and the torch glue included in the time)",
        "roofline": {"bound": "mfma", "kernel": "gemm_w4a8 (all block-linear launches of the step)",
                     "achieved": round(gemm_tops, 2), "peak": PEAK_INT8_TOPS, "unit": "TOPS",
                     "frac": round(gemm_tops / PEAK_INT8_TOPS, 4), "kernel_ms": round(pm["gemm_w4a8"], 4),
                     "algorithmic_ops_per_step": r["lin_ops"], "traffic": None},
        "breakdown_ms": breakdown,
        "breakdown_note": "parts timed alone on static inputs with the step's layers and shapes; "
                          "other_torch_ops = step minus the timed parts (norms, modulation, RoPE, GELU, "
                          "residuals, embedders, final layer, concatenations)",
        "graph_replay_equals_eager": r["replay_equal"], "output_finite": r["finite"],
        "dropin_step": {"ms": round(r["dropin_step_ms"], 4), "eager_ms": round(r["dropin_eager_ms"], 4),
                        "eager_host_wall_ms": round(r["dropin_eager_wall_ms"], 4),
                        "graph_replay_equals_eager": r["dropin_replay_equal"],
                        "output_cosine_vs_fused_step": round(r["dropin_cos_vs_fused"], 7),
                        "note": "the same model with every quantized linear an IntCrushOps.Linear "
                                "(make_intcrush_ops('int4_crush', 256), ComfyUI stand-in from tests/fake_comfy): "
                                "per linear prep + W4A8 GEMM, adaLN / GELU-tanh / residuals as torch ops, "
                                "whole step in one hipGraph (ms) and launched eagerly layer by layer (eager_ms)"},
    }
    peaks = measure_peaks()
    line["peak_measured"] = peaks
    line["roofline"]["frac_of_measured_peak"] = round(gemm_tops / peaks["int8_tops"], 4)
    if not args.no_cpu:
        tops, cores = flux_step_cpu_baseline()
        line["cpu_baseline"] = {"value": round(tops / 1e12, 5), "unit": "TOPS", "cores": cores, "cpu": cpu_model(),
                                "kind": "port",
                                "extrapolated_linears_s": round(total_ops / tops, 2),
                                "sample": "one layer of each Flux linear shape (qkv, proj, mlp_up, mlp_down) at "
                                          "512 tokens, fp32 dequant + prep + F.linear per call, median of 3; "
                                          "the time of the step's quantized linears extrapolated from that "
                                          "throughput (attention and glue not included)"}
    print(json.dumps(line), flush=True)


def measure_peaks():
    """Rates this GPU sustains at its loaded clock: dense INT8 and FP16 MFMA
    from register-only loops (bench_peak.hip) and HBM from a 1 GiB
    device-to-device copy (read + write bytes).  Reported beside the
    published peaks the roofline fractions use."""
    import ctypes

    import torch

    import __graft_entry__

    if not os.path.exists(__graft_entry__.PEAK_LIB):
        __graft_entry__.build_peak_probe()
    lib = ctypes.CDLL(__graft_entry__.PEAK_LIB)
    lib.bp_grid.restype = ctypes.c_int
    lib.bp_ops_per_launch.restype = ctypes.c_double
    lib.bp_ops_per_launch.argtypes = [ctypes.c_int, ctypes.c_int]
    lib.bp_mfma_i8.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    lib.bp_mfma_f16.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    lib.bp_mfma_i8.restype = lib.bp_mfma_f16.restype = lib.bp_wall_clock_khz.restype = ctypes.c_int
    out = torch.empty(lib.bp_grid() * 256, dtype=torch.int32, device="cuda:0")
    clk = torch.zeros(4, dtype=torch.int64, device="cuda:0")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    iters = 4000
    launch = {0: lambda c=None: lib.bp_mfma_i8(iters, ctypes.c_void_p(out.data_ptr()), c, stream),
              1: lambda c=None: lib.bp_mfma_f16(iters, ctypes.c_void_p(out.data_ptr()), stream)}
    rates = {}
    for kind in (0, 1):
        for _ in range(2):  # warm-up: clocks settle under load
            if launch[kind]() != 0:
                raise RuntimeError("peak probe launch failed")
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record()
        for i in range(5):
            launch[kind](ctypes.c_void_p(clk.data_ptr()) if kind == 0 and i == 4 else None)
        e.record()
        e.synchronize()
        rates[kind] = 5 * lib.bp_ops_per_launch(kind, iters) / (s.elapsed_time(e) * 1e-3) / 1e12
    c0, c1, w0, w1 = clk.tolist()
    wall_khz = lib.bp_wall_clock_khz()
    sclk_mhz = (c1 - c0) / (w1 - w0) * wall_khz / 1e3 if w1 > w0 and wall_khz > 0 else None
    # L2 / Infinity Cache -> LDS by global_load_lds_dwordx4, the GEMMs' operand path
    lib.bp_lds_delivery.argtypes = [ctypes.c_void_p, ctypes.c_longlong, ctypes.c_int, ctypes.c_void_p,
                                    ctypes.c_void_p]
    lib.bp_lds_delivery.restype = ctypes.c_int
    lib.bp_lds_delivery_bytes.argtypes = [ctypes.c_int]
    lib.bp_lds_delivery_bytes.restype = ctypes.c_double
    sink = torch.empty(lib.bp_grid() // 2, dtype=torch.int32, device="cuda:0")
    deliv = {}
    for name, size in (("l2", 2 << 20), ("infinity_cache", 64 << 20)):
        buf = torch.ones(size, dtype=torch.uint8, device="cuda:0")
        d_iters = 400
        run = lambda: lib.bp_lds_delivery(ctypes.c_void_p(buf.data_ptr()), size, d_iters,
                                          ctypes.c_void_p(sink.data_ptr()), stream)
        for _ in range(2):
            if run() != 0:
                raise RuntimeError("LDS delivery probe launch failed")
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(3):
            run()
        e.record()
        e.synchronize()
        deliv[name] = 3 * lib.bp_lds_delivery_bytes(d_iters) / (s.elapsed_time(e) * 1e-3)
        del buf
    cus = lib.bp_grid() // 2
    a = torch.empty(1 << 30, dtype=torch.uint8, device="cuda:0")
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(5):
        b.copy_(a)
    e.record()
    e.synchronize()
    hbm = 5 * 2 * a.numel() / (s.elapsed_time(e) * 1e-3) / 1e9
    del a, b
    return {"int8_tops": round(rates[0], 1), "fp16_tflops": round(rates[1], 1), "hbm_copy_gbps": round(hbm, 1),
            "lds_delivery_tbps": {k: round(v / 1e12, 2) for k, v in deliv.items()},
            "lds_delivery_bytes_per_clk_cu": ({k: round(v / cus / (sclk_mhz * 1e6), 1) for k, v in deliv.items()}
                                              if sclk_mhz else None),
            "sclk_mhz": round(sclk_mhz) if sclk_mhz else None,
            "int8_peak_at_sclk_tops": round(PEAK_INT8_TOPS * sclk_mhz / PEAK_SCLK_MHZ, 1) if sclk_mhz else None,
            "method": "register-only MFMA loops (v_mfma_i32_32x32x32_i8, v_mfma_f32_32x32x16_f16), "
                      "2 workgroups of 4 waves per CU, 4 independent accumulator chains per wave; "
                      "sclk: shader-clock ticks over wall-clock ticks across one wave's INT8 loop; "
                      f"int8_peak_at_sclk: the published peak scaled by sclk / {PEAK_SCLK_MHZ} MHz; "
                      "HBM: 1 GiB device copy, read + write bytes; LDS delivery: global_load_lds_dwordx4 "
                      "into LDS, 56 KB stages per CU with two in flight, from a 2 MB (L2-resident) and a "
                      "64 MB (Infinity Cache) buffer"}


def vendor_reference(cfg, reps=20):
    """The vendor library on the same GEMM shape, as a reference point for
    the roofline fraction: hipBLASLt through torch._int_mm (int8 x int8 ->
    int32, no dequant epilogue, no INT4 unpack, no group fold) for the INT8
    MFMA configs, torch.matmul in the activation dtype on a dense
    pre-dequantized weight for W4A16.  Synthetic operands of the config's
    shape; not part of the timed step."""
    import torch

    M, K, N = cfg["M"], cfg["K"], cfg["N"]
    g = torch.Generator(device="cuda:0").manual_seed(7)
    if cfg["fmt"] == "w4a16":
        act = torch.float16 if cfg["act"] == "fp16" else torch.bfloat16
        a = torch.randn(M, K, generator=g, device="cuda:0").to(act)
        b = (torch.randn(K, N, generator=g, device="cuda:0") * 0.02).to(act)
        fn, kernel, ops_unit = (lambda: torch.matmul(a, b)), f"torch.matmul {cfg['act']} (hipBLASLt)", "TFLOP/s"
    else:
        a = torch.randint(-127, 128, (M, K), generator=g, device="cuda:0", dtype=torch.int8)
        b = torch.randint(-127, 128, (K, N), generator=g, device="cuda:0", dtype=torch.int8)
        fn, kernel, ops_unit = (lambda: torch._int_mm(a, b)), "torch._int_mm int8->int32 (hipBLASLt)", "TOPS"
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    e.synchronize()
    ms = s.elapsed_time(e) / reps
    return {"kernel": kernel, "kernel_ms": round(ms, 5), "achieved": round(2.0 * M * N * K / (ms * 1e-3) / 1e12, 1),
            "unit": ops_unit, "note": "same M, K, N; plain GEMM without this path's fused work"}


def set_main(args, rt):
    """A set of linears (the C5 Wan block): each member's prep + GEMM step timed
    as in a single-linear config, one after another; the line reports the
    set's ops over the summed step times, the GEMMs' roofline over their
    summed kernel times, and the CPU fallback on each member's bounded
    token slice."""
    import torch

    st = SETS[args.config]
    tot_ops = step_ms = gemm_ms = prep_ms = 0.0
    cpu_s = cpu_ops = 0.0
    members = []
    cores = None
    for key in st["members"]:
        cfg = CONFIGS[key]
        inp = make_inputs(cfg)
        s_ms, _wall, g_ms, p_ms, copies = gpu_bench(cfg, inp, args.steps, args.warmup, rt, args.w4_order,
                                                      args.w16_layout)
        ops, _gb, _pb = algorithmic(cfg)
        tot_ops += ops
        step_ms += s_ms
        gemm_ms += g_ms
        prep_ms += p_ms or 0.0
        members.append({"linear": cfg["name"], "ms_per_step": round(s_ms, 5), "gemm_ms": round(g_ms, 5),
                        "prep_ms": round(p_ms, 5) if p_ms is not None else None,
                        "gemm_tops": round(ops / (g_ms * 1e-3) / 1e12, 1)})
        if not args.no_cpu:
            cb = cpu_baseline(cfg, inp)
            cpu_s += cb["seconds_per_call"]
            rows = min(cfg["M"], cfg.get("cpu_rows", cfg["M"]))
            cpu_ops += 2.0 * rows * cfg["N"] * cfg["K"]
            cores = cb["cores"]
        del inp
        torch.cuda.empty_cache()
    first = CONFIGS[st["members"][0]]
    fmt = first["fmt"]
    achieved = tot_ops / (gemm_ms * 1e-3) / 1e12
    line = {
        "metric": METRIC, "value": round(tot_ops / (step_ms * 1e-3) / 1e12, 3), "unit": "TOPS",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(step_ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": st["name"], "M": first["M"], "members": members, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "kernel": "gemm_w4a8" if fmt == "int4" else "gemm_w8a8",
                     "achieved": round(achieved, 2), "peak": PEAK_INT8_TOPS, "unit": "TOPS",
                     "frac": round(achieved / PEAK_INT8_TOPS, 4), "kernel_ms": round(gemm_ms, 5),
                     "algorithmic_ops_per_step": tot_ops, "traffic": None},
        "prep_quant_ms": round(prep_ms, 5),
    }
    line["peak_measured"] = measure_peaks()
    line["roofline"]["frac_of_measured_peak"] = round(achieved / line["peak_measured"]["int8_tops"], 4)
    if not args.no_cpu:
        line["cpu_baseline"] = {"value": round(cpu_ops / cpu_s / 1e12, 5), "unit": "TOPS", "cores": cores,
                                "cpu": cpu_model(), "kind": "port", "seconds": round(cpu_s, 3),
                                "sample": "each member's first 2048 of 32760 tokens, fp32 dequant + prep + "
                                          "F.linear per call, median of 3 after 1 warm-up, summed"}
    print(json.dumps(line), flush=True)


# ------------------------------------------------ C4 MLP: chained epilogue
# The Flux MLP between its two quantized linears, two ways: (a) the up-
# projection GEMM with its GELU-tanh epilogue, then the down-projection's full
# prep (SmoothRot divide, R = 256 Hadamard, perm, per-row INT8 quantization);
# (b) the chained up-projection (ic_gemm_*_chain: GELU, divide and Hadamard
# in the GEMM's epilogue), then the rest of the prep (perm and quantization).
MLP_CONFIG = "c4mlp"
MLP_SHAPES = ((4096, "double-block image stream"), (512, "double-block text stream"), (4608, "C3 rows"))


def mlp_chain_main(args, rt):
    import torch

    dev = torch.device("cuda:0")
    K, N, R = 3072, 12288, 256
    dt = torch.bfloat16
    rows = []
    for kind in ("w4a8", "w8a8"):
        for M, what in MLP_SHAPES:
            g = torch.Generator().manual_seed(M)
            xq = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8).to(dev)
            s_a = (torch.rand(M, generator=g) * 0.02 + 0.005).to(dev)
            bias = (torch.randn(N, generator=g) * 0.1).to(dev)
            if kind == "w8a8":
                w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).to(dev)
                s_w = (torch.rand(N, generator=g) * 2e-3 + 1e-4).to(dev)
            else:
                w = torch.randint(0, 256, (N, K // 2), generator=g, dtype=torch.uint8).to(dev)
                s_w = (torch.rand(N, K // 128, generator=g) * 0.02 + 1e-3).to(dev)
            srf = rt.prepare_factors(torch.exp(torch.randn(N, generator=g) * 0.5).to(dev), dt)
            perm = rt.prepare_perm(torch.randperm(N, generator=g).to(dev), N)
            h = torch.empty(M, N, dtype=dt, device=dev)
            y = torch.empty_like(h)
            q = torch.empty(M, N, dtype=torch.int8, device=dev)
            sq = torch.empty(M, dtype=torch.float32, device=dev)
            q2 = torch.empty_like(q)
            sq2 = torch.empty_like(sq)

            def up():
                if kind == "w8a8":
                    rt.fused_int8_gemm_dequant(xq, w, s_w, s_a, bias=bias, out_dtype=dt, activation=rt.ACT_GELU_TANH,
                                               out=h)
                else:
                    rt.gemm_w4a8(xq, w, s_w, s_a, bias=bias, out_dtype=dt, activation=rt.ACT_GELU_TANH, out=h)

            def prep_full():
                rt.rotate_quantize(h, rot_size=R, w_in=N, smoothrot=srf, perm=perm, s_a_out=sq, x_int8_out=q)

            def chain():
                rt.gemm_chain(xq, w, s_w, s_a, rot_size=R, smoothrot=srf, bias=bias, out_dtype=dt,
                              activation=rt.ACT_GELU_TANH, out=y)

            def prep_rest():
                rt.rotate_quantize(y, rot_size=0, w_in=N, perm=perm, s_a_out=sq2, x_int8_out=q2)

            t = {"up": [], "prep_full": [], "chain": [], "prep_rest": []}
            for _ in range(3):  # interleaved repeats, averaged
                for name, fn in (("up", up), ("prep_full", prep_full), ("chain", chain), ("prep_rest", prep_rest)):
                    t[name].append(_time_graph(fn, args.steps)[0] * 1e3)
            up(); prep_full(); chain(); prep_rest()
            torch.cuda.synchronize()
            same = bool(torch.equal(q, q2) and torch.equal(sq, sq2))
            a = {k: sum(v) / len(v) for k, v in t.items()}
            rows.append({"weights": kind, "M": M, "rows": what, "gemm_gelu_us": round(a["up"], 1),
                         "prep_full_us": round(a["prep_full"], 1), "two_kernel_us": round(a["up"] + a["prep_full"], 1),
                         "chain_gemm_us": round(a["chain"], 1), "prep_rest_us": round(a["prep_rest"], 1),
                         "chained_us": round(a["chain"] + a["prep_rest"], 1), "codes_identical": same})
            del xq, w, h, y, q, q2
            torch.cuda.empty_cache()
    head = rows[0]
    line = {
        "metric": "Flux MLP up-projection + down-projection prep, chained epilogue against two kernels",
        "value": head["chained_us"], "unit": "us", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(head["chained_us"] / 1e3, 5), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": f"C4 MLP 3072->12288 (GELU-tanh) -> prep of 12288->3072 (R=256, SmoothRot, perm), "
                               f"bf16; value: W4A8 g128 at M={head['M']}", "parallelism": "single GPU",
                   "rows": rows},
    }
    print(json.dumps(line), flush=True)


# ------------------------------------------- C3 GEMM on e3m2 operands (fp6)
# The grouped W4A8 GEMM of C3 two ways in one process: the int8 MFMA kernel
# (gemm_w4a8, what the library routes to) and the f8f6f4 MFMA kernel on
# e3m2 operands (gemm_w4a8_f6: no group-sum converts, no INT4 expansion, 1.5x
# the operand bytes), on the C3 prep's own codes.  Alternating rounds; the
# outputs are compared bit for bit.
F6_CONFIG = "c3f6"


def f6_main(args, rt):
    import torch

    cfg = CONFIGS["c3"]
    inp = make_inputs(cfg)
    dev = torch.device("cuda:0")
    M, K, N = cfg["M"], cfg["K"], cfg["N"]
    act = inp["x"].dtype
    per_copy = inp["w"].numel() * 3 // 2  # e3m2 weight bytes per copy
    copies = max(2, min(64, math.ceil(640e6 / per_copy)))
    ws = [inp["w"].to(dev) for _ in range(copies)]
    w6s = [rt.f6_repack_weights(w, K) for w in ws]
    s_w = inp["s_w"].to(dev)
    sr = rt.prepare_factors(inp["smoothrot"].to(dev), act)
    perm = rt.prepare_perm(inp["perm"].to(dev), K)
    q, s_a = rt.rotate_quantize(inp["x"].to(dev), rot_size=cfg["rot"], w_in=K, smoothrot=sr, perm=perm)
    a6 = rt.f6_split_activations(q)
    out_i8 = torch.empty(M, N, dtype=act, device=dev)
    out_f6 = torch.empty_like(out_i8)

    def i8(i):
        rt.gemm_w4a8(q, ws[i % copies], s_w, s_a, out_dtype=act, out=out_i8)

    def f6(i):
        rt.gemm_w4a8_f6(a6, M, K, w6s[i % copies], N, s_w, s_a, out_dtype=act, out=out_f6)

    def split(i):
        rt.f6_split_activations(q)

    for i in range(max(1, args.warmup)):
        i8(i)
        f6(i)
    torch.cuda.synchronize()
    same = bool(torch.equal(out_i8, out_f6))
    t = {"int8": [], "f6": []}
    for _ in range(3):
        t["int8"].append(_time_loop(i8, args.steps))
        t["f6"].append(_time_loop(f6, args.steps))
    split_ms = _time_loop(split, args.steps)
    ops, _gb, _pb = algorithmic(cfg)
    med = {k: statistics.median(v) for k, v in t.items()}
    tops = {k: ops / (v * 1e-3) / 1e12 for k, v in med.items()}
    line = {
        "metric": "C3 grouped W4A8 GEMM: int8 MFMA kernel against the e3m2 f8f6f4 MFMA kernel",
        "value": round(tops["f6"], 2), "unit": "TOPS", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(med["f6"], 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8", "data": "synthetic",
        "config": {"workload": "C3 GEMM 4608 x 12288 -> 3072, g128, on the C3 prep's codes", "input_copies": copies,
                   "parallelism": "single GPU"},
        "int8_kernel": {"ms": [round(v, 5) for v in t["int8"]], "tops": round(tops["int8"], 1),
                        "frac": round(tops["int8"] / PEAK_INT8_TOPS, 4)},
        "f6_kernel": {"ms": [round(v, 5) for v in t["f6"]], "tops": round(tops["f6"], 1),
                      "frac": round(tops["f6"] / PEAK_INT8_TOPS, 4)},
        "outputs_bit_identical": same,
        "split_activations_ms": round(split_ms, 5),
        "note": "the e3m2 route would also need the prep to write the split activations "
                "(1.5 bytes per code instead of 1), or the split pass timed here",
    }
    print(json.dumps(line), flush=True)


def traffic_for(workload_key):
    """HBM bytes per launch of the dominant kernel from committed rocprofv3 counters."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get(workload_key, {}).get("hbm_bytes_per_launch")


def main():
    args = _parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "multi-GPU sharding is a design note (token split), not a measured path.", file=sys.stderr)
        sys.exit(2)
    import torch

    import __graft_entry__

    rt = __graft_entry__._submodule("_hip_runtime")
    if not torch.cuda.is_available() or not rt.KERNELS_AVAILABLE:
        print(f"bench.py needs an MI355X and the built kernels ({rt.LOAD_ERROR})", file=sys.stderr)
        sys.exit(1)
    global EAGER
    EAGER = args.eager
    if args.config == STEP_CONFIG:
        flux_step_main(args, rt)
        return
    if args.config in SETS:
        set_main(args, rt)
        return
    if args.config == MLP_CONFIG:
        mlp_chain_main(args, rt)
        return
    if args.config == F6_CONFIG:
        f6_main(args, rt)
        return
    cfg = CONFIGS[args.config]
    if args.rows is not None:
        cfg = dict(cfg, M=int(args.rows), name=f"{cfg['name']} (M overridden to {int(args.rows)})")
    inp = make_inputs(cfg)
    if args.calib_copy:
        a = torch.empty(256 << 20, dtype=torch.uint8, device="cuda:0")
        b = torch.empty_like(a)
        b.copy_(a)
        torch.cuda.synchronize()
        del a, b
    step_ms, wall, g_ms, p_ms, copies = gpu_bench(cfg, inp, args.steps, args.warmup, rt, args.w4_order,
                                                      args.w16_layout)
    M, K, N = cfg["M"], cfg["K"], cfg["N"]
    ops, gemv_bytes, prep_bytes = algorithmic(cfg)
    is_fp = cfg["fmt"] == "w4a16"
    kname = "gemm_w4a16" if is_fp else ("gemm_w8a8" if cfg["fmt"] == "int8" else "gemm_w4a8")
    if M <= rt.GEMV_MAX_M:
        kname = kname.replace("gemm", "gemv")
        achieved = gemv_bytes / (g_ms * 1e-3) / 1e9
        roof = {"bound": "hbm", "kernel": kname, "achieved": round(achieved, 1), "peak": PEAK_HBM_GBPS,
                "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBPS, 4), "kernel_ms": round(g_ms, 5),
                "algorithmic_bytes_per_launch": gemv_bytes,
                "traffic": traffic_for(args.config) if args.rows is None else None}
    else:
        peak = PEAK_FP16_TFLOPS if is_fp else PEAK_INT8_TOPS
        achieved = ops / (g_ms * 1e-3) / 1e12
        roof = {"bound": "mfma", "kernel": kname, "achieved": round(achieved, 2), "peak": peak,
                "unit": "TFLOP/s" if is_fp else "TOPS", "frac": round(achieved / peak, 4),
                "kernel_ms": round(g_ms, 5), "algorithmic_ops_per_launch": ops,
                "traffic": traffic_for(args.config) if args.rows is None else None}
    line = {
        "metric": METRIC, "value": round(ops / (step_ms * 1e-3) / 1e12, 3), "unit": "TOPS",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(step_ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": cfg["act"] if is_fp else "int8", "data": "synthetic",
        "config": {"workload": cfg["name"], "M": M, "K_in": cfg.get("K_in", K), "K": K, "N": N,
                   "group_size": K // cfg["G"],
                   "rot_size": cfg["rot"], "smoothrot": cfg["smoothrot"], "perm": cfg["perm"],
                   "activation": cfg["act"], "input_copies": copies, "parallelism": "single GPU",
                   **({"w4_order": args.w4_order} if cfg["fmt"] == "int4" else {}),
                   **({"w16_layout": args.w16_layout} if is_fp else {})},
        "roofline": roof,
        "host_wall_ms_per_step": round(wall * 1e3 / args.steps, 5),
    }
    peaks = measure_peaks()
    line["peak_measured"] = peaks
    meas = peaks["hbm_copy_gbps"] if roof["bound"] == "hbm" else (peaks["fp16_tflops"] if is_fp else peaks["int8_tops"])
    roof["frac_of_measured_peak"] = round(roof["achieved"] / meas, 4)
    if p_ms is not None:
        pach = prep_bytes / (p_ms * 1e-3) / 1e9
        line["prep_quant"] = {"kernel": "rotate_quantize", "bound": "hbm", "kernel_ms": round(p_ms, 5),
                              "algorithmic_bytes": prep_bytes, "achieved": round(pach, 1),
                              "peak": PEAK_HBM_GBPS, "unit": "GB/s", "frac": round(pach / PEAK_HBM_GBPS, 4),
                              "frac_of_measured_peak": round(pach / peaks["hbm_copy_gbps"], 4)}
    if M > rt.GEMV_MAX_M and not args.no_vendor:
        line["vendor_gemm"] = vendor_reference(cfg)
    if args.config == "c3" and not args.no_step:
        # the metric's second half ("denoise step ms"), on the same box and run
        torch.cuda.empty_cache()
        line["denoise_step"] = denoise_step_times(rt)
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(cfg, inp)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
