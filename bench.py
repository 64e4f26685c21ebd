"""Benchmark of the Aurora GEMM / causal-attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--only LEG]

Workload: one "step" is one pass over the fp32 GEMM sweep
with M = B·T = 8192 — A@B and A@Bᵀ for (K,N) ∈ {(512,1536), (512,512),
(512,2048), (2048,512)}, the tied LM head [8192,512]·[8192,512]ᵀ and the
weight-gradient accumulate dest[2048,512] += dYᵀ·X with t = 8192 — on
seeded U(-1,1) inputs already resident in HBM.  `value` is the sweep's
total algorithmic FLOP (2·M·N·K per GEMM) divided by the measured time.

Prints ONE JSON line (the driver's contract) with a `roofline` object for
the dominant kernel (the tied-head GEMM launch, timed with HIP events on
the library's stream) and a `cpu_baseline` object: the reference CPU path's
GEMM (its linear_forward, restated in oracle/) timed on this host's cores on
a bounded sample of the same workload, with the host (nproc, affinity, CPU
model), the same GEMM on one thread, a config-2 attention sample, a
config-4 decode sample and one whole measured config-3 training step.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

PEAK_FP32_MFMA = 157.3  # TFLOP/s, MI355X dense fp32 matrix
PEAK_HBM = 8000.0       # GB/s

CLOCK_RAMP_S = 0.25     # untimed sustained work before a timed GEMM region
COPY_MIB = 256          # calibration copy of the --only traffic leg
# HBM bytes per head-GEMM launch from the two counter passes of
# profiles/gemm_head_nt_8192x8192x512_traffic.md: FETCH_SIZE 156261.9 KiB × 2.000
# + WRITE_SIZE 262144.4 KiB × 1.000 (factors from the 256 MiB copy).
HEAD_TRAFFIC_BYTES = (156261.9 * 2.000 + 262144.4 * 1.000) * 1024
SWEEP_KN = [(512, 1536), (512, 512), (512, 2048), (2048, 512)]
M = 8192


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def build_sweep(ctx, rng):
    """Device buffers for every GEMM of the sweep; returns a list of
    (name, flops, launch) where launch() enqueues that GEMM."""
    from aurora_amd.gpu import GpuBuffer

    def u(n):
        return GpuBuffer.from_slice(ctx, rng.uniform(-1, 1, n).astype(np.float32))

    items = []
    for k, n in SWEEP_KN:
        a, b_nn, b_nt = u(M * k), u(k * n), u(n * k)
        c = GpuBuffer.empty(ctx, M * n)
        fl = 2.0 * M * n * k
        items.append((f"nn_{M}x{n}x{k}", fl,
                      lambda a=a, b=b_nn, c=c, n=n, k=k: ctx.call("aur_gemm_nn", a.ptr, b.ptr, c.ptr, M, n, k)))
        items.append((f"nt_{M}x{n}x{k}", fl,
                      lambda a=a, b=b_nt, c=c, n=n, k=k: ctx.call("aur_gemm_nt", a.ptr, b.ptr, c.ptr, M, n, k)))
    h, w_tok = u(M * 512), u(8192 * 512)
    logits = GpuBuffer.empty(ctx, M * 8192)
    items.append(("head_nt_8192x8192x512", 2.0 * M * 8192 * 512,
                  lambda: ctx.call("aur_gemm_nt", h.ptr, w_tok.ptr, logits.ptr, M, 8192, 512)))
    x, dy, dest = u(M * 512), u(M * 2048), u(2048 * 512)
    items.append(("wgrad_accum_2048x512_t8192", 2.0 * 2048 * 512 * M,
                  lambda: ctx.call("aur_outer_accum", x.ptr, dy.ptr, dest.ptr, 2048, 512, M)))
    return items


def gemm_shape_list(m_sweep: int, m_c3: int) -> list[tuple[str, str, int, int, int]]:
    """(group, form, M or d_out, N or d_in, K or t) of the GEMMs one training
    step runs.  Group "c1": the config-1 sweep at M = m_sweep rows.  Group
    "c3": the config-3 (d_model 1024) training GEMMs at M = m_c3 rows —
    forward A@Bᵀ (fused QKV, W_o, fc, proj, tied head), backward dX = dY·W
    (A@B) and the weight-gradient accumulates dest += dYᵀ·X (form "acc":
    d_out, d_in, t)."""
    out = []
    for k, n in SWEEP_KN:
        out.append(("c1", "nn", m_sweep, n, k))
        out.append(("c1", "nt", m_sweep, n, k))
    out.append(("c1", "nt", m_sweep, 8192, 512))
    out.append(("c1", "acc", 2048, 512, m_sweep))
    d, F, V = C3["d_model"], C3["d_ff"], C3["vocab"]
    lin = [("qkv", 3 * d, d), ("w_o", d, d), ("fc", F, d), ("proj", d, F), ("head", V, d)]
    for _, n_out, n_in in lin:
        out.append(("c3", "nt", m_c3, n_out, n_in))
    for _, n_out, n_in in lin:
        out.append(("c3", "nn", m_c3, n_in, n_out))
    for _, n_out, n_in in lin:
        out.append(("c3", "acc", n_out, n_in, m_c3))
    return out


def bench_shapes(ctx, steps: int, m_sweep: int, m_c3: int, groups=("c1", "c3")) -> list[dict]:
    """TFLOP/s of every GEMM of gemm_shape_list(m_sweep, m_c3) in `groups`,
    each timed alone with HIP events after a warm-up (inputs U(-1,1), resident)."""
    from aurora_amd.gpu import GpuBuffer

    shapes = [s for s in gemm_shape_list(m_sweep, m_c3) if s[0] in groups]

    def need(form, a, b, c):
        if form == "acc":  # x [t, d_in], dy [t, d_out], dest [d_out, d_in]
            return c * b, c * a, a * b
        return a * c, b * c, a * b

    na = max(need(*s[1:])[0] for s in shapes)
    nb = max(need(*s[1:])[1] for s in shapes)
    nc = max(need(*s[1:])[2] for s in shapes)
    rng = np.random.default_rng(3)
    bufs = [GpuBuffer.from_slice(ctx, (2 * rng.random(n, dtype=np.float32) - 1)) for n in (na, nb, nc)]
    pa, pb, pc = (b.ptr for b in bufs)
    first = shapes[0]
    ramp_end = time.perf_counter() + CLOCK_RAMP_S
    while time.perf_counter() < ramp_end:  # clock ramp (see main)
        for _ in range(10):
            if first[1] == "acc":
                ctx.call("aur_outer_accum", pa, pb, pc, first[2], first[3], first[4])
            else:
                ctx.call("aur_gemm_nn" if first[1] == "nn" else "aur_gemm_nt", pa, pb, pc, *first[2:])
        ctx.sync()
    res = []
    for group, form, a, b, c in shapes:
        if form == "acc":
            fn = lambda a=a, b=b, c=c: ctx.call("aur_outer_accum", pa, pb, pc, a, b, c)
            name = f"acc_{a}x{b}_t{c}"
        else:
            sym = "aur_gemm_nn" if form == "nn" else "aur_gemm_nt"
            fn = lambda sym=sym, a=a, b=b, c=c: ctx.call(sym, pa, pb, pc, a, b, c)
            name = f"{form}_{a}x{b}x{c}"
        for _ in range(3):
            fn()
        ms = time_region(ctx, fn, steps)
        tf = 2.0 * a * b * c / (ms * 1e-3) / 1e12
        res.append({"group": group, "gemm": name, "ms": round(ms, 4), "tflops": round(tf, 2),
                    "pct_peak": round(100 * tf / PEAK_FP32_MFMA, 1)})
        log(f"[bench]   {group} {name:28s} {ms:8.4f} ms {tf:7.1f} TFLOP/s {100 * tf / PEAK_FP32_MFMA:5.1f}%")
    for x in bufs:
        x.free()
    return res


def shapes_summary(rows: list[dict], group: str) -> dict:
    sel = [r for r in rows if r["group"] == group]
    ms = sum(r["ms"] for r in sel)
    fl = sum(r["tflops"] * 1e12 * r["ms"] * 1e-3 for r in sel)
    return {"n_gemms": len(sel), "total_ms": round(ms, 4), "tflops": round(fl / (ms * 1e-3) / 1e12, 2),
            "min_pct_peak": min(r["pct_peak"] for r in sel),
            "pct_peak": round(100 * fl / (ms * 1e-3) / 1e12 / PEAK_FP32_MFMA, 1)}


def bench_c3_and_shards(ctx, steps: int) -> dict:
    """The config-3 training GEMMs at full size (M = B·T = 16384, the shapes the
    ≥ 60 % target is stated on) and one GPU's share of both workloads under
    8-way data parallelism (config 1 at M = 1024 rows, config 3 at M = 2048,
    weight-gradient t likewise)."""
    full = bench_shapes(ctx, steps, M, 16384, groups=("c3",))
    shard = bench_shapes(ctx, steps, M // 8, 16384 // 8)
    return {"c3_gemms": {**shapes_summary(full, "c3"), "per": full},
            "dp8_shard": {"c1_m1024": shapes_summary(shard, "c1"), "c3_m2048": shapes_summary(shard, "c3"),
                          "per": shard}}


def time_region(ctx, fn, steps: int) -> float:
    """ms per call of fn() over `steps` calls, bracketed by HIP events on the
    library's stream after a full synchronisation."""
    ctx.sync()
    e0, e1 = ctx.event(), ctx.event()
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    ms = e0.elapsed_ms(e1) / steps
    ctx.sync()
    e0.destroy()
    e1.destroy()
    return ms


def bench_ceilings(ctx, cus: int) -> dict:
    """What this GPU sustains, measured with the probes of
    aurora_amd/probes/ceilings.hip on the library's stream: fp32 MFMA with
    register operands (2 blocks of 4 waves per CU, 8 independent chains per
    wave), a streaming read of 2 GiB (the best of 2-16 blocks per CU with 4
    or 8 float4 loads in flight per lane), and an empty kernel replayed from a HIP graph (per
    launch, over 100 captured launches).  The roofline fractions keep the
    published peaks; these say how much of them the silicon reaches."""
    import ctypes as C

    from aurora_amd.build import PROBE_LIB
    from aurora_amd.gpu import GpuBuffer, _lib

    if not PROBE_LIB.exists():
        raise RuntimeError(f"{PROBE_LIB} is missing: run __graft_entry__.build()")
    lib = C.CDLL(str(PROBE_LIB))
    lib.ceil_mfma_f32_flop.restype = C.c_double
    lib.ceil_mfma_f32_flop.argtypes = [C.c_int, C.c_int]
    lib.ceil_mfma_f32.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_void_p]
    lib.ceil_mfma_f32_32x32_flop.restype = C.c_double
    lib.ceil_mfma_f32_32x32_flop.argtypes = [C.c_int, C.c_int]
    lib.ceil_mfma_f32_32x32.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_void_p]
    lib.ceil_stream_read.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_int, C.c_void_p]
    lib.ceil_graph_create.argtypes = [C.c_void_p, C.c_int, C.POINTER(C.c_void_p)]
    lib.ceil_graph_reads_create.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_int, C.c_int,
                                            C.c_int, C.c_void_p, C.POINTER(C.c_void_p)]
    lib.ceil_graph_launch.argtypes = [C.c_void_p, C.c_void_p]
    lib.ceil_graph_destroy.argtypes = [C.c_void_p]
    stream = _lib.load().aur_stream(ctx.ptr)

    def ok(rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed with HIP error {rc}")

    mfma_blocks, iters = 2 * cus, 20000
    sink = GpuBuffer.empty(ctx, 16 * cus * 256)
    ramp_end = time.perf_counter() + CLOCK_RAMP_S
    while time.perf_counter() < ramp_end:
        ok(lib.ceil_mfma_f32(stream, mfma_blocks, iters, sink.ptr), "ceil_mfma_f32")
        ctx.sync()
    ms = time_region(ctx, lambda: ok(lib.ceil_mfma_f32(stream, mfma_blocks, iters, sink.ptr), "ceil_mfma_f32"), 5)
    mfma_tf = lib.ceil_mfma_f32_flop(mfma_blocks, iters) / (ms * 1e-3) / 1e12
    # the 32x32x2 form, same FLOP per launch (half the iterations)
    ms32 = time_region(ctx, lambda: ok(lib.ceil_mfma_f32_32x32(stream, mfma_blocks, iters // 2, sink.ptr),
                                        "ceil_mfma_f32_32x32"), 5)
    mfma32_tf = lib.ceil_mfma_f32_32x32_flop(mfma_blocks, iters // 2) / (ms32 * 1e-3) / 1e12

    nbytes = 2 << 30
    src = GpuBuffer.zeros(ctx, nbytes // 4)
    reads = {}
    for mode, depth in ((0, "4 loads"), (1, "8 loads"), (2, "8 non-temporal loads")):
        for per_cu in (2, 4, 8, 16):
            blocks = per_cu * cus

            def rd(mode=mode, blocks=blocks):
                ok(lib.ceil_stream_read(stream, src.ptr, nbytes, blocks, mode, sink.ptr), "ceil_stream_read")

            for _ in range(2):
                rd()
            reads[f"{depth}, {per_cu} blocks/CU"] = nbytes / (time_region(ctx, rd, 5) * 1e-3) / 1e9
    best = max(reads, key=reads.get)
    read_gbs = reads[best]
    src.free()

    n_launch = 100
    ex = C.c_void_p()
    ok(lib.ceil_graph_create(stream, n_launch, C.byref(ex)), "ceil_graph_create")
    for _ in range(5):
        ok(lib.ceil_graph_launch(stream, ex), "ceil_graph_launch")
    ms_g = time_region(ctx, lambda: ok(lib.ceil_graph_launch(stream, ex), "ceil_graph_launch"), 20)
    ok(lib.ceil_graph_destroy(ex), "ceil_graph_destroy")

    # Reads the size of one decode weight matrix (W_o 4 MB, QKV 12.6 MB,
    # fc / W_proj 16.8 MB), replayed from a graph as the decode step is:
    # cold = every launch reads its own slice of 1 GiB (beyond the 256 MB
    # last-level cache), warm = every launch reads the same slice.
    big = GpuBuffer.zeros(ctx, (1 << 30) // 4)
    small_reads = {}
    for mib in (4, 8, 16):
        slice_b = mib << 20
        n = (1 << 30) // slice_b
        for cold in (1, 0):
            best_us, best_cfg = None, None
            for blocks, mode in ((cus, 1), (cus, 2), (2 * cus, 1), (2 * cus, 2)):
                ok(lib.ceil_graph_reads_create(stream, big.ptr, slice_b, n, blocks, mode, cold, sink.ptr,
                                               C.byref(ex)), "ceil_graph_reads_create")
                for _ in range(2):
                    ok(lib.ceil_graph_launch(stream, ex), "ceil_graph_launch")
                us = time_region(ctx, lambda: ok(lib.ceil_graph_launch(stream, ex), "ceil_graph_launch"), 5) \
                    * 1e3 / n
                ok(lib.ceil_graph_destroy(ex), "ceil_graph_destroy")
                if best_us is None or us < best_us:
                    best_us, best_cfg = us, f"{blocks // cus} blocks/CU, {'NT ' if mode == 2 else ''}8 loads"
            small_reads[f"{mib} MiB {'cold' if cold else 'warm'}"] = {
                "us": round(best_us, 2), "gbs": round(slice_b / (best_us * 1e-6) / 1e9, 1), "best": best_cfg}
    big.free()
    sink.free()
    out = {"mfma_fp32_tflops": round(mfma_tf, 1), "mfma_fp32_frac_of_peak": round(mfma_tf / PEAK_FP32_MFMA, 3),
           "mfma_fp32_32x32x2_tflops": round(mfma32_tf, 1),
           "hbm_read_gbs": round(read_gbs, 1), "hbm_read_frac_of_peak": round(read_gbs / PEAK_HBM, 3),
           "hbm_read_best": best, "hbm_read_all_gbs": {k: round(v, 1) for k, v in reads.items()},
           "graph_empty_kernel_us": round(ms_g * 1e3 / n_launch, 2),
           "graph_reads": small_reads,
           "probes": "register-operand fp32 MFMA (16x16x4, and 32x32x2), 2 GiB streaming read, "
                     "empty kernel in a HIP graph, 4-16 MiB reads replayed from a HIP graph (cold / warm)"}
    log(f"[bench] ceilings {out}")
    return out


PLANNER_TILES = ["256x128", "128x128", "128x64", "64x64", "64x32", "32x32"]
PLANNER_SPLITS = [1, 2, 4, 8, 16]


def planner_shapes(which: str) -> list[tuple[str, int, int, int]]:
    """(form, M, N, K) of the planner sweep: form nt (A@Bᵀ), nn (A@B) or acc
    (weight-gradient accumulate: M = d_out, N = d_in, K = t) — the config-1
    and config-3 GEMMs at M = 8192 / 16384 and at one GPU's 8-way
    data-parallel share, M = 1024 / 2048."""
    c3_nk = [(3072, 1024), (1024, 1024), (4096, 1024), (1024, 4096), (8192, 1024)]  # forward N, K
    c3_nn = [(1024, 3072), (1024, 1024), (1024, 4096), (4096, 1024), (1024, 8192)]  # dX N, K
    out = []
    for m in ([8192] if which in ("c1", "all") else []) + ([1024] if which in ("dp8", "all") else []):
        for k, n in SWEEP_KN:
            out += [("nn", m, n, k), ("nt", m, n, k)]
        out += [("nt", m, 8192, 512), ("acc", 2048, 512, m)]
    for m in ([16384] if which in ("c3", "all") else []) + ([2048] if which in ("dp8", "all") else []):
        out += [("nt", m, n, k) for n, k in c3_nk]
        out += [("nn", m, n, k) for n, k in c3_nn]
        out += [("acc", o, i, m) for o, i in c3_nk]
    return out


def bench_planner(ctx, steps: int, which: str) -> None:
    """The GEMM launch-plan sweep the planner constants in gemm.hip
    (choose_plan) are fitted to: every forced tile / split-K configuration
    (AUR_GEMM_CFG="BMxBN:splits", which the library reads on every call) of
    each shape, next to the planner's own pick.  One line per (form, shape)
    on stdout: "form MxNxK: auto=<TFLOP/s> cfg=<TFLOP/s> ..."; inputs are
    seeded U(-1,1) fp32 in HBM."""
    from aurora_amd.gpu import GpuBuffer

    rng = np.random.default_rng(0)
    shapes = planner_shapes(which)
    big = max(max(m * k, n * k, m * n) for _, m, n, k in shapes)
    a, b, c = (GpuBuffer.from_slice(ctx, rng.uniform(-1, 1, big).astype(np.float32)) for _ in range(3))

    def launch(form, m, n, k):
        if form == "acc":  # dest[m,n] += Σ_t d_y[t,m]·x[t,n]
            ctx.call("aur_outer_accum", a.ptr, b.ptr, c.ptr, m, n, k)
        else:
            ctx.call("aur_gemm_" + form, a.ptr, b.ptr, c.ptr, m, n, k)

    def tflops(cfg, form, m, n, k):
        if cfg is None:
            os.environ.pop("AUR_GEMM_CFG", None)
        else:
            os.environ["AUR_GEMM_CFG"] = cfg
        for _ in range(5):
            launch(form, m, n, k)
        ms = time_region(ctx, lambda: launch(form, m, n, k), steps)
        return 2.0 * m * n * k / (ms * 1e-3) / 1e12

    ramp_end = time.perf_counter() + CLOCK_RAMP_S
    while time.perf_counter() < ramp_end:
        for _ in range(10):
            launch("nt", 8192, 8192, 512)
        ctx.sync()
    for form, m, n, k in shapes:
        res = [f"auto={tflops(None, form, m, n, k):.1f}"]
        for t in PLANNER_TILES:
            if t == "256x128" and form == "acc":
                continue  # the 256-row tile needs A k-contiguous (planner: allow_wide)
            for sp in PLANNER_SPLITS:
                if sp > 1 and k // sp < 64:
                    break
                res.append(f"{t}:{sp}={tflops(f'{t}:{sp}', form, m, n, k):.1f}")
        print(f"{form} {m}x{n}x{k}: " + " ".join(res), flush=True)
    os.environ.pop("AUR_GEMM_CFG", None)
    for x in (a, b, c):
        x.free()


def bench_vendor(steps: int) -> None:
    """The vendor library on this bench's GEMM shapes, for comparison only
    (not part of the product path): torch.matmul (hipBLASLt) fp32 A@Bᵀ and
    A@B after the same clock ramp, timed with torch events over `steps`
    calls.  Runs in a process that never loads libaurora_hip.so: torch ships
    its own HIP runtime, and the two do not share one process on this image.
    This library's figures for the same shapes come from --only sweep /
    --only shapes."""
    import torch

    shapes = [(8192, 8192, 512), (8192, 1536, 512), (8192, 512, 512), (8192, 512, 2048),
              (16384, 3072, 1024), (16384, 1024, 4096), (16384, 4096, 1024),
              (1024, 1536, 512), (1024, 512, 512), (1024, 512, 2048), (2048, 1024, 1024)]
    dev = torch.device("cuda", 0)
    log(f"[bench] vendor: torch {torch.__version__} on {torch.cuda.get_device_name(0)}")
    for m, n, k in shapes:
        x = torch.rand(m, k, device=dev) - 0.5
        w = torch.rand(n, k, device=dev) - 0.5
        wt = w.t().contiguous()
        res = {}
        for form, fn in (("NT", lambda: x @ w.t()), ("NN", lambda: x @ wt)):
            end = time.perf_counter() + CLOCK_RAMP_S
            while time.perf_counter() < end:
                for _ in range(10):
                    fn()
                torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(steps):
                fn()
            e1.record()
            torch.cuda.synchronize()
            res[form] = 2.0 * m * n * k / (e0.elapsed_time(e1) / steps * 1e-3) / 1e12
        log(f"[bench] vendor {m}x{n}x{k}: NT {res['NT']:.1f} NN {res['NN']:.1f} TFLOP/s")
        del x, w, wt
    # the weight-gradient accumulate dest[d_out, d_in] += dYᵀ·X (both operands
    # k-strided: t runs down their rows) as torch.addmm on transposed views
    for d_out, d_in, t in ((2048, 512, 8192), (3072, 1024, 16384), (1024, 1024, 16384), (4096, 1024, 16384),
                           (1024, 4096, 16384), (8192, 1024, 16384)):
        dy = torch.rand(t, d_out, device=dev) - 0.5
        x = torch.rand(t, d_in, device=dev) - 0.5
        dest = torch.rand(d_out, d_in, device=dev) - 0.5
        fn = lambda: dest.addmm_(dy.t(), x)  # noqa: E731
        end = time.perf_counter() + CLOCK_RAMP_S
        while time.perf_counter() < end:
            for _ in range(10):
                fn()
            torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        tf = 2.0 * d_out * d_in * t / (e0.elapsed_time(e1) / steps * 1e-3) / 1e12
        log(f"[bench] vendor acc {d_out}x{d_in}_t{t}: {tf:.1f} TFLOP/s")
        del dy, x, dest


C3 = dict(vocab=8192, d_model=1024, n_layer=12, n_head=16, d_ff=4096, seq_len_max=1024)


def init_c3_model(ctx, max_batch, seed):
    """BASELINE config-3 model: every weight N(0,0.02), W_o and W_proj ×
    1/sqrt(2·12), LN γ = 1, β = 0 (random init, no checkpoint)."""
    from aurora_amd.model import DecoderTransformerGpu

    m = DecoderTransformerGpu(ctx, max_batch=max_batch, **C3)
    rng = np.random.default_rng(seed)
    n = m.tensor_ptr("params")[1]
    m.set("params", rng.standard_normal(n, dtype=np.float32) * np.float32(0.02))
    d, L = C3["d_model"], C3["n_layer"]
    res = np.float32(1.0 / np.sqrt(2.0 * L))
    for l in range(L):
        m.set("w_o", m.get("w_o", l) * res, l)
        m.set("w_proj", m.get("w_proj", l) * res, l)
        for k in ("ln1_g", "ln2_g"):
            m.set(k, np.ones(d, np.float32), l)
        for k in ("ln1_b", "ln2_b"):
            m.set(k, np.zeros(d, np.float32), l)
    m.set("lnf_g", np.ones(d, np.float32))
    m.set("lnf_b", np.zeros(d, np.float32))
    return m


def c3_step_flops(B=16, T=1024) -> float:
    """Algorithmic FLOP of one config-3 training step: 6·tokens·(linear + head
    params) for the GEMMs plus causal attention (4·dh per causal pair forward,
    10·dh backward) — 17.11 TFLOP at B16 T1024."""
    d, L, F, V, H = C3["d_model"], C3["n_layer"], C3["d_ff"], C3["vocab"], C3["n_head"]
    tokens = B * T
    lin = L * (4 * d * d + 2 * d * F) + V * d
    pairs = B * H * T * (T + 1) / 2
    return 6.0 * tokens * lin + L * 14.0 * (d // H) * pairs


def bench_train(ctx, steps: int, warmup: int) -> dict:
    """Config 3: one full training step (forward, CE, backward, clip 1.0,
    AdamW lr 3e-4 wd 0.1) on B16 × T1024 synthetic tokens, timed with events."""
    B, T = 16, 1024
    m = init_c3_model(ctx, B, seed=2)
    rng = np.random.default_rng(2)
    seq = rng.integers(0, C3["vocab"], (B, T + 1)).astype(np.uint32)
    tok, tgt = seq[:, :T].copy(), seq[:, 1:].copy()

    losses = []

    def step():
        m.zero_grad()
        losses.append(m.train_step_batch(tok, tgt) / B)
        m.clip_step_adamw(1.0, lr=3e-4, weight_decay=0.1)

    for _ in range(warmup):
        step()
    ms = time_region(ctx, step, steps)
    # The reference trainer's default optimizer on the same gradients: subset
    # clip 1.0 + Muon (NS5) on the GEMM weights, AdamW on embeddings and LN.
    def muon():
        m.clip_grads_adamw_subset(1.0)
        m.step_muon_hybrid(muon_lr=0.02, lr=3e-4, weight_decay=0.1)

    muon()
    muon_ms = time_region(ctx, muon, 3)
    m.destroy()
    tok_s = B * T / (ms * 1e-3)
    tf = c3_step_flops(B, T) / (ms * 1e-3) / 1e12
    log(f"[bench] train C3: {ms:.2f} ms/step {tok_s:.0f} tok/s {tf:.1f} TFLOP/s "
        f"loss {losses[0]:.4f} -> {losses[-1]:.4f}; Muon optimizer step {muon_ms:.2f} ms")
    return {"ms_per_step": round(ms, 3), "tok_per_s": round(tok_s, 1), "tflops": round(tf, 2),
            "pct_peak": round(100 * tf / PEAK_FP32_MFMA, 1), "loss_first": round(losses[0], 5),
            "loss_last": round(losses[-1], 5), "steps": steps,
            "muon_step_ms": round(muon_ms, 3),
            "config": "V8192 d1024 L12 H16 d_ff4096 T1024 B16 fp32, clip 1.0, AdamW lr 3e-4 wd 0.1 "
                      "(muon_step_ms: subset clip + Muon NS5 hybrid on the same gradients, not in ms_per_step)"}


def bench_decode(ctx, n_steps: int = 256) -> dict:
    """Config 4: prefill 32 prompts × 512 tokens, then n_steps greedy
    generate_step calls for all 32 sequences (KV ≤ 768), device-resident."""
    B, T0 = 32, 512
    max_len = T0 + n_steps
    m = init_c3_model(ctx, B, seed=2)
    rng = np.random.default_rng(4)
    prompts = rng.integers(0, C3["vocab"], (B, T0)).astype(np.uint32)
    cache = m.kv_cache(B, max_len)
    ramp_end = time.perf_counter() + CLOCK_RAMP_S
    while time.perf_counter() < ramp_end:  # clock ramp: untimed prefills (each resets the cache)
        m.prefill_kv(cache, prompts)
        ctx.sync()
    e0, e1 = ctx.event(), ctx.event()
    e0.record()
    m.prefill_kv(cache, prompts)
    e1.record()
    prefill_ms = e0.elapsed_ms(e1)
    # prefill_kv also captured the decode-step graph (its cost is in
    # prefill_ms); the timed region is the n_steps graph replays
    ctx.sync()
    e0.record()
    m.generate_greedy(cache, n_steps, collect=False)
    e1.record()
    ms = e0.elapsed_ms(e1)
    d, L, F, V = C3["d_model"], C3["n_layer"], C3["d_ff"], C3["vocab"]
    w_bytes = 4.0 * (L * (4 * d * d + 2 * d * F + 4 * d) + V * d + 2 * d + B * d)
    kv_read = sum(4.0 * 2 * L * B * (T0 + s + 1) * d for s in range(n_steps))
    kv_write = 4.0 * 2 * L * B * d * n_steps
    logits = 4.0 * B * V * n_steps
    total = w_bytes * n_steps + kv_read + kv_write + logits
    gbs = total / (ms * 1e-3) / 1e9
    tok_s = B * n_steps / (ms * 1e-3)
    cache.destroy()
    m.destroy()
    log(f"[bench] decode C4: prefill {prefill_ms:.2f} ms, {n_steps} steps {ms:.2f} ms "
        f"({ms / n_steps:.3f} ms/step) {tok_s:.0f} tok/s {gbs:.0f} GB/s")
    return {"prefill_ms": round(prefill_ms, 3), "ms_per_step": round(ms / n_steps, 4),
            "tok_per_s": round(tok_s, 1), "gb_per_s": round(gbs, 1),
            "pct_hbm": round(100 * gbs / PEAK_HBM, 1), "bytes_per_step": round(total / n_steps),
            "config": f"C3 model, {B} prompts x {T0} tokens prefill, {n_steps} greedy steps, KV<= {max_len}"}


def bench_attention(ctx, steps: int) -> dict:
    """Config 2: causal MHA forward + 3-pass backward, B16 H8 T1024 dh64."""
    from aurora_amd.gpu import CausalMhaBackwardKernel, CausalMhaForwardKernel, GpuBuffer

    B, T, H, dh = 16, 1024, 8, 64
    n = B * T * H * dh
    rng = np.random.default_rng(1)
    q, k, v, do = (GpuBuffer.from_slice(ctx, rng.standard_normal(n, dtype=np.float32)) for _ in range(4))
    o, lse = GpuBuffer.empty(ctx, n), GpuBuffer.empty(ctx, B * H * T)
    dq, dk, dv = (GpuBuffer.zeros(ctx, n) for _ in range(3))
    ws = GpuBuffer.empty(ctx, CausalMhaBackwardKernel.workspace_len(T, H, B))
    fwd, bwd = CausalMhaForwardKernel(), CausalMhaBackwardKernel()
    f = lambda: fwd.dispatch_into(ctx, q, k, v, o, lse, T, H, dh, b=B)
    g = lambda: bwd.dispatch_into(ctx, q, k, v, o, lse, do, dq, dk, dv, ws, T, H, dh, b=B)
    ramp_end = time.perf_counter() + CLOCK_RAMP_S
    while time.perf_counter() < ramp_end:  # clock ramp, as before the GEMM sweep
        f()
        g()
        ctx.sync()
    ms_f = time_region(ctx, f, steps)
    ms_b = time_region(ctx, g, steps)
    pairs = B * H * T * (T + 1) / 2
    tf_f = 4.0 * dh * pairs / (ms_f * 1e-3) / 1e12
    tf_b = 10.0 * dh * pairs / (ms_b * 1e-3) / 1e12
    for x in (q, k, v, do, o, lse, dq, dk, dv, ws):
        x.free()
    log(f"[bench] attention C2: fwd {ms_f:.3f} ms {tf_f:.1f} TFLOP/s, bwd {ms_b:.3f} ms {tf_b:.1f} TFLOP/s")
    return {"fwd_ms": round(ms_f, 4), "fwd_tflops": round(tf_f, 2), "bwd_ms": round(ms_b, 4),
            "bwd_tflops": round(tf_b, 2), "config": "B16 H8 T1024 dh64 causal fp32"}


CPU_SHARE = 16  # host cores that one GPU's jobs may use on this pool (its worker-pool bound)


def cpu_host() -> dict:
    """The host the CPU legs run on, and the threads they use: all cores of
    one GPU's CPU share (min(16, affinity)), one sequence per thread as the
    reference's rayon loops over a batch (examples/aurora_train.rs:828-838)."""
    aff = len(os.sched_getaffinity(0))
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "affinity": aff, "cpu_model": model, "threads": min(CPU_SHARE, aff),
            "note": f"threads = min({CPU_SHARE}, affinity): one GPU's CPU share on this pool is {CPU_SHARE} cores"}


def cpu_baseline(threads: int, budget_s: float = 10.0) -> dict:
    """The reference CPU path's GEMM: linear_forward (src/attention.rs:219-238)
    restated in oracle/, one 64-row "sequence" per task over `threads`
    threads as the reference's rayon loop does, on the sweep's QKV shape
    [rows,512]·[1536,512]ᵀ until `budget_s` of wall time is used; then the
    same GEMM on one thread for a fifth of the budget."""
    import oracle

    rng = np.random.default_rng(0)
    k, n, rows = 512, 1536, 1024
    x = rng.uniform(-1, 1, rows * k).astype(np.float32)
    w = rng.uniform(-1, 1, n * k).astype(np.float32)

    def rate(nthreads, budget):
        oracle.linear_forward_seqs(w, x, k, n, 64, nthreads)  # warm-up
        t0 = time.perf_counter()
        reps = 0
        while True:
            oracle.linear_forward_seqs(w, x, k, n, 64, nthreads)
            reps += 1
            el = time.perf_counter() - t0
            if el >= budget:
                return 2.0 * rows * k * n * reps / el / 1e12, reps, el

    tf, reps, el = rate(threads, budget_s)
    tf1, reps1, el1 = rate(1, budget_s / 5)
    return {"value": round(tf, 5), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"linear_forward [{rows},512]x[1536,512]^T (the sweep's QKV GEMM, "
                      f"1/8 of its rows) x{reps} in {el:.1f}s, 64-row sequences over {threads} threads",
            "gemm_1thread_tflops": round(tf1, 5),
            "gemm_1thread_sample": f"the same GEMM x{reps1} in {el1:.1f}s on one thread"}


def cpu_attention_sample(threads: int) -> dict:
    """Config 2 on the reference CPU path: scaled_dot_product_attention and
    its backward (src/attention.rs:396-550, restated in oracle/) for one
    (sequence, head) — T 1024, d_head 64, causal — one per thread on `threads`
    threads at once, timed; the 128 (b, h) pairs of config 2 take
    128 / threads such rounds."""
    import oracle
    from concurrent.futures import ThreadPoolExecutor

    T, dh = 1024, 64
    rng = np.random.default_rng(1)
    heads = [tuple(rng.standard_normal(T * dh, dtype=np.float32) for _ in range(4)) for _ in range(threads)]

    def one(h):
        q, k, v, do = h
        out, probs = oracle.sdpa_forward(q, k, v, dh, dh, causal=True)
        oracle.sdpa_backward(q, k, v, probs, do, dh, dh)

    one(heads[0])  # warm-up
    with ThreadPoolExecutor(max_workers=threads) as ex:
        t0 = time.perf_counter()
        list(ex.map(one, heads))
        el = time.perf_counter() - t0
    rounds = (16 * 8 + threads - 1) // threads
    return {"s_per_round": round(el, 3), "threads": threads, "c2_fwd_bwd_s_est": round(el * rounds, 2),
            "sample": f"oracle sdpa forward + backward, one (sequence, head) of T 1024 d_head 64 per thread, "
                      f"{threads} at once in {el:.2f}s; config 2 (B16 x H8 = 128 heads) = {rounds} such rounds"}


def cpu_decode_sample(threads: int, n_steps: int = 4) -> dict:
    """The reference CPU decode path (kv_cache.rs generate_step, restated in
    oracle/model.py) on the config-4 model: `threads` sequences decoded at
    once, one per thread (the reference runs sequences in parallel), each
    with its KV cache pre-filled to 640 positions (the average length of the
    256-step config-4 run), n_steps greedy steps each, timed."""
    from concurrent.futures import ThreadPoolExecutor

    from oracle import model as om

    cfg = om.Config(vocab=C3["vocab"], d_model=C3["d_model"], n_layer=C3["n_layer"], n_head=C3["n_head"],
                    d_ff=C3["d_ff"], seq_len_max=768 + 64)
    P = om.init_params(cfg, 2)
    rng = np.random.default_rng(5)
    t0 = 640
    caches = []
    for _ in range(threads):
        kv = om.KvCache(cfg)
        for l in range(cfg.n_layer):
            kv.k[l] = rng.standard_normal(t0 * cfg.d_model, dtype=np.float32)
            kv.v[l] = rng.standard_normal(t0 * cfg.d_model, dtype=np.float32)
        kv.current_len = t0
        caches.append(kv)

    def run(kv, steps):
        tok = 17
        for _ in range(steps):
            tok = om.argmax(om.generate_step(P, cfg, kv, tok))

    run(caches[0], 1)  # warm-up (one sequence one step longer)
    with ThreadPoolExecutor(max_workers=threads) as ex:
        ts = time.perf_counter()
        list(ex.map(lambda kv: run(kv, n_steps), caches))
        el = time.perf_counter() - ts
    tok_s = threads * n_steps / el
    return {"tok_per_s": round(tok_s, 1), "threads": threads, "s_per_step": round(el / n_steps, 4),
            "sample": f"oracle generate_step, config-4 model, {threads} sequences at once (one per thread) at KV "
                      f"length {t0}..{t0 + n_steps}, {n_steps} greedy steps each in {el:.2f}s"}


def cpu_train_step(threads: int, full: bool = True) -> dict:
    """The reference CPU training path on config 3 (model.rs forward, CE,
    backward; aurora_train.rs:812-848 batch loop; clip 1.0; AdamW): one whole
    step of 16 sequences × 1024 tokens, the sequences' gradients computed
    `threads` at a time (one per thread, as rayon par_iter over the batch),
    summed in sequence order and scaled by 1/16, then clip + AdamW — timed
    once, measured, no extrapolation.  full=False times one 32-token
    sequence instead (a quick sample for profiling runs)."""
    from oracle import model as om

    cfg = om.Config(vocab=C3["vocab"], d_model=C3["d_model"], n_layer=C3["n_layer"], n_head=C3["n_head"],
                    d_ff=C3["d_ff"], seq_len_max=C3["seq_len_max"])
    P = om.init_params(cfg, 2)
    B, T = (16, 1024) if full else (1, 32)
    seq = np.random.default_rng(2).integers(0, cfg.vocab, (B, T + 1)).astype(np.uint32)
    state = om.new_adam_state(P)
    t0 = time.perf_counter()
    loss, G = om.batch_grads(P, cfg, seq[:, :T], seq[:, 1:], threads=threads)
    t1 = time.perf_counter()
    om.clip_grads(G, 1.0)
    om.step_adamw(P, G, state, lr=3e-4, wd=0.1)
    t2 = time.perf_counter()
    out = {"s_fwd_bwd": round(t1 - t0, 2), "s_clip_adamw": round(t2 - t1, 2), "threads": threads,
           "loss": round(loss / B, 4)}
    if full:
        out["c3_step_s"] = round(t2 - t0, 2)
        out["sample"] = (f"oracle batch_grads over the full config-3 batch (16 x 1024 tokens, {threads} sequences "
                         f"at a time), then clip + AdamW: one measured step")
    else:
        out["sample"] = "oracle batch_grads + clip + AdamW on one 32-token sequence (not a config-3 step)"
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--only", choices=["head", "sweep", "train", "decode", "attention", "traffic", "shapes",
                                       "ceilings", "vendor", "planner"],
                    default=None,
                    help="profile helper: time only this part and skip the CPU baseline")
    ap.add_argument("--decode-steps", type=int, default=256)
    ap.add_argument("--planner-set", choices=["all", "c1", "c3", "dp8"], default="all",
                    help="shapes of --only planner")
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    ap.add_argument("--cpu-train", choices=["full", "sample"], default="full",
                    help="full: time a whole config-3 CPU step (about a minute on 16 cores); "
                         "sample: one 32-token sequence")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build measures ONE GPU only (every box has one GPU; "
              "sharding across GPUs is designed, not built)", file=sys.stderr)
        return 2

    if args.only == "vendor":  # before anything loads libaurora_hip.so
        bench_vendor(args.steps)
        return 0

    from aurora_amd.gpu import GpuContext

    ctx = GpuContext.new(0)
    name, cus = ctx.device_info()
    log(f"[bench] device {name}, {cus} CUs")
    rng = np.random.default_rng(1)
    items = build_sweep(ctx, rng)
    head = [it for it in items if it[0].startswith("head")][0]

    if args.only == "head":
        ramp_end = time.perf_counter() + CLOCK_RAMP_S
        while time.perf_counter() < ramp_end:  # clock ramp (see below)
            for _ in range(10):
                head[2]()
            ctx.sync()
        for _ in range(args.warmup):
            head[2]()
        ms = time_region(ctx, head[2], args.steps)
        log(f"[bench] head gemm {ms:.4f} ms  {head[1] / ms / 1e9:.1f} TFLOP/s")
        return 0
    if args.only == "traffic":
        # For `rocprofv3 --pmc FETCH_SIZE` / `WRITE_SIZE` passes: the head GEMM,
        # then a device copy of COPY_MIB as the counters' calibration (its
        # algorithmic bytes are known: COPY_MIB read + COPY_MIB written).
        from aurora_amd.gpu import GpuBuffer
        src = GpuBuffer.zeros(ctx, COPY_MIB << 18)
        dst = GpuBuffer.empty(ctx, COPY_MIB << 18)
        for _ in range(max(1, args.steps)):
            head[2]()
        for _ in range(max(1, args.steps)):
            ctx.call("aur_d2d", dst.ptr, src.ptr, COPY_MIB << 20)
        ctx.sync()
        log(f"[bench] traffic leg: {args.steps} head GEMMs, {args.steps} copies of {COPY_MIB} MiB")
        return 0
    if args.only == "train":
        bench_train(ctx, max(1, args.steps), args.warmup)
        return 0
    if args.only == "decode":
        bench_decode(ctx, args.decode_steps)
        return 0
    if args.only == "attention":
        bench_attention(ctx, args.steps)
        return 0
    if args.only == "shapes":
        bench_c3_and_shards(ctx, args.steps)
        return 0
    if args.only == "planner":
        bench_planner(ctx, args.steps, args.planner_set)
        return 0
    if args.only == "ceilings":
        bench_ceilings(ctx, cus)
        return 0

    def step():
        for _, _, fn in items:
            fn()

    # Clock ramp: the GPU leaves its idle clocks only after some ~100 ms of
    # sustained work (measured: 3 warm-up sweeps → 120.4 TFLOP/s, 100 → 125.7),
    # so the sweep first runs untimed for CLOCK_RAMP_S of wall time, then the
    # W warm-up steps, then the K timed steps.
    ramp_end = time.perf_counter() + CLOCK_RAMP_S
    while time.perf_counter() < ramp_end:
        for _ in range(10):
            step()
        ctx.sync()
    for _ in range(args.warmup):
        step()
    ctx.sync()
    t_wall = time.perf_counter()
    ms_step = time_region(ctx, step, args.steps)
    wall = time.perf_counter() - t_wall
    total_flops = sum(fl for _, fl, _ in items)
    value = total_flops / (ms_step * 1e-3) / 1e12
    log(f"[bench] sweep {ms_step:.3f} ms/step, {value:.1f} TFLOP/s (wall {wall:.2f}s)")

    per = []
    for nm, fl, fn in items:
        ms = time_region(ctx, fn, max(5, args.steps // 2))
        tf = fl / (ms * 1e-3) / 1e12
        per.append({"gemm": nm, "ms": round(ms, 4), "tflops": round(tf, 2),
                    "pct_peak": round(100 * tf / PEAK_FP32_MFMA, 1)})
        log(f"[bench]   {nm:32s} {ms:8.4f} ms {tf:7.1f} TFLOP/s {100 * tf / PEAK_FP32_MFMA:5.1f}%")
    head_ms = [p for p in per if p["gemm"].startswith("head")][0]["ms"]
    head_tf = head[1] / (head_ms * 1e-3) / 1e12

    if args.only == "sweep":
        return 0
    shapes = bench_c3_and_shards(ctx, max(5, args.steps // 2))
    attn = bench_attention(ctx, max(3, args.steps // 4))
    train = bench_train(ctx, max(2, min(args.steps, 5)), min(args.warmup, 2))
    decode = bench_decode(ctx, args.decode_steps)
    ceilings = bench_ceilings(ctx, cus)
    host = cpu_host()
    thr = host["threads"]
    cpu = cpu_baseline(thr, args.cpu_budget)
    cpu["host"] = host
    log(f"[bench] cpu gemm {cpu['value']} TFLOP/s on {thr} threads, {cpu['gemm_1thread_tflops']} on one")
    # The same leg also times the reference CPU attention (config 2), decode
    # (config 4) and training step (config 3).
    cpu["attention"] = cpu_attention_sample(thr)
    cpu["attention"]["gpu_speedup"] = round(
        cpu["attention"]["c2_fwd_bwd_s_est"] / ((attn["fwd_ms"] + attn["bwd_ms"]) * 1e-3), 1)
    log(f"[bench] cpu attention {cpu['attention']}")
    cpu["decode"] = cpu_decode_sample(thr)
    cpu["decode"]["gpu_speedup"] = round(decode["tok_per_s"] / cpu["decode"]["tok_per_s"], 1)
    log(f"[bench] cpu decode {cpu['decode']}")
    cpu["train"] = cpu_train_step(thr, full=args.cpu_train == "full")
    if "c3_step_s" in cpu["train"]:
        cpu["train"]["gpu_speedup"] = round(cpu["train"]["c3_step_s"] / (train["ms_per_step"] * 1e-3), 1)
    log(f"[bench] cpu train {cpu['train']}")

    line = {
        "metric": "fp32 GEMM TFLOP/s (% MFMA peak); train tok/s d1024 L12; decode tok/s + GB/s",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded U(-1,1) operands resident in HBM)",
        "config": {"workload": "BASELINE config 1: fp32 GEMM sweep, M=8192, NN+NT for "
                               "(K,N) in {(512,1536),(512,512),(512,2048),(2048,512)}, tied head "
                               "8192x8192x512 NT, weight-grad accumulate 2048x512 t=8192",
                   "parallelism": "single GPU"},
        "pct_peak": round(100 * value / PEAK_FP32_MFMA, 2),
        "sweep": per,
        "c3_gemms": shapes["c3_gemms"],
        "dp8_shard": shapes["dp8_shard"],
        "attention": attn,
        "train": train,
        "decode": decode,
        "ceilings": ceilings,
        "roofline": {"bound": "mfma", "kernel": "gemm_f32_mfma_direct<256,128> (tied head, NT 8192x8192x512)",
                     "achieved": round(head_tf, 3), "peak": PEAK_FP32_MFMA, "unit": "TFLOP/s",
                     "frac": round(head_tf / PEAK_FP32_MFMA, 4), "traffic": round(HEAD_TRAFFIC_BYTES),
                     "traffic_unit": "bytes per launch (rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-calibrated)",
                     "algorithmic_bytes": 4 * (2 * 8192 * 512 + 8192 * 8192)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    ctx.destroy()
    return 0


if __name__ == "__main__":
    sys.exit(main())
