"""GEMM launch-plan sweep: every forced tile / split-K configuration of the
fp32 GEMM family, timed on the BASELINE shapes and on one GPU's share of them
under 8-way data parallelism, next to the planner's own pick.

    python -m aurora_amd.tune_gemm [--reps 20] [--set all|c1|c3|dp8]

Prints one line per (form, shape): "form MxNxK: auto=<TFLOP/s>[<pick>]
cfg=<TFLOP/s> ...", cfg being AUR_GEMM_CFG="BMxBN:splits" (the override the
library reads on every call).  The planner constants in gemm.hip
(choose_plan) are fitted to this table; the summary kept under profiles/
is its output.  Needs a GPU; inputs are seeded U(-1,1) fp32 in HBM.
"""
from __future__ import annotations

import argparse
import os
import sys

import numpy as np

TILES = ["256x128", "128x128", "128x64", "64x64", "64x32", "32x32"]
SPLITS = [1, 2, 4, 8, 16]

C1_KN = [(512, 1536), (512, 512), (512, 2048), (2048, 512)]
C3_NK = [(3072, 1024), (1024, 1024), (4096, 1024), (1024, 4096), (8192, 1024)]  # forward N, K
C3_NN = [(1024, 3072), (1024, 1024), (1024, 4096), (4096, 1024), (1024, 8192)]  # dX N, K
C3_ACC = [(3072, 1024), (1024, 1024), (4096, 1024), (1024, 4096), (8192, 1024)]  # d_out, d_in


def shape_set(which: str):
    """(form, M, N, K) with form nt (A@Bᵀ), nn (A@B) or acc (weight-gradient
    accumulate: M = d_out, N = d_in, K = t)."""
    out = []
    for m in ([8192] if which in ("c1", "all") else []) + ([1024] if which in ("dp8", "all") else []):
        for k, n in C1_KN:
            out += [("nn", m, n, k), ("nt", m, n, k)]
        out += [("nt", m, 8192, 512), ("acc", 2048, 512, m)]
    for m in ([16384] if which in ("c3", "all") else []) + ([2048] if which in ("dp8", "all") else []):
        out += [("nt", m, n, k) for n, k in C3_NK]
        out += [("nn", m, n, k) for n, k in C3_NN]
        out += [("acc", o, i, m) for o, i in C3_ACC]
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reps", type=int, default=20)
    ap.add_argument("--set", choices=["all", "c1", "c3", "dp8"], default="all")
    args = ap.parse_args()
    from aurora_amd.gpu import GpuBuffer, GpuContext

    ctx = GpuContext.new(0)
    rng = np.random.default_rng(0)
    shapes = shape_set(args.set)
    big = max(max(m * k, n * k, m * n) for _, m, n, k in shapes)
    a, b, c = (GpuBuffer.from_slice(ctx, rng.uniform(-1, 1, big).astype(np.float32)) for _ in range(3))
    e0, e1 = ctx.event(), ctx.event()

    def launch(form, m, n, k):
        if form == "acc":  # dest[m,n] += Σ_t d_y[t,m]·x[t,n]
            ctx.call("aur_outer_accum", a.ptr, b.ptr, c.ptr, m, n, k)
        else:
            ctx.call("aur_gemm_" + form, a.ptr, b.ptr, c.ptr, m, n, k)

    def time_cfg(cfg, form, m, n, k):
        if cfg is None:
            os.environ.pop("AUR_GEMM_CFG", None)
        else:
            os.environ["AUR_GEMM_CFG"] = cfg
        for _ in range(5):
            launch(form, m, n, k)
        ctx.sync()
        e0.record()
        for _ in range(args.reps):
            launch(form, m, n, k)
        e1.record()
        ms = e0.elapsed_ms(e1) / args.reps
        return 2.0 * m * n * k / (ms * 1e-3) / 1e12

    # clock ramp
    for _ in range(200):
        launch("nt", 8192, 8192, 512)
    ctx.sync()
    for form, m, n, k in shapes:
        res = [f"auto={time_cfg(None, form, m, n, k):.1f}"]
        for t in TILES:
            if t == "256x128" and form == "acc":
                continue  # the 256-row tile needs A k-contiguous (planner: allow_wide)
            for s in SPLITS:
                if s > 1 and k // s < 64:
                    break
                res.append(f"{t}:{s}={time_cfg(f'{t}:{s}', form, m, n, k):.1f}")
        print(f"{form} {m}x{n}x{k}: " + " ".join(res), flush=True)
    os.environ.pop("AUR_GEMM_CFG", None)
    ctx.destroy()
    return 0


if __name__ == "__main__":
    sys.exit(main())
