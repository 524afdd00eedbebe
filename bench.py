#!/usr/bin/env python3
"""Benchmark of the IFKFAC curvature hot path on one MI355X.

One step = one factor update plus one preconditioned weight update for a
single Linear layer, exactly the work IFKFAC.step does for that layer with
factor_update_freq=1 in bf16 mode:

  the damped bf16 factors of X (p x n_in) and delta (p x n_out), each side by
  the Gram matrix + blocked Cholesky (the panel TPQRT fold for a side it
  flags), the two sides concurrently, each side's triangular inverse (with
  its bf16 copies) right behind its factor                     (factor update)
  nat = (R_G^T R_G)^-1 grad (R_X^T R_X)^-1 from the inverses    (four solves)
  heavy-ball momentum + weight step                              (update)

Headline workload: Linear 4096 -> 11008 at p = 16384 rows, inputs resident in
HBM.  value = algorithmic TFLOP/s of the step, with the algorithmic count
2 p (n_in^2 + n_out^2) + 2 n_out n_in (n_in + n_out).

roofline: the dominant kernel of the workload -- the family with the largest
summed launch time in a survey step with every GEMM launch and every
block-Cholesky step bracketed by HIP events on its own stream -- timed by
such event pairs over as many steps again, run right after the timed steps
(which run with no events armed: an event pair per launch costs host time,
which a launch-bound chain would add to the step): algorithmic work per
launch over its average launch time, against the bf16 MFMA, fp32 MFMA or
HBM peak as its intensity says.

Extra keys on the same JSON line (unless --no-extras): the other benchmark
layers (Linear 1024 -> 1024 streamed over 8 chunks, 4096 -> 4096 at p = 8192,
11008 -> 4096 at p = 16384, one ViT-B block's capture folds), each with the
roofline of its own dominant kernel, IFKFAC.step() itself on a
Linear(4096, 11008) model and on the 4 x (Linear(4096, 4096) + GELU) stack,
the same step in fp32 arithmetic (the reference's regime), the same step with
its factors by the other two factor paths (CholeskyQR2 blocks, the panel
TPQRT fold), the step under the
default hardware-queue count (child process), kappa of the damped factors,
and a roofline per phase.  --workload measures one of the other layers as the
line's own workload (for its kernel-trace and counter runs).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
       [--no-extras] [--factor-path gram|cqr|panel]
Prints one JSON line.
"""
from __future__ import annotations

import argparse
import contextlib
import io
import json
import math
import os
import subprocess
import sys
import time

# HIP maps streams onto a pool of hardware queues (GPU_MAX_HW_QUEUES, 4 by
# default), and streams that share a queue run in submission order.  A layer's
# factor update runs each side on its own stream with two helper streams
# (Gram columns; panel work beside the Cholesky chain), so with 4 queues some
# of them share one.  HIP reads the variable when it initialises, so it is
# raised here, before torch touches the GPU (a larger setting is kept); with
# --hw-queues-default it is left alone (the drop-in user's default).
if "--hw-queues-default" not in sys.argv:
    try:
        _queues = int(os.environ.get("GPU_MAX_HW_QUEUES", "0"))
    except ValueError:
        _queues = 0
    if _queues < 8:
        os.environ["GPU_MAX_HW_QUEUES"] = "8"

METRIC = "ms per factor-update + precond step per layer; bf16 TFLOP/s vs MFMA peak"
PEAK_BF16_TFLOPS = 2500.0
PEAK_F32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0
# HBM bytes per launch of a workload's dominant kernel, from two rocprofv3
# --pmc runs (FETCH_SIZE, WRITE_SIZE) of that workload, scaled by the same
# counters on a 256 MiB copy (profiles/pmc_traffic_*.txt: fetch factor 2.0,
# write factor 1.0), averaged over the kernel's dispatches in the run, keyed
# by (workload, factor path, kernel); None where no counter run was made.
# (The dominant kernel of a run is the one with the largest summed launch time
# in its survey step; for these workloads that is either of two kernels.)
TRAFFIC = {
    ("linear_4096x11008_p16384", "gram", "gemm_bb_kernel<BbCfg<256, 256, 2, 4, 1, true>>"):
        861.65e6,
    ("linear_4096x11008_p16384", "gram", "cholb_step_kernel"): 5.14e6,
    ("vit_b_block_capture_p4096", "gram", "gemm_bb_kernel<BbCfg<256, 256, 2, 4, 1, true>>"):
        1068.91e6,
    ("vit_b_block_capture_p4096", "gram", "cholb_step_kernel"): 15.18e6,
}

WORKLOADS = {
    # name: (n_in, n_out, p, chunks) of a Linear layer's step, or ("vit",) for
    # one ViT-B block's capture folds
    "linear_4096x11008_p16384": (4096, 11008, 16384, 1),
    "linear_11008x4096_p16384": (11008, 4096, 16384, 1),
    "linear_4096x4096_p8192": (4096, 4096, 8192, 1),
    "linear_1024x1024_p4096": (1024, 1024, 4096, 1),
    "linear_1024x1024_p4096_8_chunks": (1024, 1024, 4096, 8),
    "vit_b_block_capture_p4096": ("vit",),
}


def algorithmic_flops(n_in: int, n_out: int, p: int) -> float:
    return 2.0 * p * (n_in ** 2 + n_out ** 2) + 2.0 * n_out * n_in * (n_in + n_out)


def update_flops(n_in: int, n_out: int, p: int) -> float:
    return 2.0 * p * (n_in ** 2 + n_out ** 2)


def precond_flops(n_in: int, n_out: int) -> float:
    return 2.0 * n_out * n_in * (n_in + n_out)


def kappa_matrix(p: int, n: int, kappa: float, seed: int, dtype):
    """p x n with singular values log-spaced from 1 to 1/kappa (Haar-like U, V by
    CholeskyQR of Gaussian matrices in fp64 on the GPU); setup only."""
    import torch
    g = torch.Generator(device="cuda").manual_seed(seed)
    k = min(p, n)

    def orth(m):
        G = torch.randn(m, k, device="cuda", dtype=torch.float64, generator=g)
        L = torch.linalg.cholesky(G.t() @ G)
        return torch.linalg.solve_triangular(L, G.t(), upper=False).t()

    U = orth(p)
    V = orth(n)
    s = torch.logspace(0, -math.log10(kappa), k, device="cuda", dtype=torch.float64)
    X = (U * s) @ V.t()
    del U, V
    return X.to(dtype).contiguous()


def cpu_info(threads: int) -> dict:
    import torch
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    cfg = torch.__config__.show()
    lapack = "unknown"
    for key in ("LAPACK is enabled", "BLAS_INFO", "LAPACK_INFO"):
        for line in cfg.splitlines():
            if key in line:
                lapack = line.strip()
                break
        if lapack != "unknown":
            break
    mkl = [l.strip() for l in cfg.splitlines() if "Math Kernel Library" in l or "MKL" in l[:12]]
    return {"cpu_model": model, "threads": threads,
            "lapack": (mkl[0] if mkl else lapack)[:120]}


def cpu_baseline(threads: int):
    """The reference's CPU call sequence (oracle/ref_recipe.py) timed on host cores:
    one step of the headline layer (a single rep: about half a minute of CPU work),
    and the median of three steps of Linear 4096 -> 4096 at p = 8192 after a warm-up."""
    import torch
    from oracle import ref_recipe
    torch.set_num_threads(threads)

    def one(n_in, n_out, p, seed):
        g = torch.Generator().manual_seed(seed)
        X = torch.randn(p, n_in, generator=g)
        D = torch.randn(p, n_out, generator=g)
        grad = torch.randn(n_out, n_in, generator=g) * 0.1
        W = torch.randn(n_out, n_in, generator=g) * 0.01
        t0 = time.perf_counter()
        ref_recipe.factor_update_precond_step([X], [D], grad, W, None, 1e-3, 0.9, 1e-2, True)
        return time.perf_counter() - t0

    n_in, n_out, p = WORKLOADS["linear_4096x11008_p16384"][:3]
    dt = one(n_in, n_out, p, 0)
    fl = algorithmic_flops(n_in, n_out, p)
    s_in, s_out, s_p = WORKLOADS["linear_4096x4096_p8192"][:3]
    one(s_in, s_out, s_p, 1)   # warm-up
    reps = sorted(one(s_in, s_out, s_p, 2 + i) for i in range(3))
    med = reps[1]
    out = {
        "value": round(fl / dt / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "ms_per_step": round(dt * 1e3, 1),
        "sample": (f"one factor-update + precondition step of Linear {n_in}->{n_out} at p={p} "
                   f"(bf16 factors) through the reference's torch-CPU call sequence (LAPACK "
                   f"qr/solve_triangular), a single rep, {threads} threads, torch "
                   f"{torch.__version__}"),
        "small_sample": {"workload": f"Linear {s_in}->{s_out} p={s_p}",
                         "ms_per_step_median_of_3": round(med * 1e3, 1),
                         "tflops": round(algorithmic_flops(s_in, s_out, s_p) / med / 1e12, 4)},
    }
    out.update(cpu_info(threads))
    return out


def default_queue_child(args) -> dict:
    """The headline step in a child process left at the default hardware-queue
    count (HIP reads it at start-up, so it takes a process of its own)."""
    env = dict(os.environ)
    env.pop("GPU_MAX_HW_QUEUES", None)
    cmd = [sys.executable, os.path.abspath(__file__), "--hw-queues-default", "--no-extras",
           "--no-cpu-baseline", "--steps", str(max(5, args.steps)), "--warmup",
           str(max(3, args.warmup)), "--factor-path", args.factor_path]
    try:
        r = subprocess.run(cmd, env=env, capture_output=True, text=True, timeout=600)
        line = [l for l in r.stdout.strip().splitlines() if l.startswith("{")][-1]
        d = json.loads(line)
        return {"ms_per_step": d["ms_per_step"], "value": d["value"],
                "GPU_MAX_HW_QUEUES": "default (unset)"}
    except Exception as e:   # reported, never fatal: the headline does not depend on it
        return {"error": f"{type(e).__name__}: {e}"[:200]}


# ----------------------------------------------------------------------------
# the per-layer chain
# ----------------------------------------------------------------------------
class LayerChain:
    """The backend calls of one IFKFAC step for one Linear layer (factor update
    with freq 1, bf16 factors), on resident synthetic inputs."""

    def __init__(self, be, n_in, n_out, p, factor_path="gram", math_=1, chunks=1,
                 kappa_x=1e2, kappa_d=1e1, lam=1e-2, seed=1):
        import torch
        self.be, self.n_in, self.n_out, self.p = be, n_in, n_out, p
        self.path, self.math, self.lam = factor_path, math_, lam
        self.X = kappa_matrix(p, n_in, kappa_x, seed, torch.bfloat16)
        self.D = kappa_matrix(p, n_out, kappa_d, seed + 1, torch.bfloat16)
        self.chunks = chunks
        gg = torch.Generator(device="cuda").manual_seed(seed + 2)
        self.grad = torch.randn(n_out, n_in, device="cuda", generator=gg) * 0.1
        self.W = torch.randn(n_out, n_in, device="cuda", generator=gg) * 0.01
        self.buf = torch.zeros_like(self.W)
        self.dev = torch.device("cuda", 0)
        self.factors = None
        if chunks > 1:
            self.RX = torch.zeros(n_in, n_in, device=self.dev)
            self.RG = torch.zeros(n_out, n_out, device=self.dev)

    def _chunk_folds(self, fq, accs):
        """As the hooks: the chunks of a streamed step but the last, both
        sides in arrival order (a batch's input chunk in the forward pass, its
        output-gradient chunk in the backward pass), small ones held until a
        fold of them pays, and in bf16 arithmetic each fold that pays held for
        one batched fold with the other side's (a factor's next fold first
        folds everything held), with no status read.  Returns each side's row
        count."""
        from ifkfac_amd._backend import MATH_BF16
        from ifkfac_amd.activation_hooks import FoldGroups, RowAccumulator
        q = self.p // self.chunks
        r = {"X": 0, "G": 0}
        groups = FoldGroups()
        grouping = self.math == MATH_BF16 and hasattr(self.be, "fold_gram_batched_")
        for c in range(self.chunks - 1):
            for side, T, R in (("X", self.X, self.RX), ("G", self.D, self.RG)):
                if side in groups:
                    groups.flush(self.math, fq)
                acc = accs.setdefault(side, RowAccumulator())
                chunk = T[c * q:(c + 1) * q]
                if grouping:
                    rows, private = acc.offer(r[side], R.shape[1], chunk)
                    if rows is not None:
                        groups.hold(side, R, r[side], rows, private)
                        r[side] = R.shape[1]
                else:
                    r[side] = acc.add(R, r[side], chunk, self.math, fq)
        groups.flush(self.math, fq)
        return r

    def _last_rows(self, T, acc):
        """The rows the factor update folds: the whole input, or with chunks the
        last chunk with the rows still held in front of it."""
        import torch
        if self.chunks == 1:
            return T
        last = T[(self.chunks - 1) * (self.p // self.chunks):]
        rows = acc.take() if acc is not None else None
        return last if rows is None else torch.cat([rows, last], dim=0)

    def _side(self, last, R, how, math_=None, r=0):
        import torch
        from ifkfac_amd._backend import MATH_BF16
        be, p = self.be, self.p
        am = self.math if math_ is None else math_
        out_dtype = torch.bfloat16
        # as IFKFAC's factor update: the Gram path in bf16 arithmetic (the
        # factor's inverse formed in the same call), CholeskyQR2 blocks in fp32
        # arithmetic
        gram = how == "gram" and am == MATH_BF16
        if gram:
            F, st, _, (Z, Zb, ZT) = be.fold_finalize_gram_batched(
                [R] if r > 0 else None, r, [last], 1 / math.sqrt(p), self.lam, out_dtype,
                with_inverse=True)
            return F[0], st, (Z[0], Zb[0], ZT[0])
        cqr = how == "cqr" or (how == "gram" and not gram)
        F, st = be.fold_finalize(R if r > 0 else None, r, last, 1 / math.sqrt(p), self.lam,
                                 out_dtype, am, cqr=cqr, gram=gram)
        return F, st, (be.tri_inverse_bf16(F) if am == MATH_BF16
                       else be.tri_inverse(F, 0))

    def factor_update(self):
        import torch
        from ifkfac_amd._backend import MATH_BF16, run_pair
        from ifkfac_amd.activation_hooks import FoldStatusQueue
        RX = getattr(self, "RX", None)
        RG = getattr(self, "RG", None)
        r = {"X": 0, "G": 0}
        accs = {}
        if self.chunks > 1:
            fq = FoldStatusQueue()
            r = self._chunk_folds(fq, accs)
            # the factor update reads the folds' statuses first (a refused
            # fold goes into its factor by the panel path)
            fq.drain()
        lx = self._last_rows(self.X, accs.get("X"))
        lg = self._last_rows(self.D, accs.get("G"))
        if (self.path == "gram" and self.math == MATH_BF16 and r["X"] == r["G"] and
                lx.shape == lg.shape and lx.dtype == lg.dtype and lx.stride() == lg.stride()):
            # as the hooks: a square layer's two sides in one batched call
            F, st, _, (Z, Zb, ZT) = self.be.fold_finalize_gram_batched(
                [RX, RG] if r["X"] > 0 else None, r["X"], [lx, lg], 1 / math.sqrt(self.p),
                self.lam, torch.bfloat16, with_inverse=True)
            out = [(F[i], st[i:i + 1], (Z[i], Zb[i], ZT[i])) for i in range(2)]
        else:
            out = list(run_pair(self.dev,
                                lambda: self._side(lx, RX, self.path, r=r["X"]),
                                lambda: self._side(lg, RG, self.path, r=r["G"]),
                                b_first=self.n_out > self.n_in))
        st = torch.cat([out[0][1], out[1][1]]).cpu()
        self.flagged = False
        for i, (last, R, side) in enumerate(((lx, RX, "X"), (lg, RG, "G"))):
            if int(st[i]) == 2:
                # as the hooks: a flagged side is refactored in fp32 arithmetic
                out[i] = self._side(last, R, "panel", math_=0, r=r[side])
                self.flagged = True
        self.factors = out
        return out

    def step(self, first, mark=lambda: None):
        import torch
        mark()
        (_, _, ix), (_, _, ig) = self.factor_update()
        mark()
        if self.math == 1 and not self.flagged:
            nat = self.be.precondition_apply_bf16(self.grad, ix[1:], ig[1:])
        else:
            # fp32 arithmetic, or a side refactored in fp32: the fp32 apply on
            # both sides' fp32 inverses
            zx, zg = (z if isinstance(z, torch.Tensor) else z[0] for z in (ix, ig))
            nat = self.be.precondition_apply(self.grad, zx, zg, 0)
        mark()
        self.be.momentum_update_(nat, self.buf, self.W, 1e-3, 0.9, 0.0, first)
        mark()


def timed(fn, steps, warmup):
    import torch
    for i in range(warmup):
        fn(i == 0)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn(False)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


# ----------------------------------------------------------------------------
# launch profiler: every GEMM launch and every block-Cholesky step of the
# library bracketed by HIP events on its own stream (ifk_profile_*)
# ----------------------------------------------------------------------------
# family -> (kernel name as rocprofv3 prints it, what it is, bound)
FAMILIES = {
    0: ("gemm_kernel", "128x128 MFMA GEMM engine", "mfma"),
    1: ("gemm_big_kernel", "256x128x32 bf16 MFMA GEMM, register staged", "mfma"),
    2: ("gemm_bb_kernel<BbCfg<256, 256, 2, 4, 1, true>>",
        "256x256x32 bf16 MFMA GEMM, direct-to-LDS ring (data-parallel or stream-K)", "mfma"),
    3: ("gemm_bb_kernel<BbCfg<128, 128, 2, 2, 2, false>>",
        "128x128x32 bf16 MFMA GEMM, direct-to-LDS ring (data-parallel or stream-K)", "mfma"),
    5: ("cholb_first_kernel", "first launch of the 1024-block Cholesky (fp32 MFMA)", "mfma_f32"),
    6: ("cholb_step_kernel",
        "one 64-column step of the 1024-block Cholesky with its inverse (fp32 MFMA)", "mfma_f32"),
}
ARM = {0: -4, 1: -3, 2: -5, 3: -6, 5: -7, 6: -8}
KVID = 1 << 12


def family(vid: int) -> int:
    if vid >= KVID:
        return 5 + (vid - KVID)
    if (vid >> 6) & 1:
        return 3 if (vid >> 7) & 1 else 2
    return (vid >> 5) & 1


def read_profile(lib, count: int) -> list:
    """(variant, ms, algorithmic flops, algorithmic bytes) of each recorded launch."""
    from ifkfac_amd import _lib
    C = _lib.ctypes
    v, ms, fl, by = C.c_int(0), C.c_float(0), C.c_double(0), C.c_double(0)
    m_, n_, k_ = C.c_int64(0), C.c_int64(0), C.c_int64(0)
    recs = []
    for i in range(count):
        _lib.check(lib.ifk_profile_get(i, *(C.byref(x) for x in (v, ms, fl, by, m_, n_, k_))),
                   "profile_get")
        recs.append((v.value, ms.value, fl.value, by.value))
    return recs


def profiled(lib, arm: int, fn) -> list:
    """Run fn with the launch profiler armed (arm as ifk_profile_begin takes it)."""
    import torch
    from ifkfac_amd import _lib
    torch.cuda.synchronize()
    _lib.check(lib.ifk_profile_begin(arm), "profile_begin")
    try:
        fn()
        torch.cuda.synchronize()
    finally:
        n = _lib.ctypes.c_int64(0)
        _lib.check(lib.ifk_profile_end(_lib.ctypes.byref(n)), "profile_end")
    return read_profile(lib, n.value)


def per_family(recs: list, steps: int) -> dict:
    out = {}
    for vid, ms, fl, by in recs:
        a = out.setdefault(family(vid), [0.0, 0, 0.0, 0.0])
        a[0] += ms / steps
        a[1] += 1.0 / steps
        a[2] += fl
        a[3] += by
    return out


def roofline(fam: int, recs: list, steps: int, ms_per_step: float, traffic_key=None) -> dict:
    """Roofline of one kernel family over the given launches: algorithmic work per
    launch over the launches' average event-measured duration."""
    name, desc, bound = FAMILIES[fam]
    tot_ms = sum(r[1] for r in recs)
    tot_fl = sum(r[2] for r in recs)
    tot_by = sum(r[3] for r in recs)
    n = max(len(recs), 1)
    if bound == "mfma_f32":
        peak, bf16_share = PEAK_F32_TFLOPS, 0.0
    else:
        bf16_share = sum(r[2] for r in recs if (r[0] >> 4) & 1) / max(tot_fl, 1.0)
        peak = PEAK_BF16_TFLOPS if bf16_share >= 0.5 else PEAK_F32_TFLOPS
    intensity = tot_fl / max(tot_by, 1.0)
    ridge = peak * 1e12 / (PEAK_HBM_GBS * 1e9)
    if intensity < ridge:
        ach = tot_by / (tot_ms * 1e-3) / 1e9
        r = {"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
             "frac": round(ach / PEAK_HBM_GBS, 4)}
    else:
        ach = tot_fl / (tot_ms * 1e-3) / 1e12
        r = {"bound": "mfma", "achieved": round(ach, 2), "peak": peak, "unit": "TFLOP/s",
             "frac": round(ach / peak, 4)}
    r.update({
        "traffic": TRAFFIC.get(traffic_key + (name,)) if traffic_key else None,
        "kernel": f"{name} ({desc})",
        "bf16_share_of_flops": round(bf16_share, 3),
        "launches_per_step": round(len(recs) / steps, 1),
        "avg_launch_ms": round(tot_ms / n, 4),
        "share_of_step": round(tot_ms / steps / ms_per_step, 3),
        "algorithmic_flops_per_launch": round(tot_fl / n),
        "algorithmic_bytes_per_launch": round(tot_by / n),
    })
    return r


def measure(lib, step, steps: int, warmup: int, traffic_key=None, marks=None):
    """warmup steps; one survey step with every family armed (the dominant
    family: the largest summed launch time per step, as a kernel-trace summary
    ranks kernels); then the timed steps, with nothing armed; then the same
    number of steps again with the dominant family armed, whose launches give
    the roofline (an event pair per launch costs host time, which a
    launch-bound chain would otherwise add to the timed steps).  Returns
    (ms_per_step, roofline of the dominant family, survey table, phases)."""
    import torch
    for i in range(warmup):
        step(i == 0)
    torch.cuda.synchronize()
    ev = []

    def mark():
        e = torch.cuda.Event(enable_timing=True)
        e.record()
        ev.append(e)
    survey = per_family(profiled(lib, -2, lambda: step(False, mark)), 1)
    phases = None
    if marks:
        torch.cuda.synchronize()
        phases = {marks[i]: round(ev[i].elapsed_time(ev[i + 1]), 3) for i in range(len(marks))}
    fam = max(survey, key=lambda f: survey[f][0])
    timing = {}

    def run():
        t0 = time.perf_counter()
        for _ in range(steps):
            step(False)
        torch.cuda.synchronize()
        timing["ms"] = (time.perf_counter() - t0) * 1e3 / steps
    run()
    ms = timing["ms"]
    recs = profiled(lib, ARM[fam], run)
    table = {FAMILIES[f][0]: {"ms_per_step": round(a[0], 3), "launches": round(a[1], 1),
                              "tflops": round(a[2] / (a[0] * 1e-3) / 1e12, 2) if a[0] else None}
             for f, a in sorted(survey.items(), key=lambda kv: -kv[1][0])}
    return ms, roofline(fam, recs, steps, ms, traffic_key), table, phases


class VitCapture:
    """One ViT-B block's factor capture per step: the folds of one 4096-row batch
    into the running factors of both sides of qkv 768->2304, proj 768->768,
    fc1 768->3072 and fc2 3072->768 (bf16 arithmetic, the Gram route with the
    panel fold for a refused fold, the statuses read without blocking), as the
    hooks issue them: held, then one batched fold per shape)."""

    shapes = [(768, 2304), (768, 768), (768, 3072), (3072, 768)]
    rows = 4096

    def __init__(self, be, seed=13):
        import torch
        from ifkfac_amd._backend import MATH_BF16
        from ifkfac_amd.activation_hooks import FoldStatusQueue
        g = torch.Generator(device="cuda").manual_seed(seed)
        self.be = be
        self.queue = FoldStatusQueue()
        self.Rs, self.chunks = [], []
        self.accs = None
        for (a, b) in self.shapes:
            for nn_ in (a, b):
                R = torch.zeros(nn_, nn_, device="cuda")
                T = torch.randn(self.rows, nn_, device="cuda", generator=g)
                be.fold_(R, 0, T, MATH_BF16)
                self.Rs.append(R)
                self.chunks.append(T)
        self.flops = sum(2.0 * self.rows * nn_ ** 2 for (a, b) in self.shapes for nn_ in (a, b))

    def step(self, first, mark=lambda: None):
        from ifkfac_amd._backend import MATH_BF16
        from ifkfac_amd.activation_hooks import FoldGroups, RowAccumulator
        mark()
        self.queue.poll()
        # as the hooks: each factor's chunk offered to its row accumulator
        # (a square factor folds two widths' worth of rows at a time, so the
        # 2304- and 3072-wide factors fold every other batch), each fold that
        # pays held, then one batched Gram-route fold per shape
        if self.accs is None:
            self.accs = [RowAccumulator() for _ in self.Rs]
        groups = FoldGroups()
        for i, (R, T) in enumerate(zip(self.Rs, self.chunks)):
            rows, private = self.accs[i].offer(R.shape[0], R.shape[1], T)
            if rows is not None:
                groups.hold(i, R, R.shape[0], rows, private)
        groups.flush(MATH_BF16, self.queue)
        mark()


def extras(be, args, head_kappa):
    """The other benchmark layers, each with the roofline of its dominant kernel,
    and IFKFAC.step() itself (see the module doc)."""
    import torch
    import torch.nn as nn
    from ifkfac_amd import IFKFAC
    from ifkfac_amd._backend import MATH_BF16
    lib = be.lib
    res = {}
    steps, warm = max(3, args.steps // 2), 2

    def layer(name, n_in, n_out, p, chunks=1, math_=1, path=None):
        path = path or args.factor_path
        c = LayerChain(be, n_in, n_out, p, path, math_=math_, chunks=chunks)
        ms, roof, table, _ = measure(lib, c.step, steps, warm, (name, path))
        del c
        torch.cuda.empty_cache()
        return {"ms_per_step": round(ms, 3),
                "tflops": round(algorithmic_flops(n_in, n_out, p) / ms / 1e9, 1),
                "roofline": roof, "kernels": table}

    res["layers"] = {
        "linear_1024x1024_p4096_8_chunks": layer("linear_1024x1024_p4096_8_chunks", 1024, 1024,
                                                 4096, chunks=8),
        "linear_4096x4096_p8192": layer("linear_4096x4096_p8192", 4096, 4096, 8192),
        "linear_11008x4096_p16384": layer("linear_11008x4096_p16384", 11008, 4096, 16384),
    }
    h_in, h_out, h_p = WORKLOADS["linear_4096x11008_p16384"][:3]
    res["fp32_arithmetic"] = dict(layer("fp32", h_in, h_out, h_p, math_=0), **{
        "note": "the headline step in fp32 arithmetic (CholeskyQR2 fp32 factor update, fp32 "
                "inverses and solves): the reference's regime"})

    # the headline step on the other factor paths: the north star's streaming
    # TSQR and Householder pieces, which the Gram route runs only as its
    # fallback
    res["other_factor_paths"] = {
        path: dict(layer(f"path_{path}", h_in, h_out, h_p, path=path), **{"note": note})
        for path, note in (
            ("cqr", "the headline step with each side factored by 1024-column CholeskyQR2 "
                    "blocks (bf16 arithmetic)"),
            ("panel", "the headline step with each side factored by the panel TPQRT fold "
                      "(blocked Householder, bf16 arithmetic)"))
        if path != args.factor_path}

    quiet = contextlib.redirect_stdout(io.StringIO())

    # IFKFAC.step() on a Linear(4096, 11008) model: forward and backward outside the timer
    def ifkfac_model(model, x, target, steps_, warm_):
        opt = IFKFAC(model, lr=1e-3, damping=1e-2, factor_update_freq=1, momentum=0.9,
                     use_true_bf16=True)
        times = []
        with quiet:
            for i in range(warm_ + steps_):
                model.zero_grad(set_to_none=True)
                loss = ((model(x) - target) ** 2).mean()
                loss.backward()
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                opt.step()
                torch.cuda.synchronize()
                if i >= warm_:
                    times.append((time.perf_counter() - t0) * 1e3)
        opt.cleanup() if hasattr(opt, "cleanup") else None
        return sorted(times)[len(times) // 2]

    torch.manual_seed(0)
    lin = nn.Linear(h_in, h_out, bias=False).cuda()
    x = kappa_matrix(h_p, h_in, 1e2, 11, torch.float32)
    tgt = torch.randn(h_p, h_out, device="cuda") * 0.1
    ms = ifkfac_model(lin, x, tgt, 3, 2)
    res["ifkfac_step_linear_4096x11008_p16384"] = {
        "ms_per_step_median": round(ms, 3),
        "note": "IFKFAC(use_true_bf16=True, factor_update_freq=1, momentum=0.9).step() with "
                "fp32 activations captured by the hooks; forward and backward untimed"}
    del lin, x, tgt
    torch.cuda.empty_cache()

    n, p = 4096, 8192
    layers = [nn.Linear(n, n) for _ in range(4)]
    mlp = nn.Sequential(*[m for l in layers for m in (l, nn.GELU())]).cuda()
    x = kappa_matrix(p, n, 1e2, 12, torch.float32)
    tgt = torch.randn(p, n, device="cuda") * 0.1
    ms = ifkfac_model(mlp, x, tgt, 3, 2)
    res["ifkfac_step_mlp_4x4096_gelu_p8192"] = {
        "ms_per_step_median": round(ms, 3),
        "tflops": round(4 * algorithmic_flops(n, n, p) / ms / 1e9, 1),
        "note": "4 x (Linear(4096, 4096) + GELU), one same-shape bucket, IFKFAC.step() "
                "end to end; forward and backward untimed"}
    del mlp, layers, x, tgt
    torch.cuda.empty_cache()

    # one ViT-B block's factor capture per batch, then get_factors() once
    cap = VitCapture(be)
    # an even number of batches: the 2304- and 3072-wide factors fold every
    # other batch
    ms_b, roof_b, table_b, _ = measure(lib, cap.step, 2 * ((steps + 1) // 2), warm,
                                       ("vit_b_block_capture_p4096", args.factor_path))
    rows = cap.rows

    def finalize_all(_first):
        # as get_factors() in bf16 arithmetic: every side by the Gram route,
        # grouped by width (grouped_gram_finalize), one host read of the
        # flags, the panel finalize for a side flagged 2
        from ifkfac_amd.activation_hooks import grouped_gram_finalize
        got = grouped_gram_finalize([(i, R, rows * 200) for i, R in enumerate(cap.Rs)], 1e-3,
                                    torch.float32)
        st = torch.cat([got[i][1] for i in range(len(cap.Rs))]).cpu()
        for i, R in enumerate(cap.Rs):
            if int(st[i]) == 2:
                be.finalize(R, 1 / math.sqrt(rows * 200), 1e-3, torch.float32, MATH_BF16)
    ms_f = timed(finalize_all, 3, 1)
    res["vit_b_block_capture_p4096"] = {
        "ms_per_batch": round(ms_b, 3), "tflops_per_batch": round(cap.flops / ms_b / 1e9, 1),
        "roofline": roof_b, "kernels": table_b,
        "ms_get_factors": round(ms_f, 3),
        "note": "one 4096-row batch per step into the 8 running factors (bf16 arithmetic, "
                "held as the hooks hold them -- a square factor folds two widths' worth of "
                "rows, so the 2304- and 3072-wide ones every other batch -- and folded by "
                "one batched Gram-route fold per shape, the panel fold for a refused fold), "
                "averaged over an even number of batches; 200 batches x 12 "
                "blocks take 2400 x ms_per_batch; get_factors() of the 8 sides by the Gram "
                "route, grouped by width"}
    del cap
    torch.cuda.empty_cache()
    res["kappa_R_damped_headline"] = head_kappa
    return res


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="linear_4096x11008_p16384", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--hw-queues-default", action="store_true",
                    help="leave GPU_MAX_HW_QUEUES at HIP's default (used by the child that "
                         "reports the step under the default)")
    ap.add_argument("--factor-path", default="gram", choices=["gram", "cqr", "panel"],
                    help="the consuming factor update: Gram matrix + blocked Cholesky, "
                         "CholeskyQR2 outer blocks, or the panel TPQRT fold (a side "
                         "flagged by the first two is recomputed by the panel path)")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="before the warmup, copy a device buffer of this many MiB three "
                         "times (a kernel of known HBM traffic for counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only (the curvature path is "
              "benchmarked on a single MI355X); run with --gpus 1", file=sys.stderr)
        return 2

    child = None
    if (not args.no_extras and not args.hw_queues_default and
            args.workload == "linear_4096x11008_p16384"):
        child = default_queue_child(args)   # before this process initialises HIP

    import torch
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from ifkfac_amd import _backend, _lib

    be = _backend.get_backend()
    lib = be.lib
    torch.cuda.set_device(0)

    if args.calib_copy_mib > 0:
        src = torch.ones(args.calib_copy_mib << 18, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    wl = WORKLOADS[args.workload]
    if wl[0] == "vit":
        runner = VitCapture(be)
        flops = runner.flops
        marks = ["folds"]
        desc = ("ViT-B block factor capture: the folds of one 4096-row batch into the running "
                "factors of qkv 768->2304, proj 768->768, fc1 768->3072, fc2 3072->768 (both "
                "sides, bf16 arithmetic)")
        cfg = {"rows_per_batch": VitCapture.rows, "sides": 8}
    else:
        n_in, n_out, p, chunks = wl
        runner = LayerChain(be, n_in, n_out, p, args.factor_path, chunks=chunks)
        flops = algorithmic_flops(n_in, n_out, p)
        marks = ["factor_update_and_inverse", "precondition", "update"]
        desc = (f"IFKFAC factor update + precondition, Linear {n_in}->{n_out}, p={p} rows"
                + (f" in {chunks} streamed chunks" if chunks > 1 else "")
                + ", bf16 factors (use_true_bf16), damping 1e-2, momentum 0.9")
        cfg = {"n_in": n_in, "n_out": n_out, "p": p, "chunks": chunks}

    ms_per_step, roof, table, phases = measure(lib, runner.step, args.steps, args.warmup,
                                               (args.workload, args.factor_path), marks)
    value = flops / (ms_per_step * 1e-3) / 1e12

    out_extra = {}
    if wl[0] != "vit":
        # a roofline per phase: algorithmic work over the phase's time in the
        # survey step (the whole GPU, all streams)
        ph_upd = phases["factor_update_and_inverse"]
        ph_pre = phases["precondition"]
        ph_mom = phases["update"]
        upd_fl = update_flops(n_in, n_out, p)
        pre_fl = precond_flops(n_in, n_out)
        mom_by = 20.0 * n_in * n_out   # read nat, read/write buf, read/write W (fp32)
        out_extra["phase_rooflines"] = {
            "factor_update_and_inverse": {
                "bound": "mfma", "achieved": round(upd_fl / ph_upd / 1e9, 1),
                "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(upd_fl / ph_upd / 1e9 / PEAK_BF16_TFLOPS, 4),
                "algorithmic": "2 p (n_in^2 + n_out^2)"},
            "precondition": {
                "bound": "mfma", "achieved": round(pre_fl / ph_pre / 1e9, 1),
                "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(pre_fl / ph_pre / 1e9 / PEAK_BF16_TFLOPS, 4),
                "algorithmic": "2 n_out n_in (n_in + n_out)"},
            "update": {
                "bound": "hbm", "achieved": round(mom_by / ph_mom / 1e6, 1),
                "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(mom_by / ph_mom / 1e6 / PEAK_HBM_GBS, 4),
                "algorithmic": "20 n_out n_in bytes"},
        }
        # kappa_2 of the damped factors of the timed step
        (FX, _, ix), (FG, _, ig) = runner.factors
        zx, zg = (z if isinstance(z, torch.Tensor) else z[0] for z in (ix, ig))
        kx = float(be.cond_estimate(FX, zx).item())
        kg = float(be.cond_estimate(FG, zg).item())
        out_extra["kappa_R_damped"] = {"R_X": round(kx, 4), "R_G": round(kg, 4)}
    head_kappa = out_extra.get("kappa_R_damped")

    cfg.update({"workload": desc,
                "factor_path": {
                    "gram": "Gram matrix + 1024-block Cholesky with split-bf16 updates (panel "
                            "path if flagged)",
                    "cqr": "1024-column blocks by CholeskyQR2 (panel path if flagged)",
                    "panel": "panel TPQRT fold"}[args.factor_path],
                "algorithmic_gflop_per_step": round(flops / 1e9, 1),
                "frac_of_bf16_peak": round(value / PEAK_BF16_TFLOPS, 4),
                "GPU_MAX_HW_QUEUES": os.environ.get("GPU_MAX_HW_QUEUES", "default (unset)")})
    out = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded; X kappa=1e2 and delta kappa=1e1 log-spaced singular values, "
                "grad ~ N(0, 0.01))",
        "config": cfg,
        "phases_ms": phases,
        "roofline": roof,
        "kernels": table,
    }
    out.update(out_extra)
    if child is not None:
        out["default_hw_queues"] = child
    if not args.no_extras and args.workload == "linear_4096x11008_p16384":
        del runner
        torch.cuda.empty_cache()
        out["extras"] = extras(be, args, head_kappa)
    if not args.no_cpu_baseline:
        # the cores this process may run on (a container's share, not the host's count)
        out["cpu_baseline"] = cpu_baseline(len(os.sched_getaffinity(0)) or 1)
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
