#!/usr/bin/env python3
"""Benchmark of the dot_amd hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c3|c1|c4|c5]
                    [--method vanilla|momentum|anderson|adam] [--schedule linear|exponential|cosine]

One "step" is one pass of the hot path over one batch of synthetic input, as
the reference's users run it: ``result = dot.sinkhorn(C, reg, n_iters)``
followed by ``result.cost.sum().backward()``.  The default workload is config
C3 of BASELINE.json (B=64, M=N=512 fp32, squared Euclidean costs between
seeded 64-d Gaussian clouds normalised to max 1, uniform marginals, reg=0.1,
n_iters=200, tol=1e-6): the configuration the Sinkhorn headline metric is
quoted on.  Inputs are generated on the CPU from fixed seeds and are resident
in HBM before the timed region starts.

Printed: one JSON line.  ``value`` is Sinkhorn element-iterations per second,
E * (T_f + T_b) per step with E = B*M*N, T_f = forward iterations executed
and T_b = adjoint sweeps executed (averaged over the batch: the one-launch
tiers end each element's sweeps once converged, ``result.adjoint_sweeps``), so
it falls as the step gets shorter; ``ms_per_step`` is the step's wall time.
The steps do not read ``n_iters_used`` (a wait for the forward): every step
runs the same input, and the count is read once after the timed steps.
The same line carries

* ``roofline`` — the dominant kernel (the most time per step) against the
  roof it comes closer to, with its average launch duration measured with HIP
  events on the launch stream over a second pass of the same K steps run right
  after the timed ones (the events would otherwise add their own cost to
  ``value``).  Its algorithmic work per launch (KERNEL_WORK) is the
  irreducible traffic of its tier — inputs read and output written once (8
  bytes per element in the forward, 12 in the adjoint), plus 4 bytes per
  element-sweep for tiers that re-read the matrix every sweep (the
  register-resident tier keeps it in VGPRs) — and its arithmetic, 8 flops per
  element-iteration in the forward and 4 per element-sweep in the adjoint, over
  the sweeps it executed.  ``hbm`` and ``valu`` give both fractions (8 TB/s,
  157.3 TFLOP/s); ``bound`` names the larger;
* ``cpu_baseline`` — the reference's own CPU kernels (oracle/_ref, compiled
  from the reference sources) timed on a bounded sample of the same input,
  pinned to one host core with one torch thread, or the numpy oracle when
  oracle/_ref is absent;
* ``bidirectional_softmax`` — config C2 (B=32, 1024x1024, fwd+bwd) in GB/s of
  algorithmic traffic (20 bytes per element over the whole step), with the
  one-pass kernels' own traffic beside it, and ``two_sweep_shape``: the same
  element count at 128 x 512 x 512 (not a BASELINE configuration), where rows
  of at most 512 take the two-sweep kernels;
* ``other_configs`` — C1, C4 and C5 measured the same way (``--headline-only``
  skips them).

``--method`` / ``--schedule`` (with ``--omega``, ``--lr``, ``--anderson-k``,
``--reg-start``) time the accelerated solvers instead, on the same workload and
through the same public call; the line's ``config`` names the method the
reference's resolution rules select (sinkhorn.py:1362-1390).  Their backward
recomputes the plain forward at ``n_iters_used`` iterations, as the
reference's does; ``value`` still counts E * (T_f + T_b).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time

HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E, 8 TB/s
FP32_PEAK_TFLOPS = 157.3  # MI355X fp32 vector peak (packed dual-issue)
FP32_NONPACKED_TFLOPS = 78.6  # the same without packed fp32 instructions (this build disables them)
ROOT = os.path.dirname(os.path.abspath(__file__))

WORKLOADS = {
    "c1": dict(B=8, M=64, N=64, reg=1.0, n_iters=100, tol=1e-6, seed=0),
    "c3": dict(B=64, M=512, N=512, reg=0.1, n_iters=200, tol=1e-6, seed=3),
    "c4": dict(B=16, M=1024, N=2048, reg=0.05, n_iters=500, tol=1e-6, seed=4),
    "c5": dict(B=4, M=4096, N=4096, reg=0.02, n_iters=1000, tol=1e-6, seed=5),
    # not a BASELINE configuration: rows of 16384 columns, the strips x chunks
    # tiles of the streaming sweeps (``--workload wide``; never in other_configs)
    "wide": dict(B=4, M=1024, N=16384, reg=0.05, n_iters=100, tol=0.0, seed=6),
    # not BASELINE configurations: C3's shape, inputs and solver at larger
    # batches (``batch_scaling`` in the default line): B = 128 and 256 take the
    # persistent tier, B = 512 the per-iteration sweeps
    "c3b128": dict(B=128, M=512, N=512, reg=0.1, n_iters=200, tol=1e-6, seed=3),
    "c3b256": dict(B=256, M=512, N=512, reg=0.1, n_iters=200, tol=1e-6, seed=3),
    "c3b512": dict(B=512, M=512, N=512, reg=0.1, n_iters=200, tol=1e-6, seed=3),
}
BATCH_SCALING = ("c3b128", "c3b256", "c3b512")


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def make_inputs(name: str, torch, device):
    """Seeded inputs of BASELINE.md section 3; returns (C, a, b) with a, b None for uniform."""
    cfg = WORKLOADS[name]
    g = torch.Generator().manual_seed(cfg["seed"])
    B, M, N = cfg["B"], cfg["M"], cfg["N"]
    a = b = None
    if name in ("c1", "wide"):
        C = torch.rand(B, M, N, generator=g)
    elif name.startswith("c3"):
        x = torch.randn(B, M, 64, generator=g)
        y = torch.randn(B, N, 64, generator=g)
        C = torch.cdist(x.to(device), y.to(device)).square()
        C = C / C.amax(dim=(-2, -1), keepdim=True)
    elif name == "c4":
        C = torch.rand(B, M, N, generator=g)
        ea = -torch.log(torch.rand(B, M, generator=g))
        eb = -torch.log(torch.rand(B, N, generator=g))
        a = ea / ea.sum(-1, keepdim=True)
        b = eb / eb.sum(-1, keepdim=True)
    elif name == "c5":
        x = torch.randn(B, M, 128, generator=g)
        y = torch.randn(B, N, 128, generator=g)
        C = torch.cdist(x.to(device), y.to(device))
        C = C / C.amax(dim=(-2, -1), keepdim=True)
    else:
        raise ValueError(name)
    C = C.to(device=device, dtype=torch.float32).contiguous()
    if a is not None:
        a, b = a.to(device), b.to(device)
    return C, a, b


def kernel_stats(profiler, names):
    out = {}
    for n in names:
        launches, ms = profiler.query(n)
        if launches:
            out[n] = {"launches": launches, "total_ms": ms, "avg_us": 1000.0 * ms / launches}
    return out


# ---------------------------------------------------------------------------
# CPU baselines (bounded samples)
# ---------------------------------------------------------------------------
class one_core:
    """Pins this process to one host CPU and torch to one thread for the
    duration (the reference's CPU kernels are single-threaded); restores both."""

    def __enter__(self):
        import torch

        self.threads = torch.get_num_threads()
        self.mask = os.sched_getaffinity(0) if hasattr(os, "sched_getaffinity") else None
        self.core = min(self.mask) if self.mask else None
        if self.core is not None:
            os.sched_setaffinity(0, {self.core})
        torch.set_num_threads(1)
        return self

    def __exit__(self, *exc):
        import torch

        torch.set_num_threads(self.threads)
        if self.mask is not None:
            os.sched_setaffinity(0, self.mask)
        return False

    def label(self):
        return f"pinned to CPU {self.core}, 1 torch thread" if self.core is not None else "1 torch thread"


def sinkhorn_cpu_baseline(C_cpu, reg, a, b, target_s):
    """Reference CPU path, as torch_cpu.cpp runs it: forward T, then backward =
    recomputed forward T + adjoint T (here with tol 0 so the adjoint runs all T
    sweeps).  Timed on a growing number of batch elements until ~target_s."""
    import numpy as np

    sys.path.insert(0, ROOT)
    from oracle import ref

    kind = "reference" if ref.available() else "port"
    T = 20
    la = (-C_cpu).numpy()
    lga = None if a is None else np.log(a.cpu().numpy())
    lgb = None if b is None else np.log(b.cpu().numpy())
    Bt, M, N = la.shape

    def run(nb):
        sl = slice(0, nb)
        x = la[sl]
        A = None if lga is None else lga[sl]
        Bm = None if lgb is None else lgb[sl]
        t0 = time.perf_counter()
        if kind == "reference":
            P = ref.sinkhorn_forward(x, reg, T, A, Bm)
            P2 = ref.sinkhorn_forward(x, reg, T, A, Bm)
            ref.sinkhorn_backward_implicit(x, P2, -x, reg, T, 0.0)
        else:
            from oracle import sinkhorn as osk

            f = osk.dual_forward(x, reg, T, 0.0, A, Bm, dtype=np.float32)
            f2 = osk.dual_forward(x, reg, T, 0.0, A, Bm, dtype=np.float32)
            osk.implicit_backward(x, f2.P, -x, reg, T, None, dtype=np.float32)
        return time.perf_counter() - t0

    with one_core() as pin:
        t1 = run(1)
        nb = max(1, min(Bt, int(target_s / max(t1, 1e-6))))
        t = run(nb) if nb > 1 else t1
        reps = _repeats(t, target_s)
        if reps > 1:
            t = sum(run(nb) for _ in range(reps))
    elem_iters = reps * nb * M * N * (T + T)  # the metric counts forward + adjoint, not the recompute
    return {
        "value": elem_iters / t,
        "unit": "elem-iters/s",
        "cores": 1,
        "kind": kind,
        "sample": f"{nb} of {Bt} batch elements of this workload ({M}x{N}), {T} forward + "
                  f"{T} recomputed forward + {T} adjoint iterations"
                  + (f", {reps} times" if reps > 1 else "") + f", single-threaded, {pin.label()} "
                  f"({t:.1f} s on {_cpu_model()}, host has {os.cpu_count()} logical CPUs)",
    }


def _repeats(t, target_s):
    """Whole-sample repetitions that bring a sample shorter than half the target
    near it (small workloads finish the whole batch in milliseconds)."""
    if t >= 0.5 * target_s:
        return 1
    return int(min(10000, max(2, target_s / max(t, 1e-6))))


def bidi_cpu_baseline(sim_cpu, G_cpu, lengths_np, tau, target_s):
    import numpy as np

    sys.path.insert(0, ROOT)
    from oracle import ref

    kind = "reference" if ref.available() else "port"
    s = sim_cpu.numpy()
    g = G_cpu.numpy()
    B, L1, L2 = s.shape

    def run(nb):
        t0 = time.perf_counter()
        if kind == "reference":
            out, r, c = ref.bidirectional_softmax(s[:nb], tau, lengths_np[:nb])
            ref.bidirectional_softmax_backward(s[:nb], out, g[:nb], r, c, tau, lengths_np[:nb])
        else:
            from oracle import bidirectional_softmax as obs

            out, r, c = obs.forward(s[:nb], tau, lengths_np[:nb], dtype=np.float32)
            obs.backward(s[:nb], out, g[:nb], r, c, tau, lengths_np[:nb], dtype=np.float32)
        return time.perf_counter() - t0

    with one_core() as pin:
        t1 = run(1)
        nb = max(1, min(B, int(target_s / max(t1, 1e-6))))
        t = run(nb) if nb > 1 else t1
        reps = _repeats(t, target_s)
        if reps > 1:
            t = sum(run(nb) for _ in range(reps))
    return {
        "value": 20.0 * reps * nb * L1 * L2 / t / 1e9,
        "unit": "GB/s",
        "cores": 1,
        "kind": kind,
        "sample": f"{nb} of {B} batch elements ({L1}x{L2}) forward + backward"
                  + (f", {reps} times" if reps > 1 else "") + f", single-threaded, {pin.label()} "
                  f"({t:.1f} s on {_cpu_model()})",
    }


# ---------------------------------------------------------------------------
def profiled_pass(profiler, names, step, steps, torch):
    """Per-kernel durations for the roofline: the same ``steps`` steps run again
    right after the timed ones, with every launch of ``names`` bracketed by HIP
    events on its own stream.  The events are kept out of the timed steps: on
    the short bidirectional-softmax kernels they add ~25 us to a 200 us step."""
    profiler.reset()
    profiler.enable(True, kernels=names)
    torch.cuda.synchronize()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    profiler.enable(False)
    profiler.collect()
    return kernel_stats(profiler, names)


# Algorithmic work of each Sinkhorn kernel per matrix element: (HBM bytes once
# per launch, HBM bytes per sweep, flops per sweep, which count the sweeps are).
# Bytes are the irreducible traffic of the kernel's tier: the register-resident
# kernels read their inputs and write their output once (the matrix then stays
# in VGPRs: no bytes per sweep); the persistent and streaming kernels also
# re-read the matrix every sweep.  Forward: read C, write P (8); adjoint: read
# P and C, write the gradient (12).  Flops per sweep: the forward's row update
# and shared-exponential column sum (FMA, max, subtract, exp2, add, FMA, plus
# the column FMA: 8), the adjoint's row dot and column sum (two FMAs: 4).
KERNEL_WORK = {
    "sk_fwd_resident": (8.0, 0.0, 8.0, "T_f"),
    "sk_imp_resident": (12.0, 0.0, 4.0, "T_b"),
    "sk_fwd_persistent": (8.0, 4.0, 8.0, "T_f"),
    "sk_imp_persistent": (12.0, 4.0, 4.0, "T_b"),
    "sk_fwd_sweep": (0.0, 4.0, 8.0, "one"),
    "sk_imp_sweep": (0.0, 4.0, 4.0, "one"),
    "sk_unr_step": (0.0, 12.0, 0.0, "one"),
    "sk_unr_persistent": (12.0, 12.0, 0.0, "T_b"),
}


def sinkhorn_roofline(dominant, stats, E, T_f, T_b, workload):
    """Roofline object of the dominant Sinkhorn kernel (see the module docstring):
    its algorithmic bytes and flops per launch over its event-timed average
    duration, against the HBM and fp32 vector peaks; ``bound`` is the roof the
    kernel comes closer to."""
    once, per_sweep, flops_sweep, count = KERNEL_WORK.get(dominant, (0.0, 4.0, 0.0, "one"))
    sweeps = {"T_f": T_f, "T_b": T_b, "one": 1}[count]
    avg_s = stats[dominant]["avg_us"] * 1e-6
    bytes_launch = (once + per_sweep * sweeps) * E
    flops_launch = flops_sweep * sweeps * E
    hbm = bytes_launch / avg_s / 1e9
    valu = flops_launch / avg_s / 1e12
    traffic = _pmc_traffic(dominant, workload)
    measured = None if traffic is None else {
        "GBps": round(traffic / avg_s / 1e9, 1), "frac": round(traffic / avg_s / 1e9 / HBM_PEAK_GBPS, 4)}
    tier = ("register-resident (one launch, the matrix held in VGPRs for every sweep)" if "resident" in dominant
            else "persistent streaming (one launch; the matrix is re-read every sweep)" if "persistent" in dominant
            else "streaming sweeps (one launch per sweep)")
    common = {"kernel": dominant, "tier": tier, "sweeps_per_launch": sweeps, "avg_us": round(avg_s * 1e6, 2),
              "bytes_per_launch": bytes_launch, "bytes_per_elem": {"once": once, "per_sweep": per_sweep},
              "flops_per_launch": flops_launch, "flops_per_elem_sweep": flops_sweep,
              "hbm": {"achieved_GBps": round(hbm, 1), "frac": round(hbm / HBM_PEAK_GBPS, 4)},
              "valu": {"achieved_TFLOPs": round(valu, 2), "frac": round(valu / FP32_PEAK_TFLOPS, 4),
                       "frac_of_nonpacked_peak": round(valu / FP32_NONPACKED_TFLOPS, 4)},
              "traffic": traffic, "traffic_source": TRAFFIC_SOURCE, "hbm_measured": measured}
    if valu / FP32_PEAK_TFLOPS > hbm / HBM_PEAK_GBPS:
        return {"bound": "valu", "achieved": round(valu, 2), "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(valu / FP32_PEAK_TFLOPS, 4), **common}
    return {"bound": "hbm", "achieved": round(hbm, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(hbm / HBM_PEAK_GBPS, 4), **common}


SINKHORN_KERNELS = ["sk_fwd_sweep", "sk_imp_sweep", "sk_fwd_resident", "sk_imp_resident",
                    "sk_fwd_persistent", "sk_imp_persistent", "mth_sweep", "mth_vfinish",
                    "sk_fwd_wide_rows", "sk_fwd_wide_cols", "sk_imp_wide_rows", "sk_imp_wide_cols",
                    "sk_unr_step", "sk_unr_init", "sk_unr_fold", "sk_unr_resident", "sk_unr_persistent"]


def bench_sinkhorn(args, workload, steps, warmup, torch, dot_amd, profiler, solver=None):
    cfg = WORKLOADS[workload]
    dev = torch.device("cuda", 0)
    C, a, b = make_inputs(workload, torch, dev)
    B, M, N = C.shape
    E = B * M * N
    reg, n_iters, tol = cfg["reg"], cfg["n_iters"], cfg["tol"]
    solver = solver or {}

    last = {}

    def step():
        leaf = C.detach().requires_grad_(True)
        res = dot_amd.sinkhorn(leaf, reg=reg, n_iters=n_iters, tol=tol, a=a, b=b, **solver)
        res.cost.sum().backward()
        last["res"] = res

    from dot_amd.sinkhorn import _effective_method
    _, effective, eff_schedule, _ = _effective_method(
        solver.get("method", "vanilla"), solver.get("schedule"), solver.get("reg_start"),
        solver.get("omega"), reg, solver.get("lr", 1.0), 0.9, 0.999, 1e-8, True,
        "implicit", True, True, (M, N))

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    # Every step runs the same input, so every step executes the same
    # iterations: the count is read once, after the timed steps.  Reading it
    # inside a step (a device-to-host wait for that step's forward) would
    # time a loop that stalls the launch queue once per step.
    T_f = float(last["res"].n_iters_used)
    stats = profiled_pass(profiler, SINKHORN_KERNELS, step, steps, torch)

    # implicit: the sweeps each element's adjoint executed (at most backward_iters =
    # n_iters; the one-launch tiers end an element's sweeps once converged), averaged
    # over the batch (same input every step, same counts); unrolled: one reverse step
    # per recorded forward iteration
    sweeps = last["res"].adjoint_sweeps
    if solver.get("backward_mode") == "unrolled":
        T_b = T_f
    else:
        T_b = sum(sweeps) / len(sweeps) if sweeps else n_iters
    sec_per_step = (t1 - t0) / steps
    value = E * (T_f + T_b) / sec_per_step

    dominant = max(stats, key=lambda k: stats[k]["total_ms"]) if stats else None
    roofline = sinkhorn_roofline(dominant, stats, E, T_f, T_b, workload) if dominant else None
    algo_bytes = 4.0 * E * (T_f + T_b) + 20.0 * E
    return {
        "value": value,
        "unit": "elem-iters/s",
        "ms_per_step": 1000.0 * sec_per_step,
        "E": E,
        "T_f": T_f,
        "T_b": T_b,
        "config": {"workload": f"{workload}: sinkhorn fwd+bwd B={B} M={M} N={N} reg={reg} "
                               f"n_iters={n_iters} tol={tol}"
                               + ("" if effective == "vanilla" and eff_schedule is None else
                                  f" method={effective} schedule={eff_schedule}"),
                   "method": effective, "schedule": eff_schedule,
                   "B": B, "M": M, "N": N, "reg": reg, "n_iters": n_iters, "tol": tol,
                   "n_iters_used": int(T_f), "backward_iters": n_iters,
                   "adjoint_sweeps_executed": T_b,
                   "backward_mode": solver.get("backward_mode", "implicit")},
        "algorithmic_GBps": algo_bytes / sec_per_step / 1e9,
        "frac_of_hbm_peak": algo_bytes / sec_per_step / 1e9 / HBM_PEAK_GBPS,
        "frac_of_hbm_peak_note": ("algorithmic bytes (4 per element-iteration + 20 per element) over "
                                  "ms_per_step against 8 TB/s: HBM-equivalent, above 1 when the tier keeps "
                                  "the matrix on chip (register-resident); `roofline` gives the bound of "
                                  "the dominant kernel's tier"),
        "kernels": stats,
        "roofline": roofline,
        "C_cpu": C.cpu(), "a": a, "b": b, "reg": reg,
    }


# bytes per element each kernel moves itself: the two-sweep kernels, and the
# one-pass kernels that read each input once (full C2 tiles take those)
BIDI_KERNEL_BYTES = {"bidi_fwd_stats": 4.0, "bidi_fwd_write": 8.0, "bidi_bwd_dots": 8.0, "bidi_bwd_write": 12.0,
                     "bidi_fwd_onepass": 8.0, "bidi_bwd_onepass": 12.0}


def bench_bidi(args, torch, dot_amd, profiler):
    dev = torch.device("cuda", 0)
    B, L1, L2 = 32, 1024, 1024
    sim = torch.randn(B, L1, L2, generator=torch.Generator().manual_seed(1))
    G = torch.randn(B, L1, L2, generator=torch.Generator().manual_seed(2))
    sim_d, G_d = sim.to(dev), G.to(dev)
    lengths = torch.tensor([[L1, L2]] * B, dtype=torch.int32, device=dev)

    def step():
        # no lengths: every element is full (the reference's default)
        leaf = sim_d.detach().requires_grad_(True)
        P = dot_amd.bidirectional_softmax(leaf, 1.0)
        P.backward(G_d)

    for _ in range(args.warmup):
        step()
    names = sorted(BIDI_KERNEL_BYTES) + ["bidi_fwd_fused", "bidi_bwd_fused"]
    torch.cuda.synchronize()
    steps = max(args.steps, 10)
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    stats = profiled_pass(profiler, names, step, steps, torch)
    E = B * L1 * L2
    sec = (t1 - t0) / steps
    algo = 20.0 * E / sec / 1e9  # read sim, write P; read sim and grad, write grad: 20 B/elem per step
    # each sweep's own traffic (its reads and writes of [B,L1,L2] fp32 arrays) over its duration
    own = {}
    for k, st in stats.items():
        per_elem = BIDI_KERNEL_BYTES.get(k)
        if per_elem:
            bw = per_elem * E / (st["avg_us"] * 1e-6) / 1e9
            own[k] = {"bytes_per_launch": per_elem * E, "GBps": round(bw, 1),
                      "frac": round(bw / HBM_PEAK_GBPS, 4), "traffic": _pmc_traffic(k, "c2")}
    traffic = [v["traffic"] for v in own.values()]
    roofline = {"bound": "hbm", "kernel": "fwd+bwd step (" + ", ".join(sorted(stats)) + ")",
                "achieved": round(algo, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(algo / HBM_PEAK_GBPS, 4),
                "traffic": sum(traffic) if traffic and None not in traffic else None,
                "traffic_source": TRAFFIC_SOURCE,
                "bytes_per_step": 20.0 * E,
                "note": "20 B/elem algorithmic over ms_per_step; kernels_own_traffic gives each "
                        "sweep's own bytes over its event-timed duration"}
    return {
        "metric": "bidirectional softmax fwd+bwd algorithmic GB/s (20 B/elem)",
        "value": algo,
        "unit": "GB/s",
        "ms_per_step": 1000.0 * sec,
        "frac_of_hbm_peak": algo / HBM_PEAK_GBPS,
        "config": {"workload": "c2: bidirectional_softmax fwd+bwd B=32 L1=L2=1024 tau=1.0"},
        "kernels": stats,
        "kernels_own_traffic": own,
        "roofline": roofline,
        "two_sweep_shape": bench_bidi_two_sweep(args, torch, dot_amd, profiler),
        "_cpu": (sim, G, lengths.cpu().numpy()),
    }


def bench_bidi_two_sweep(args, torch, dot_amd, profiler):
    """C2's element count at 128 x 512 x 512 (not a BASELINE configuration):
    rows of at most 512 take the two-sweep kernels, which read sim twice in
    the forward and sim and grad_out twice in the backward (32 B/elem against
    the 20 of one pass; the metric counts 20)."""
    dev = torch.device("cuda", 0)
    B, L1, L2 = 128, 512, 512
    gen = torch.Generator(device=dev).manual_seed(7)
    sim = torch.randn(B, L1, L2, generator=gen, device=dev)
    G = torch.randn(B, L1, L2, generator=gen, device=dev)

    def step():
        leaf = sim.detach().requires_grad_(True)
        P = dot_amd.bidirectional_softmax(leaf, 1.0)
        P.backward(G)

    for _ in range(max(args.warmup, 2)):
        step()
    torch.cuda.synchronize()
    steps = max(args.steps, 10)
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    sec = (time.perf_counter() - t0) / steps
    stats = profiled_pass(profiler, sorted(BIDI_KERNEL_BYTES), step, steps, torch)
    E = B * L1 * L2
    own = {k: round(BIDI_KERNEL_BYTES[k] * E / (st["avg_us"] * 1e-6) / 1e9, 1) for k, st in stats.items()}
    return {"config": {"workload": f"bidirectional_softmax fwd+bwd B={B} L1=L2={L2} tau=1.0 (not a BASELINE config)"},
            "ms_per_step": 1000.0 * sec, "algorithmic_GBps": 20.0 * E / sec / 1e9,
            "frac_of_hbm_peak": 20.0 * E / sec / 1e9 / HBM_PEAK_GBPS,
            "kernels": stats, "kernels_own_GBps": own}


TRAFFIC_SOURCE = ("profiles/pmc_traffic.json: HBM bytes per dispatch from committed rocprofv3 --pmc "
                  "FETCH_SIZE and WRITE_SIZE runs, calibrated on a device copy; not measured in this run")


def _pmc_traffic(kernel, workload):
    """HBM bytes per dispatch from committed rocprofv3 --pmc summaries, if present."""
    path = os.path.join(ROOT, "profiles", "pmc_traffic.json")
    try:
        with open(path) as f:
            table = json.load(f)
        return table.get(workload, {}).get(kernel)
    except (OSError, ValueError):
        return None


def _public(d):
    return {k: v for k, v in d.items() if k not in ("C_cpu", "a", "b", "reg", "E")}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="c3", choices=sorted(WORKLOADS))
    ap.add_argument("--method", default="vanilla", choices=["vanilla", "momentum", "anderson", "adam"])
    ap.add_argument("--schedule", default=None, choices=["linear", "exponential", "cosine"])
    ap.add_argument("--omega", type=float, default=None)
    ap.add_argument("--lr", type=float, default=1.0)
    ap.add_argument("--anderson-k", type=int, default=5)
    ap.add_argument("--reg-start", type=float, default=None)
    ap.add_argument("--backward-mode", default="implicit", choices=["implicit", "unrolled"],
                    help="the backward the step runs (unrolled: the reverse pass through the "
                         "n_iters_used recorded iterations)")
    ap.add_argument("--no-bidi", action="store_true", help="skip the bidirectional-softmax leg")
    ap.add_argument("--headline-only", action="store_true",
                    help="skip the other Sinkhorn configurations (C1, C4, C5 besides the headline)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="approximate CPU time of each CPU-baseline sample (half of it for the "
                         "other configurations)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run 20 device copies of MIB MiB each (calibrates rocprofv3 "
                         "FETCH_SIZE / WRITE_SIZE against a known byte count) and exit")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported by this build "
              "(the batch shards across GPUs with no communication; see DESIGN.md)", file=sys.stderr)
        sys.exit(2)

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    if args.copy_probe:
        n = args.copy_probe * (1 << 20) // 4
        src = torch.rand(n, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(20):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes_read": 4 * n, "copy_probe_bytes_written": 4 * n,
                          "copies": 20}), flush=True)
        return

    sys.path.insert(0, ROOT)
    import dot_amd
    from dot_amd import profiler

    solver = dict(method=args.method, schedule=args.schedule, omega=args.omega, lr=args.lr,
                  anderson_k=args.anderson_k, reg_start=args.reg_start)
    if args.backward_mode != "implicit":
        solver["backward_mode"] = args.backward_mode
    sk = bench_sinkhorn(args, args.workload, args.steps, args.warmup, torch, dot_amd, profiler, solver)
    bidi = None if args.no_bidi else bench_bidi(args, torch, dot_amd, profiler)
    others = {}
    if (not args.headline_only and args.method == "vanilla" and args.schedule is None
            and args.backward_mode == "implicit"):
        for w in ("c1", "c3", "c4", "c5"):
            if w != args.workload:
                others[w] = bench_sinkhorn(args, w, args.steps, min(args.warmup, 2), torch, dot_amd, profiler)

    batch = {}
    if (not args.headline_only and args.workload == "c3" and args.method == "vanilla" and args.schedule is None
            and args.backward_mode == "implicit"):
        for w in BATCH_SCALING:
            r = bench_sinkhorn(args, w, args.steps, min(args.warmup, 2), torch, dot_amd, profiler)
            batch[w] = {"ms_per_step": r["ms_per_step"], "ratio_to_c3": r["ms_per_step"] / sk["ms_per_step"],
                        "T_f": r["T_f"], "T_b": r["T_b"], "value": r["value"], "unit": r["unit"],
                        "kernels": r["kernels"], "config": r["config"]}

    cpu = None
    if not args.no_cpu_baseline:
        cpu = sinkhorn_cpu_baseline(sk["C_cpu"], sk["reg"], sk["a"], sk["b"], args.cpu_seconds)
        if bidi is not None:
            sim, G, ln = bidi["_cpu"]
            bidi["cpu_baseline"] = bidi_cpu_baseline(sim, G, ln, 1.0, args.cpu_seconds)
            bidi["speedup_vs_cpu"] = bidi["value"] / bidi["cpu_baseline"]["value"]
        for w, o in others.items():
            o["cpu_baseline"] = sinkhorn_cpu_baseline(o["C_cpu"], o["reg"], o["a"], o["b"],
                                                      0.5 * args.cpu_seconds)
            o["speedup_vs_cpu"] = o["value"] / o["cpu_baseline"]["value"]
    profiler.shutdown()

    line = {
        "metric": "Sinkhorn fwd+bwd elem-iters/s and % HBM peak; bidir-softmax GB/s, 1 GPU",
        "value": sk["value"],
        "unit": "elem-iters/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": sk["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded inputs per BASELINE.md section 3)",
        "config": sk["config"],
        "n_iters_used": sk["T_f"],
        "backward_iters": sk["config"]["backward_iters"],
        "adjoint_sweeps_executed": sk["T_b"],
        "algorithmic_GBps": sk["algorithmic_GBps"],
        "frac_of_hbm_peak": sk["frac_of_hbm_peak"],
        "frac_of_hbm_peak_note": sk["frac_of_hbm_peak_note"],
        "roofline": sk["roofline"],
        "kernels": sk["kernels"],
        "cpu_baseline": cpu,
        "speedup_vs_cpu": (sk["value"] / cpu["value"]) if cpu else None,
    }
    if bidi is not None:
        bidi.pop("_cpu", None)
        line["bidirectional_softmax"] = bidi
    if others:
        line["other_configs"] = {w: _public(o) for w, o in others.items()}
    if batch:
        line["batch_scaling"] = {"note": "not BASELINE configurations: C3's shape, inputs and solver at B = 128, "
                                         "256, 512; ratio_to_c3 = ms_per_step over the headline's", **batch}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
