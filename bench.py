#!/usr/bin/env python3
"""Benchmark of the MI355X kernel surface at BASELINE.json's configurations.

The headline line measures configs[1] (the GPT-2-small memory-bound set), which fits one GPU:
one "step" is one pass of GELU fwd (bf16 [8,1024,3072]), sparse cross-entropy fwd and bwd
(fp32 [8192, 50257]), GELU bwd and one multi-tensor AdamW step over the 148 GPT-2-small
tensors (124,439,808 fp32 parameters), in that order so that no kernel finds its inputs in the
256 MB last-level cache from the previous one. `value` = algorithmic bytes of the step / step
time (GB/s, the reference's byte conventions, README.md:186-199).

`roofline` is for the step's dominant kernel (longest average duration, found in an untimed
pass with events around every kernel), timed live inside the timed steps with HIP events around
it alone, on the launch stream; its `mix_ceiling` is the rate hk_hbm_stream reaches with the same
read/write mix and byte count (AdamW: 4 arrays in, 3 out). `cpu_baseline` is the repository's
CPU oracle (a restatement of the reference harnesses' CPU references) timed on this host on a
bounded sample of the same step, on every core the host gives the process and on one thread.
`per_kernel` lists each kernel of the surface at its BASELINE config, timed alone: after 25
untimed repetitions, each of 100 repetitions flushes the caches and times one burst of
launches between one pair of events (memory-bound kernels: one launch per distinct buffer
set, ~1 GiB touched in all, so every launch reads HBM; compute-bound kernels: 5 launches of
the same operands); `achieved` comes from the median. Memory-bound entries carry the
fraction of their mix ceiling, and each entry of configs[0], [1], [2]/[3] and [4] the
oracle's time for the full config (`cpu`: one thread and all cores, sampled and scaled where
the sample says so). `ceilings` lists the hk_hbm_stream rates themselves.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
                       [--suite headline|all|kernels|compute|ceiling|copy] [--cases a,b]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np


def _args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--suite", choices=["headline", "all", "copy", "compute", "kernels",
                                        "ceiling"],
                    default="all",
                    help="copy: only the plain-copy kernel used to calibrate rocprofv3's "
                         "FETCH_SIZE / WRITE_SIZE counters (prints its byte count); compute: "
                         "only the MFMA kernels (GEMMs, attention) of the per-kernel suite, for "
                         "counter runs; kernels: only the per-kernel suite; ceiling: only the "
                         "HBM read/write-mix streams that bound the memory-bound kernels")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cases", default="",
                    help="with --suite compute or kernels: comma-separated names of the "
                         "per-kernel cases to run (default: all)")
    ap.add_argument("--reps", type=int, default=100,
                    help="timed repetitions per per-kernel timing (the median is reported)")
    ap.add_argument("--warmup-reps", type=int, default=25,
                    help="untimed repetitions before each per-kernel timing")
    return ap.parse_args()


ARGS = _args()
if ARGS.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
    print("bench.py: this build measures one GPU only (every kernel runs on one MI355X; "
          "sharding across GPUs is not built). Run with --gpus 1.", file=sys.stderr)
    sys.exit(2)

import torch  # noqa: E402

from hyperkernels_amd import kernels as hk  # noqa: E402
from hyperkernels_amd import workloads as W  # noqa: E402
from hyperkernels_amd.rocprof_summary import read_traffic  # noqa: E402

DEV = torch.device("cuda", 0)
torch.cuda.set_device(DEV)
hk.lib()  # fail loudly if the HIP library is missing


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


class Flusher:
    """Reads 512 MiB between repetitions so a timed kernel starts with a cold L2 and MALL.
    A read leaves the caches holding clean lines of an unrelated buffer; a write flush would
    leave them dirty, and the timed kernel would pay for their write-back (measured +30% on
    a 25 MB LayerNorm)."""

    def __init__(self):
        self.buf = torch.ones(512 << 18, dtype=torch.float32, device=DEV)

    def __call__(self):
        self.buf.sum()  # one reduction kernel over the fp32 buffer: reads only


def time_burst(fns, reps, flush, warmup=0):
    """Duration (ms) of one launch in a burst: each repetition flushes the caches, then
    launches every fn of `fns` back to back between one pair of events on the current stream
    and divides by len(fns). For memory-bound kernels `fns` run on distinct buffer sets (each
    set is read from HBM once per burst), for compute-bound ones they repeat one launch.
    One event pair per burst keeps the ~5 us event overhead out of short kernels (the host
    enqueues faster than these kernels run: the same bursts replayed from a HIP graph measured
    2-4% slower, not faster). `warmup` untimed repetitions come first; mean, median and
    minimum of the `reps` timed ones are returned (the reference reports the median of 100
    runs after 25 warm-ups with the L2 flushed, README.md:137-139)."""
    def body():
        for f in fns:
            f()
    for _ in range(max(1, warmup)):
        flush()
        body()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(reps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(reps)]
    for i in range(reps):
        flush()
        starts[i].record()
        body()
        ends[i].record()
    torch.cuda.synchronize()
    ts = sorted(s.elapsed_time(e) / len(fns) for s, e in zip(starts, ends))
    return {"avg_ms": sum(ts) / len(ts), "median_ms": ts[len(ts) // 2], "min_ms": ts[0]}


BURST_BYTES = 1 << 30  # a burst of memory-bound launches touches about this many distinct bytes
COMPUTE_BURST = 5      # launches per burst of a compute-bound kernel


def n_sets(footprint: int) -> int:
    """Buffer sets for a memory-bound burst: enough that a burst touches ~1 GiB, at most 32."""
    return max(1, min(32, -(-BURST_BYTES // max(footprint, 1))))


# ------------------------------------------------------------------------------------------------
# headline step: configs[1]
# ------------------------------------------------------------------------------------------------
def make_step():
    g = torch.Generator(device=DEV)
    g.manual_seed(1234)
    n = 8 * 1024 * 3072
    gx = torch.randn(n, generator=g, device=DEV).to(torch.bfloat16)
    gdy = torch.randn(n, generator=g, device=DEV).to(torch.bfloat16)
    gy = torch.empty_like(gx)
    gdx = torch.empty_like(gx)
    R, V = W.CE["rows"], W.CE["vocab"]
    logits = torch.randn(R, V, generator=g, device=DEV) * 2.0
    targets = torch.randint(0, V, (R,), generator=g, device=DEV, dtype=torch.int32)
    loss = torch.empty(R, device=DEV)
    mx = torch.empty(R, device=DEV)
    sm = torch.empty(R, device=DEV)
    grad = torch.empty_like(logits)
    gout = torch.ones(1, device=DEV)
    shapes = W.gpt2_param_shapes()
    P = [torch.randn(W.numel(s), generator=g, device=DEV) * 0.02 for s in shapes]
    G = [torch.randn(W.numel(s), generator=g, device=DEV) * 1e-2 for s in shapes]
    M = [torch.rand(W.numel(s), generator=g, device=DEV) * 0.1 for s in shapes]
    Vv = [torch.rand(W.numel(s), generator=g, device=DEV) * 0.1 for s in shapes]
    plan = hk.AdamPlan(P, G, M, Vv)
    c = W.ADAMW
    hyper = (c["lr"], c["beta1"], c["beta2"], c["eps"], c["weight_decay"], 1 - c["beta1"],
             1 - c["beta2"])
    ks = [
        ("gelu_fwd_bf16", lambda: hk.gelu_forward(gx, gy), W.gelu_fwd_bytes(n, 2)),
        ("ce_fwd", lambda: hk.sparse_ce_forward(logits, targets, loss, mx, sm), W.ce_fwd_bytes(R, V)),
        ("ce_bwd", lambda: hk.sparse_ce_backward(logits, targets, mx, sm, gout, 1.0, grad),
         W.ce_bwd_bytes(R, V)),
        ("gelu_bwd_bf16", lambda: hk.gelu_backward(gdy, gx, gdx), W.gelu_bwd_bytes(n, 2)),
        ("adamw_148", lambda: plan.step(*hyper), W.adamw_bytes(W.GPT2_NUM_PARAMS)),
    ]
    return ks, (plan, P, G, M, Vv)


def _event_pair():
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


def run_headline():
    """Returns (kernels, step bytes, ms per step, per-kernel ms, dominant kernel, its ms).

    A pass of ARGS.steps steps with HIP events around every kernel finds each kernel's time and
    the dominant one. The timed region is then ARGS.steps further steps with events around the
    dominant kernel only: an event pair around each of the five kernels adds about 38 us to a
    1.41 ms step on MI355X (the gaps it opens between kernels), which would be charged to the
    headline value."""
    ks, keep = make_step()
    step_bytes = sum(b for _, _, b in ks)
    names = [k for k, _, _ in ks]
    for _ in range(ARGS.warmup):
        for _, f, _ in ks:
            f()
    torch.cuda.synchronize()
    ev = [[_event_pair() for _ in ks] for _ in range(ARGS.steps)]
    for s in range(ARGS.steps):
        for (a, b), (_, f, _) in zip(ev[s], ks):
            a.record()
            f()
            b.record()
    torch.cuda.synchronize()
    per = {n: sum(ev[s][i][0].elapsed_time(ev[s][i][1]) for s in range(ARGS.steps)) / ARGS.steps
           for i, n in enumerate(names)}
    dom = max(per, key=per.get)
    di = names.index(dom)
    ev_dom = [_event_pair() for _ in range(ARGS.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(ARGS.steps):
        for i, (_, f, _) in enumerate(ks):
            if i == di:
                ev_dom[s][0].record()
                f()
                ev_dom[s][1].record()
            else:
                f()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_dom = sum(a.elapsed_time(b) for a, b in ev_dom) / ARGS.steps
    del keep
    return ks, step_bytes, wall / ARGS.steps * 1e3, per, dom, ms_dom


# ------------------------------------------------------------------------------------------------
# CPU baseline: the oracle on bounded samples, on one thread and on every core the host gives
# ------------------------------------------------------------------------------------------------
def cpu_threads():
    """(threads for the all-core leg, host facts). The all-core leg uses every core of this
    process's affinity mask, or OMP_NUM_THREADS when the host sets it (the GPU boxes set it to
    the process's CPU share, which can be fewer than the machine's cores)."""
    import oracle

    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    env = os.environ.get("OMP_NUM_THREADS")
    threads = int(env) if env and env.isdigit() and int(env) > 0 else affinity
    facts = {"hardware_concurrency": oracle.hardware_concurrency(), "affinity_cores": affinity,
             "omp_num_threads_env": env}
    return max(1, threads), facts


def _cpu_time(fn, min_s=0.2):
    """Mean seconds per call of fn: one untimed call, then calls until min_s has elapsed."""
    fn()
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        dt = time.perf_counter() - t0
        if dt >= min_s:
            return dt / n


def run_cpu_baseline():
    """configs[1] steps through the oracle: all cores on the full step, repeated until ~10 s of
    CPU work is timed; one thread on a quarter of the step (a quarter of the GELU elements, CE
    rows and AdamW parameters; every element is independent), scaled by 4.

    Inputs come from numpy's generator (untimed); the timed region is the five oracle calls,
    so the figure is directly comparable with the headline value. Returns the cpu_baseline
    object and each step kernel's CPU time (ms, full size)."""
    import oracle

    threads, facts = cpu_threads()
    rng = np.random.default_rng(7)
    n = 8 * 1024 * 3072
    x = oracle.f32_to_bf16(rng.standard_normal(n, dtype=np.float32))
    dy = oracle.f32_to_bf16(rng.standard_normal(n, dtype=np.float32))
    rows, V = W.CE["rows"], W.CE["vocab"]
    logits = rng.standard_normal((rows, V), dtype=np.float32)
    logits *= 2.0
    targets = rng.integers(0, V, rows, dtype=np.int32)
    P = W.GPT2_NUM_PARAMS
    p = rng.standard_normal(P, dtype=np.float32) * np.float32(0.02)
    g = rng.standard_normal(P, dtype=np.float32) * np.float32(1e-2)
    m = rng.random(P, dtype=np.float32) * np.float32(0.1)
    v = rng.random(P, dtype=np.float32) * np.float32(0.1)
    grad = np.zeros_like(logits)  # output pages touched before the timed region
    c = W.ADAMW
    names = ["gelu_fwd_bf16", "ce_fwd", "ce_bwd", "gelu_bwd_bf16", "adamw_148"]

    def step(frac):
        ne, nr, npar = n // frac, rows // frac, P // frac
        t = []
        t0 = time.perf_counter()
        oracle.gelu_forward(x[:ne])
        t.append(time.perf_counter())
        _, mx, sm = oracle.sparse_ce_forward(logits[:nr], targets[:nr])
        t.append(time.perf_counter())
        oracle.sparse_ce_backward(logits[:nr], targets[:nr], mx, sm, 1.0, out=grad[:nr])
        t.append(time.perf_counter())
        oracle.gelu_backward(dy[:ne], x[:ne])
        t.append(time.perf_counter())
        oracle.adamw_(p[:npar], g[:npar], m[:npar], v[:npar], c["lr"], c["beta1"], c["beta2"],
                      c["eps"], c["weight_decay"], 1 - c["beta1"], 1 - c["beta2"])
        t.append(time.perf_counter())
        return [b - a for a, b in zip([t0] + t[:-1], t)]

    oracle.set_threads(threads)
    reps, per = 0, [0.0] * 5
    while sum(per) < 10.0 and reps < 50:  # repeat the full step until ~10 s of CPU work is timed
        per = [a + b for a, b in zip(per, step(1))]
        reps += 1
    dt = sum(per)
    oracle.set_threads(1)
    per1 = [4 * t for t in step(4)]  # a quarter of the step, scaled to the full step
    oracle.set_threads(threads)
    del logits, grad
    nbytes = (W.gelu_fwd_bytes(n, 2) + W.gelu_bwd_bytes(n, 2) + W.ce_fwd_bytes(rows, V)
              + W.ce_bwd_bytes(rows, V) + W.adamw_bytes(P))
    base = {"value": round(reps * nbytes / dt / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": (f"{reps} full configs[1] steps (GELU fwd+bwd bf16 {n} elements, CE fwd+bwd "
                       f"{rows}x{V}, AdamW {P} params) through the oracle, the C++ restatement of "
                       f"the reference harnesses' CPU references; {dt:.2f} s on {threads} threads"),
            "value_1thread": round(nbytes / sum(per1) / 1e9, 3),
            "sample_1thread": ("a quarter of one configs[1] step (1/4 of the GELU elements, CE "
                               "rows and AdamW parameters) on 1 thread, scaled by 4: "
                               f"{sum(per1) / 4:.2f} s"),
            **facts}
    kernels = {k: {"ms_all_cores": round(a / reps * 1e3, 3), "ms_1thread": round(b * 1e3, 3),
                   "threads": threads, "sample": "configs[1] step (see cpu_baseline)"}
               for k, a, b in zip(names, per, per1)}
    return base, kernels


def run_cpu_configs():
    """The oracle at configs[0], [2]/[3] and [4] (and the reduce at the README shape), on one
    thread and on every core, each figure scaled to the full config (ms). Large configs are
    sampled: attention runs whole heads (1 on one thread, one per thread on all cores) and is
    scaled to the 96 heads of the config; the GEMMs and the reduce run whole output rows and are
    scaled to the config's rows. Every sampled unit is independent work of the same size."""
    import oracle

    threads, _ = cpu_threads()
    rng = np.random.default_rng(11)
    out = {}

    def both(name, make, full_units, units_per_thread, unit):
        """make(units) -> fn timing `units` units; scaled by full_units / units."""
        entry = {"threads": threads}
        for leg, th in (("ms_1thread", 1), ("ms_all_cores", threads)):
            oracle.set_threads(th)
            u = min(full_units, units_per_thread * th)
            entry[leg] = round(_cpu_time(make(u)) * full_units / u * 1e3, 3)
            entry["sample_" + leg[3:]] = (f"{u} of {full_units} {unit}"
                                          + (f", scaled by {full_units / u:g}" if u < full_units
                                             else ""))
        out[name] = entry
        log("cpu", name, entry)

    # LayerNorm fp32 4096 x 768, whole
    R, C = W.LN["rows"], W.LN["cols"]
    x = rng.standard_normal((R, C), dtype=np.float32)
    dyl = rng.standard_normal((R, C), dtype=np.float32)
    gam = (rng.random(C, dtype=np.float32) + np.float32(0.5))
    bet = rng.standard_normal(C, dtype=np.float32) * np.float32(0.1)
    _, mu, rs = oracle.layer_norm_forward(x, gam, bet, W.LN["eps"])
    both("ln_fwd", lambda u: lambda: oracle.layer_norm_forward(x[:u], gam, bet, W.LN["eps"]),
         R, R, "rows")
    both("ln_bwd_input", lambda u: lambda: oracle.ln_backward_input(dyl[:u], x[:u], mu[:u],
                                                                   rs[:u], gam), R, R, "rows")
    both("ln_bwd_gamma_beta", lambda u: lambda: oracle.ln_backward_gamma_beta(dyl[:u], x[:u],
                                                                           mu[:u], rs[:u]),
         R, R, "rows")
    fused = {}
    for leg in ("ms_1thread", "ms_all_cores"):  # the oracle has no fused form: the two summed
        fused[leg] = round(out["ln_bwd_input"][leg] + out["ln_bwd_gamma_beta"][leg], 3)
        fused["sample_" + leg[3:]] = "ln_bwd_input + ln_bwd_gamma_beta"
    out["ln_bwd_fused"] = {"threads": threads, **fused}
    # configs[2] / [3]: attention B=8 H=12 T=1024 d=64
    A = W.ATTN
    heads, T, D = A["B"] * A["H"], A["T"], A["d"]
    nh = min(heads, threads)
    q, k, v, do = (rng.standard_normal((1, nh, T, D), dtype=np.float32) for _ in range(4))
    scale = D ** -0.5
    for causal in (False, True):
        tag = "causal" if causal else "noncausal"
        o, lse = oracle.attn_forward(q, k, v, scale, causal)
        shape = f"{A['B']}x{A['H']}x{T}x{D}"
        both(f"attn_fwd_{tag}_{shape}", lambda u, causal=causal: lambda: oracle.attn_forward(
            q[:, :u], k[:, :u], v[:, :u], scale, causal), heads, 1, "(b, h) heads")
        both(f"attn_bwd_{tag}_{shape}", lambda u, causal=causal, o=o, lse=lse: lambda: oracle.attn_backward(
            q[:, :u], k[:, :u], v[:, :u], o[:, :u], do[:, :u], lse[:, :u], scale, causal),
            heads, 1, "(b, h) heads")
    # BF16 GEMM 8192 x 5120 x 1280 in four layouts, its dA / dB, SGEMM 4096^3 + bias
    G = W.BGEMM
    M, N, K = G["M"], G["N"], G["K"]
    bf = lambda *shape: oracle.f32_to_bf16(  # noqa: E731
        rng.standard_normal(shape, dtype=np.float32) * np.float32(0.05))
    rows_pt = 16
    a_mk, b_kn = bf(rows_pt * threads, K), bf(K, N)
    a_km, b_nk = np.ascontiguousarray(a_mk.T), np.ascontiguousarray(b_kn.T)
    for ta, tb in ((0, 0), (0, 1), (1, 0), (1, 1)):
        bb = b_nk if tb else b_kn
        name = f"bgemm_{'T' if ta else 'N'}{'T' if tb else 'N'}_8192x5120x1280"
        both(name, lambda u, ta=ta, tb=tb, bb=bb: lambda: oracle.bgemm(
            ta, tb, np.ascontiguousarray(a_km[:, :u]) if ta else a_mk[:u], bb), M, rows_pt,
            "output rows")
    # dA = dY W^T: [M, N] x [K, N]^T; dB = X^T dY: [M, K]^T x [M, N] (M rows of the product are K)
    dy_mn, w_kn = bf(rows_pt * threads, N), bf(K, N)
    both("bgemm_dA_NT_8192x1280x5120", lambda u: lambda: oracle.bgemm(0, 1, dy_mn[:u], w_kn), M,
         rows_pt, "output rows")
    x_mk, dy_full = bf(M, 4 * threads), bf(M, N)
    both("bgemm_dB_TN_1280x5120x8192", lambda u: lambda: oracle.bgemm(
        1, 0, np.ascontiguousarray(x_mk[:, :u]), dy_full), K, 4, "output rows")
    S = W.SGEMM
    sa = rng.standard_normal((4 * threads, S["K"]), dtype=np.float32)
    sb = rng.standard_normal((S["K"], S["N"]), dtype=np.float32)
    sbias = rng.standard_normal(S["N"], dtype=np.float32)
    # one CPU figure serves both GPU lines (the split is a GPU scheduling choice)
    both("sgemm_NN_4096^3_splitk4_bias", lambda u: lambda: oracle.sgemm(0, 0, sa[:u], sb,
                                                                       bias=sbias), S["M"], 4,
         "output rows")
    out["sgemm_NN_4096^3_auto_split_bias"] = out["sgemm_NN_4096^3_splitk4_bias"]
    # unified reduce, README shape 16384 x 50304 (inner axis)
    rsrc = rng.standard_normal((1024 * threads, 50304), dtype=np.float32)
    both("reduce_inner_16384x50304", lambda u: lambda: oracle.reduce_inner(rsrc[:u], u, 50304),
         16384, 1024, "output rows")
    oracle.set_threads(threads)
    return out


# ------------------------------------------------------------------------------------------------
# per-kernel suite
# ------------------------------------------------------------------------------------------------
def per_kernel_suite(flush, compute_only=False):
    out = {}
    g = torch.Generator(device=DEV)
    g.manual_seed(99)
    if compute_only:
        return time_cases(select(gemm_cases(g) + attention_cases(g)), flush, out)
    # LayerNorm configs[0], in fp32 and in bf16 / fp16 storage (fp32 statistics); gamma and
    # beta are shared by the buffer sets
    R, C = W.LN["rows"], W.LN["cols"]
    gamma = torch.rand(C, generator=g, device=DEV) + 0.5
    beta = torch.randn(C, generator=g, device=DEV) * 0.1
    cases = []
    for dt, tag, es in ((torch.float32, "", 4), (torch.bfloat16, "_bf16", 2),
                        (torch.float16, "_f16", 2)):
        g16, b16 = gamma.to(dt), beta.to(dt)
        dgam = torch.zeros(C, device=DEV)
        dbet = torch.zeros(C, device=DEV)
        fwd, bwd, bin_, bgb = [], [], [], []
        for _ in range(n_sets(W.ln_bwd_bytes(R, C, es))):
            x = torch.randn(R, C, generator=g, device=DEV).to(dt)
            dy = torch.randn(R, C, generator=g, device=DEV).to(dt)
            y, dx = torch.empty_like(x), torch.empty_like(x)
            mean = torch.empty(R, device=DEV)
            rstd = torch.empty(R, device=DEV)
            hk.layer_norm_forward(x, g16, b16, W.LN["eps"], y, mean, rstd)
            fwd.append(lambda x=x, y=y, mean=mean, rstd=rstd, g16=g16, b16=b16:
                       hk.layer_norm_forward(x, g16, b16, W.LN["eps"], y, mean, rstd))
            bwd.append(lambda dy=dy, x=x, mean=mean, rstd=rstd, dx=dx, g16=g16, dgam=dgam,
                       dbet=dbet: hk.layer_norm_backward(dy, x, mean, rstd, g16, dgam, dbet, dx))
            bin_.append(lambda dy=dy, x=x, mean=mean, rstd=rstd, dx=dx, g16=g16:
                        hk.ln_backward_input(dy, x, mean, rstd, g16, dx))
            bgb.append(lambda dy=dy, x=x, mean=mean, rstd=rstd, dgam=dgam, dbet=dbet:
                       hk.ln_backward_gamma_beta(dy, x, mean, rstd, dgam, dbet))
        cases += [(f"ln_fwd{tag}", fwd, W.ln_fwd_bytes(R, C, es), "hbm"),
                  (f"ln_bwd_fused{tag}", bwd, W.ln_bwd_bytes(R, C, es), "hbm")]
        if not tag:  # the two separate backward entry points, fp32
            cases += [("ln_bwd_input", bin_, W.ln_bwd_bytes(R, C, es), "hbm"),
                      ("ln_bwd_gamma_beta", bgb, W.ln_fwd_bytes(R, C, es), "hbm")]
    # GELU in fp16 at the configs[1] shape (the headline step runs the bf16 form)
    n = W.numel(W.GELU["shape"])
    gf, gb = [], []
    for _ in range(n_sets(W.gelu_bwd_bytes(n, 2))):
        gx = torch.randn(n, generator=g, device=DEV).half()
        gg = torch.randn(n, generator=g, device=DEV).half()
        gy, gi = torch.empty_like(gx), torch.empty_like(gx)
        gf.append(lambda gx=gx, gy=gy: hk.gelu_forward(gx, gy))
        gb.append(lambda gg=gg, gx=gx, gi=gi: hk.gelu_backward(gg, gx, gi))
    cases += [("gelu_fwd_f16", gf, W.gelu_fwd_bytes(n, 2), "hbm"),
              ("gelu_bwd_f16", gb, W.gelu_bwd_bytes(n, 2), "hbm")]
    # unified reduce at the README shape
    rs = torch.randn(16384, 50304, generator=g, device=DEV)
    lay = hk.ReductionLayout()
    lay.path, lay.num_outputs, lay.reduced_count = hk.REDUCE_INNER, 16384, 50304
    lay.input_outer_stride = 50304
    rdst = torch.empty(16384, device=DEV)
    cases.append(("reduce_inner_16384x50304", lambda: hk.unified_reduce_sum(rs, lay, rdst),
                  16384 * 50304 * 4, "hbm"))
    cases += step_alone_cases(g)
    cases += gemm_cases(g)
    cases += gemv_cases(g)
    cases += attention_cases(g)
    return time_cases(select(cases), flush, out)


def step_alone_cases(g):
    """The five configs[1] step kernels timed alone like every other memory-bound case (bursts
    over distinct buffer sets after a cache flush, median of the repetitions), beside their
    inside-the-step figures: an event pair around each launch inside the step adds a few us,
    which is a sizeable part of the ~17-25 us GELU kernels."""
    n = W.numel(W.GELU["shape"])
    gf, gb = [], []
    for _ in range(n_sets(W.gelu_bwd_bytes(n, 2))):
        gx = torch.randn(n, generator=g, device=DEV).to(torch.bfloat16)
        gg = torch.randn(n, generator=g, device=DEV).to(torch.bfloat16)
        gy, gi = torch.empty_like(gx), torch.empty_like(gx)
        gf.append(lambda gx=gx, gy=gy: hk.gelu_forward(gx, gy))
        gb.append(lambda gg=gg, gx=gx, gi=gi: hk.gelu_backward(gg, gx, gi))
    R, V = W.CE["rows"], W.CE["vocab"]
    logits = torch.randn(R, V, generator=g, device=DEV) * 2.0
    targets = torch.randint(0, V, (R,), generator=g, device=DEV, dtype=torch.int32)
    loss, mx, sm = (torch.empty(R, device=DEV) for _ in range(3))
    grad = torch.empty_like(logits)
    gout = torch.ones(1, device=DEV)
    hk.sparse_ce_forward(logits, targets, loss, mx, sm)
    shapes = W.gpt2_param_shapes()
    P = [torch.randn(W.numel(sh), generator=g, device=DEV) * 0.02 for sh in shapes]
    G = [torch.randn(W.numel(sh), generator=g, device=DEV) * 1e-2 for sh in shapes]
    M = [torch.rand(W.numel(sh), generator=g, device=DEV) * 0.1 for sh in shapes]
    Vv = [torch.rand(W.numel(sh), generator=g, device=DEV) * 0.1 for sh in shapes]
    plan = hk.AdamPlan(P, G, M, Vv)
    c = W.ADAMW
    hyper = (c["lr"], c["beta1"], c["beta2"], c["eps"], c["weight_decay"], 1 - c["beta1"],
             1 - c["beta2"])
    return [
        ("gelu_fwd_bf16_alone", gf, W.gelu_fwd_bytes(n, 2), "hbm"),
        ("ce_fwd_alone", [lambda: hk.sparse_ce_forward(logits, targets, loss, mx, sm)],
         W.ce_fwd_bytes(R, V), "hbm"),
        ("ce_bwd_alone", [lambda: hk.sparse_ce_backward(logits, targets, mx, sm, gout, 1.0, grad)],
         W.ce_bwd_bytes(R, V), "hbm"),
        ("gelu_bwd_bf16_alone", gb, W.gelu_bwd_bytes(n, 2), "hbm"),
        ("adamw_148_alone", [lambda: plan.step(*hyper)], W.adamw_bytes(W.GPT2_NUM_PARAMS), "hbm"),
    ]


def select(cases):
    """The cases --cases names (all when it is empty)."""
    if not ARGS.cases:
        return cases
    keep = set(ARGS.cases.split(","))
    unknown = keep - {c[0] for c in cases}
    if unknown:
        raise SystemExit(f"bench.py: unknown case(s) {sorted(unknown)}")
    return [c for c in cases if c[0] in keep]


def time_cases(cases, flush, out):
    """Times each (name, fn or [fns], work, bound) case; fills and returns `out`. `achieved` and
    `frac` come from the median burst (the reference's statistic); the mean is listed beside."""
    for name, fn, work, bound in cases:
        fns = fn if isinstance(fn, list) else [fn] * (1 if bound == "hbm" else COMPUTE_BURST)
        t = time_burst(fns, ARGS.reps, flush, ARGS.warmup_reps)
        ms = t["median_ms"]
        entry = {"median_ms": round(ms, 5), "avg_ms": round(t["avg_ms"], 5),
                 "reps": ARGS.reps, "warmup_reps": ARGS.warmup_reps}
        if bound == "hbm":
            ach = work / (ms * 1e-3) / 1e9
            entry.update({"achieved": round(ach, 1), "unit": "GB/s",
                          "frac": round(ach / W.PEAK_HBM_GBS, 4)})
        else:
            ach = work / (ms * 1e-3) / 1e12
            peak = W.PEAK_TFLOPS[bound]
            entry.update({"achieved": round(ach, 1), "unit": "TFLOP/s", "peak": peak,
                          "frac": round(ach / peak, 4)})
        out[name] = entry
        log(name, entry)
    return out


def attention_cases(g):
    """attention fwd and bwd, B=8 H=12 T=1024 d=64, fp32 I/O."""
    A = W.ATTN
    B, H, T, D = A["B"], A["H"], A["T"], A["d"]
    q, k, v, do = (torch.randn(B, H, T, D, generator=g, device=DEV) for _ in range(4))
    cases = []
    for causal in (True, False):
        o, lse = hk.fused_attn_forward(q, k, v, causal)
        Dt = hk.attn_bwd_precompute_D(do, o)
        dq, dk, dv = torch.zeros_like(q), torch.empty_like(k), torch.empty_like(v)
        tag = "causal" if causal else "noncausal"
        cases.append((f"attn_fwd_{tag}_8x12x1024x64",
                      lambda c=causal, o=o, lse=lse: hk.fused_attn_forward(q, k, v, c, o=o, lse=lse),
                      W.attn_fwd_flop(B, H, T, D, causal), "bf16x3"))
        mask = (torch.rand(B, H, T, T, generator=g, device=DEV) >= 0.1).float() / 0.9
        cases.append((f"attn_fwd_dropout_{tag}_8x12x1024x64",
                      lambda c=causal, o=o, lse=lse, mask=mask: hk.fused_attn_forward(
                          q, k, v, c, o=o, lse=lse, dropout_p=0.1, dropout_mask=mask),
                      W.attn_fwd_flop(B, H, T, D, causal), "bf16x3"))
        cases.append((f"attn_bwd_{tag}_8x12x1024x64",
                      lambda c=causal, lse=lse, Dt=Dt, dq=dq, dk=dk, dv=dv: hk.attn_backward(
                          q, k, v, do, lse, Dt, c, dq=dq, dk=dk, dv=dv),
                      W.attn_bwd_flop(B, H, T, D, causal), "bf16x3"))
    # the vendor path on the same tensors, for comparison (not part of the surface): torch's
    # scaled_dot_product_attention in fp32 on its memory-efficient backend (AOTriton)
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    def sdpa(c):
        with sdpa_kernel([SDPBackend.EFFICIENT_ATTENTION]):
            F.scaled_dot_product_attention(q, k, v, is_causal=c)
    for causal in (True, False):
        tag = "causal" if causal else "noncausal"
        cases.append((f"vendor_torch_sdpa_fp32_fwd_{tag}_8x12x1024x64",
                      lambda c=causal: sdpa(c), W.attn_fwd_flop(B, H, T, D, causal),
                      "fp32_matrix"))
    return cases


def gemv_cases(g):
    """BF16 GEMV (the M == 1 products) at GPT-2 decode shapes: logits = x wte^T (nt_row,
    [50257, 768] weight) and x W for a [4096, 16384] weight (nn_row). HBM-bound: the weight
    is read once (2 K N bytes)."""
    import ctypes

    lib = hk.lib()
    stream = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)  # noqa: E731
    one, zero = 0x3F80, 0
    cases = []
    V, C = 50257, 768
    nt = []
    for _ in range(n_sets(2 * V * C)):
        x = torch.randn(C, generator=g, device=DEV).to(torch.bfloat16)
        wte = (torch.randn(V, C, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
        logits = torch.empty(V, device=DEV, dtype=torch.bfloat16)

        def run_nt(x=x, wte=wte, logits=logits):
            assert lib.hk_bgemv_nt_row(V, C, one, x.data_ptr(), wte.data_ptr(), C, zero,
                                       logits.data_ptr(), 1, 0, 0, 0, stream()) == 0
        nt.append(run_nt)
    cases.append(("bgemv_nt_row_50257x768", nt, 2 * V * C + 2 * (V + C), "hbm"))
    K, N = 4096, 16384
    nn = []
    for _ in range(n_sets(2 * K * N)):
        xk = torch.randn(K, generator=g, device=DEV).to(torch.bfloat16)
        w = (torch.randn(K, N, generator=g, device=DEV) * K ** -0.5).to(torch.bfloat16)
        y = torch.empty(N, device=DEV, dtype=torch.bfloat16)

        def run_nn(xk=xk, w=w, y=y):
            assert lib.hk_bgemv_nn_row(N, K, one, xk.data_ptr(), w.data_ptr(), N, zero,
                                       y.data_ptr(), 1, 0, 0, 0, stream()) == 0
        nn.append(run_nn)
    cases.append(("bgemv_nn_row_4096x16384", nn, 2 * K * N + 2 * (K + N), "hbm"))
    return cases


def gemm_cases(g):
    """BF16 GEMM M=8192 K=1280 N=5120 in NN/NT/TN/TT plus dA (NT) and dB (TN)."""
    import ctypes

    lib = hk.lib()
    M, N, K = W.BGEMM["M"], W.BGEMM["N"], W.BGEMM["K"]
    one = 0x3F80  # bf16 1.0
    zero = 0
    stream = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)  # noqa: E731
    A_mk = (torch.randn(M, K, generator=g, device=DEV) * K ** -0.5).to(torch.bfloat16)
    A_km = A_mk.t().contiguous()
    B_kn = (torch.randn(K, N, generator=g, device=DEV) * K ** -0.5).to(torch.bfloat16)
    B_nk = B_kn.t().contiguous()
    C = torch.empty(M, N, device=DEV, dtype=torch.bfloat16)
    flop = W.gemm_flop(M, N, K)
    cases = []
    for ta, tb in ((0, 0), (0, 1), (1, 0), (1, 1)):
        a = A_km if ta else A_mk
        b = B_nk if tb else B_kn

        def run(ta=ta, tb=tb, a=a, b=b):
            st = lib.hk_bgemm(ta, tb, M, N, K, one, a.data_ptr(), a.shape[1], 0, b.data_ptr(),
                              b.shape[1], 0, zero, C.data_ptr(), N, 0, 1, stream())
            assert st == 0
        cases.append((f"bgemm_{'T' if ta else 'N'}{'T' if tb else 'N'}_8192x5120x1280", run, flop,
                      "bf16"))
    # backward of Y[M,N] = X[M,K] W[K,N]: dX = dY W^T (NT, [M,N]x[N,K]); dW = X^T dY (TN)
    dY = (torch.randn(M, N, generator=g, device=DEV) * N ** -0.5).to(torch.bfloat16)
    dX = torch.empty(M, K, device=DEV, dtype=torch.bfloat16)
    dW = torch.empty(K, N, device=DEV, dtype=torch.bfloat16)

    def run_da():
        assert lib.hk_bgemm_nt_backward(M, K, N, one, dY.data_ptr(), N, 0, B_kn.data_ptr(), N, 0,
                                        zero, dX.data_ptr(), K, 0, 1, stream()) == 0

    def run_db():
        assert lib.hk_bgemm_tn_backward(K, N, M, one, A_mk.data_ptr(), K, 0, dY.data_ptr(), N, 0,
                                        zero, dW.data_ptr(), N, 0, 1, stream()) == 0
    cases.append(("bgemm_dA_NT_8192x1280x5120", run_da, flop, "bf16"))
    cases.append(("bgemm_dB_TN_1280x5120x8192", run_db, flop, "bf16"))
    # FP32 SGEMM 4096^3, split-K 4, fused bias (added once), NN
    S = W.SGEMM
    sa = torch.randn(S["M"], S["K"], generator=g, device=DEV) * S["K"] ** -0.5
    sb = torch.randn(S["K"], S["N"], generator=g, device=DEV) * S["K"] ** -0.5
    sbias = torch.randn(S["N"], generator=g, device=DEV) * 0.02
    sc = torch.empty(S["M"], S["N"], device=DEV)

    def run_sgemm(split_k):
        assert lib.hk_sgemm(2, S["M"], S["N"], S["K"], 1.0, sa.data_ptr(), S["K"], 0,
                            sb.data_ptr(), S["N"], 0, 0.0, sc.data_ptr(), S["N"], 0,
                            sbias.data_ptr(), S["N"], 1, split_k, stream()) == 0
    # the config as stated (4 k splits summed by the finalize), and the library's own plan
    assert lib.hk_sgemm_split_count(2, S["M"], S["N"], S["K"], 1, S["split_k"]) == S["split_k"]
    cases.append(("sgemm_NN_4096^3_splitk4_bias", lambda: run_sgemm(S["split_k"]),
                  W.gemm_flop(S["M"], S["N"], S["K"]), "bf16x3"))
    cases.append(("sgemm_NN_4096^3_auto_split_bias", lambda: run_sgemm(0),
                  W.gemm_flop(S["M"], S["N"], S["K"]), "bf16x3"))
    # the vendor library on the same shapes, for comparison (not part of the surface):
    # torch.matmul -> hipBLASLt; bf16 NN / NT / TN and the fp32 GEMM + bias (fp32 MFMA)
    cases += [
        ("vendor_hipblaslt_bf16_NN_8192x5120x1280", lambda: torch.matmul(A_mk, B_kn, out=C),
         flop, "bf16"),
        ("vendor_hipblaslt_bf16_NT_8192x5120x1280",
         lambda: torch.matmul(A_mk, B_nk.t(), out=C), flop, "bf16"),
        ("vendor_hipblaslt_bf16_TN_8192x5120x1280",
         lambda: torch.matmul(A_km.t(), B_kn, out=C), flop, "bf16"),
        ("vendor_hipblaslt_bf16_dA_NT_8192x1280x5120",
         lambda: torch.matmul(dY, B_kn.t(), out=dX), flop, "bf16"),
        ("vendor_hipblaslt_bf16_dB_TN_1280x5120x8192",
         lambda: torch.matmul(A_mk.t(), dY, out=dW), flop, "bf16"),
        ("vendor_hipblaslt_fp32_NN_4096^3_bias", lambda: torch.addmm(sbias, sa, sb, out=sc),
         W.gemm_flop(S["M"], S["N"], S["K"]), "fp32_matrix"),
    ]
    return cases


COPY_BYTES = 1 << 30
TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                            "traffic_configs1_step.txt")


# ------------------------------------------------------------------------------------------------
# HBM read/write-mix ceilings
# ------------------------------------------------------------------------------------------------
# (name, fp32 elements per array, arrays read, arrays written): each memory-bound kernel of the
# surface at its own mix and byte count, plus 1 GiB-per-array read, write and copy streams.
CEILINGS = [
    ("ceiling_1r1w_ln_fp32", 4096 * 768, 1, 1),         # LayerNorm forward fp32, configs[0]
    ("ceiling_2r1w_ln_fp32", 4096 * 768, 2, 1),         # LayerNorm backward fp32
    ("ceiling_1r1w_ln_16bit", 4096 * 768 // 2, 1, 1),   # LayerNorm forward bf16 / fp16
    ("ceiling_2r1w_ln_16bit", 4096 * 768 // 2, 2, 1),   # LayerNorm backward bf16 / fp16
    ("ceiling_1r1w_gelu_16bit", 8 * 1024 * 3072 // 2, 1, 1),  # GELU forward, configs[1]
    ("ceiling_2r1w_gelu_16bit", 8 * 1024 * 3072 // 2, 2, 1),  # GELU backward
    ("ceiling_1r0w_ce", 8192 * 50257, 1, 0),            # CE forward reads the logits
    ("ceiling_1r1w_ce", 8192 * 50257, 1, 1),            # CE backward: logits in, grad out
    ("ceiling_4r3w_adamw", 124_439_808, 4, 3),          # AdamW: p, g, m, v in; p, m, v out
    ("ceiling_1r0w_1GiB", 1 << 28, 1, 0),
    ("ceiling_0r1w_1GiB", 1 << 28, 0, 1),
    ("ceiling_1r1w_1GiB", 1 << 28, 1, 1),
]
# memory-bound per-kernel case -> the ceiling of its mix and size
CEILING_OF = {
    "ln_fwd": "ceiling_1r1w_ln_fp32", "ln_bwd_fused": "ceiling_2r1w_ln_fp32",
    "ln_bwd_input": "ceiling_2r1w_ln_fp32",
    "ln_fwd_bf16": "ceiling_1r1w_ln_16bit", "ln_bwd_fused_bf16": "ceiling_2r1w_ln_16bit",
    "ln_fwd_f16": "ceiling_1r1w_ln_16bit", "ln_bwd_fused_f16": "ceiling_2r1w_ln_16bit",
    "gelu_fwd_bf16": "ceiling_1r1w_gelu_16bit", "gelu_bwd_bf16": "ceiling_2r1w_gelu_16bit",
    "gelu_fwd_f16": "ceiling_1r1w_gelu_16bit", "gelu_bwd_f16": "ceiling_2r1w_gelu_16bit",
    "ce_fwd": "ceiling_1r0w_ce", "ce_bwd": "ceiling_1r1w_ce", "adamw_148": "ceiling_4r3w_adamw",
    "gelu_fwd_bf16_alone": "ceiling_1r1w_gelu_16bit",
    "gelu_bwd_bf16_alone": "ceiling_2r1w_gelu_16bit",
    "ce_fwd_alone": "ceiling_1r0w_ce", "ce_bwd_alone": "ceiling_1r1w_ce",
    "adamw_148_alone": "ceiling_4r3w_adamw",
    "reduce_inner_16384x50304": "ceiling_1r0w_1GiB",
}


def ceiling_suite(flush, names=None):
    """Times hk_hbm_stream at each CEILINGS mix (the best of 1, 2 and 4 spans per workgroup),
    each burst over distinct buffer sets as for the memory-bound kernels."""
    import ctypes

    lib = hk.lib()
    out = {}
    for name, n, nin, nout in CEILINGS:
        if names is not None and name not in names:
            continue
        nbytes = 4 * n * (nin + nout)
        sets = []
        for _ in range(n_sets(nbytes)):
            ins = [torch.randn(n, device=DEV) for _ in range(nin)]
            outs = [torch.empty(n, device=DEV) for _ in range(nout)]
            sets.append((ins, outs))
        sink = torch.empty(-(-n // 1024), device=DEV)
        best = None
        for unroll in (1, 2, 4):
            fns = []
            for ins, outs in sets:
                pin = (ctypes.c_void_p * 4)(*[t.data_ptr() for t in ins])
                pout = (ctypes.c_void_p * 3)(*[t.data_ptr() for t in outs])

                def run(pin=pin, pout=pout, unroll=unroll):
                    st = lib.hk_hbm_stream(pin, nin, pout, nout, n, unroll, sink.data_ptr(),
                                           ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
                    assert st == 0
                fns.append(run)
            t = time_burst(fns, ARGS.reps, flush, ARGS.warmup_reps)
            if best is None or t["median_ms"] < best[1]["median_ms"]:
                best = (unroll, t)
        unroll, t = best
        ach = nbytes / (t["median_ms"] * 1e-3) / 1e9
        out[name] = {"median_ms": round(t["median_ms"], 5), "avg_ms": round(t["avg_ms"], 5),
                     "achieved": round(ach, 1), "unit": "GB/s",
                     "frac": round(ach / W.PEAK_HBM_GBS, 4), "bytes": nbytes,
                     "reads": nin, "writes": nout, "spans_per_workgroup": unroll}
        log(name, out[name])
        del sets, sink
    return out


def attach_ceilings(per_kernel, ceilings):
    """Adds the measured mix ceiling and the fraction of it to every memory-bound entry."""
    for k, c in CEILING_OF.items():
        if k in per_kernel and c in ceilings and per_kernel[k].get("unit") == "GB/s":
            per_kernel[k]["mix_ceiling"] = c
            per_kernel[k]["frac_of_mix_ceiling"] = round(
                per_kernel[k]["achieved"] / ceilings[c]["achieved"], 4)


def run_copy_calibration():
    """A plain copy of known size (1 GiB read, 1 GiB written) for counter calibration."""
    src = torch.randn(COPY_BYTES // 4, device=DEV)
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": COPY_BYTES, "dispatches": 3}), flush=True)


def main():
    log(f"device: {torch.cuda.get_device_name(0)}")
    if ARGS.suite == "copy":
        run_copy_calibration()
        return
    if ARGS.suite == "compute":
        print(json.dumps({"per_kernel": per_kernel_suite(Flusher(), compute_only=True)}),
              flush=True)
        return
    if ARGS.suite == "kernels":
        print(json.dumps({"per_kernel": per_kernel_suite(Flusher())}), flush=True)
        return
    if ARGS.suite == "ceiling":
        print(json.dumps({"ceilings": ceiling_suite(Flusher())}), flush=True)
        return
    ks, step_bytes, ms_step, per, dom, ms_dom = run_headline()
    value = step_bytes / (ms_step * 1e-3) / 1e9
    byte_of = {n: b for n, _, b in ks}
    # the dominant kernel's mean duration inside the timed region (HIP events on its stream)
    ach = byte_of[dom] / (ms_dom * 1e-3) / 1e9
    # HBM bytes per dispatch measured by rocprofv3 FETCH_SIZE + WRITE_SIZE (copy-calibrated)
    traffic = {k: int(v) for k, v in read_traffic(TRAFFIC_FILE).items()}
    for n in per:
        log(f"step kernel {n}: {per[n]:.4f} ms, {byte_of[n] / (per[n] * 1e-3) / 1e9:.1f} GB/s")
    result = {
        "metric": "TFLOP/s (attn, GEMM) & GB/s (LN/GELU/CE/Adam) vs MI355X roofline",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": ARGS.steps,
        "warmup": ARGS.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {"workload": "configs[1] GPT-2-small memory-bound set: GELU(tanh) fwd+bwd bf16 "
                               "[8,1024,3072]; sparse CE fwd+bwd fp32 [8192,50257] int32 targets; "
                               "multi-tensor AdamW 148 tensors / 124,439,808 fp32 params",
                   "step_bytes": step_bytes},
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": round(ach, 1),
                     "peak": W.PEAK_HBM_GBS, "unit": "GB/s", "frac": round(ach / W.PEAK_HBM_GBS, 4),
                     "traffic": traffic.get(dom), "algorithmic_bytes": byte_of[dom],
                     "avg_ms": round(ms_dom, 5)},
    }
    flush = Flusher()
    # the HBM rate the dominant kernel's read/write mix reaches at its size (hk_hbm_stream)
    ceilings = ceiling_suite(flush, None if ARGS.suite == "all" else {CEILING_OF[dom]})
    c = ceilings[CEILING_OF[dom]]
    result["roofline"]["mix_ceiling"] = {"stream": CEILING_OF[dom], "achieved": c["achieved"],
                                         "frac_of_mix_ceiling": round(ach / c["achieved"], 4)}
    if ARGS.suite == "all":
        result["per_kernel"] = {n: {"avg_ms": round(per[n], 5),
                                    "achieved": round(byte_of[n] / (per[n] * 1e-3) / 1e9, 1),
                                    "unit": "GB/s",
                                    "frac": round(byte_of[n] / (per[n] * 1e-3) / 1e9
                                                  / W.PEAK_HBM_GBS, 4),
                                    "timing": ("inside the step, mean of steps of a pass with "
                                               "events around every kernel")}
                                for n in per}
        result["per_kernel"].update(per_kernel_suite(flush))
        attach_ceilings(result["per_kernel"], ceilings)
        result["ceilings"] = ceilings
    if not ARGS.no_cpu:
        result["cpu_baseline"], cpu_kernels = run_cpu_baseline()
        if ARGS.suite == "all":
            cpu_kernels.update(run_cpu_configs())
            for k, e in cpu_kernels.items():
                for name in (k, k + "_alone"):
                    if name in result["per_kernel"]:
                        result["per_kernel"][name]["cpu"] = e
    print(json.dumps(result), flush=True)
    print_summary(result)


# BASELINE.json's configs in order, each with the per-kernel entries that measure it
SUMMARY = [
    ("configs[0] LayerNorm fp32 4096x768",
     ["ln_fwd", "ln_bwd_fused", "ln_bwd_input", "ln_bwd_gamma_beta"]),
    ("configs[1] GELU bf16 / CE / AdamW, alone; then inside the step (events per launch)",
     ["gelu_fwd_bf16_alone", "ce_fwd_alone", "ce_bwd_alone", "gelu_bwd_bf16_alone",
      "adamw_148_alone", "gelu_fwd_bf16", "ce_fwd", "ce_bwd", "gelu_bwd_bf16", "adamw_148"]),
    ("configs[2] attention fwd 8x12x1024x64",
     ["attn_fwd_causal_8x12x1024x64", "attn_fwd_noncausal_8x12x1024x64"]),
    ("configs[3] attention bwd 8x12x1024x64",
     ["attn_bwd_causal_8x12x1024x64", "attn_bwd_noncausal_8x12x1024x64"]),
    ("configs[4] BGEMM 8192x5120x1280 / SGEMM 4096^3",
     ["bgemm_NN_8192x5120x1280", "bgemm_NT_8192x5120x1280", "bgemm_TN_8192x5120x1280",
      "bgemm_TT_8192x5120x1280", "bgemm_dA_NT_8192x1280x5120", "bgemm_dB_TN_1280x5120x8192",
      "sgemm_NN_4096^3_splitk4_bias", "sgemm_NN_4096^3_auto_split_bias"]),
]


def print_summary(result):
    """The last lines on stderr: one short line per BASELINE config entry (time in us, rate,
    fraction of the peak, the oracle's time on one thread and on all cores), so that a reader
    of only the end of the log sees every config."""
    per = result.get("per_kernel", {})
    if not per:
        return
    short = {"_8x12x1024x64": "", "_8192x5120x1280": "", "_8192x1280x5120": "",
             "_1280x5120x8192": "", "_4096^3": "", "_bias": ""}
    lines = [f"[summary] headline {result['value']:.0f} GB/s, {result['ms_per_step']:.4f} ms/step; "
             "name us rate frac cpu-1t/cpu-all ms"]
    for title, names in SUMMARY:
        lines.append(f"[summary] {title}")
        for n in names:
            e = per.get(n)
            if e is None:
                continue
            label = n
            for k, v in short.items():
                label = label.replace(k, v)
            ms = e.get("median_ms", e.get("avg_ms"))
            unit = "G" if e.get("unit") == "GB/s" else "T"
            cpu = e.get("cpu", {})
            cpu_s = (f" {cpu['ms_1thread']:.4g}/{cpu['ms_all_cores']:.4g}"
                     if "ms_1thread" in cpu else "")
            lines.append(f"  {label} {ms * 1e3:.1f} {e['achieved']:.0f}{unit} "
                         f"{e['frac']:.3f}{cpu_s}")
    print("\n".join(lines), file=sys.stderr, flush=True)


if __name__ == "__main__":
    main()
