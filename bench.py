#!/usr/bin/env python3
"""Palettized-LUT contraction benchmark on one MI355X.

Default workload (BASELINE.json metric): 4-bit palettized GEMV at batch 1,
K=4096, N=14336 ("hero").  A step is one GEMV over one weight matrix with
the activations already in HBM.  Steps rotate over enough distinct device
copies of the weights (>= 2 x the 256 MB Infinity Cache) that every step
reads its weights from HBM.  The timed region holds exactly K back-to-back
kernels and no host launch cost: a bounded device-side spin runs while the
host enqueues them (up to 200 steps eagerly, right after the warm-up
launches; more steps captured once into a HIP graph and replayed), and
events on the launch stream bracket the K launches.  In the same process the
library's streaming-read kernel is timed the same way over as many bytes per
launch ("floor": the kernel's ratio to a pure read of its bytes).

value = effective weight bytes (index + LUT bytes) x K / timed seconds.

Other workloads (--workload): cfg1 (4-bit 4864x896), cfg2 (gate_up+SwiGLU
2x18944x3584), cfg4 (8-bit 14336x4096, --batch B), cfg5 (prefill GEMM
2048x4096x14336, TFLOP/s; --batch sets M), gemm8 (the cfg5 shape with 8-bit
weights), cfg3 (one decode step of a random-init
Qwen2.5-0.5B-architecture model, 4-bit, KV length 512: tokens/s; a step is
one token, KV rolled back to 512 after each so every step does the same
work), palettize (the palette compiler: one step palettizes every matrix of
a Qwen2.5-0.5B-architecture model, fp32 N(0, 0.02) weights resident in HBM,
k=16, max_iter=50 as compile_to_cimage uses: fp32 params/s), floor (the
read floor the GEMVs are held to: one launch of the library's streaming-read
kernel over as many bytes as the hero GEMV reads, rotated the same way;
floor8 the same over config 4's 66 MB, floor1 over config 1's 2.3 MB), load (a step is one load_cimage of a Qwen2.5-0.5B-sized 4-bit .cimage: mmap,
every tensor through the pinned staging ring, one wait; GB/s of payload), launch (an empty kernel launched back to
back: the cost of one dependent launch, us), mfma (register-only matrix-core work on every CU and on three quarters
of them: TFLOP/s and the rate per CU).
"""
from __future__ import annotations

import argparse
import ctypes
import dataclasses
import importlib
import json
import os
import platform
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
FP16_MFMA_PEAK_TFLOPS = 2500.0
MALL_BYTES = 256 << 20
# HBM bytes per launch measured with rocprofv3 (FETCH_SIZE x 1.999 + WRITE_SIZE x 1,
# scales from a 64 MiB copy in the same run), by (workload, batch): (bytes, the kernel
# the profile measured, the profile).  A line carries the figure only when the
# library reports that the same kernel ran.
PMC_TRAFFIC = {
    ("hero", 1): (30110612, "k_gemv_lpr<8, 1, 1, 0, 16>", "profiles/k_gemv_lpr_hero_4bit_b1.md"),
    ("cfg2", 1): (69368052, "k_gemv_lpr_hg<8, 2, 1, 1, 14>", "profiles/k_gemv_lpr_hg_cfg2_gateup_swiglu.md"),
    ("cfg4", 1): (66438202, "k_gemv_lpr8<8, 1, 1, 0, 32>", "profiles/k_gemv_lpr8_cfg4_8bit.md"),
}

WORKLOADS = {
    # name: (kind, bits, N, K, batch/M)
    "hero": ("gemv", 4, 14336, 4096, 1),
    "cfg1": ("gemv", 4, 4864, 896, 1),
    "cfg2": ("gateup", 4, 18944, 3584, 1),
    "cfg4": ("gemv", 8, 14336, 4096, 1),
    # config 2's gate matrix alone (74 rows per CU: the half-group GI layout), for batch sweeps
    "hgmat": ("gemv", 4, 18944, 3584, 1),
    "cfg5": ("gemm", 4, 14336, 4096, 2048),
    "gemm8": ("gemm", 8, 14336, 4096, 2048),  # the cfg5 shape with 8-bit weights (not a BASELINE config)
    "cfg3": ("decode", 4, 0, 0, 1),
    "palettize": ("palettize", 4, 0, 0, 1),
    # the read floor: one streaming-read launch over the hero's weight bytes
    "floor": ("floor", 4, 14336, 4096, 1),
    # the same over config 4's bytes (8-bit 14336 x 4096: 66 MB)
    "floor8": ("floor", 8, 14336, 4096, 1),
    # and over config 1's (4-bit 4864 x 896: 2.3 MB, a latency-bound launch)
    "floor1": ("floor", 4, 4864, 896, 1),
    # .cimage -> device: load_cimage of a Qwen2.5-0.5B-sized file
    "load": ("load", 4, 0, 0, 1),
    # measuring sticks: one dependent launch, the matrix cores' rate
    "launch": ("launch", 0, 0, 0, 1),
    "mfma": ("mfma", 0, 0, 0, 1),
    # instruction issue rates (v_fma_f32, v_dot2_f32_f16, v_perm_b32, v_mfma_f32_4x4x4f16) at 1 / 2 / 4 waves per SIMD
    "issue": ("issue", 0, 0, 0, 1),
}
PCIE_PEAK_GBS = 63.0  # PCIe 5.0 x16, one direction
DECODE_KV_LEN = 512


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def cpu_model() -> str:
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except Exception:
        pass
    return platform.processor() or "unknown"


def weight_bytes(bits: int, N: int, K: int) -> int:
    return N * (2 << bits) + N * (K // 2 if bits == 4 else K)


class _pinned_core:
    """Run the enclosed single-thread baseline on one host core."""

    def __enter__(self):
        self.old = None
        self.core = None
        try:
            self.old = os.sched_getaffinity(0)
            self.core = min(self.old)
            os.sched_setaffinity(0, {self.core})
        except (AttributeError, OSError):
            self.old = None
        return self

    def __exit__(self, *a):
        if self.old is not None:
            os.sched_setaffinity(0, self.old)


def device_busy(stream, ms: float = 2.0) -> None:
    """Enqueue a bounded spin of about `ms` on `stream`, so that the work
    recorded after it (an event, a graph) is submitted while the GPU is busy
    and the timed region holds device work only, not the host's submission
    latency.  The spin's cycles-per-ms is measured on first use."""
    import torch
    global _SPIN_CYCLES_PER_MS
    if _SPIN_CYCLES_PER_MS is None:
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            torch.cuda._sleep(1 << 18)  # warm
            a.record(stream)
            torch.cuda._sleep(1 << 20)
            b.record(stream)
        torch.cuda.synchronize()
        _SPIN_CYCLES_PER_MS = (1 << 20) / max(a.elapsed_time(b), 1e-3)
    with torch.cuda.stream(stream):
        torch.cuda._sleep(int(ms * _SPIN_CYCLES_PER_MS))


_SPIN_CYCLES_PER_MS = None

# HIP event flags (hip_runtime_api.h).  The timed region is bracketed by
# events created with hipEventDisableSystemFence, which HIP documents for
# timing: recording such an event does not write back and invalidate the
# caches at system scope, a cost (and a disturbance of the next kernel) that
# an event window of a few launches would otherwise carry at both edges.
HIP_EVENT_DISABLE_SYSTEM_FENCE = 0x20000000
HIP_EVENT_RELEASE_TO_DEVICE = 0x40000000
TIMING_EVENT_FLAGS = HIP_EVENT_DISABLE_SYSTEM_FENCE


class HipEvent:
    """A timing event of the HIP runtime (the library torch already loaded),
    created with explicit flags; record() on a torch stream."""
    _hip = None

    def __init__(self, flags: int = TIMING_EVENT_FLAGS):
        import ctypes
        if HipEvent._hip is None:
            # the HIP runtime this process already runs on (torch's copy, which
            # libprism_hip.so binds to by soname); loading another copy by name
            # would start a second runtime
            with open("/proc/self/maps") as f:
                paths = sorted({ln.split()[-1] for ln in f if "libamdhip64" in ln and "/" in ln})
            if not paths:
                raise RuntimeError("no HIP runtime loaded in this process")
            hip = ctypes.CDLL(paths[0])
            hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
            hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
            hip.hipEventSynchronize.argtypes = [ctypes.c_void_p]
            hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
            hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
            HipEvent._hip = hip
        self.h = ctypes.c_void_p()
        self._check(HipEvent._hip.hipEventCreateWithFlags(ctypes.byref(self.h), flags), "hipEventCreateWithFlags")

    @staticmethod
    def _check(rc: int, what: str) -> None:
        if rc != 0:
            raise RuntimeError(f"{what} failed: hipError {rc}")

    def record(self, stream) -> None:
        self._check(HipEvent._hip.hipEventRecord(self.h, stream.cuda_stream), "hipEventRecord")

    def elapsed_time(self, end: "HipEvent") -> float:
        import ctypes
        self._check(HipEvent._hip.hipEventSynchronize(end.h), "hipEventSynchronize")
        ms = ctypes.c_float()
        self._check(HipEvent._hip.hipEventElapsedTime(ctypes.byref(ms), self.h, end.h), "hipEventElapsedTime")
        return ms.value

    def __del__(self):
        if HipEvent._hip is not None and self.h:
            HipEvent._hip.hipEventDestroy(self.h)


# Up to this many timed steps the launches are issued eagerly (the spin ahead
# of them covers the host's enqueue of every launch); beyond it they are
# replayed from one HIP graph, whose fixed cost per replay (about 11 us on
# MI355X, inside any event window around the replay) a short run cannot
# amortise.  MI355X, hero, one box: eager 20 steps 6.63-6.73 us per launch,
# graph 2000 steps 6.44 (a graph replay of 20 steps: 6.93-7.0).
EAGER_MAX_STEPS = 200


def time_launches(launch, steps: int, warmup: int, stream, use_graph: bool, copies: int = 1,
                  event_flags: int = TIMING_EVENT_FLAGS):
    """Time exactly `steps` launches with events on `stream`, behind a
    device-side spin (device_busy) so that the window holds device work only.

    launch(i) works on rotated input copy i % copies.  First one untimed
    launch per copy, so that the timed launches find every copy's address
    translations warm, as in the steady state of a long run (MI355X, hero, 20
    eager steps: 7.36-7.55 us per launch when 15 of the 20 copies were last
    touched at upload, 6.65-6.68 once each has been read).  Then the `warmup`
    launches (indices 0..warmup-1) and the timed ones, which continue the
    rotation (indices warmup..warmup+steps-1), so no timed launch reads a copy
    read within the last few launches (still in the 256 MB MALL).

    Up to EAGER_MAX_STEPS (or without use_graph) the warm-up and the timed
    launches go eagerly one after the other with no synchronisation between
    them; above it the timed launches are captured once into a HIP graph and
    the timed replay follows an untimed one.  That whole sequence runs once
    untimed, then once timed.  Returns (device ms, wall ms, launch mode)."""
    import torch
    with torch.cuda.stream(stream):
        for i in range(copies):
            launch(i)
        for i in range(warmup):
            launch(i)
    torch.cuda.synchronize()
    graph = None
    if use_graph and steps > EAGER_MAX_STEPS:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(steps):
                launch(warmup + i)
        torch.cuda.synchronize()
    e0 = HipEvent(event_flags)
    e1 = HipEvent(event_flags)

    def sequence() -> None:
        with torch.cuda.stream(stream):
            if graph is not None:
                device_busy(stream)
                graph.replay()  # untimed replay right before the timed one
                e0.record(stream)
                graph.replay()
                e1.record(stream)
            else:
                # the host enqueues every launch while the GPU spins (Python
                # issues a launch in 5-12 us); 10 ms also brings the GPU's
                # clocks back up after the idle of the parity check
                device_busy(stream, max(10.0, 0.03 * (warmup + steps)))
                for i in range(warmup):
                    launch(i)
                e0.record(stream)
                for i in range(steps):
                    launch(warmup + i)
                e1.record(stream)

    # the whole sequence once untimed: the first one in a process reads
    # 4-5 % slower (MI355X, hero, 20 steps: 6.87-6.90 against 6.58-6.65 us)
    sequence()
    torch.cuda.synchronize()
    t_wall = time.perf_counter()
    sequence()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_wall
    del graph
    return e0.elapsed_time(e1), wall * 1e3, ("hip_graph" if use_graph and steps > EAGER_MAX_STEPS else "eager")


def time_two_streams(launch, steps: int, warmup: int, s0, s1, copies: int) -> float:
    """A probe, not the headline: `steps` launches alternating between two
    streams (launch(i, stream)), so a launch never waits for its neighbour
    and the start of one can overlap the end of the other.  Eager, behind a
    device-side spin on s0; the window opens on s0 before the first timed
    launch (s1 waits for it) and closes on s0 after both streams' last
    launches.  Returns device ms."""
    import torch
    for i in range(copies):
        launch(i, s0)
    torch.cuda.synchronize()
    e0, e1, e_end1 = HipEvent(), HipEvent(), HipEvent()
    ms = None
    for rep in range(2):  # the first sequence untimed
        device_busy(s0, max(10.0, 0.03 * (warmup + steps)))
        for i in range(warmup):
            launch(i, s0)
        e0.record(s0)
        HipEvent._hip.hipStreamWaitEvent.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint]
        HipEvent._check(HipEvent._hip.hipStreamWaitEvent(s1.cuda_stream, e0.h, 0), "hipStreamWaitEvent")
        for i in range(steps):
            launch(warmup + i, (s0, s1)[i % 2])
        e_end1.record(s1)
        HipEvent._check(HipEvent._hip.hipStreamWaitEvent(s0.cuda_stream, e_end1.h, 0), "hipStreamWaitEvent")
        e1.record(s0)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1)
    return ms


def cpu_baseline(kind, bits, N, K, batch, tensors, x, budget_s=12.0):
    """The oracle (a C restatement of lut_gemv_cpu, single thread like the
    reference) timed on this host on a bounded sample of the workload."""
    oracle = importlib.import_module("oracle")
    oracle.lib()
    t0 = tensors[0]
    if kind == "gemm":
        # M independent GEMV rows; sample rows until the budget is spent
        with _pinned_core() as pin:
            rows, t_start = 0, time.perf_counter()
            while time.perf_counter() - t_start < budget_s and rows < batch:
                oracle.gemm(np.ascontiguousarray(x[rows:rows + 1]), t0.payload, N, K, bits, threads=1)
                rows += 1
            dt = time.perf_counter() - t_start
        flops = 2.0 * rows * N * K
        return {"value": round(flops / dt / 1e12, 6), "unit": "TFLOP/s", "cores": 1, "kind": "port",
                "sample": f"{rows} of {batch} GEMM rows (oracle, 1 thread) in {dt:.1f} s",
                "pinned_core": pin.core, "cpu": cpu_model(), "host_cpus": os.cpu_count()}

    def one():
        if kind == "gateup":
            oracle.gateup_swiglu(x[0], tensors[0].payload, tensors[1].payload, N, K, bits, threads=1)
        else:
            oracle.gemv(x, t0.payload, N, K, bits, threads=1)

    with _pinned_core() as pin:
        t_start = time.perf_counter()
        one()
        t1 = time.perf_counter() - t_start
        n = max(1, min(1000, int(budget_s / max(t1, 1e-6))))
        t_start = time.perf_counter()
        for _ in range(n):
            one()
        dt = (time.perf_counter() - t_start) / n
    nbytes = weight_bytes(bits, N, K) * (2 if kind == "gateup" else 1)
    # informational: the row-parallel variant on every host core (bit-identical)
    threads = min(os.cpu_count() or 1, 16)
    ts = time.perf_counter()
    if kind == "gateup":
        oracle.gateup_swiglu(x[0], tensors[0].payload, tensors[1].payload, N, K, bits, threads=threads)
    else:
        oracle.gemv(x, t0.payload, N, K, bits, threads=threads)
    dt_mt = time.perf_counter() - ts
    return {"value": round(nbytes / dt / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{n + 1} full {kind} calls of the workload (oracle, 1 thread), {dt * 1e3:.2f} ms each",
            "pinned_core": pin.core, "all_core_value": round(nbytes / dt_mt / 1e9, 4), "all_core_threads": threads,
            "cpu": cpu_model(), "host_cpus": os.cpu_count()}


def run_decode(args, pe, seed) -> int:
    """Config 3: the GPU-resident decode step (prism_hip_model_step_dev).
    --layers / --vocab shrink the model (a probe of where the weights sit:
    inside the L2s or the MALL); the headline is the full model."""
    import torch
    oracle = importlib.import_module("oracle")
    cfg = pe.Qwen2Config()
    if args.layers is not None:
        cfg = dataclasses.replace(cfg, n_layers=args.layers)
    if args.vocab is not None:
        cfg = dataclasses.replace(cfg, vocab=args.vocab)
    L0 = DECODE_KV_LEN
    log(f"[bench] workload=cfg3 decode step: Qwen2.5-0.5B architecture, 4-bit, KV {L0}, seed={seed}")
    embed, layers = pe.synth_weights(cfg, seed)
    emb_p, lay_p = pe.model.payloads(embed, layers)
    kvs = pe.synth_kv(cfg, L0, seed)
    ctx = pe.Context(0)
    m = pe.Model.from_tensors(ctx, cfg, embed, layers, max_seq=L0 + 64)
    for l, (k, v) in enumerate(kvs):
        m.kv_append(l, k, v)
    step_bytes = cfg.weight_bytes() + cfg.kv_bytes(L0)
    log(f"[bench] {step_bytes / 1e6:.2f} MB read per token (weights {cfg.weight_bytes() / 1e6:.2f} MB + "
        f"INT8 KV {cfg.kv_bytes(L0) / 1e6:.2f} MB)")

    # parity guard: one step against the oracle (the tests hold the full bar)
    kv = oracle.KVState(cfg.n_layers, cfg.kv_dim, L0 + 1)
    for l, (k, v) in enumerate(kvs):
        for t in range(L0):
            kv.append(l, k[t], v[t])
    got = m.step(42, L0)
    want = oracle.decode_step(cfg.oracle_dims(), cfg.rms_eps, emb_p, lay_p, kv, 42, L0,
                              threads=min(os.cpu_count() or 1, 16))
    err = pe.rel_err(got, want)
    log(f"[bench] parity check (logits) rel_err={err:.3e}")
    if not err <= 1e-2:
        log("[bench] PARITY FAILURE")
        return 1
    m.kv_truncate(L0)

    stream = torch.cuda.Stream(device=torch.device("cuda", 0))

    def step(i: int) -> None:
        m.step_dev((i * 7919) % cfg.vocab, L0, stream)
        m.kv_truncate(L0)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    log(f"[bench] warmup {args.warmup} done")
    e0 = HipEvent()
    e1 = HipEvent()
    torch.cuda.synchronize()
    t_wall = time.perf_counter()
    device_busy(stream)
    e0.record(stream)
    for i in range(args.steps):
        step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_wall
    ms = e0.elapsed_time(e1)
    ms_step = ms / args.steps
    log(f"[bench] timed {args.steps} steps: {ms:.3f} ms on device events, {wall * 1e3:.3f} ms wall")
    tps = 1e3 / ms_step
    gbs = step_bytes / (ms_step * 1e-3) / 1e9

    cpu = None
    if not args.no_cpu:
        log("[bench] cpu baseline ...")
        kv_c = oracle.KVState(cfg.n_layers, cfg.kv_dim, L0 + 1)
        for l, (k, v) in enumerate(kvs):
            for t in range(L0):
                kv_c.append(l, k[t], v[t])
        with _pinned_core() as pin:
            n, t0 = 0, time.perf_counter()
            while n < 1 or time.perf_counter() - t0 < 8.0:
                kv_c.len[:] = L0
                oracle.decode_step(cfg.oracle_dims(), cfg.rms_eps, emb_p, lay_p, kv_c, 42 + n, L0, threads=1)
                n += 1
            dt = (time.perf_counter() - t0) / n
        cpu = {"value": round(1.0 / dt, 4), "unit": "tokens/s", "cores": 1, "kind": "port",
               "sample": f"{n} decode steps at KV {L0} (oracle, 1 thread), {dt * 1e3:.0f} ms each",
               "pinned_core": pin.core, "cpu": cpu_model(), "host_cpus": os.cpu_count()}
        log(f"[bench] cpu baseline {cpu['value']} tokens/s")

    rec = {
        "metric": "Qwen2.5-0.5B-architecture decode step tokens/s (4-bit palettized, batch 1, KV 512)"
                  + ("" if (args.layers is None and args.vocab is None) else
                     f" -- probe: {cfg.n_layers} layers, vocabulary {cfg.vocab}"),
        "value": round(tps, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u4-index/fp16-LUT, fp32 accumulate; INT8 KV",
        "data": "synthetic (seeded PCG64: random-init weights, sorted N(0,0.02) fp16 LUTs, KV fp16 N(0,1))",
        "config": {"workload": "cfg3", "kind": "decode", "layers": cfg.n_layers, "hidden": cfg.hidden,
                   "heads": cfg.n_heads, "kv_heads": cfg.n_kv_heads, "intermediate": cfg.intermediate,
                   "vocab": cfg.vocab, "kv_len": L0, "launch": "one HIP graph per token", "seed": seed},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "decode step (k_step_begin + one graph: 5 launches per layer + LM head)",
                     "algorithmic_per_launch": step_bytes},
        "cpu_baseline": cpu,
        "parity_rel_err": err,
    }
    print(json.dumps(rec), flush=True)
    return 0


def run_palettize(args, pe, seed) -> int:
    """The palette compiler over a whole model (prism_hip_palettize_dev)."""
    import torch
    oracle = importlib.import_module("oracle")
    cfg = pe.Qwen2Config()
    shapes = cfg.shapes()
    mats = [(cfg.vocab, cfg.hidden)] + [shapes[r] for _ in range(cfg.n_layers) for r in pe.model.LAYER_ROLES]
    params = sum(m * n for m, n in mats)
    log(f"[bench] workload=palettize: {len(mats)} matrices, {params / 1e6:.1f} M fp32 params, seed={seed}")
    g = torch.Generator(device="cuda").manual_seed(seed)
    ws = [torch.randn(m, n, generator=g, device="cuda", dtype=torch.float32).mul_(0.02) for m, n in mats]
    ctx = pe.Context(0)
    outs = [torch.empty(ctx.palettize_bytes(m, n), dtype=torch.uint8, device="cuda") for m, n in mats]
    out_bytes = sum(o.numel() for o in outs)
    stream = torch.cuda.Stream(device=torch.device("cuda", 0))

    def step() -> None:
        for (m, n), w, o in zip(mats, ws, outs):
            ctx.palettize_dev(w, m, n, o, stream=stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    log(f"[bench] warmup {args.warmup} done")
    e0 = HipEvent()
    e1 = HipEvent()
    t_wall = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_wall
    ms_step = e0.elapsed_time(e1) / args.steps
    log(f"[bench] timed {args.steps} steps: {ms_step:.3f} ms per model on device events, "
        f"{wall * 1e3 / args.steps:.3f} ms wall")

    # parity guard: layer 0's k_proj and the embedding's first 256 rows,
    # byte for byte against the oracle (the tests hold the full bar)
    def rows_of(payload, m, n, r0, r1):
        rb = (n + 1) // 2
        return np.concatenate([payload[r0 * 32:r1 * 32], payload[m * 32 + r0 * rb:m * 32 + r1 * rb]])

    ok = True
    for i, (r0, r1) in ((2, (0, cfg.kv_dim)), (0, (0, 256))):
        m, n = mats[i]
        want, _ = oracle.palettize_payload(ws[i][r0:r1].cpu().numpy(), 16, 50,
                                           threads=min(os.cpu_count() or 1, 16))
        ok &= bool(np.array_equal(rows_of(outs[i].cpu().numpy(), m, n, r0, r1), want))
    log(f"[bench] parity check (payload bytes vs oracle): {'identical' if ok else 'DIFFERENT'}")
    if not ok:
        log("[bench] PARITY FAILURE")
        return 1

    cpu = None
    if not args.no_cpu:
        log("[bench] cpu baseline ...")
        host = [(w[:max(1, w.shape[0] // 8)].cpu().numpy()) for w in ws]
        with _pinned_core() as pin:
            t0 = time.perf_counter()
            done = 0
            for h in host:
                oracle.palettize_payload(h, 16, 50, threads=1)
                done += h.size
            dt = time.perf_counter() - t0
        cpu = {"value": round(done / dt / 1e6, 4), "unit": "Mparams/s", "cores": 1, "kind": "port",
               "sample": f"first 1/8 of the rows of every matrix ({done / 1e6:.1f} M params, oracle, 1 thread), "
                         f"{dt:.1f} s",
               "pinned_core": pin.core, "cpu": cpu_model(), "host_cpus": os.cpu_count()}
        log(f"[bench] cpu baseline {cpu['value']} Mparams/s")

    value = params / (ms_step * 1e-3) / 1e6
    gbs = (params * 4 + out_bytes) / (ms_step * 1e-3) / 1e9
    rec = {
        "metric": "palette compile throughput, Qwen2.5-0.5B-architecture fp32 weights (k=16, max_iter=50)",
        "value": round(value, 2),
        "unit": "Mparams/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 k-means, fp16 LUT + u4 index out",
        "data": "synthetic (torch CUDA generator: fp32 N(0, 0.02) random-init weights)",
        "config": {"workload": "palettize", "kind": "palettize", "matrices": len(mats), "params": params,
                   "k": 16, "max_iter": 50, "seed": seed},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 5), "traffic": None,
                     "kernel": "k_palettize (whole model: fp32 read + payload write per step)",
                     "algorithmic_per_launch": params * 4 + out_bytes},
        "cpu_baseline": cpu,
    }
    print(json.dumps(rec), flush=True)
    return 0


def run_load(args, pe, seed) -> int:
    """load_cimage timed end to end: mmap of the file, every palettized
    tensor through the context's pinned staging ring (GI regrouping on
    the device where it applies), one wait.  The file is a Qwen2.5-0.5B-
    sized 4-bit .cimage with random payload bytes, written to the host's
    temporary directory first (so it is read from the page cache)."""
    import tempfile

    import torch
    cfg = pe.Qwen2Config()
    names = pe.tensor_names(cfg)
    shapes = cfg.shapes()
    tensors = [(names["embed"], cfg.vocab, cfg.hidden)]
    for l in range(cfg.n_layers):
        for role, key in names["layers"][l].items():
            tensors.append((key, shapes[role][0], shapes[role][1]))
    rng = np.random.Generator(np.random.PCG64(seed))
    fd, path = tempfile.mkstemp(suffix=".cimage")
    os.close(fd)
    total = 0
    try:
        w = pe.CImageWriter(path)
        for key, m, n in tensors:
            nb = m * 32 + m * n // 2
            w.append_palettized(key, rng.integers(0, 256, size=nb, dtype=np.uint8), m, n, 4)
            total += nb
        w.finalize()
        fsize = os.path.getsize(path)
        log(f"[bench] workload=load: {len(tensors)} tensors, {total / 1e6:.1f} MB of payload, file {fsize / 1e6:.1f} MB")

        def one() -> float:
            t0 = time.perf_counter()
            b = pe.load_cimage(path)
            dt = time.perf_counter() - t0
            n = len(b)
            b.close()
            if n != len(tensors):
                raise RuntimeError(f"loaded {n} of {len(tensors)} tensors")
            return dt

        for _ in range(args.warmup):
            one()
        times = [one() for _ in range(args.steps)]
        dt = float(np.median(times))
        value = total / dt / 1e9
        log(f"[bench] {args.steps} loads: median {dt * 1e3:.1f} ms ({value:.2f} GB/s), "
            f"min {min(times) * 1e3:.1f} ms")

        # context: each payload copied from the mapping as a pageable torch
        # tensor with a wait per tensor (the per-tensor synchronous pattern)
        r = pe.CImageReader(path)
        dev = torch.device("cuda", 0)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for key, m, n in tensors:
            torch.from_numpy(np.asarray(r.payload(key))).to(dev)
            torch.cuda.synchronize()
        pageable = total / (time.perf_counter() - t0) / 1e9
        r.close()

        cpu = None
        if not args.no_cpu:
            # the reference's host side: fs::read of the whole file, then a
            # copy of each payload (MetalBackend::new's newBufferWithBytes)
            with _pinned_core() as pin:
                t0 = time.perf_counter()
                with open(path, "rb") as f:
                    data = f.read()
                rr = pe.CImageReader(path)
                for key, m, n in tensors:
                    rec = rr.tensors[key]
                    bytearray(data[rec["offset"]:rec["offset"] + rec["size"]])
                rr.close()
                dc = time.perf_counter() - t0
            cpu = {"value": round(total / dc / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
                   "sample": f"one read of the {fsize / 1e6:.0f} MB file plus a copy of each payload, {dc * 1e3:.0f} ms",
                   "pinned_core": pin.core, "cpu": cpu_model(), "host_cpus": os.cpu_count()}
    finally:
        os.unlink(path)
    rec = {
        "metric": "load_cimage GB/s (.cimage mmap -> device, Qwen2.5-0.5B size, 4-bit)",
        "value": round(value, 3), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "u8", "data": "synthetic (random payload bytes, Qwen2.5-0.5B tensor shapes)",
        "config": {"workload": "load", "kind": "load", "tensors": len(tensors), "payload_bytes": total,
                   "file_bytes": fsize, "seed": seed},
        "roofline": {"bound": "pcie", "achieved": round(value, 3), "peak": PCIE_PEAK_GBS, "unit": "GB/s",
                     "frac": round(value / PCIE_PEAK_GBS, 4), "traffic": None, "kernel": "hipMemcpyAsync H2D"},
        "pageable_per_tensor_GBps": round(pageable, 3),
        "cpu_baseline": cpu,
    }
    print(json.dumps(rec), flush=True)
    return 0


def run_probe(args, pe, kind: str) -> int:
    """The two measuring sticks behind claims about the chains of small
    kernels and about the GEMM (measure_kernels.hpp; no counterpart in the
    reference).  launch: one empty one-wave kernel per step, launched back
    to back like the decode step's dependent kernels (value: us per launch).
    mfma: register-only matrix-core work, every CU (num_cu workgroups of one
    wave per SIMD) and three quarters of them, timed the same way as the
    GEMV workloads (value: TFLOP/s over all CUs; the line also carries the
    rate per CU at 3/4 of them).  issue: the issue rate of four instruction
    kinds (v_fma_f32, v_dot2_f32_f16, v_perm_b32, v_mfma_f32_4x4x4f16) with 1,
    2 and 4 waves per SIMD on every CU, in ns per instruction per SIMD
    (value: v_mfma_f32_4x4x4f16 at 2 waves per SIMD, the lane-per-row GEMVs'
    occupancy; the line carries the whole table)."""
    import torch
    ctx = pe.Context(0)
    dev = torch.device("cuda", 0)
    stream = torch.cuda.Stream(device=dev)
    ncu = torch.cuda.get_device_properties(dev).multi_processor_count
    if kind == "issue":
        sink = torch.zeros(256, dtype=torch.float32, device=dev)
        iters = 2000
        names = ["v_fma_f32", "v_dot2_f32_f16", "v_perm_b32", "v_mfma_f32_4x4x4f16"]
        table = {}
        for op, name in enumerate(names):
            for wps in (1, 2, 4):
                def launch(i: int, o=op, w=wps) -> None:
                    ctx.issue_probe_dev(o, ncu, w, iters, sink, stream)
                ms, _, mode = time_launches(launch, args.steps, args.warmup, stream, not args.no_graph)
                ns = ms / args.steps * 1e6 / (iters * 8 * wps)  # per instruction per SIMD
                table.setdefault(name, {})[f"{wps}_waves_per_simd"] = round(ns, 3)
                log(f"[bench] {name}, {wps} wave(s) per SIMD: {ns:.3f} ns per instruction per SIMD ({mode})")
        v = table["v_mfma_f32_4x4x4f16"]["2_waves_per_simd"]
        rec = {"metric": "ns per v_mfma_f32_4x4x4f16 per SIMD (2 waves per SIMD, every CU)", "value": v,
               "unit": "ns", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
               "ms_per_step": None, "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
               "dtype": "fp32 / fp16 register operands", "data": "synthetic register operands",
               "config": {"workload": "issue", "kind": "probe", "workgroups": ncu, "rounds": iters,
                          "chains_per_wave": 8},
               "issue_ns_per_instruction_per_simd": table, "roofline": None, "cpu_baseline": None}
        print(json.dumps(rec), flush=True)
        return 0
    if kind == "launch":
        def launch(i: int) -> None:
            ctx.launch_empty_dev(stream)
        ms, wall_ms, mode = time_launches(launch, args.steps, args.warmup, stream, not args.no_graph)
        us = ms / args.steps * 1e3
        log(f"[bench] empty kernel, {args.steps} launches ({mode}): {us:.3f} us per launch")
        rec = {"metric": "dependent launch us (empty one-wave kernel, back to back)", "value": round(us, 4),
               "unit": "us", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
               "ms_per_step": round(ms / args.steps, 6), "higher_is_better": False, "scaling": "weak",
               "vs_baseline": None, "dtype": "none", "data": "none",
               "config": {"workload": "launch", "kind": "probe", "launch": mode},
               "roofline": None, "cpu_baseline": None}
        print(json.dumps(rec), flush=True)
        return 0
    sink = torch.zeros(256, dtype=torch.float32, device=dev)
    iters = 512
    flop_per_group = 4 * iters * 16 * 2 * 32 * 32 * 16
    out = {}
    for groups in (ncu, (3 * ncu) // 4):
        def launch(i: int, g=groups) -> None:
            ctx.mfma_probe_dev(g, iters, sink, stream)
        ms, _, mode = time_launches(launch, args.steps, args.warmup, stream, not args.no_graph)
        tflops = flop_per_group * groups * args.steps / (ms * 1e-3) / 1e12
        out[groups] = (ms / args.steps, tflops)
        log(f"[bench] MFMA probe, {groups} workgroups x 4 waves x {iters} rounds: {ms / args.steps * 1e3:.2f} us, "
            f"{tflops:.1f} TFLOP/s, {tflops / groups:.3f} per CU")
    full, part = out[ncu], out[(3 * ncu) // 4]
    rec = {"metric": "register-only fp16 MFMA TFLOP/s (v_mfma_f32_32x32x16_f16, one wave per SIMD, every CU)",
           "value": round(full[1], 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": round(full[0], 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "dtype": "fp16 in, fp32 accumulate", "data": "synthetic register operands",
           "config": {"workload": "mfma", "kind": "probe", "workgroups": ncu, "rounds": iters, "launch": "per step"},
           "roofline": {"bound": "mfma", "achieved": round(full[1], 2), "peak": FP16_MFMA_PEAK_TFLOPS,
                        "unit": "TFLOP/s", "frac": round(full[1] / FP16_MFMA_PEAK_TFLOPS, 4), "traffic": None,
                        "kernel": "k_mfma_probe"},
           "three_quarters": {"workgroups": (3 * ncu) // 4, "TFLOPs": round(part[1], 2),
                              "per_cu_over_all_cus": round((part[1] / ((3 * ncu) // 4)) / (full[1] / ncu), 4)},
           "cpu_baseline": None}
    print(json.dumps(rec), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed steps (default 2000; palettize: 10)")
    ap.add_argument("--warmup", type=int, default=None, help="untimed steps (default 50; palettize: 2)")
    ap.add_argument("--workload", default="hero", choices=sorted(WORKLOADS))
    ap.add_argument("--batch", type=int, default=None,
                    help="batch for gemv workloads (cfg4 sweep), rows of X (M) for the GEMM")
    ap.add_argument("--no-graph", action="store_true", help="launch eagerly instead of replaying a HIP graph")
    ap.add_argument("--no-cpu", action="store_true", help="skip the cpu_baseline leg")
    ap.add_argument("--no-floor", action="store_true", help="skip the same-process read-floor leg")
    ap.add_argument("--rotate-mb", type=int, default=640, help="distinct weight bytes the steps rotate over")
    ap.add_argument("--streams", type=int, default=1, choices=(1, 2),
                    help="probe (hero and floor only): 2 alternates the launches between two streams, so "
                         "neighbouring launches do not wait for each other (the headline is 1: a dependent chain)")
    ap.add_argument("--layers", type=int, default=None, help="cfg3: decoder layers (default 24)")
    ap.add_argument("--vocab", type=int, default=None, help="cfg3: vocabulary, the LM head's rows (default 151936)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MB",
                    help="after timing, run one untimed device copy of MB MiB (scale reference for "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    # a palettize step compiles a whole model (about 0.1 s)
    if args.steps is None:
        args.steps = 10 if args.workload in ("palettize", "load") else 2000
    if args.warmup is None:
        args.warmup = 2 if args.workload in ("palettize", "load") else 50

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build measures one GPU: the palettized contraction runs on a single "
                                   "MI355X; multi-GPU sharding is design-only (rows per GPU + all-gather of y)",
                          "n_gpus": args.gpus}))
        return 2

    import torch
    pe = importlib.import_module("prism-engine_amd")
    kind, bits, N, K, batch = WORKLOADS[args.workload]
    if args.streams == 2 and not (kind == "floor" or (args.workload == "hero" and (args.batch or 1) == 1)):
        print(json.dumps({"error": "--streams 2 is a probe for the hero GEMV and the read floor"}))
        return 2
    if (args.layers is not None or args.vocab is not None) and kind != "decode":
        print(json.dumps({"error": "--layers / --vocab apply to cfg3"}))
        return 2
    if kind == "decode":
        return run_decode(args, pe, pe.SEEDS.get(args.workload, 1003))
    if kind == "palettize":
        return run_palettize(args, pe, pe.SEEDS.get(args.workload, 1006))
    if kind == "load":
        return run_load(args, pe, pe.SEEDS.get(args.workload, 1007))
    if kind in ("launch", "mfma", "issue"):
        return run_probe(args, pe, kind)
    if args.batch is not None and kind in ("gemv", "gemm"):
        batch = args.batch  # batch vectors, or the GEMM's rows of X
    seed = pe.SEEDS.get(args.workload, 1000)

    log(f"[bench] workload={args.workload} kind={kind} bits={bits} N={N} K={K} batch/M={batch} seed={seed}")
    nmat = 2 if kind == "gateup" else 1
    wb = weight_bytes(bits, N, K) * nmat
    copies = 1 if kind == "gemm" else max(2, -(-(args.rotate_mb << 20) // wb))
    ctx = pe.Context(0)
    dev = torch.device("cuda", 0)
    stream = torch.cuda.Stream(device=dev)

    if kind == "floor":
        # random bytes, so the kernel's XOR never matches and nothing is written
        g = torch.Generator(device=dev).manual_seed(seed)
        bufs = [torch.randint(0, 256, (wb,), dtype=torch.uint8, device=dev, generator=g) for _ in range(copies)]
        sink = torch.zeros(256, dtype=torch.int32, device=dev)
        log(f"[bench] {copies} buffers x {wb / 1e6:.2f} MB = {copies * wb / 1e6:.0f} MB rotated")

        def launch(i: int, st=stream) -> None:
            ctx.stream_read_dev(bufs[i % copies], wb, sink, st)
        err = None
        args.no_cpu = True
    else:
        tensors = [pe.synth_tensor(N, K, bits, seed=seed + i) for i in range(nmat)]
        x = pe.synth_x(batch, K, seed=seed)
        weights = [[ctx.upload_tensor(t) for t in tensors] for _ in range(copies)]
        dx = torch.from_numpy(x.view(np.int16)).to(dev)
        ny = (batch * N) if kind != "gateup" else N
        dy = torch.empty(ny, dtype=torch.int16, device=dev)
        dy2 = torch.empty(ny, dtype=torch.int16, device=dev)  # the second stream's output (--streams 2)
        log(f"[bench] {copies} weight copies x {wb / 1e6:.2f} MB = {copies * wb / 1e6:.0f} MB rotated")

        def launch(i: int, st=None) -> None:
            w = weights[i % copies]
            if st is not None and st is not stream:
                ctx.gemv_dev(w[0], dx, batch, dy2, st)
            elif kind == "gemv":
                ctx.gemv_dev(w[0], dx, batch, dy, stream)
            elif kind == "gateup":
                ctx.gateup_swiglu_dev(w[0], w[1], dx, dy, stream)
            else:
                ctx.gemm_dev(w[0], dx, batch, dy, stream)

    # correctness guard on a sample before timing (the tests hold the full bar)
    launch(0)
    torch.cuda.synchronize()
    if kind == "gemv":
        oracle = importlib.import_module("oracle")
        yk = dy.cpu().numpy().view(np.uint16)
        ref = oracle.gemv(x, tensors[0].payload, N, K, bits, threads=min(os.cpu_count() or 1, 16))
        err = max(pe.rel_err(yk.reshape(batch, N)[b], ref[b]) for b in range(batch))
    elif kind == "gateup":
        oracle = importlib.import_module("oracle")
        yk = dy.cpu().numpy().view(np.uint16)
        ref = oracle.gateup_swiglu(x[0], tensors[0].payload, tensors[1].payload, N, K, bits,
                                   threads=min(os.cpu_count() or 1, 16))
        err = pe.rel_err(yk, ref)
    elif kind == "gemm":
        oracle = importlib.import_module("oracle")
        yk = dy.cpu().numpy().view(np.uint16)
        rows = [0, batch // 2, batch - 1]
        ref = oracle.gemm(np.ascontiguousarray(x[rows]), tensors[0].payload, N, K, bits, threads=8)
        err = max(pe.rel_err(yk.reshape(batch, N)[r], ref[i]) for i, r in enumerate(rows))
    if err is not None:
        log(f"[bench] parity check rel_err={err:.3e}")
        if not err <= 2e-3:
            log("[bench] PARITY FAILURE")
            return 1

    # the kernels the library's dispatch picked for one step, as it reports them
    kernel_name = ctx.last_kernels()
    log(f"[bench] kernels of one step: {kernel_name}")

    if args.streams == 2:
        # probe: neighbouring launches independent, on two streams
        ms = time_two_streams(launch, args.steps, args.warmup, stream, torch.cuda.Stream(device=dev), copies)
        wall_ms, launch_mode = float("nan"), "eager, two streams (neighbouring launches independent)"
    else:
        ms, wall_ms, launch_mode = time_launches(launch, args.steps, args.warmup, stream, not args.no_graph, copies)
    ms_step = ms / args.steps
    log(f"[bench] timed {args.steps} steps ({launch_mode}, behind a device-side spin): {ms:.3f} ms on device "
        f"events, {wall_ms:.3f} ms wall")

    # the read floor in the same process: k_stream_read over as many bytes
    # per launch, rotated over as many distinct buffers, timed the same way
    floor = None
    if kind in ("gemv", "gateup") and not args.no_floor and args.streams == 1:
        g = torch.Generator(device=dev).manual_seed(seed + 1)
        fbufs = [torch.randint(0, 256, (wb,), dtype=torch.uint8, device=dev, generator=g) for _ in range(copies)]
        fsink = torch.zeros(256, dtype=torch.int32, device=dev)

        def flaunch(i: int) -> None:
            ctx.stream_read_dev(fbufs[i % copies], wb, fsink, stream)
        fms, _, _ = time_launches(flaunch, args.steps, args.warmup, stream, not args.no_graph, copies)
        f_us = fms / args.steps * 1e3
        floor = {"kernel": "k_stream_read", "us_per_launch": round(f_us, 4),
                 "GBps": round(wb / (f_us * 1e-6) / 1e9, 2), "kernel_over_floor": round(ms_step * 1e3 / f_us, 4),
                 "bytes_per_launch": wb, "buffers_rotated": copies}
        log(f"[bench] read floor (same process, same bytes and rotation): {f_us:.3f} us per launch; "
            f"this workload takes {floor['kernel_over_floor']:.3f} x the floor")
        del fbufs, fsink

    if args.copy_calibration > 0:
        src = torch.empty(args.copy_calibration << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] copy calibration: {args.copy_calibration} MiB device-to-device copy done")
        del src, dst

    if kind == "gemm":
        flops = 2.0 * batch * N * K
        value = flops / (ms_step * 1e-3) / 1e12
        unit, metric = "TFLOP/s", "palettized GEMM fp16-MFMA TFLOP/s (% of 2.5 PFLOP/s dense fp16)"
        roof = {"bound": "mfma", "achieved": round(value, 3), "peak": FP16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(value / FP16_MFMA_PEAK_TFLOPS, 4), "traffic": None}
    else:
        value = wb / (ms_step * 1e-3) / 1e9
        unit = "GB/s"
        metric = ("palettized GEMV effective HBM GB/s (% of 8 TB/s peak), 4-bit, batch 1"
                  if args.workload == "hero" and batch == 1 and args.streams == 1 else
                  "palettized GEMV HBM GB/s with neighbouring launches overlapping (two streams; a probe, "
                  "not the dependent-chain headline), 4-bit, batch 1"
                  if args.workload == "hero" and batch == 1 else
                  "streaming-read floor GB/s, neighbouring launches overlapping (two streams)"
                  if kind == "floor" and args.streams == 2 else
                  f"streaming-read floor GB/s (one launch over the "
                  f"{'config-1' if args.workload == 'floor1' else 'hero' if bits == 4 else 'config-4'} weight bytes)"
                  if kind == "floor" else
                  f"palettized {kind} effective HBM GB/s (% of 8 TB/s peak), {bits}-bit, batch {batch}")
        roof = {"bound": "hbm", "achieved": round(value, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(value / HBM_PEAK_GBS, 4), "traffic": None}
        pmc = PMC_TRAFFIC.get((args.workload, batch))
        if pmc is not None and pmc[1] == kernel_name:
            roof["traffic"] = pmc[0]
            roof["traffic_source"] = f"{pmc[2]} (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of {pmc[1]})"
    roof["kernel"] = kernel_name
    roof["algorithmic_per_launch"] = (2.0 * batch * N * K) if kind == "gemm" else wb

    cpu = None
    if not args.no_cpu:
        log("[bench] cpu baseline ...")
        cpu = cpu_baseline(kind, bits, N, K, batch, tensors, x)
        log(f"[bench] cpu baseline {cpu['value']} {cpu['unit']}")

    rec = {
        "metric": metric,
        "value": round(value, 3),
        "unit": unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("u8" if kind == "floor" else
                  "u4-index/fp16-LUT, fp32 accumulate" if bits == 4 else "u8-index/fp16-LUT, fp32 accumulate"),
        "data": ("synthetic (uniform random bytes)" if kind == "floor" else
                 "synthetic (seeded PCG64: x~N(0,1) fp16, uniform indices, sorted N(0,0.02) fp16 LUTs)"),
        "config": {"workload": args.workload, "kind": kind, "bits": bits, "N": N, "K": K,
                   ("M" if kind == "gemm" else "batch"): batch, "weight_copies_rotated": copies,
                   "launch": launch_mode, "streams": args.streams, "seed": seed},
        "roofline": roof,
        "floor": floor,
        "cpu_baseline": cpu,
        "parity_rel_err": err,
    }
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
