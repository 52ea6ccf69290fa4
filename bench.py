#!/usr/bin/env python3
"""Benchmark of the MI355X DVAttn operators on the five BASELINE configurations.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs 1,2,2u,3,4,5,5v,5f] [--no-cpu]
    python bench.py --read-ceiling | --mfma-ceiling | --small-crossover      (measurement probes only)

One "step" is one call of the operator over one batch of synthetic, seeded
inputs already resident in HBM.  The headline line (``value``) is configuration
2 (bf16 paged GQA-16 decode, batch 32, KV length U[1024, 8192], page 16): K
steps are timed back to back between two synchronisations; ``value`` is the
achieved algorithmic HBM rate in TB/s and ``ms_per_step`` the time per call.
Before each timed region the same calls run untimed for ``--prewarm-ms``
(default 50 ms) besides the W warm-up steps, so that the GPU's clock has left
its idle state (its governor takes 10-20 ms of load to reach the steady clock).
Inputs rotate over enough replicas that consecutive calls never find their K/V
in the 256 MB Infinity Cache (cold HBM reads, as in a real multi-layer decode
step).  Every configuration is also reported under ``per_config`` (``5v``:
configuration 5's 16-token chunks packed through the varlen op, its cross-check;
``2u``: configuration 2 with all 32 sequences at 8192 keys, the north star's
"batch 32 x 8k context" read literally -- supplementary, the headline stays
configuration 2; ``5f``: configuration 5's shape in fp32, the fp32 multi-query
kernel), and the
cache-side kernels around the path (K-side append, merge_caches re-rotation,
view metadata) under ``cache_rows``.

``roofline`` covers the decode kernel family (decode + split-merge launch of one
call): algorithmic bytes over the per-call time of the back-to-back timed region
(HIP events on the stream the kernels run on); ``traffic`` is the
HBM bytes per call measured with rocprofv3 counters (profiles/).  ``cpu_baseline``
times the CPU oracle (the fp32 restatement of the reference's eager path) on a
bounded sample of configuration 2, on this host's cores.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

HBM_PEAK_GBS = 8000.0            # MI355X HBM3E
MFMA_BF16_PEAK_TFLOPS = 2500.0   # dense bf16/fp16
METRIC = "paged decode-attn µs/call + achieved HBM TB/s (% of peak), bf16 GQA-16"
MALL_BYTES = 256 << 20


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def replicas_for(wl_bytes: int, max_replicas: int = 4096) -> int:
    # enough distinct inputs that the rotation's footprint is >= 4x the Infinity
    # Cache, so every call reads its K/V from HBM (configuration 1's 0.5 MB
    # takes about 1900 replicas)
    need = max(1, -(-4 * MALL_BYTES // max(1, wl_bytes)))
    return min(max_replicas, need)


# Configurations other than the headline time at least this much GPU work per
# measurement (more calls than --steps when a call is short): a few tens of
# calls of a 10 us call are dominated by the first launch's host latency.
MIN_TIMED_US = 2000.0

# Before each timed region the GPU runs the measured calls themselves for at
# least this long (wall clock), besides the --warmup steps: the shader clock
# idles at ~100 MHz while the host builds inputs and its governor needs 10-20 ms
# of load to reach the steady clock (1.7 -> 2.3 GHz measured), so a handful of
# 0.1 ms warm-up calls would time part of the ramp (configuration 5's first 30
# calls after a pause: 219 us each, then 185).  --prewarm-ms 0: exactly W
# warm-up steps.
PREWARM_MS = 50.0


def prewarm(call, ms: float) -> None:
    """Run call(j) for at least `ms` milliseconds of wall time, in batches of 16
    between synchronisations (so the queue stays short)."""
    if ms <= 0:
        return
    t0 = time.perf_counter()
    j = 0
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(16):
            call(j)
            j += 1
        torch.cuda.synchronize()


def time_config(i, steps: int, warmup: int, device, exact: bool = False) -> dict:
    """Per-call time of configuration i (1-5, "5v", "5f" or "2u").  exact: time exactly
    `steps` calls (the headline); otherwise at least `steps` calls and at least
    MIN_TIMED_US of work, estimated from the warm-up calls."""
    from dvattention_amd import workloads as WL
    first = WL.workload(i, device=device, seed=1234)
    R = replicas_for(first.meta.get("kv_bytes", first.alg_bytes))
    wls = [first] + [WL.workload(i, device=device, seed=1234 + r) for r in range(1, R)]
    outs = [w.out_like() for w in wls]
    rqs = [torch.empty(w.meta["rq_shape"], dtype=w.dtype, device=device) if w.op == "fused" else None for w in wls]
    prewarm(lambda j: WL.run(wls[j % R], outs[j % R], rqs[j % R]), PREWARM_MS)
    for j in range(warmup):
        WL.run(wls[j % R], outs[j % R], rqs[j % R])
    torch.cuda.synchronize()
    if not exact:
        # 10 more untimed calls estimate the call time
        t_w = time.perf_counter()
        for j in range(10):
            WL.run(wls[j % R], outs[j % R], rqs[j % R])
        torch.cuda.synchronize()
        est_us = (time.perf_counter() - t_w) * 1e6 / 10
        steps = max(steps, min(4096, int(MIN_TIMED_US / max(est_us, 1.0)) + 1))
    stream = torch.cuda.current_stream()
    # (a) K back-to-back steps between two synchronisations (wall clock + events)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for j in range(steps):
        WL.run(wls[j % R], outs[j % R], rqs[j % R])
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    ms_step = ev0.elapsed_time(ev1) / steps
    # (b) per-call kernel time: events around each call on the launch stream
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for j in range(steps):
        a, b = evs[j]
        a.record(stream)
        WL.run(wls[j % R], outs[j % R], rqs[j % R])
        b.record(stream)
    torch.cuda.synchronize()
    per_call = sorted(a.elapsed_time(b) for a, b in evs)
    kern_ms = sum(per_call) / len(per_call)
    med_ms = per_call[len(per_call) // 2]
    alg = sum(w.alg_bytes for w in wls) / R
    flops = sum(w.flops for w in wls) / R
    res = {
        "config": i,
        "workload": first.name,
        "op": first.op,
        "dtype": str(first.dtype).replace("torch.", ""),
        "replicas": R,
        "steps": steps,
        "us_per_call": round(ms_step * 1e3, 2),
        "us_per_call_wall": round(wall * 1e6, 2),
        "kernel_us_mean": round(kern_ms * 1e3, 2),
        "kernel_us_median": round(med_ms * 1e3, 2),
        "alg_bytes": int(alg),
        "alg_flops": int(flops),
        "achieved_GBs": round(alg / (kern_ms * 1e-3) / 1e9, 1),
        "hbm_frac": round(alg / (kern_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "achieved_TFLOPs": round(flops / (kern_ms * 1e-3) / 1e12, 2),
        "mfma_frac": round(flops / (kern_ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
    }
    del wls, outs, rqs
    torch.cuda.empty_cache()
    return res


def read_ceiling(i: int, steps: int, warmup: int, device) -> dict:
    """The paged-read probe (dvattention_amd/csrc/dv_probe.hip, libdvattn_probe.so)
    on configuration i's inputs: the decode kernel's K/V stream -- same work
    split, launch shape, page-id cache, direct-to-LDS ring and waits -- with the
    attention taken out.  Timed like time_config (back-to-back calls over the
    same input replicas, HIP events on the launch stream); the rate is the
    visible K/V bytes per call over the time."""
    import ctypes
    from dvattention_amd import capi
    from dvattention_amd import workloads as WL
    lib = ctypes.CDLL(os.path.join(HERE, "dvattention_amd", "libdvattn_probe.so"))
    lib.dvprobe_last_error.restype = ctypes.c_char_p
    lib.dvprobe_paged_read.restype = ctypes.c_int
    lib.dvprobe_paged_read.argtypes = [ctypes.c_int] + [ctypes.c_void_p] * 6 + [ctypes.c_void_p, ctypes.c_size_t,
                                                                                  ctypes.c_void_p, ctypes.c_longlong,
                                                                                  ctypes.c_void_p]
    first = WL.config(i, device=device, seed=1234)
    if first.op != "paged" or first.meta["S"] != 1:
        raise ValueError(f"config {i}: the read probe covers one-view paged decode configurations")
    R = replicas_for(first.meta.get("kv_bytes", first.alg_bytes))
    wls = [first] + [WL.config(i, device=device, seed=1234 + r) for r in range(1, R)]
    args = []
    for w in wls:
        t = w.t
        shp = capi.paged_shape(t["queries"], t["locations"], t["cosines"], t["k_cache"], t["v_cache"],
                               t["block_tables"])
        ws = torch.empty(1 << 20, dtype=torch.uint8, device=device)
        sink = torch.empty(4 * 4096, dtype=torch.int32, device=device)
        args.append((shp, ws, sink, t))
    stream = torch.cuda.current_stream()

    def call(j):
        shp, ws, sink, t = args[j % R]
        rc = lib.dvprobe_paged_read(capi.dtype_code(first.dtype), t["locations"].data_ptr(),
                                    t["fragment_lengths"].data_ptr(), t["k_cache"].data_ptr(),
                                    t["v_cache"].data_ptr(), t["block_tables"].data_ptr(), ctypes.byref(shp),
                                    ws.data_ptr(), ws.numel(), sink.data_ptr(), sink.numel(), stream.cuda_stream)
        if rc != 0:
            raise RuntimeError(lib.dvprobe_last_error().decode())

    prewarm(call, PREWARM_MS)
    for j in range(warmup):
        call(j)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for j in range(steps):
        call(j)
    ev1.record(stream)
    torch.cuda.synchronize()
    us = ev0.elapsed_time(ev1) * 1e3 / steps
    kv = sum(w.meta["kv_bytes"] for w in wls) / R
    del wls, args
    torch.cuda.empty_cache()
    return {"config": i, "workload": first.name, "probe_us_per_call": round(us, 2), "kv_bytes": int(kv),
            "read_GBs": round(kv / (us * 1e-6) / 1e9, 1), "read_frac": round(kv / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}


def plain_read(device, gib: int = 4, calls: int = 10) -> dict:
    """A plain full-chip streaming read of a contiguous buffer (dv_probe.hip
    `dvprobe_plain_read`: 16-byte loads, grid-stride), with non-temporal and with
    default-policy loads: the part's read rate without paging, for scale."""
    import ctypes
    lib = ctypes.CDLL(os.path.join(HERE, "dvattention_amd", "libdvattn_probe.so"))
    lib.dvprobe_last_error.restype = ctypes.c_char_p
    lib.dvprobe_plain_read.restype = ctypes.c_int
    lib.dvprobe_plain_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_void_p,
                                       ctypes.c_longlong, ctypes.c_void_p]
    nbytes = gib << 30
    buf = torch.ones(nbytes // 4, dtype=torch.int32, device=device)
    sink = torch.empty(4 * 8192, dtype=torch.int32, device=device)
    stream = torch.cuda.current_stream()
    out = {"bytes": nbytes}
    for nt in (1, 0):
        def call():
            if lib.dvprobe_plain_read(buf.data_ptr(), nbytes, nt, sink.data_ptr(), sink.numel(),
                                      stream.cuda_stream) != 0:
                raise RuntimeError(lib.dvprobe_last_error().decode())
        prewarm(lambda j: call(), PREWARM_MS)
        for _ in range(3):
            call()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record(stream)
        for _ in range(calls):
            call()
        b.record(stream)
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / calls
        out["nontemporal_GBs" if nt else "default_GBs"] = round(nbytes / (us * 1e-6) / 1e9, 1)
    del buf
    torch.cuda.empty_cache()
    return out


def mfma_ceiling(device, iters: int = 2000, calls: int = 10) -> dict:
    """The MFMA rate probe (dv_probe.hip `dvprobe_mfma_rate`): back-to-back
    v_mfma_f32_16x16x32_bf16 on every SIMD at the chunk kernel's occupancy (eight
    waves per CU), alone and with n independent fp32 FMAs or v_exp_f32 per MFMA;
    then v_mfma_f32_32x32x16_bf16 with n FMAs per MFMA (`dvprobe_mfma_rate32`).
    Per mix: TFLOP/s, the shader clock the waves ran at (s_memtime against the
    100 MHz s_memrealtime counter), and SIMD cycles per MFMA at that clock."""
    import ctypes
    lib = ctypes.CDLL(os.path.join(HERE, "dvattention_amd", "libdvattn_probe.so"))
    lib.dvprobe_last_error.restype = ctypes.c_char_p
    lib.dvprobe_mfma_rate.restype = ctypes.c_int
    lib.dvprobe_mfma_rate.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_longlong,
                                      ctypes.c_void_p, ctypes.c_longlong, ctypes.c_void_p]
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    sink = torch.empty(512 * cus, dtype=torch.float32, device=device)
    clocks = torch.zeros(16 * cus, dtype=torch.int64, device=device)
    stream = torch.cuda.current_stream()
    rows = []
    for n, ex in ((0, 0), (1, 0), (2, 0), (3, 0), (4, 0), (6, 0), (1, 1), (2, 1), (0, 0)):
        def call():
            wgs = lib.dvprobe_mfma_rate(n, ex, iters, sink.data_ptr(), sink.numel(), clocks.data_ptr(),
                                        clocks.numel(), stream.cuda_stream)
            if wgs < 0:
                raise RuntimeError(lib.dvprobe_last_error().decode())
            return wgs
        for _ in range(2):
            wgs = call()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(calls):
            call()
        b.record(stream)
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / calls
        ck = clocks.view(-1, 2).double().sum(0).tolist()
        mhz = ck[0] / ck[1] * 100.0 if ck[1] > 0 else 0.0
        mfma_per_simd = iters * 8 * 2                 # two waves per SIMD, eight MFMAs per round
        rows.append({"shape": "16x16x32", "other_per_mfma": n, "kind": "exp" if ex else "fma", "us": round(us, 1),
                     "tflops": round(wgs * 8 * iters * 8 * 16384 / (us * 1e-6) / 1e12, 1),
                     "clock_mhz": round(mhz), "simd_cycles_per_mfma": round(mhz * us / mfma_per_simd, 2)})
    # v_mfma_f32_32x32x16_bf16 (twice the work per instruction, half the rounds):
    # n FMAs per MFMA = n/2 per 16x16x32-equivalent
    lib.dvprobe_mfma_rate32.restype = ctypes.c_int
    lib.dvprobe_mfma_rate32.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_longlong,
                                        ctypes.c_void_p, ctypes.c_longlong, ctypes.c_void_p]
    it32 = iters // 2
    for n in (0, 2, 4, 6, 8, 12):
        def call():
            wgs = lib.dvprobe_mfma_rate32(n, it32, sink.data_ptr(), sink.numel(), clocks.data_ptr(),
                                          clocks.numel(), stream.cuda_stream)
            if wgs < 0:
                raise RuntimeError(lib.dvprobe_last_error().decode())
            return wgs
        for _ in range(2):
            wgs = call()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(calls):
            call()
        b.record(stream)
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / calls
        ck = clocks.view(-1, 2).double().sum(0).tolist()
        mhz = ck[0] / ck[1] * 100.0 if ck[1] > 0 else 0.0
        mfma_per_simd = it32 * 8 * 2
        rows.append({"shape": "32x32x16", "other_per_mfma": n, "kind": "fma", "us": round(us, 1),
                     "tflops": round(wgs * 8 * it32 * 8 * 32768 / (us * 1e-6) / 1e12, 1),
                     "clock_mhz": round(mhz), "simd_cycles_per_mfma": round(mhz * us / mfma_per_simd, 2)})
    return {"cus": cus, "iters": iters, "rows": rows}


# Calls of the crossover table: (W, Hkv, fragment lengths); the query of each
# sequence sits after its views and sees every key.
CROSSOVER_CALLS = [(1, 1, [512]), (1, 8, [512]), (1, 1, [4096]), (2, 8, [256, 64]), (2, 8, [512]),
                   (4, 8, [512]), (32, 8, [64]), (1, 8, [2048]), (8, 8, [256])]


def small_crossover(device, min_us: float = 3000.0) -> dict:
    """dvattn_fused through the single-launch path (library option small_path =
    force) and through the general path (off) on the same calls: µs per call, back to
    back, over enough input replicas that every call reads its K/V from HBM.
    Its rows set the workgroup limit of the single-launch path (dv_capi.hip
    small_path_chunks): past it the merge protocol's fences cost more than the
    general path's three launches."""
    from dvattention_amd import attention as A
    from dvattention_amd import capi
    from dvattention_amd import workloads as WL
    rows = []
    saved = capi.get_option("small_path")
    try:
        for dtype in (torch.float32, torch.bfloat16):
            es = 4 if dtype == torch.float32 else 2
            for W, Hkv, lens in CROSSOVER_CALLS:
                Hq, E, R, F = 16 * Hkv, 128, 64, len(lens)
                kv = W * Hkv * sum(lens) * 2 * E * es
                nrep = replicas_for(kv, max_replicas=2048)
                gen = torch.Generator(device=device).manual_seed(7)
                pos = sum(lens)
                loc = torch.tensor([[[pos - sum(lens[:f])]] * W for f in range(F)], dtype=torch.int32, device=device)
                c, s_ = WL.hf_cos_sin(loc.cpu().numpy(), R, 1e4)
                c, s_ = c.to(device), s_.to(device)
                fl = torch.tensor(lens, dtype=torch.int32, device=device)
                reps = []
                for _ in range(nrep):
                    q = torch.randn(W, Hq, 1, E, generator=gen, device=device).to(dtype)
                    ks = [torch.randn(W, Hkv, L, E, generator=gen, device=device).to(dtype) for L in lens]
                    vs = [torch.randn(W, Hkv, L, E, generator=gen, device=device).to(dtype) for L in lens]
                    reps.append((q, ks, vs, torch.empty(F, W, Hq, 1, E, dtype=dtype, device=device),
                                 torch.empty(W, Hq, 1, E, dtype=dtype, device=device)))

                def call(j):
                    q, ks, vs, rq, out = reps[j % nrep]
                    A.dvattn_fused(q, loc, ks, vs, E ** -0.5, fl, c, s_, rotated_queries=rq, out=out)

                row = {"dtype": str(dtype).replace("torch.", ""), "W": W, "Hkv": Hkv, "lens": lens,
                       "chunks": sum(-(-L // 64) for L in lens)}
                row["workgroups"] = W * Hkv * row["chunks"]
                for mode in ("force", "off"):
                    capi.set_option("small_path", capi.SMALL_PATH[mode])
                    prewarm(call, PREWARM_MS)
                    for j in range(5):
                        call(j)
                    torch.cuda.synchronize()
                    t = time.perf_counter()
                    for j in range(10):
                        call(j)
                    torch.cuda.synchronize()
                    est = (time.perf_counter() - t) * 1e6 / 10
                    n = max(50, int(min_us / max(est, 1.0)))
                    stream = torch.cuda.current_stream()
                    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    a.record(stream)
                    for j in range(n):
                        call(j)
                    b.record(stream)
                    torch.cuda.synchronize()
                    row["single_us" if mode == "force" else "general_us"] = round(a.elapsed_time(b) * 1e3 / n, 2)
                rows.append(row)
                log(f"[bench] {row['dtype']} W={W} Hkv={Hkv} lens={lens}: {row['workgroups']} workgroups, single "
                    f"{row['single_us']} us, general {row['general_us']} us per call")
                del reps
                torch.cuda.empty_cache()
    finally:
        capi.set_option("small_path", saved)
    return {"rows": rows}


def _time_calls(fn, n_inputs: int, steps: int, warmup: int) -> tuple:
    """Mean µs per call of fn(j % n_inputs): (a) `steps` eager back-to-back calls
    (HIP events; small kernels are bound by the host's launch rate there) and
    (b) the same calls captured in one HIP graph and replayed (the GPU-side cost
    of a call, as in a graph-captured decode step)."""
    prewarm(lambda j: fn(j % n_inputs), PREWARM_MS)
    for j in range(warmup):
        fn(j % n_inputs)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for j in range(steps):
        fn(j % n_inputs)
    b.record(stream)
    torch.cuda.synchronize()
    eager = a.elapsed_time(b) * 1e3 / steps
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for j in range(steps):
            fn(j % n_inputs)
    graph.replay()
    torch.cuda.synchronize()
    a.record(stream)
    graph.replay()
    b.record(stream)
    torch.cuda.synchronize()
    replay = a.elapsed_time(b) * 1e3 / steps
    del graph
    return replay, eager


def time_cache_rows(device, steps: int, warmup: int) -> list:
    """The rows around the decode path: the K-side append (key rotation + page
    writes) at a decode step of configuration 2 and at an 8192-token prefill,
    merge_caches' re-rotation of a 32768-token source, and the on-device view
    metadata of a configuration-2 step with 4 views.  Algorithmic bytes: keys and
    values read once and written once, cos/sin, positions and table entries read
    once (metadata: lengths/orders read, locations and cos/sin written)."""
    import dvattention_amd as dv
    g = torch.Generator(device="cpu").manual_seed(7)
    rows = []

    def append_case(name, W, S, Hkv, cos_rows, n_in, merge=False):
        E, bs = 128, 16
        maxB = -(-S // bs)
        P = W * maxB
        bt = torch.randperm(P, generator=g).to(torch.int32).reshape(W, maxB).to(device)
        kc = torch.empty(P, bs, Hkv, E, dtype=torch.bfloat16, device=device)
        vc = torch.empty_like(kc)
        pos = torch.arange(S, dtype=torch.int32).repeat(W, 1).to(device)
        ins = []
        for _ in range(n_in):
            k = torch.randn(W, S, Hkv, E, device=device).to(torch.bfloat16).transpose(1, 2)  # k_proj view
            v = torch.randn(W, S, Hkv, E, device=device).to(torch.bfloat16).transpose(1, 2)
            c = torch.rand(1 if merge else W, cos_rows, 128, device=device)
            ins.append((k, v, c, c.clone()))

        def fn(j):
            k, v, c, sn = ins[j]
            dv.dvattn_paged_kv_append(k, v, pos, c, sn, kc, vc, bt)

        us, eager = _time_calls(fn, n_in, steps, warmup)
        kv = W * S * Hkv * E * 2
        alg = 4 * kv + 2 * ins[0][2].numel() * 4 + W * S * 4 + W * maxB * 4
        rows.append({"row": name, "us_per_call": round(us, 2), "us_per_call_eager": round(eager, 2), "alg_bytes": alg,
                     "achieved_GBs": round(alg / (us * 1e-6) / 1e9, 1),
                     "hbm_frac": round(alg / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
        del ins, kc, vc

    append_case("kv_append_decode_cfg2 (W=32,S=1,Hkv=8)", 32, 1, 8, 1, 4)
    append_case("kv_append_prefill (W=1,S=8192,Hkv=8)", 1, 8192, 8, 8192, 4)
    append_case("merge_caches (L=32768,Hkv=8, one cos/sin row)", 1, 32768, 8, 1, 2, merge=True)
    F, W, S, R = 4, 32, 1, 128
    fl = torch.tensor([4096, 512, 2048, 1], dtype=torch.int32, device=device)
    order = torch.stack([torch.randperm(F, generator=g) for _ in range(W)]).to(torch.int32).to(device)
    inv = (1.0 / (1e4 ** (torch.arange(0, R, 2, dtype=torch.float) / R))).to(device)
    loc = torch.empty(F, W, S, dtype=torch.int32, device=device)
    cos = torch.empty(F, W, S, R, device=device)
    sin = torch.empty_like(cos)
    us, eager = _time_calls(
        lambda j: torch.ops.libdvatt.dvattn_view_metadata(loc, cos, sin, fl, order, inv, 1.0, None), 1, steps, warmup)
    alg = F * 4 + W * F * 4 + R // 2 * 4 + loc.numel() * 4 + 2 * cos.numel() * 4
    rows.append({"row": f"view_metadata (F={F},W={W},S={S},R={R})", "us_per_call": round(us, 2),
                 "us_per_call_eager": round(eager, 2), "alg_bytes": alg,
                 "achieved_GBs": round(alg / (us * 1e-6) / 1e9, 1),
                 "hbm_frac": round(alg / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
    torch.cuda.empty_cache()
    return rows


def measure_copy(device, nbytes: int = 1 << 30, reps: int = 10) -> float:
    """Achievable HBM rate of a plain device-to-device copy (read + write bytes / time)."""
    src = torch.empty(nbytes, dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        dst.copy_(src)
    b.record()
    torch.cuda.synchronize()
    gbs = 2 * nbytes * reps / (a.elapsed_time(b) * 1e-3) / 1e9
    del src, dst
    torch.cuda.empty_cache()
    return gbs


def cpu_baseline(device, budget_s: float = 10.0) -> dict:
    """The CPU oracle (fp32 torch-CPU restatement of the reference's eager path,
    attention.py:309-312, plus the page-table gather) on the full configuration 2
    input: one warm-up, then repeated runs for about ``budget_s`` seconds; the
    median run time gives the rate."""
    from dvattention_amd import workloads as WL
    from oracle import dvattn_oracle as O
    # every core of the host (the CPU baseline's protocol: all cores the
    # process may use): os.cpu_count(), which on the MI355X box equals its
    # scheduler affinity and its cgroup CPU quota
    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else cores
    quota = None
    try:
        q, period = open("/sys/fs/cgroup/cpu.max").read().split()
        quota = None if q == "max" else round(int(q) / int(period), 2)
    except (OSError, ValueError):
        pass
    wl = WL.config(2, device="cpu", seed=1234)
    t = wl.t

    def once():
        t0 = time.perf_counter()
        O.paged_sdpa(wl.scale, t["locations"], t["queries"], t["cosines"], t["sines"], t["fragment_lengths"],
                     t["k_cache"], t["v_cache"], t["block_tables"])
        return time.perf_counter() - t0

    once()
    runs = []
    while sum(runs) < budget_s or len(runs) < 3:
        runs.append(once())
    runs.sort()
    med = runs[len(runs) // 2]
    cpu_model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": round(wl.alg_bytes / med / 1e12, 6),
        "unit": "TB/s",
        "cores": cores,
        "kind": "port",
        "host_cpus": {"cpu_count": os.cpu_count(), "affinity": avail, "cgroup_quota": quota,
                      "model": cpu_model or platform.processor()},
        "sample": f"full config 2 input ({wl.alg_bytes / 1e6:.0f} MB algorithmic), median of {len(runs)} runs = "
                  f"{med * 1e3:.1f} ms/call, fp32 torch-CPU oracle on {cores} threads, "
                  f"{cpu_model or platform.processor()}, torch {torch.__version__}",
    }


def main() -> int:
    global PREWARM_MS
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--configs", default="1,2,2u,3,4,5,5v,5f")
    ap.add_argument("--prewarm-ms", type=float, default=PREWARM_MS,
                    help="wall-clock ms of untimed calls before each timed region, besides --warmup "
                         "(the GPU clock's ramp from idle; 0: exactly --warmup steps)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-cache-rows", action="store_true", help="skip the K-side append / view metadata rows")
    ap.add_argument("--read-ceiling", action="store_true",
                    help="only the paged-read probe on configurations 2 and 4 (one JSON line)")
    ap.add_argument("--mfma-ceiling", action="store_true",
                    help="only the MFMA rate probe, alone and with other VALU work per MFMA (one JSON line)")
    ap.add_argument("--small-crossover", action="store_true",
                    help="only the single-launch vs general path timings of dvattn_fused (one JSON line)")
    args = ap.parse_args()
    PREWARM_MS = args.prewarm_ms
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the operator has no multi-GPU path); "
              "run with --gpus 1", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py: no HIP device visible", file=sys.stderr)
        return 2
    import dvattention_amd  # noqa: F401  (loads the HIP libraries; fails loudly if missing)
    device = torch.device("cuda", 0)
    if args.read_ceiling:
        rows = []
        for i in (2, 4):
            rows.append(read_ceiling(i, args.steps, args.warmup, device))
            dec = time_config(i, args.steps, args.warmup, device)
            rows[-1]["decode_us_per_call"] = dec["us_per_call"]
            rows[-1]["decode_kernel_us"] = dec["kernel_us_mean"]
            log(f"[bench] read probe cfg{i}: {rows[-1]['probe_us_per_call']} us/call, {rows[-1]['read_GBs']} GB/s "
                f"(decode {dec['us_per_call']} us/call)")
        plain = plain_read(device)
        log(f"[bench] plain streaming read of {plain['bytes'] >> 30} GiB: {plain['nontemporal_GBs']} GB/s "
            f"non-temporal, {plain['default_GBs']} GB/s default policy")
        print(json.dumps({"read_ceiling": rows, "plain_read": plain}), flush=True)
        return 0
    if args.small_crossover:
        print(json.dumps({"small_crossover": small_crossover(device)}), flush=True)
        return 0
    if args.mfma_ceiling:
        res = mfma_ceiling(device)
        for r in res["rows"]:
            log(f"[bench] mfma {r['shape']} bf16 + {r['other_per_mfma']} {r['kind']}/MFMA: {r['tflops']} TFLOP/s at "
                f"{r['clock_mhz']} MHz, {r['simd_cycles_per_mfma']} SIMD cycles per MFMA")
        print(json.dumps({"mfma_ceiling": res}), flush=True)
        return 0
    cfgs = [x if x in ("5v", "2u", "5f") else int(x) for x in args.configs.split(",") if x]
    if 2 not in cfgs:
        cfgs = [2] + cfgs
    per = {}
    for i in cfgs:
        r = time_config(i, args.steps, args.warmup, device, exact=(i == 2))
        per[i] = r
        log(f"[bench] cfg{i} {r['workload']}: {r['us_per_call']} us/call (events, back-to-back), "
            f"kernel {r['kernel_us_mean']} us, {r['achieved_GBs']} GB/s = {100 * r['hbm_frac']:.1f}% HBM, "
            f"{r['achieved_TFLOPs']} TFLOP/s")
    cache_rows = [] if args.no_cache_rows else time_cache_rows(device, args.steps, args.warmup)
    for r in cache_rows:
        log(f"[bench] {r['row']}: {r['us_per_call']} us/call in a graph ({r['us_per_call_eager']} eager), "
            f"{r['achieved_GBs']} GB/s = {100 * r['hbm_frac']:.1f}% HBM")
    head = per[2]
    # HBM bytes per call from the committed rocprofv3 --pmc summary (FETCH_SIZE / WRITE_SIZE
    # scaled by a 1 GiB copy); absent -> null
    traffic = {}
    tpath = os.path.join(HERE, "profiles", "hbm_traffic_configs2-5.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = next((t for t in json.load(f) if t.get("config") == head["config"]), {})
    copy_gbs = measure_copy(device)
    log(f"[bench] device copy (1 GiB read + 1 GiB write): {copy_gbs:.0f} GB/s")
    ceiling = read_ceiling(2, args.steps, args.warmup, device)
    log(f"[bench] read probe cfg2 (decode access pattern, no compute): {ceiling['probe_us_per_call']} us/call, "
        f"{ceiling['read_GBs']} GB/s")
    cpu = None if args.no_cpu else cpu_baseline(device)
    line = {
        "metric": METRIC,
        "value": round(head["alg_bytes"] / (head["us_per_call"] * 1e-6) / 1e12, 4),
        "unit": "TB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "prewarm_ms": args.prewarm_ms,
        "ms_per_step": round(head["us_per_call"] / 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/k/v, random page permutation)",
        "config": {"workload": head["workload"], "op": "dvattn_paged_sdpa", "batch": 32, "kv_heads": 8,
                   "q_heads": 128, "head_dim": 128, "page_size": 16, "kv_len": "U[1024,8192]",
                   "rotary_dim": 128, "replicas": head["replicas"]},
        "roofline": {"bound": "hbm", "achieved": round(head["alg_bytes"] / (head["us_per_call"] * 1e-6) / 1e9, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(head["alg_bytes"] / (head["us_per_call"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                     "traffic": traffic.get("traffic_bytes_per_call"),
                     "traffic_source": traffic.get("source"),
                     "kernel": "dv_stream + dv_merge (one call)", "alg_bytes_per_launch": head["alg_bytes"],
                     "launch_us": head["us_per_call"], "launch_us_source": "back-to-back timed region, per call",
                     "launch_us_single_events": head["kernel_us_mean"], "copy_GBs": round(copy_gbs, 1),
                     "read_ceiling": ceiling},
        "cpu_baseline": cpu,
        "per_config": [per[i] for i in sorted(per, key=str)],
        "cache_rows": cache_rows,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
