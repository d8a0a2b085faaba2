#!/usr/bin/env python3
"""Decode benchmarks of the MI355X path on one GPU.

Default workload (the metric's): the config-3 Qwen3-style MoE layer at batch
1 -- d_model 2048, 128 experts, expert d_ffn 768, top-8, fp32 router, Q4_K
expert weights, SiLU, renormalised top-k weights.  One step = one token
through the layer (router -> softmax / top-k -> expert gate/up -> down ->
weighted combine), inputs resident in HBM.

Other workloads (--workload): cfg1 dense Q8_0 FFN (896 -> 4864 -> 896), cfg2
Q4_K matvec 4096 x 4096, cfg2b Q6_K matvec 151936 x 1024 (K padded from
896), cfg4 Gemma4-A4B-like layer (Q8_0 router and shared FFN, Q4_K experts),
prefill (config 5, 512 tokens), gemma4 (the config-4 layer inside the Gemma4
block), formats (the APEX expert formats on a large dense matvec).

Measurement (every workload):
  * Weight copies are rotated so that the bytes of one rotation exceed the
    256 MB Infinity Cache, and (decode layers) the input x cycles through a
    pool so the selected experts change from step to step.
  * The timed steps replay hipGraphs of G captured steps; every graph is
    launched twice before timing.  At least 256 steps are timed whatever
    --steps says (more when --steps asks); `steps` is the count timed,
    `steps_requested` what was asked.  `value` is host wall time per step
    around the replays; `device_us_per_step` is the HIP-event time on the
    library's stream over the same replays.
  * roofline: the dominant kernel's mean launch duration from back-to-back
    launches between one HIP event pair on the library stream; achieved =
    algorithmic bytes per launch / that duration.  traffic = HBM bytes per
    launch from rocprofv3 FETCH_SIZE + WRITE_SIZE runs committed under
    profiles/ (scaled by the counters' reading on a copy of known size), or
    null when no counter summary exists for the workload; traffic_gbps =
    those bytes over the same launch duration (the counter-side GB/s).
  * cpu_baseline: the oracle's restatement of the reference CPU path
    (quantMatvecPar row split over a persistent pool + moeForward) on this
    host, min(usable cores, 64) threads (the reference's job arrays hold 64),
    on a bounded sample of the same inputs; a 1-thread figure too.

Prints one JSON line on stdout; progress goes to stderr.
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
sys.path[:0] = [os.path.join(ROOT, "llmtoy-zig_amd"), os.path.join(ROOT, "oracle")]

METRIC = "MoE-layer decode µs/token + achieved HBM GB/s (% of 8 TB/s) at batch 1"
PEAK_GBPS = 8000.0
MIN_TIMED_STEPS = 256
D, E, F, K = 2048, 128, 768, 8
Q4K_ROW_D = (D // 256) * 144          # 1152 B: one gate or up row
Q4K_ROW_F = (F // 256) * 144          # 432 B: one down row
EXPERT_BYTES = 2 * F * Q4K_ROW_D + D * Q4K_ROW_F      # 2,654,208 B per expert
SELECTED_BYTES = K * EXPERT_BYTES                      # 21,233,664 B (metric denominator)
LAYER_BYTES = SELECTED_BYTES + E * D * 4 + 4 * D * 4   # + fp32 router + x/out/h traffic -> 22,347,776 B
FUSED_BYTES = SELECTED_BYTES + E * D * 4 + 2 * D * 4    # + router + x + out = 22,298,624 B per launch
GATE_UP_WEIGHT_BYTES = K * 2 * F * Q4K_ROW_D           # 14,155,776 B
GATE_UP_BYTES = GATE_UP_WEIGHT_BYTES + D * 4 + K * F * 4   # + x read + h write = 14,188,544 B
DOWN_BYTES = K * D * Q4K_ROW_F + K * F * 4 + D * 4          # 7,077,888 + h + out
DTYPE_Q4K_DECODE = ("Q4_K weights x fp32 activations split into two int8 limbs per 16-element group "
                    "(v_dot4 int32 dots), fp32 scales and accumulation; fp32 router in dotf32 order")


def log(msg: str):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_threads(args) -> int:
    """min(usable cores, 64): the cores this process may run on (the box's
    share, not the whole host), capped at the reference's 64 job slots
    (ops/math.zig:300)."""
    if args.cpu_threads:
        return args.cpu_threads
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, 64))


def cpu_info() -> dict:
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next(l.split(":", 1)[1].strip() for l in f if l.startswith("model name"))
    except (OSError, StopIteration):
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = None
    return {"nproc": os.cpu_count(), "usable_cores": usable, "cpu_model": model}


def pmc_traffic(name: str):
    """HBM bytes per launch of the dominant kernel from a committed rocprofv3
    counter summary (profiles/<name>_pmc.json), and its path."""
    path = os.path.join(ROOT, "profiles", f"{name}_pmc.json")
    if not os.path.exists(path):
        return None, None
    with open(path) as f:
        p = json.load(f)
    try:
        fetch = p["kernels"][p["dominant"]]["FETCH_SIZE_kib"] / p["copy_calibration"]["fetch_factor"]
        write = p["kernels"][p["dominant"]]["WRITE_SIZE_kib"] / p["copy_calibration"]["write_factor"]
        return (fetch + write) * 1024.0, os.path.relpath(path, ROOT)
    except (KeyError, ZeroDivisionError):
        return None, os.path.relpath(path, ROOT)


def roofline(kernel: str, algo_bytes: int, mean_us: float, pmc_name: str | None, iters: int) -> dict:
    gbps = algo_bytes / (mean_us * 1e-6) / 1e9
    traffic, src = pmc_traffic(pmc_name) if pmc_name else (None, None)
    r = {"bound": "hbm", "achieved": round(gbps, 1), "peak": PEAK_GBPS, "unit": "GB/s",
         "frac": round(gbps / PEAK_GBPS, 4), "traffic": None if traffic is None else round(traffic),
         "kernel": kernel, "algorithmic_bytes": algo_bytes, "mean_launch_us": round(mean_us, 3),
         "timing": f"{iters} back-to-back launches, one HIP event pair on the library stream"}
    r["traffic_source"] = (f"committed counters {src} (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE per dispatch, "
                           "scaled by a 256 MiB copy), not measured in this run") if traffic is not None else None
    # the second derivation: counter bytes (FETCH + WRITE) over the same launch time
    r["traffic_gbps"] = None if traffic is None else round(traffic / (mean_us * 1e-6) / 1e9, 1)
    return r


class Timer:
    """Graph replay timing on the library's stream."""

    def __init__(self, stream):
        self.stream = stream

    def graph_steps(self, step, n_steps: int, G: int = 64):
        """Capture G consecutive steps into one graph, launch it twice
        (warm), then time ceil(n_steps / G) launches: host wall clock and a
        HIP event pair on the stream.  Returns (wall us/step, device
        us/step, steps timed)."""
        from llmtoy_amd.hip import Event, Graph, sync_stream
        graph = Graph(self.stream, lambda: [step(i) for i in range(G)])
        graph.launch()
        graph.launch()
        sync_stream(self.stream)
        n_graphs = max(1, math.ceil(n_steps / G))
        e0, e1 = Event(), Event()
        t = time.perf_counter()
        e0.record(self.stream)
        for _ in range(n_graphs):
            graph.launch()
        e1.record(self.stream)
        sync_stream(self.stream)
        wall = time.perf_counter() - t
        steps = n_graphs * G
        dev = e0.elapsed_ms(e1) * 1e3 / steps
        graph.destroy()
        e0.destroy()
        e1.destroy()
        return wall / steps * 1e6, dev, steps

    def launches(self, fn, n: int) -> float:
        """Mean launch duration: n back-to-back launches between one HIP
        event pair on the library's stream (per-launch event pairs would add
        their own overhead to every launch)."""
        from llmtoy_amd.hip import Event, sync_stream
        for i in range(min(n, 32)):
            fn(i)
        sync_stream(self.stream)
        a, b = Event(), Event()
        a.record(self.stream)
        for i in range(n):
            fn(i)
        b.record(self.stream)
        sync_stream(self.stream)
        us = a.elapsed_ms(b) * 1e3 / n
        a.destroy()
        b.destroy()
        return us


def rnd(v, n=3):
    return None if v is None else round(v, n)


def timed_steps(args) -> int:
    return max(args.steps or 0, MIN_TIMED_STEPS)


def base_record(args, metric, value, unit, steps, higher_is_better, dtype, config, extra=None) -> dict:
    r = {"metric": metric, "value": value, "unit": unit, "n_gpus": 1, "steps": steps,
         "steps_requested": args.steps, "warmup": args.warmup, "higher_is_better": higher_is_better,
         "scaling": "weak", "vs_baseline": None, "dtype": dtype, "data": "synthetic (seeded; BASELINE value scheme)",
         "config": config}
    if extra:
        r.update(extra)
    return r


def cpu_sample(fn, seconds: float, min_n: int = 20, max_n: int = 5000):
    """Median seconds per call of fn(i) over a time-bounded sample."""
    fn(0)
    ts, t_end, i = [], time.perf_counter() + seconds, 0
    while (time.perf_counter() < t_end or len(ts) < min_n) and len(ts) < max_n:
        t0 = time.perf_counter()
        fn(i)
        ts.append(time.perf_counter() - t0)
        i += 1
    return statistics.median(ts), len(ts)


def cpu_baseline_record(args, fn_for_pool, unit_scale, unit, what):
    """Times fn(pool)(i) with min(usable cores, 64) threads and 1 thread."""
    import pyoracle as orc
    nt = cpu_threads(args)
    res = {}
    for threads, budget in ((nt, args.cpu_seconds), (1, max(2.0, args.cpu_seconds / 4))):
        with orc.Pool(threads) as pool:
            med, n = cpu_sample(fn_for_pool(pool), budget)
        res[threads] = (med * unit_scale, n)
        log(f"cpu baseline {threads} thread(s): {res[threads][0]:.1f} {unit} over {n} calls")
        if threads == 1:
            break
    rec = {"value": round(res[nt][0], 2), "unit": unit, "cores": nt, "kind": "port",
           "sample": f"{res[nt][1]} calls, median; {what}, --threads {nt}",
           "value_1_thread": round(res[1][0], 2)}
    rec.update(cpu_info())
    return rec


# ------------------------------------------------------------------ config 3 (default)
def calibrate_copy(ctx, nbytes=256 << 20):
    """A device-to-device copy of known size (the runtime's copy kernel), for
    scaling the FETCH_SIZE / WRITE_SIZE counters in a rocprofv3 --pmc run."""
    from llmtoy_amd.hip import D2D, DeviceArray, check, hip
    a, b = DeviceArray((nbytes // 4,), "float32"), DeviceArray((nbytes // 4,), "float32")
    for _ in range(3):
        check(hip().hipMemcpy(b.ptr, a.ptr, nbytes, D2D), "hipMemcpy D2D")
    a.free()
    b.free()
    log(f"calibration: 3 x {nbytes >> 20} MiB device copies")


def gguf_load(ctx, w, x, base):
    """The config-3 layer written to a GGUF file, read back through the GGUF
    reader (mapped, parsed, tensors viewed in place) and uploaded: parse and
    upload times, and whether the decode output from the file's tensors is
    bit-identical to the output from the in-memory weights."""
    import tempfile

    import numpy as np

    import llmtoy_amd as lt
    from llmtoy_amd import gguf

    with tempfile.TemporaryDirectory() as td:
        path = gguf.write_moe_layer(os.path.join(td, "cfg3_layer.gguf"), w, k=K)
        t = time.perf_counter()
        r = gguf.GgufReader(path)
        cfg = gguf.moe_config(r)
        L = gguf.load_moe_layer(r, 0, cfg)
        parse_ms = (time.perf_counter() - t) * 1e3
        t = time.perf_counter()
        tens = lt.upload_moe(ctx, L)
        ctx.sync()
        upload_s = time.perf_counter() - t
        outs = []
        for tt in (tens, base):
            o = np.zeros(D, np.float32)
            ctx.moe_forward(o, x, *tt, cfg.n_experts_used, cfg.d_expert, norm_topk=True, deterministic=True)
            outs.append(o)
        nbytes = sum(tt.nbytes for tt in tens)
        for tt in tens:
            tt.free()
        t = time.perf_counter()
        tens = lt.upload_moe(ctx, w)
        ctx.sync()
        mem_s = time.perf_counter() - t
        for tt in tens:
            tt.free()
        res = {"file_bytes": os.path.getsize(path), "parse_ms": round(parse_ms, 3),
               "upload_ms": round(upload_s * 1e3, 2), "upload_gbps": round(nbytes / upload_s / 1e9, 2),
               "upload_gbps_from_memory": round(nbytes / mem_s / 1e9, 2),
               "output_bit_identical": bool(np.array_equal(outs[0], outs[1])),
               "note": "host->device over PCIe through pinned 4 MiB staging pieces, planes split on the device; "
                       "outside the timed decode"}
        del L, r
    return res


def bench_decode(args):
    import numpy as np

    import llmtoy_amd as lt
    import pyoracle as orc
    from llmtoy_amd import synth
    from llmtoy_amd.hip import DeviceArray, sync_stream

    t0 = time.time()
    log("generating config-3 weights (128 experts, Q4_K) ...")
    c = synth.config3()
    w = c["weights"]
    xs = [c["x"]] + [synth.config3_x(i) for i in range(1, args.xpool)]
    log(f"generated in {time.time() - t0:.1f}s; uploading {args.copies} copies")

    ctx = lt.Context(0)
    stream = ctx.stream
    timer = Timer(stream)
    base = lt.upload_moe(ctx, w)
    copies = [base] + [tuple(t.clone() for t in base) for _ in range(args.copies - 1)]
    dev_bytes = sum(t.nbytes for cp in copies for t in cp)
    log(f"{args.copies} weight copies resident: {dev_bytes / 2**30:.2f} GiB")

    # parity of the benchmarked configuration against the oracle, both combines
    parity = {}
    with orc.Pool(min(16, cpu_threads(args))) as p:
        ref, rids, _, _ = orc.moe_forward(w, xs[0], K, norm_topk=True, pool=p)
    for det in (False, True):
        out_h = np.zeros(D, np.float32)
        ids_h = np.zeros(K, np.uint32)
        ctx.moe_forward(out_h, xs[0], *base, K, F, norm_topk=True, out_ids=ids_h, deterministic=det)
        parity["deterministic" if det else "atomic"] = {
            "ids_bit_exact": bool(np.array_equal(ids_h, rids)),
            "rel_l2": float(np.linalg.norm(out_h - ref) / np.linalg.norm(ref))}
    log(f"parity: {parity}")
    gguf_res = None
    if not args.no_gguf:
        gguf_res = gguf_load(ctx, w, xs[0], base)
        log(f"GGUF file load: {gguf_res}")

    X = DeviceArray.from_numpy(np.stack(xs))
    out = DeviceArray((D,), np.float32)

    def step(i, det=False):
        r, g, d = copies[i % args.copies]
        ctx.moe_forward(out, X.row(i % args.xpool), r, g, d, K, F, norm_topk=True, deterministic=det)

    # ---- eager warmup + eager rate
    for i in range(args.warmup):
        step(i)
    sync_stream(stream)
    n_eager = 1024
    t = time.perf_counter()
    for i in range(n_eager):
        step(i)
    sync_stream(stream)
    eager_us = (time.perf_counter() - t) / n_eager * 1e6
    log(f"eager: {eager_us:.2f} us/token")

    # host buffers in and out (LT_HOST_IO: H2D of x, D2H of out, synchronous) -- PCIe-inclusive
    host_out = np.zeros(D, np.float32)
    for i in range(16):
        r, g, d = copies[i % args.copies]
        ctx.moe_forward(host_out, xs[i % args.xpool], r, g, d, K, F, norm_topk=True)
    n_host = 256
    t = time.perf_counter()
    for i in range(n_host):
        r, g, d = copies[i % args.copies]
        ctx.moe_forward(host_out, xs[i % args.xpool], r, g, d, K, F, norm_topk=True)
    host_io_us = (time.perf_counter() - t) / n_host * 1e6
    log(f"host-buffer (PCIe-inclusive) calls: {host_io_us:.2f} us/token")

    # ---- graph replay: one graph holds G consecutive steps (copy and x cycle with period G)
    G = int(np.lcm(args.copies, args.xpool))
    while G < 64:
        G *= 2
    n_steps = timed_steps(args)
    us_per_token, dev_us, steps = timer.graph_steps(step, n_steps, G)
    log(f"graph replay ({steps} steps): {us_per_token:.3f} us/token wall, {dev_us:.3f} us/token device")
    det_us = det_dev_us = None
    if not args.atomic_only:
        det_us, det_dev_us, _ = timer.graph_steps(lambda i: step(i, True), n_steps, G)
        log(f"deterministic (slot-order combine): {det_us:.3f} us/token wall, {det_dev_us:.3f} device")

    # ---- per-kernel launch durations
    ids_pool = []
    for i in range(args.xpool):
        ids = np.zeros(K, np.uint32)
        wt = np.zeros(K, np.float32)
        ctx.router_topk(base[0], xs[i], K, ids, wt, norm_topk=True)
        ids_pool.append((ids, wt))
    IDS = DeviceArray.from_numpy(np.stack([a for a, _ in ids_pool]))
    WTS = DeviceArray.from_numpy(np.stack([b for _, b in ids_pool]))
    H = DeviceArray((K, F), np.float32)
    dids = DeviceArray((K,), np.uint32)
    dw = DeviceArray((K,), np.float32)

    def gu(i):
        r, g, d = copies[i % args.copies]
        ctx.expert_gate_up_id(g, X.row(i % args.xpool), IDS.row(i % args.xpool), K, F, F, H)

    def dn(i):
        r, g, d = copies[i % args.copies]
        ctx.expert_down_id(d, H, IDS.row(i % args.xpool), WTS.row(i % args.xpool), K, out)

    def rt(i):
        r, g, d = copies[i % args.copies]
        ctx.router_topk(r, X.row(i % args.xpool), K, dids, dw, norm_topk=True)

    fu_mean = timer.launches(step, args.kernel_iters)
    fu_det_mean = None if args.atomic_only else timer.launches(lambda i: step(i, True), args.kernel_iters)
    gu_mean = timer.launches(gu, args.kernel_iters)
    dn_mean = timer.launches(dn, args.kernel_iters)
    rt_mean = timer.launches(rt, args.kernel_iters)
    log(f"fused layer kernel {fu_mean:.2f} us per launch ({fu_det_mean} deterministic); three-launch path "
        f"kernels alone: gate/up {gu_mean:.2f} us, down {dn_mean:.2f} us, router+topk {rt_mean:.2f} us")

    layer_gbps = SELECTED_BYTES / (us_per_token * 1e-6) / 1e9
    result = base_record(
        args, METRIC, round(us_per_token, 3), "us/token", steps, False, DTYPE_Q4K_DECODE,
        {"workload": "qwen3_moe_decode_cfg3", "d_model": D, "n_experts": E, "d_expert": F, "top_k": K,
         "expert_quant": "Q4_K", "router": "f32", "act": "silu", "norm_topk": True, "batch": 1,
         "weight_copies": args.copies, "x_pool": args.xpool, "graph_steps": G},
        {"ms_per_step": round(us_per_token / 1e3, 6),
         "achieved_gbps_selected_experts": round(layer_gbps, 1),
         "hbm_frac_selected_experts": round(layer_gbps / PEAK_GBPS, 4),
         "achieved_gbps_full_layer": round(LAYER_BYTES / (us_per_token * 1e-6) / 1e9, 1),
         "device_us_per_step": round(dev_us, 3),
         "deterministic_us_per_token": rnd(det_us),
         "deterministic_device_us_per_token": rnd(det_dev_us),
         "eager_us_per_token": round(eager_us, 3),
         "host_io_us_per_token": round(host_io_us, 3),
         "kernel_us": {"moe_fused": round(fu_mean, 3), "moe_fused_deterministic": rnd(fu_det_mean)},
         "unfused_kernel_us": {"router_topk": round(rt_mean, 3), "expert_gate_up": round(gu_mean, 3),
                               "expert_down": round(dn_mean, 3)},
         "unfused_kernel_gbps": {"expert_gate_up": round(GATE_UP_BYTES / (gu_mean * 1e-6) / 1e9, 1),
                                 "expert_down": round(DOWN_BYTES / (dn_mean * 1e-6) / 1e9, 1)},
         "roofline": roofline("k_moe_fused", FUSED_BYTES, fu_mean, "moe_fused_cfg3", args.kernel_iters),
         "parity": parity})
    if gguf_res is not None:
        result["gguf_load"] = gguf_res

    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline_record(
            args, lambda pool: (lambda i: orc.moe_forward(w, xs[i % len(xs)], K, norm_topk=True, pool=pool)),
            1e6, "us/token", f"config-3 tokens (x pool of {args.xpool}); oracle/lt_oracle.c quantMatvecPar + "
                             "moeForward")

    if args.calibrate:
        calibrate_copy(ctx)
    print(json.dumps(result), flush=True)
    for a in (X, out, IDS, WTS, H, dids, dw):
        a.free()
    for cp in copies:
        for tns in cp:
            tns.free()
    ctx.close()
    if args.timeline:
        timeline_report(args, w, xs)


def timeline_report(args, w, xs, n=200):
    """n decode steps in a context created with LT_PROFILE=timeline (rotated
    weight copies, x pool), each followed by lt_sync so that every launch's
    phase stamps are collected; writes lt_profile_report's text to the path."""
    import llmtoy_amd as lt
    from llmtoy_amd.hip import DeviceArray
    os.environ["LT_PROFILE"] = "timeline"
    try:
        ctx = lt.Context(0)
    finally:
        del os.environ["LT_PROFILE"]
    base = lt.upload_moe(ctx, w)
    copies = [base] + [tuple(t.clone() for t in base) for _ in range(args.copies - 1)]
    import numpy as np
    X = DeviceArray.from_numpy(np.stack(xs))
    out = DeviceArray((D,), np.float32)
    for i in range(n):
        ctx.moe_forward(out, X.row(i % len(xs)), *copies[i % args.copies], K, F, norm_topk=True)
        ctx.sync()
    rep = ctx.profile_report()
    head = (f"Command (GPU box, repo root): python3 {' '.join(sys.argv)}\n"
            f"Workload: config-3 decode layer, {n} eager launches, {args.copies} weight copies rotated, "
            f"x pool of {len(xs)}; LT_PROFILE=timeline adds one store per workgroup at its end.\n\n")
    with open(args.timeline, "w") as f:
        f.write(head + rep)
    log("timeline report:\n" + rep)
    X.free()
    out.free()
    for cp in copies:
        for t in cp:
            t.free()
    ctx.close()


# ------------------------------------------------------------------ configs 1, 2, 2b
MALL_BYTES = 256 << 20


def n_copies(bytes_per_copy: int, minimum: int = 2) -> int:
    """Copies whose total exceeds the Infinity Cache by a margin (>= 1.2x)."""
    return max(minimum, math.ceil(1.2 * MALL_BYTES / bytes_per_copy))


def bench_matvec(args):
    """Config 2 (Q4_K 4096 x 4096) or config 2b (Q6_K 151936 x 1024, K
    padded from 896): one matvec per step, rotated weight copies."""
    import numpy as np

    import llmtoy_amd as lt
    import pyoracle as orc
    from llmtoy_amd import ggml, synth
    from llmtoy_amd.hip import DeviceArray

    if args.workload == "cfg2":
        c, gtype, kname, wl = synth.config2(), ggml.Q4_K, "k_matvec_q4k", "q4k_matvec_cfg2"
    else:
        c, gtype, kname, wl = synth.config2_q6k(), ggml.Q6_K, "k_matvec_q6k", "q6k_matvec_cfg2b"
    rows, cols = c["rows"], c["cols"]
    ctx = lt.Context(0)
    timer = Timer(ctx.stream)
    t0 = ctx.upload(c["w"], gtype, rows, cols)
    nb = t0.nbytes
    copies = [t0] + [t0.clone() for _ in range(n_copies(nb) - 1)]
    log(f"{args.workload}: {rows} x {cols} {ggml.NAMES[gtype]}, {nb} B, {len(copies)} copies")
    # parity: the whole matvec against the oracle (rows split over the pool)
    y = np.zeros(rows, np.float32)
    ctx.quant_matvec(y, t0, c["x"])
    with orc.Pool(min(16, cpu_threads(args))) as p:
        ref = orc.quant_matvec(c["w"], gtype, c["x"], rows, cols, pool=p)
    parity = {"max_rel": float(np.max(np.abs(y - ref)) / np.max(np.abs(ref))),
              "rel_l2": float(np.linalg.norm(y - ref) / np.linalg.norm(ref))}
    log(f"parity: {parity}")
    X = DeviceArray.from_numpy(c["x"])
    Y = DeviceArray((rows,), np.float32)

    def step(i):
        ctx.quant_matvec(Y, copies[i % len(copies)], X)

    n_steps = timed_steps(args)
    G = 64
    us, dev_us, steps = timer.graph_steps(step, n_steps, G)
    mean = timer.launches(step, args.kernel_iters)
    algo = nb + cols * 4 + rows * 4
    useful = rows * c.get("valid_cols", cols) * 210 // 256 if gtype == ggml.Q6_K else nb
    log(f"{kname}: {us:.2f} us wall / {dev_us:.2f} device per matvec; {mean:.2f} us per launch, "
        f"{algo / (mean * 1e-6) / 1e9:.0f} GB/s")
    result = base_record(
        args, f"{ggml.NAMES[gtype]} matvec µs + achieved HBM GB/s at batch 1 ({rows} x {cols})", round(us, 3),
        "us/matvec", steps, False,
        f"{ggml.NAMES[gtype]} weights x fp32 activations split into two int8 limbs per 16-element group "
        "(v_dot4 int32 dots), fp32 scales and accumulation",
        {"workload": wl, "rows": rows, "cols": cols, "valid_cols": c.get("valid_cols", cols), "batch": 1,
         "weight_copies": len(copies), "graph_steps": G},
        {"device_us_per_step": round(dev_us, 3), "gbps_tensor_bytes": round(nb / (mean * 1e-6) / 1e9, 1),
         "useful_weight_bytes": useful,
         "roofline": roofline(kname, algo, mean, wl, args.kernel_iters), "parity": parity})
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline_record(
            args, lambda pool: (lambda i: orc.quant_matvec(c["w"], gtype, c["x"], rows, cols, pool=pool)), 1e6,
            "us/matvec", f"oracle quantMatvecPar ({ggml.NAMES[gtype]} dequantRow + dotf32 per row)")
    if args.calibrate:
        calibrate_copy(ctx)
    print(json.dumps(result), flush=True)
    X.free()
    Y.free()
    for t in copies:
        t.free()
    ctx.close()


# weights 13,891,584 B + activations 84,992 B (x and out, gate/up/h vectors written and read)
CFG1_BYTES = 13_976_576


def bench_ffn(args):
    """Config 1: dense Q8_0 FFN, Qwen2.5-0.5B shape (896 -> 4864 -> 896),
    out = Wd (SiLU(Wg x) * Wu x); one FFN per step, rotated weight copies."""
    import numpy as np

    import llmtoy_amd as lt
    import pyoracle as orc
    from llmtoy_amd import ggml, synth
    from llmtoy_amd.hip import DeviceArray

    c = synth.config1()
    Dm, Ff = c["d_model"], c["d_ffn"]
    ctx = lt.Context(0)
    timer = Timer(ctx.stream)
    base = (ctx.upload(c["w_gate"], ggml.Q8_0, Ff, Dm), ctx.upload(c["w_up"], ggml.Q8_0, Ff, Dm),
            ctx.upload(c["w_down"], ggml.Q8_0, Dm, Ff))
    nb = sum(t.nbytes for t in base)
    copies = [base] + [tuple(t.clone() for t in base) for _ in range(n_copies(nb) - 1)]
    log(f"cfg1: dense Q8_0 FFN {Dm} -> {Ff} -> {Dm}, {nb} B of weights, {len(copies)} copies")
    out_h = np.zeros(Dm, np.float32)
    ctx.ffn_dense(out_h, *base, c["x"], act=lt.ACT_SILU)
    with orc.Pool(min(16, cpu_threads(args))) as p:
        ref = orc.ffn_dense(c["w_gate"], c["w_up"], c["w_down"], orc.Q8_0, c["x"], Dm, Ff, pool=p)
    parity = {"rel_l2": float(np.linalg.norm(out_h - ref) / np.linalg.norm(ref))}
    log(f"parity: {parity}")
    X = DeviceArray.from_numpy(c["x"])
    Y = DeviceArray((Dm,), np.float32)

    def step(i):
        ctx.ffn_dense(Y, *copies[i % len(copies)], X, act=lt.ACT_SILU)

    n_steps = timed_steps(args)
    us, dev_us, steps = timer.graph_steps(step, n_steps, 64)
    mean = timer.launches(step, args.kernel_iters)
    algo = CFG1_BYTES
    log(f"cfg1: {us:.2f} us wall / {dev_us:.2f} device per FFN; {mean:.2f} us per call (one launch)")
    result = base_record(
        args, "Dense FFN decode µs/token + achieved HBM GB/s at batch 1 (Q8_0, 896 -> 4864 -> 896)",
        round(us, 3), "us/token", steps, False, "Q8_0 weights x fp32 activations, fp32 accumulation",
        {"workload": "dense_ffn_q8_0_cfg1", "d_model": Dm, "d_ffn": Ff, "act": "silu", "batch": 1,
         "weight_copies": len(copies), "graph_steps": 64},
        {"device_us_per_step": round(dev_us, 3),
         "roofline": roofline("k_ffn_fused", algo, mean, "dense_ffn_cfg1",
                              args.kernel_iters), "parity": parity})
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline_record(
            args, lambda pool: (lambda i: orc.ffn_dense(c["w_gate"], c["w_up"], c["w_down"], orc.Q8_0, c["x"], Dm,
                                                        Ff, pool=pool)),
            1e6, "us/token", "oracle ffn_dense: three quantMatvecPar calls (fused dotQ8_0)")
    if args.calibrate:
        calibrate_copy(ctx)
    print(json.dumps(result), flush=True)
    X.free()
    Y.free()
    for cp in copies:
        for t in cp:
            t.free()
    ctx.close()


# ------------------------------------------------------------------ config 4
G4_D, G4_E, G4_F, G4_KD, G4_S = 2816, 128, 704, 768, 2112
G4_EXPERT_BYTES = 2 * G4_F * (G4_D // 256) * 144 + G4_D * (G4_KD // 256) * 144  # 3,446,784 B
G4_ROUTER_BYTES = G4_E * (G4_D // 32) * 34                                        # 382,976 B
G4_SHARED_BYTES = 3 * G4_S * (G4_D // 32) * 34                                    # 18,957,312 B
CFG4_BYTES = K * G4_EXPERT_BYTES + G4_SHARED_BYTES + G4_ROUTER_BYTES + 34 * G4_D  # 47,010,304 B (x, out ~ 95,744)


def bench_cfg4(args):
    """Config 4: Gemma4-A4B-like layer through lt_moe_forward -- Q8_0 router,
    Q8_0 shared FFN (d_ffn 2112), 8 of 128 Q4_K experts (d_expert 704, down K
    padded to 768), GELU-tanh, softmax top-8 without renormalisation;
    out = shared(x) + sum_k p_k expert_k(x)."""
    import numpy as np

    import llmtoy_amd as lt
    import pyoracle as orc
    from llmtoy_amd import ggml, synth
    from llmtoy_amd.hip import DeviceArray

    c = synth.config4()
    w = c["weights"]
    Dm, S = w.d_model, c["d_shared"]
    ctx = lt.Context(0)
    timer = Timer(ctx.stream)

    def upload_all():
        r, g, d = lt.upload_moe(ctx, w)
        sh = (ctx.upload(c["sh_gate"], ggml.Q8_0, S, Dm), ctx.upload(c["sh_up"], ggml.Q8_0, S, Dm),
              ctx.upload(c["sh_down"], ggml.Q8_0, Dm, S))
        return (r, g, d) + sh

    base = upload_all()
    copies = [base] + [tuple(t.clone() for t in base) for _ in range(args.copies - 1)]
    xs = np.stack([c["x"]] + [synth.normal(synth.stream(4, 300 + i), (Dm,)) for i in range(1, args.xpool)])
    log(f"cfg4: {args.copies} copies of {sum(t.nbytes for t in base) / 2**20:.0f} MiB")
    parity = {}
    with orc.Pool(min(16, cpu_threads(args))) as pool:
        ref, rids, rw = orc.moe_layer_shared(w, xs[0], K, c["sh_gate"], c["sh_up"], c["sh_down"], S, pool=pool)
    for det in (False, True):
        out_h = np.zeros(Dm, np.float32)
        ids = np.zeros(K, np.uint32)
        ctx.moe_forward(out_h, xs[0], *base[:3], K, G4_F, act=lt.ACT_GELU_TANH, shared=base[3:], out_ids=ids,
                        deterministic=det)
        parity["deterministic" if det else "atomic"] = {
            "ids_bit_exact": bool(np.array_equal(ids, rids)),
            "rel_l2": float(np.linalg.norm(out_h - ref) / np.linalg.norm(ref))}
    log(f"parity: {parity}")
    X = DeviceArray.from_numpy(xs)
    out = DeviceArray((Dm,), np.float32)

    def step(i, det=False):
        t = copies[i % args.copies]
        ctx.moe_forward(out, X.row(i % args.xpool), *t[:3], K, G4_F, act=lt.ACT_GELU_TANH, shared=t[3:],
                        deterministic=det)

    for i in range(args.warmup):
        step(i)
    G = int(np.lcm(args.copies, args.xpool))
    while G < 64:
        G *= 2
    n_steps = timed_steps(args)
    us, dev_us, steps = timer.graph_steps(step, n_steps, G)
    det_us = det_dev_us = None
    if not args.atomic_only:
        det_us, det_dev_us, _ = timer.graph_steps(lambda i: step(i, True), n_steps, G)
    mean = timer.launches(step, args.kernel_iters)
    log(f"cfg4: {us:.2f} us/token wall, {dev_us:.2f} device, {mean:.2f} per call; deterministic {det_us}")
    result = base_record(
        args, "Gemma4-A4B-like MoE layer decode µs/token + achieved HBM GB/s at batch 1 (config 4)", round(us, 3),
        "us/token", steps, False,
        "Q4_K experts x fp32 activations in int8-limb pairs (v_dot4), Q8_0 router and shared FFN x fp32 "
        "activations; fp32 accumulation",
        {"workload": "gemma4_like_moe_cfg4", "d_model": Dm, "n_experts": G4_E, "d_expert": G4_F,
         "down_cols": G4_KD, "d_shared": S, "top_k": K, "router": "Q8_0", "shared_ffn": "Q8_0",
         "experts": "Q4_K", "act": "gelu_tanh", "norm_topk": False, "weight_copies": args.copies,
         "x_pool": args.xpool, "graph_steps": G},
        {"device_us_per_step": round(dev_us, 3), "deterministic_us_per_token": rnd(det_us),
         "deterministic_device_us_per_token": rnd(det_dev_us),
         "roofline": roofline("lt_moe_forward with shared FFN (whole call)", CFG4_BYTES, mean, "moe_fused_cfg4",
                              args.kernel_iters), "parity": parity})
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline_record(
            args, lambda pool: (lambda i: orc.moe_layer_shared(w, xs[i % len(xs)], K, c["sh_gate"], c["sh_up"],
                                                               c["sh_down"], S, pool=pool)),
            1e6, "us/token", "oracle moe_layer_shared (shared FFN + Q8_0 routerTopKSoftmax + expert loop)")
    if args.calibrate:
        calibrate_copy(ctx)
    print(json.dumps(result), flush=True)
    X.free()
    out.free()
    for cp in copies:
        for t in cp:
            t.free()
    ctx.close()
    if args.timeline:
        timeline_cfg4(args, c, w, xs)


def timeline_cfg4(args, c, w, xs, n=200):
    """The config-4 layer's phase timeline: n eager launches in a context
    created with LT_PROFILE=timeline (rotated weight copies, x pool), each
    followed by lt_sync; writes lt_profile_report's text to args.timeline."""
    import llmtoy_amd as lt
    from llmtoy_amd import ggml
    from llmtoy_amd.hip import DeviceArray
    import numpy as np
    os.environ["LT_PROFILE"] = "timeline"
    try:
        ctx = lt.Context(0)
    finally:
        del os.environ["LT_PROFILE"]
    Dm, S = w.d_model, c["d_shared"]
    base = lt.upload_moe(ctx, w) + (ctx.upload(c["sh_gate"], ggml.Q8_0, S, Dm),
                                    ctx.upload(c["sh_up"], ggml.Q8_0, S, Dm),
                                    ctx.upload(c["sh_down"], ggml.Q8_0, Dm, S))
    copies = [base] + [tuple(t.clone() for t in base) for _ in range(args.copies - 1)]
    X = DeviceArray.from_numpy(np.asarray(xs))
    out = DeviceArray((Dm,), np.float32)
    for i in range(n):
        t = copies[i % args.copies]
        ctx.moe_forward(out, X.row(i % len(xs)), *t[:3], K, G4_F, act=lt.ACT_GELU_TANH, shared=t[3:])
        ctx.sync()
    rep = ctx.profile_report()
    head = (f"Command (GPU box, repo root): python3 {' '.join(sys.argv)}\n"
            f"Workload: config-4 layer (shared FFN in the same launch), {n} eager launches, {args.copies} weight "
            f"copies rotated, x pool of {len(xs)}; LT_PROFILE=timeline adds one store per workgroup at its end.\n\n")
    with open(args.timeline, "w") as f:
        f.write(head + rep)
    log("timeline report:\n" + rep)
    X.free()
    out.free()
    for cp in copies:
        for t in cp:
            t.free()
    ctx.close()


# ------------------------------------------------------------------ config 5
PREFILL_FLOP = 512 * K * (2 * 2 * F * D + 2 * D * F)  # 38,654,705,664 (gate, up, down)


def bench_prefill(args):
    """Config-5 batched prefill (512 tokens): the MFMA path."""
    import numpy as np

    import llmtoy_amd as lt
    import pyoracle as orc
    from llmtoy_amd import synth
    from llmtoy_amd.hip import DeviceArray

    c = synth.config3()
    w = c["weights"]
    p = synth.config5(512, weights=w)
    ctx = lt.Context(0)
    timer = Timer(ctx.stream)
    base = lt.upload_moe(ctx, w)
    copies = [base] + [tuple(t.clone() for t in base) for _ in range(max(1, args.copies // 2) - 1)]
    out_h = np.zeros((512, D), np.float32)
    ctx.moe_prefill(out_h, p["X"], *base, K, F, norm_topk=True, bias=p["bias"])
    with orc.Pool(min(16, cpu_threads(args))) as pool:
        ref, _, _ = orc.moe_prefill(w, p["X"], K, norm_topk=True, bias=p["bias"], pool=pool)
    parity = {"rel_l2": float(np.linalg.norm(out_h - ref) / np.linalg.norm(ref))}
    X = DeviceArray.from_numpy(p["X"])
    B = DeviceArray.from_numpy(p["bias"])
    out = DeviceArray((512, D), np.float32)

    def call(i):
        ctx.moe_prefill(out, X, *copies[i % len(copies)], K, F, norm_topk=True, bias=B)

    for i in range(args.warmup):
        call(i)
    steps_req = max(args.steps or 0, 64)
    us, dev_us, steps = timer.graph_steps(call, steps_req, 16)
    result = base_record(
        args, "MoE-layer batched prefill tokens/s (config 5, 512 tokens)", round(512 / (us * 1e-6)), "tokens/s",
        steps, True, "f16 MFMA (Q4_K dequantised to f16 in LDS; X per-row power-of-two scaled to f16), fp32 accumulation",
        {"workload": "qwen3_moe_prefill_cfg5", "tokens": 512, "d_model": D, "n_experts": E, "d_expert": F,
         "top_k": K, "router_bias": "zipf(1.1)", "graph_steps": 16},
        {"ms_per_step": round(us / 1e3, 4), "us_per_call": round(us, 2), "device_us_per_call": round(dev_us, 2),
         "achieved_tflops": round(PREFILL_FLOP / (us * 1e-6) / 1e12, 2),
         "roofline": {"bound": "mfma", "achieved": round(PREFILL_FLOP / (dev_us * 1e-6) / 1e12, 2),
                      "peak": 2500.0, "unit": "TFLOP/s",
                      "frac": round(PREFILL_FLOP / (dev_us * 1e-6) / 1e12 / 2500.0, 4), "traffic": None,
                      "kernel": "whole prefill call (device time per call; f16 dense MFMA peak)",
                      "algorithmic_flops": PREFILL_FLOP},
         "parity": parity})
    if not args.no_cpu:
        # the reference prefills token by token: the oracle's per-token MoE
        # layer on the first 16 prompt rows per call
        X16 = np.ascontiguousarray(p["X"][:16])
        result["cpu_baseline"] = cpu_baseline_record(
            args, lambda pool: (lambda i: orc.moe_prefill(w, X16, K, norm_topk=True, bias=p["bias"], pool=pool)),
            1e6 / 16, "us/token", "oracle moe_prefill on 16 of the 512 tokens per call (per-token moeForward, "
            "quantMatvecPar)")
        result["cpu_baseline"]["tokens_per_s"] = round(1e6 / result["cpu_baseline"]["value"])
    if args.calibrate:
        calibrate_copy(ctx)
    print(json.dumps(result), flush=True)
    X.free()
    B.free()
    out.free()
    for cp in copies:
        for t in cp:
            t.free()
    ctx.close()


# ------------------------------------------------------------------ Gemma4 block
# selected experts + router + x read/written + dense + 5 norm vectors (4 x d, 1 x E)
G4_BLOCK_BYTES = K * G4_EXPERT_BYTES + G4_ROUTER_BYTES + 3 * G4_D * 4 + 4 * G4_D * 4 + G4_E * 4


def bench_gemma4(args):
    """Config-4 layer inside the Gemma4 block (router-input prep, Q8_0 router,
    Q4_K experts with down_exps_scale, GELU, MoE tail): one decode token per step."""
    import numpy as np

    import llmtoy_amd as lt
    import pyoracle as orc
    from llmtoy_amd import ggml, lib as ltlib, synth
    from llmtoy_amd.hip import DeviceArray

    c = synth.config4_block()
    if args.apex:  # the Gemma4 APEX expert formats: Q3_K gate/up, IQ4_NL down (K = d_expert, no padding)
        c["weights"] = synth.moe_weights(4, G4_D, G4_E, G4_F, router_type=ggml.Q8_0, gate_up_type=ggml.Q3_K,
                                         down_type=ggml.IQ4_NL)
    w, nm = c["weights"], c["norms"]
    ctx = lt.Context(0)
    timer = Timer(ctx.stream)
    base = lt.upload_moe(ctx, w)
    copies = [base] + [tuple(t.clone() for t in base) for _ in range(args.copies - 1)]
    xs = np.stack([c["x"]] + [synth.normal(synth.stream(4, 70 + i), (G4_D,)) for i in range(1, args.xpool)])
    parity = {}
    with orc.Pool(min(16, cpu_threads(args))) as pool:
        ref, rids, _ = orc.gemma4_moe_block(w, xs[0], c["dense_ffn"], K, nm, c["layer_output_scale"], c["eps"],
                                            pool=pool)
    for precise in (True, False):
        ids = np.zeros(K, np.uint32)
        got = ltlib.gemma4_moe_block(ctx, xs[0].copy(), c["dense_ffn"], *base, K, G4_F, nm, c["layer_output_scale"],
                                     c["eps"], precise=precise, out_ids=ids)
        parity["precise" if precise else "tree"] = {
            "ids_bit_exact": bool(np.array_equal(ids, rids)),
            "rel_l2": float(np.linalg.norm(got - ref) / np.linalg.norm(ref))}
    log(f"gemma4 block parity: {parity}")
    X = DeviceArray.from_numpy(xs)
    dense = DeviceArray.from_numpy(c["dense_ffn"])
    dn = {k: (DeviceArray.from_numpy(v) if v is not None else None) for k, v in nm.items()}

    def step(i):
        r, g, d = copies[i % args.copies]
        ltlib.gemma4_moe_block(ctx, X.row(i % args.xpool), dense, r, g, d, K, G4_F, dn, c["layer_output_scale"],
                               c["eps"])

    for i in range(args.warmup):
        step(i)
    G = 64
    us, dev_us, steps = timer.graph_steps(step, timed_steps(args), G)
    expert_bytes = (w.gate_up.nbytes + w.down.nbytes) // G4_E
    block_bytes = G4_BLOCK_BYTES - K * G4_EXPERT_BYTES + K * expert_bytes
    gbps = block_bytes / (dev_us * 1e-6) / 1e9
    log(f"gemma4 block: {us:.2f} us/token wall, {dev_us:.2f} us/token device, {gbps:.0f} GB/s")
    result = base_record(
        args, "Gemma4 MoE block decode us/token (config-4 layer + router-input prep + MoE tail)", round(us, 3),
        "us/token", steps, False,
        ("expert weights x fp32 activations in int8-limb pairs (v_dot4)" if args.apex else
         "Q4_K gate/up x fp32 activations in int8-limb pairs (v_dot4), Q4_K down x fp32 h")
        + ", Q8_0 router x fp32 activations; fp32 accumulation and norms",
        {"workload": "gemma4_moe_block_cfg4", "d_model": G4_D, "n_experts": G4_E, "d_expert": G4_F,
         "down_cols": w.down_cols, "top_k": K, "router": "Q8_0",
         "experts": f"{ggml.NAMES[w.gate_up_type]} gate/up, {ggml.NAMES[w.down_type]} down",
         "act": "gelu_tanh", "norm_sum": "tree", "weight_copies": args.copies, "x_pool": args.xpool,
         "graph_steps": G},
        {"ms_per_step": round(us / 1e3, 6), "device_us_per_step": round(dev_us, 3),
         "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": PEAK_GBPS, "unit": "GB/s",
                      "frac": round(gbps / PEAK_GBPS, 4), "traffic": None,
                      "kernel": "whole block (device time per token)", "algorithmic_bytes": block_bytes},
         "parity": parity})
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline_record(
            args, lambda pool: (lambda i: orc.gemma4_moe_block(w, xs[i % len(xs)], c["dense_ffn"], K, nm,
                                                               c["layer_output_scale"], c["eps"], pool=pool)),
            1e6, "us/token", "config-4 block tokens; oracle lto_gemma4_moe_block (quantMatvecPar rows)")
    print(json.dumps(result), flush=True)
    if args.timeline:
        timeline_gemma4(args, c, w, X, dense, dn)
    for a in [X, dense] + [v for v in dn.values() if v is not None]:
        a.free()


def timeline_gemma4(args, c, w, X, dense, dn, n=200):
    """The Gemma4 block's phase timeline: n eager launches in a context
    created with LT_PROFILE=timeline (rotated weight copies, the bench's x
    pool, which the block overwrites in place), each followed by lt_sync;
    writes lt_profile_report's text to args.timeline."""
    import llmtoy_amd as lt
    from llmtoy_amd import lib as ltlib
    os.environ["LT_PROFILE"] = "timeline"
    try:
        ctx = lt.Context(0)
    finally:
        del os.environ["LT_PROFILE"]
    base = lt.upload_moe(ctx, w)
    copies = [base] + [tuple(t.clone() for t in base) for _ in range(args.copies - 1)]
    for i in range(n):
        r, g, d = copies[i % len(copies)]
        ltlib.gemma4_moe_block(ctx, X.row(i % args.xpool), dense, r, g, d, K, G4_F, dn, c["layer_output_scale"],
                               c["eps"])
        ctx.sync()
    rep = ctx.profile_report()
    head = (f"Command (GPU box, repo root): python3 {' '.join(sys.argv)}\n"
            f"Workload: Gemma4 block (config-4 layer, router-input prep, MoE tail in the same launch), {n} eager "
            f"launches, {len(copies)} weight copies rotated, x pool of {args.xpool}; LT_PROFILE=timeline adds one "
            f"store per workgroup at its end.\n\n")
    with open(args.timeline, "w") as f:
        f.write(head + rep)
    log("timeline report:\n" + rep)
    for cp in copies:
        for t in cp:
            t.free()
    ctx.close()
    for cp in copies:
        for tns in cp:
            tns.free()
    ctx.close()


def bench_formats(args):
    """Dense matvec over the Gemma4 APEX expert formats (Q5_0, Q5_1, IQ4_NL,
    Q3_K) and Q4_K for comparison: one [131072 x 4096] matrix per format, two
    copies alternated so reads come from HBM; mean launch duration from a HIP
    event pair on the library stream around back-to-back launches."""
    import numpy as np

    import llmtoy_amd as lt
    import pyoracle as orc
    from llmtoy_amd import ggml, synth
    from llmtoy_amd.hip import DeviceArray

    rows, cols = 131072, 4096
    ctx = lt.Context(0)
    timer = Timer(ctx.stream)
    g = np.random.default_rng(7)
    x = synth.normal(g, (cols,))
    X = DeviceArray.from_numpy(x)
    Y = DeviceArray((rows,), np.float32)
    per = {}
    for gtype in (ggml.Q5_0, ggml.Q5_1, ggml.IQ4_NL, ggml.Q3_K, ggml.Q4_K):
        name = ggml.NAMES[gtype]
        m = np.concatenate([synth.quant_matrix(np.random.default_rng(100 + i), gtype, 8192, cols)
                            for i in range(rows // 8192)])
        t0 = ctx.upload(m, gtype, rows, cols)
        t1 = t0.clone()
        y = np.zeros(rows, np.float32)
        ctx.quant_matvec(y, t0, x)
        ref = orc.quant_matvec(m[:512], gtype, x, 512, cols)
        err = float(np.max(np.abs(y[:512] - ref)) / np.max(np.abs(ref)))
        nbytes = m.nbytes
        del m
        us = timer.launches(lambda i: ctx.quant_matvec(Y, (t0, t1)[i & 1], X), 64)
        gbps = (nbytes + cols * 4 + rows * 4) / (us * 1e-6) / 1e9
        per[name] = {"us": round(us, 2), "gbps": round(gbps, 1), "frac": round(gbps / PEAK_GBPS, 4),
                     "weight_bytes": nbytes, "max_rel_err": err}
        log(f"matvec {name} {rows}x{cols}: {us:.1f} us, {gbps:.0f} GB/s, parity max rel {err:.2e}")
        t0.free()
        t1.free()
    result = {"metric": "dense matvec GB/s per GGUF format (131072 x 4096, batch 1)", "unit": "GB/s",
              "value": per["Q3_K"]["gbps"], "higher_is_better": True, "n_gpus": 1,
              "dtype": "weights x fp32 activations split into two int8 limbs per 16-element group (v_dot4 int32 dots), fp32 scales and accumulation",
              "data": "synthetic", "config": {"workload": "matvec_formats", "rows": rows, "cols": cols},
              "per_format": per}
    print(json.dumps(result), flush=True)
    X.free()
    Y.free()
    ctx.close()


def bench_stream(args):
    """The read ceiling of one launch: lt_stream_read (16-byte loads, every
    load in flight before any is used, nothing else) over each config's
    algorithmic byte count, cold (each launch reads a fresh region of a 4 GiB
    buffer, far past the 256 MB Infinity Cache) and hot (the same region
    every launch).  Timed like the roofline figures of the other workloads:
    back-to-back launches between one HIP event pair, and graph replay."""
    from llmtoy_amd.hip import DeviceArray, check, hip
    import llmtoy_amd as lt
    import numpy as np

    ctx = lt.Context(0)
    timer = Timer(ctx.stream)
    total = 4 << 30
    buf = DeviceArray((total,), np.uint8)
    check(hip().hipMemset(buf.ptr, 1, total), "hipMemset")
    sizes = {"cfg2": 9469952, "cfg1": 13976576, "cfg3": FUSED_BYTES, "cfg4": CFG4_BYTES, "cfg2b": 128238080,
             "q4k_131072x4096": 131072 * 16 * 144}
    rows = {}
    for name, nb in sizes.items():
        nb = nb // 256 * 256
        nreg = total // nb
        for mode in ("cold", "hot"):
            def step(i, nb=nb, nreg=nreg, mode=mode):
                off = ((i * 7 + 3) % nreg) * nb if mode == "cold" else 0
                ctx.stream_read(buf.ptr + off, nb)
            mean = timer.launches(step, args.kernel_iters)
            wall, dev, _ = timer.graph_steps(step, timed_steps(args), 64)
            rows[f"{name}_{mode}"] = {"bytes": nb, "mean_launch_us": round(mean, 3), "graph_us": round(dev, 3),
                                      "gbps": round(nb / (mean * 1e-6) / 1e9, 1),
                                      "frac_of_8tbs": round(nb / (mean * 1e-6) / 1e9 / PEAK_GBPS, 4)}
            log(f"stream {name} {mode}: {nb} B {mean:.3f} us per launch, {rows[f'{name}_{mode}']['gbps']} GB/s")
    big = rows["cfg2b_cold"]
    result = base_record(
        args, "read ceiling of one launch: GB/s of a streaming read kernel (lt_stream_read)", big["gbps"], "GB/s",
        args.kernel_iters, True, "u8 (16-byte loads, no arithmetic)",
        {"workload": "stream_read", "buffer_bytes": total, "sizes": {k: v for k, v in sizes.items()}},
        {"rows": rows, "roofline": {"bound": "hbm", "achieved": big["gbps"], "peak": PEAK_GBPS, "unit": "GB/s",
                                    "frac": big["frac_of_8tbs"], "traffic": None, "kernel": "k_stream_read",
                                    "algorithmic_bytes": big["bytes"], "mean_launch_us": big["mean_launch_us"]}})
    print(json.dumps(result), flush=True)
    buf.free()
    ctx.close()


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help=f"timed steps (at least {MIN_TIMED_STEPS} are timed whatever this says)")
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--copies", type=int, default=8)
    ap.add_argument("--xpool", type=int, default=64)
    ap.add_argument("--kernel-iters", type=int, default=512)
    ap.add_argument("--cpu-threads", type=int, default=None)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-gguf", action="store_true", help="skip the GGUF file load + upload check")
    ap.add_argument("--atomic-only", action="store_true",
                    help="decode, cfg4: time the default (atomic) combine only, so that a kernel trace of the run holds "
                         "no slot-order-combine dispatches of the same kernel")
    ap.add_argument("--apex", action="store_true",
                    help="--workload gemma4 with the APEX expert formats (Q3_K gate/up, IQ4_NL down)")
    ap.add_argument("--workload", choices=["decode", "cfg1", "cfg2", "cfg2b", "cfg4", "prefill", "gemma4", "formats",
                                           "stream"],
                    default="decode")
    ap.add_argument("--calibrate", action="store_true",
                    help="finish with device copies of known size (for rocprofv3 --pmc scaling)")
    ap.add_argument("--timeline", metavar="PATH", default=None,
                    help="decode, cfg4, gemma4: afterwards run LT_PROFILE=timeline steps in a fresh context and "
                         "write the library's per-phase report to PATH")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); sharding the layer "
              "over several GPUs (experts split across them, one all-to-all of the routed activations each way) "
              "is a design, not something this build runs", file=sys.stderr)
        sys.exit(2)
    if args.warmup is None:
        args.warmup = 5 if args.workload == "prefill" else 64
    {"decode": bench_decode, "cfg1": bench_ffn, "cfg2": bench_matvec, "cfg2b": bench_matvec, "cfg4": bench_cfg4,
     "prefill": bench_prefill, "gemma4": bench_gemma4, "formats": bench_formats, "stream": bench_stream}[args.workload](args)


if __name__ == "__main__":
    main()
