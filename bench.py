#!/usr/bin/env python3
"""MoE-layer benchmark on one MI355X (gfx950).

One step = one call of rmda_moe_layer (router -> top-k -> ranks/offsets ->
permutation -> grouped SwiGLU gate_up GEMM -> grouped down GEMM -> combine)
over one batch of synthetic tokens already resident in HBM.  The default
workload is BASELINE configuration 3 (T=2048, d=2048, 128 experts, top-8,
I=768), the configuration the headline metric is quoted on.

Prints ONE JSON line.  Besides the driver's fields it carries
  roofline      the dominant kernel's algorithmic bytes (or FLOPs) per launch
                divided by its average duration, measured with hipEvents on
                the stream the kernels run on (the library's stage profiler);
  stages        every stage's average duration and achieved rate;
  gemm          grouped-GEMM FLOP rate against the dense fp16 MFMA peak and
                against the weight-streaming ceiling min(peak, BW * AI);
  cpu_baseline  the CPU oracle (a C restatement of the reference shaders)
                timed on this host on a bounded sample of the same workload;
  decode        (config-3 runs) BASELINE configuration 2, T=128, timed the
                same way: the weight-streaming regime's tokens/s and its two
                GEMMs' HBM GB/s;
  skew          (config-3 runs) BASELINE configuration 4 (Zipf-skewed load,
                the compute tile): tokens/s and the GEMMs' TFLOP/s against
                the dense fp16 MFMA peak;
  fine_shared   (config-3 runs) BASELINE configuration 5 (512 experts,
                top-10, shared expert);
  mixed_load    (config-3 runs) config 3's shape with four hot experts
                holding ~35% of the rows: the per-call tile choice against
                each tile forced for the whole call;
  teacher       (config-3 runs) the reference teacher's own MoE shape (d 2560,
                512 experts, top-10, width 640 + shared) at 2048 tokens: the
                fused layer with fp16 and with fp32 (slot-scaled)
                activations, and the reference-structured recording;
  fp32_activations  (config-3 runs) config 3 through the slot-scaled
                fp32-activation input;
  alternating_layers  (config-3 runs) configs 3 and 4 alternating on one
                context under the adaptive and the auto tile policy;
  dropin        (config-3 runs) the reference-equivalent stage entry points
                (route, scan, scatter into xp, combine, the grouped GEMM, the
                whole recording) on the same inputs: warm legs (inputs
                cache-resident) and cold legs (buffer sets rotated past the
                256 MB Infinity Cache) for the copy-shaped ones.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 3]
"""
import argparse
import json
import os
import re
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(REPO, "r-mda_amd"), REPO):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "MoE-layer tokens/sec at T=2048; grouped-GEMM % fp16 MFMA peak; HBM GB/s"
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E, published
PEAK_FP16_TFLOPS = 2500.0   # MI355X dense fp16 MFMA, published
TRAFFIC_FILE = os.path.join(REPO, "profiles", "gate_up_prefill_traffic.txt")


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=140)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--config", type=int, default=3, choices=range(1, 7),
                    help="BASELINE configuration (1-5), or 6: the reference teacher's own MoE shape")
    ap.add_argument("--cpu-tokens", type=int, default=None,
                    help="tokens in the CPU-baseline sample (default: sized for ~10-30 s)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-peaks", action="store_true", help="skip re-measuring the copy and GEMM peaks")
    ap.add_argument("--upload", action="store_true",
                    help="also time rmda_moe_upload_layer from a bf16 safetensors file of this config's layer")
    ap.add_argument("--calib-copy", action="store_true",
                    help="also run a device copy of known size (HBM counter calibration)")
    ap.add_argument("--stages", action="store_true", help="print the stage table to stderr")
    ap.add_argument("--hf-layout", action="store_true",
                    help="stream the HF-layout weights instead of the packed ones")
    ap.add_argument("--no-decode", action="store_true",
                    help="skip the config-2 (T=128 decode) weight-streaming line added to the config-3 run")
    ap.add_argument("--no-others", action="store_true",
                    help="skip the config-4 (skewed, compute tile) and config-5 lines added to the config-3 run")
    ap.add_argument("--no-dropin", action="store_true",
                    help="skip timing the reference-equivalent stage entry points (route, scan, scatter, combine)")
    ap.add_argument("--dropin-only", action="store_true",
                    help="time only the reference-equivalent stage entry points (config 3 inputs), for profiling")
    ap.add_argument("--transient", action="store_true",
                    help="before the warm-up, time each of the first 400 layer calls of this fresh process, "
                         "then 60 more after a 2 s idle (the GPU's warm-up transient)")
    ap.add_argument("--sustain", type=float, default=0.0, metavar="SECS",
                    help="after the warm-up, run the layer back to back for SECS seconds with amd-smi sampling "
                         "socket power and clocks, then profile the stages at that clock; prints that line only")
    return ap.parse_args()


def cpu_threads():
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


def read_traffic():
    """HBM bytes per gate_up launch from the committed PMC summary, or None."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", open(TRAFFIC_FILE).read(), re.M)
    return float(m.group(1)) if m else None


def cpu_baseline(inp, cfg, n_tokens, rounds=7):
    """The CPU oracle's layer (a C restatement of the reference shaders, with
    pthreads over tokens and pairs) timed on this host: warm-up, then `rounds`
    rounds, best and median, with the oracle's own per-stage wall clock.  A
    round routes all T tokens (router, top-k, offsets, ranks) and runs the
    expert FFNs and the combine for a sample of n_tokens of them, so a round
    takes seconds; tokens/s is over the sample.  A smaller sample on one
    thread gives the single-thread figure (the reference's bench discipline,
    src/bench.c:32-53,93-105)."""
    import numpy as np
    from oracle import oracle as orc
    from rmda_moe import inputs

    host = inputs.to_host(inp)
    T = cfg["rows"]
    n = min(n_tokens, T)
    sel = np.arange(0, T, max(1, T // n), dtype=np.uint32)[:n]
    th = cpu_threads()
    orc.lib()
    orc.layer(host, tile=1, rows_sel=sel[: max(1, n // 8)], threads=th)  # warm-up: pages, threads
    times, stages = [], []
    for _ in range(rounds):
        t0 = time.perf_counter()
        r = orc.layer(host, tile=1, rows_sel=sel, threads=th)
        times.append(time.perf_counter() - t0)
        stages.append(r["stage_ms"])
    times.sort()
    best, med = times[0], times[len(times) // 2]
    stage_med = {k: round(sorted(st[k] for st in stages)[len(stages) // 2], 2) for k in stages[0]}
    n1 = max(1, min(32, n))
    sel1 = sel[:: max(1, len(sel) // n1)][:n1]
    t0 = time.perf_counter()
    orc.layer(host, tile=1, rows_sel=sel1, threads=1)
    dt1 = time.perf_counter() - t0
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count() or 1
    return {
        "value": round(len(sel) / med, 2),
        "unit": "tokens/s",
        "cores": th,
        "kind": "port",
        "best_tokens/s": round(len(sel) / best, 2),
        "rounds": rounds,
        "best_s": round(best, 3),
        "median_s": round(med, 3),
        "stage_ms_median": stage_med,
        "host": {"cpu": model, "nproc": os.cpu_count(), "affinity": affinity, "threads_used": th},
        "sample": "per round: routing of all %d tokens, expert FFNs + combine for %d of them (every %d-th); "
                  "%d threads (the box's CPU share for one GPU is 16); median of %d rounds after a warm-up"
                  % (T, len(sel), max(1, T // n), th, rounds),
        "single_thread": {"value": round(len(sel1) / dt1, 2), "unit": "tokens/s",
                          "sample": "routing of all %d tokens + FFNs of %d, 1 thread, %.1f s" % (T, len(sel1), dt1)},
    }


def measure_peaks(torch):
    """This box's achievable peaks, re-measured as the reference measures
    them: a device copy timed as 2*bytes/t (src/probe_memory.c:41-63,86) and
    a large dense fp16 GEMM (rocBLAS/hipBLASLt through torch.matmul)."""
    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device="cuda")
    src.fill_(1)
    dst = torch.empty_like(src)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    for _ in range(2):
        dst.copy_(src)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(5):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    copy_gbs = 2 * n / (e0.elapsed_time(e1) / 5 * 1e-3) / 1e9
    del src, dst
    m = 8192
    a = torch.randn(m, m, dtype=torch.float16, device="cuda")
    b = torch.randn(m, m, dtype=torch.float16, device="cuda")
    for _ in range(2):
        c = a @ b
    torch.cuda.synchronize()
    e0.record()
    for _ in range(5):
        c = a @ b
    e1.record()
    torch.cuda.synchronize()
    tf = 2.0 * m ** 3 / (e0.elapsed_time(e1) / 5 * 1e-3) / 1e12
    del a, b, c
    # the vendor GEMM on the hot experts' shape of BASELINE config 4's
    # gate_up: ten experts of 2048 rows, d 2048 -> 2I 1536, as one batched
    # product on contiguous fp16 operands
    nb, mr, kd, nn = 10, 2048, 2048, 1536
    a = torch.randn(nb, mr, kd, dtype=torch.float16, device="cuda")
    b = torch.randn(nb, kd, nn, dtype=torch.float16, device="cuda").contiguous()
    for _ in range(2):
        c = torch.bmm(a, b)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(10):
        c = torch.bmm(a, b)
    e1.record()
    torch.cuda.synchronize()
    tf_hot = 2.0 * nb * mr * kd * nn / (e0.elapsed_time(e1) / 10 * 1e-3) / 1e12
    del a, b, c
    torch.cuda.empty_cache()
    return {"hbm_copy_GB/s": round(copy_gbs, 1), "hbm_copy": "1 GiB device copy, 2*bytes/t",
            "fp16_gemm_TFLOP/s": round(tf, 1), "fp16_gemm": "8192^3 torch.matmul",
            "fp16_gemm_hot_shape_TFLOP/s": round(tf_hot, 1),
            "fp16_gemm_hot_shape": "torch.bmm 10 x (2048 x 2048) x (2048 x 1536), contiguous operands"}


def measure_transient(step, torch, n=400, n_after=60, idle_s=2.0):
    """Per-call GPU time of the first n layer calls of a fresh process, one
    event between consecutive calls, then n_after calls after idle_s of
    idling.  Shows how long the GPU takes to reach its steady rate, and
    whether the slow calls return after an idle gap with every buffer already
    touched (which rules out first-touch and TLB costs)."""
    def run(k):
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(k + 1)]
        torch.cuda.synchronize()
        evs[0].record()
        for i in range(k):
            step()
            evs[i + 1].record()
        torch.cuda.synchronize()
        return [evs[i].elapsed_time(evs[i + 1]) for i in range(k)]

    first = run(n)
    time.sleep(idle_s)
    after = run(n_after)
    blocks = [first[a:a + 20] for a in range(0, n, 20)]
    return {"what": "per-call ms of the first %d calls of the process (before any warm-up), in blocks of 20, "
                    "then %d calls after %.0f s idle" % (n, n_after, idle_s),
            "block_mean_ms": [round(sum(b) / len(b), 4) for b in blocks],
            "block_min_ms": [round(min(b), 4) for b in blocks],
            "after_idle_ms": [round(x, 4) for x in after]}


def parse_smi(txt):
    """Socket power (W), the GFX clock of each XCD and the memory clock (MHz)
    from the text of `amd-smi metric --power --clock`; None when the text
    holds no socket power (amd-smi prints "N/A" where a sensor is missing)."""
    pw = re.search(r"SOCKET_POWER:\s*([0-9.]+)\s*W", txt)
    if pw is None:
        return None
    gfx = [float(v) for v in re.findall(r"GFX_\d+:\s*\n\s*CLK:\s*([0-9.]+)\s*MHz", txt)]
    mem = re.search(r"MEM_0:\s*\n\s*CLK:\s*([0-9.]+)\s*MHz", txt)
    return {"socket_W": float(pw.group(1)), "gfx_MHz": gfx, "mem_MHz": float(mem.group(1)) if mem else None}


def smi_sample():
    """parse_smi of GPU 0's current report, or None where amd-smi is missing
    or prints no power line."""
    import subprocess
    try:
        r = subprocess.run(["amd-smi", "metric", "-g", "0", "--power", "--clock"], capture_output=True, text=True,
                           timeout=30)
    except (OSError, subprocess.TimeoutExpired):
        return None
    return parse_smi(r.stdout)


def measure_sustained(step, ctx, torch, secs, prof_calls=200):
    """The layer run back to back for `secs` seconds (batches of 200 calls,
    one synchronisation each), with amd-smi sampled about once a second
    after the first two seconds: sustained ms per call, socket power and the
    GFX clock of each XCD (averaged over samples).  Then, still warm, the
    stage profiler over `prof_calls` calls: each stage's time at the
    sustained clock.  Shows whether a long run is held at the board's power
    limit, and by how much that lowers the clock."""
    import threading

    samples = []
    done = threading.Event()
    t_start = time.perf_counter()

    def sampler():
        while not done.wait(1.0):
            if time.perf_counter() - t_start >= 2.0:
                s = smi_sample()
                if s is not None:
                    samples.append(s)

    th = threading.Thread(target=sampler, daemon=True)
    th.start()
    n = 0
    ctx.sync()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < secs:
        for _ in range(200):
            step()
        ctx.sync()
        n += 200
    dt = time.perf_counter() - t0
    done.set()
    th.join()
    ctx.prof_begin()
    for _ in range(prof_calls):
        step()
    stage_ms, nc = ctx.prof_end()
    event_us = 1000.0 * ctx.prof_empty_ms() / max(nc, 1)
    res = {"seconds": round(dt, 2), "calls": n, "ms_per_call": round(1e3 * dt / n, 4),
           "stage_us": {k: round(1e3 * v / max(nc, 1) - event_us, 2) for k, v in stage_ms.items() if v > 0},
           "smi_samples": len(samples)}
    if samples:
        gfx = [sum(s["gfx_MHz"]) / len(s["gfx_MHz"]) for s in samples if s["gfx_MHz"]]
        res["socket_W_mean"] = round(sum(s["socket_W"] for s in samples) / len(samples), 1)
        res["socket_W_max"] = max(s["socket_W"] for s in samples)
        if gfx:
            res["gfx_MHz_mean"] = round(sum(gfx) / len(gfx), 1)
            res["gfx_MHz_min_xcd"] = min(min(s["gfx_MHz"]) for s in samples if s["gfx_MHz"])
        res["mem_MHz"] = samples[-1]["mem_MHz"]
    return res


def measure_config(ctx, torch, cfg_id, steps=100, warmup=50, policy=None, x32=False):
    """Another configuration on the same context, timed as the main line:
    the layer's rate, and each grouped GEMM's time, TFLOP/s and HBM GB/s
    against the published peaks (algorithmic work; experts touched counted
    from the run's routing).  cfg_id is a BASELINE configuration number or a
    configuration dict.  Config 2 is the weight-streaming regime
    (HBM-bound), config 4 the compute-bound one (hot experts).  policy: a
    tile policy for this measurement (the context's is restored after);
    x32: the fp32-activation input (slot-scaled)."""
    from rmda_moe import api, configs, inputs

    cfg = configs.CONFIGS[cfg_id] if isinstance(cfg_id, int) else cfg_id
    inp = inputs.make_inputs(ctx, cfg, seed=0)
    shape = inp["shape"]
    if x32:
        ws = torch.empty(api.workspace_bytes_x32(shape), dtype=torch.uint8, device="cuda")
        xf = inp["x"].float()
    else:
        ws = inputs.workspace_for(shape)
    out = torch.empty(shape["rows"], shape["d"], dtype=torch.float16, device="cuda")
    packed = ctx.pack_weights(shape, inp["w_router"], inp["w_gate_up"], inp["w_down"], inp["w_sh_gate_up"],
                              inp["w_sh_down"])
    if policy is not None:
        ctx.set_tile_policy(policy)

    def step():
        if x32:
            ctx.layer(shape, None, inp["w_router"], inp["bias"], None, None, None, None, out, ws, packed=packed,
                      x32=xf)
        else:
            ctx.layer(shape, inp["x"], inp["w_router"], inp["bias"], None, None, None, None, out, ws, packed=packed)

    for _ in range(warmup):
        step()
    ctx.sync()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    ctx.prof_begin()
    for _ in range(steps):
        step()
    stage_ms, n_prof = ctx.prof_end()
    event_us = 1000.0 * ctx.prof_empty_ms() / max(n_prof, 1)
    views = api.ws_views(shape, ws)
    counts = views["count"].cpu().numpy()
    hot = int(views["n_items_hot"].cpu().numpy()[0]) > 0
    work = configs.algorithmic_work(cfg, touched=int((counts > 0).sum()))
    res = {"workload": workload_name(cfg, shape, cfg_id if isinstance(cfg_id, int) else None) +
                       (", fp32 activations (slot-scaled)" if x32 else ""),
           "tokens/s": round(shape["rows"] / (ms * 1e-3), 1), "ms_per_step": round(ms, 5), "steps": steps,
           "experts_touched": int((counts > 0).sum()), "gemm_tile": "compute (hot experts)" if hot else "streaming"}
    hot_min = 256
    res["rows_on_hot_experts"] = round(float(counts[counts >= hot_min].sum()) / max(1, counts.sum()), 4)
    gemm_us = 0.0
    for k in ("gate_up", "down"):
        us = 1000.0 * stage_ms[k] / max(n_prof, 1) - event_us
        gemm_us += us
        gbs = work[k + "_bytes"] / (us * 1e-6) / 1e9
        tf = work[k + "_flops"] / (us * 1e-6) / 1e12
        res[k] = {"us": round(us, 2), "TFLOP/s": round(tf, 1), "frac_of_fp16_peak": round(tf / PEAK_FP16_TFLOPS, 4),
                  "GB/s": round(gbs, 1), "frac_of_hbm_peak": round(gbs / PEAK_HBM_GBS, 4)}
    tf = work["gemm_flops"] / (gemm_us * 1e-6) / 1e12
    res["gemm"] = {"us": round(gemm_us, 2), "TFLOP/s": round(tf, 1), "frac_of_fp16_peak": round(tf / PEAK_FP16_TFLOPS, 4)}
    if policy is not None:
        ctx.set_tile_policy(api.Context.TILE_ADAPTIVE)
    del inp, ws, out, packed
    torch.cuda.empty_cache()
    return res


def workload_name(cfg, shape, cfg_id=None):
    skew = {True: " skewed", "mixed": " mixed load"}.get(cfg.get("skew"), "")
    return "%s: T=%d d=%d experts=%d top-%d inter=%d shared=%d%s%s" % (
        cfg["name"], shape["rows"], shape["d"], shape["experts"], shape["topk"], shape["inter"], shape["shared"],
        skew, " (BASELINE config %d)" % cfg_id if cfg_id else "")


def measure_mixed(ctx, torch):
    """Config 3's shape with four hot experts holding ~35% of the rows (the
    rest on 124 cold experts): the per-call tile choice (the streaming tile,
    since the hot bucket holds under half the rows) against each tile forced
    for the whole call.  The gap is what a per-expert tile choice inside one
    call could win at most."""
    from rmda_moe import api, configs
    res = {"per_call_choice": measure_config(ctx, torch, configs.MIXED, policy=api.Context.TILE_ADAPTIVE),
           "stream_tile": measure_config(ctx, torch, configs.MIXED, policy=api.Context.TILE_STREAM),
           "compute_tile": measure_config(ctx, torch, configs.MIXED, policy=api.Context.TILE_HOT)}
    best = min(res["stream_tile"]["gemm"]["us"], res["compute_tile"]["gemm"]["us"])
    res["gemm_us_per_call_choice_over_best_forced"] = round(res["per_call_choice"]["gemm"]["us"] / best, 4)
    return res


def measure_alternating(ctx, torch, pairs=100, warmup=20):
    """Two layers on one context, config 3 (streaming tile) and config 4
    (compute tile) alternating call by call, as a model's layers would:
    ms per layer call under RMDA_TILE_ADAPTIVE (each layer's own last choice,
    keyed by its packed weights) and RMDA_TILE_AUTO (both tiles launched)."""
    from rmda_moe import api, configs, inputs
    L = []
    for k in (3, 4):
        inp = inputs.make_inputs(ctx, configs.CONFIGS[k], seed=0)
        sh = inp["shape"]
        packed = ctx.pack_weights(sh, inp["w_router"], inp["w_gate_up"], inp["w_down"])
        L.append((inp, sh, packed, inputs.workspace_for(sh),
                  torch.empty(sh["rows"], sh["d"], dtype=torch.float16, device="cuda")))
    res = {"what": "config 3 and config 4 layers alternating on one context, ms per layer call"}
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    for name, pol in (("adaptive", api.Context.TILE_ADAPTIVE), ("auto", api.Context.TILE_AUTO)):
        ctx.set_tile_policy(pol)

        def pair():
            for inp, sh, packed, ws, out in L:
                ctx.layer(sh, inp["x"], inp["w_router"], inp["bias"], None, None, None, None, out, ws,
                          packed=packed)
        for _ in range(warmup):
            pair()
        ctx.sync()
        e0.record()
        for _ in range(pairs):
            pair()
        e1.record()
        torch.cuda.synchronize()
        res[name + "_ms_per_layer"] = round(e0.elapsed_time(e1) / (2 * pairs), 5)
    ctx.set_tile_policy(api.Context.TILE_ADAPTIVE)
    del L
    torch.cuda.empty_cache()
    return res


def measure_teacher(ctx, torch, steps=50, warmup=20):
    """The reference teacher's own MoE shape (d 2560, 512 experts, top-10,
    width 640 with a shared expert; src/qwen.c:11-37) at the training batch
    of 2048 tokens: the fused layer on packed weights, and the reference's
    recording (rmda_qwen_moe_rec: 128-row segments, slot-scaled casts, fp32
    rows, hyper-connection streams out) on the HF-layout weights; the fused
    layer also with fp32 activations (slot-scaled)."""
    from rmda_moe import api, configs, inputs
    cfg = configs.TEACHER
    res = {"fused": measure_config(ctx, torch, cfg, steps=steps, warmup=warmup)}
    # the path qwen.c's fused forwarder takes: the chunk's fp32 activations
    # through the reference's slot-scaled casts
    res["fused_fp32_activations"] = measure_config(ctx, torch, cfg, steps=steps, warmup=warmup, x32=True)
    inp = inputs.make_inputs(ctx, cfg, seed=0)
    s = inp["shape"]
    T, d = s["rows"], s["d"]
    hc, hc_pad, hc_rank = 4, 384, 320  # MDA_QWEN_HC, MDA_QWEN_HC_PAD, cfg.hc_rank (src/qwen.h:20-21)
    qm = api.QwenMoe(ctx, s, inp["w_router"], inp["w_gate_up"], inp["w_down"], inp["w_sh_gate_up"],
                     inp["w_sh_down"], hc=hc, hc_rank=hc_rank, inj_stride=hc_pad)
    x32 = inp["x"].float()
    h = torch.zeros(T, hc, d, dtype=torch.float32, device="cuda")
    inj = torch.zeros(T, hc_pad, dtype=torch.float32, device="cuda")
    for _ in range(3):
        qm.moe_rec(x32, T, inj=inj, h=h)
    ctx.sync()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(10):
        qm.moe_rec(x32, T, inj=inj, h=h)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / 10
    res["qwen_moe_rec"] = {"ms_per_step": round(ms, 4), "tokens/s": round(T / (ms * 1e-3), 1),
                           "what": "rmda_qwen_moe_rec at the teacher shape, HF weights, 4 hc streams"}
    del qm, x32, h, inj, inp
    torch.cuda.empty_cache()
    return res


def measure_dropins(ctx, torch, inp, iters=50, warmup=10):
    """The reference-equivalent stage entry points on the same inputs, with
    the reference's 128-row segments and fp32 expert outputs: route, scan,
    scatter (materialises xp like shader/moe_scatter.comp), combine into four
    hyper-connection streams and plain combine.  Bytes are the algorithmic
    ones (padding and zero-fills excluded); route and scan are latency-bound."""
    s = inp["shape"]
    T, d, E, K = s["rows"], s["d"], s["experts"], s["topk"]
    P, HC, HC_PAD = 128, 4, 8
    mrows = (T * K + E * (P - 1) + P - 1) // P * P
    dev = "cuda"
    proj = torch.empty(T, E, dtype=torch.float32, device=dev)
    ctx.router(T, d, E, E, 0, inp["x"], inp["w_router"], None, proj)
    idx = torch.empty(T * K, dtype=torch.int32, device=dev)
    wt = torch.empty(T * K, dtype=torch.float32, device=dev)
    count = torch.empty(E, dtype=torch.int32, device=dev)
    off = torch.empty(E, dtype=torch.int32, device=dev)
    tiles = torch.empty(mrows // P, dtype=torch.int32, device=dev)
    fill = torch.empty(E, dtype=torch.int32, device=dev)
    slot = torch.empty(T * K, dtype=torch.int32, device=dev)
    xp = torch.zeros(mrows, d, dtype=torch.float16, device=dev)
    y = torch.randn(mrows, d, dtype=torch.float32, device=dev)
    h = torch.zeros(T, HC, d, dtype=torch.float32, device=dev)
    inj = torch.randn(T, HC_PAD, dtype=torch.float32, device=dev)
    out = torch.empty(T, d, dtype=torch.float16, device=dev)
    fields = (T, d, K, E, E, HC_PAD, 0, HC)
    ctx.scatter_experts(E)
    stages = [
        ("route", lambda: ctx.route(T, E, K, E, proj, idx, wt, count), T * E * 4 + T * K * 8 + E * 4),
        ("scan", lambda: ctx.scan(E, P, count, off, tiles, mrows // P), 0),
        ("scatter", lambda: ctx.scatter(T, K, d // 8, idx, off, fill, inp["x"], xp, slot),
         T * d * 2 + T * K * d * 2 + T * K * 8),
        ("combine_hc", lambda: ctx.combine(fields, wt, slot, y, proj, None, inj, h),
         T * K * d * 4 + T * K * 8 + T * HC * d * 4 * 2 + T * HC_PAD * 4),
        ("combine_plain", lambda: ctx.combine_plain(fields, wt, slot, y, proj, None, out),
         T * K * d * 4 + T * K * 8 + T * d * 2),
    ]
    res = {"workload": "BASELINE config 3 inputs, reference segments P=%d (mrows %d), fp32 expert outputs" % (P, mrows),
           "rates": "algorithmic bytes / time.  The plain legs repeat one call on the same buffers, so inputs "
                    "that fit the 256 MB Infinity Cache (scatter's x, combine's 134 MB of y) are served from it "
                    "(cache_resident); the *_cold legs rotate through buffer sets totalling over 256 MB so every "
                    "call reads HBM, and only they carry frac_of_hbm_peak"}
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    for name, fn, nbytes in stages:
        for _ in range(warmup):
            fn()
        ctx.sync()
        e0.record()
        for _ in range(iters):
            fn()
        e1.record()
        torch.cuda.synchronize()
        us = 1000.0 * e0.elapsed_time(e1) / iters
        res[name] = {"us": round(us, 2)}
        if nbytes:
            gbs = nbytes / (us * 1e-6) / 1e9
            res[name].update({"bytes": nbytes, "GB/s": round(gbs, 1),
                              "cache_resident": "inputs re-read every call (Infinity Cache)"})
    # cold: NSET buffer sets used in turn, so a set's bytes were evicted by
    # the other sets' since its last use (each combine set holds 134 MB of y,
    # each scatter set 134 MB of xp and its own 8 MB of x)
    NSET = 3
    ys = [torch.randn(mrows, d, dtype=torch.float32, device=dev) for _ in range(NSET)]
    hs = [torch.zeros(T, HC, d, dtype=torch.float32, device=dev) for _ in range(NSET)]
    xps = [torch.zeros(mrows, d, dtype=torch.float16, device=dev) for _ in range(NSET)]
    xs = [inp["x"].clone() for _ in range(NSET)]
    cold = [
        ("scatter_cold", lambda i: ctx.scatter(T, K, d // 8, idx, off, fill, xs[i], xps[i], slot), res["scatter"]["bytes"]),
        ("combine_hc_cold", lambda i: ctx.combine(fields, wt, slot, ys[i], proj, None, inj, hs[i]),
         res["combine_hc"]["bytes"]),
        ("combine_plain_cold", lambda i: ctx.combine_plain(fields, wt, slot, ys[i], proj, None, out),
         res["combine_plain"]["bytes"]),
    ]
    for name, fn, nbytes in cold:
        for i in range(2 * NSET):
            fn(i % NSET)
        ctx.sync()
        e0.record()
        for i in range(iters):
            fn(i % NSET)
        e1.record()
        torch.cuda.synchronize()
        us = 1000.0 * e0.elapsed_time(e1) / iters
        gbs = nbytes / (us * 1e-6) / 1e9
        res[name] = {"us": round(us, 2), "bytes": nbytes, "GB/s": round(gbs, 1),
                     "frac_of_hbm_peak": round(gbs / PEAK_HBM_GBS, 4),
                     "what": "%d buffer sets in turn (%.0f MB), every call's inputs from HBM"
                             % (NSET, NSET * (ys[0].numel() * 4 if "combine" in name else xps[0].numel() * 2) / 1e6)}
    del ys, hs, xps, xs
    # the reference's grouped GEMM (matmul_f16_moe): 128-row tiles of xp,
    # HF [E][n][k] weights, fp32 C; gate_up then down on a fp16 stand-in for hp16
    I = s["inter"]
    NO_SLOT = 0xFFFFFFFF
    g32 = torch.empty(mrows, 2 * I, dtype=torch.float32, device=dev)
    hp16 = torch.randn(mrows, I, dtype=torch.float16, device=dev)
    ye32 = torch.empty(mrows, d, dtype=torch.float32, device=dev)
    mm = [
        ("mm_gate_up", lambda: ctx.mm(mrows, 2 * I, d, NO_SLOT, NO_SLOT, xp, inp["w_gate_up"], g32, None, tiles),
         4 * T * K * d * I, E * 2 * I * d * 2 + T * K * d * 2 + T * K * 2 * I * 4),
        ("mm_down", lambda: ctx.mm(mrows, d, I, NO_SLOT, NO_SLOT, hp16, inp["w_down"], ye32, None, tiles),
         2 * T * K * d * I, E * d * I * 2 + T * K * I * 2 + T * K * d * 4),
    ]
    for name, fn, flops, nbytes in mm:
        for _ in range(3):
            fn()
        ctx.sync()
        e0.record()
        for _ in range(10):
            fn()
        e1.record()
        torch.cuda.synchronize()
        us = 1000.0 * e0.elapsed_time(e1) / 10
        gbs = nbytes / (us * 1e-6) / 1e9
        res[name] = {"us": round(us, 2), "TFLOP/s": round(flops / (us * 1e-6) / 1e12, 1), "bytes": nbytes,
                     "GB/s": round(gbs, 1), "frac_of_hbm_peak": round(gbs / PEAK_HBM_GBS, 4)}
    del g32, hp16, ye32
    # the whole reference-structured recording (mda_qwen_moe_rec's sequence
    # over these entry points), fp32 activations in, hc streams out
    from rmda_moe import api
    qm = api.QwenMoe(ctx, s, inp["w_router"], inp["w_gate_up"], inp["w_down"], inp["w_sh_gate_up"],
                     inp["w_sh_down"], hc=HC, hc_rank=0, inj_stride=HC_PAD)
    x32 = inp["x"].float()
    for _ in range(3):
        qm.moe_rec(x32, T, inj=inj, h=h)
    ctx.sync()
    e0.record()
    for _ in range(10):
        qm.moe_rec(x32, T, inj=inj, h=h)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / 10
    res["qwen_moe_rec"] = {"ms_per_step": round(ms, 4), "tokens/s": round(T / (ms * 1e-3), 1),
                           "what": "rmda_qwen_moe_rec: the reference's recording stage by stage, HF weights"}
    del qm, x32
    sc_b = res["scatter_cold"]["bytes"] + res["combine_hc_cold"]["bytes"]
    sc_us = res["scatter_cold"]["us"] + res["combine_hc_cold"]["us"]
    res["scatter+combine_hc_cold_GB/s"] = round(sc_b / (sc_us * 1e-6) / 1e9, 1)
    del proj, idx, wt, count, off, tiles, fill, slot, xp, y, h, inj, out
    torch.cuda.empty_cache()
    return res


def measure_upload(ctx, shape, torch):
    """Write one layer's bf16 weights as safetensors (reference tensor names),
    then time rmda_moe_upload_layer (mapped file -> pinned staging -> device ->
    packed), three times so both staging banks are used."""
    import tempfile
    import numpy as np
    from rmda_moe import st

    prefix = "model.language_model.layers.0.mlp."
    rng = np.random.default_rng(0)
    ts = st.moe_layer_tensors(prefix, shape, rng)
    nbytes = sum(a.nbytes for _, a in ts.values())
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "layer.safetensors")
        st.write(path, ts)
        del ts
        with st.SafeTensors(path) as f:
            packed = ctx.upload_layer(f, prefix, shape)  # first touch: maps pages, sizes the staging
            ctx.upload_wait()
            ctx.sync()
            times = []
            for _ in range(3):
                t0 = time.perf_counter()
                ctx.upload_layer(f, prefix, shape, packed=packed)
                ctx.upload_wait()
                ctx.sync()
                times.append(time.perf_counter() - t0)
    best = min(times)
    return {"GB/s": round(nbytes / best / 1e9, 2), "file_bytes": nbytes, "best_ms": round(best * 1e3, 2),
            "what": "bf16 safetensors layer in the page cache -> pinned staging (host threads) -> device -> "
                    "packed fp16, one rmda_moe_upload_layer + sync"}


def main():
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build runs the MoE layer on a single MI355X "
              "(expert-parallel sharding is a design note, not built); use --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    from rmda_moe import api, configs, inputs

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    torch.cuda.set_device(0)
    cfg = configs.CONFIGS[args.config] if args.config in configs.CONFIGS else configs.TEACHER
    ctx = api.Context(0)
    inp = inputs.make_inputs(ctx, cfg, seed=0)
    shape = inp["shape"]
    if args.dropin_only:
        d = measure_dropins(ctx, torch, inp)
        ctx.close()
        print(json.dumps({"dropin": d}), flush=True)
        return
    ws = inputs.workspace_for(shape)
    out = torch.empty(shape["rows"], shape["d"], dtype=torch.float16, device="cuda")

    # expert weights are packed once, as at weight upload (the reference
    # converts them bf16 -> fp16 at upload, outside the MoE layer)
    torch.cuda.synchronize()
    p0 = time.perf_counter()
    packed = None
    if not args.hf_layout:
        packed = ctx.pack_weights(shape, inp["w_router"], inp["w_gate_up"], inp["w_down"], inp["w_sh_gate_up"],
                                  inp["w_sh_down"])
        ctx.sync()
    pack_ms = 1000.0 * (time.perf_counter() - p0)

    def step():
        if packed is None:
            ctx.layer(shape, inp["x"], inp["w_router"], inp["bias"], inp["w_gate_up"], inp["w_down"],
                      inp["w_sh_gate_up"], inp["w_sh_down"], out, ws)
        else:
            ctx.layer(shape, inp["x"], inp["w_router"], inp["bias"], None, None, None, None, out, ws,
                      packed=packed)

    transient = measure_transient(step, torch) if args.transient else None
    for _ in range(args.warmup):
        step()
    ctx.sync()
    torch.cuda.synchronize()
    if args.sustain > 0:
        idle = smi_sample()
        s = measure_sustained(step, ctx, torch, args.sustain)
        s["idle_before"] = None if idle is None else {"socket_W": idle["socket_W"], "mem_MHz": idle["mem_MHz"]}
        ctx.close()
        print(json.dumps({"sustained": s, "config": {"workload": cfg["name"], "tokens": shape["rows"]}}),
              flush=True)
        return

    # timed region: K layer calls, bracketed by device synchronisation; events
    # between equal rounds of the K calls (no synchronisation inside) give the
    # best and median round, the reference's bench discipline
    # (src/bench.c:32-53,93-105)
    n_rounds = max(1, min(7, args.steps))
    cuts = [args.steps * r // n_rounds for r in range(n_rounds + 1)]
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(n_rounds + 1)]
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    evs[0].record()
    for r in range(n_rounds):
        for _ in range(cuts[r + 1] - cuts[r]):
            step()
        evs[r + 1].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    ms = evs[0].elapsed_time(evs[-1]) / args.steps
    round_seq = [evs[r].elapsed_time(evs[r + 1]) / (cuts[r + 1] - cuts[r]) for r in range(n_rounds)]
    round_ms = sorted(round_seq)

    # per-stage durations: the same K calls again with the stage profiler on
    ctx.prof_begin()
    for _ in range(args.steps):
        step()
    stage_ms, n_prof = ctx.prof_end()
    # per-stage GPU time net of what a stage boundary (one event) costs by
    # itself; stages whose launch every call skipped are left out
    event_us = 1000.0 * ctx.prof_empty_ms() / max(n_prof, 1)
    stage_us = {k: 1000.0 * v / max(n_prof, 1) - event_us for k, v in stage_ms.items() if v > 0}

    # steady state, reported beside (never in place of) the timed region:
    # the GPU's clocks take tens of milliseconds of back-to-back calls to
    # settle, so a short --warmup times part of that transient
    for _ in range(100):
        step()
    e_s0 = torch.cuda.Event(enable_timing=True)
    e_s1 = torch.cuda.Event(enable_timing=True)
    e_s0.record()
    for _ in range(100):
        step()
    e_s1.record()
    torch.cuda.synchronize()
    steady_ms = e_s0.elapsed_time(e_s1) / 100

    views = api.ws_views(shape, ws)
    counts = views["count"].cpu().numpy()
    touched = int((counts > 0).sum())
    work = configs.algorithmic_work(cfg, touched=touched)

    rate = {
        "router": (work["router_bytes"], work["router_flops"]),
        "route": (work["route_bytes"], 0),
        "rank": (0, 0),
        "permute": (0, 0),
        "gate_up": (work["gate_up_bytes"], work["gate_up_flops"]),
        "down": (work["down_bytes"], work["down_flops"]),
        "combine": (work["combine_bytes"], 0),
    }
    stages = {}
    for k, us in stage_us.items():
        b, f = rate[k]
        stages[k] = {"us": round(us, 2)}
        if b:
            stages[k]["GB/s"] = round(b / (us * 1e-6) / 1e9, 1)
        if f:
            stages[k]["TFLOP/s"] = round(f / (us * 1e-6) / 1e12, 1)

    dom = max(stage_us, key=stage_us.get)
    b, f = rate[dom]
    ridge = PEAK_FP16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)
    t_dom = stage_us[dom] * 1e-6
    if f and b and f / b > ridge:
        roof = {"bound": "mfma", "achieved": round(f / t_dom / 1e12, 2), "peak": PEAK_FP16_TFLOPS,
                "unit": "TFLOP/s"}
    else:
        roof = {"bound": "hbm", "achieved": round(b / t_dom / 1e9, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s"}
    roof["frac"] = round(roof["achieved"] / roof["peak"], 4)
    roof["kernel"] = dom
    roof["algorithmic_bytes"] = b
    roof["algorithmic_flops"] = f
    roof["avg_us"] = round(stage_us[dom], 2)
    roof["traffic"] = read_traffic() if (dom == "gate_up" and args.config == 3) else None

    gemm_us = stage_us["gate_up"] + stage_us["down"]
    gemm_tf = work["gemm_flops"] / (gemm_us * 1e-6) / 1e12
    ai = work["gemm_flops"] / (work["gate_up_bytes"] + work["down_bytes"])
    ceiling = min(PEAK_FP16_TFLOPS, PEAK_HBM_GBS * 1e9 * ai / 1e12)
    gemm = {"TFLOP/s": round(gemm_tf, 1), "frac_of_fp16_peak": round(gemm_tf / PEAK_FP16_TFLOPS, 4),
            "ai_flop_per_byte": round(ai, 1), "ceiling_TFLOP/s": round(ceiling, 1),
            "frac_of_ceiling": round(gemm_tf / ceiling, 4), "experts_touched": touched}
    # the layer's combine reads the 67 MB of fp16 rows the down GEMM wrote
    # just before, from the Infinity Cache: a cache-resident rate
    hbm_small = {"combine_GB/s": stages.get("combine", {}).get("GB/s"),
                 "combine_inputs": "cache_resident: the fp16 expert rows written by the down GEMM just before"}
    stages["event_interval_us"] = round(event_us, 2)

    if args.calib_copy:
        # a plain device copy of known size, for scaling FETCH_SIZE / WRITE_SIZE
        n = 256 << 20
        src = torch.empty(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print("calib copy: %d bytes read, %d bytes written per launch" % (n, n), file=sys.stderr)

    peaks = None if args.no_peaks else measure_peaks(torch)
    upload = measure_upload(ctx, shape, torch) if args.upload else None
    decode = measure_config(ctx, torch, 2) if (args.config == 3 and not args.no_decode) else None
    others = {}
    if args.config == 3 and not args.no_others:
        others["skew"] = measure_config(ctx, torch, 4)
        others["fine_shared"] = measure_config(ctx, torch, 5)
        others["mixed_load"] = measure_mixed(ctx, torch)
        others["teacher"] = measure_teacher(ctx, torch)
        others["fp32_activations"] = measure_config(ctx, torch, 3, x32=True)
        others["alternating_layers"] = measure_alternating(ctx, torch)
    dropin = measure_dropins(ctx, torch, inp) if (args.config == 3 and not args.no_dropin) else None

    cpu = None
    if not args.no_cpu_baseline:
        n_tok = args.cpu_tokens
        if n_tok is None:
            n_tok = {1: 256, 2: 128, 3: 512, 4: 512, 5: 256, 6: 128}[args.config]
        cpu = cpu_baseline(inp, cfg, n_tok)

    if args.stages:
        for k, v in stages.items():
            print("%-8s %s" % (k, v), file=sys.stderr)

    T = shape["rows"]
    line = {
        "metric": METRIC,
        "value": round(T / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (counter-hash N(0,1) activations, N(0,0.02) weights, seed 0)",
        "config": {"workload": workload_name(cfg, shape, args.config if args.config in configs.CONFIGS else None),
                   "tokens": T, "d": shape["d"], "experts": shape["experts"], "topk": shape["topk"],
                   "inter": shape["inter"], "shared": shape["shared"], "parallelism": "single GPU"},
        "wall_ms_per_step": round(1000.0 * wall / args.steps, 5),
        "rounds": {"n": n_rounds, "best_ms": round(round_ms[0], 5),
                   "median_ms": round(round_ms[len(round_ms) // 2], 5),
                   "ms_in_order": [round(x, 4) for x in round_seq]},
        "steady_state": {"ms_per_step": round(steady_ms, 5), "tokens/s": round(T / (steady_ms * 1e-3), 1),
                         "what": "100 calls timed after the timed region, the stage profile and 100 more calls"},
        "weights": "HF layout" if args.hf_layout else "packed once before timing (%.1f ms, host-timed)" % pack_ms,
        "roofline": roof,
        "gemm": gemm,
        "bandwidth": hbm_small,
        "stages": stages,
        "decode": decode,
        "skew": others.get("skew"),
        "fine_shared": others.get("fine_shared"),
        "mixed_load": others.get("mixed_load"),
        "teacher": others.get("teacher"),
        "fp32_activations": others.get("fp32_activations"),
        "alternating_layers": others.get("alternating_layers"),
        "dropin": dropin,
        "cpu_baseline": cpu,
    }
    if cpu is not None:
        line["cpu_baseline"]["gpu_over_cpu"] = round(line["value"] / cpu["value"], 1)
    if upload is not None:
        line["upload"] = upload
    if transient is not None:
        line["transient"] = transient
    if peaks is not None:
        line["peaks_measured"] = peaks
        if roof["unit"] == "GB/s":
            roof["frac_of_measured_copy"] = round(roof["achieved"] / peaks["hbm_copy_GB/s"], 4)
        # the copy-shaped stages beside this box's own device-copy rate: a
        # scatter or combine cannot stream faster than a plain copy does
        cp = peaks["hbm_copy_GB/s"]
        if hbm_small.get("combine_GB/s"):
            hbm_small["combine_frac_of_measured_copy"] = round(hbm_small["combine_GB/s"] / cp, 4)
        if dropin is not None:
            for k in ("scatter", "combine_hc", "combine_plain", "scatter_cold", "combine_hc_cold",
                      "combine_plain_cold"):
                if "GB/s" in dropin.get(k, {}):
                    dropin[k]["frac_of_measured_copy"] = round(dropin[k]["GB/s"] / cp, 4)
    ctx.close()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
