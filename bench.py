#!/usr/bin/env python3
"""Routed-MoE decode benchmark on one MI355X.

Workload (benchmark config 1): one MoE layer of 288 routed experts, top-8, SwiGLU H=5120 I=1536, EXL3 3 bits/weight,
M = 1..4 decode tokens with fp16 N(0,1) activations and sigmoid top-8 routing of N(0,1) fp32 logits. A step is one
layer call (split -> 8*M expert GEMVs -> weighted combine) through the C ABI. Steps cycle through `--layers` distinct
288-expert layers (2.56 GB each) and 32 routings, so expert bytes come from HBM, not the 256 MB Infinity Cache.
Steps are captured in a HIP graph and replayed; the timed region is bracketed by synchronisation. Before it, after
the --warmup eager steps, the captured graphs are replayed until 30 ms of device time has passed: the device's first
~10 ms of sustained load run up to 25% slower, which a short timed region (--steps 20) would otherwise measure.

value        = microseconds per token at M=1 (lower is better): the median over exactly --steps timed steps of the
               per-step times (device events between replays of up to 8 captured graphs of up to --graph-steps steps,
               replayed round-robin so a graph's layers come back only after GBs of others); p10/p90 and the mean
               over the whole timed region beside it. per_M holds M=1..4. All run the EXACT mode, whose outputs are
               bit-identical to the reference's EXACT expert (--mode mfma times GFL_MODE_MFMA instead).
roofline     = the gate|up GEMV kernel (the dominant one) at M=1: algorithmic quantized bytes per launch (union of
               routed experts x (gate+up trellis + their suh/svh)) / its mean execution time, from start/stop events
               the runtime stamps on each launch's own dispatch (hipExtLaunchKernelGGL, through gfl_profile_*) during
               an eager pass on the launch stream; peak = 8 TB/s HBM; traffic = HBM bytes per launch from the
               FETCH_SIZE/WRITE_SIZE counter file (--pmc-probe / --pmc-digest).
per_M_end_to_end = the decode step a routing_fn caller pays at M=1..4, from router logits to the layer output:
               gfl_route_split + gfl_moe_forward + gfl_combine in one captured step (128 steps, same protocol).
configs      = benchmark configs 0 (one expert per call), 2 (mixed bitrates, Zipf routing), 3 (M=16/32/64) and 4 (42
               resident layers decoded at M=1; prefill of M=2048 tokens through the EXACT path, as TFLOP/s against
               the 157.3 TF dense fp32 MFMA peak its chain steps run on, and through the MFMA grouped path, against
               2.5 PF dense fp16); the router (gfl_route) per call; routed layer + shared expert: sequential,
               overlapped on a side stream, and fused into the routed call's launches (gfl_moe_forward_shared).
cpu_baseline = the reference's own AVX2 expert engine (kernels/cpu_avx2/ft_core.h, built into oracle/_ref) timed on
               this host: decode calls of M tokens x 8 experts cycling a DRAM-cold pool of 288 experts; value = I16
               at M=1; EXACT at M=1..4, AFFINE at M=2..4 and the single expert of config 0 beside it, with the CPU
               model.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "glm-flash-lite_amd"))

METRIC = "MoE-layer decode µs/token at M=1..4 + % HBM roofline on quantized bytes"
HBM_PEAK_GBPS = 8000.0
MODE = 1   # decode mode of every gfl_moe_forward call (1 EXACT, 3 MFMA-accumulate GEMVs); set by --mode
MFMA_PEAK_TFLOPS = 2500.0   # dense fp16 MFMA
MFMA_FP32_PEAK_TFLOPS = 157.3   # dense fp32 MFMA
H, I, E, TOPK, KBITS = 5120, 1536, 288, 8, 3
XSTEPS = 128   # steps per line of the configs beside the headline
WARM_MS = 30.0   # device time of graph replays before each graph-timed region (graph_time)


def physical_cpus(skip=2, cap=16):
    """One logical CPU per physical core among the allowed CPUs, minus the first `skip` (auto_cpus rule of the
    reference, glm53/cpu_tier.py:114-127), capped at the GPU box's CPU share."""
    allowed = sorted(os.sched_getaffinity(0))
    seen, firsts = set(), []
    for c in allowed:
        try:
            core = open(f"/sys/devices/system/cpu/cpu{c}/topology/core_id").read().strip()
            pkg = open(f"/sys/devices/system/cpu/cpu{c}/topology/physical_package_id").read().strip()
        except OSError:
            core, pkg = str(c), "0"
        if (pkg, core) not in seen:
            seen.add((pkg, core))
            firsts.append(c)
    cpus = firsts[skip:] if len(firsts) > skip + 1 else firsts[-1:]
    return cpus[:cap]


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(iters, warmup):
    """Reference AVX2 engine timing; returns the cpu_baseline object or None when the engine is not built.
    Decode calls of M tokens x 8 experts (1 expert for config 0) cycling a DRAM-cold pool of 288 experts, as
    tools/bench/kernel-ab-harness.cpp HARNESS_TIME does: I16 (the production decode mode) and EXACT at M=1, EXACT and
    AFFINE at M=2..4 (the reference's I16 scale arrays are sized for H=4096 and overrun at H=5120 once an expert
    carries two tokens), and the single-expert config 0 in I16 and EXACT. Median and p10/p90 per call."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from oracle import REFLIB, Mat, Oracle, RefEngine
    if not os.path.exists(REFLIB):
        return None
    cpus = physical_cpus()
    O = Oracle()
    eng = RefEngine(threads=len(cpus), cpus=cpus)
    t0 = time.time()
    pool = []
    for e in range(E):
        mats = []
        for p, (k, n) in enumerate(((H, I), (H, I), (I, H))):
            s = O.seed(90, e, p)
            tr = O.synth_trellis(s, (k // 16) * (n // 16) * 32 * KBITS)
            suh, svh = O.synth_scales(s, k, n, k)
            mats.append(Mat(tr, suh, svh, k, n, KBITS))
        pool.append(tuple(mats))
    gen_s = time.time() - t0
    per_expert = sum(m.tr.size + 2 * (m.k + m.n) for m in pool[0])
    rng = np.random.default_rng(4242)
    xs = rng.standard_normal((4, H)).astype(np.float16).astype(np.float32)

    def run(M, topk, mode, n):
        secs = np.asarray(eng.time_decode(pool, xs[:M], topk, n, warmup, mode)) * 1e6 / M
        return {"median": round(float(np.median(secs)), 2), "p10": round(float(np.percentile(secs, 10)), 2),
                "p90": round(float(np.percentile(secs, 90)), 2), "calls": n,
                "GBps": round(M * topk * per_expert / (float(np.median(secs)) * M * 1e-6) / 1e9, 2)}

    t1 = time.time()
    res = {"M1_i16": run(1, TOPK, 2, iters), "M1_exact": run(1, TOPK, 1, iters)}
    for M in (2, 3, 4):
        res[f"M{M}_exact"] = run(M, TOPK, 1, max(20, iters // 3))
        res[f"M{M}_affine"] = run(M, TOPK, 0, max(20, iters // 3))
    res["config0_i16"] = run(1, 1, 2, iters)
    res["config0_exact"] = run(1, 1, 1, iters)
    return {"value": res["M1_i16"]["median"], "unit": "us/token", "cores": len(cpus), "kind": "reference",
            "cpu_model": cpu_model(),
            "sample": f"decode calls (after {warmup} warm-up each) of M tokens x {TOPK} experts (config 0: 1 x 1), "
                      f"expert sets cycling a DRAM-cold pool of {E} experts (H={H} I={I} K={KBITS}, "
                      f"{E * per_expert / 1e9:.2f} GB); value = I16 at M=1, median of {iters} calls; "
                      f"per-mode medians and p10/p90 in us/token below",
            "modes_us_per_token": res, "cpus": cpus, "pool_gen_s": round(gen_s, 1),
            "timed_s": round(time.time() - t1, 1)}


COPY_BYTES = 1 << 30
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_gate_up_config1_M1.json")
# the gate|up launch of a config-1 M=1 call: 8 picks (1,536 gate|up tile columns) run the relay launches, 2 waves per
# column (gfl_moe_forward's launch choice)
GATE_UP_KERNEL = "gu_relay_kernel<3, 2>"


def pmc_probe(ctx, layers, steps=64, M=1):
    """Dispatches whose HBM counters calibrate and measure the gate|up kernel: four launches of an elementwise
    negation over COPY_BYTES of fp32 (reads COPY_BYTES, writes COPY_BYTES; 4x the 256 MB Infinity Cache), then
    `steps` eager M-token layer calls cycling the layers and 32 routings, as the timed benchmark does."""
    import numpy as np
    import torch
    import synth
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(4):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    del src, dst
    rng = np.random.default_rng(1001)
    xs, sels, ws = [], [], []
    for r in range(32):
        x = rng.standard_normal((M, H)).astype(np.float16)
        (sel, w16), _ = synth.route_uniform(M, E, TOPK, rng)
        xs.append(torch.from_numpy(x.view(np.int16)).view(torch.float16).cuda())
        sels.append(torch.from_numpy(sel).cuda())
        ws.append(torch.from_numpy(w16.view(np.int16)).view(torch.float16).cuda())
    out = torch.empty((M, H), dtype=torch.float32, device="cuda")
    for i in range(steps):
        ctx.moe_forward(i % len(layers), xs[i % 32], sels[i % 32], ws[i % 32], out, mode=MODE)
    torch.cuda.synchronize()
    print(f"pmc probe: {4} copies of {COPY_BYTES} B, {steps} M={M} layer calls", flush=True)


def pmc_table(folders):
    """Markdown table of per-kernel means of every counter in rocprofv3 --pmc outputs (counter_collection.csv) and
    of the kernel-trace statistics (kernel_stats.csv) under the given folders: the decode kernels and the copy."""
    import csv
    import glob
    from collections import defaultdict
    acc, stats = defaultdict(list), {}
    for folder in folders:
        for f in glob.glob(os.path.join(folder, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                acc[(r["Kernel_Name"].split("(")[0][:48], r["Counter_Name"])].append(float(r["Counter_Value"]))
        for f in glob.glob(os.path.join(folder, "**", "*kernel_stats.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                stats[r["Name"].split("(")[0][:48]] = (int(r["Calls"]), float(r["AverageNs"]) / 1e3)
    print("| kernel | counter | mean per dispatch | dispatches |")
    print("|---|---|---|---|")
    for (k, c), v in sorted(acc.items()):
        if "gfl::" in k or "neg" in k:
            print(f"| `{k}` | {c} | {sum(v) / len(v):,.1f} | {len(v)} |")
    for k, (n, us) in sorted(stats.items()):
        if "gfl::" in k:
            print(f"| `{k}` | mean duration (us) | {us:.2f} | {n} |")


def _pmc_rows(folder, counter):
    import csv
    import glob
    files = glob.glob(os.path.join(folder, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no counter_collection.csv under {folder}")
    rows = []
    for f in files:
        for r in csv.DictReader(open(f)):
            if r.get("Counter_Name") == counter:
                rows.append((r["Kernel_Name"], float(r["Counter_Value"])))
    return rows


def pmc_digest(fetch_dir, write_dir):
    """HBM bytes per gate|up launch from FETCH_SIZE and WRITE_SIZE (KiB per dispatch), each scaled by the factor
    that makes the calibration copy read / write exactly COPY_BYTES."""
    import numpy as np
    res = {}
    for name, folder in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        rows = _pmc_rows(folder, name)
        cal = [v for k, v in rows if "neg" in k.lower()]
        gu = [v for k, v in rows if GATE_UP_KERNEL in k]
        if not cal or not gu:
            raise SystemExit(f"{name}: calibration or gate|up dispatches missing ({len(cal)}, {len(gu)})")
        factor = COPY_BYTES / (float(np.median(cal)) * 1024.0)
        res[name] = {"copy_kib_median": float(np.median(cal)), "scale": round(factor, 4),
                     "gate_up_kib_mean": round(float(np.mean(gu)), 1), "dispatches": len(gu),
                     "gate_up_bytes_scaled": round(float(np.mean(gu)) * 1024.0 * factor)}
    total = res["FETCH_SIZE"]["gate_up_bytes_scaled"] + res["WRITE_SIZE"]["gate_up_bytes_scaled"]
    doc = {"kernel": GATE_UP_KERNEL, "workload": "config1 M=1 decode, eager calls cycling 4 layers",
           "hbm_bytes_per_launch": total, "counters": res}
    json.dump(doc, open(TRAFFIC_FILE, "w"), indent=1)
    print(json.dumps(doc))


def make_routes(M, rng, n, kind):
    """n routings of M tokens: (x fp16 [M,H], sel int64 [M,8], w fp16 [M,8], union size) on the GPU.
    kind: "uniform" (N(0,1) logits) or "zipf" (Zipf s=1.1 skew over a seeded expert ranking)."""
    import numpy as np
    import torch
    import synth
    out = []
    for _ in range(n):
        x = rng.standard_normal((M, H)).astype(np.float16)
        if kind == "zipf":
            sel, w16 = synth.route(synth.zipf_logits(M, E, 1.1, rng), TOPK)
        else:
            (sel, w16), _ = synth.route_uniform(M, E, TOPK, rng)
        out.append((torch.from_numpy(x.view(np.int16)).view(torch.float16).cuda(), torch.from_numpy(sel).cuda(),
                    torch.from_numpy(w16.view(np.int16)).view(torch.float16).cuda(), len(np.unique(sel))))
    return out


def graph_size(steps, gmax):
    """Steps per captured graph: the largest divisor of `steps` that is <= gmax, so exactly `steps` steps are timed."""
    for g in range(max(1, min(gmax, steps)), 0, -1):
        if steps % g == 0:
            return g
    return 1


def replay_samples(graphs, reps):
    """Replays graphs[r % len(graphs)] for r < reps back to back on the current stream, with a device event between
    consecutive replays. Returns (per-replay ms list, ms from the first event to the last)."""
    import torch
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    torch.cuda.synchronize()
    ev[0].record()
    for r in range(reps):
        graphs[r % len(graphs)].replay()
        ev[r + 1].record()
    torch.cuda.synchronize()
    return [ev[r].elapsed_time(ev[r + 1]) for r in range(reps)], ev[0].elapsed_time(ev[reps])


def warm_graphs(graphs):
    """Replay `graphs` round-robin until WARM_MS of device time has passed (each at least once): the device's first
    ~10 ms of sustained load run slower (20-step measurements of config 1 M=4 repeated back to back in one process
    gave 42.1, 41.2, 35.8, 34.6, ... 33.7 us/token), so a timed region right after capture would measure that ramp
    rather than the kernels."""
    import torch
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    while True:
        for g in graphs:
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        if e0.elapsed_time(e1) >= WARM_MS:
            return


def _dist(ms_per_step, M):
    import numpy as np
    a = np.asarray(ms_per_step) * 1e3 / M
    return {"median": round(float(np.median(a)), 3), "p10": round(float(np.percentile(a, 10)), 3),
            "p90": round(float(np.percentile(a, 90)), 3)}


def graph_time(step, out, steps, G, warmup, ngraphs=8):
    """Graph-timed steps: step(s) enqueues step s on the current stream. Up to `ngraphs` graphs of G consecutive steps
    each are captured (graph j holds steps jG .. jG+G-1) and replayed round-robin, steps / G replays in all, so exactly
    `steps` steps are timed and a graph comes back only after the others' steps have streamed through. Returns
    (per-step ms from device events between replays, ms over the whole timed region, graphs, whether the last graph's
    final step replayed equals the same step run eagerly, compared on `out`)."""
    import torch
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        for i in range(2):
            step(i)
    torch.cuda.current_stream().wait_stream(st)
    reps = steps // G
    ng = max(1, min(ngraphs, reps))
    graphs = []
    for j in range(ng):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(G):
                step(j * G + i)
        graphs.append(g)
    warm_graphs(graphs)
    samples, total_ms = replay_samples(graphs, reps)
    graphs[-1].replay()
    torch.cuda.synchronize()
    got = out.clone()
    step(ng * G - 1)
    torch.cuda.synchronize()
    graph_ok = bool(torch.equal(got, out))
    del graphs
    return [t / G for t in samples], total_ms, ng, graph_ok


def time_layer_steps(ctx, layer_ids, routes, M, steps, G, warmup, bytes_per_expert, per_step=1, ngraphs=8):
    """Graph-timed decode steps (graph_time). A step is `per_step` consecutive layer calls (call c = s * per_step + i
    of step s runs layer layer_ids[c % len] with routing c % len(routes)); with many layers cycled a graph comes back
    only after far more bytes than the 256 MB Infinity Cache. The headline is the median of the per-step times;
    p10/p90 and the mean over the whole timed region are reported beside it."""
    import numpy as np
    import torch
    out = torch.empty((M, H), dtype=torch.float32, device="cuda")
    NR, NL = len(routes), len(layer_ids)

    def step(s_):
        for i in range(per_step):
            c = s_ * per_step + i
            x, sel, w, _ = routes[c % NR]
            ctx.moe_forward(layer_ids[c % NL], x, sel, w, out, mode=MODE)

    per_step_ms, total_ms, ng, graph_ok = graph_time(step, out, steps, G, warmup, ngraphs)
    ms = float(np.median(per_step_ms))
    calls = [(s_ * per_step + i) for s_ in range(ng * G) for i in range(per_step)]
    step_bytes = (sum(routes[c % NR][3] * bytes_per_expert(layer_ids[c % NL]) for c in calls) / (ng * G)
                  + per_step * M * H * 6)
    gbps = step_bytes / (ms * 1e-3) / 1e9
    return {"us_per_token": round(ms * 1e3 / M, 3), "ms_per_step": round(ms, 5),
            "us_per_token_dist": _dist(per_step_ms, M), "us_per_token_mean": round(total_ms / steps * 1e3 / M, 3),
            "steps": steps, "graph_steps": G, "graphs": ng,
            "union_experts": round(float(np.mean([r[3] for r in routes])), 2), "GBps": round(gbps, 1),
            "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4), "graph_replay_matches_eager": graph_ok}


def time_e2e_steps(ctx, layer_ids, M, steps, G, warmup, bytes_per_expert):
    """The decode step a routing_fn caller pays, from the router's logits to the layer output: one step is
    gfl_route_split (sigmoid top-8 of fp32 N(0,1) logits [M, 288] and ft_split at full residency, which publishes
    nothing), gfl_moe_forward on the split's selection, and gfl_combine (no job: it returns without waiting). The
    router's projection z @ W^T, a plain library GEMM, is outside it. Graph-timed as the headline (graph_time), with
    32 routings and the layers cycled."""
    import numpy as np
    import torch
    import _native
    import synth
    rng = np.random.default_rng(9000 + M)
    routes = []
    for _ in range(32):
        x = rng.standard_normal((M, H)).astype(np.float16)
        lg = rng.standard_normal((M, E)).astype(np.float32)
        routes.append((torch.from_numpy(x.view(np.int16)).view(torch.float16).cuda(), torch.from_numpy(lg).cuda(),
                       len(np.unique(synth.route(lg, TOPK)[0]))))
    dev = "cuda"
    n = M * TOPK
    sel = torch.empty((M, TOPK), dtype=torch.int64, device=dev)
    w = torch.empty((M, TOPK), dtype=torch.float16, device=dev)
    so = torch.empty(n, dtype=torch.int64, device=dev)
    wo = torch.empty(n, dtype=torch.float16, device=dev)
    ctrl = torch.zeros(16, dtype=torch.int64, device=dev)
    hx = torch.zeros(n * H, dtype=torch.float16, device=dev)
    picks = torch.zeros(n * 3, dtype=torch.int32, device=dev)
    hout = torch.zeros(M * H, dtype=torch.float32, device=dev)
    dflag = torch.zeros(1, dtype=torch.int64, device=dev)
    stats = torch.zeros(8, dtype=torch.int64, device=dev)
    slotof = torch.arange(E, dtype=torch.int32, device=dev)
    score = torch.zeros(E, dtype=torch.float32, device=dev)
    pol = torch.tensor([0.4, 0.023, 0.11, 0.104, 0.2, 32, -1, 0] + [0.0] * 12, dtype=torch.float32, device=dev)
    out = torch.empty((M, H), dtype=torch.float32, device=dev)
    NR, NL = len(routes), len(layer_ids)

    def step(s_):
        x, lg, _ = routes[s_ % NR]
        li = layer_ids[s_ % NL]
        _native.route_split(lg, TOPK, x, E, 0, slotof, score, pol, ctrl.data_ptr(), hx.data_ptr(), picks.data_ptr(),
                            s_ + 1, li, 0, sel, w, so, wo, dflag, stats, None)
        ctx.moe_forward(li, x, so.view(M, TOPK), wo.view(M, TOPK), out, mode=MODE)
        _native.combine(out, dflag, ctrl.data_ptr(), hout.data_ptr(), stats, 2_000_000_000)

    per_step_ms, total_ms, ng, graph_ok = graph_time(step, out, steps, G, warmup)
    ms = float(np.median(per_step_ms))
    union = float(np.mean([r[2] for r in routes]))
    gbps = (union * bytes_per_expert + M * H * 6) / (ms * 1e-3) / 1e9
    return {"us_per_token": round(ms * 1e3 / M, 3), "ms_per_step": round(ms, 5),
            "us_per_token_dist": _dist(per_step_ms, M), "us_per_token_mean": round(total_ms / steps * 1e3 / M, 3),
            "steps": steps, "graph_steps": G, "graphs": ng, "union_experts": round(union, 2), "GBps": round(gbps, 1),
            "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4), "graph_replay_matches_eager": graph_ok,
            "combine_timeouts": int(stats[6].item()), "split_calls": int(stats[3].item()),
            "experts_sent_to_host": int(stats[2].item())}


def extra_configs(ctx, layers, args):
    """Benchmark configs 0, 2, 3 and 4 (42-layer resident stack, prefill through both paths), timed like config 1:
    XSTEPS steps per line (fewer for the long ones), graphs of 4 steps."""
    import numpy as np
    import synth
    res = {}
    t0 = time.time()
    res["config0_single_expert"] = time_config0(ctx, list(range(args.layers)), layers[0].quant_bytes_per_expert)
    print(f"bench: config 0 done ({time.time() - t0:.0f} s)", file=sys.stderr, flush=True)
    # config 2: mixed bitrates, Zipf-skewed routing; two layers of each kind cycled (3.1 GB per layer)
    base = 100
    mixed = {"A_gate_up4_down3": (4, 4, 3), "B_gate_up3_down5": (3, 3, 5)}
    for j, (name, ks) in enumerate(mixed.items()):
        ids = []
        for r in range(2):
            li = base + 2 * j + r
            L = synth.SynthLayer(li, E, H, I, ks)
            L.register(ctx, li)
            layers.append(L)
            ids.append(li)
        bpe = L.quant_bytes_per_expert
        per = {}
        for M in (1, 2, 3, 4):
            routes = make_routes(M, np.random.default_rng(2000 + 10 * j + M), 32, "zipf")
            per[str(M)] = time_layer_steps(ctx, ids, routes, M, XSTEPS, 4, 8, lambda li, b=bpe: b)
        res["config2_" + name] = per
        print(f"bench: config 2 {name} done ({time.time() - t0:.0f} s)", file=sys.stderr, flush=True)
    # config 3: batched decode across conversations on the config-1 layers
    per = {}
    for M in (16, 32, 64):
        routes = make_routes(M, np.random.default_rng(3000 + M), 16, "uniform")
        per[str(M)] = time_layer_steps(ctx, list(range(args.layers)), routes, M, XSTEPS // 2, 4, 4,
                                       lambda li: layers[0].quant_bytes_per_expert)
    res["config3_batched"] = per
    print(f"bench: config 3 done ({time.time() - t0:.0f} s)", file=sys.stderr, flush=True)
    # config 4 (decode half): a stack of 42 config-1 layers resident at once, one token through all of them per step
    nst = args.stack_layers
    ids = []
    for r in range(nst):
        li = 200 + r
        L = synth.SynthLayer(li, E, H, I, (KBITS,) * 3)
        L.register(ctx, li)
        layers.append(L)
        ids.append(li)
    print(f"bench: {nst}-layer stack resident ({time.time() - t0:.0f} s)", file=sys.stderr, flush=True)
    routes = make_routes(1, np.random.default_rng(4000), nst, "uniform")
    r = time_layer_steps(ctx, ids, routes, 1, 16, 2, 1, lambda li: layers[0].quant_bytes_per_expert, per_step=nst,
                         ngraphs=4)
    r["layers"] = nst
    r["resident_GB"] = round(nst * E * layers[0].quant_bytes_per_expert / 1e9, 1)
    res["config4_stack_decode"] = r
    print(f"bench: config 4 stack done ({time.time() - t0:.0f} s)", file=sys.stderr, flush=True)
    res["config4_prefill"] = time_prefill(ctx, list(range(args.layers)), layers[0].quant_bytes_per_expert, 2048, 8)
    print(f"bench: config 4 prefill (MFMA grouped) done ({time.time() - t0:.0f} s)", file=sys.stderr, flush=True)
    res["config4_prefill_exact"] = time_prefill(ctx, list(range(args.layers)), layers[0].quant_bytes_per_expert,
                                                2048, 2, G=2, exact=True)
    print(f"bench: config 4 prefill done ({time.time() - t0:.0f} s)", file=sys.stderr, flush=True)
    res["router"] = {f"M{M}": time_router(M) for M in (1, 4, 64, 2048)}
    res["shared_overlap"] = time_shared(ctx, list(range(args.layers)), 32, 4)
    print(f"bench: shared-expert overlap done ({time.time() - t0:.0f} s)", file=sys.stderr, flush=True)
    res["setup_and_time_s"] = round(time.time() - t0, 1)
    return res


def time_config0(ctx, layer_ids, bytes_per_expert, steps=XSTEPS):
    """Config 0: one expert (H=5120, I=1536, K=3) on one token per call: top-1 routing with weight 1.0, the expert id
    cycling over the 288 of each config-1 layer (and the layers cycled), so every call streams a cold expert."""
    import numpy as np
    import torch
    rng = np.random.default_rng(8000)
    routes = []
    for r in range(32):
        x = rng.standard_normal((1, H)).astype(np.float16)
        sel = torch.tensor([[int(rng.integers(0, E))]], dtype=torch.int64, device="cuda")
        w = torch.ones((1, 1), dtype=torch.float32, device="cuda")
        routes.append((torch.from_numpy(x.view(np.int16)).view(torch.float16).cuda(), sel, w, 1))
    r = time_layer_steps(ctx, layer_ids, routes, 1, steps, 4, 8, lambda li: bytes_per_expert)
    r["expert_bytes"] = bytes_per_expert
    return r


def time_shared(ctx, layer_ids, G, reps):
    """Routed layer + the layer's shared expert (one more config-0-shaped expert at 3 bpw), per token: the shared
    expert after the routed call on one stream ("sequential", the stock order); through k_overlap.SharedOverlap with
    overlap requested and the shared expert in its own context only ("overlapped": on a side stream, except at M = 1
    where SharedOverlap keeps the stock order); and with the routed context holding the shared expert too ("fused":
    both in the routed call's launches, gfl_moe_forward_shared). Graph-timed like the decode steps."""
    import numpy as np
    import torch
    import k_overlap
    import synth
    so = k_overlap.SharedOverlap(0)
    sof = k_overlap.SharedOverlap(0)
    keep = []
    for li in layer_ids:
        S = synth.SynthLayer(300 + li, 1, H, I, (KBITS,) * 3)
        so.register(li, H, I, S.Ks, S.ptr_table, keep=S)
        sof.register(li, H, I, S.Ks, S.ptr_table, keep=S, routed=ctx)
        keep.append(S)
    res = {}
    for M in (1, 2, 4):
        routes = make_routes(M, np.random.default_rng(7000 + M), 32, "uniform")
        out = torch.empty((M, H), dtype=torch.float32, device="cuda")
        r = {}
        for mode in ("sequential", "overlapped", "fused"):
            ov = mode != "sequential"
            obj = sof if mode == "fused" else so

            def step(i):
                x, sel, w, _ = routes[i % len(routes)]
                obj.forward(ctx, layer_ids[i % len(layer_ids)], x, sel, w, out, overlap=ov)

            for i in range(8):
                step(i)
            torch.cuda.synchronize()
            st = torch.cuda.Stream()
            st.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(st):
                step(0)
            torch.cuda.current_stream().wait_stream(st)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for i in range(G):
                    step(i)
            warm_graphs([g])
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                g.replay()
            e1.record()
            torch.cuda.synchronize()
            del g
            r[mode] = round(e0.elapsed_time(e1) * 1e3 / (reps * G) / M, 3)
        r["overlap_gain"] = round(r["sequential"] / r["overlapped"], 3)
        r["fused_gain"] = round(r["sequential"] / r["fused"], 3)
        res[f"M{M}_us_per_token"] = r
    return res


def time_router(M, reps=8, G=32):
    """gfl_route on fp32 N(0,1) logits [M, 288] -> top-8 sel / fp16 w: mean µs per call, G calls captured in a HIP
    graph replayed `reps` times (device events around the replays)."""
    import numpy as np
    import torch
    import _native
    lg = torch.from_numpy(np.random.default_rng(6000 + M).standard_normal((M, E)).astype(np.float32)).cuda()
    sel = torch.empty((M, TOPK), dtype=torch.int64, device="cuda")
    w = torch.empty((M, TOPK), dtype=torch.float16, device="cuda")
    for _ in range(3):
        _native.route(lg, TOPK, sel, w)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(G):
            _native.route(lg, TOPK, sel, w)
    warm_graphs([g])
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    del g
    return {"us_per_call": round(e0.elapsed_time(e1) * 1e3 / (reps * G), 2), "tokens": M, "experts": E, "topk": TOPK}


def time_prefill(ctx, layer_ids, bytes_per_expert, M, reps, G=4, exact=False):
    """Config 4 prefill: M tokens, uniform top-8 routing, through gfl_grouped_forward (MFMA grouped GEMMs), or with
    exact=True through gfl_moe_forward in EXACT mode (above 1,024 picks the accumulator-chain GEMMs on the grouped
    plan, bit-identical to the reference's EXACT mode). G layer calls (layers cycled) are captured in one HIP graph and replayed `reps` times.
    Algorithmic work per call: 2 * picks * 3 * H * I flops (gate, up, down GEMMs) and the union's quantized expert
    bytes."""
    import numpy as np
    import torch
    routes = make_routes(M, np.random.default_rng(5000 + M), 2, "uniform")
    out = torch.empty((M, H), dtype=torch.float32, device="cuda")
    NL = len(layer_ids)

    def call(i):
        x, sel, w, _ = routes[i % 2]
        if exact:
            ctx.moe_forward(layer_ids[i % NL], x, sel, w, out, mode=1)
        else:
            ctx.grouped_forward(layer_ids[i % NL], x, sel, w, out)

    for i in range(3):
        call(i)
    torch.cuda.synchronize()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        call(0)
    torch.cuda.current_stream().wait_stream(st)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(G):
            call(i)
    g.replay()
    torch.cuda.synchronize()
    got = out.clone()
    call(G - 1)
    torch.cuda.synchronize()
    graph_ok = bool(torch.equal(got, out))
    warm_graphs([g])
    samples, total = replay_samples([g], reps)
    ms = total / (reps * G)
    del g
    picks = M * TOPK
    flops = 2.0 * picks * 3 * H * I
    tflops = flops / (ms * 1e-3) / 1e12
    union = float(np.mean([r[3] for r in routes]))
    gbps = (union * bytes_per_expert + M * H * 6) / (ms * 1e-3) / 1e9
    # the EXACT chains run on fp32 MFMAs (v_mfma_f32_16x16x1_4b_f32, each element an fmaf), the grouped GEMMs on
    # fp16 MFMAs (v_mfma_f32_16x16x32_f16): each is priced against its own dense peak
    peak = MFMA_FP32_PEAK_TFLOPS if exact else MFMA_PEAK_TFLOPS
    return {"path": "EXACT (gfl_moe_forward)" if exact else "MFMA grouped (gfl_grouped_forward)",
            "tokens": M, "ms_per_layer": round(ms, 4), "us_per_token": round(ms * 1e3 / M, 4),
            "ms_per_layer_replays": [round(t / G, 4) for t in samples],
            "TFLOPs": round(tflops, 1), "mfma_peak_TFLOPs": peak,
            "mfma_peak_kind": "fp32 MFMA (dense)" if exact else "fp16 MFMA (dense)",
            "mfma_frac": round(tflops / peak, 4), "GBps": round(gbps, 1), "union_experts": union,
            "graph_replay_matches_eager": graph_ok}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--mode", choices=("exact", "mfma"), default="exact")
    ap.add_argument("--steps", type=int, default=320)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--layers", type=int, default=4)
    ap.add_argument("--Ms", default="1,2,3,4")
    ap.add_argument("--graph-steps", type=int, default=4,
                    help="most steps per captured graph (the largest divisor of --steps up to this is used)")
    ap.add_argument("--profile-steps", type=int, default=64)
    ap.add_argument("--cpu-iters", type=int, default=300)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the config 2 / 3 / 42-layer-stack measurements (config 1 only)")
    ap.add_argument("--stack-layers", type=int, default=42)
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the config-4 prefill measurement (M=2048 through the grouped path), one JSON line")
    ap.add_argument("--prefill-exact", action="store_true",
                    help="with --prefill-only: the EXACT path (gfl_moe_forward, accumulator chains) instead")
    ap.add_argument("--shared-only", action="store_true",
                    help="only the routed + shared expert measurement (stock order, overlapped, fused), one JSON line")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="counter run: the calibration copy, then eager M=1 steps (run under rocprofv3 --pmc)")
    ap.add_argument("--probe-M", type=int, default=1, help="tokens per layer call of --pmc-probe")
    ap.add_argument("--pmc-table", nargs="+", metavar="DIR",
                    help="print per-kernel counter means and kernel-trace durations of rocprofv3 output folders")
    ap.add_argument("--pmc-digest", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="turn two rocprofv3 --pmc output folders (FETCH_SIZE, WRITE_SIZE) into the traffic file")
    args = ap.parse_args()
    if args.pmc_digest:
        pmc_digest(*args.pmc_digest)
        return
    if args.pmc_table:
        pmc_table(args.pmc_table)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures the routed-expert path on one GPU; multi-GPU runs are not part of this build "
              "(run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    import _native
    import synth
    global MODE
    MODE = _native.MODE_MFMA if args.mode == "mfma" else _native.MODE_EXACT

    torch.cuda.set_device(0)
    ctx = _native.Context(0)
    t0 = time.time()
    layers = []
    for li in range(args.layers):
        L = synth.SynthLayer(li, E, H, I, (KBITS,) * 3)
        L.register(ctx, li)
        layers.append(L)
    setup_s = time.time() - t0
    if args.pmc_probe:
        pmc_probe(ctx, layers, M=args.probe_M)
        return
    if args.shared_only:
        print(json.dumps({"shared_overlap": time_shared(ctx, list(range(args.layers)), 32, 4)}), flush=True)
        return
    if args.prefill_only:
        if args.prefill_exact:
            r = time_prefill(ctx, list(range(args.layers)), layers[0].quant_bytes_per_expert, 2048, 2, G=2,
                             exact=True)
            print(json.dumps({"config4_prefill_exact": r}), flush=True)
            return
        r = time_prefill(ctx, list(range(args.layers)), layers[0].quant_bytes_per_expert, 2048,
                         max(4, args.steps // 64))
        print(json.dumps({"config4_prefill": r}), flush=True)
        return
    per_expert = layers[0].quant_bytes_per_expert
    gu_per_expert = layers[0].tbytes[0] + layers[0].tbytes[1] + 2 * 2 * (H + I)
    steps = max(1, args.steps)
    G = graph_size(steps, args.graph_steps)
    per_M, e2e = {}, {}
    roof = None
    for M in [int(m) for m in args.Ms.split(",")]:
        rng = np.random.default_rng(1000 + M)
        routes = make_routes(M, rng, 32, "uniform")
        r = time_layer_steps(ctx, list(range(args.layers)), routes, M, steps, G, args.warmup,
                             lambda li: layers[li].quant_bytes_per_expert)
        per_M[str(M)] = r
        e2e[str(M)] = time_e2e_steps(ctx, list(range(args.layers)), M, min(steps, XSTEPS),
                                     graph_size(min(steps, XSTEPS), args.graph_steps), 8, per_expert)
        if M == 1:
            # live per-kernel timing of the dominant kernel (gate|up GEMV): start/stop events on every launch's dispatch
            out = torch.empty((1, H), dtype=torch.float32, device="cuda")
            NR = len(routes)
            ctx.profile(True)
            torch.cuda.synchronize()
            for i in range(args.profile_steps):
                x, sel, w, _ = routes[i % NR]
                ctx.moe_forward(i % args.layers, x, sel, w, out, mode=MODE)
            prof = ctx.profile_read()
            ctx.profile(False)
            gu_ms, gu_n = prof["gate_up"]
            gu_bytes = float(np.mean([routes[i % NR][3] for i in range(args.profile_steps)])) * gu_per_expert
            ach = gu_bytes / (gu_ms / gu_n * 1e-3) / 1e9
            stage_us = {k: round(v[0] / max(1, v[1]) * 1e3, 2) for k, v in prof.items()}
            roof = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                    "frac": round(ach / HBM_PEAK_GBPS, 4), "traffic": None, "kernel": GATE_UP_KERNEL + " (gate|up GEMV + SwiGLU)",
                    "algorithmic_bytes_per_launch": round(gu_bytes), "mean_launch_us": round(gu_ms / gu_n * 1e3, 2),
                    "stage_mean_us": stage_us}
    configs = {}
    if not args.no_extra:
        configs = extra_configs(ctx, layers, args)
    if roof is not None and os.path.exists(TRAFFIC_FILE):
        try:
            roof["traffic"] = json.load(open(TRAFFIC_FILE)).get("hbm_bytes_per_launch")
        except (OSError, ValueError):
            pass
    cpu = None if args.no_cpu else cpu_baseline(args.cpu_iters, 20)
    m1 = per_M.get("1") or next(iter(per_M.values()))
    line = {"metric": METRIC, "value": m1["us_per_token"], "unit": "us/token", "n_gpus": 1, "steps": steps,
            "warmup": args.warmup, "ms_per_step": m1["ms_per_step"], "higher_is_better": False, "scaling": "weak",
            "vs_baseline": None, "dtype": "f32 (fp16 operands)", "data": "synthetic",
            "config": {"workload": "config1: one 288-expert top-8 MoE layer decode, M=1, H=5120 I=1536 K=3 bpw",
                       "experts": E, "topk": TOPK, "hidden": H, "intermediate": I, "bits": KBITS,
                       "layers_cycled": args.layers, "graph_steps": G},
            "per_M": per_M, "per_M_end_to_end": e2e, "configs": configs, "roofline": roof, "cpu_baseline": cpu, "setup_s": round(setup_s, 1)}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
