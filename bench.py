#!/usr/bin/env python3
"""Recall hot path on one MI355X: select + stage-in per layer at 128K context.

Workload (default): a 64-layer stack, 131072 tokens per layer, 8 kv-heads x
head_dim 128, fp16 K and V, pages of 256 tokens (512 pages), one decode query
row of 32 q-heads (GQA group 4), Mean head aggregation, top-32 pages per
layer gathered (K and V) from pinned host history into an 8192-token device
slot array per layer.  K is resident in HBM for scoring; page summaries are
rebuilt from it inside every select.

Timed step: scoring + selection of the whole stack, one kvr_recall_stack
call (layer l's softmax/top-k inside layer l+1's summary launch, one select
stream, descriptors built beforehand).

Reported:
  value        scored-KV GB/s = layers x (K bytes + fp16 summary bytes +
               Q bytes) / step time
  roofline     the stack launch (dominant): algorithmic bytes per launch /
               its mean duration (HIP events the library records around it on
               the select stream, inside the timed steps, on sampled layers)
  latency      select + stage-in per layer with every layer's stage-in on one
               copy stream beside the following selects (latency_us_per_layer)
  stage-in     gather GB/s per layer (separate pass) vs measured pinned H2D peak
  cpu_baseline the reference's own CPU select path (oracle/_ref: RawKvStore
               fp16 capture + mean_k + page_softmax_scores + pick_scored_blocks),
               single thread, on a bounded sample of layers
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_baseline(args, geo, gpu_selection, dev_k, dev_q):
    """The reference's CPU select path on a bounded sample of layers, fed the
    same K and Q the GPU scored (copied back)."""
    import oracle as O
    T, HKV, D, PT, HQ, KSEL = geo["T"], geo["HKV"], geo["D"], geo["PT"], geo["HQ"], geo["K"]
    W = HKV * D
    kind = "reference" if O.ref_available() else "port"
    times, match = [], True
    budget_s = args.cpu_seconds
    t_start = time.perf_counter()
    layer = 0
    while layer < geo["L"] and (layer < 1 or time.perf_counter() - t_start < budget_s):
        keys = dev_k[layer].cpu().numpy().view(np.uint16).reshape(1, T, W)
        q = dev_q[layer].cpu().numpy().view(np.float16).astype(np.float32).reshape(1, 1, HQ, D)
        t0 = time.perf_counter()
        if kind == "reference":
            _, scores = O.ref_scores_f16_keys(keys, T, HKV, D, PT, q, [1], HQ, O.AGG_MEAN)
            sel = O.ref_pick_scored_blocks(scores, KSEL)
        else:
            _, means = O.page_summaries(keys[0], O.FMT_F16, T, W, PT)
            scores = O.page_softmax_scores(means[None], q, [1], HQ, HKV, D, O.AGG_MEAN)
            sel = O.pick_scored_blocks(scores, KSEL, (), O.TIE_HIGHER_FIRST)
        times.append(time.perf_counter() - t0)
        match &= bool(np.array_equal(sel, gpu_selection[layer]))
        layer += 1
    per_layer = float(np.mean(times))
    return {
        "value": round(geo["scored_bytes"] / per_layer / 1e9, 4),
        "unit": "GB/s",
        "cores": 1,
        "kind": kind,
        "sample": f"{len(times)} of {geo['L']} layers, select path (summaries from fp16 K + page "
                  f"softmax + top-{KSEL}), {per_layer * 1e3:.1f} ms per layer, single thread",
        "select_us_per_layer": round(per_layer * 1e6, 1),
        "selection_matches_gpu": match,
        "host_cpu": _cpu_model(),
        "host_cores": os.cpu_count(),
    }


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def run(args):
    import torch
    import kvmem_amd as K
    from kvmem_amd.hip import runtime

    hip = runtime()
    ctxs = [K.Context(0)]
    for c in ctxs:
        c.set_option(K._capi.OPT_GATHER_WORKGROUPS, args.gather_wgs)
        c.set_option(K._capi.OPT_GATHER_CHUNK_ROWS, args.chunk_rows)
        c.set_option(K._capi.OPT_GATHER_THREADS, args.gather_threads)
    ctx = ctxs[0]
    L, T, HKV, D, HQ, PT, KSEL, R = args.layers, 131072, 8, 128, 32, 256, 32, 1
    G = K._capi.STACK_GROUP  # layers per stack launch
    W = HKV * D
    P = T // PT
    geo = dict(L=L, T=T, HKV=HKV, D=D, HQ=HQ, PT=PT, K=KSEL)
    k_bytes = T * W * 2
    geo["scored_bytes"] = k_bytes + P * W * 2 + HQ * D * 2
    plane_bytes = T * W * 2
    stage_bytes = 2 * KSEL * PT * W * 2  # K and V of the selected pages, fp16
    log(f"workload: {L} layers x {T} tokens, Hq {HQ}/Hkv {HKV}, D {D}, page {PT} ({P} pages), top-{KSEL}")

    # ---- inputs: resident K per layer; pinned K/V history per layer --------
    dev_k = torch.empty((L, T * W), dtype=torch.int16, device="cuda")
    dev_q = torch.empty((L, HQ * D), dtype=torch.int16, device="cuda")
    tmp_v = torch.empty(T * W, dtype=torch.int16, device="cuda")
    torch.cuda.synchronize()
    ring = L
    pins = []
    try:
        for l in range(L):
            pins.append((K.PinnedBuffer(plane_bytes), K.PinnedBuffer(plane_bytes)))
    except K.KvrError as e:
        ring = max(1, len(pins))
        log(f"pinned allocation stopped at {len(pins)} layers ({e}); aliasing a ring of {ring}")
    for l in range(L):
        src = l % ring
        ctx.synth_normal_f16(args.seed, 1000 + src, T * W, dev_k[l])
        ctx.synth_normal_f16(args.seed, 3000 + src, HQ * D, dev_q[l])
        if l < ring:
            ctx.check()
            hip.d2h(pins[l][0].ptr, dev_k[l].data_ptr(), plane_bytes)
            ctx.synth_normal_f16(args.seed, 2000 + src, T * W, tmp_v)
            ctx.check()
            hip.d2h(pins[l][1].ptr, tmp_v.data_ptr(), plane_bytes)
    ctx.check()
    del tmp_v
    log(f"inputs ready ({L} x {plane_bytes >> 20} MiB resident K, {ring} x 2 x {plane_bytes >> 20} MiB pinned)")

    s16 = torch.empty((L, P * W), dtype=torch.int16, device="cuda")
    scores = torch.empty((L, P), dtype=torch.float64, device="cuda")
    sel = torch.empty((L, KSEL), dtype=torch.int32, device="cuda")
    cnt = torch.empty((L, 1), dtype=torch.int32, device="cuda")
    kslots = torch.empty((L, KSEL * PT * W), dtype=torch.int16, device="cuda")
    vslots = torch.empty((L, KSEL * PT * W), dtype=torch.int16, device="cuda")
    torch.cuda.synchronize()

    engine = {"auto": K.ENGINE_AUTO, "kernel": K.ENGINE_KERNEL, "sdma": K.ENGINE_SDMA}[args.engine]
    keys = [K.make_keys(dev_k[l], K.FMT_F16, T, HKV, D, PT) for l in range(L)]
    queries = [K.make_query(dev_q[l], K.FMT_F16, R, HQ, HKV, D) for l in range(L)]
    planes = [[K.make_plane(pins[l % ring][0], K.FMT_F16, W, T, K.GATHER_COPY, kslots[l]),
               K.make_plane(pins[l % ring][1], K.FMT_F16, W, T, K.GATHER_COPY, vslots[l])] for l in range(L)]
    copy_stream = ctx.copy_stream  # every layer's stage-in, in layer order

    # Every event recorded between two kernels of the select stream costs a
    # few microseconds of stream time, so per-layer events go on a sample of
    # layers (three inside the stack, plus the first and last for its span).
    sampled = sorted({0, L // 4, L // 2, 3 * L // 4, L - 1})

    def events():
        return {n: {l: hip.event() for l in sampled} for n in ("kb", "ke", "se")}

    def descriptors(ev, with_planes):
        return [K.Context.layer_recall(keys=keys[l], summaries=s16[l], query=queries[l], scores=scores[l],
                                       selected=sel[l], count=cnt[l], k=KSEL, aggregation=K.AGG_MEAN,
                                       planes=planes[l] if with_planes else (), engine=engine,
                                       summary_events=(ev["kb"][l], ev["ke"][l]) if l in ev["kb"] else (None, None),
                                       select_end=ev["se"].get(l))
                for l in range(L)]

    def stack(descs, ev):
        # one call per stack: layer l's softmax/top-k runs inside layer l+1's
        # summary launch
        keep.append(ctx.recall_stack(descs, None, copy_stream))

    keep = []

    def drain():
        for c in ctxs:
            c.check()
        keep.clear()

    def layer_times(ev):
        """sampled layers: summary kernel, summary start -> selection written"""
        inner = [l for l in sampled if 0 < l < L - 1] or sampled
        kern = [hip.elapsed_ms(ev["kb"][l], ev["ke"][l]) * 1e3 for l in inner]
        selt = [hip.elapsed_ms(ev["kb"][l], ev["se"][l]) * 1e3 for l in inner]
        return kern, selt, hip.elapsed_ms(ev["kb"][0], ev["se"][L - 1]) * 1e3

    # ---- timed: scoring + selection of the whole stack ----------------------
    ev_w = events()
    d_w = descriptors(ev_w, False)
    for _ in range(args.warmup):
        stack(d_w, ev_w)
        drain()
    ev_t = [events() for _ in range(args.steps)]
    d_t = [descriptors(e, False) for e in ev_t]
    drain()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(args.steps):
        stack(d_t[s], ev_t[s])
    drain()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_per_step = (t1 - t0) * 1e3 / args.steps
    kern_us, sel_us, stack_us = [], [], []
    for e in ev_t:
        a, b, c = layer_times(e)
        kern_us += a
        sel_us += b
        stack_us.append(c)
    kern_us_mean = float(np.mean(kern_us))
    select_us = float(np.mean(sel_us))
    stack_gpu_us = float(np.mean(stack_us))
    log(f"select stack {ms_per_step:.3f} ms/step ({ms_per_step / L * 1e3:.1f} us/layer; GPU "
        f"{stack_gpu_us / L:.1f} us/layer); stack launch ({G} layers) {kern_us_mean:.1f} us, "
        f"summary start -> selection {select_us:.1f} us")

    # ---- one layer alone (kvr_recall_layer): summary start -> selection ---
    ev_a, ev_b = hip.event(), hip.event()
    lone = []
    for rep in range(max(3, args.steps)):
        for l in range(min(L, 4)):
            ctx.recall(K.Context.layer_recall(keys=keys[l], summaries=s16[l], query=queries[l], scores=scores[l],
                                              selected=sel[l], count=cnt[l], k=KSEL, aggregation=K.AGG_MEAN,
                                              summary_events=(ev_a, None), select_end=ev_b))
            ctx.check()
            if rep:
                lone.append(hip.elapsed_ms(ev_a, ev_b) * 1e3)
    lone_us = float(np.median(lone))
    log(f"one layer alone (kvr_recall_layer): summary start -> selection {lone_us:.1f} us")

    # ---- pipelined recall: each layer's stage-in beside the next selects ---
    ev_p = events()
    d_p = descriptors(ev_p, True)
    for rep in range(2):
        drain()
        p0 = time.perf_counter()
        stack(d_p, ev_p)
        drain()
        p1 = time.perf_counter()
    pipe_us = (p1 - p0) * 1e6 / L
    pk, ps, _ = layer_times(ev_p)
    pipe_kern_us, pipe_sel_us = float(np.mean(pk)), float(np.mean(ps))
    log(f"select+stage-in pipelined {pipe_us:.1f} us/layer; beside the stage-in: stack launch "
        f"{pipe_kern_us:.1f} us, summary start -> selection {pipe_sel_us:.1f} us")

    # ---- stage-in alone (same selections, copy stream) ---------------------
    stage_us = []
    a, b = hip.event(), hip.event()
    for rep in range(2):
        for l in range(L):
            hip.record(a, copy_stream)
            ctx.stage_in(planes[l], PT, sel[l], cnt[l], KSEL, engine=engine)
            hip.record(b, copy_stream)
            ctx.check()
            if rep:
                stage_us.append(hip.elapsed_ms(a, b) * 1e3)
    stage_us = float(np.mean(stage_us))
    h2d = ctx.h2d_peak_gbps(1 << 30, 5)
    stage_gbps = stage_bytes / (stage_us * 1e-6) / 1e9
    log(f"stage-in {stage_us:.1f} us/layer = {stage_gbps:.2f} GB/s; pinned H2D peak {h2d:.2f} GB/s")

    gpu_sel = sel.cpu().numpy().view(np.uint32)
    assert (cnt.cpu().numpy() == KSEL).all(), "every layer must select k pages"

    # one stack launch, per layer of its group: the layer's K read and fp16
    # summaries written; per layer of the previous group: summaries and Q
    # read (logits stay in LDS), terms written and read back, scores written
    logit_bytes = HQ * R * P * 8
    alg_kernel_bytes = G * (k_bytes + 2 * P * W * 2 + HQ * D * 2 + 2 * logit_bytes + P * 8)
    achieved = alg_kernel_bytes / (kern_us_mean * 1e-6) / 1e9
    scored_gbps = L * geo["scored_bytes"] / (ms_per_step * 1e-3) / 1e9
    traffic = None
    pmc = os.path.join(ROOT, "profiles", "pmc_stack_resident64.json")
    if os.path.exists(pmc):
        try:
            traffic = json.load(open(pmc)).get("traffic_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None

    line = {
        "metric": "select+stage-in latency/layer at 128K ctx; scored-KV GB/s vs HBM peak",
        "value": round(scored_gbps, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 operands, f32 summaries, f64 scores",
        "data": f"synthetic seeded N(0,1) (Box-Muller), seed {args.seed}",
        "config": {
            "workload": "resident-history scoring + recall, 64-layer stack at 131072 tokens",
            "step": "summaries + scores + softmax + top-k for every layer (scored-KV throughput); "
                    "stage-in measured pipelined and alone beside it",
            "layers": L, "tokens": T, "kv_heads": HKV, "head_dim": D, "query_heads": HQ,
            "query_rows": R, "page_tokens": PT, "pages": P, "top_k": KSEL,
            "aggregation": "mean", "gather": "fp16 K+V copy into 8192-token slots",
            "engine": args.engine, "pinned_layers": ring,
            "gather_workgroups": args.gather_wgs or "16 x 64 threads (copy default)", "gather_chunk_rows": args.chunk_rows or 8,
        },
        "select_us_per_layer": round(select_us, 2),
        "select_one_layer_us": round(lone_us, 2),
        "select_stack_us_per_layer": round(ms_per_step / L * 1e3, 2),
        "scored_frac_hbm": round(scored_gbps / HBM_PEAK_GBPS, 4),
        "latency_us_per_layer": round(pipe_us, 2),
        "select_us_beside_stagein": round(pipe_sel_us, 2),
        "summary_kernel_beside_stagein_us": round(pipe_kern_us, 2),
        "stagein_us_per_layer": round(stage_us, 2),
        "stagein_GBps": round(stage_gbps, 3),
        "h2d_peak_GBps": round(h2d, 3),
        "stagein_frac_h2d": round(stage_gbps / h2d, 4),
        "roofline": {
            "bound": "hbm",
            "kernel": f"k_stack_group<f16> ({G} layers' summaries beside the previous {G} layers' "
                      "logits, softmax and top-k)",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "bytes_per_launch": alg_kernel_bytes,
            "mean_launch_us": round(kern_us_mean, 3),
        },
    }
    if not args.no_cpu:
        log("CPU baseline ...")
        line["cpu_baseline"] = cpu_baseline(args, geo, gpu_sel, dev_k, dev_q)
    for c in ctxs:
        c.close()
    print(json.dumps(line), flush=True)


def calibration_copies(ctx) -> int:
    """Three device copies of 256 MiB in 64 KiB ops (k_copy_ops): known byte
    counts that calibrate FETCH_SIZE / WRITE_SIZE in a counter pass."""
    import torch
    op, cb = 1 << 16, 256 << 20
    src_t = torch.empty(cb, dtype=torch.uint8, device="cuda")
    dst_t = torch.empty(cb, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    n = cb // op
    for _ in range(3):
        ctx.d2d_batched([src_t.data_ptr() + i * op for i in range(n)], [dst_t.data_ptr() + i * op for i in range(n)],
                        [op] * n)
        ctx.check()
    return cb


def pmc_pass(args):
    """Counter pass (run under rocprofv3 --pmc): a stack of eight distinct
    128K-token layers in three launches (k_stack_group: the first group's
    summaries alone, then the second group's beside the first group's
    selections, then the second group's selections alone) and three 256 MiB
    device copies (4096 ops of 64 KiB, k_copy_ops) that calibrate
    FETCH_SIZE / WRITE_SIZE against known byte counts."""
    import torch
    import kvmem_amd as K
    T, HKV, D, HQ, PT, KSEL = 131072, 8, 128, 32, 256, 32
    W, P = HKV * D, T // PT
    L = 2 * K._capi.STACK_GROUP
    ctx = K.Context(0)
    kd = torch.empty((L, T * W), dtype=torch.int16, device="cuda")
    qd = torch.empty((L, HQ * D), dtype=torch.int16, device="cuda")
    dst = torch.empty(T * W, dtype=torch.int16, device="cuda")
    s16 = torch.empty((L, P * W), dtype=torch.int16, device="cuda")
    scores = torch.empty((L, P), dtype=torch.float64, device="cuda")
    sel = torch.empty((L, KSEL), dtype=torch.int32, device="cuda")
    cnt = torch.empty((L, 1), dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    for l in range(L):
        ctx.synth_normal_f16(args.seed, 1000 + l, T * W, kd[l])
        ctx.synth_normal_f16(args.seed, 3000 + l, HQ * D, qd[l])
    ctx.check()
    descs = [K.Context.layer_recall(keys=K.make_keys(kd[l], K.FMT_F16, T, HKV, D, PT),
                                    summaries=s16[l], query=K.make_query(qd[l], K.FMT_F16, 1, HQ, HKV, D),
                                    scores=scores[l], selected=sel[l], count=cnt[l], k=KSEL,
                                    aggregation=K.AGG_MEAN) for l in range(L)]
    keep = ctx.recall_stack(descs)
    ctx.check()
    del keep
    op = 1 << 16
    n = T * W * 2 // op
    srcs = [kd[0].data_ptr() + i * op for i in range(n)]
    dsts = [dst.data_ptr() + i * op for i in range(n)]
    for _ in range(3):
        ctx.d2d_batched(srcs, dsts, [op] * n)
        ctx.check()
    ctx.close()
    print(json.dumps({"pass": "pmc", "layers": L, "summary_bytes_read": T * W * 2 + HQ * D * 2,
                      "copy_bytes": T * W * 2, "copy_ops": n}), flush=True)


# ---------------------------------------------------------------------------
# The other workloads (--workload).  Each prints one JSON line of the same
# shape: value = scored-KV GB/s of the select stack, the per-layer select
# latency, select+stage-in pipelined latency and stage-in GB/s, the roofline
# of the dominant launch, the reference's CPU select path on a bounded sample
# and a parity check of every layer's (lane's) selection against the oracle.
WORKLOADS = {
    # 64 distinct 32768-token layers (4 GiB of K: HBM, not the 256 MB cache),
    # K = N(0,1) x per-channel U(0.5, 2), Max, top-16
    "single32k": dict(layers=64, repeat=1, lanes=1, T=32768, HQ=32, HKV=8, D=128, PT=256, R=1, K=16,
                      agg="max", kfmt="f16_scaled", vfmt="f16", kmode="copy", vmode="copy", resident=False, ring=8),
    # q8_0 K (scores from dequantized K) + q4_1-layout V, dequantized on gather
    "k8v4": dict(layers=16, repeat=1, lanes=1, T=131072, HQ=32, HKV=8, D=128, PT=256, R=1, K=32,
                 agg="mean", kfmt="q8_0", vfmt="q4_1", kmode="dequant", vmode="dequant", resident=False),
    # 8 lanes x 262144 tokens, 40/8 heads, 4 query rows (matrix-core logits), top-64 per lane
    "lanes8": dict(layers=1, repeat=8, lanes=8, T=262144, HQ=40, HKV=8, D=128, PT=256, R=4, K=64,
                   agg="mean", kfmt="f16", vfmt="f16", kmode="copy", vmode="copy", resident=False),
    # raw q8_0 K staged with the transform (decode, NeoX RoPE at the original
    # position, Walsh-Hadamard over 128, requantize) + fp16 V copied
    "rawk": dict(layers=16, repeat=1, lanes=1, T=131072, HQ=32, HKV=8, D=128, PT=256, R=1, K=32,
                 agg="mean", kfmt="q8_0", vfmt="f16", kmode="rope_fwht", vmode="copy", resident=False),
    # 40 layers x 1048576 tokens, 16/2 heads, D 256, q8_0 K + fp16 V, resident
    # summaries, top-48 (pinned history aliased over a ring of 4 layers)
    "layerwise40": dict(layers=40, repeat=1, lanes=1, T=1048576, HQ=16, HKV=2, D=256, PT=256, R=1, K=48,
                        agg="mean", kfmt="q8_0", vfmt="f16", kmode="dequant", vmode="copy", resident=True,
                        ring=4),
}


def _q8_rows_f32(raw: np.ndarray, width: int) -> np.ndarray:
    """q8_0 token rows -> binary32 rows (code * d, exact)."""
    blk = raw.reshape(-1, 34)
    d = blk[:, :2].copy().view(np.float16).astype(np.float32)
    return (blk[:, 2:].view(np.int8).astype(np.float32) * d).reshape(-1, width)


def workload_checks(args, w, name, host_units, gpu_sel, gpu_scores, tie, scored_unit_bytes):
    """Parity of every unit (layer or lane) against the oracle, and the
    reference's own CPU select path on a bounded sample of units.
    host_units: callables returning (kind, data, query) per unit, where kind
    is 'f16' (uint16 keys), 'q8_0' (raw bytes) or 'summaries' (fp16)."""
    import oracle as O
    T, HQ, HKV, D, PT, R, KSEL = w["T"], w["HQ"], w["HKV"], w["D"], w["PT"], w["R"], w["K"]
    W = HKV * D
    agg = {"mean": O.AGG_MEAN, "max": O.AGG_MAX}[w["agg"]]
    equal, worst = True, 0.0
    ref_kind = "reference" if O.ref_available() else "port"
    cpu_times, ref_match = [], True
    t_start = time.perf_counter()
    for u, fetch in enumerate(host_units):
        kind, data, q = fetch()
        q4 = q.reshape(1, R, HQ, D)
        if kind == "summaries":
            means = data.view(np.float16).astype(np.float32).reshape(1, -1, W)
        else:
            _, m = O.page_summaries(data, O.FMT_F16 if kind == "f16" else O.FMT_Q8_0, T, W, PT)
            means = m[None]
        want = O.page_softmax_scores(means, q4, [R], HQ, HKV, D, agg)
        worst = max(worst, float(np.max(np.abs(gpu_scores[u] - want) / np.maximum(want, 1e-300))))
        equal &= bool(np.array_equal(gpu_sel[u], O.pick_scored_blocks(want, KSEL, (), tie)))
        if args.no_cpu or (cpu_times and time.perf_counter() - t_start > args.cpu_seconds):
            continue
        # the reference's select path: capture, mean-K, page softmax, pick
        c0 = time.perf_counter()
        if ref_kind == "reference":
            if kind == "f16":
                _, sc = O.ref_scores_f16_keys(data.reshape(1, T, W), T, HKV, D, PT, q4, [R], HQ, agg)
            elif kind == "q8_0":
                _, sc = O.ref_scores_f32_keys(_q8_rows_f32(data, W)[None], T, HKV, D, PT, q4, [R], HQ, agg)
            else:
                sc = O.ref_scores_from_sums(means * np.float32(PT), HKV, D, PT, q4, [R], HQ, agg)
            pick = O.ref_pick_scored_blocks(sc, KSEL)
        else:
            sc, pick = want, O.pick_scored_blocks(want, KSEL, (), O.TIE_HIGHER_FIRST)
        cpu_times.append(time.perf_counter() - c0)
        ref_match &= bool(np.array_equal(pick, gpu_sel[u]))
    parity = {"units_checked": len(host_units), "selections_equal": equal, "max_rel_score_diff": worst,
              "oracle": "oracle/kvr_oracle.c summaries + page softmax + pick with the GPU's tie rule"}
    cpu = None
    if cpu_times:
        per = float(np.mean(cpu_times))
        src = {"f16": "fp16 K capture (write_layer_tokens_f16)", "q8_0": "dequantized q8_0 K capture "
               "(write_layer_mean_k)", "summaries": "resident page sums (write_layer_mean_sum)"}[kind]
        cpu = {"value": round(scored_unit_bytes / per / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": ref_kind,
               "sample": f"{len(cpu_times)} of {len(host_units)} {name}s, select path ({src} + mean_k + "
                         f"page_softmax_scores + pick_scored_blocks), {per * 1e3:.1f} ms each, single thread",
               "select_us_per_unit": round(per * 1e6, 1), "selection_matches_gpu": ref_match,
               "host_cpu": _cpu_model(), "host_cores": os.cpu_count()}
    return parity, cpu


def run_workload(args):
    import torch
    import kvmem_amd as K
    from kvmem_amd.hip import runtime

    w = dict(WORKLOADS[args.workload])
    if args.pmc_pass:  # a short stack: three launches of distinct layers
        w["layers"] = min(w["layers"], 2 * K._capi.STACK_GROUP) if w["lanes"] == 1 else 1
        w["repeat"] = 1
        w["ring"] = min(w.get("ring", w["layers"]), w["layers"])
    hip = runtime()
    ctx = K.Context(0)
    ctx.set_option(K._capi.OPT_GATHER_WORKGROUPS, args.gather_wgs)
    ctx.set_option(K._capi.OPT_GATHER_CHUNK_ROWS, args.chunk_rows)
    ctx.set_option(K._capi.OPT_GATHER_THREADS, args.gather_threads)
    L, NL, T, HQ, HKV, D, PT, R, KSEL = w["layers"], w["lanes"], w["T"], w["HQ"], w["HKV"], w["D"], w["PT"], \
        w["R"], w["K"]
    G = K._capi.STACK_GROUP
    W, P = HKV * D, T // PT
    ring = w.get("ring", L)
    fmt = {"f16": K.FMT_F16, "f16_scaled": K.FMT_F16, "q8_0": K.FMT_Q8_0, "q4_1": K.FMT_Q4_1}
    row = lambda f: K.row_bytes(fmt[f], W)
    kfmt, vfmt = fmt[w["kfmt"]], fmt[w["vfmt"]]
    mode = {"copy": K.GATHER_COPY, "dequant": K.GATHER_DEQUANT_F16, "rope_fwht": K.GATHER_ROPE_FWHT}
    # rotation angles of the raw-K transform: theta_i = 10000^(-2i/D)
    theta = torch.from_numpy((10000.0 ** (-np.arange(D // 2) * 2 / D)).astype(np.float32)).cuda()
    rope = dict(head_dim=D, n_rot=D, theta=theta, fwht=128, pos_base=0) if w["kmode"] == "rope_fwht" else None
    agg = {"mean": K.AGG_MEAN, "max": K.AGG_MAX}[w["agg"]]
    tie = K.TIE_LOWER_FIRST
    seed = args.seed
    log(f"workload {args.workload}: {L} layer(s) x {NL} lane(s) x {T} tokens, Hq {HQ}/Hkv {HKV}, D {D}, "
        f"page {PT} ({P} pages), {R} query row(s), top-{KSEL}, K {w['kfmt']}, V {w['vfmt']}")

    def synth(f, sid, nrows, out):
        n = nrows * W
        if f == "f16":
            ctx.synth_normal_f16(seed, sid, n, out)
        elif f == "f16_scaled":
            # per-(kv-head, dim) channel scale U(0.5, 2)
            scale = torch.from_numpy(np.random.default_rng(seed + sid).uniform(0.5, 2.0, W).astype(np.float32))
            scale = scale.cuda()
            torch.cuda.synchronize()
            ctx.synth_scaled_normal_f16(seed, sid, nrows, W, scale, out)
        elif f == "q8_0":
            if w["resident"]:
                ctx.synth_normal_q8_0(seed, sid, n // 32, out)
            else:
                ctx.synth_q8_0(seed, sid, n // 32, 0.01, 0.05, out)
        elif f == "q4_1":
            ctx.synth_q4_1(seed, sid, n // 32, 0.01, 0.05, -0.4, 0.0, out)
        ctx.check()

    lane_rows = NL * T
    kb, vb = lane_rows * row(w["kfmt"]), lane_rows * row(w["vfmt"])
    pins, s16, dev_k = [], [], []
    tmp = torch.empty(max(kb, vb), dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    for r in range(ring):
        pk, pv = K.PinnedBuffer(kb), K.PinnedBuffer(vb)
        synth(w["kfmt"], 1000 + r, lane_rows, tmp)
        hip.d2h(pk.ptr, tmp.data_ptr(), kb)
        if w["resident"]:
            srow = torch.empty(NL * P * W, dtype=torch.int16, device="cuda")
            torch.cuda.synchronize()
            ctx.summary_build(K.make_keys(tmp, kfmt, T, HKV, D, PT, lanes=NL), None, srow)
            ctx.check()
            s16.append(srow)
        synth(w["vfmt"], 2000 + r, lane_rows, tmp)
        hip.d2h(pv.ptr, tmp.data_ptr(), vb)
        pins.append((pk, pv))
    del tmp
    if not w["resident"]:
        for l in range(L):
            t = torch.empty(kb, dtype=torch.uint8, device="cuda")
            torch.cuda.synchronize()
            synth(w["kfmt"], 1000 + l, lane_rows, t)  # distinct K per layer
            dev_k.append(t)
    else:
        s16 = [s16[l % ring].clone() for l in range(L)]
    qd = []
    for l in range(L):
        q = torch.empty(NL * R * HQ * D, dtype=torch.int16, device="cuda")
        torch.cuda.synchronize()
        ctx.synth_normal_f16(seed, 3000 + l, q.numel(), q)
        qd.append(q)
    if not w["resident"]:
        s16 = [torch.empty(NL * P * W, dtype=torch.int16, device="cuda") for _ in range(L)]
    order = [l for l in range(L) for _ in range(w["repeat"])]
    N = len(order)  # stack positions (a layer may be scored more than once)
    scores = [torch.empty(NL * P, dtype=torch.float64, device="cuda") for _ in range(N)]
    sel = [torch.empty(NL * KSEL, dtype=torch.int32, device="cuda") for _ in range(N)]
    cnt = [torch.empty(NL, dtype=torch.int32, device="cuda") for _ in range(N)]
    kslots = [torch.empty(NL * KSEL * PT * K.gather_row_bytes(kfmt, mode[w["kmode"]], W), dtype=torch.uint8,
                          device="cuda") for _ in range(L)]
    vslots = [torch.empty(NL * KSEL * PT * K.gather_row_bytes(vfmt, mode[w["vmode"]], W), dtype=torch.uint8,
                          device="cuda") for _ in range(L)]
    torch.cuda.synchronize()
    ctx.check()
    log(f"inputs ready ({L} distinct layer(s); {ring} pinned K/V set(s) of {kb >> 20} + {vb >> 20} MiB)")

    def desc(i, with_planes, ev=(None, None), se=None):
        l = order[i]
        planes = [K.make_plane(pins[l % ring][0], kfmt, W, T, mode[w["kmode"]], kslots[l], rope=rope),
                  K.make_plane(pins[l % ring][1], vfmt, W, T, mode[w["vmode"]], vslots[l])]
        src = dict(keys=None, pages=P, page_tokens=PT, lanes=NL) if w["resident"] else \
            dict(keys=K.make_keys(dev_k[l], kfmt, T, HKV, D, PT, lanes=NL))
        return K.Context.layer_recall(summaries=s16[l], query=K.make_query(qd[l], K.FMT_F16, R, HQ, HKV, D, lanes=NL),
                                      scores=scores[i], selected=sel[i], count=cnt[i], k=KSEL, aggregation=agg,
                                      tie_rule=tie, planes=planes if with_planes else (), summary_events=ev,
                                      select_end=se, **src)

    fused = R * (HQ // HKV) < 16  # vector logits: layers fuse into stack launches of G
    if args.pmc_pass:
        keep = ctx.recall_stack([desc(i, False) for i in range(N)])
        ctx.check()
        del keep
        cb = calibration_copies(ctx)
        ctx.close()
        print(json.dumps({"pass": "pmc", "workload": args.workload, "layers": N, "copy_bytes": cb,
                          "copy_ops": cb >> 16}), flush=True)
        return

    # (a) select latency of one layer: summary start -> selection written
    ev_a, ev_b = hip.event(), hip.event()
    lat = []
    for rep in range(max(3, args.steps)):
        for i in range(min(N, 4)):
            ctx.recall(desc(i, False, (ev_a, None), ev_b))
            ctx.check()
            if rep:
                lat.append(hip.elapsed_ms(ev_a, ev_b) * 1e3)
    select_us = float(np.median(lat))
    # (b) timed: the select stack; launch events on sampled inner positions
    # (steady launches: each beside the previous group's softmax and top-k)
    sampled = sorted({i for i in (N // 4, N // 2, 3 * N // 4) if (G <= i < N - G) or not fused} or {N // 2})
    ev_t = [{i: (hip.event(), hip.event()) for i in sampled} for _ in range(args.steps)]
    d_w = [desc(i, False) for i in range(N)]
    d_t = [[desc(i, False, e.get(i, (None, None))) for i in range(N)] for e in ev_t]
    keep = None
    for _ in range(args.warmup):
        keep = ctx.recall_stack(d_w)
        ctx.check()
    torch.cuda.synchronize()
    keeps = []
    t0 = time.perf_counter()
    for s_ in range(args.steps):
        keeps.append(ctx.recall_stack(d_t[s_]))
    ctx.check()
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / args.steps
    del keep, keeps
    launch_us = float(np.mean([hip.elapsed_ms(*e[i]) * 1e3 for e in ev_t for i in sampled]))
    k_read = 0 if w["resident"] else lane_rows * row(w["kfmt"])
    q_bytes = NL * R * HQ * D * 2
    scored_layer = k_read + NL * P * W * 2 + q_bytes
    value = N * scored_layer / (ms_per_step * 1e-3) / 1e9
    log(f"select {select_us:.1f} us/layer; stack {ms_per_step * 1e3 / N:.1f} us/layer = {value:.1f} GB/s; "
        f"dominant launch {launch_us:.1f} us")
    # algorithmic bytes of the dominant launch
    logits = NL * R * HQ * P * 8
    if not fused:
        kernel = "k_summary<f16> (summaries of every lane; logits on the matrix cores follow)"
        alg = k_read + NL * P * W * 2
    elif w["resident"]:
        # per layer: summaries + Q read, logits written by the summary
        # workgroups and read by the softmax units, terms written in place
        # and read back by the tail, scores written
        kernel = f"k_stack_group<summaries> ({G} resident layers' logits beside the previous {G} layers' " \
                 f"softmax and top-k)"
        alg = G * (NL * P * W * 2 + q_bytes + 4 * logits + NL * P * 8)
    else:
        kernel = f"k_stack_group<{'q8_0' if kfmt == K.FMT_Q8_0 else 'f16'}> ({G} layers' summaries beside the " \
                 f"previous {G} layers' logits, softmax and top-k)"
        alg = G * (k_read + 2 * NL * P * W * 2 + q_bytes + 2 * logits + NL * P * 8)
    achieved = alg / (launch_us * 1e-6) / 1e9
    traffic, traffic_src = None, os.path.join(ROOT, "profiles", f"pmc_{args.workload}.json")
    if os.path.exists(traffic_src):
        try:
            traffic = json.load(open(traffic_src)).get("traffic_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None
    # (c) select + stage-in pipelined over the layers
    pdescs = [desc(i, True) for i in range(N)]
    for rep in range(2):
        ctx.check()
        p0 = time.perf_counter()
        keep = ctx.recall_stack(pdescs, None, ctx.copy_stream)
        ctx.check()
        pipe_us = (time.perf_counter() - p0) * 1e6 / N
    del keep
    # (d) stage-in alone
    stage = []
    eng = {"auto": K.ENGINE_AUTO, "kernel": K.ENGINE_KERNEL, "sdma": K.ENGINE_SDMA}[args.engine]
    for rep in range(2):
        for i in range(N):
            l = order[i]
            planes = [K.make_plane(pins[l % ring][0], kfmt, W, T, mode[w["kmode"]], kslots[l], rope=rope),
                      K.make_plane(pins[l % ring][1], vfmt, W, T, mode[w["vmode"]], vslots[l])]
            hip.record(ev_a, ctx.copy_stream)
            ctx.stage_in(planes, PT, sel[i], cnt[i], KSEL, lanes=NL, engine=eng)
            hip.record(ev_b, ctx.copy_stream)
            ctx.check()
            if rep:
                stage.append(hip.elapsed_ms(ev_a, ev_b) * 1e3)
    stage_us = float(np.mean(stage))
    stage_bytes = NL * KSEL * PT * (row(w["kfmt"]) + row(w["vfmt"]))
    link = ctx.h2d_ceiling_gbps(1 << 30, 5)
    stage_gbps = stage_bytes / (stage_us * 1e-6) / 1e9
    log(f"pipelined {pipe_us:.1f} us/layer; stage-in {stage_us:.1f} us/layer = {stage_gbps:.2f} GB/s "
        f"(host link: copy {link['copy_GBps']}, kernel read {link['kernel_read_GBps']} GB/s)")
    line = {
        "metric": "select+stage-in latency/layer at 128K ctx; scored-KV GB/s vs HBM peak",
        "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16/q8_0/q4_1 operands, f32 summaries, f64 scores",
        "data": f"synthetic seeded (device generator, Box-Muller normals), seed {seed}",
        "config": {"workload": args.workload, **{k: v for k, v in w.items()}, "stack_layers": N},
        "select_us_per_layer": round(select_us, 2),
        "select_stack_us_per_layer": round(ms_per_step * 1e3 / N, 2),
        "scored_frac_hbm": round(value / HBM_PEAK_GBPS, 4),
        "latency_us_per_layer": round(pipe_us, 2),
        "stagein_us_per_layer": round(stage_us, 2),
        "stagein_bytes_per_layer": stage_bytes,
        "stagein_GBps": round(stage_gbps, 3), "h2d_link": link, "h2d_peak_GBps": link["ceiling_GBps"],
        "stagein_frac_h2d": round(stage_gbps / link["ceiling_GBps"], 4),
        "roofline": {"bound": "hbm", "kernel": kernel, "achieved": round(achieved, 2), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "bytes_per_launch": alg, "mean_launch_us": round(launch_us, 3)},
    }
    # parity of every unit and the reference's CPU select path
    log("parity of every layer/lane against the oracle; reference CPU baseline ...")
    gsel = [x.cpu().numpy().view(np.uint32).reshape(NL, KSEL) for x in sel]
    gsc = [x.cpu().numpy().reshape(NL, P) for x in scores]
    units, usel, usc = [], [], []
    seen = set()
    for i in range(N):
        l = order[i]
        if l in seen:
            continue
        seen.add(l)
        for lane in range(NL):
            def fetch(l=l, lane=lane):
                q = qd[l].cpu().numpy().view(np.float16).astype(np.float32).reshape(NL, R * HQ * D)[lane]
                if w["resident"]:
                    return "summaries", s16[l].cpu().numpy().view(np.uint16).reshape(NL, -1)[lane], q
                raw = dev_k[l][lane * T * row(w["kfmt"]):(lane + 1) * T * row(w["kfmt"])].cpu().numpy()
                return ("q8_0", raw, q) if kfmt == K.FMT_Q8_0 else ("f16", raw.view(np.uint16), q)
            units.append(fetch)
            usel.append(gsel[i][lane])
            usc.append(gsc[i][lane])
    parity, cpu = workload_checks(args, w, "lane" if NL > 1 else "layer", units, usel, usc, tie, scored_layer // NL)
    line["parity"] = parity
    if cpu:
        line["cpu_baseline"] = cpu
    log(f"parity: {parity}; cpu: {cpu}")
    for pk, pv in pins:
        pk.free()
        pv.free()
    ctx.close()
    print(json.dumps(line), flush=True)


# ---------------------------------------------------------------------------
# Sampled attention page masses (--workload attn128k / attn128k_q8): one
# layer's attention-feedback observer at 131072 tokens, 8 kv-heads x 128,
# 32 query heads, 4 sampled rows (every 128th row of a 512-row ubatch),
# causal fp16 mask, pages of 256 tokens.
ATTN_WORKLOADS = {"attn128k": "f16", "attn128k_q8": "q8_0"}


def run_stageout(args):
    """Stage-out (--workload stageout32m): 64 scattered 512 KiB device records
    packed into one 32 MiB pinned slot by one kvr_d2d_batched launch that
    writes over the host link, against a measured device-to-host copy peak."""
    import torch
    import kvmem_amd as K
    from kvmem_amd.hip import runtime

    hip = runtime()
    ctx = K.Context(0)
    n, rec = 64, 512 << 10
    src = torch.empty(n * 2 * rec, dtype=torch.uint8, device="cuda")  # records at every other 512 KiB
    torch.cuda.synchronize()
    ctx.synth_normal_f16(args.seed, 6000, src.numel() // 2, src)
    slot = K.PinnedBuffer(n * rec)
    srcs = [src.data_ptr() + (2 * i) * rec for i in range(n)]
    dsts = [slot.ptr + i * rec for i in range(n)]
    sizes = [rec] * n
    ev_a, ev_b = hip.event(), hip.event()
    for _ in range(args.warmup):
        ctx.d2d_batched(srcs, dsts, sizes, ctx.copy_stream)
    ctx.check()
    times = []
    for _ in range(args.steps):
        hip.record(ev_a, ctx.copy_stream)
        ctx.d2d_batched(srcs, dsts, sizes, ctx.copy_stream)
        hip.record(ev_b, ctx.copy_stream)
        ctx.check()
        times.append(hip.elapsed_ms(ev_a, ev_b) * 1e3)
    torch.cuda.synchronize()
    got = slot.numpy()
    ok = all(np.array_equal(got[i * rec:(i + 1) * rec], src[2 * i * rec:(2 * i + 1) * rec].cpu().numpy())
             for i in (0, n // 2, n - 1))
    # device-to-host copy peak: 1 GiB into pinned memory, best of 5
    big = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    pin = torch.empty(1 << 30, dtype=torch.uint8, pin_memory=True)
    best = 0.0
    for _ in range(5):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        pin.copy_(big, non_blocking=True)
        e1.record()
        torch.cuda.synchronize()
        best = max(best, (1 << 30) / (e0.elapsed_time(e1) * 1e-3) / 1e9)
    us = float(np.median(times))
    gbps = n * rec / (us * 1e-6) / 1e9
    log(f"stage-out {n} x {rec >> 10} KiB: {us:.1f} us = {gbps:.2f} GB/s; D2H peak {best:.2f} GB/s; bytes ok {ok}")
    line = {"metric": "stage-out GB/s (device records -> pinned slot) vs measured D2H peak", "value": round(gbps, 3),
            "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(us / 1e3, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "bytes", "data": f"synthetic seeded (device generator), seed {args.seed}",
            "config": {"workload": "stageout32m", "records": n, "record_bytes": rec},
            "d2h_peak_GBps": round(best, 3), "frac_d2h": round(gbps / best, 4), "bytes_match": bool(ok)}
    slot.free()
    ctx.close()
    print(json.dumps(line), flush=True)


def run_attention(args):
    import torch
    import kvmem_amd as K
    import oracle as O
    from kvmem_amd.hip import runtime

    hip = runtime()
    ctx = K.Context(0)
    kname = ATTN_WORKLOADS[args.workload]
    T, HKV, HQ, D, PT, UB = 131072, 8, 32, 128, 256, 512
    rows = [127, 255, 383, 511]
    P = T // PT
    kfmt = {"f16": K.FMT_F16, "q8_0": K.FMT_Q8_0}[kname]
    hrow = D * 2 if kname == "f16" else D // 32 * 34
    krow = HKV * hrow
    kdev = torch.empty(T * krow, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    if kname == "f16":
        ctx.synth_normal_f16(args.seed, 5000, T * HKV * D, kdev)
    else:
        ctx.synth_normal_q8_0(args.seed, 5001, T * HKV * D // 32, kdev)
    ctx.check()
    q = torch.empty(UB * HQ * D, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    ctx.synth_normal_f32(args.seed, 5002, q.numel(), q)
    ctx.check()
    # causal mask of the ubatch's last 512 positions: row r sees t <= T-UB+r
    t_idx = torch.arange(T, device="cuda")[None, :]
    r_idx = torch.arange(UB, device="cuda")[:, None]
    mask = torch.where(t_idx <= T - UB + r_idx, 0.0, float("-inf")).to(torch.float16).contiguous()
    mass = torch.empty(len(rows) * P, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    scale = 1 / np.sqrt(D)
    log(f"workload {args.workload}: {T} tokens, Hq {HQ}/Hkv {HKV}, D {D}, K {kname}, page {PT} ({P} pages), "
        f"{len(rows)} sampled rows of a {UB}-row ubatch, causal f16 mask")

    def call():
        ctx.attention_page_mass(q=q, q_format=K.FMT_F32, q_row_stride=HQ * D * 4, q_head_stride=D * 4, k=kdev,
                                k_format=kfmt, k_row_stride=krow, k_head_stride=hrow, mask=mask,
                                mask_format=K.FMT_F16, mask_row_stride=T * 2, head_dim=D, query_heads=HQ,
                                kv_heads=HKV, tokens=T, page_tokens=PT, scale=scale, softcap=0.0, rows=rows,
                                mass=mass)

    if args.pmc_pass:  # three calls, then the calibration copies
        for _ in range(3):
            call()
        ctx.check()
        cb = calibration_copies(ctx)
        ctx.close()
        print(json.dumps({"pass": "pmc", "workload": args.workload, "calls": 3, "copy_bytes": cb}), flush=True)
        return
    ev_a, ev_b = hip.event(), hip.event()
    for _ in range(args.warmup):
        call()
    ctx.check()
    # throughput: the K calls back to back between one pair of events on
    # the calls' stream (both launches of every call inside)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    hip.record(ev_a, ctx.select_stream)
    for _ in range(args.steps):
        call()
    hip.record(ev_b, ctx.select_stream)
    ctx.check()
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / args.steps
    call_us = hip.elapsed_ms(ev_a, ev_b) * 1e3 / args.steps
    # latency: one call alone between events (host launch time included)
    alone = []
    for _ in range(5):
        hip.record(ev_a, ctx.select_stream)
        call()
        hip.record(ev_b, ctx.select_stream)
        ctx.check()
        alone.append(hip.elapsed_ms(ev_a, ev_b) * 1e3)
    alone_us = float(np.median(alone))
    R = len(rows)
    alg = T * krow + R * HQ * D * 4 + R * T * 2 + 2 * R * HQ * P * 4 + R * P * 4
    achieved = alg / (call_us * 1e-6) / 1e9
    got = mass.cpu().numpy().reshape(R, P)
    traffic, traffic_src = None, os.path.join(ROOT, "profiles", f"pmc_{args.workload}.json")
    if os.path.exists(traffic_src):
        try:
            traffic = json.load(open(traffic_src)).get("traffic_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None
    log(f"call {call_us:.1f} us back to back ({args.steps} calls, both launches) = {achieved:.1f} GB/s algorithmic; "
        f"one call alone {alone_us:.1f} us; mass sums {got.sum(axis=1).round(6).tolist()}")
    line = {
        "metric": "sampled attention page masses at 128K ctx: key GB/s vs HBM peak",
        "value": round(achieved, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": f"{kname} keys, f32 query, f16 mask, f32 arithmetic",
        "data": f"synthetic seeded (device generator), seed {args.seed}",
        "config": {"workload": args.workload, "tokens": T, "kv_heads": HKV, "query_heads": HQ, "head_dim": D,
                   "page_tokens": PT, "pages": P, "sampled_rows": rows, "ubatch": UB, "key_format": kname},
        "roofline": {"bound": "hbm", "kernel": "k_attn_lse + k_attn_mass (one call)",
                     "achieved": round(achieved, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic, "bytes_per_call": alg,
                     "mean_call_us": round(call_us, 3)},
        "call_alone_us": round(alone_us, 3),
    }
    if not args.no_cpu:
        # the FP64 dense restatement on one sampled row, scaled to the call
        kh = kdev.cpu().numpy()
        qh = q.cpu().numpy().view(np.uint8)
        mh = mask.cpu().numpy().view(np.uint8)
        c0 = time.perf_counter()
        want = O.attention_page_mass(qh, O.FMT_F32, HQ * D * 4, D * 4, kh, kfmt, krow, hrow, mh, O.FMT_F16, T * 2,
                                     D, HQ, HKV, T, PT, scale, 0.0, rows[-1:])
        cpu_s = time.perf_counter() - c0
        err = float(np.max(np.abs(got[-1] - want[0])))
        line["cpu_baseline"] = {"value": round(alg / (cpu_s * R) / 1e9, 4), "unit": "GB/s", "cores": 1,
                                "kind": "port",
                                "sample": f"1 of {R} sampled rows (row {rows[-1]}), full layer, FP64 dense "
                                          f"restatement, {cpu_s:.2f} s, single thread; scaled to {R} rows",
                                "max_abs_diff_vs_gpu": err}
        log(f"cpu: {cpu_s:.2f} s for one row; max |gpu - oracle| = {err:.3e}")
    ctx.close()
    print(json.dumps(line), flush=True)


GRAPH_WORKLOADS = {"graph4096": (1, 4096, 48), "graph8x1024": (8, 1024, 64)}  # lanes, pages, budget


def run_graph(args):
    """Graph propagation + LRFU preview + selection of one Query's page
    scores (the stage between scoring and top-k), timed with HIP events."""
    import torch
    import kvmem_amd as K
    import oracle as O
    from kvmem_amd.hip import runtime

    hip = runtime()
    ctx = K.Context(0)
    lanes, P, budget = GRAPH_WORKLOADS[args.workload]
    rng = np.random.default_rng(args.seed)
    topk, alpha, lam, frac, cross, span = 4, 0.2, 0.5, 0.9, 0.25, 37
    raws, hists, graphs, nws, dev_graphs, keep = [], [], [], [], [], []
    for _ in range(lanes):
        x = rng.exponential(1.0, P) ** 3
        raws.append(x / x.sum())
        hists.append(O.lrfu_preview(rng.exponential(1.0, P) / P, None, lam, frac))
        rows = []
        for src in range(1, P):  # every page a sealed source: up to 4 earlier targets
            tg = np.unique(rng.integers(0, src, min(topk, src)))
            m = rng.exponential(1.0, tg.size)
            rows.append((src, [(int(t), float(v)) for t, v in zip(tg, m / m.sum())]))
        g = O.PageGraph(rows)
        nw = O.span_coefficients([(b * 64, min(P, b + span) * 64, True) for b in range(0, P, span)], 64, P, cross)
        graphs.append(g)
        nws.append(nw)
        t = [torch.from_numpy(a.view(np.int32) if a.dtype == np.uint32 else a).cuda()
             for a in (g.row_source, g.row_begin, g.edge_target, g.edge_mass, nw)]
        keep.append(t)
        dev_graphs.append(K.make_page_graph(g.n_rows, g.n_edges, *t[:4], neighbor_weight=t[4]))
    raw_d = torch.from_numpy(np.concatenate(raws)).cuda()
    hist_d = torch.from_numpy(np.concatenate(hists)).cuda()
    sc = torch.empty_like(raw_d)
    cand = torch.empty_like(raw_d)
    sel = torch.empty(lanes * budget, dtype=torch.int32, device="cuda")
    cnt = torch.empty(lanes, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    E = sum(g.n_edges for g in graphs)
    log(f"workload {args.workload}: {lanes} lane(s) x {P} pages, {graphs[0].n_rows} graph rows and "
        f"{graphs[0].n_edges} edges per lane, alpha {alpha}, LRFU lambda {lam} fraction {frac}, budget {budget}")

    def call():
        ctx.propagate_lrfu(sc, P, cand, dev_graphs, alpha, None, hist_d, P, lam, frac, lanes, ctx.select_stream)
        ctx.select_topk(cand, P, budget, sel, cnt, lanes=lanes, tie_rule=K.TIE_HIGHER_FIRST, signed_scores=True,
                        stream=ctx.select_stream)

    ev_a, ev_b = hip.event(), hip.event()
    for _ in range(args.warmup):
        sc.copy_(raw_d)
        torch.cuda.synchronize()
        call()
        ctx.check()
    times = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        sc.copy_(raw_d)  # propagation works in place: every step starts from the raw scores
        torch.cuda.synchronize()
        hip.record(ev_a, ctx.select_stream)
        call()
        hip.record(ev_b, ctx.select_stream)
        ctx.check()
        times.append(hip.elapsed_ms(ev_a, ev_b) * 1e3)
    ms_per_step = (time.perf_counter() - t0) * 1e3 / args.steps
    call_us = float(np.mean(times))
    got_c = cand.cpu().numpy().reshape(lanes, P)
    got_s = sel.cpu().numpy().view(np.uint32).reshape(lanes, budget)
    errs, same = [], True
    for l in range(lanes):
        want = O.lrfu_preview(O.propagate_scores(raws[l], graphs[l], alpha, None, nws[l]), hists[l], lam, frac)
        errs.append(float(np.max(np.abs(got_c[l] - want))))
        same &= bool(np.array_equal(got_s[l], O.pick_scored_blocks(want, budget, tie_rule=O.TIE_HIGHER_FIRST,
                                                                   signed_scores=True)))
    # bytes the two launches must move: propagation reads scores, weights,
    # rows and edges and writes scores; LRFU (same launch) reads the history
    # and writes the candidate; selection reads the candidate, writes the ids
    alg = lanes * (P * 8 * 2 + (P - 1) * 8 + P * 8 * 2 + P * 8 + budget * 4 + 4) + \
        sum(g.n_rows * 8 + 4 + g.n_edges * 12 for g in graphs)
    achieved = alg / (call_us * 1e-6) / 1e9
    log(f"call {call_us:.2f} us (propagate+LRFU launch, select launch; events) for {lanes * P} pages; "
        f"max |gpu - oracle| {max(errs):.2e}; selections equal {same}")
    line = {
        "metric": "graph propagation + LRFU + top-k of one Query's page scores: microseconds per call",
        "value": round(call_us, 3), "unit": "us", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f64", "data": f"synthetic seeded (numpy), seed {args.seed}",
        "config": {"workload": args.workload, "lanes": lanes, "pages": P, "budget": budget, "graph_rows": P - 1,
                   "edges": E, "alpha": alpha, "lrfu_lambda": lam, "lrfu_top_fraction": frac,
                   "message_span_pages": span},
        "roofline": {"bound": "hbm", "kernel": "k_graph_lrfu + k_select (one call)",
                     "achieved": round(achieved, 3), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 6), "traffic": None, "bytes_per_call": alg,
                     "mean_call_us": round(call_us, 3),
                     "note": "two dependent launches over ~100 KiB: launch and barrier latency, not HBM"},
        "parity": {"max_abs_diff_vs_oracle": max(errs), "selections_equal": same},
    }
    if not args.no_cpu:
        reps = 0
        c0 = time.perf_counter()
        while time.perf_counter() - c0 < min(args.cpu_seconds, 5.0) or reps == 0:
            for l in range(lanes):
                v = O.lrfu_preview(O.propagate_scores(raws[l], graphs[l], alpha, None, nws[l]), hists[l], lam, frac)
                O.pick_scored_blocks(v, budget, tie_rule=O.TIE_HIGHER_FIRST, signed_scores=True)
            reps += 1
        cpu_us = (time.perf_counter() - c0) / reps * 1e6
        line["cpu_baseline"] = {"value": round(cpu_us, 2), "unit": "us", "cores": 1, "kind": "port",
                                "sample": f"the whole call ({lanes} lane(s)), {reps} repetitions, single thread: "
                                          f"propagation, LRFU and the pick restated in C"}
        log(f"cpu: {cpu_us:.1f} us per call")
    ctx.close()
    print(json.dumps(line), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=64)
    ap.add_argument("--seed", type=int, default=42)
    ap.add_argument("--engine", choices=["auto", "kernel", "sdma"], default="kernel")
    ap.add_argument("--gather-wgs", type=int, default=0, help="gather grid bound (0 = library default)")
    ap.add_argument("--chunk-rows", type=int, default=0, help="gather rows per work item (0 = default)")
    ap.add_argument("--gather-threads", type=int, default=0, help="gather workgroup size (0 = default)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--workload", choices=["resident64", *WORKLOADS, *ATTN_WORKLOADS, *GRAPH_WORKLOADS,
                                           "stageout32m"],
                    default="resident64",
                    help="resident64 (default): the 64-layer 128K stack; the others are the remaining "
                         "workloads, each measured the same way")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="only the short counter pass of the workload (a stack of three launches, or one launch, "
                         "then three 256 MiB calibration copies)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        if int(os.environ.get("RANK", "0")) == 0:
            print("bench.py measures one GPU: the recall path runs on a single MI355X in this build "
                  "(multi-GPU sharding is a design note, not a measured mode). Use --gpus 1.", flush=True)
        sys.exit(2)
    if args.pmc_pass and args.workload in WORKLOADS:
        run_workload(args)
        return
    if args.pmc_pass and args.workload in ATTN_WORKLOADS:
        run_attention(args)
        return
    if args.pmc_pass:
        pmc_pass(args)
        return
    if args.workload in ATTN_WORKLOADS:
        run_attention(args)
        return
    if args.workload in GRAPH_WORKLOADS:
        run_graph(args)
        return
    if args.workload == "stageout32m":
        run_stageout(args)
        return
    if args.workload != "resident64":
        run_workload(args)
        return
    run(args)


if __name__ == "__main__":
    main()
