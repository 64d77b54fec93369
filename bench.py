"""Benchmark of the MI355X MoE forward (one GPU).

    python bench.py [--gpus 1] [--steps 64] [--warmup 10] [--workload qwen-bf16-t17]

A step is one full router-inclusive MoE layer forward (router -> planner ->
gate/up+SwiGLU -> down -> combine) over inputs already resident in HBM,
replayed from HIP graphs of 8 forwards each (BASELINE's timing protocol).  Two
copies of the weights alternate between forwards so the 256 MB Infinity Cache
cannot serve a forward from the previous one (more copies where one is small,
up to 8; a workload that still fits is marked ``cache_resident``).  The
JSON line's ``value`` is tokens/s of ``--workload`` (default: BASELINE
configs[1], Qwen3-30B-A3B shape, BF16, T=17); ``sweep`` carries every
BASELINE MoE configuration.  ``roofline`` is the dominant kernel
(gate/up+SwiGLU) timed live with HIP events on the stream it runs on;
``cpu_baseline`` times the FP32 CPU oracle on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import torch

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
METRIC = "MoE layer µs + tokens/s at T=17/193/1024 (BF16, W4A16); % HBM/MFMA roofline"

WORKLOADS = {
    "qwen-bf16-t17": dict(shape="qwen", T=17, routing="uniform", w4=False),
    "qwen-bf16-t193": dict(shape="qwen", T=193, routing="uniform", w4=False),
    "qwen-bf16-t1024-zipf": dict(shape="qwen", T=1024, routing="zipf", w4=False),
    "qwen-w4-t17": dict(shape="qwen", T=17, routing="uniform", w4=True),
    "qwen-w4-t193": dict(shape="qwen", T=193, routing="uniform", w4=True),
    "qwen-w4-t1024": dict(shape="qwen", T=1024, routing="uniform", w4=True),
    # The opt-in folded W4 decode (group scale on the fp32 group sum; effective
    # weights q * scale, not the reference's bf16_rn(q * scale)).
    "qwen-w4fold-t17": dict(shape="qwen", T=17, routing="uniform", w4=True, fold=True),
    "qwen-w4fold-t193": dict(shape="qwen", T=193, routing="uniform", w4=True, fold=True),
    "tiny-bf16-t17": dict(shape="tiny", T=17, routing="uniform", w4=False),
    # One GPU's share of the Qwen layer under 8-way expert / tensor parallelism
    # (the local kernels at their real shard shapes; no collectives).
    "qwen-ep8-bf16-t17": dict(shape="qwen-ep8", T=17, routing="uniform", w4=False),
    "qwen-ep8-bf16-t1024": dict(shape="qwen-ep8", T=1024, routing="uniform", w4=False),
    "qwen-tp8-bf16-t17": dict(shape="qwen-tp8", T=17, routing="uniform", w4=False),
    "qwen-tp8-bf16-t1024-zipf": dict(shape="qwen-tp8", T=1024, routing="zipf", w4=False),
    "qwen-tp8-w4-t17": dict(shape="qwen-tp8", T=17, routing="uniform", w4=True),
}


def log(msg):
    print(msg, file=sys.stderr, flush=True)


MALL_BYTES = 256 << 20  # MI355X Infinity Cache
MAX_COPIES = FORWARDS_PER_GRAPH = 8


def weight_bytes(spec, lay):
    """Bytes of one copy of the layer's expert weights (all experts)."""
    e, h, inter = lay["E"], lay["H"], lay["I"]
    gu = 2 * inter * h // 2 + 2 * inter * (h // 128) * 2 if spec["w4"] else 2 * inter * h * 2
    return e * (gu + h * inter * 2)


def build_plans(spec, device):
    """Prepared layers sharing inputs, each with its own weight copy.  Enough
    copies rotate through the graphs that the set of weights they touch is at
    least 1.5 x the Infinity Cache (a cyclic walk over more than the cache
    finds nothing of the previous forward in it), at most 8 (one graph's
    forwards); a workload whose 8 copies still fit is marked cache-resident."""
    from llm_gpu_kernels_amd import prepare_routed_moe, quantize_gate_up, tile_gate_up
    from llm_gpu_kernels_amd.workloads import make_layer
    lay = make_layer(spec["shape"], spec["T"], routing=spec["routing"], seed=0, device=device)
    gate_up = lay["gate_up"]
    if spec["w4"]:
        gate_up = tile_gate_up(quantize_gate_up(gate_up.cpu())).to(device)
    one = weight_bytes(spec, lay)
    copies = min(MAX_COPIES, max(2, -(-(3 * MALL_BYTES // 2) // one)))
    lay["weight_copies"] = copies
    lay["cache_resident"] = copies * one < 3 * MALL_BYTES // 2
    plans = []
    for c in range(copies):
        if c == 0:
            gu, dn = gate_up, lay["down"]
        elif spec["w4"]:
            gu = type(gate_up)(gate_up.words.clone(), gate_up.scales.clone(), gate_up.logical_shape)
            dn = lay["down"].clone()
        else:
            gu, dn = gate_up.clone(), lay["down"].clone()
        plans.append(prepare_routed_moe(lay["x"], lay["logits"], gu, dn, lay["K"],
                                        w4_decode="fold" if spec.get("fold") else "exact"))
    torch.cuda.synchronize()
    return lay, plans


def algorithmic(spec, lay, plan):
    """Bytes and FLOPs one forward must move / compute (weights of active experts once)."""
    e, h, inter, k, t = lay["E"], lay["H"], lay["I"], lay["K"], spec["T"]
    counts = plan.counts.cpu()
    active = int((counts > 0).sum())
    if spec["w4"]:
        gu_bytes = 2 * inter * h // 2 + 2 * inter * (h // 128) * 2
    else:
        gu_bytes = 2 * inter * h * 2
    dn_bytes = h * inter * 2
    layer_bytes = active * (gu_bytes + dn_bytes) + t * h * 2 + t * e * 4 + t * h * 2
    gate_up_bytes = active * gu_bytes + t * h * 2 + t * k * inter * 2
    flops = 6 * t * k * h * inter + 3 * t * e
    return dict(active_experts=active, layer_bytes=layer_bytes, gate_up_bytes=gate_up_bytes,
                flops=flops, gate_up_flops=4 * t * k * h * inter)


def time_layer(plans, steps, warmup):
    """Time exactly `steps` forwards; returns (ms per forward, per-graph samples).

    BASELINE's protocol (benchmark.py:68-98 of the reference): HIP graphs of
    FORWARDS_PER_GRAPH forwards, device time from HIP events on the replay
    stream.  Two graphs cycle through the weight copies, one starting at copy
    0 and one at copy 1 (A B A B ... and B A B A ... with two copies), and
    replays alternate between them (AB/BA rounds), so no copy always runs
    first.  A third graph holds the
    remainder steps % 8.  Warmup replays at least max(W, 32) forwards so the
    timed region starts at steady clocks.  Every full replay inside the timed
    region is also an event-timed sample (/8), and 16 more replays after it
    give p50/p95; the mean is total time / steps over the timed region."""
    stream = torch.cuda.Stream()
    for p in plans:
        for _ in range(2):
            p.run()
    torch.cuda.synchronize()

    def capture(n, first):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(n):
                plans[(first + i) % len(plans)].run()
        return graph

    rounds = [capture(FORWARDS_PER_GRAPH, 0), capture(FORWARDS_PER_GRAPH, 1)]
    replays, rem = divmod(steps, FORWARDS_PER_GRAPH)
    tail = capture(rem, replays % 2) if rem else None
    for i in range(max(4, -(-warmup // FORWARDS_PER_GRAPH))):
        rounds[i % 2].replay()
    if tail is not None:  # a graph's first replay also uploads it
        tail.replay()
        tail.replay()
    torch.cuda.synchronize()
    ev = lambda: torch.cuda.Event(enable_timing=True)
    marks = [ev() for _ in range(replays + 1)]
    end = ev()
    with torch.cuda.stream(stream):
        # Keep the GPU busy up to the timed region (an idle gap lets the clocks
        # drop, and the first timed replays would then run slower than the rest).
        for i in range(4):
            rounds[i % 2].replay()
        marks[0].record(stream)
        for i in range(replays):
            rounds[i % 2].replay()
            marks[i + 1].record(stream)
        if tail is not None:
            tail.replay()
        end.record(stream)
    end.synchronize()
    total_ms = marks[0].elapsed_time(end)
    samples = [marks[i].elapsed_time(marks[i + 1]) / FORWARDS_PER_GRAPH for i in range(replays)]
    extra = [ev() for _ in range(17)]
    with torch.cuda.stream(stream):
        extra[0].record(stream)
        for i in range(16):
            rounds[i % 2].replay()
            extra[i + 1].record(stream)
    extra[-1].synchronize()
    samples += [extra[i].elapsed_time(extra[i + 1]) / FORWARDS_PER_GRAPH for i in range(16)]
    return total_ms / max(steps, 1), samples


def time_stage(plans, stage, reps=40):
    """Average duration (ms) of one launch of `stage`: a HIP graph of `reps`
    back-to-back launches (alternating weight copies) timed with HIP events on
    the stream the launches run on, so host launch latency is not counted."""
    for p in plans:
        p.run()
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(reps):
            plans[i % len(plans)].run_stage(stage)
    graph.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        a.record(stream)
        graph.replay()
        b.record(stream)
    b.synchronize()
    return a.elapsed_time(b) / reps


def measure(name, steps, warmup, device):
    spec = WORKLOADS[name]
    lay, plans = build_plans(spec, device)
    alg = algorithmic(spec, lay, plans[0])
    ms, samples = time_layer(plans, steps, warmup)
    gate_idx = plans[0].launch_names.index("gate_up_swiglu")
    gu_ms = time_stage(plans, gate_idx)
    stage_ms = {n: round(time_stage(plans, i, reps=20) * 1e3, 2) for i, n in enumerate(plans[0].launch_names)}
    t = spec["T"]
    layer_gbs = alg["layer_bytes"] / (ms * 1e-3) / 1e9
    tflops = alg["flops"] / (ms * 1e-3) / 1e12
    attainable = min(BF16_PEAK_TFLOPS, alg["flops"] / alg["layer_bytes"] * HBM_PEAK_GBS / 1e3)
    res = dict(
        workload=name, T=t,
        weights=("w4g128-fold+bf16-down" if spec.get("fold") else "w4g128+bf16-down") if spec["w4"] else "bf16",
        routing=spec["routing"], us_per_layer=round(ms * 1e3, 2),
        p50_us=round(statistics.median(samples) * 1e3, 2),
        p95_us=round(sorted(samples)[int(0.95 * (len(samples) - 1))] * 1e3, 2),
        tokens_per_s=round(t / (ms * 1e-3), 1), active_experts=alg["active_experts"],
        layer_bytes=alg["layer_bytes"], layer_hbm_gbs=round(layer_gbs, 1),
        weight_copies=lay["weight_copies"], cache_resident=lay["cache_resident"],
        # A cache-resident workload's bytes per second are not HBM bandwidth.
        layer_hbm_frac=None if lay["cache_resident"] else round(layer_gbs / HBM_PEAK_GBS, 4),
        layer_tflops=round(tflops, 2), mfma_frac=round(tflops / BF16_PEAK_TFLOPS, 4),
        attainable_roofline_frac=round(tflops / attainable, 4),
        stage_us=stage_ms,
        gate_up=dict(us=round(gu_ms * 1e3, 2), bytes=alg["gate_up_bytes"],
                     gbs=round(alg["gate_up_bytes"] / (gu_ms * 1e-3) / 1e9, 1)),
    )
    return res, lay, plans


def measure_attention(tokens, device, reps=20, per_graph=10):
    """Segmented-KV GQA prefill: Q [T,32,128], KV segments
    1024/512/256/T with 8 KV heads.  FLOPs = 32*4*128*(T*1792 + T(T+1)/2);
    bytes = K,V once per KV head + Q + O.  One graph holds `per_graph` runs so
    the figure is device time, not host graph-launch rate."""
    from llm_gpu_kernels_amd import prepare_segmented_gqa
    g = torch.Generator(device=device).manual_seed(tokens)
    rnd = lambda shape: torch.randn(shape, generator=g, device=device).to(torch.bfloat16)
    q = rnd((tokens, 32, 128))
    segs = [(rnd((L, 8, 128)), rnd((L, 8, 128))) for L in (1024, 512, 256, tokens)]
    plan = prepare_segmented_gqa(q, segs)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for _ in range(per_graph):
            plan.run()
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        graph.replay()
    b.record()
    b.synchronize()
    us = a.elapsed_time(b) / (reps * per_graph) * 1e3
    flops = 32 * 4 * 128 * (tokens * 1792 + tokens * (tokens + 1) // 2)
    nbytes = (1792 + tokens) * 8 * 128 * 2 * 2 + 2 * tokens * 32 * 128 * 2
    tflops = flops / (us * 1e-6) / 1e12
    gbs = nbytes / (us * 1e-6) / 1e9
    attain = min(BF16_PEAK_TFLOPS, flops / nbytes * HBM_PEAK_GBS / 1e3)
    return dict(workload=f"gqa-seg-t{tokens}", T=tokens, us=round(us, 2), tflops=round(tflops, 2),
                hbm_gbs=round(gbs, 1), mfma_frac=round(tflops / BF16_PEAK_TFLOPS, 4),
                attainable_roofline_frac=round(tflops / attain, 4),
                arithmetic_intensity=round(flops / nbytes, 1))


def _cpu_sample(fn, budget_s, max_runs):
    """Mean seconds of fn() over a bounded sample (at least one run)."""
    times = []
    t_end = time.perf_counter() + budget_s
    while not times or (time.perf_counter() < t_end and len(times) < max_runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.mean(times), len(times)


def cpu_baseline(lay, spec, budget_s=10.0, max_runs=20):
    """FP32 CPU oracle (reference.py:17-45 restated) + CPU router, bounded
    sample, on this host's cores.  W4 layers run it on the dequantised
    gate/up weights (dequantised once, outside the timed sample)."""
    from oracle.moe_oracle import dequantize_w4, moe_reference, route_topk
    x, dn, logits = lay["x"].cpu(), lay["down"].cpu(), lay["logits"].cpu()
    gu = lay["gate_up"].cpu()
    if spec["w4"]:
        from llm_gpu_kernels_amd import quantize_gate_up
        packed = quantize_gate_up(gu)
        gu = dequantize_w4(packed.words, packed.scales)

    def forward():
        ids, w = route_topk(logits, lay["K"])
        moe_reference(x, gu, dn, ids, w)

    mean, n = _cpu_sample(forward, budget_s, max_runs)
    return {"value": round(spec["T"] / mean, 2), "unit": "tokens/s", "cores": torch.get_num_threads(),
            "kind": "port", "us_per_layer": round(mean * 1e6, 1),
            "sample": f"{n} full forwards of the {spec['shape']} T={spec['T']} layer "
                      f"(oracle.moe_oracle.route_topk + moe_reference, FP32, torch CPU, "
                      f"{torch.get_num_threads()} threads, os.cpu_count()={os.cpu_count()})"}


def cpu_attention_baseline(tokens, budget_s=3.0):
    """FP32 SDPA-math oracle of the segmented GQA attention (the reference's
    own test oracle, tests/e2e/test_compact_attention.py:49-78) on this host."""
    from oracle.moe_oracle import gqa_segmented_reference
    g = torch.Generator().manual_seed(tokens)
    rnd = lambda shape: torch.randn(shape, generator=g).to(torch.bfloat16)
    q = rnd((tokens, 32, 128))
    segs = [(rnd((L, 8, 128)), rnd((L, 8, 128))) for L in (1024, 512, 256, tokens)]
    mean, n = _cpu_sample(lambda: gqa_segmented_reference(q, segs), budget_s, 50)
    return {"cpu_us": round(mean * 1e6, 1), "cpu_cores": torch.get_num_threads(),
            "cpu_sample": f"{n} calls of oracle.moe_oracle.gqa_segmented_reference (FP32)"}


def copy_calibration(mib: int):
    """A plain device copy of known size, for scaling rocprofv3 FETCH_SIZE /
    WRITE_SIZE readings (KiB per dispatch) into HBM bytes."""
    n = mib * (1 << 20) // 2
    src = torch.randn(n, device="cuda:0").to(torch.bfloat16)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_read": n * 2, "copy_calibration_bytes_written": n * 2,
                      "dispatches": 10}), flush=True)


def profiled_traffic(workload: str):
    """HBM bytes per gate/up launch from the committed rocprofv3 PMC summary, if any."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        f"gate_up_traffic_{workload}.txt")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def _attach_cpu(rec, cpu):
    """The CPU FP32 baseline of one sweep record, in the record's own terms."""
    rec["cpu_us_per_layer"] = cpu["us_per_layer"]
    rec["cpu_tokens_per_s"] = cpu["value"]
    rec["cores"] = cpu["cores"]
    rec["cpu_sample"] = cpu["sample"]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="qwen-bf16-t17", choices=sorted(WORKLOADS))
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--attention-only", action="store_true",
                    help="only time the segmented-KV GQA attention (BASELINE config 5) and print "
                         "its records as one JSON line")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain MIB-MiB device copy 10 times (PMC scaling)")
    args = ap.parse_args()
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(one MI355X per box); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs an MI355X", file=sys.stderr)
        sys.exit(1)
    device = torch.device("cuda:0")
    if args.attention_only:
        print(json.dumps({"attention": [measure_attention(t, device) for t in (32, 96, 256)]}),
              flush=True)
        return
    log(f"[bench] workload {args.workload}")
    main_res, lay, plans = measure(args.workload, args.steps, args.warmup, device)
    spec = WORKLOADS[args.workload]
    cpu = None
    if not args.no_cpu:
        log("[bench] cpu baseline")
        cpu = cpu_baseline(lay, spec)
        _attach_cpu(main_res, cpu)
    del plans
    sweep = []
    if not args.no_sweep:
        for name in WORKLOADS:
            if name == args.workload:
                sweep.append(main_res)
                continue
            log(f"[bench] sweep {name}")
            r, lay_s, p = measure(name, args.steps, args.warmup, device)
            del p
            if not args.no_cpu:
                _attach_cpu(r, cpu_baseline(lay_s, WORKLOADS[name], budget_s=3.0, max_runs=10))
            sweep.append(r)
            del lay_s
            torch.cuda.empty_cache()
    attention = []
    if not args.no_sweep:
        for t in (32, 96, 256):
            log(f"[bench] attention T={t}")
            rec = measure_attention(t, device)
            if not args.no_cpu:
                c = cpu_attention_baseline(t)
                rec.update(c)
                rec["cpu_tokens_per_s"] = round(t / (c["cpu_us"] * 1e-6), 1)
            attention.append(rec)
    gu = main_res["gate_up"]
    line = {
        "metric": METRIC, "value": main_res["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(main_res["us_per_layer"] / 1e3, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": args.workload, "shape": spec["shape"], "T": spec["T"],
                   "E": lay["E"], "H": lay["H"], "I": lay["I"], "top_k": lay["K"],
                   "weights": main_res["weights"], "routing": spec["routing"],
                   "router": "on-GPU softmax-topk-renorm", "parallelism": "single-gpu"},
        "us_per_layer": main_res["us_per_layer"],
        "stage_us": main_res["stage_us"],
        "roofline": {"bound": "hbm", "kernel": "gate_up_swiglu", "achieved": gu["gbs"],
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gu["gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": profiled_traffic(args.workload), "avg_us": gu["us"],
                     "algorithmic_bytes": gu["bytes"]},
        "layer_roofline": {"bound": "hbm", "achieved": main_res["layer_hbm_gbs"],
                           "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": main_res["layer_hbm_frac"]},
        "cpu_baseline": cpu,
        "sweep": sweep,
        "attention": attention,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
