"""Benchmark: one decode-step tree-attention layer at 128 x 8192 (8128 shared) on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--method cube] [--no-graph]

Workload: 128 requests, one 8128-token shared root plus 64 private tokens each
(16,320 physical vs 1,048,576 logical KV positions), 32 query / 8 KV heads,
head dim 128, bf16, Q/K/V ~ N(0, 1) from a fixed seed, subset-DP (``cube``)
plan under the MI355X cost model.  One step = one ``attention_matrix`` call
(segment kernels + merge) on resident pools.  Steps rotate over 8 distinct KV
pools (535 MB, above the 256 MB MALL) so the bandwidth is HBM bandwidth.

Timing: HIP events on the launch stream around exactly K steps after W
warm-up steps, with a device synchronize on both sides.  By default the K
steps are replays of a HIP graph that holds one layer per pool (launch gaps
of the Python host loop removed); ``--no-graph`` times eager calls.  Graph
replays are checked against eager results before timing.

Prints one JSON line (see the repository's bench contract).
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "tree-attention-scheduling_amd"))
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16
R, HQ, HK, D = 128, 32, 8, 128
SHARED, PRIVATE = 8128, 64
POOLS = 8


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--method", default="cube")
    ap.add_argument("--cost-model", default="mi355x", choices=["mi355x", "reference"])
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--cpu-budget-s", type=float, default=20.0)
    ap.add_argument("--seed", type=int, default=101)
    return ap.parse_args()


def physical_kv_bytes(tokens: int) -> int:
    return tokens * HK * D * 2 * 2


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(the attention path is single-device; see DESIGN.md for how it would shard)", file=sys.stderr)
        sys.exit(2)
    import torch
    from tree_attention import CostModel, schedule, shapes
    from tree_attention import _native
    from tree_attention.kernels import attention_matrix, merge, pack_kv, prepare, segment

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    tree = shapes.tree(shapes.headline())
    T = tree.storage_tokens
    model = CostModel.mi355x() if args.cost_model == "mi355x" else CostModel()

    g = torch.Generator().manual_seed(args.seed)
    q = torch.randn(R, HQ, D, generator=g).bfloat16()
    k = torch.randn(T, HK, D, generator=g).bfloat16()
    v = torch.randn(T, HK, D, generator=g).bfloat16()
    qd = q.to(dev)
    kp0, vp0 = pack_kv(k.to(dev), v.to(dev))
    pools = [(kp0, vp0)] + [(kp0.clone(), vp0.clone()) for _ in range(POOLS - 1)]

    t0 = time.perf_counter()
    plan = schedule(tree, HQ, HK, D, args.method, model)
    plan_us = (time.perf_counter() - t0) * 1e6
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    prepared = prepare(plan, qd)
    torch.cuda.synchronize()
    metadata_us = (time.perf_counter() - t0) * 1e6

    stream = torch.cuda.current_stream(dev)

    def layer(i):
        kp, vp = pools[i % POOLS]
        return attention_matrix(qd, kp, vp, prepared)

    # correctness gate (oracle on the host) before any timing
    eager = [layer(i).clone() for i in range(POOLS)]
    torch.cuda.synchronize()
    from oracle.attention_oracle import relative_l2, request_attention
    ref = request_attention(q.float(), k.float(), v.float(), tree)
    rel = relative_l2(eager[0].cpu(), ref)
    if rel > 3e-3 or not all(torch.equal(eager[0], e) for e in eager[1:]):
        print(json.dumps({"error": "parity gate failed", "rel_l2": rel}), flush=True)
        sys.exit(1)

    def time_steps(fn, steps, warmup):
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for i in range(steps):
            fn(i)
        end.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(end) * 1e3 / steps  # us per step

    use_graph = not args.no_graph
    if use_graph:
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            layer(0)  # warm the side stream
        stream.wait_stream(side)
        outs = []
        with torch.cuda.graph(graph, stream=side):
            for i in range(POOLS):
                outs.append(layer(i).clone())
        torch.cuda.synchronize()
        for rep in range(3):  # replays interleaved with eager work must match eager results
            graph.replay()
            torch.cuda.synchronize()
            for i in range(POOLS):
                if not torch.equal(outs[i], eager[i]):
                    print(json.dumps({"error": f"graph replay {rep} differs from eager for pool {i}"}), flush=True)
                    sys.exit(1)
            layer(rep).clone()
            torch.cuda.synchronize()
        reps = max(1, args.steps // POOLS)
        us_per_layer = time_steps(lambda i: graph.replay(), reps, max(1, args.warmup // POOLS)) / POOLS
        steps_timed = reps * POOLS
    else:
        us_per_layer = time_steps(layer, args.steps, args.warmup)
        steps_timed = args.steps
    eager_us = time_steps(layer, max(POOLS, args.steps // 2), args.warmup)

    # per-kernel averages (graph of back-to-back launches of one kernel kind, rotating pools)
    kernel_us = {}
    kind_names = {_native.TA_SMALL: "segment_small", _native.TA_LARGE64: "segment_large64",
                  _native.TA_LARGE128: "segment_large128", _native.TA_LARGE256: "segment_large256"}
    launches = {}
    for kind, name in kind_names.items():
        if prepared.abi.n_items[kind] == 0:
            continue
        launches[name] = lambda i, kind=kind: segment(qd, pools[i % POOLS][0], pools[i % POOLS][1], prepared, kind)
    launches["merge"] = lambda i: merge(prepared)
    for name, fn in launches.items():
        kg = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            fn(0)
        stream.wait_stream(side)
        with torch.cuda.graph(kg, stream=side):
            for i in range(POOLS):
                fn(i)
        kernel_us[name] = time_steps(lambda i: kg.replay(), max(1, args.steps // POOLS),
                                     max(1, args.warmup // POOLS)) / POOLS

    # per-request execution through the same kernels (the "faster than per-request" check)
    req_prepared = prepare(schedule(tree, HQ, HK, D, "request", model), qd)
    per_request_us = time_steps(lambda i: attention_matrix(qd, *pools[i % POOLS], req_prepared),
                                max(POOLS, args.steps // 4), max(2, args.warmup // 2))

    # ---- roofline of the dominant kernel
    jobs = prepared.jobs
    small_tokens = sum(len(j.tokens) for j in jobs if len(j.requests) * (HQ // HK) <= 16)
    large_tokens = sum(len(j.tokens) for j in jobs if len(j.requests) * (HQ // HK) > 16)
    large_flops = sum(4 * len(j.requests) * HQ * len(j.tokens) * D for j in jobs
                      if len(j.requests) * (HQ // HK) > 16)
    seg_kernels = {n: t for n, t in kernel_us.items() if n.startswith("segment")}
    dominant = max(kernel_us, key=kernel_us.get)
    traffic = _pmc_traffic(dominant)
    if dominant.startswith("segment_large"):
        achieved = large_flops / (kernel_us[dominant] * 1e-6) / 1e12
        roofline = {"kernel": dominant, "bound": "mfma", "achieved": round(achieved, 1),
                    "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                    "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": traffic,
                    "algorithmic": f"{large_flops} FLOP per launch (4*rows*tokens*D over large jobs)"}
    else:
        nbytes = physical_kv_bytes(small_tokens) if dominant == "segment_small" else \
            2 * sum(len(j.requests) for j in jobs) * HQ * (D + 1) * 4
        achieved = nbytes / (kernel_us[dominant] * 1e-6) / 1e9
        roofline = {"kernel": dominant, "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                    "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                    "algorithmic": f"{nbytes} B per launch"}

    kv_bytes = physical_kv_bytes(T)
    value = kv_bytes / (us_per_layer * 1e-6) / 1e9
    cpu = cpu_baseline(q, k, v, tree, plan, args.cpu_budget_s)
    line = {
        "metric": "tree-attn decode µs/layer at 128×8192 (8128 shared); physical-KV HBM GB/s",
        "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": steps_timed, "warmup": args.warmup,
        "ms_per_step": round(us_per_layer / 1e3, 6), "us_per_layer": round(us_per_layer, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic N(0,1) Q/K/V, seed %d" % args.seed,
        "config": {"workload": "128 requests x 8192-token context, 8128-token shared root + 64 private each "
                               "(16,320 physical / 1,048,576 logical KV positions), 32Q/8KV heads, d=128, "
                               "one decode-step attention layer",
                   "method": args.method, "cost_model": args.cost_model, "kv_pools": POOLS,
                   "timing": "hip-graph replay" if use_graph else "eager", "physical_kv_bytes": kv_bytes},
        "layer_hbm_frac": round(value / HBM_PEAK_GBS, 4),
        "eager_us_per_layer": round(eager_us, 3),
        "per_request_us_per_layer": round(per_request_us, 3),
        "speedup_vs_per_request": round(per_request_us / eager_us, 3),
        "kernel_us": {n: round(t, 3) for n, t in kernel_us.items()},
        "plan": {"jobs": len(jobs), "small_jobs": prepared.small_jobs, "plan_us": round(plan_us, 1),
                 "metadata_us": round(metadata_us, 1), "estimated_us": plan.estimated_us,
                 "small_tokens": small_tokens, "large_tokens": large_tokens},
        "rel_l2_vs_fp32": rel,
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def _pmc_traffic(kernel_name):
    """HBM bytes per launch from the committed rocprofv3 PMC summary, if one exists."""
    path = ROOT / "profiles" / "pmc_traffic.json"
    if not path.exists():
        return None
    try:
        data = json.loads(path.read_text())
        return data.get("kernels", {}).get(kernel_name, {}).get("hbm_bytes_per_launch")
    except (ValueError, OSError):
        return None


def cpu_baseline(q, k, v, tree, plan, budget_s):
    """Oracle (FP32 torch-CPU restatement of reference.py) on the same layer, host cores."""
    import torch
    from oracle.attention_oracle import segmented_attention
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    qf, kf, vf = q.float(), k.float(), v.float()
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 1:
        t0 = time.perf_counter()
        segmented_attention(qf, kf, vf, plan)
        times.append(time.perf_counter() - t0)
        if len(times) >= 5:
            break
    us = statistics.median(times) * 1e6
    gbs = physical_kv_bytes(tree.storage_tokens) / (us * 1e-6) / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "us_per_layer": round(us, 1), "cores": cores,
            "threads": torch.get_num_threads(), "kind": "port",
            "sample": f"{len(times)} full layer(s) of the same workload and plan through the oracle's "
                      f"segmented_attention in fp32 (median)",
            "cpu": platform.processor() or platform.machine()}


if __name__ == "__main__":
    main()
