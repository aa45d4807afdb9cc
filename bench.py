"""Benchmark: one decode-step tree-attention layer at 128 x 8192 (8128 shared) on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--method cube]

Workload: 128 requests, one 8128-token shared root plus 64 private tokens each
(16,320 physical vs 1,048,576 logical KV positions), 32 query / 8 KV heads,
head dim 128, bf16, Q/K/V ~ N(0, 1) from a fixed seed, subset-DP (``cube``)
plan under the MI355X cost model.  One step = one ``attention_matrix`` call
(the root's segment kernel, then the tail kernel whose work items also merge
each request) on resident pools.  Steps rotate over 8 distinct KV
pools (535 MB, above the 256 MB MALL) so the bandwidth is HBM bandwidth.

Timing: HIP events on the launch stream around exactly K eager steps after W
warm-up steps, with a device synchronize on both sides.  The same layers are
also replayed from a HIP graph (one layer per pool), checked against the
eager results and reported as ``graph_us_per_layer``: on this path graph
replay is slightly slower than back-to-back eager launches.  Per-kernel
``kernel_us`` are the kernels' own durations (dispatch begin/end stamps of
every launch through hipExtLaunchKernel events); ``kernel_graph_slot_us`` is
each kernel's share of a graph of back-to-back launches, gaps included.  The
roofline figure divides the dominant kernel's algorithmic work by its
``kernel_us``; ``roofline.stream_frac`` divides that rate by the box's read
ceiling, measured in the same run by the library's read-only stream over
1 GiB (``ta_read_stream``), and ``layer_stream_frac`` does the same for the
whole layer.

The parity gate comes first: the GPU output must be within 0.3% relative L2
of the FP32 oracle's per-request attention (oracle/attention_oracle.py, the
restatement of the reference's reference.py).  The CPU leg times the oracle
on the host cores on the same layer after the GPU timing, so that the GPU
does not idle (and drop its clocks) right before the timed steps.

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
REL_L2_BOUND = 3e-3
STREAM_BLOCKS = 16384  # workgroups of the read-ceiling stream (the fastest of 1024 / 4096 / 16384 measured)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--method", default="cube")
    ap.add_argument("--cost-model", default="mi355x", choices=["mi355x", "reference"])
    ap.add_argument("--cpu-budget-s", type=float, default=20.0)
    ap.add_argument("--seed", type=int, default=101)
    return ap.parse_args()


def physical_kv_bytes(tokens: int) -> int:
    return tokens * HK * D * 2 * 2


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(the attention path runs on one device)", file=sys.stderr)
        sys.exit(2)
    import torch
    from tree_attention import CostModel, schedule, shapes
    from tree_attention import _native, _planner
    from tree_attention.kernels import (attention_matrix, launch_durations_us, merge, pack_kv, prepare, segment,
                                        tail_merge)

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

    # host planning: the first call (library load, id tuples) and the median of warm calls
    plan_times, meta_times = [], []
    for _ in range(6):
        t0 = time.perf_counter()
        plan = schedule(tree, HQ, HK, D, args.method, model)
        plan_times.append((time.perf_counter() - t0) * 1e6)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        prepared = prepare(plan, qd)
        torch.cuda.synchronize()
        meta_times.append((time.perf_counter() - t0) * 1e6)
    plan_us, metadata_us = statistics.median(plan_times[1:]), statistics.median(meta_times[1:])

    stream = torch.cuda.current_stream(dev)

    def layer(i):
        kp, vp = pools[i % POOLS]
        return attention_matrix(qd, kp, vp, prepared)

    eager = [layer(i).clone() for i in range(POOLS)]
    torch.cuda.synchronize()
    if not all(torch.equal(eager[0], e) for e in eager[1:]):
        print(json.dumps({"error": "pools with equal contents gave different outputs"}), flush=True)
        sys.exit(1)

    # parity gate before any timing: the GPU layer against the oracle's per-request attention
    rel = parity_rel_l2(q, k, v, tree, eager[0].cpu())
    if not rel <= REL_L2_BOUND:
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

    def capture(fn, n):
        """A HIP graph of fn(0..n-1), captured on a side stream that the current stream joins."""
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            fn(0)
        stream.wait_stream(side)
        outs = []
        with torch.cuda.graph(graph, stream=side):
            for i in range(n):
                outs.append(fn(i))
        torch.cuda.synchronize()
        return graph, outs

    # the timed steps: K eager layers, each one attention_matrix call, rotating over the pools
    us_per_layer = time_steps(layer, args.steps, args.warmup)
    steps_timed = args.steps

    # the same layers replayed from a HIP graph (a checking graph first keeps a copy of every output)
    check, outs = capture(lambda i: layer(i).clone(), POOLS)
    for rep in range(3):  # replays interleaved with eager work must match eager results
        check.replay()
        torch.cuda.synchronize()
        for i in range(POOLS):
            if not torch.equal(outs[i], eager[i]):
                print(json.dumps({"error": f"graph replay {rep} differs from eager for pool {i}"}), flush=True)
                sys.exit(1)
        layer(rep).clone()
        torch.cuda.synchronize()
    del check, outs
    graph, _ = capture(layer, POOLS)
    graph.replay()
    torch.cuda.synchronize()
    if not torch.equal(prepared.out, eager[POOLS - 1]):
        print(json.dumps({"error": "timed graph's last layer differs from eager"}), flush=True)
        sys.exit(1)
    graph_us = time_steps(lambda i: graph.replay(), max(1, args.steps // POOLS), max(1, args.warmup // POOLS)) / POOLS

    # per-kernel averages over launches of one kernel kind, rotating pools
    kernel_us = {}
    kind_names = {_native.TA_SMALL: "segment_small", _native.TA_LARGE64: "segment_large64",
                  _native.TA_LARGE128: "segment_large128", _native.TA_LARGE256: "segment_large256"}
    launches = {}
    for kind, name in kind_names.items():
        if prepared.abi.n_items[kind] == 0:
            continue
        launches[name] = lambda i, kind=kind: segment(qd, pools[i % POOLS][0], pools[i % POOLS][1], prepared, kind)
    if prepared.abi.n_items[_native.TA_TAIL]:
        # the fused kind: each tail item attends its request's tail and merges the request
        launches["segment_tail_merge"] = lambda i: tail_merge(qd, pools[i % POOLS][0], pools[i % POOLS][1], prepared)
    if prepared.abi.n_rest:
        launches["merge"] = lambda i: merge(prepared)  # all requests; the layer merges only `rest`
    kernel_slot_us = {}
    for name, fn in launches.items():
        # the kernel's own duration: dispatch begin/end stamps of every launch (hipExtLaunchKernel events)
        for i in range(args.warmup):
            fn(i)
        kernel_us[name] = statistics.mean(launch_durations_us(fn, max(POOLS, args.steps)))
        # its slot in a graph of back-to-back launches, inter-launch gaps included
        kg, _ = capture(fn, POOLS)
        kernel_slot_us[name] = time_steps(lambda i: kg.replay(), max(1, args.steps // POOLS),
                                          max(1, args.warmup // POOLS)) / POOLS

    # the box's read ceiling in the same run: the library's read-only stream over 1 GiB
    # (ta_read_stream, 16,384 workgroups), the kernel's own duration from dispatch stamps
    lib = _native.load()
    stream_bytes = 1 << 30
    src = torch.ones(stream_bytes, dtype=torch.uint8, device=dev)
    sink = torch.zeros(4 * STREAM_BLOCKS, dtype=torch.int32, device=dev)

    def read_stream(i):
        _native.check(lib.ta_read_stream(src.data_ptr(), stream_bytes, sink.data_ptr(), STREAM_BLOCKS,
                                         stream.cuda_stream))

    for i in range(3):
        read_stream(i)
    stream_us = statistics.median(launch_durations_us(read_stream, 10))
    stream_gbs = stream_bytes / (stream_us * 1e-6) / 1e9
    del src, sink

    # per-request execution through the same kernels (the "faster than per-request" check)
    req_prepared = prepare(schedule(tree, HQ, HK, D, "request", model), qd)
    per_request_us = time_steps(lambda i: attention_matrix(qd, *pools[i % POOLS], req_prepared),
                                max(POOLS, args.steps // 4), max(2, args.warmup // 2))

    # CPU leg after the GPU timing (the GPU would idle through it and start the timing cold)
    cpu = cpu_baseline(q, k, v, tree, plan, args.cpu_budget_s, args.seed)

    # ---- roofline of the dominant kernel: both floors from its algorithmic work, the larger binds
    jobs = prepared.jobs
    small_rows = HQ // HK
    small_tokens = sum(len(j.tokens) for j in jobs if len(j.requests) * small_rows <= 16)
    tail_jobs = sorted({j for j, _, _ in prepared.items[_native.TA_TAIL].view(-1, 3).tolist()})
    tail_requests = [jobs[j].requests[0] for j in tail_jobs]
    counts = prepared.counts.tolist()
    large_jobs = [j for j in jobs if len(j.requests) * small_rows > 16]
    attached = [t for segs in prepared.attached.values() for t, _ in segs]
    # the large kernels' work: their jobs, plus the private segments attached to their items
    large_flops = (sum(4 * len(j.requests) * HQ * len(j.tokens) * D for j in large_jobs)
                   + sum(4 * HQ * len(t.tokens) * D for t in attached))
    # their physical KV: every token of a large job or attached segment, read once per KV head
    large_kv_bytes = physical_kv_bytes(sum(len(j.tokens) for j in large_jobs) + sum(len(t.tokens) for t in attached))
    partial_row = HQ * (2 * D + 8)  # one slot: fp16 row per query head + (lse, exponent) fp32 pair
    dominant = max(kernel_us, key=kernel_us.get)
    traffic = _pmc_traffic(dominant)
    t_s = kernel_us[dominant] * 1e-6
    if dominant.startswith("segment_large"):
        nbytes, flops = large_kv_bytes, large_flops
        work = (f"{large_kv_bytes} B of physical KV (K and V of every token of the large jobs and their "
                f"attached private segments, per KV head) and {large_flops} FLOP (4 x rows x tokens x D) per launch")
    elif dominant == "segment_small":
        nbytes, flops = physical_kv_bytes(small_tokens), 0
        work = f"{nbytes} B of physical KV per launch"
    elif dominant == "segment_tail_merge":
        # tail KV, the other partial slots of each tail request, the output rows
        nbytes = (physical_kv_bytes(sum(len(jobs[j].tokens) for j in tail_jobs))
                  + sum(counts[r] - 1 for r in tail_requests) * partial_row + len(tail_requests) * HQ * D * 2)
        flops = 0
        work = f"{nbytes} B per launch (tail KV, partial slots, output)"
    else:  # merge: every slot's partial row and (lse, exponent), then the output row
        nbytes, flops = sum(counts) * partial_row + len(counts) * HQ * D * 2, 0
        work = f"{nbytes} B per launch (partial slots and output)"
    hbm_floor_s = nbytes / (HBM_PEAK_GBS * 1e9)
    mfma_floor_s = flops / (MFMA_BF16_PEAK_TFLOPS * 1e12)
    hbm = {"achieved": round(nbytes / t_s / 1e9, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
           "frac": round(hbm_floor_s / t_s, 4), "floor_us": round(hbm_floor_s * 1e6, 3)}
    mfma = {"achieved": round(flops / t_s / 1e12, 1), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(mfma_floor_s / t_s, 4), "floor_us": round(mfma_floor_s * 1e6, 3)}
    bound, other = ("hbm", mfma) if hbm_floor_s >= mfma_floor_s else ("mfma", hbm)
    main = hbm if bound == "hbm" else mfma
    roofline = {"kernel": dominant, "bound": bound, "achieved": main["achieved"], "peak": main["peak"],
                "unit": main["unit"], "frac": main["frac"], "traffic": traffic, "kernel_us": round(kernel_us[dominant], 3),
                "floor_us": main["floor_us"], "algorithmic": work,
                ("mfma" if bound == "hbm" else "hbm"): other,
                # against the box's measured read ceiling instead of the 8 TB/s peak
                "stream_gbs": round(stream_gbs, 1), "stream_frac": round(hbm["achieved"] / stream_gbs, 4),
                "stream": f"ta_read_stream over {stream_bytes} B, {STREAM_BLOCKS} workgroups, median of 10 "
                          f"dispatch-stamped launches: {stream_us:.1f} us"}

    kv_bytes = physical_kv_bytes(T)
    value = kv_bytes / (us_per_layer * 1e-6) / 1e9
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
                   "timing": "eager", "physical_kv_bytes": kv_bytes},
        "layer_hbm_frac": round(value / HBM_PEAK_GBS, 4),
        "layer_stream_frac": round(value / stream_gbs, 4),
        "graph_us_per_layer": round(graph_us, 3),
        "per_request_us_per_layer": round(per_request_us, 3),
        "speedup_vs_per_request": round(per_request_us / us_per_layer, 3),
        "kernel_us": {n: round(t, 3) for n, t in kernel_us.items()},
        "kernel_graph_slot_us": {n: round(t, 3) for n, t in kernel_slot_us.items()},
        "plan": {"jobs": len(jobs), "small_jobs": prepared.small_jobs, "plan_us": round(plan_us, 1),
                 "plan_first_call_us": round(plan_times[0], 1), "metadata_first_call_us": round(meta_times[0], 1),
                 "planner": "cpp" if _planner.available() else "python",
                 "metadata_us": round(metadata_us, 1), "estimated_us": plan.estimated_us,
                 "small_tokens": small_tokens, "large_flops": large_flops},
        "rel_l2_vs_fp32": rel,
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def _pmc_traffic(kernel_name):
    """HBM bytes per launch of ``kernel_name`` from the committed rocprofv3 PMC summary, if any."""
    path = ROOT / "profiles" / "pmc_traffic.json"
    if not path.exists():
        return None
    try:
        data = json.loads(path.read_text())
        return data.get("kernels", {}).get(kernel_name, {}).get("hbm_bytes_per_launch")
    except (ValueError, OSError):
        return None


def parity_rel_l2(q, k, v, tree, gpu_out):
    """Relative L2 of ``gpu_out`` against the oracle's FP32 ``request_attention`` (reference.py:4-13)."""
    import torch
    from oracle.attention_oracle import relative_l2, request_attention
    torch.set_num_threads(len(os.sched_getaffinity(0)))
    return relative_l2(gpu_out, request_attention(q.float(), k.float(), v.float(), tree))


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), else the architecture."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def _time_cpu(fn, warmup, iters, budget_s):
    for _ in range(warmup):
        fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < iters and (time.perf_counter() < t_end or len(times) < 1):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times) * 1e6, len(times)


def cpu_baseline(q, k, v, tree, plan, budget_s, seed):
    """CPU leg: the FP32 oracle's plan-driven ``segmented_attention``
    (reference.py:16-33) on the host cores.

    ``value``: the CPU-baseline configuration (8 requests, 1024-token shared
    root + 64 private tokens each, fp32 N(0,1) Q/K/V from ``seed``, per-request
    plan; 2 warm-ups, then the median of 20 runs).  ``same_layer``: the timed
    GPU layer and plan in fp32 (median of up to 5 runs within ``budget_s``).
    Both in physical-KV GB/s (bf16 K and V bytes of the tree, the metric's
    denominator)."""
    import torch
    from oracle.attention_oracle import request_attention, segmented_attention
    from tree_attention import schedule, shapes
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    small = shapes.tree(shapes.cpu_baseline_shape())
    g = torch.Generator().manual_seed(seed)
    q1 = torch.randn(len(small.paths), HQ, D, generator=g)
    k1 = torch.randn(small.storage_tokens, HK, D, generator=g)
    v1 = torch.randn(small.storage_tokens, HK, D, generator=g)
    plan1 = schedule(small, HQ, HK, D, "request")
    a = segmented_attention(q1, k1, v1, plan1)
    b = request_attention(q1, k1, v1, small)  # cross-check of the timed function
    if not torch.allclose(a, b, atol=2e-5, rtol=2e-5):
        raise RuntimeError("oracle segmented_attention disagrees with request_attention on the CPU-baseline shape")
    us1, n1 = _time_cpu(lambda: segmented_attention(q1, k1, v1, plan1), 2, 20, budget_s)
    qf, kf, vf = q.float(), k.float(), v.float()
    us2, n2 = _time_cpu(lambda: segmented_attention(qf, kf, vf, plan), 0, 5, budget_s)
    gb = lambda tokens, us: round(physical_kv_bytes(tokens) / (us * 1e-6) / 1e9, 3)  # noqa: E731
    return {"value": gb(small.storage_tokens, us1), "unit": "GB/s", "us_per_layer": round(us1, 1),
            "cores": cores, "threads": torch.get_num_threads(), "kind": "port",
            "sample": (f"CPU-baseline configuration: 8 requests x (1024 shared + 64 private) tokens, 32Q/8KV, "
                       f"d=128, fp32, per-request plan ({len(plan1.jobs)} jobs) through the oracle's "
                       f"segmented_attention; median of {n1} runs after 2 warm-ups"),
            "cpu": cpu_model(),
            "same_layer": {"value": gb(tree.storage_tokens, us2), "unit": "GB/s", "us_per_layer": round(us2, 1),
                           "sample": f"the timed 128 x 8192 layer and plan in fp32, median of {n2} run(s)"}}


if __name__ == "__main__":
    main()
