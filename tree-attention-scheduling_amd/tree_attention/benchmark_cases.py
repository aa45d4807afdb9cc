"""The six representative cases of scripts/benchmark.py on one MI355X, in its row schema.

    python -m tree_attention.benchmark_cases [--cases wide_long ...] [--repeats 3] [--iters 30]
        [--cost-model mi355x|reference] [--output PATH]

Cases (scripts/benchmark.py:14-23, ``shapes.benchmark_cases``): ``no_share``,
``wide``, ``unequal``, ``deep``, ``wide_long`` (the 128 x 8192 headline) and
``no_share_long`` (128 x 8192, nothing shared).  Per case: bf16 Q/K/V ~ N(0, 1)
drawn on the host after ``torch.manual_seed(seed)`` (scripts/benchmark.py:67-70),
32 Q / 8 KV heads, d = 128; then, per planning method, ``schedule``,
``prepare``, one checked call and the timed calls.

Differences from the reference script, all deliberate:

* The output is checked against ``harness.reference_fp32`` (the reference's
  reference.py arithmetic in fp32 on the device) with the reference's
  tolerance before anything is timed (scripts/benchmark.py:96), and the row
  also carries the relative L2 error.
* The timed calls rotate over copies of the K/V pools that together span at
  least 535 MB, so every case reads HBM (the reference timed one pool).
* ``steady_us`` are HIP-event times of ``--iters`` back-to-back calls per
  repeat (the reference used host timers around synchronized loops).
* The Ascend vendor-operator rows (``vendor``, ``vendor_bsh``,
  scripts/benchmark.py:47-59) have no counterpart: that operator exists only
  in torch_npu.

Row fields follow scripts/benchmark.py:100-105 (``case``, ``method``,
``run_id``, ``seed``, ``steady_us``, ``median_us``, ``plan_us``,
``metadata_us``, ``layout_us``, ``first_call_ms``, ``jobs``,
``full_plan_refresh_us``, ``peak_allocated_bytes``, ``shared_tokens``,
``logical_tokens``, ``max_abs_error``), plus ``rel_l2``, ``cost_model``,
``kv_pools``, ``kv_pool_bytes`` and ``device``.  ``peak_allocated_bytes``
leaves out the rotated pool copies (``kv_pool_bytes`` counts them), so it
measures one pool plus what the method allocates, as the reference's did.
"""
from __future__ import annotations

import argparse
import json
import statistics
import time
from pathlib import Path

import torch

from . import CostModel, schedule, shapes
from .harness import check, pool_bytes, reference_fp32, rotated_pools
from .kernels import attention_matrix, pack_kv, prepare

METHODS = ("request", "fixed", "greedy", "cube")
HQ, HK, D = 32, 8, 128


def _events_us(fn, iters, warmup):
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(iters):
        fn(i)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1e3 / iters


def run_case(name, spec, methods, model, model_name, repeats, iters, seed, run_id, dev, log):
    tree = shapes.tree(spec)
    torch.manual_seed(seed)
    q = torch.randn(len(tree.paths), HQ, D, dtype=torch.bfloat16).to(dev)
    k = torch.randn(tree.storage_tokens, HK, D, dtype=torch.bfloat16).to(dev)
    v = torch.randn_like(k)
    ref = reference_fp32(q, k, v, tree)
    kp, vp = pack_kv(k, v)
    pools = rotated_pools(kp, vp)
    layout = [_events_us(lambda i: pack_kv(k, v), 5, 2) for _ in range(repeats)]
    rows = []
    for method in methods:
        torch.cuda.synchronize()
        first = time.perf_counter()
        t0 = time.perf_counter()
        plan = schedule(tree, HQ, HK, D, method, model)
        plan_us = (time.perf_counter() - t0) * 1e6
        plan.validate(tree)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        prepared = prepare(plan, q)
        torch.cuda.synchronize()
        metadata_us = (time.perf_counter() - t0) * 1e6
        out = attention_matrix(q, kp, vp, prepared).clone()
        torch.cuda.synchronize()
        first_call_ms = (time.perf_counter() - first) * 1e3
        err = check(out, ref, f"{name}/{method}")
        torch.cuda.reset_peak_memory_stats(dev)

        def layer(i):
            kpi, vpi = pools[i % len(pools)]
            attention_matrix(q, kpi, vpi, prepared)

        steady = [_events_us(layer, iters, 5) for _ in range(repeats)]
        median = statistics.median(steady)
        row = {"case": name, "method": method, "run_id": run_id, "seed": seed, "steady_us": steady,
               "median_us": median, "plan_us": plan_us, "metadata_us": metadata_us, "layout_us": layout,
               "first_call_ms": first_call_ms, "jobs": len(prepared.jobs),
               "full_plan_refresh_us": plan_us + metadata_us + statistics.median(layout) + median,
               # the rotated pool copies exist only to defeat the caches; one pool is the workload's
               "peak_allocated_bytes": torch.cuda.max_memory_allocated(dev) - pool_bytes(pools[1:]),
               "shared_tokens": tree.storage_tokens, "logical_tokens": sum(map(len, tree.paths)),
               "max_abs_error": err["max_abs_error"], "rel_l2": err["rel_l2"], "cost_model": model_name,
               "kv_pools": len(pools), "kv_pool_bytes": pool_bytes(pools),
               "device": torch.cuda.get_device_name(dev)}
        log(json.dumps(row))
        rows.append(row)
    return rows


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--cases", nargs="*")
    ap.add_argument("--methods", nargs="*", default=list(METHODS))
    ap.add_argument("--repeats", type=int, default=3)
    ap.add_argument("--iters", type=int, default=30)
    ap.add_argument("--seed", type=int, default=101)
    ap.add_argument("--run-id", type=int, default=0)
    ap.add_argument("--cost-model", default="mi355x", choices=["mi355x", "reference"])
    ap.add_argument("--output", default=None)
    args = ap.parse_args(argv)
    dev = torch.device("cuda:0")
    model = CostModel.mi355x() if args.cost_model == "mi355x" else CostModel()
    cases = {n: s for n, s in shapes.benchmark_cases().items() if not args.cases or n in args.cases}
    rows = []
    for name, spec in cases.items():
        rows += run_case(name, spec, args.methods, model, args.cost_model, args.repeats, args.iters, args.seed,
                         args.run_id, dev, lambda s: print(s, flush=True))
        if args.output:
            Path(args.output).write_text(json.dumps(rows, indent=2) + "\n")


if __name__ == "__main__":
    main()
