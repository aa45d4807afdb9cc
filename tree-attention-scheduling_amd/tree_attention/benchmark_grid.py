"""Planner comparison over a grid of tree shapes (counterpart of scripts/benchmark_tree_grid.py
and the comparison block of scripts/analyze_planning.py:60-64).

    python -m tree_attention.benchmark_grid [--grid config|reference|nested] [--iters 10]
        [--cost-model mi355x|reference] [--route-items N] [--output PATH]

``--grid config`` (default) is the 81-shape requests x context x shared fraction x
depth factorial of ``shapes.config_grid``; ``--grid reference`` is the reference's own
81 trees (``shapes.reference_grid``, scripts/tree_shapes.py:5-19); ``--grid nested`` is the
one nested unequal-prefix tree of ``shapes.nested_unequal`` (root 4096 -> 8 x 1024 -> 32 x 256,
a request ending at an inner node, two duplicate paths).  Every shape runs
the four planning methods on one MI355X with bf16 Q/K/V ~ N(0, 1) from ``--seed``,
32 Q / 8 KV heads, d = 128.

Rows keep the reference's result schema (scripts/benchmark_tree_grid.py:48-52):
``kernel_us`` is the mean time of one ``attention_matrix`` call on resident pools
(HIP events around ``--iters`` calls, rotating over copies of the K/V pools that
span at least 535 MB, so small shapes read HBM rather than the MALL),
``plan_us`` / ``metadata_us`` time ``schedule`` and ``prepare``, ``refresh_us``
is their sum.  As in the reference (scripts/benchmark_tree_grid.py:40-41) every
method's output is checked before it is timed, here against
``harness.reference_fp32`` (per-request attention in fp32 on the device) with the
reference's device tolerance atol .008 / rtol .03; ``max_abs_error`` and
``rel_l2`` are recorded.  The CPU oracle comparison of the same shapes is the GPU
test suite's (tests/test_gpu_configs.py).
``--route-items`` sets ``prepare``'s limit for running large jobs in the small-job kernel
(default ``kernels.ROUTE_ITEMS``; 0 never routes).
``comparisons`` holds, per baseline method and metric, the geometric-mean speedup of
``cube`` over it, as scripts/analyze_planning.py:60-64 computes it.
"""
from __future__ import annotations

import argparse
import json
import math
import statistics
import time
from pathlib import Path

import torch

from . import CostModel, schedule, shapes
from .harness import check, pool_bytes, reference_fp32, rotated_pools
from .kernels import ROUTE_ITEMS, attention_matrix, pack_kv, prepare

METHODS = ("request", "fixed", "greedy", "cube")
HQ, HK, D = 32, 8, 128


def _time_layer(q, pools, prepared, iters):
    for i in range(3):
        attention_matrix(q, *pools[i % len(pools)], prepared)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(iters):
        attention_matrix(q, *pools[i % len(pools)], prepared)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1e3 / iters


def run_shape(params, spec, model, iters, seed, dev, log, route_items=ROUTE_ITEMS):
    tree = shapes.tree(spec)
    g = torch.Generator().manual_seed(seed)
    t8 = (tree.storage_tokens + 7) // 8 * 8
    q = torch.randn(len(tree.paths), HQ, D, generator=g).bfloat16().to(dev)
    k = torch.randn(t8, HK, D, generator=g).bfloat16().to(dev)
    v = torch.randn(t8, HK, D, generator=g).bfloat16().to(dev)
    ref = reference_fp32(q, k, v, tree)
    kp, vp = pack_kv(k, v)
    del k, v
    pools = rotated_pools(kp, vp)
    rows = []
    for method in METHODS:
        t0 = time.perf_counter()
        plan = schedule(tree, HQ, HK, D, method, model)
        plan_us = (time.perf_counter() - t0) * 1e6
        plan.validate(tree)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        prepared = prepare(plan, q, route_items=route_items)
        torch.cuda.synchronize()
        metadata_us = (time.perf_counter() - t0) * 1e6
        err = check(attention_matrix(q, kp, vp, prepared), ref, f"{params} {method}")
        kernel_us = _time_layer(q, pools, prepared, iters)
        row = {"shape": params, "requests": len(tree.paths), "storage_tokens": tree.storage_tokens,
               "method": method, "seed": seed, "kernel_us": kernel_us, "plan_us": plan_us,
               "metadata_us": metadata_us, "refresh_us": kernel_us + plan_us + metadata_us,
               "jobs": len(prepared.jobs), "logical_jobs": len(plan.jobs),
               "estimated_us": plan.estimated_us, "max_abs_error": err["max_abs_error"],
               "rel_l2": err["rel_l2"], "kv_pools": len(pools), "kv_pool_bytes": pool_bytes(pools)}
        rows.append(row)
        log(json.dumps(row))
    return rows


def comparisons(rows):
    """Speedup of ``cube`` over each baseline (scripts/analyze_planning.py:60-64)."""
    by_shape = {}
    for r in rows:
        by_shape.setdefault(json.dumps(r["shape"], sort_keys=True), {})[r["method"]] = r
    out = {}
    for metric in ("kernel_us", "refresh_us"):
        for baseline in ("request", "fixed", "greedy"):
            ratios = [m[baseline][metric] / m["cube"][metric] for m in by_shape.values()]
            out[f"{metric}_vs_{baseline}"] = {
                "geometric_mean_speedup": math.exp(sum(map(math.log, ratios)) / len(ratios)),
                "median_speedup": statistics.median(ratios), "range": [min(ratios), max(ratios)],
                "faster_shapes": sum(x > 1 for x in ratios), "shapes": len(ratios)}
    return out


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--grid", default="config", choices=["config", "reference", "nested"])
    ap.add_argument("--iters", type=int, default=10)
    ap.add_argument("--seed", type=int, default=201)
    ap.add_argument("--cost-model", default="mi355x", choices=["mi355x", "reference"])
    ap.add_argument("--limit", type=int, default=0, help="run only the first N shapes")
    ap.add_argument("--route-items", type=int, default=ROUTE_ITEMS)
    ap.add_argument("--output", default=None)
    args = ap.parse_args(argv)
    dev = torch.device("cuda:0")
    model = CostModel.mi355x() if args.cost_model == "mi355x" else CostModel()
    if args.grid == "nested":
        grid = [({"tree": "nested_unequal"}, shapes.nested_unequal())]
    else:
        grid = list(shapes.config_grid() if args.grid == "config" else shapes.reference_grid())
    if args.limit:
        grid = grid[:args.limit]
    # one untimed pass over the first shape: library loads and first calls stay out of the rows
    run_shape(*grid[0], model, 1, args.seed, dev, lambda s: None)
    rows = []
    for params, spec in grid:
        rows += run_shape(params, spec, model, args.iters, args.seed, dev, lambda s: print(s, flush=True),
                          args.route_items)
    doc = {"grid": args.grid, "cost_model": args.cost_model, "route_items": args.route_items,
           "device": torch.cuda.get_device_name(0),
           "rows": rows, "comparisons": comparisons(rows)}
    print(json.dumps({"comparisons": doc["comparisons"]}), flush=True)
    if args.output:
        Path(args.output).write_text(json.dumps(doc, indent=1) + "\n")


if __name__ == "__main__":
    main()
