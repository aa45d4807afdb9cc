"""Rebuild-per-step vs cached decode plans (counterpart of scripts/benchmark_decode_plan.py
and the ``decode`` aggregation of scripts/analyze_planning.py:19-39).

    python -m tree_attention.benchmark_decode_plan [--steps 16] [--seeds 301 302 303]
        [--planner auto|cpp|python] [--cost-model reference|mi355x] [--output PATH]

Workload (scripts/benchmark_decode_plan.py:21-27): 32 requests sharing a
1024-token root, each with a private 64-token node; bf16 Q [32, 32, 128] and
K/V pools of prefix + 32 x steps tokens, 8 KV heads, ~ N(0, 1) from the seed.
For each method (fixed, greedy, cube) and mode:

* ``rebuild``: every step appends one token per request to the tree
  (``extend_leaves``) and calls ``prepare(schedule(tree))``;
* ``cached``: one ``CachedDecodePlan`` over the prompt plan with reserved
  tails, then ``update(step + 1)`` per step.

Per step, ``planning_us`` is the host time of that planning work (device
synchronised on both sides) and ``kernel_us`` the mean of 10 resident
``attention_matrix`` calls after one warm call, as the reference measures
them (:45-56).  ``initial_plan_us`` is the cached plan's construction, and
``amortized_us`` = (initial + sum of step totals) / steps.  At the first and
last step the output is checked against the per-request plan of the same
tree (the ``request`` method, a different kernel path) within the
reference's device tolerance (atol .008, rtol .03); the oracle comparison of
the same protocol is in the GPU test suite.

``--cost-model`` selects the planner's parameters: ``reference`` (the
reference's defaults, as its script plans) or ``mi355x`` (the fitted MI355X
parameters the decoders of this package use).  ``--planner`` selects the
greedy / cube decision code of ``schedule``
(``cpp``: libtree_plan.so, ``python``: the Python planner; both give the same
plans).  Output: one JSON object per (method, mode, seed) as it finishes,
then the aggregate over seeds in the reference's ``results/decode_plan.json``
schema (median and [min, max] of each metric).
"""
from __future__ import annotations

import argparse
import copy
import json
import time
from collections import defaultdict
from pathlib import Path
from statistics import median

import torch

from . import CostModel, KVTree, schedule
from .kernels import CachedDecodePlan, attention_matrix, pack_kv, prepare

REQUESTS, ROOT, PRIVATE, HQ, HK, D = 32, 1024, 64, 32, 8, 128
METHODS = ("fixed", "greedy", "cube")
MODES = ("rebuild", "cached")
NATIVE = {"auto": None, "cpp": True, "python": False}


def _sync_time(fn):
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    out = fn()
    torch.cuda.synchronize()
    return out, (time.perf_counter() - t0) * 1e6


def run_seed(seed, steps, native, dev, log, model=None):
    base = KVTree.synthetic([-1] + [0] * REQUESTS, [ROOT] + [PRIVATE] * REQUESTS, list(range(1, REQUESTS + 1)))
    prefix = base.storage_tokens
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(REQUESTS, HQ, D, generator=g).bfloat16().to(dev)
    k = torch.randn(prefix + REQUESTS * steps, HK, D, generator=g).bfloat16().to(dev)
    v = torch.randn(k.shape, generator=g).bfloat16().to(dev)
    kp, vp = pack_kv(k, v)
    warm = CachedDecodePlan(schedule(base, method="fixed", model=model, native=native), q, prefix, steps)
    attention_matrix(q, kp, vp, warm.update(1))
    torch.cuda.synchronize()
    del warm
    rows = []
    for method in METHODS:
        for mode in MODES:
            tree = copy.deepcopy(base)
            leaves = list(range(1, REQUESTS + 1))
            if mode == "cached":
                cached, initial_us = _sync_time(
                    lambda: CachedDecodePlan(schedule(tree, method=method, model=model, native=native), q, prefix,
                                             steps))
            else:
                cached, initial_us = None, _sync_time(lambda: None)[1]
            costs = []
            for step in range(steps):
                if mode == "rebuild":
                    def plan_step():
                        tree.extend_leaves(leaves, [prefix + r * steps + step for r in range(REQUESTS)])
                        return prepare(schedule(tree, method=method, model=model, native=native), q)
                    prepared, planning_us = _sync_time(plan_step)
                else:
                    prepared, planning_us = _sync_time(lambda: cached.update(step + 1))
                attention_matrix(q, kp, vp, prepared)
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                for _ in range(10):
                    actual = attention_matrix(q, kp, vp, prepared)
                torch.cuda.synchronize()
                kernel_us = (time.perf_counter() - t0) * 1e6 / 10
                if step in (0, steps - 1):
                    check = copy.deepcopy(base)
                    for r in range(REQUESTS):
                        tail = tuple(prefix + r * steps + t for t in range(step + 1))
                        check.paths[r] = check.paths[r] + tail
                        check.nodes[r + 1].tokens = check.nodes[r + 1].tokens + tail
                    want = attention_matrix(q, kp, vp, prepare(schedule(check, method="request"), q))
                    torch.testing.assert_close(actual, want, atol=0.008, rtol=0.03)
                costs.append({"step": step + 1, "planning_us": planning_us, "kernel_us": kernel_us,
                              "total_us": planning_us + kernel_us})
            row = {"method": method, "mode": mode, "seed": seed, "initial_plan_us": initial_us, "steps": costs,
                   "amortized_us": (initial_us + sum(c["total_us"] for c in costs)) / steps}
            rows.append(row)
            log(json.dumps(row))
    return rows


def aggregate(runs):
    """scripts/analyze_planning.py:19-39 for ``decode``: per (method, mode), median and range over seeds."""
    groups = defaultdict(list)
    for row in runs:
        groups[(row["method"], row["mode"])].append(row)
    out = []
    for (method, mode), values in groups.items():
        row = {"method": method, "mode": mode, "seeds": [v["seed"] for v in values]}
        for v in values:
            v["planning_us"] = sum(s["planning_us"] for s in v["steps"]) / len(v["steps"])
            v["kernel_us"] = sum(s["kernel_us"] for s in v["steps"]) / len(v["steps"])
        for metric in ("initial_plan_us", "planning_us", "kernel_us", "amortized_us"):
            row[metric] = median(v[metric] for v in values)
            row[metric + "_range"] = [min(v[metric] for v in values), max(v[metric] for v in values)]
        out.append(row)
    return out


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=16)
    ap.add_argument("--seeds", type=int, nargs="+", default=[301, 302, 303])
    ap.add_argument("--planner", choices=sorted(NATIVE), default="auto")
    ap.add_argument("--cost-model", choices=["reference", "mi355x"], default="reference")
    ap.add_argument("--output", default=None)
    args = ap.parse_args(argv)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    model = CostModel.mi355x() if args.cost_model == "mi355x" else CostModel()
    runs = []
    for seed in args.seeds:
        runs += run_seed(seed, args.steps, NATIVE[args.planner], dev, lambda s: print(s, flush=True), model)
    result = {"inputs": [f"seed {s}" for s in args.seeds], "planner": args.planner, "cost_model": args.cost_model,
              "results": aggregate(runs)}
    if args.output:
        Path(args.output).write_text(json.dumps(result, indent=2))
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
