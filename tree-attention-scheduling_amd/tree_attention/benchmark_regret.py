"""Calibration regret: per evaluation shape, the fastest measured plan over every planning method
and cost-model parameter set, against the plan the fitted model's subset DP (``cube``) makes.

    python -m tree_attention.benchmark_regret [--grid nested|config|reference|headline|decode]
        [--iters 10] [--output PATH]

Parameter sets: the reference's Ascend 910B defaults (``CostModel()``, schedule.py:29-39) and
every candidate of the MI355X calibration -- the continuous terms tuned for each
``kv_split`` x ``max_query_rows`` pair, ``candidates`` of mi355x_cost_model.json -- among them
the chosen one (``fitted``), and each candidate's least-squares terms before the tuning.  Methods: request, fixed, greedy, cube (schedule.py:327-458).
Identical plans are timed once.  Every plan's output is checked against per-request attention in
fp32 on the device (atol .008 / rtol .03, scripts/benchmark.py:96) before it is timed; timing is
the device time of ``--iters`` resident ``attention_matrix`` calls captured in one HIP graph and
replayed (``harness.graph_layer_us``), rotating over copies of the K/V pools that span at least
535 MB.  Eager calls between two events would time the host's submission for the layers of
10-20 us.

Per shape: ``fitted_cube_us``, ``best_us`` and the (method, parameter set) that gave it, and
``regret`` = fitted_cube_us / best_us (1.0 when the fitted DP plan is the fastest measured).

``--grid decode`` times the two decode-step layers of ``shapes.decode_layers`` (the
decode-plan protocol of scripts/benchmark_decode_plan.py:21-64 and the Qwen3-4B-shaped
workload's layer), each at one step of its growing tails.  There every (method, parameter
set) gives two plans, as the protocol's two modes do: ``cached`` (a ``CachedDecodePlan`` over
the prompt plan, what the decoders run) and ``rebuild`` (the tree with the tails appended,
planned afresh); the fitted plan is the cached one of the fitted model's ``cube`` schedule.
"""
from __future__ import annotations

import argparse
import json
import math
import statistics
import copy
from dataclasses import asdict
from pathlib import Path

import torch

from . import CostModel, schedule, shapes
from .calibrate import OUT as FITTED_JSON
from .harness import check, graph_layer_us, reference_fp32, rotated_pools
from .kernels import CachedDecodePlan, attention_matrix, pack_kv, prepare

METHODS = ("request", "fixed", "greedy", "cube")
HQ, HK, D = 32, 8, 128


def parameter_sets():
    """{name: CostModel}: the reference defaults, the fitted model and every calibration candidate."""
    doc = json.loads(Path(FITTED_JSON).read_text())
    sets = {"reference": CostModel(), "fitted": CostModel(**doc["params"])}
    for c in doc["candidates"]:
        p = c["params"]
        name = f"candidate_s{p['kv_split']}_q{p['max_query_rows']}"
        if CostModel(**p) != sets["fitted"]:
            sets[name] = CostModel(**p)
        lsq = c.get("least_squares_params")
        if lsq and CostModel(**lsq) not in sets.values():
            sets["least_squares_" + name[len("candidate_"):]] = CostModel(**lsq)
    return sets


def plan_key(plan):
    return tuple((j.requests, j.tokens) for j in plan.jobs)


def distinct_plans(tree, sets):
    """[(key, plan, [(method, set name), ...])]: every (method, parameter set) plan, deduplicated."""
    out = {}
    for method in METHODS:
        for name, model in sets.items():
            plan = schedule(tree, HQ, HK, D, method, model)
            key = plan_key(plan)
            if key not in out:
                out[key] = (plan, [])
            out[key][1].append((method, name))
    return [(k, plan, who) for k, (plan, who) in out.items()]


def summarize(rows):
    regrets = [r["regret"] for r in rows]
    return {"shapes": len(rows),
            "geomean_regret": math.exp(sum(map(math.log, regrets)) / len(regrets)),
            "median_regret": statistics.median(regrets), "max_regret": max(regrets),
            "fitted_cube_within_2pct": sum(x <= 1.02 for x in regrets),
            # shapes whose fitted cube plan is more than 3 % slower than the per-request plan
            "cube_slower_than_request_3pct": [r["shape"] for r in rows
                                              if r["fitted_cube_us"] > 1.03 * r["request_us"]],
            "max_cube_over_request": max(r["fitted_cube_us"] / r["request_us"] for r in rows),
            "best_by": _count(r["best_by"] for r in rows),
            "worst": sorted(rows, key=lambda r: -r["regret"])[:5]}


def _count(items):
    out = {}
    for method, name in items:
        out[f"{method}/{name}"] = out.get(f"{method}/{name}", 0) + 1
    return out


def _time(q, pools, prepared, iters):
    return graph_layer_us(lambda i: attention_matrix(q, *pools[i % len(pools)], prepared), iters)


def run_shape(params, spec, sets, iters, seed, dev):
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
    timed = []
    for key, plan, who in distinct_plans(tree, sets):
        prepared = prepare(plan, q)
        check(attention_matrix(q, kp, vp, prepared), ref, f"{params} {who[0]}")
        timed.append((_time(q, pools, prepared, iters), key, who))
    fitted = plan_key(schedule(tree, HQ, HK, D, "cube", sets["fitted"]))
    fitted_us = next(t for t, key, _ in timed if key == fitted)
    request = plan_key(schedule(tree, HQ, HK, D, "request", sets["fitted"]))
    request_us = next(t for t, key, _ in timed if key == request)
    best_us, _, best_who = min(timed, key=lambda x: x[0])
    return {"shape": params, "requests": len(tree.paths), "storage_tokens": tree.storage_tokens,
            "fitted_cube_us": fitted_us, "request_us": request_us, "best_us": best_us, "best_by": best_who[0],
            "best_also": best_who[1:], "regret": fitted_us / best_us, "distinct_plans": len(timed),
            "plans": [{"us": t, "by": who} for t, _, who in sorted(timed, key=lambda x: x[0])]}


def run_decode_layer(name, tree, reserved, generated, sets, iters, seed, dev):
    """Regret of one decode-step layer: cached and rebuilt plans of every (method, set)."""
    nreq, prefix = len(tree.paths), tree.storage_tokens
    g = torch.Generator().manual_seed(seed)
    t8 = (prefix + nreq * reserved + 7) // 8 * 8
    q = torch.randn(nreq, HQ, D, generator=g).bfloat16().to(dev)
    k = torch.randn(t8, HK, D, generator=g).bfloat16().to(dev)
    v = torch.randn(t8, HK, D, generator=g).bfloat16().to(dev)
    tails = [[prefix + r * reserved + t for t in range(generated)] for r in range(nreq)]
    context = type("Context", (), {"paths": [list(p) + t for p, t in zip(tree.paths, tails)]})
    ref = reference_fp32(q, k, v, context)
    grown = copy.deepcopy(tree)
    leaves = [next(i for i, n in enumerate(grown.nodes) if r in n.terminal) for r in range(nreq)]
    for t in range(generated):
        grown.extend_leaves(leaves, [prefix + r * reserved + t for r in range(nreq)])
    kp, vp = pack_kv(k, v)
    del k, v
    pools = rotated_pools(kp, vp)
    plans = {}
    for method in METHODS:
        for set_name, model in sets.items():
            prompt = schedule(tree, HQ, HK, D, method, model)
            rebuilt = schedule(grown, HQ, HK, D, method, model)
            for mode, plan in (("cached", prompt), ("rebuild", rebuilt)):
                key = (mode, plan_key(plan))
                if key not in plans:
                    plans[key] = (plan, [])
                plans[key][1].append((f"{method}/{mode}", set_name))
    timed = []
    for key, (plan, who) in plans.items():
        if key[0] == "cached":
            prepared = CachedDecodePlan(plan, q, prefix, reserved).update(generated)
        else:
            prepared = prepare(plan, q)
        check(attention_matrix(q, kp, vp, prepared), ref, f"{name} {who[0]}")
        timed.append((_time(q, pools, prepared, iters), key, who))
    fitted = ("cached", plan_key(schedule(tree, HQ, HK, D, "cube", sets["fitted"])))
    fitted_us = next(t for t, key, _ in timed if key == fitted)
    request_us = next(t for t, key, who in timed if ("request/cached", "fitted") in who)
    best_us, _, best_who = min(timed, key=lambda x: x[0])
    return {"shape": {"layer": name, "reserved": reserved, "generated": generated}, "requests": nreq,
            "storage_tokens": prefix, "fitted_cube_us": fitted_us, "request_us": request_us, "best_us": best_us,
            "best_by": best_who[0], "best_also": best_who[1:], "regret": fitted_us / best_us,
            "distinct_plans": len(timed),
            "plans": [{"us": t, "by": who} for t, _, who in sorted(timed, key=lambda x: x[0])]}


def grid_of(name):
    if name == "nested":
        return [({"tree": "nested_unequal"}, shapes.nested_unequal())]
    if name == "headline":
        return [({"tree": "headline"}, shapes.headline())]
    return list(shapes.config_grid() if name == "config" else shapes.reference_grid())


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--grid", default="nested", choices=["nested", "config", "reference", "headline", "decode"])
    ap.add_argument("--iters", type=int, default=10)
    ap.add_argument("--seed", type=int, default=201)
    ap.add_argument("--limit", type=int, default=0, help="run only the first N shapes")
    ap.add_argument("--output", default=None)
    args = ap.parse_args(argv)
    dev = torch.device("cuda:0")
    sets = parameter_sets()
    if args.grid == "decode":
        layers = list(shapes.decode_layers())[:args.limit or None]
        run_decode_layer(*layers[0], {"fitted": sets["fitted"]}, 1, args.seed, dev)  # untimed first calls
        jobs = [lambda layer=layer: run_decode_layer(*layer, sets, args.iters, args.seed, dev) for layer in layers]
    else:
        grid = grid_of(args.grid)[:args.limit or None]
        run_shape(*grid[0], {"fitted": sets["fitted"]}, 1, args.seed, dev)  # untimed: first loads and calls
        jobs = [lambda p=p, spec=spec: run_shape(p, spec, sets, args.iters, args.seed, dev) for p, spec in grid]
    rows = []
    for job in jobs:
        row = job()
        print(json.dumps({k: v for k, v in row.items() if k != "plans"}), flush=True)
        rows.append(row)
    doc = {"grid": args.grid, "device": torch.cuda.get_device_name(0),
           "parameter_sets": {k: asdict(v) for k, v in sets.items()},
           "summary": summarize(rows), "rows": rows}
    print(json.dumps({"summary": {k: v for k, v in doc["summary"].items() if k != "worst"}}), flush=True)
    if args.output:
        Path(args.output).write_text(json.dumps(doc, indent=1) + "\n")


if __name__ == "__main__":
    main()
