"""Fit the MI355X cost-model terms from measured attention layers.

    python -m tree_attention.calibrate [--out PATH] [--iters 20]

The reference fits its ``CostModel`` (schedule.py:29-52) for Ascend 910B from
tile sweeps on two calibration trees (scripts/calibrate_tiles.py:13-22).  Here
the same formula is kept and only its parameters are refitted on one MI355X:

* ``cube_rows`` (16) and ``key_tile`` (64) are the kernels' own constants: jobs
  of at most 16 query rows run on the one-wave small-job path, K/V are staged
  in 64-token tiles and large jobs step through them 32 tokens at a time
  (``key_tile // 2``).
* ``kv_split`` and ``max_query_rows`` are structural: for every candidate pair
  the continuous terms are fitted and the pair whose subset-DP (``cube``) plans
  measure fastest on the calibration grid is kept.  "Fastest" is a weighted
  geometric mean of the cube plans' times: the static trees share one half of
  the weight and the decode-step layers the other, so the few decode layers
  are not outvoted by the many static trees.
* ``bandwidth``, ``cube_flops``, ``task_us`` and ``merge_us`` are fitted by
  least squares on log((launch + estimated_us) / measured_us) over every plan
  of every method on the calibration grid, with the layer's fixed launch cost
  as a nuisance term that the planner does not use.  Plans of ``greedy`` / ``cube`` depend on the
  parameters, so the fit is repeated with plans re-made from the fitted values.
* The least-squares terms predict times, not which plan is fastest.  A coordinate
  search then scales one term at a time by 1/4, 1/2, 2 or 4, or sets a per-job
  term (``task_us``, ``merge_us``) to one of a few absolute levels (3 ns .. 1 us),
  and keeps a change when the measured ``cube`` plans of the calibration grid get
  at least 1 % faster (the same weighted geometric mean), for up to three passes.
  The levels matter because the fit's layer-constant term absorbs the per-job
  costs, which it then leaves at their lower bounds.  The formula is unchanged;
  only its parameters move.

The calibration trees (``shapes.calibration_grid``) and decode-step layers
(``shapes.decode_calibration_grid``: a prompt tree whose ``CachedDecodePlan``
carries a growing tail per request, timed at one step, as the decoders run
it) share no request count or segment length with any evaluation shape.  A
decode layer's features are its prompt plan's jobs, the part the planner
decides.  Every plan is timed over copies of the
K/V pools that span at least 535 MB (``harness.rotated_pools``), as the evaluation
harnesses time theirs, on the device alone: ``iters`` layers captured in one
HIP graph and replayed (``harness.graph_layer_us``).  The fitted parameters are written
to ``mi355x_cost_model.json`` next to this module, together with the fit
residuals and the command that produced them.
"""
from __future__ import annotations

import argparse
import json
import math
import sys
import time
from dataclasses import asdict, replace
from pathlib import Path

import numpy as np
import torch

from . import shapes
from .harness import graph_layer_us, rotated_pools
from .kernels import CachedDecodePlan, attention_matrix, pack_kv, prepare
from .schedule import CostModel, physical_jobs, schedule

METHODS = ("request", "fixed", "greedy", "cube")
HQ, HK, D = 32, 8, 128
FIT_FIELDS = ("bandwidth", "cube_flops", "task_us", "merge_us")
OUT = Path(__file__).with_name("mi355x_cost_model.json")


def _features(plan):
    """Per-physical-job (nreq, ntok) pairs of a plan, in job order."""
    return [(len(j.requests), len(j.tokens)) for j in physical_jobs(plan.jobs)]


def _estimate(feats, model: CostModel) -> float:
    total = 0.0
    for nreq, ntok in feats:
        total += model._cost_n(nreq, ntok, HQ, HK, D)
    return total


class Bench:
    """Device inputs of one tree and a timer for its plans.

    ``decode = (reserved, generated)`` times a plan as a decode step does: a
    ``CachedDecodePlan`` with ``reserved`` tail tokens per request, updated to
    ``generated``."""

    def __init__(self, tree, dev, seed=11, decode=None):
        g = torch.Generator().manual_seed(seed)
        t = tree.storage_tokens + (len(tree.paths) * decode[0] if decode else 0)
        t8 = (t + 7) // 8 * 8  # an 8-aligned pool, as the model's pools are
        self.tree = tree
        self.decode = decode
        self.q = torch.randn(len(tree.paths), HQ, D, generator=g).bfloat16().to(dev)
        k = torch.randn(t8, HK, D, generator=g).bfloat16().to(dev)
        v = torch.randn(t8, HK, D, generator=g).bfloat16().to(dev)
        kp, vp = pack_kv(k, v)
        del k, v
        self.pools = rotated_pools(kp, vp)

    def time_plan(self, plan, iters: int) -> float:
        if self.decode:
            reserved, generated = self.decode
            prepared = CachedDecodePlan(plan, self.q, self.tree.storage_tokens, reserved).update(generated)
        else:
            prepared = prepare(plan, self.q)
        return graph_layer_us(lambda i: attention_matrix(self.q, *self.pools[i % len(self.pools)], prepared),
                              iters)


def fit_terms(samples, model: CostModel):
    """Least-squares fit of the continuous terms on log((launch + estimate) / measured).

    ``launch`` -- the fixed cost of one layer's kernel launches, which every plan
    pays alike -- is fitted alongside as a nuisance term; the planner's formula
    has no such term and compares plans without it.  Returns (model, launch_us).
    """
    from scipy.optimize import least_squares

    x0 = np.log([getattr(model, f) for f in FIT_FIELDS] + [5.0])

    def unpack(x):
        e = np.exp(x)
        return CostModel(**{**asdict(model), **dict(zip(FIT_FIELDS, map(float, e[:4])))}), float(e[4])

    def residual(x):
        m, launch = unpack(x)
        return np.array([math.log((launch + _estimate(f, m)) / t) for f, t in samples])

    # 0.1-20 TB/s, 0.1-10 PFLOP/s, 1 ns-100 us per task, 0.1 ns-10 us per merged request, 0.1-100 us launch
    lo = np.log([1e5, 1e8, 1e-3, 1e-4, 1e-1])
    hi = np.log([2e7, 1e10, 1e2, 1e1, 1e2])
    res = least_squares(residual, np.clip(x0, lo + 1e-9, hi - 1e-9), bounds=(lo, hi), method="trf")
    return unpack(res.x)


def _geomean(values):
    return float(np.exp(np.mean(np.log(values))))


def _weighted_geomean(values, weights):
    return float(np.exp(np.dot(weights, np.log(values)) / np.sum(weights)))


# absolute values the coordinate search also tries for the per-job terms (us): the
# least-squares fit leaves them at their bounds when the layer's fixed cost absorbs them
LEVELS = {"task_us": (0.003, 0.01, 0.03, 0.1, 0.3, 1.0), "merge_us": (0.003, 0.01, 0.03, 0.1, 0.3, 1.0)}


def tune_terms(model, cube_times, passes=3, factors=(0.25, 0.5, 2.0, 4.0), gain=0.01, score=_geomean,
               levels=None):
    """Coordinate search of the continuous terms on measured plan quality.

    ``cube_times(model)`` returns the measured times of ``model``'s cube plans on the
    calibration trees.  Each pass tries every term scaled by every factor, and set to
    each of its ``levels`` (absolute values, ``LEVELS`` by default), and keeps the best
    change if it lowers their ``score`` (geometric mean by default) by at least
    ``gain``.  Returns (model, score, steps taken); a step is (term, factor) or
    (term, "=", value).
    """
    levels = LEVELS if levels is None else levels
    best, best_s = model, score(cube_times(model))
    steps = []
    for _ in range(passes):
        trial = None
        for f in FIT_FIELDS:
            moves = [((f, k), replace(best, **{f: getattr(best, f) * k})) for k in factors]
            moves += [((f, "=", x), replace(best, **{f: x})) for x in levels.get(f, ())]
            for step, m in moves:
                if m == best:
                    continue
                s_ = score(cube_times(m))
                if s_ < best_s * (1 - gain) and (trial is None or s_ < trial[1]):
                    trial = (m, s_, step)
        if trial is None:
            break
        best, best_s = trial[0], trial[1]
        steps.append(trial[2])
    return best, best_s, steps


def calibrate(iters=20, kv_splits=(256, 512, 1024), query_rows=(64, 128, 256, 512), log=print):
    dev = torch.device("cuda:0")
    benches = [(name, Bench(shapes.tree(spec), dev)) for name, spec in shapes.calibration_grid()]
    benches += [(name, Bench(shapes.tree(spec), dev, decode=(reserved, generated)))
                for name, spec, reserved, generated in shapes.decode_calibration_grid()]
    # the static trees and the decode-step layers weigh half each in the score
    n_dec = sum(b.decode is not None for _, b in benches)
    weights = np.array([0.5 / n_dec if b.decode else 0.5 / (len(benches) - n_dec) for _, b in benches])

    def score(times):
        return _weighted_geomean(times, weights)

    start = CostModel(bandwidth=5.0e6, cube_flops=1.0e9, task_us=0.5, merge_us=0.01, cube_rows=16,
                      key_tile=64)
    measured = {}

    def measure(bench_name, bench, plan):
        key = (bench_name, tuple((j.requests, j.tokens) for j in plan.jobs))
        if key not in measured:
            measured[key] = bench.time_plan(plan, iters)
        return measured[key]

    candidates = []
    for kv_split in kv_splits:
        for mqr in query_rows:
            model = CostModel(**{**asdict(start), "kv_split": kv_split, "max_query_rows": mqr})
            samples = []
            for _round in range(2):
                for name, b in benches:
                    for method in METHODS:
                        plan = schedule(b.tree, HQ, HK, D, method, model)
                        samples.append((_features(plan), measure(name, b, plan)))
                model, launch = fit_terms(samples, model)
            fitted = model

            def cube_times(m):
                return [measure(name, b, schedule(b.tree, HQ, HK, D, "cube", m)) for name, b in benches]
            lsq_score = score(cube_times(model))
            model, _, steps = tune_terms(model, cube_times, score=score)
            cube = {name: measure(name, b, schedule(b.tree, HQ, HK, D, "cube", model)) for name, b in benches}
            req = {name: measure(name, b, schedule(b.tree, HQ, HK, D, "request", model)) for name, b in benches}
            cube_us, req_us = sum(cube.values()), sum(req.values())
            err = [math.log((launch + _estimate(f, model)) / t) for f, t in samples]
            err_lsq = [math.log((launch + _estimate(f, fitted)) / t) for f, t in samples]
            row = {"params": asdict(model), "least_squares_params": asdict(fitted), "tuning_steps": steps,
                   "launch_us": launch, "cube_total_us": cube_us, "request_total_us": req_us,
                   "cube_geomean_us": _geomean(list(cube.values())), "cube_score_us": score(list(cube.values())),
                   "least_squares_cube_score_us": lsq_score,
                   "cube_us": cube, "fit_rms_log_error": float(np.sqrt(np.mean(np.square(err)))),
                   "least_squares_rms_log_error": float(np.sqrt(np.mean(np.square(err_lsq)))),
                   "samples": len(samples), "plans_timed": len(measured)}
            candidates.append(row)
            log(json.dumps(row))
    # the static trees and the decode layers count alike: weighted geometric mean of the cube plans' times
    best = min(candidates, key=lambda r: r["cube_score_us"])
    return best, candidates


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--out", default=str(OUT))
    ap.add_argument("--iters", type=int, default=20)
    args = ap.parse_args(argv)
    t0 = time.time()
    best, candidates = calibrate(iters=args.iters, log=lambda s: print(s, flush=True))
    doc = {
        "status": "fitted on one MI355X",
        "command": "python -m tree_attention.calibrate " + " ".join(argv or sys.argv[1:]),
        "device": torch.cuda.get_device_name(0),
        "calibration_grid": [name for name, _ in shapes.calibration_grid()]
        + [name for name, *_ in shapes.decode_calibration_grid()],
        "params": best["params"],
        "launch_us": best["launch_us"],
        "fit_rms_log_error": best["fit_rms_log_error"],
        "cube_total_us": best["cube_total_us"],
        "cube_geomean_us": best["cube_geomean_us"],
        "cube_score_us": best["cube_score_us"],
        "request_total_us": best["request_total_us"],
        "candidates": candidates,
        "seconds": round(time.time() - t0, 1),
    }
    Path(args.out).write_text(json.dumps(doc, indent=1) + "\n")
    print(json.dumps({"best": best["params"], "out": args.out}), flush=True)


if __name__ == "__main__":
    main()
