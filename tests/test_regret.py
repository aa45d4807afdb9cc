"""Host logic of the calibration-regret harness (tree_attention/benchmark_regret.py), on CPU."""
import math

from tree_attention import CostModel, schedule, shapes
from tree_attention.benchmark_regret import (METHODS, distinct_plans, parameter_sets, plan_key,
                                             summarize)


def test_parameter_sets_hold_the_reference_the_fit_and_the_candidates():
    sets = parameter_sets()
    assert sets["reference"] == CostModel()
    assert sets["fitted"] == CostModel.mi355x()
    cands = [m for name, m in sets.items() if name.startswith("candidate_")]
    assert len(cands) == 11 and CostModel.mi355x() not in cands
    lsq = [m for name, m in sets.items() if name.startswith("least_squares_")]
    assert lsq and all(m not in cands for m in lsq)
    fitted = CostModel.mi355x()
    pairs = {(m.kv_split, m.max_query_rows) for m in cands} | {(fitted.kv_split, fitted.max_query_rows)}
    assert pairs == {(s, r) for s in (256, 512, 1024) for r in (64, 128, 256, 512)}


def test_distinct_plans_cover_every_method_and_set_once():
    sets = parameter_sets()
    tree = shapes.tree(shapes.nested_unequal())
    plans = distinct_plans(tree, sets)
    keys = [k for k, _, _ in plans]
    assert len(set(keys)) == len(keys)
    who = [w for _, _, ws in plans for w in ws]
    assert sorted(who) == sorted((m, s) for m in METHODS for s in sets)
    for key, plan, ws in plans:
        for method, name in ws:
            assert plan_key(schedule(tree, 32, 8, 128, method, sets[name])) == key


def test_summarize():
    rows = [{"regret": 1.0, "best_by": ("cube", "fitted"), "shape": "a", "fitted_cube_us": 10.0, "request_us": 10.0},
            {"regret": 1.21, "best_by": ("greedy", "reference"), "shape": "b", "fitted_cube_us": 12.1,
             "request_us": 11.0},
            {"regret": 1.01, "best_by": ("cube", "fitted"), "shape": "c", "fitted_cube_us": 10.2, "request_us": 10.0}]
    s = summarize(rows)
    assert s["cube_slower_than_request_3pct"] == ["b"]
    assert math.isclose(s["max_cube_over_request"], 1.1)
    assert math.isclose(s["geomean_regret"], (1.21 * 1.01) ** (1 / 3))
    assert s["max_regret"] == 1.21 and s["fitted_cube_within_2pct"] == 2
    assert s["best_by"] == {"cube/fitted": 2, "greedy/reference": 1}
    assert s["worst"][0]["regret"] == 1.21


def test_decode_layers_are_the_protocol_and_the_qwen_workload():
    """The decode grid's two layers: 32 x (1024 + 64) (scripts/benchmark_decode_plan.py:21-27) and
    the Qwen3-4B-shaped prompt tree (2048 + 4 x 64 + 32 x 128), 16 reserved tail tokens, 8 generated."""
    layers = {name: (t, reserved, generated) for name, t, reserved, generated in shapes.decode_layers()}
    t, reserved, generated = layers["protocol_r32_1024_64"]
    assert (len(t.paths), t.storage_tokens, reserved, generated) == (32, 1024 + 32 * 64, 16, 8)
    t, reserved, generated = layers["qwen3_4b"]
    assert (len(t.paths), t.storage_tokens) == (32, 2048 + 4 * 64 + 32 * 128)
    assert sorted(map(len, t.paths)) == [2048 + 64 + 128] * 32
