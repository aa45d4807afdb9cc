"""Evaluation and calibration tree shapes (tree_attention.shapes)."""
import pytest

from tree_attention import shapes


def _lengths_and_requests(spec):
    parents, lengths, terminals = spec
    return {n for n in lengths if n}, {len(terminals)}


def _evaluation_specs():
    specs = [shapes.headline(), shapes.cpu_baseline_shape(), shapes.nested_unequal()]
    specs += list(shapes.benchmark_cases().values())
    specs += [s for _, s in shapes.reference_grid()]
    specs += [s for _, s in shapes.config_grid()]
    # decode-step layers: the prompt trees plus their reserved and generated tail lengths
    for _, t, reserved, generated in shapes.decode_layers():
        lengths = [len(n.tokens) for n in t.nodes] + [reserved, generated]
        specs.append(([-1] * len(lengths), lengths, [0] * len(t.paths)))
    return specs


def test_calibration_grid_is_disjoint_from_evaluation_shapes():
    """The MI355X cost model is fitted on shapes that no evaluation uses."""
    cal_len, cal_req = set(), set()
    for _, spec in shapes.calibration_grid():
        lengths, reqs = _lengths_and_requests(spec)
        cal_len |= lengths
        cal_req |= reqs
    for _, spec, reserved, generated in shapes.decode_calibration_grid():
        lengths, reqs = _lengths_and_requests(spec)
        cal_len |= lengths | {reserved, generated}
        cal_req |= reqs
    ev_len, ev_req = set(), set()
    for spec in _evaluation_specs():
        lengths, reqs = _lengths_and_requests(spec)
        ev_len |= lengths
        ev_req |= reqs
    assert not cal_len & ev_len
    assert not cal_req & ev_req


def test_headline_and_nested_shapes():
    t = shapes.tree(shapes.headline())
    assert t.storage_tokens == 16_320
    assert sum(map(len, t.paths)) == 1_048_576
    n = shapes.tree(shapes.nested_unequal())
    assert n.storage_tokens == 20_480 and len(n.paths) == 35
    assert len(n.paths[32]) == 4096 + 1024          # terminates at an internal node
    assert n.paths[33] == n.paths[0] and n.paths[34] == n.paths[1]  # duplicates


def test_config_grid_is_a_full_factorial():
    rows = list(shapes.config_grid())
    assert len(rows) == 81
    for params, spec in rows:
        t = shapes.tree(spec)
        assert len(t.paths) == params["requests"]
        assert all(len(p) == params["context"] for p in t.paths)
        shared = int(params["fraction"] * params["context"] + 0.5)
        # every request shares exactly the `shared` prefix of the root chain with request 0's subtree
        leaves = 2 ** (params["depth"] - 1)
        assert t.storage_tokens == sum(
            (2 ** i) * (shared // params["depth"] + (1 if i < shared % params["depth"] else 0))
            for i in range(params["depth"])) + params["requests"] * (params["context"] - shared)
        assert leaves <= params["requests"]


def test_grid_comparisons_geometric_mean():
    """benchmark_grid.comparisons follows scripts/analyze_planning.py:60-64."""
    from tree_attention.benchmark_grid import comparisons
    rows = []
    for i, (req, cube) in enumerate([(4.0, 1.0), (9.0, 1.0), (2.0, 4.0)]):
        for method, t in (("request", req), ("fixed", 2.0), ("greedy", 1.0), ("cube", cube)):
            rows.append({"shape": {"i": i}, "method": method, "kernel_us": t, "refresh_us": 2 * t})
    c = comparisons(rows)
    r = c["kernel_us_vs_request"]
    assert abs(r["geometric_mean_speedup"] - (4 * 9 * 0.5) ** (1 / 3)) < 1e-12
    assert r["median_speedup"] == 4.0 and r["range"] == [0.5, 9.0] and r["faster_shapes"] == 2
    assert c["refresh_us_vs_greedy"]["shapes"] == 3


def test_decode_plan_aggregate_matches_reference_schema():
    """benchmark_decode_plan.aggregate follows scripts/analyze_planning.py:19-39 (decode): per
    (method, mode), the mean over steps per seed, then median and [min, max] over seeds."""
    pytest.importorskip("torch")
    from tree_attention.benchmark_decode_plan import aggregate

    def run(seed, scale):
        steps = [{"step": i + 1, "planning_us": scale * (i + 1), "kernel_us": 10.0 * scale,
                  "total_us": scale * (i + 1) + 10.0 * scale} for i in range(4)]
        return {"method": "cube", "mode": "cached", "seed": seed, "initial_plan_us": 100.0 * scale,
                "steps": steps, "amortized_us": (100.0 * scale + sum(s["total_us"] for s in steps)) / 4}

    rows = aggregate([run(301, 1.0), run(302, 2.0), run(303, 3.0)])
    assert len(rows) == 1
    row = rows[0]
    assert (row["method"], row["mode"], row["seeds"]) == ("cube", "cached", [301, 302, 303])
    assert row["planning_us"] == 5.0 and row["planning_us_range"] == [2.5, 7.5]  # mean of 1..4 is 2.5 per unit
    assert row["kernel_us"] == 20.0 and row["kernel_us_range"] == [10.0, 30.0]
    assert row["initial_plan_us"] == 200.0 and row["amortized_us_range"][0] == (100.0 + 10.0 + 40.0) / 4
