"""The C++ grouped planner (libtree_plan.so) against the Python planner.

The reference-pinned checks (published costs, reference plans at default and
non-default parameters) run over both implementations in test_planner.py;
here the two are compared on random trees, deep chains and random cost
parameters, where any difference in a decision or in the last bit of a cost
shows up as a different job list or estimate.
"""
import ctypes
import random
import re
from pathlib import Path

import numpy as np
import pytest

from tree_attention import CostModel, KVTree, schedule, shapes
from tree_attention import _planner

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "tree_plan.h"


def _both(tree, method, model=None, heads=(32, 8, 128)):
    a = schedule(tree, *heads, method, model, native=True)
    b = schedule(tree, *heads, method, model, native=False)
    assert a.jobs == b.jobs
    assert a.estimated_us == b.estimated_us
    return a


def _random_tree(rng, nodes, max_len, deep=False):
    parents = [-1]
    for v in range(1, nodes):
        parents.append(v - 1 if deep and rng.random() < 0.7 else rng.randrange(v))
    children = [[] for _ in parents]
    for v, p in enumerate(parents[1:], 1):
        children[p].append(v)
    lengths = [rng.randint(1, max_len) for _ in parents]
    leaves = [v for v in range(nodes) if not children[v]]
    inner = [v for v in range(1, nodes) if children[v]]
    terminals = leaves + rng.sample(inner, min(len(inner), rng.randint(0, 3)))
    rng.shuffle(terminals)
    return KVTree.synthetic(parents, lengths, terminals)


def _random_model(rng):
    return CostModel(bandwidth=rng.choice([900_000.0, 5_300_000.0, 1e6 / 3]),
                     cube_flops=rng.choice([1e8, 1.9e9, 7e7]),
                     task_us=rng.choice([0.15, 0.5, 0.0]), merge_us=rng.choice([0.03, 0.1, 1 / 7]),
                     cube_rows=rng.choice([16, 32]), key_tile=rng.choice([64, 128, 256]),
                     kv_split=rng.choice([64, 128, 512, 1000]), max_query_rows=rng.choice([16, 64, 128]))


def test_library_exports_declared_symbols():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    declared = set(re.findall(r"\b(tp_\w+)\s*\(", text))
    assert declared == set(_planner.EXPORTS)
    lib = _planner.load()
    for name in declared:
        assert hasattr(lib, name)


def test_invalid_arguments_are_rejected():
    lib = _planner.load()
    assert lib.tp_grouped_plan(1, 0, *([None] * 11)) == 1
    one = np.zeros(4, dtype=np.int64)
    p = one.ctypes.data_as(ctypes.c_void_p)
    assert lib.tp_grouped_plan(2, 1, *([p] * 11)) == 1  # unknown method
    iparams = np.array([16, 128, 512, 64, 30, 8, 128], dtype=np.int64)  # 30 % 8 != 0
    args = [p] * 11  # parent .. fparams, iparams (index 8), pushed, total
    args[8] = iparams.ctypes.data_as(ctypes.c_void_p)
    assert lib.tp_grouped_plan(1, 1, *args) == 1


@pytest.mark.parametrize("method", ["greedy", "cube"])
def test_shape_grids(method):
    for model in (None, CostModel.mi355x()):
        for _, spec in shapes.reference_grid():
            _both(shapes.tree(spec), method, model)
        for _, spec in shapes.config_grid():
            _both(shapes.tree(spec), method, model)
        for spec in (shapes.headline(), shapes.nested_unequal(), shapes.cpu_baseline_shape()):
            _both(shapes.tree(spec), method, model)
        _both(KVTree.from_sequences(shapes.qwen3_4b_workload()), method, model)


@pytest.mark.parametrize("seed", range(12))
def test_random_trees_and_parameters(seed):
    rng = random.Random(seed)
    for _ in range(6):
        tree = _random_tree(rng, rng.randint(2, 40), rng.choice([4, 64, 700]), deep=rng.random() < 0.3)
        model = _random_model(rng)
        heads = rng.choice([(32, 8, 128), (8, 2, 64), (16, 16, 32), (64, 4, 128)])
        for method in ("greedy", "cube"):
            _both(tree, method, model, heads).validate(tree)


def _chain(nodes):
    parents, lengths = [-1], [5]
    for v in range(1, nodes):
        parents.append(v - 1 if v % 3 else v - 2)
        lengths.append(1 + v % 7)
    children = set(parents[1:])
    return KVTree.synthetic(parents, lengths, [v for v in range(nodes) if v not in children])


def test_deep_chains():
    """Chains with short branches; neither planner recurses (the subset DP is cubic in depth here)."""
    tree = _chain(200)
    for method in ("greedy", "cube"):
        _both(tree, method).validate(tree)
    tree = _chain(3000)
    _both(tree, "greedy").validate(tree)


def test_uncovered_cases_fall_back_or_raise():
    """Grown tails break the increasing-chain condition; subclassed costs are Python-only."""
    tree = shapes.tree(shapes.shared_prefix(4, 600, 40))
    leaves = [1, 2, 3, 4]
    tree.extend_leaves(leaves, [tree.storage_tokens + i for i in range(4)])
    assert schedule(tree, method="cube", native=True).jobs == schedule(tree, method="cube", native=False).jobs
    tree.extend_leaves(leaves, [5, 6, 7, 8])  # ids below the leaves' first ids: chains no longer increase
    with pytest.raises(ValueError):
        schedule(tree, method="cube", native=True)
    assert schedule(tree, method="cube").jobs == schedule(tree, method="cube", native=False).jobs

    class Scaled(CostModel):
        def _cost_n(self, nreq, ntok, qheads, kvheads, dim):
            return 2.0 * super()._cost_n(nreq, ntok, qheads, kvheads, dim)
    tree = shapes.tree(shapes.headline())
    with pytest.raises(ValueError):
        schedule(tree, method="cube", model=Scaled(), native=True)
    assert schedule(tree, method="cube", model=Scaled()).estimated_us == 2.0 * schedule(tree).estimated_us


@pytest.mark.parametrize("seed", range(8))
def test_native_tail_attachment_equals_python(seed):
    """tp_attach_tails against kernels._attach_tails_py on random job sets: same attachments, same
    order, for single-request tails and for candidates of a few requests, scattered or consecutive
    (attachable only at consecutive rows of one wave)."""
    from tree_attention import kernels
    from tree_attention.schedule import Job
    rng = random.Random(seed)
    nreq = rng.randint(4, 300)
    large, base = [], 0
    for _ in range(rng.randint(1, 12)):
        reqs = tuple(sorted(rng.sample(range(nreq), rng.randint(1, nreq))))
        n = rng.randint(8, 900)
        large.append(Job(reqs, tuple(range(base, base + n))))
        base += n
    small = []
    for _ in range(rng.randint(0, 200)):
        u = rng.random()
        if u < 0.7:
            reqs = (rng.randrange(nreq),)
        elif u < 0.85:
            reqs = tuple(sorted(rng.sample(range(nreq), 2)))
        else:  # a node over consecutive requests
            r0 = rng.randrange(nreq)
            reqs = tuple(range(r0, min(nreq, r0 + rng.randint(2, 8))))
        n = rng.randint(1, 300)
        small.append(Job(reqs, tuple(range(base, base + n))))
        base += n
    fixed = {id(j) for j in small if rng.random() < 0.1}
    for group in (1, 4, 8, 16):
        for tile_rows in (128, 256):
            args = (small, large, group, tile_rows, lambda j: id(j) in fixed)
            left, attached = kernels._attach_tails(*args)
            left_py, attached_py = kernels._attach_tails_py(*args)
            assert [id(j) for j in left] == [id(j) for j in left_py]
            assert list(attached) == list(attached_py)
            for key in attached:
                assert [(id(j), r) for j, r in attached[key]] == [(id(j), r) for j, r in attached_py[key]]


def test_native_metadata_equals_numpy():
    """tp_build_metadata against the numpy builder: same buffer, sections and scalars, over
    every method on the shape sets, cached decode plans and random trees."""
    import torch
    from tree_attention import kernels
    from tree_attention.kernels import CachedDecodePlan

    captured = []
    native = kernels._metadata_native

    def both(*args):
        a, b = native(*args), kernels._metadata_numpy(*args)
        captured.append((a, b))
        return a

    kernels._metadata_native = both
    try:
        trees = [shapes.tree(shapes.headline()), shapes.tree(shapes.nested_unequal()),
                 shapes.tree(shapes.cpu_baseline_shape())]
        trees += [shapes.tree(spec) for _, spec in list(shapes.reference_grid())[::10]]
        rng = random.Random(5)
        trees += [_random_tree(rng, rng.randint(2, 30), rng.choice([16, 300])) for _ in range(6)]
        for tree in trees:
            q = torch.empty(len(tree.paths), 32, 128, dtype=torch.bfloat16)
            for method in ("request", "fixed", "cube"):
                for tile_rows in (256, 128):
                    kernels.prepare(schedule(tree, method=method, model=CostModel.mi355x()), q, tile_rows)
            CachedDecodePlan(schedule(tree, method="cube"), q, tree.storage_tokens, 4)
    finally:
        kernels._metadata_native = native
    assert len(captured) > 100
    for a, b in captured:
        assert np.array_equal(a["buf"], b["buf"])
        assert [tuple(s) for s in a["shapes"]] == [tuple(s) for s in b["shapes"]]
        for key in ("maxr", "maxs", "nslot", "contiguous_q", "slot_stride"):
            assert a[key] == b[key], key
        assert np.array_equal(a["qbase"], b["qbase"])
