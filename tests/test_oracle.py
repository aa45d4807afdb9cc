"""Pins of the CPU oracle (oracle/attention_oracle.py) -- reference src/tree_attention/reference.py.

Each oracle function is checked against something independent of its own
formula: a float64 numpy restatement, closed forms, the reference's own
segmented == request invariant (tests/test_semantics.py:23-34), and planted
mistakes that the checks must catch.
"""
import math

import numpy as np
import pytest
import torch

from oracle.attention_oracle import attention_f64, relative_l2, request_attention, segmented_attention
from tree_attention import CostModel, KVTree, schedule
from tree_attention.schedule import Plan, physical_jobs

METHODS = ("request", "fixed", "greedy", "cube")


def semantics_trees():
    """The trees of the reference's tests/test_semantics.py."""
    t = KVTree.from_sequences([[1, 2], [1, 2], [3, 4]])
    leaves = [next(i for i, n in enumerate(t.nodes) if r in n.terminal) for r in range(3)]
    t.extend_leaves(leaves, [4, 5, 6])
    t.extend_leaves(leaves, [7, 8, 9])
    return {
        "unequal": (KVTree.from_sequences([[1, 2, 3], [1, 2], [1, 2, 4, 5, 6], [7, 8], [1, 2, 3]]), 1),
        "noshare": (KVTree.from_sequences([[1, 2, 3], [4], [5, 6, 7, 8, 9]]), 1),
        "deep": (KVTree.synthetic([-1, 0, 1, 1, 0], [129, 65, 17, 33, 81], [2, 3, 4]), 30),
        "extended": (t, 1),
    }


def inputs(tree, scale, seed=17):
    torch.manual_seed(seed)
    q = torch.randn(len(tree.paths), 8, 32) * scale
    k = torch.randn(tree.storage_tokens, 2, 32)
    v = torch.randn_like(k)
    return q, k, v


@pytest.mark.parametrize("name", ["unequal", "noshare", "deep", "extended"])
def test_segmented_equals_request_for_every_plan(name):
    tree, scale = semantics_trees()[name]
    q, k, v = inputs(tree, scale)
    ref = request_attention(q, k, v, tree)
    for method in METHODS:
        plan = schedule(tree, 8, 2, 32, method, CostModel(kv_split=48))
        plan = Plan(physical_jobs(plan.jobs), method, plan.estimated_us, plan.settings)
        torch.testing.assert_close(segmented_attention(q, k, v, plan), ref, atol=2e-5, rtol=2e-5)


@pytest.mark.parametrize("name", ["unequal", "deep"])
def test_request_attention_vs_float64(name):
    tree, scale = semantics_trees()[name]
    q, k, v = inputs(tree, scale)
    got = request_attention(q, k, v, tree).double().numpy()
    want = attention_f64(q.numpy(), k.numpy(), v.numpy(), tree)
    np.testing.assert_allclose(got, want, atol=2e-5, rtol=2e-5)


def test_float64_vs_independent_softmax():
    torch.manual_seed(3)
    tree = KVTree.synthetic([-1, 0, 0], [40, 9, 13], [1, 2, 2])
    q = torch.randn(3, 6, 16, dtype=torch.float64)
    k = torch.randn(tree.storage_tokens, 3, 16, dtype=torch.float64)
    v = torch.randn_like(k)
    want = attention_f64(q.numpy(), k.numpy(), v.numpy(), tree)
    for r, path in enumerate(tree.paths):
        idx = torch.tensor(path)
        for h in range(6):
            s = (k[idx, h // 2] @ q[r, h]) / 4.0
            o = torch.softmax(s, 0) @ v[idx, h // 2]
            np.testing.assert_allclose(want[r, h], o.numpy(), atol=1e-12)


def test_closed_forms():
    torch.manual_seed(5)
    # one-token context: output is that token's V row for every query head of its KV head
    tree = KVTree.synthetic([-1, 0], [0, 1], [1])
    q = torch.randn(1, 4, 8)
    k = torch.randn(1, 2, 8)
    v = torch.randn(1, 2, 8)
    out = request_attention(q, k, v, tree)
    torch.testing.assert_close(out[0], v[0].repeat_interleave(2, 0))
    # equal scores (q = 0): mean of V over the path
    tree = KVTree.synthetic([-1, 0, 0], [5, 3, 2], [1, 2])
    q = torch.zeros(2, 4, 8)
    k = torch.randn(tree.storage_tokens, 2, 8)
    v = torch.randn_like(k)
    out = request_attention(q, k, v, tree)
    for r, path in enumerate(tree.paths):
        torch.testing.assert_close(out[r], v[list(path)].mean(0).repeat_interleave(2, 0))
    # a planted dominant key selects its V row
    k = torch.zeros(tree.storage_tokens, 2, 8)
    q = torch.zeros(2, 4, 8)
    q[:, :, 0] = 1.0
    k[6, :, 0] = 1000.0  # token 6 belongs to request 0's private node (ids 5..7)
    out = request_attention(q, k, v, tree)
    torch.testing.assert_close(out[0], v[6].repeat_interleave(2, 0))
    # GQA head mapping: query head h reads KV head h // G
    assert not torch.allclose(out[0, 0], out[0, 3])


def test_planted_mistakes_are_caught():
    tree, _ = semantics_trees()["unequal"]
    q, k, v = inputs(tree, 1)
    ref = request_attention(q, k, v, tree)
    plan = schedule(tree, 8, 2, 32, "fixed", CostModel(kv_split=48))
    # dropping one job (whose requests keep other jobs) changes their outputs
    drop = next(i for i, j in enumerate(plan.jobs)
                if all(any(r in o.requests for o in plan.jobs if o is not j) for r in j.requests))
    broken = Plan(plan.jobs[:drop] + plan.jobs[drop + 1:], "fixed", 0.0, plan.settings)
    with pytest.raises(AssertionError):
        torch.testing.assert_close(segmented_attention(q, k, v, broken), ref, atol=2e-5, rtol=2e-5)
    # a wrong softmax scale (sqrt(D) dropped) is caught by the float64 check
    bad = request_attention(q * math.sqrt(32), k, v, tree).double().numpy()
    want = attention_f64(q.numpy(), k.numpy(), v.numpy(), tree)
    assert np.abs(bad - want).max() > 1e-2
    # a transposed head mapping (h % HK instead of h // G) is caught
    want_t = attention_f64(q[:, [0, 4, 1, 5, 2, 6, 3, 7]].numpy(), k.numpy(), v.numpy(), tree)
    assert np.abs(want_t[:, [0, 2, 4, 6, 1, 3, 5, 7]] - want).max() > 1e-2


def test_output_dtype_and_relative_l2():
    tree, _ = semantics_trees()["noshare"]
    q, k, v = inputs(tree, 1)
    out = request_attention(q.bfloat16(), k.bfloat16(), v.bfloat16(), tree)
    assert out.dtype == torch.bfloat16
    assert relative_l2(out, out) == 0.0
    assert abs(relative_l2(2 * out.float(), out.float()) - 1.0) < 1e-12
