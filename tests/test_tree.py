"""KVTree behaviour (reference src/tree_attention/tree.py; tests/test_semantics.py:11-14,36-43)."""
import json
from pathlib import Path

import pytest

from tree_attention import KVTree

GOLDEN = Path(__file__).parent / "golden"


def test_unequal_nested_terminal_and_duplicate_sequences():
    tree = KVTree.from_sequences([[1, 2, 3], [1, 2], [1, 2, 4, 5, 6], [7, 8], [1, 2, 3]])
    assert tree.storage_tokens == 8
    assert tree.paths[0] == tree.paths[4]
    assert tree.paths[1] == tree.paths[0][:2]
    assert tree.token_ids == [1, 2, 3, 4, 5, 6, 7, 8]


def test_extension_keeps_private_paths_compressed():
    tree = KVTree.from_sequences([[1, 2], [1, 2], [3, 4]])
    leaves = [next(i for i, n in enumerate(tree.nodes) if r in n.terminal) for r in range(3)]
    tree.extend_leaves(leaves, [4, 5, 6])
    assert len(tree.nodes) == 5
    tree.extend_leaves(leaves, [7, 8, 9])
    assert len(tree.nodes) == 5
    assert tree.paths[0] == (0, 1, 4, 7) and tree.paths[2] == (2, 3, 6, 9)


def test_synthetic_ids_are_closed_form():
    parents, lengths = [-1, 0, 1, 1, 0], [129, 65, 17, 33, 81]
    tree = KVTree.synthetic(parents, lengths, [2, 3, 4])
    starts = [sum(lengths[:i]) for i in range(len(lengths))]
    for i, node in enumerate(tree.nodes):
        assert node.tokens == tuple(range(starts[i], starts[i] + lengths[i]))
    assert tree.paths[0] == tree.nodes[0].tokens + tree.nodes[1].tokens + tree.nodes[2].tokens
    assert tree.nodes[1].requests == (0, 1) and tree.nodes[0].requests == (0, 1, 2)


@pytest.mark.parametrize("bad", [[], [[1], []]])
def test_empty_context_raises(bad):
    with pytest.raises(ValueError):
        KVTree.from_sequences(bad)


def test_synthetic_validation():
    with pytest.raises(ValueError):
        KVTree.synthetic([0, 0], [1, 1], [1])
    with pytest.raises(ValueError):
        KVTree.synthetic([-1, 0], [0, 0], [1])


def test_deep_chain_without_recursion_limit():
    # 3000 requests, each one token longer than the previous: a 3000-deep chain
    seqs = [list(range(1, n + 2)) for n in range(3000)]
    tree = KVTree.from_sequences(seqs)
    assert tree.storage_tokens == 3000
    assert tree.paths[-1] == tuple(range(3000))


def test_real_token_workloads_storage():
    """configs/qwen_workloads.json trees: storage = allocated - 8 x 16 in results/qwen4b.json."""
    data = json.loads((GOLDEN / "qwen_workload_trees.json").read_text())
    for name, w in data["workloads"].items():
        tree = KVTree.from_sequences(w["sequences"])
        assert tree.storage_tokens == w["allocated_kv_tokens"] - 8 * data["new_tokens_per_request"], name
        assert sum(map(len, tree.paths)) == sum(map(len, w["sequences"]))


def test_node_structure_matches_reference():
    """Exact node order / ids of from_sequences vs the reference implementation's output."""
    data = json.loads((GOLDEN / "plan_fixtures.json").read_text())
    checked = 0
    for case in data["cases"]:
        if "tree" not in case:  # digest-only plan cases
            continue
        if case["kind"] == "sequences":
            tree = KVTree.from_sequences(case["spec"])
        else:
            tree = KVTree.synthetic(*case["spec"])
        want = case["tree"]
        assert tree.storage_tokens == want["storage_tokens"], case["name"]
        got = [[n.parent, _runs(n.tokens), list(n.children), list(n.terminal), list(n.requests)]
               for n in tree.nodes]
        assert got == want["nodes"], case["name"]
        assert [_runs(p) for p in tree.paths] == want["paths"], case["name"]
        checked += 1
    assert checked >= 50


def _runs(tokens):
    out = []
    for t in tokens:
        if out and out[-1][0] + out[-1][1] == t:
            out[-1][1] += 1
        else:
            out.append([t, 1])
    return out
