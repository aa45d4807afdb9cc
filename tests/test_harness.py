"""Benchmark-harness helpers (tree_attention/harness.py), on CPU tensors.

``reference_fp32`` must be the reference's reference.py:4-13 arithmetic: it is
compared with the oracle's ``request_attention`` (itself pinned by a float64
brute force in test_oracle.py) on the reference's semantic trees and on a
shared-prefix tree with GQA group 4; ``check`` must reject a planted error.
"""
import pytest
import torch

from oracle.attention_oracle import request_attention
from tree_attention import KVTree, shapes
from tree_attention.harness import check, pool_bytes, reference_fp32, rotated_pools


@pytest.mark.parametrize("tree", [
    KVTree.from_sequences([[1, 2, 3], [1, 2], [1, 2, 4, 5, 6], [7, 8], [1, 2, 3]]),
    shapes.tree(shapes.shared_prefix(6, 40, [3, 9, 1, 17, 5, 8])),
    shapes.tree(shapes.benchmark_cases()["deep"]),
], ids=["semantics", "shared_prefix", "deep"])
def test_reference_fp32_equals_oracle(tree):
    g = torch.Generator().manual_seed(5)
    hq, hk, d = 8, 2, 32
    q = torch.randn(len(tree.paths), hq, d, generator=g)
    k = torch.randn(tree.storage_tokens, hk, d, generator=g)
    v = torch.randn(tree.storage_tokens, hk, d, generator=g)
    got = reference_fp32(q, k, v, tree)
    want = request_attention(q, k, v, tree)
    torch.testing.assert_close(got, want.float(), atol=2e-6, rtol=2e-5)


def test_check_rejects_a_planted_error():
    tree = shapes.tree(shapes.shared_prefix(4, 16, 4))
    g = torch.Generator().manual_seed(1)
    q = torch.randn(4, 8, 32, generator=g).bfloat16()
    k = torch.randn(tree.storage_tokens, 2, 32, generator=g).bfloat16()
    v = torch.randn(tree.storage_tokens, 2, 32, generator=g).bfloat16()
    ref = reference_fp32(q, k, v, tree)
    out = ref.bfloat16()
    err = check(out, ref, "exact")
    assert err["rel_l2"] < 4e-3
    bad = out.clone()
    bad[2, 3, 7] += 0.5
    with pytest.raises(AssertionError, match="planted"):
        check(bad, ref, "planted")


def test_rotated_pools_span_the_requested_bytes():
    kp = torch.zeros(2, 16, 1000, dtype=torch.bfloat16)
    vp = torch.zeros(2, 1000, 16, dtype=torch.bfloat16)
    pools = rotated_pools(kp, vp, min_bytes=1_000_000)
    per = 2 * kp.numel() * 2
    assert len(pools) == -(-1_000_000 // per) and pool_bytes(pools) >= 1_000_000
    assert pools[0][0] is kp and all(p[0].data_ptr() != kp.data_ptr() for p in pools[1:])
    assert len(rotated_pools(kp, vp, min_bytes=1)) == 1
