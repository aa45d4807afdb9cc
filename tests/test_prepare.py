"""Plan lowering (reference kernels.py:103-141, 171-186) checked on CPU tensors, no launches."""
import pytest
import torch

from tree_attention import CostModel, KVTree, schedule, shapes
from tree_attention import _native
from tree_attention.kernels import CachedDecodePlan, prepare
from tree_attention.schedule import Job, Plan


def test_metadata_layout_small_first_and_compact_slots():
    tree = shapes.tree(shapes.headline())
    q = torch.empty(128, 32, 128, dtype=torch.bfloat16)
    p = prepare(schedule(tree, 32, 8, 128, "cube"), q)
    assert len(p.jobs) == 256 and p.small_jobs == 128
    assert all(len(j.requests) == 1 for j in p.jobs[:128])
    assert p.contiguous_k
    qlen = p.qlen.tolist()
    rowbase = p.rowbase.tolist()
    assert rowbase == [sum(qlen[:i]) for i in range(len(qlen))]
    counts = p.counts.tolist()
    assert counts == [17] * 128
    # every request's slots point at rows of jobs that contain it
    slot_owner = {}
    for j, job in enumerate(p.jobs):
        for i, r in enumerate(job.requests):
            slot_owner[rowbase[j] + i] = r
    for r in range(128):
        assert {slot_owner[s] for s in p.slots[r, :counts[r]].tolist()} == {r}
    assert p.part.shape == (sum(qlen), 32, 128) and p.lse.shape == (sum(qlen), 32)
    # work items: 128 small jobs; large jobs of 16 requests = 64 rows -> one 64-row tile per head
    assert p.abi.n_items[_native.TA_SMALL] == 128 * 8
    small = p.items[_native.TA_SMALL].view(-1, 3).tolist()
    assert sorted(small) == [[j, 0, h] for j in range(128) for h in range(8)]
    assert p.abi.n_items[_native.TA_LARGE64] == 128 * 8
    items = p.items[_native.TA_LARGE64].view(-1, 3).tolist()
    assert sorted(set((j, h) for j, _, h in items)) == [(j, h) for j in range(128, 256) for h in range(8)]


def test_large_row_tiles():
    tree = shapes.tree(shapes.headline())
    q = torch.empty(128, 32, 128, dtype=torch.bfloat16)
    model = CostModel(max_query_rows=512, kv_split=256)
    p = prepare(schedule(tree, 32, 8, 128, "cube", model), q)
    n256 = p.abi.n_items[_native.TA_LARGE256]
    big = [j for j in p.jobs if len(j.requests) == 128]
    assert len(big) == 32 and n256 == 32 * 8 * 2


def test_rejects_bad_jobs():
    q = torch.empty(2, 8, 32)
    settings = dict(kvheads=2)
    with pytest.raises(ValueError):
        prepare(Plan([Job((0,), (0, 1)), Job((5,), (2,))], "x", 0.0, settings), q)
    with pytest.raises(ValueError):
        prepare(Plan([Job((0, 1), (0, 2, 1, 3))], "x", 0.0, settings), q)


def test_cached_decode_plan_tails():
    """kernels.py:171-186: tails are reserved contiguous runs; update sets their lengths."""
    base = shapes.tree(shapes.shared_prefix(4, 32, 8))
    prefix = base.storage_tokens
    q = torch.empty(4, 8, 32, dtype=torch.float16)
    cached = CachedDecodePlan(schedule(base, 8, 2, 32, "fixed"), q, prefix, 5)
    p = cached.prepared
    tails = cached.tail_indices.tolist()
    assert len(tails) == 4
    for i in tails:
        assert p.jobs[i].tokens[0] >= prefix and len(p.jobs[i].tokens) == 5
    cached.update(3)
    assert [p.klen[i].item() for i in tails] == [3, 3, 3, 3]
    others = [i for i in range(len(p.jobs)) if i not in tails]
    assert all(p.klen[i].item() == len(p.jobs[i].tokens) for i in others)
    with pytest.raises(ValueError):
        cached.update(6)
