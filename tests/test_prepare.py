"""Plan lowering (reference kernels.py:103-141, 171-186) checked on CPU tensors, no launches."""
import pytest
import torch

from tree_attention import CostModel, KVTree, schedule, shapes
from tree_attention import _native, _planner, kernels
from tree_attention.kernels import CachedDecodePlan, prepare
from tree_attention.schedule import Job, Plan


def _covers_paths(prepared, tree):
    """Every request's execution jobs and attached segments cover its path exactly once."""
    seen = [[] for _ in tree.paths]
    for job in prepared.jobs:
        for r in job.requests:
            seen[r].extend(job.tokens)
    for segs in prepared.attached.values():
        for job, _ in segs:
            for r in job.requests:
                seen[r].extend(job.tokens)
    return all(sorted(seen[r]) == sorted(path) for r, path in enumerate(tree.paths))


def test_metadata_layout_small_first_and_compact_slots():
    tree = shapes.tree(shapes.headline())
    q = torch.empty(128, 32, 128, dtype=torch.bfloat16)
    p = prepare(schedule(tree, 32, 8, 128, "cube"), q, fuse_rows=0)
    # default model: 16-request groups x 512-token chunks of the root; each group's
    # chunks are re-cut into 4 chunks of 2032 tokens (8 groups x 4 x 8 heads = 256
    # one-tile workgroups), the 128 private tails stay small jobs
    assert p.small_jobs == 128 and len(p.jobs) == 128 + 32
    assert all(len(j.requests) == 1 and len(j.tokens) == 64 for j in p.jobs[:128])
    assert all(len(j.requests) == 16 and len(j.tokens) == 2032 for j in p.jobs[128:])
    assert _covers_paths(p, tree)
    assert p.contiguous_k
    qlen = p.qlen.tolist()
    rowbase = p.rowbase.tolist()
    assert rowbase == [sum(qlen[:i]) for i in range(len(qlen))]
    counts = p.counts.tolist()
    assert counts == [5] * 128
    # every request's slots point at rows of jobs that contain it
    slot_owner = {}
    for j, job in enumerate(p.jobs):
        for i, r in enumerate(job.requests):
            slot_owner[rowbase[j] + i] = r
    for r in range(128):
        assert {slot_owner[s] for s in p.slots[r, :counts[r]].tolist()} == {r}
    assert p.part.shape == (sum(qlen), 32, 128) and p.lse.shape == (sum(qlen), 32, 2)
    assert p.part.dtype == torch.float16 and p.lse.dtype == torch.float32
    # work items: one per (small job, head); every private tail is its request's only
    # small job, so all are TA_TAIL items that merge their request and no request is
    # left for the merge kernel; large jobs of 16 requests = 64 rows -> one 64-row tile per head
    assert p.abi.n_items[_native.TA_SMALL] == 0
    assert p.abi.n_items[_native.TA_TAIL] == 128 * 8
    tails = p.items[_native.TA_TAIL].view(-1, 3).tolist()
    assert sorted(tails) == [[j, 0, h] for j in range(128) for h in range(8)]
    assert p.abi.n_rest == 0 and p.rest.numel() == 0
    assert p.abi.n_items[_native.TA_LARGE64] == 32 * 8
    items = p.items[_native.TA_LARGE64].view(-1, 3).tolist()
    assert sorted(set((j, h) for j, _, h in items)) == [(j, h) for j in range(128, 160) for h in range(8)]


def test_recut_is_independent_of_the_plans_kv_split():
    """The GPU work split depends on the request groups, not on where the plan cut them."""
    tree = shapes.tree(shapes.headline())
    q = torch.empty(128, 32, 128, dtype=torch.bfloat16)
    splits = []
    for kv_split in (128, 256, 512, 8192):
        p = prepare(schedule(tree, 32, 8, 128, "cube", CostModel(kv_split=kv_split, max_query_rows=512)), q)
        assert _covers_paths(p, tree)
        splits.append([(j.requests, j.tokens[0], len(j.tokens)) for j in p.jobs])
    assert all(s == splits[0] for s in splits[1:])
    # 16 root chunks (512 rows = 2 tiles x 8 heads = 16 workgroups each): 256 workgroups
    assert sum(len(r) == 128 for r, _, _ in splits[0]) == 16


def test_recut_keeps_cached_tails_fixed():
    tree = shapes.tree(shapes.shared_prefix(4, 100, 20))
    prefix = tree.storage_tokens
    q = torch.empty(4, 32, 32, dtype=torch.float16)
    cached = CachedDecodePlan(schedule(tree, 32, 2, 32, "request", CostModel(kv_split=16)), q, prefix, 6)
    tails = [cached.prepared.jobs[i] for i in cached.tail_indices.tolist()]
    assert sorted((j.requests, j.tokens[0], len(j.tokens)) for j in tails) == [
        ((r,), prefix + 6 * r, 6) for r in range(4)]


def test_large_row_tiles():
    tree = shapes.tree(shapes.headline())
    q = torch.empty(128, 32, 128, dtype=torch.bfloat16)
    model = CostModel(max_query_rows=512, kv_split=256)
    p = prepare(schedule(tree, 32, 8, 128, "cube", model), q)
    n256 = p.abi.n_items[_native.TA_LARGE256]
    big = [j for j in p.jobs if len(j.requests) == 128]
    assert len(big) == 16 and n256 == 16 * 8 * 2
    p = prepare(schedule(tree, 32, 8, 128, "cube", model), q, tile_rows=128)
    assert p.abi.n_items[_native.TA_LARGE128] == 8 * 8 * 4  # 4 row tiles: 8 chunks fill the GPU


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


def test_tail_items_and_merge_rest():
    """TA_TAIL: single-request small jobs that are their request's only small job."""
    q = torch.empty(4, 8, 32, dtype=torch.float16)
    settings = dict(kvheads=2)
    jobs = [Job((0, 1, 2, 3), tuple(range(0, 40))),   # 16 rows: small, shared by all
            Job((0,), tuple(range(40, 50))),          # request 0 has two small jobs
            Job((1,), tuple(range(50, 60))),          # request 1: two small jobs as well
            Job((2,), tuple(range(60, 70)))]          # request 3 has only the shared job
    p = prepare(Plan(jobs, "x", 0.0, settings), q)
    assert p.abi.n_items[_native.TA_TAIL] == 0 and p.rest.tolist() == [0, 1, 2, 3]
    jobs = [Job((0, 1, 2, 3, 4, 5), tuple(range(0, 40))),  # 24 rows: large
            Job((0,), tuple(range(40, 50))), Job((1,), tuple(range(50, 60))),
            Job((2, 3), tuple(range(64, 70))), Job((1,), tuple(range(70, 74)))]
    q = torch.empty(6, 8, 32, dtype=torch.float16)
    p = prepare(Plan(jobs, "x", 0.0, settings), q, route_items=0)  # the large job stays large
    tail_jobs = sorted({j for j, _, _ in p.items[_native.TA_TAIL].view(-1, 3).tolist()})
    assert [p.jobs[j].requests for j in tail_jobs] == [(0,)]
    # request 1 has two small jobs, 2 and 3 share one, 4 and 5 have only the large job
    assert p.rest.tolist() == [1, 2, 3, 4, 5] and p.abi.n_rest == 5
    assert p.abi.n_items[_native.TA_SMALL] == 3 * 2


def test_private_tails_attach_to_root_items():
    """Headline under the MI355X model: each private tail is folded into one 256-row
    root work item holding its request's rows (four per item, on four waves)."""
    tree = shapes.tree(shapes.headline())
    q = torch.empty(128, 32, 128, dtype=torch.bfloat16)
    p = prepare(schedule(tree, 32, 8, 128, "cube", CostModel.mi355x()), q)
    # the root in 16 chunks over all 128 requests (request groups of one chunk fuse)
    assert p.small_jobs == 0 and len(p.jobs) == 16 and {len(j.requests) for j in p.jobs} == {128}
    assert _covers_paths(p, tree)
    assert p.abi.n_items[_native.TA_TAIL] == 0 and p.abi.n_items[_native.TA_SMALL] == 0
    assert p.counts.tolist() == [16] * 128 and p.abi.n_rest == 128
    assert sorted(len(v) for v in p.attached.values()) == [4] * 32
    tails = sorted(job.requests[0] for segs in p.attached.values() for job, _ in segs)
    assert tails == list(range(128))
    for (j, row0), segs in p.attached.items():
        job = p.jobs[j]
        waves = set()
        for tail, lrow in segs:
            r = tail.requests[0]
            assert lrow == job.requests.index(r) * 4 and row0 <= lrow < row0 + 256
            waves.add((lrow - row0) // 32)
        assert len(waves) == len(segs)  # one tail per wave of the item
    # device record: per TA_LARGE256 item (job, row0, head) the same segments
    stride = p.abi.xtail_stride
    xt = p.xtail.view(-1, stride).tolist()
    items = p.items[_native.TA_LARGE256].view(-1, 3).tolist()
    assert len(xt) == len(items) == 256
    for rec, (j, row0, h) in zip(xt, items):
        segs = p.attached[(j, row0)]
        assert rec[0] == len(segs)
        assert rec[1:1 + 4 * len(segs)] == [v for tail, lrow in segs
                                            for v in (tail.tokens[0], len(tail.tokens), lrow, 4)]
    # without attachment the tails are TA_TAIL jobs again
    p2 = prepare(schedule(tree, 32, 8, 128, "cube", CostModel.mi355x()), q, attach_tails=False)
    assert not p2.attached and p2.xtail is None and p2.abi.xtail is None
    assert p2.abi.n_items[_native.TA_TAIL] == 128 * 8 and _covers_paths(p2, tree)


def test_attachment_limits():
    """Tails attach only where the request's rows fit one wave, up to XTAIL_MAX segments and
    the item's own tile count -- at least ATTACH_MIN_CAP tiles when every candidate attaches
    (the layer then has no small-job launch), exactly its own when some stay small jobs;
    growing decode tails attach too, their lengths rewritten in the attachment records by
    fill_growing."""
    settings = dict(kvheads=1)
    q = torch.empty(80, 4, 32, dtype=torch.float16)   # group 4: 80 requests = 320 rows
    root = Job(tuple(range(80)), tuple(range(0, 64)))  # one tile of root tokens
    tails = [Job((r,), tuple(range(64 + 16 * r, 80 + 16 * r))) for r in range(80)]
    # two row tiles (rows 0-255, 256-319) of one job, one own tile each: each takes
    # XTAIL_MAX one-tile tails (within the ATTACH_MIN_CAP floor of attached tiles)
    assert kernels.XTAIL_MAX <= kernels.ATTACH_MIN_CAP
    left, att = kernels._attach_tails(tails, [root], 4, 256, lambda job: False)
    assert sorted((j, row0, len(s)) for (j, row0), s in att.items()) == [
        (0, 0, kernels.XTAIL_MAX), (0, 256, kernels.XTAIL_MAX)]
    assert len(left) == 80 - 2 * kernels.XTAIL_MAX
    # when every candidate fits, prepare attaches them all that way: one segment launch
    few = [t for t in tails if t.requests[0] % 64 < kernels.XTAIL_MAX]
    p = prepare(Plan([root] + few, "x", 0.0, settings), q)
    assert p.small_jobs == 0 and len(p.jobs) == 1
    assert sorted((j, row0, len(s)) for (j, row0), s in p.attached.items()) == [
        (0, 0, kernels.XTAIL_MAX), (0, 256, kernels.XTAIL_MAX)]
    # with tails left for the small-job kernel, an item takes no more tiles than its own (one)
    p = prepare(Plan([root] + tails, "x", 0.0, settings), q, route_items=0)
    assert sorted((j, row0, len(s)) for (j, row0), s in p.attached.items()) == [
        (p.small_jobs, 0, 1), (p.small_jobs, 256, 1)]
    assert len(p.jobs) == p.small_jobs + 1
    tree_paths = [tuple(range(0, 64)) + tuple(range(64 + 16 * r, 80 + 16 * r)) for r in range(80)]
    seen = [[] for _ in range(80)]
    for job in p.jobs:
        for r in job.requests:
            seen[r].extend(job.tokens)
    for segs in p.attached.values():
        for job, _ in segs:
            seen[job.requests[0]].extend(job.tokens)
    assert all(sorted(seen[r]) == list(tree_paths[r]) for r in range(80))
    # growing tails (fixed_from) attach the same way; fill_growing sets the klen of those
    # left as jobs and the token field of every record holding an attached one
    g = prepare(Plan([root] + few, "x", 0.0, settings), q, fixed_from=64)
    assert g.small_jobs == 0 and g.grow_offsets.numel() == 2 * kernels.XTAIL_MAX
    g = prepare(Plan([root] + tails, "x", 0.0, settings), q, fixed_from=64, route_items=0)
    assert {k: [(j.requests, lr) for j, lr in v] for k, v in g.attached.items()} == \
        {k: [(j.requests, lr) for j, lr in v] for k, v in p.attached.items()}
    njob_tails = sum(job.tokens[0] >= 64 for job in g.jobs)
    assert njob_tails == 80 - 2
    assert g.grow_offsets.numel() == njob_tails + 2
    g.fill_growing(3)
    assert (g.klen[torch.tensor([j.tokens[0] >= 64 for j in g.jobs])] == 3).all()
    recs = g.xtail.view(-1, 1 + 4 * kernels.XTAIL_MAX)
    assert (recs[:, 0] == 1).all()
    assert (recs[:, 2] == 3).all()  # every attached segment's token count
    assert (recs[:, 4] == 4).all()  # and its rows (one request, group 4)
    g.fill_growing(16)
    assert (recs[:, 2] == 16).all() and (g.klen[-1] == 64).all()
    # group 12: request 1's rows 12-23 lie in wave 0; request 2's rows 24-35 straddle waves 0 and 1
    q = torch.empty(24, 12, 32, dtype=torch.float16)
    root = Job(tuple(range(24)), tuple(range(0, 256)))
    p = prepare(Plan([root, Job((1,), (300, 301)), Job((2,), (302, 303))], "x", 0.0, settings), q,
                route_items=0)
    assert [(job.requests, lrow) for segs in p.attached.values() for job, lrow in segs] == [((1,), 12)]
    assert [job.requests for job in p.jobs[:p.small_jobs]] == [(2,)]


def test_affine_slot_layout():
    """The headline plan's slots are affine (request r's slot k is r + k * 128): prepare
    passes the stride, and the slot lists it still uploads hold exactly those values.
    Plans with ragged slot lists keep slot_stride 0."""
    tree = shapes.tree(shapes.headline())
    q = torch.empty(128, 32, 128, dtype=torch.bfloat16)
    p = prepare(schedule(tree, method="cube", model=CostModel.mi355x()), q)
    stride, maxs = p.abi.slot_stride, p.abi.maxs
    assert stride == 128 and maxs == 16
    slots = p.slots.reshape(128, maxs)
    assert (p.counts == maxs).all()
    assert torch.equal(slots, torch.arange(128)[:, None] + torch.arange(maxs)[None, :] * stride)
    assert int(slots.max()) < p.abi.nslot
    for spec in (shapes.nested_unequal(), shapes.cpu_baseline_shape()):
        tree = shapes.tree(spec)
        q = torch.empty(len(tree.paths), 32, 128, dtype=torch.bfloat16)
        assert prepare(schedule(tree, method="cube", model=CostModel.mi355x()), q).abi.slot_stride == 0


def test_nodes_of_a_wave_attach():
    """A job of a few requests whose rows lie in one wave of a 256-row item (a branch node over
    consecutive requests) attaches like a private tail; its record carries its row count, and
    the layer keeps one segment launch.  Jobs whose requests are not consecutive rows of one
    wave in the large job stay jobs."""
    settings = dict(kvheads=1)
    q = torch.empty(32, 4, 32, dtype=torch.float16)  # 32 requests x group 4 = 128 rows, waves of 8 requests
    root = Job(tuple(range(32)), tuple(range(0, 512)))
    branches = [Job(tuple(range(8 * b, 8 * b + 8)), tuple(range(512 + 64 * b, 576 + 64 * b))) for b in range(4)]
    misaligned = Job(tuple(range(4, 12)), tuple(range(800, 864)))    # rows 16-47: two waves
    gapped = Job((1, 3, 5, 7, 9), tuple(range(900, 932)))              # rows 4-7, 12-15, ...: not consecutive
    # root: 8 one-tile items of 4 segments each; 16 tails leave room for the nodes
    tails = [Job((r,), tuple(range(1000 + 16 * r, 1016 + 16 * r))) for r in range(0, 32, 2)]
    plan = Plan([root] + branches + [misaligned, gapped] + tails, "x", 0.0, settings)
    for native in (True, False):
        if native and not _planner.available():
            continue
        # consolidate_rows=0: the 20-row gapped job would otherwise take the root into 64-row items
        p = prepare(plan, q, consolidate_rows=0) if native else _prepare_python_attach(plan, q, consolidate_rows=0)
        segs = [(job.requests, lrow) for s in p.attached.values() for job, lrow in s]
        for b in range(4):
            assert (tuple(range(8 * b, 8 * b + 8)), 32 * b) in segs
        assert not any(req == misaligned.requests or req == gapped.requests for req, _ in segs)
        left = [job.requests for job in p.jobs]
        assert misaligned.requests in left and gapped.requests in left
        assert all(job.requests not in [br.requests for br in branches] for job in p.jobs)
        for (j, row0), s in p.attached.items():
            rec = p.xtail.view(-1, p.abi.xtail_stride)[[i for i, (jj, r0, h) in enumerate(
                p.items[_native.TA_LARGE256].view(-1, 3).tolist()) if (jj, r0) == (j, row0)][0]].tolist()
            assert rec[4:1 + 4 * len(s):4] == [4 * len(job.requests) for job, _ in s]
        assert _covers_paths_plan(p, plan, 32)


def _prepare_python_attach(plan, q, **kw):
    """prepare() with the Python attachment (kernels._attach_tails_py) instead of the host library's."""
    orig = kernels._attach_tails
    kernels._attach_tails = kernels._attach_tails_py
    try:
        return prepare(plan, q, **kw)
    finally:
        kernels._attach_tails = orig


def _covers_paths_plan(p, plan, nreq):
    """Every request's tokens in the prepared jobs and attachments are exactly its plan tokens."""
    want = [[] for _ in range(nreq)]
    for job in plan.jobs:
        for r in job.requests:
            want[r].extend(job.tokens)
    seen = [[] for _ in range(nreq)]
    for job in p.jobs:
        for r in job.requests:
            seen[r].extend(job.tokens)
    for segs in p.attached.values():
        for job, _ in segs:
            for r in job.requests:
                seen[r].extend(job.tokens)
    return all(sorted(seen[r]) == sorted(want[r]) for r in range(nreq))


def test_small_large_jobs_run_in_the_small_kernel():
    """When small jobs are left for the small-job kernel and the large jobs, cut into 16-row
    request groups, stream at most route_items (tile, KV head) units, the large jobs run as
    those groups in the small-job kernel: one segment launch, the same tokens per request.
    Above the limit, or when every small job attaches (no small-job launch), they stay large."""
    settings = dict(kvheads=2)
    q = torch.empty(32, 8, 32, dtype=torch.float16)   # group 4: 4 requests per 16-row group
    root = Job(tuple(range(32)), tuple(range(0, 256)))                      # 8 groups x 4 tiles
    tails = [Job((r,), tuple(range(256 + 768 * r, 256 + 768 * (r + 1)))) for r in range(32)]  # 12 tiles each
    plan = Plan([root] + tails, "x", 0.0, settings)
    p = prepare(plan, q)   # 8 groups x 4 tiles x 2 KV heads = 64 units
    assert len(p.jobs) == p.small_jobs and p.abi.n_items[_native.TA_LARGE256] == 0 and not p.attached
    assert sorted({job.requests for job in p.jobs if job.tokens[0] < 256}) == \
        [tuple(range(i, i + 4)) for i in range(0, 32, 4)]
    assert _covers_paths_plan(p, plan, 32)
    for limit, routed in ((0, False), (63, False), (64, True)):
        r = prepare(plan, q, route_items=limit)
        assert (r.small_jobs == len(r.jobs)) == routed and _covers_paths_plan(r, plan, 32)
    # one-token tails that all attach (the root's four 64-token chunks take four each): no
    # small-job launch to share, no routing
    short = [Job((r,), (256 + r,)) for r in range(16)]
    a = prepare(Plan([root] + short, "x", 0.0, settings), q)
    assert a.small_jobs == 0 and sum(map(len, a.attached.values())) == 16


def test_jobs_over_one_token_run_fuse():
    """Jobs over the same token run that together hold at least fuse_rows query rows and share
    no request run as one job over their requests: the headline under the reference's cost
    model (16-request groups of each 512-token root chunk) runs as 128-request chunks in the
    256-row kernel, with the slots of the 128-request plan.  Below the row count, or when two
    jobs share a request, they stay apart."""
    tree = shapes.tree(shapes.headline())
    q = torch.empty(128, 32, 128, dtype=torch.bfloat16)
    plan = schedule(tree, 32, 8, 128, "cube")
    assert {len(j.requests) for j in plan.jobs} == {1, 16}
    p = prepare(plan, q)
    assert {len(j.requests) for j in p.jobs[p.small_jobs:]} == {128}
    assert p.abi.n_items[_native.TA_LARGE256] == 256 and p.abi.n_items[_native.TA_LARGE64] == 0
    assert _covers_paths(p, tree)
    assert p.abi.slot_stride == 128
    settings = dict(kvheads=1)
    q = torch.empty(40, 4, 32, dtype=torch.float16)
    a, b = Job(tuple(range(0, 20)), tuple(range(0, 64))), Job(tuple(range(20, 40)), tuple(range(0, 64)))
    c = Job(tuple(range(0, 40)), tuple(range(64, 128)))
    fused = prepare(Plan([a, b, c], "x", 0.0, settings), q, fuse_rows=160)
    assert sorted(j.requests for j in fused.jobs) == [tuple(range(40))] * 2
    apart = prepare(Plan([a, b, c], "x", 0.0, settings), q, fuse_rows=161)
    assert sorted(len(j.requests) for j in apart.jobs) == [20, 20, 40]
    # per-request jobs (4 rows each) over one token run stay apart, whatever their number
    single = [Job((r,), tuple(range(0, 64))) for r in range(40)]
    alone = prepare(Plan(single + [c], "x", 0.0, settings), q, fuse_rows=1)
    assert sorted(j.requests for j in alone.jobs if j.tokens[0] < 64) == [(r,) for r in range(40)]
    shared = Job(tuple(range(19, 39)), tuple(range(0, 64)))   # request 19 in both
    q2 = torch.empty(39, 4, 32, dtype=torch.float16)
    kept = prepare(Plan([a, shared, Job((39 - 1,), (200,))], "x", 0.0, settings), q2, fuse_rows=1)
    assert sorted(len(j.requests) for j in kept.jobs if j.tokens[0] == 0) == [20, 20]


def test_wide_jobs_consolidate_into_64_row_items():
    """When 64-row items run anyway and no wider job holds more than consolidate_rows rows,
    the wider jobs run as 16-request (64-row) groups in the same kind: the layer launches one
    large-job kernel.  A group of at most 16 rows becomes a small job.  A wider job above the
    limit keeps the 256-row kind."""
    settings = dict(kvheads=2)
    q = torch.empty(40, 8, 32, dtype=torch.float16)   # group 4
    root = Job(tuple(range(35)), tuple(range(0, 640)))             # 140 rows
    half = Job(tuple(range(16)), tuple(range(640, 1280)))          # 64 rows: a 64-row item
    tails = [Job((r,), tuple(range(1280 + 40 * r, 1320 + 40 * r))) for r in range(40)]
    others = [Job(tuple(range(35, 40)), tuple(range(0, 640)))]     # the rest of the root's requests
    plan = Plan([root, half] + others + tails, "x", 0.0, settings)
    nreq = 40
    wide = prepare(plan, q, consolidate_rows=128, route_items=0)   # 140 rows > 128: kept
    assert wide.abi.n_items[_native.TA_LARGE256] > 0
    one = prepare(plan, q, consolidate_rows=160, route_items=0)
    assert one.abi.n_items[_native.TA_LARGE256] == 0 and one.abi.n_items[_native.TA_LARGE64] > 0
    groups = {j.requests for j in one.jobs if j.tokens[0] < 640}
    assert {tuple(range(0, 16)), tuple(range(16, 32))} <= groups and (32, 33, 34) in groups
    small = {j.requests for j in one.jobs[:one.small_jobs]}
    assert (32, 33, 34) in small                                   # 12 rows: a small job
    for p in (wide, one, prepare(plan, q, consolidate_rows=0, route_items=0), prepare(plan, q)):
        assert _covers_paths_plan(p, plan, nreq)
    # the 81-shape grid's 32-request, 99 %-shared, 3-level tree under the fitted model
    spec = next(s for p_, s in shapes.config_grid()
                if p_ == {"requests": 32, "context": 8192, "fraction": 0.99, "depth": 3})
    tree = shapes.tree(spec)
    q = torch.empty(32, 32, 128, dtype=torch.bfloat16)
    fitted = schedule(tree, 32, 8, 128, "cube", CostModel.mi355x())
    p = prepare(fitted, q)
    assert p.abi.n_items[_native.TA_LARGE256] == 0 and _covers_paths(p, tree)
    assert prepare(fitted, q, consolidate_rows=0).abi.n_items[_native.TA_LARGE256] > 0


def test_one_tile_chunks_lengthen_when_the_lowering_keeps_its_kinds():
    """The re-cut gives large chunks of at least LARGE_MIN_TILES tiles when the lowering
    then keeps its kernel kinds, attaches as much and still has half a work item per CU."""
    assert kernels.LARGE_MIN_TILES == 2
    # "wide": 32 requests over 2048 shared tokens + 64 private each, fitted model.  One
    # tile per chunk gives 32 chunks x 8 heads = 256 items; two tiles give 128 items
    tree = shapes.tree(shapes.benchmark_cases()["wide"])
    q = torch.empty(32, 32, 128, dtype=torch.bfloat16)
    plan = schedule(tree, 32, 8, 128, "cube", CostModel.mi355x())
    one = prepare(plan, q, large_min_tiles=1)
    two = prepare(plan, q)
    assert one.abi.n_items[_native.TA_LARGE256] == 256 and two.abi.n_items[_native.TA_LARGE256] == 128
    assert {len(j.tokens) for j in one.jobs} == {64} and {len(j.tokens) for j in two.jobs} == {128}
    # every private tail attached in both: no small-job launch
    assert one.small_jobs == two.small_jobs == 0
    assert sum(map(len, one.attached.values())) == sum(map(len, two.attached.values())) == 32
    assert two.abi.nslot * 2 == one.abi.nslot
    assert _covers_paths(one, tree) and _covers_paths(two, tree)
    # chunks of at least two tiles already (the headline root): nothing changes
    head = shapes.tree(shapes.headline())
    qh = torch.empty(128, 32, 128, dtype=torch.bfloat16)
    hp = schedule(head, 32, 8, 128, "cube", CostModel.mi355x())
    a, b = prepare(hp, qh, large_min_tiles=1), prepare(hp, qh)
    assert [(j.requests, j.tokens) for j in a.jobs] == [(j.requests, j.tokens) for j in b.jobs]
    # the Qwen3-4B-shaped decode layer: two-tile chunks would leave its tails and branch
    # nodes unattached, so the lowering stays as it is
    qt = KVTree.from_sequences(shapes.qwen3_4b_workload())
    qq = torch.empty(len(qt.paths), 32, 128, dtype=torch.bfloat16)
    qp = schedule(qt, 32, 8, 128, "cube", CostModel.mi355x())
    t0 = qt.storage_tokens   # 16 reserved tokens per request, as CachedDecodePlan lays them out
    tails = [Job((r,), tuple(range(t0 + 16 * r, t0 + 16 * (r + 1)))) for r in range(len(qt.paths))]
    qp = Plan(qp.jobs + tails, qp.method, qp.estimated_us, qp.settings)
    a, b = prepare(qp, qq, large_min_tiles=1, fixed_from=t0), prepare(qp, qq, fixed_from=t0)
    assert b.jobs == CachedDecodePlan(schedule(qt, 32, 8, 128, "cube", CostModel.mi355x()), qq, t0, 16).prepared.jobs
    assert [(j.requests, j.tokens) for j in a.jobs] == [(j.requests, j.tokens) for j in b.jobs]
    assert list(a.abi.n_items) == list(b.abi.n_items)


def test_wide_jobs_fill_the_gpu_as_64_row_groups():
    """A 128-row root whose 256-row items, cut into one-tile chunks, fill more than a quarter but
    at most half of the 256 CUs runs as two 64-row request groups per chunk instead (the
    decode-plan protocol's layer: 32 requests x 1024 shared tokens, 16 chunks x 8 KV heads = 128
    256-row items -> 64-row groups); a root long enough to fill the GPU in 256-row items keeps
    them (the Qwen3-4B-shaped layer's 2048-token root: 256 items, tails attached)."""
    from tree_attention import CostModel, schedule, shapes
    from tree_attention.kernels import CachedDecodePlan
    layers = {name: (tree, reserved) for name, tree, reserved, _ in shapes.decode_layers()}
    tree, reserved = layers["protocol_r32_1024_64"]
    q = torch.zeros(len(tree.paths), 32, 128, dtype=torch.bfloat16)
    p = CachedDecodePlan(schedule(tree, 32, 8, 128, "cube", CostModel.mi355x()), q, tree.storage_tokens, reserved)
    n = list(p.prepared.abi.n_items)
    assert n[_native.TA_LARGE256] == 0 and n[_native.TA_LARGE64] == 128
    assert all(len(j.requests) <= 16 for j in p.prepared.jobs)
    tree, reserved = layers["qwen3_4b"]
    p = CachedDecodePlan(schedule(tree, 32, 8, 128, "cube", CostModel.mi355x()), q, tree.storage_tokens, reserved)
    n = list(p.prepared.abi.n_items)
    assert n[_native.TA_LARGE256] == 256 and n[_native.TA_LARGE64] == 0 and p.prepared.attached


def test_large_recut_keeps_one_round_of_items():
    """A large-kind re-cut that would give a few more items than CUs (a second round of work
    items for the surplus) takes the next longer chunks when one round of them is shorter than
    two rounds of the shorter chunks: 32 requests over a 4096-token context, 99 % shared in three
    levels, lowers to 192 64-row items instead of 272."""
    from tree_attention import CostModel, schedule, shapes
    tree = shapes.tree(shapes.grid_tree(32, 4096, 0.99, 3))
    q = torch.zeros(len(tree.paths), 32, 128, dtype=torch.bfloat16)
    p = prepare(schedule(tree, 32, 8, 128, "cube", CostModel.mi355x()), q)
    assert p.abi.n_items[_native.TA_LARGE64] == 192
    assert _covers_paths_plan(p, schedule(tree, 32, 8, 128, "cube", CostModel.mi355x()), len(tree.paths))


def test_fill_rule_leaves_long_private_parts_attached():
    """The 64-row fill rule needs every small job to be one tile: the benchmark case `unequal`
    (32 requests over a 1024-token root, private parts of 32..993 tokens) keeps its 128-row
    root in 256-row items with private parts attached."""
    from tree_attention import CostModel, schedule, shapes
    tree = shapes.tree(shapes.benchmark_cases()["unequal"])
    q = torch.zeros(len(tree.paths), 32, 128, dtype=torch.bfloat16)
    p = prepare(schedule(tree, 32, 8, 128, "cube", CostModel.mi355x()), q)
    assert p.abi.n_items[_native.TA_LARGE256] > 0 and p.abi.n_items[_native.TA_LARGE64] == 0 and p.attached


def test_small_launch_takes_two_tile_chunks(monkeypatch):
    """A launch of small-job items alone takes two-tile chunks when one-tile chunks would fill at
    least 45 % of its 2048 waves: 32 requests over 1024-token contexts, 25 % shared, lower to
    1664 two-tile items (8 partial slots per request) instead of 3328 one-tile items (16 slots),
    and 16 such requests to 832 instead of 1664.  With 75 % shared, 16 requests give 896
    one-tile items (44 % of the waves) and keep them."""
    from tree_attention import CostModel, schedule, shapes
    for nreq, fraction, one, two in ((32, 0.25, 3328, 1664), (16, 0.25, 1664, 832), (16, 0.75, 896, 896)):
        tree = shapes.tree(shapes.grid_tree(nreq, 1024, fraction, 1))
        q = torch.zeros(len(tree.paths), 32, 128, dtype=torch.bfloat16)
        plan = schedule(tree, 32, 8, 128, "cube", CostModel.mi355x())
        p = prepare(plan, q)
        assert list(p.abi.n_items) == [two, 0, 0, 0, 0]
        assert _covers_paths(p, tree)
        monkeypatch.setattr(kernels, "SMALL_PAIRS", False)
        assert list(prepare(plan, q).abi.n_items) == [one, 0, 0, 0, 0]
        monkeypatch.setattr(kernels, "SMALL_PAIRS", True)
    # two-tile chunks of 128 tokens: 2 of the shared 256 tokens and 6 of each private 768 per request
    tree = shapes.tree(shapes.grid_tree(32, 1024, 0.25, 1))
    p = prepare(schedule(tree, 32, 8, 128, "cube", CostModel.mi355x()),
                torch.zeros(32, 32, 128, dtype=torch.bfloat16))
    assert max(len(j.tokens) for j in p.jobs) == 128 and p.abi.maxs == 8
