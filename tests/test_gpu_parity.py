"""GPU parity of the HIP backend against the CPU FP32 oracle (reference src/tree_attention/reference.py).

Tolerances are the reference's own device tolerances -- atol .006 / rtol .02
(scripts/check_npu.py:29) for the small trees and atol .008 / rtol .03
(scripts/benchmark.py:96) for the benchmark shapes -- plus the per-layer
relative L2 bound of 0.3% against the FP32 oracle evaluated on the same
(bf16/fp16-valued) Q/K/V.
"""
import ctypes
import sys

import numpy as np
import pytest
import torch

from oracle.attention_oracle import relative_l2, request_attention
from tree_attention import CostModel, KVTree, schedule, shapes
from tree_attention import _native
from tree_attention.kernels import (CachedDecodePlan, attention, attention_matrix, decode_append, merge, pack_kv,
                                    prepare, segment, tail_merge)
from tree_attention.schedule import Job, Plan

pytestmark = pytest.mark.gpu
METHODS = ("request", "fixed", "greedy", "cube")
REL_L2 = 3e-3
MI355X_LIKE = CostModel(bandwidth=5.0e6, cube_flops=1.0e9, task_us=0.5, merge_us=0.01, cube_rows=16,
                        key_tile=64, kv_split=256, max_query_rows=512)


def say(*args):
    print(*args, flush=True)
    sys.stdout.flush()


def make_inputs(tree, hq, hk, d, dtype, seed, tcap=None, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    t = tree.storage_tokens if tcap is None else tcap
    q = (torch.randn(len(tree.paths), hq, d, generator=g) * scale).to(dtype)
    k = torch.randn(t, hk, d, generator=g).to(dtype)
    v = torch.randn(t, hk, d, generator=g).to(dtype)
    return q, k, v


def oracle_fp32(q, k, v, tree):
    return request_attention(q.float(), k.float(), v.float(), tree)


def check(out, ref32, atol, rtol, what):
    ref = ref32.to(out.dtype)
    err = relative_l2(out.cpu(), ref32)
    torch.testing.assert_close(out.cpu(), ref, atol=atol, rtol=rtol, msg=lambda m: f"{what}: {m}")
    assert err <= REL_L2, (what, err)
    return err


def run(tree, method, model, q, k, v, device, heads):
    plan = schedule(tree, heads[0], heads[1], heads[2], method, model)
    plan.validate(tree)
    qd = q.to(device)
    kp, vp = pack_kv(k.to(device), v.to(device))
    prepared = prepare(plan, qd)
    out = attention_matrix(qd, kp, vp, prepared)
    torch.cuda.synchronize()
    return out


SEMANTICS = {
    "unequal": (lambda: KVTree.from_sequences([[1, 2, 3], [1, 2], [1, 2, 4, 5, 6], [7, 8], [1, 2, 3]]), 1.0),
    "noshare": (lambda: KVTree.from_sequences([[1, 2, 3], [4], [5, 6, 7, 8, 9]]), 1.0),
    "deep": (lambda: KVTree.synthetic([-1, 0, 1, 1, 0], [129, 65, 17, 33, 81], [2, 3, 4]), 30.0),
}


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("name", list(SEMANTICS))
def test_semantics_trees_d32(name, dtype, device):
    """tests/test_semantics.py trees (8 Q / 2 KV heads, d=32, kv_split=48), incl. logits x30."""
    build, scale = SEMANTICS[name]
    tree = build()
    q, k, v = make_inputs(tree, 8, 2, 32, dtype, 17, scale=scale)
    ref = oracle_fp32(q, k, v, tree)
    for method in METHODS:
        say("semantics", name, dtype, method)
        out = run(tree, method, CostModel(kv_split=48), q, k, v, device, (8, 2, 32))
        check(out, ref, 0.006, 0.02, f"{name}/{method}")


NPU_TREES = {
    "unequal": lambda: KVTree.synthetic([-1, 0, 0, 1, 1], [129, 65, 17, 33, 81], [2, 3, 4]),
    "none": lambda: KVTree.from_sequences([[1, 2, 3], [4], [5, 6, 7, 8, 9]]),
    "duplicate_terminal": lambda: KVTree.from_sequences([[1, 2], [1, 2], [1, 2, 3, 4], [1, 5, 6]]),
    "wide": lambda: KVTree.synthetic([-1] + [0] * 32, [257] + [31 + i for i in range(32)], list(range(1, 33))),
}


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("name", list(NPU_TREES))
def test_device_suite_d64(name, dtype, device):
    """scripts/check_npu.py: 4 trees x {fp16, bf16} x 4 methods, 8 Q / 2 KV, d=64, kv_split=128."""
    tree = NPU_TREES[name]()
    q, k, v = make_inputs(tree, 8, 2, 64, dtype, 2026)
    ref = oracle_fp32(q, k, v, tree)
    for method in METHODS:
        say("npu-suite", name, dtype, method)
        out = run(tree, method, CostModel(kv_split=128), q, k, v, device, (8, 2, 64))
        check(out, ref, 0.006, 0.02, f"{name}/{method}")


@pytest.mark.parametrize("name", ["no_share", "wide", "unequal", "deep"])
def test_benchmark_cases(name, device):
    """scripts/benchmark.py shapes, bf16, 32 Q / 8 KV, d=128, default and MI355X-like cost models."""
    tree = shapes.tree(shapes.benchmark_cases()[name])
    q, k, v = make_inputs(tree, 32, 8, 128, torch.bfloat16, 101)
    ref = oracle_fp32(q, k, v, tree)
    for model in (CostModel(), MI355X_LIKE):
        for method in METHODS:
            say("bench-case", name, method, model.max_query_rows)
            out = run(tree, method, model, q, k, v, device, (32, 8, 128))
            check(out, ref, 0.008, 0.03, f"{name}/{method}")


def test_headline_shape(device):
    """128 requests x 8192 tokens, 8128 shared, bf16: rel-L2 <= 0.3% for cube (both models) and request."""
    tree = shapes.tree(shapes.headline())
    q, k, v = make_inputs(tree, 32, 8, 128, torch.bfloat16, 101)
    say("headline oracle")
    ref = oracle_fp32(q, k, v, tree)
    errs = {}
    for method, model in (("cube", CostModel()), ("cube", MI355X_LIKE), ("request", CostModel()),
                          ("fixed", MI355X_LIKE)):
        say("headline", method, model.max_query_rows)
        out = run(tree, method, model, q, k, v, device, (32, 8, 128))
        errs[(method, model.max_query_rows)] = check(out, ref, 0.008, 0.03, f"headline/{method}")
    say("headline rel-L2", errs)


def test_nested_unequal_tree(device):
    """Root 4096 -> 8 x 1024 -> 4 x 256, an internal terminal and two duplicates; all methods."""
    tree = shapes.tree(shapes.nested_unequal())
    q, k, v = make_inputs(tree, 32, 8, 128, torch.bfloat16, 7)
    ref = oracle_fp32(q, k, v, tree)
    for model in (CostModel(), MI355X_LIKE):
        for method in METHODS:
            say("nested", method, model.max_query_rows)
            out = run(tree, method, model, q, k, v, device, (32, 8, 128))
            check(out, ref, 0.008, 0.03, f"nested/{method}")


def test_small_launch_two_tile_chunks(device, monkeypatch):
    """A launch of small-job items alone with two-tile chunks (prepare's SMALL_PAIRS: 32
    requests over 1024-token contexts, 25 % shared, lower to 1664 two-tile items, 8 slots per
    request) matches the oracle, as the same plan lowered to 3328 one-tile items does."""
    from tree_attention import kernels
    tree = shapes.tree(shapes.grid_tree(32, 1024, 0.25, 1))
    q, k, v = make_inputs(tree, 32, 8, 128, torch.bfloat16, 43)
    plan = schedule(tree, 32, 8, 128, "cube", CostModel.mi355x())
    qd = q.to(device)
    kp, vp = pack_kv(k.to(device), v.to(device))
    ref = oracle_fp32(q, k, v, tree)
    for pairs, items, slots in ((True, 1664, 8), (False, 3328, 16)):
        monkeypatch.setattr(kernels, "SMALL_PAIRS", pairs)
        prepared = prepare(plan, qd)
        assert list(prepared.abi.n_items) == [items, 0, 0, 0, 0] and prepared.abi.maxs == slots
        say("two-tile chunks", pairs, "items", items)
        out = attention_matrix(qd, kp, vp, prepared)
        torch.cuda.synchronize()
        check(out, ref, 0.008, 0.03, f"small launch, pairs={pairs}")


@pytest.mark.parametrize("hq,hk,d", [(8, 2, 32), (8, 2, 64), (32, 8, 128)])
def test_merge_of_many_slots(hq, hk, d, device):
    """More than 16 partial slots per request (the merge splits them into two ranges), ragged counts
    (11 to 45 slots), and 8 query heads, which fill only part of a merge workgroup at d = 32 and 64."""
    tree = shapes.tree(shapes.shared_prefix(6, 700, [1, 33, 900, 17, 2130, 64]))
    q, k, v = make_inputs(tree, hq, hk, d, torch.bfloat16, 5)
    ref = oracle_fp32(q, k, v, tree)
    model = CostModel(kv_split=64)
    plan = schedule(tree, hq, hk, d, "request", model)
    counts = prepare(plan, q.to(device)).counts.cpu()
    assert counts.max() > 16 and counts.min() < 16 and counts.max() % 2 == 1, counts
    for method in METHODS:
        say("many-slots", hq, hk, d, method)
        out = run(tree, method, model, q, k, v, device, (hq, hk, d))
        check(out, ref, 0.008, 0.03, f"many-slots{hq}/{d}/{method}")


@pytest.mark.parametrize("hq,hk", [(8, 8), (16, 2), (32, 2), (64, 4)])
def test_group_sizes(hq, hk, device):
    """GQA group sizes 1, 8, 16, 16 (rows per request up to one full 16-row block)."""
    tree = shapes.tree(shapes.shared_prefix(20, 300, [5 + 7 * i for i in range(20)]))
    q, k, v = make_inputs(tree, hq, hk, 64, torch.bfloat16, 11)
    ref = oracle_fp32(q, k, v, tree)
    for method in METHODS:
        say("group", hq, hk, method)
        out = run(tree, method, CostModel(kv_split=100, max_query_rows=96), q, k, v, device, (hq, hk, 64))
        check(out, ref, 0.008, 0.03, f"group{hq}/{hk}/{method}")


def test_misaligned_pool_and_ragged_jobs(device):
    """Odd pool capacity (rows not 16-byte aligned), odd job starts, 1-token jobs, partial tiles."""
    tree = KVTree.synthetic([-1, 0, 0, 1, 1, 2, 0], [77, 1, 130, 3, 65, 200, 9], [3, 4, 5, 5, 6, 1])
    q, k, v = make_inputs(tree, 32, 8, 128, torch.bfloat16, 5, tcap=tree.storage_tokens + 3)
    ref = oracle_fp32(q, k, v, tree)
    for model in (CostModel(kv_split=33), CostModel(kv_split=64, max_query_rows=8), MI355X_LIKE):
        for method in METHODS:
            say("ragged", method, model.kv_split)
            out = run(tree, method, model, q, k, v, device, (32, 8, 128))
            check(out, ref, 0.008, 0.03, f"ragged/{method}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("pad", [0, 3, 8])
def test_large_row_tiles_all_kinds(pad, dtype, device):
    """Jobs of 20, 40, 100 and 300 requests exercise the 64/128/256-row tile kernels.

    The pool capacity is 1016 + pad tokens: a multiple of 8 (pad 0, 8) selects the
    LDS-transpose kernels, pad 3 the register-transpose kernels for unaligned pools.
    """
    tree = KVTree.synthetic([-1, 0, 0, 0, 0], [700, 90, 33, 64, 129],
                            [1] * 20 + [2] * 40 + [3] * 100 + [4] * 140)
    q, k, v = make_inputs(tree, 32, 8, 128, dtype, 9, tcap=tree.storage_tokens + pad)
    ref = oracle_fp32(q, k, v, tree)
    qd = q.to(device)
    kp, vp = pack_kv(k.to(device), v.to(device))
    for model in (CostModel(max_query_rows=1200, kv_split=512), CostModel(max_query_rows=256, kv_split=190)):
        for tile_rows in (256, 128, 64):  # 65..256-row jobs take 256-row items unless tile_rows caps them
            say("large-tiles", pad, dtype, model.max_query_rows, tile_rows)
            prepared = prepare(schedule(tree, 32, 8, 128, "fixed", model), qd, tile_rows=tile_rows)
            n = prepared.abi.n_items
            allowed = {256: (_native.TA_LARGE64, _native.TA_LARGE256), 128: (_native.TA_LARGE64, _native.TA_LARGE128),
                       64: (_native.TA_LARGE64,)}[tile_rows]
            assert all(n[k] == 0 for k in (_native.TA_LARGE64, _native.TA_LARGE128, _native.TA_LARGE256)
                       if k not in allowed) and n[allowed[-1]] > 0
            out = attention_matrix(qd, kp, vp, prepared)
            torch.cuda.synchronize()
            check(out, ref, 0.008, 0.03, f"large-tiles/{tile_rows}")


@pytest.mark.parametrize("name", ["deep", "wide"])
def test_attention_packs_and_c_abi_phases_agree(name, device):
    """attention(q,k,v) == attention_matrix on packed pools == per-kind launches of the plan
    (kernels.segment / kernels.merge, i.e. ta_segment_plan + ta_merge_plan) and the fused
    tail-merge order (kernels.tail_merge).  The raw ta_segment / ta_merge entry points are
    covered by test_raw_segment_and_merge_entry_points."""
    tree = shapes.tree(shapes.benchmark_cases()[name])
    q, k, v = make_inputs(tree, 32, 8, 128, torch.bfloat16, 3)
    qd, kd, vd = q.to(device), k.to(device), v.to(device)
    # "wide" without attachments: its private tails are TA_TAIL items whose fused kernel merges
    prepared = prepare(schedule(tree, method="cube", model=MI355X_LIKE), qd, attach_tails=name != "wide")
    a = attention(qd, kd, vd, prepared).clone()
    kp, vp = pack_kv(kd, vd)
    b = attention_matrix(qd, kp, vp, prepared).clone()
    assert (prepared.abi.n_items[_native.TA_TAIL] > 0) == (name == "wide")
    prepared.out.zero_()
    for kind in range(_native.TA_NKINDS):
        segment(qd, kp, vp, prepared, kind)
    c = merge(prepared).clone()
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    if prepared.abi.n_rest == 0:
        # the fused path on its own: partial-producing kinds, then the tail items merge
        prepared.out.zero_()
        for kind in (_native.TA_LARGE256, _native.TA_LARGE128, _native.TA_LARGE64, _native.TA_SMALL):
            segment(qd, kp, vp, prepared, kind)
        d = tail_merge(qd, kp, vp, prepared).clone()
        torch.cuda.synchronize()
        assert torch.equal(b, d)
    # the unfused order merges in another order: equal up to rounding
    assert relative_l2(b.cpu(), c.cpu().float()) < 5e-4


@pytest.mark.parametrize("name,dtype,pad", [("deep", torch.bfloat16, 0), ("wide", torch.float16, 0),
                                            ("unequal", torch.bfloat16, 3)])
def test_raw_segment_and_merge_entry_points(name, dtype, pad, device):
    """The raw C-ABI entry points as a C or ctypes caller of the reference's _segment and
    _merge (kernels.py:8-83, launched at :158-167) binds them: ta_segment once per work-item
    kind with plain device pointers and sizes from a prepared plan, then ta_merge over every
    request's slot list, against the FP32 oracle.  No attachments (ta_segment takes no
    attachment records); pad 3 gives a pool capacity that is not a multiple of 8."""
    tree = shapes.tree(shapes.benchmark_cases()[name])
    q, k, v = make_inputs(tree, 32, 8, 128, dtype, 17, tcap=tree.storage_tokens + pad)
    ref = oracle_fp32(q, k, v, tree)
    qd = q.to(device)
    kp, vp = pack_kv(k.to(device), v.to(device))
    prepared = prepare(schedule(tree, method="cube", model=MI355X_LIKE), qd, attach_tails=False)
    abi = prepared.abi
    lib = _native.load()
    stream = torch.cuda.current_stream().cuda_stream
    tcap = kp.shape[2]
    prepared.part.zero_()
    kinds = [kind for kind in range(_native.TA_NKINDS) if abi.n_items[kind]]
    say("raw", name, dtype, pad, "kinds", kinds)
    for kind in kinds:
        _native.check(lib.ta_segment(qd.data_ptr(), kp.data_ptr(), vp.data_ptr(), abi.qids, abi.kstart, abi.qlen,
                                     abi.klen, abi.rowbase, abi.items[kind], abi.n_items[kind], kind, abi.part,
                                     abi.lse, abi.nreq, abi.hq, abi.hk, abi.d, tcap, abi.maxr, abi.dtype, stream))
    out = torch.full_like(qd, float("nan"))
    _native.check(lib.ta_merge(abi.part, abi.lse, abi.slots, abi.counts, out.data_ptr(), abi.nreq, abi.hq, abi.d,
                               abi.maxs, abi.dtype, stream))
    torch.cuda.synchronize()
    check(out, ref, 0.008, 0.03, f"raw ta_segment + ta_merge {name}")
    # the plan-level layer merges in another order: equal up to rounding
    b = attention_matrix(qd, kp, vp, prepared).clone()
    torch.cuda.synchronize()
    assert relative_l2(out.cpu().float(), b.cpu().float()) < 5e-4
    # a plan's work items of one kind cover the job rows once: ta_segment twice gives the same partials
    if kinds:
        before = prepared.part.clone()
        kind = kinds[0]
        _native.check(lib.ta_segment(qd.data_ptr(), kp.data_ptr(), vp.data_ptr(), abi.qids, abi.kstart, abi.qlen,
                                     abi.klen, abi.rowbase, abi.items[kind], abi.n_items[kind], kind, abi.part,
                                     abi.lse, abi.nreq, abi.hq, abi.hk, abi.d, tcap, abi.maxr, abi.dtype, stream))
        torch.cuda.synchronize()
        assert torch.equal(prepared.part, before)


@pytest.mark.parametrize("hq,hk,d,dtype,pad", [(32, 8, 128, torch.bfloat16, 0), (32, 4, 64, torch.float16, 8),
                                                (32, 2, 32, torch.bfloat16, 0), (32, 8, 128, torch.bfloat16, 3)])
def test_attached_tails(hq, hk, d, dtype, pad, device):
    """Private tails folded into 256-row root items: ragged lengths (1..200 tokens, unaligned
    starts, several tiles), several per item, GQA groups 4/8/16; equal to the oracle, to the
    unattached plan, and to the explicit segment + merge launches.  pad 3 (pool capacity not a
    multiple of 8) runs the unattached variant on the register-staged kernels."""
    group = hq // hk
    nreq, root = {4: (96, 3001), 8: (48, 6001), 16: (24, 12001)}[group]
    tails = [1 + (37 * r) % 200 for r in range(nreq)]
    tree = shapes.tree(shapes.shared_prefix(nreq, root, tails))
    q, k, v = make_inputs(tree, hq, hk, d, dtype, 31 + group, tcap=tree.storage_tokens + pad)
    ref = oracle_fp32(q, k, v, tree)
    qd = q.to(device)
    kp, vp = pack_kv(k.to(device), v.to(device))
    plan = schedule(tree, hq, hk, d, "cube", MI355X_LIKE)
    p1 = prepare(plan, qd)
    assert p1.attached, "the shape must attach tails"
    assert any(len(job.tokens) > 64 for segs in p1.attached.values() for job, _ in segs)
    assert group != 4 or max(len(v) for v in p1.attached.values()) >= 2
    say("attached", hq, hk, d, dtype, pad, len(p1.attached), p1.small_jobs)
    a = attention_matrix(qd, kp, vp, p1).clone()
    p2 = prepare(plan, qd, attach_tails=False)
    b = attention_matrix(qd, kp, vp, p2).clone()
    p1.out.zero_()
    for kind in range(_native.TA_NKINDS):
        segment(qd, kp, vp, p1, kind)
    c = merge(p1, kp).clone()
    torch.cuda.synchronize()
    check(a, ref, 0.008, 0.03, "attached")
    check(b, ref, 0.008, 0.03, "unattached")
    check(c, ref, 0.008, 0.03, "attached/segment+merge")


def test_large_jobs_over_scattered_requests(device):
    """256-row work items over requests that are not consecutive (the qids lookup) beside
    consecutive ones (Q addressed from the first request id), with private tails."""
    n = 160
    jobs = [Job(tuple(range(0, n, 2)), tuple(range(0, 700))),     # even requests: 320 rows, qbase -1
            Job(tuple(range(1, n, 2)), tuple(range(700, 1300))),  # odd requests
            Job(tuple(range(0, 80)), tuple(range(1300, 1555)))]   # consecutive: qbase 0
    jobs += [Job((r,), tuple(range(1560 + 9 * r, 1560 + 9 * r + 1 + r % 9))) for r in range(n)]
    paths = [[] for _ in range(n)]
    for job in jobs:
        for r in job.requests:
            paths[r].extend(job.tokens)
    tree = _Paths([tuple(p) for p in paths])
    g = torch.Generator().manual_seed(41)
    q = torch.randn(n, 32, 128, generator=g).bfloat16()
    k = torch.randn(1560 + 9 * n + 8, 8, 128, generator=g).bfloat16()
    v = torch.randn(1560 + 9 * n + 8, 8, 128, generator=g).bfloat16()
    qd = q.to(device)
    kp, vp = pack_kv(k.to(device), v.to(device))
    prepared = prepare(Plan(jobs, "x", 0.0, dict(kvheads=8)), qd)
    base = prepared.qbase_host
    assert -1 in base and 0 in base
    assert prepared.abi.n_items[_native.TA_LARGE256] > 0 and prepared.attached
    out = attention_matrix(qd, kp, vp, prepared)
    torch.cuda.synchronize()
    check(out, oracle_fp32(q, k, v, tree), 0.008, 0.03, "scattered")


def test_affine_slot_merge_equals_slot_lists(device):
    """The merge with computed slots (ta_plan.slot_stride) gives the bits of the merge that
    loads the slot lists, in the layer and through ta_merge_plan / ta_merge."""
    tree = shapes.tree(shapes.headline())
    q, k, v = make_inputs(tree, 32, 8, 128, torch.bfloat16, 29)
    qd = q.to(device)
    kp, vp = pack_kv(k.to(device), v.to(device))
    prepared = prepare(schedule(tree, 32, 8, 128, "cube", CostModel.mi355x()), qd)
    stride = prepared.abi.slot_stride
    assert stride > 0
    with_stride = attention_matrix(qd, kp, vp, prepared).clone()
    merged = merge(prepared).clone()
    prepared.abi.slot_stride = 0
    lists = attention_matrix(qd, kp, vp, prepared).clone()
    merged_lists = merge(prepared).clone()
    prepared.abi.slot_stride = stride
    torch.cuda.synchronize()
    assert torch.equal(with_stride, lists)
    assert torch.equal(merged, merged_lists) and torch.equal(merged, with_stride)
    check(with_stride.cpu(), oracle_fp32(q, k, v, tree), 0.008, 0.03, "affine slots")


@pytest.mark.parametrize("vscale", [1e5, 1e-5])
def test_partial_rows_keep_range(vscale, device):
    """Partial rows are fp16 scaled by 2^-e per row: V far outside fp16's range
    (or deep in its subnormals) still merges to the FP32 result."""
    tree = shapes.tree(shapes.benchmark_cases()["wide"])
    q, k, v = make_inputs(tree, 32, 8, 128, torch.bfloat16, 23)
    v = (v.float() * vscale).bfloat16()
    ref = oracle_fp32(q, k, v, tree)
    for method in ("cube", "request"):
        out = run(tree, method, MI355X_LIKE, q, k, v, device, (32, 8, 128))
        err = relative_l2(out.cpu(), ref)
        assert torch.isfinite(out).all() and err <= REL_L2, (method, err)


class _Paths:
    def __init__(self, paths):
        self.paths = paths


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_tail_items_with_merge_rest(dtype, device):
    """Requests merged by their TA_TAIL item next to requests left to the merge kernel."""
    jobs = [Job(tuple(range(6)), tuple(range(0, 300))),       # 24 rows: large, all requests
            Job((0,), tuple(range(300, 364))),                 # request 0: one tail (fused merge)
            Job((1,), tuple(range(370, 380))), Job((1,), tuple(range(450, 520))),  # two small jobs
            Job((2, 3), tuple(range(380, 400))),               # 2 and 3 share a small job
            Job((5,), tuple(range(400, 401))),                 # request 5: a one-token tail
            Job((4, 5), tuple(range(401, 450)))]               # ... and a large-free shared job
    paths = [[] for _ in range(6)]
    for job in jobs:
        for r in job.requests:
            paths[r].extend(job.tokens)
    tree = _Paths([tuple(p) for p in paths])
    g = torch.Generator().manual_seed(17)
    q = torch.randn(6, 16, 128, generator=g).to(dtype)
    k = torch.randn(528, 4, 128, generator=g).to(dtype)
    v = torch.randn(528, 4, 128, generator=g).to(dtype)
    qd = q.to(device)
    kp, vp = pack_kv(k.to(device), v.to(device))
    prepared = prepare(Plan(jobs, "x", 0.0, dict(kvheads=4)), qd, route_items=0)  # the large job stays large
    tails = {prepared.jobs[j].requests for j, _, _ in prepared.items[_native.TA_TAIL].view(-1, 3).tolist()}
    assert tails == {(0,)} and prepared.rest.tolist() == [1, 2, 3, 4, 5]
    out = attention_matrix(qd, kp, vp, prepared)
    torch.cuda.synchronize()
    check(out, oracle_fp32(q, k, v, tree), 0.006, 0.02, "tail+rest")


@pytest.mark.parametrize("model_name", ["reference", "mi355x"])
def test_cached_decode_plan_steps(model_name, device):
    """scripts/benchmark_decode_plan.py protocol: 32 req, 1024 + 64 prompt, growing tails, check steps,
    planned under the reference's cost model and the fitted one (whose 32-request root runs as
    64-row request groups beside the tails' small items, prepare's fill rule)."""
    model = CostModel() if model_name == "reference" else CostModel.mi355x()
    base = shapes.tree(shapes.shared_prefix(32, 1024, 64))
    prefix = base.storage_tokens
    steps = 16
    g = torch.Generator().manual_seed(301)
    q = torch.randn(32, 32, 128, generator=g).bfloat16()
    k = torch.randn(prefix + 32 * steps, 8, 128, generator=g).bfloat16()
    v = torch.randn(prefix + 32 * steps, 8, 128, generator=g).bfloat16()
    qd = q.to(device)
    kp, vp = pack_kv(k.to(device), v.to(device))
    for method in ("fixed", "cube"):
        cached = CachedDecodePlan(schedule(base, method=method, model=model), qd, prefix, steps)
        if method == "cube":
            assert cached.prepared.abi.n_items[_native.TA_LARGE64] > 0 and not cached.prepared.attached
        for step in (0, 7, steps - 1):
            say("decode", model_name, method, step)
            out = attention_matrix(qd, kp, vp, cached.update(step + 1)).cpu()
            paths = [p + tuple(prefix + r * steps + t for t in range(step + 1)) for r, p in enumerate(base.paths)]
            ref = oracle_fp32(q, k, v, KVTree([], paths))
            check(out, ref, 0.008, 0.03, f"decode/{method}/{step}")
        # zero generated tokens: tails contribute nothing (reference leaves this undefined)
        out = attention_matrix(qd, kp, vp, cached.update(0)).cpu()
        check(out, oracle_fp32(q, k, v, base), 0.008, 0.03, f"decode/{method}/empty-tail")


def test_large_items_in_one_round(device):
    """32 requests over a 4096-token context, 99 % shared in three levels: the large re-cut takes
    one round of longer chunks (192 64-row items instead of 272) under the fitted model; the
    layer matches the oracle, as the same plan with the shorter cut does."""
    tree = shapes.tree(shapes.grid_tree(32, 4096, 0.99, 3))
    q, k, v = make_inputs(tree, 32, 8, 128, torch.bfloat16, 47)
    qd = q.to(device)
    kp, vp = pack_kv(k.to(device), v.to(device))
    plan = schedule(tree, 32, 8, 128, "cube", CostModel.mi355x())
    prepared = prepare(plan, qd)
    assert prepared.abi.n_items[_native.TA_LARGE64] == 192
    out = attention_matrix(qd, kp, vp, prepared)
    torch.cuda.synchronize()
    check(out, oracle_fp32(q, k, v, tree), 0.008, 0.03, "one round")


@pytest.mark.parametrize("model_name", ["mi355x", "mi355x-like"])
def test_attached_growing_tails(model_name, device):
    """The decode-plan protocol's form with a 2048-token root (32 requests, 2048 + 64 prompt,
    16 reserved tail tokens each), whose 256-row root items fill the GPU, so that the private
    and growing tails attach to them: the layer is one segment launch plus the merge, and each
    step's tail length is read from the attachment records that update() rewrites.  (The
    protocol's own 1024-token root runs as 64-row groups, see test_prepare.)  Steps 0, 1, 8
    and 16 against the oracle."""
    base = shapes.tree(shapes.shared_prefix(32, 2048, 64))
    prefix = base.storage_tokens
    steps = 16
    g = torch.Generator().manual_seed(307)
    q = torch.randn(32, 32, 128, generator=g).bfloat16()
    k = torch.randn(prefix + 32 * steps, 8, 128, generator=g).bfloat16()
    v = torch.randn(prefix + 32 * steps, 8, 128, generator=g).bfloat16()
    qd = q.to(device)
    kp, vp = pack_kv(k.to(device), v.to(device))
    model = CostModel.mi355x() if model_name == "mi355x" else MI355X_LIKE
    cached = CachedDecodePlan(schedule(base, 32, 8, 128, "cube", model), qd, prefix, steps)
    p = cached.prepared
    grown = [job for segs in p.attached.values() for job, _ in segs if job.tokens[0] >= prefix]
    assert len(grown) == 32 and not [j for j in p.jobs if j.tokens[0] >= prefix]
    assert p.abi.n_items[_native.TA_SMALL] == 0 and p.abi.n_items[_native.TA_TAIL] == 0
    for step in (0, 1, 8, 16, 3):
        say("attached growing tails", model_name, step)
        out = attention_matrix(qd, kp, vp, cached.update(step)).cpu()
        paths = [p_ + tuple(prefix + r * steps + t for t in range(step)) for r, p_ in enumerate(base.paths)]
        ref = oracle_fp32(q, k, v, KVTree([], paths))
        check(out, ref, 0.008, 0.03, f"attached-growing/{model_name}/{step}")


def test_reuse_across_calls_and_streams(device):
    """prepared.out is overwritten per call; launches follow torch's current stream."""
    tree = shapes.tree(shapes.benchmark_cases()["wide"])
    q, k, v = make_inputs(tree, 32, 8, 128, torch.bfloat16, 1)
    q2 = torch.flip(q, [0]).contiguous()
    qd, q2d = q.to(device), q2.to(device)
    kp, vp = pack_kv(k.to(device), v.to(device))
    prepared = prepare(schedule(tree, method="cube"), qd)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        out1 = attention_matrix(qd, kp, vp, prepared).clone()
        out2 = attention_matrix(q2d, kp, vp, prepared).clone()
    s.synchronize()
    check(out1, oracle_fp32(q, k, v, tree), 0.008, 0.03, "stream/1")
    check(out2, oracle_fp32(q2, k, v, tree), 0.008, 0.03, "stream/2")


def test_full_size_properties(device):
    """Headline size: equal keys give the path mean of V; permuting requests permutes outputs."""
    tree = shapes.tree(shapes.headline())
    g = torch.Generator().manual_seed(4)
    t = tree.storage_tokens
    q = torch.randn(128, 32, 128, generator=g).bfloat16()
    k = torch.ones(t, 8, 128).bfloat16()
    v = torch.randn(t, 8, 128, generator=g).bfloat16()
    qd = q.to(device)
    kp, vp = pack_kv(k.to(device), v.to(device))
    prepared = prepare(schedule(tree, 32, 8, 128, "cube", MI355X_LIKE), qd)
    out = attention_matrix(qd, kp, vp, prepared).float().cpu()
    vf = v.float()
    root_sum = vf[:8128].sum(0)
    for r in (0, 63, 127):
        mean = (root_sum + vf[8128 + 64 * r: 8128 + 64 * (r + 1)].sum(0)) / 8192
        torch.testing.assert_close(out[r], mean.repeat_interleave(4, 0), atol=4e-3, rtol=0.02)
    # request permutation equivariance (the tree is symmetric in its requests)
    perm = torch.randperm(128, generator=g)
    k2 = torch.randn(t, 8, 128, generator=g).bfloat16()
    kp2, _ = pack_kv(k2.to(device), v.to(device))
    a = attention_matrix(qd, kp2, vp, prepared).clone()
    # swapping request r's query with request perm[r] and its private KV rows with perm[r]'s
    idx = torch.arange(t)
    for r in range(128):
        idx[8128 + 64 * r: 8128 + 64 * (r + 1)] = torch.arange(8128 + 64 * perm[r], 8128 + 64 * (perm[r] + 1))
    kp3, vp3 = pack_kv(k2[idx].to(device), v[idx].to(device))
    b = attention_matrix(q[perm].contiguous().to(device), kp3, vp3, prepared).clone()
    torch.cuda.synchronize()
    # each private tail is attended inside the root chunk item its request index selects, so a
    # permuted request's tail joins another chunk's fp16 partial: equal up to partial rounding
    # (an indexing mistake gives O(1) differences)
    assert relative_l2(b.cpu(), a[perm.to(device)].cpu()) < 2e-3
    plain = prepare(schedule(tree, 32, 8, 128, "cube", MI355X_LIKE), qd, attach_tails=False)
    a = attention_matrix(qd, kp2, vp, plain).clone()
    b = attention_matrix(q[perm].contiguous().to(device), kp3, vp3, plain).clone()
    torch.cuda.synchronize()
    assert relative_l2(b.cpu(), a[perm.to(device)].cpu()) < 1e-6  # symmetric work split: exact


def test_bad_inputs_raise(device):
    tree = shapes.tree(shapes.benchmark_cases()["wide"])
    q, k, v = make_inputs(tree, 32, 8, 128, torch.bfloat16, 1)
    qd = q.to(device)
    kp, vp = pack_kv(k.to(device), v.to(device))
    prepared = prepare(schedule(tree, method="cube"), qd)
    with pytest.raises(ValueError):
        attention_matrix(qd.half(), kp, vp, prepared)
    with pytest.raises(ValueError):
        attention_matrix(qd[:3], kp, vp, prepared)
    with pytest.raises(ValueError):
        attention_matrix(qd, kp.transpose(1, 2), vp, prepared)
    lib = _native.load()
    bad = ctypes.c_void_p(qd.data_ptr() + 2)
    rc = lib.ta_attention_matrix(bad, kp.data_ptr(), vp.data_ptr(), kp.shape[2], ctypes.byref(prepared.abi),
                                 prepared.out.data_ptr(), None)
    assert rc == 1002


def test_graph_replay_matches_eager(device):
    """A captured layer replays to the eager result every time, with eager work in between."""
    tree = shapes.tree(shapes.benchmark_cases()["unequal"])
    q, k, v = make_inputs(tree, 32, 8, 128, torch.bfloat16, 12)
    qd = q.to(device)
    kp, vp = pack_kv(k.to(device), v.to(device))
    prepared = prepare(schedule(tree, method="cube"), qd)
    eager = attention_matrix(qd, kp, vp, prepared).clone()
    stream = torch.cuda.current_stream()
    side = torch.cuda.Stream()
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        attention_matrix(qd, kp, vp, prepared)
    stream.wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        captured = attention_matrix(qd, kp, vp, prepared).clone()
    for rep in range(4):
        prepared.out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, eager), rep
        other = attention_matrix(torch.flip(qd, [0]).contiguous(), kp, vp, prepared).clone()
        torch.cuda.synchronize()
        assert not torch.equal(other, eager)


@pytest.mark.parametrize("d,dtype", [(128, torch.bfloat16), (64, torch.float16), (32, torch.bfloat16)])
def test_mixed_kinds_launch_equals_kind_by_kind(d, dtype, device):
    """A layer with 256-row, 64-row and small work items runs them in one launch
    (seg_mix_kernel): the output has the bits of the kinds launched one after another
    (ta_segment_plan per kind, then the merge) and matches the oracle."""
    n = 96
    jobs = [Job(tuple(range(64)), tuple(range(0, 300))),            # 256 rows: TA_LARGE256
            Job(tuple(range(64, 80)), tuple(range(300, 500)))]      # 64 rows: TA_LARGE64
    # two private runs per request (apart, so that neither is a merging tail): small jobs
    jobs += [Job((r,), tuple(range(500 + 60 * r + o, 525 + 60 * r + o))) for r in range(80) for o in (0, 30)]
    jobs += [Job((r,), tuple(range(5300 + 20 * (r - 80), 5320 + 20 * (r - 80)))) for r in range(80, n)]
    jobs += [Job((r,), tuple(range(5700 + 20 * (r - 80), 5710 + 20 * (r - 80)))) for r in range(80, n)]
    paths = [[] for _ in range(n)]
    for job in jobs:
        for r in job.requests:
            paths[r].extend(job.tokens)
    tree = _Paths([tuple(p) for p in paths])
    g = torch.Generator().manual_seed(d)
    q = torch.randn(n, 32, d, generator=g).to(dtype)
    k = torch.randn(6024, 8, d, generator=g).to(dtype)
    v = torch.randn(6024, 8, d, generator=g).to(dtype)
    qd = q.to(device)
    kp, vp = pack_kv(k.to(device), v.to(device))
    # no routing and no attachment: every kind keeps its items (the grid and nested-tree
    # tests run the mixed launch with attached segments)
    prepared = prepare(Plan(jobs, "x", 0.0, dict(kvheads=8)), qd, route_items=0, attach_tails=False)
    kinds = [kd for kd in (_native.TA_LARGE256, _native.TA_LARGE64, _native.TA_SMALL) if prepared.abi.n_items[kd] > 0]
    say("mixed kinds", d, dtype, list(prepared.abi.n_items))
    assert len(kinds) == 3 and prepared.abi.n_items[_native.TA_TAIL] == 0 and prepared.abi.n_items[_native.TA_LARGE128] == 0
    a = attention_matrix(qd, kp, vp, prepared).clone()
    prepared.out.zero_()
    for kd in kinds:
        segment(qd, kp, vp, prepared, kd)
    b = merge(prepared, kp).clone()
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    check(a, oracle_fp32(q, k, v, tree), 0.008, 0.03, f"mixed/{d}")


def _rotate_half(x):
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hq,hk,d,shared_rope", [(32, 8, 128, False), (16, 2, 64, True), (8, 8, 32, False)])
def test_decode_append_matches_eager_ops(hq, hk, d, shared_rope, dtype, device):
    """The fused decode glue equals the eager RoPE + index_copy_ + contiguous of the adapter
    (reference qwen.py:86-91) bit for bit; slots outside the pool write nothing."""
    g = torch.Generator().manual_seed(hq + d)
    nreq, tcap = 24, 200
    q = torch.randn(nreq, 1, hq, d, generator=g).to(dtype).to(device)
    k = torch.randn(nreq, 1, hk, d, generator=g).to(dtype).to(device)
    v = torch.randn(nreq, 1, hk, d, generator=g).to(dtype).to(device)
    pos = torch.arange(nreq, dtype=torch.float32)[:, None] * 7 + 3
    inv = 1.0 / (1e6 ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    emb = torch.cat([pos * inv, pos * inv], dim=-1)[:, None, :]  # [R, 1, D]
    if shared_rope:
        emb = emb[:1]
    cos, sin = emb.cos().to(dtype).to(device), emb.sin().to(dtype).to(device)
    slots = torch.randperm(tcap, generator=g)[:nreq].to(torch.int32)
    slots[0] = tcap - 1
    slots[1] = tcap + 5  # outside the pool: no write
    kp0 = torch.randn(hk, d, tcap, generator=g).to(dtype).to(device)
    vp0 = torch.randn(hk, tcap, d, generator=g).to(dtype).to(device)
    # eager ops, as the unfused adapter runs them
    qt, kt = q.transpose(1, 2), k.transpose(1, 2)
    c, s_ = cos[:, None], sin[:, None]
    q_ref = (qt * c) + (_rotate_half(qt) * s_)
    k_ref = (kt * c) + (_rotate_half(kt) * s_)
    kp_ref, vp_ref = kp0.clone(), vp0.clone()
    ok = slots < tcap
    idx = slots[ok].long().to(device)
    kp_ref.index_copy_(2, idx, k_ref[ok.to(device), :, 0, :].permute(1, 2, 0))
    vp_ref.index_copy_(1, idx, v.transpose(1, 2)[ok.to(device), :, 0, :].permute(1, 0, 2))
    kp, vp = kp0.clone(), vp0.clone()
    out = decode_append(q, k, v, cos, sin, slots.to(device), kp, vp)
    torch.cuda.synchronize()
    assert torch.equal(out, q_ref[:, :, 0, :].contiguous())
    assert torch.equal(kp, kp_ref) and torch.equal(vp, vp_ref)


@pytest.mark.gpu
@pytest.mark.parametrize("blocks", [1, 7, 256])
def test_read_stream_reads_every_byte(blocks, device):
    """ta_read_stream (the read ceiling of the memory-bound kinds) folds every 16-byte chunk
    exactly once: the XOR of its per-wave words equals the XOR of all words of the buffer."""
    lib = _native.load()
    g = torch.Generator().manual_seed(3)
    words = torch.randint(-2**31, 2**31 - 1, ((1 << 18) + 4 * 37,), generator=g, dtype=torch.int64).to(torch.int32)
    src = words.to(device)
    sink = torch.zeros(4 * blocks, dtype=torch.int32, device=device)
    _native.check(lib.ta_read_stream(src.data_ptr(), src.numel() * 4, sink.data_ptr(), blocks,
                                     torch.cuda.current_stream().cuda_stream))
    folded = int(np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32)))
    assert folded == int(np.bitwise_xor.reduce(words.numpy().view(np.uint32)))
    assert lib.ta_read_stream(src.data_ptr(), 12, sink.data_ptr(), blocks, None) == _native.TA_ERR_ARG
