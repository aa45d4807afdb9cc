"""Execution backend: plan lowering plus the HIP segment / merge kernels.

Drop-in for the reference's ``src/tree_attention/kernels.py``: ``PreparedPlan``
(:86-100), ``prepare`` (:103-141), ``pack_kv`` (:144-145), ``attention``
(:148-149), ``attention_matrix`` (:152-168) and ``CachedDecodePlan``
(:171-186) keep their names, arguments and results.  The Triton kernels are
replaced by the gfx950 library ``libtree_attn.so`` (include/tree_attn.h),
called through ctypes on torch's current HIP stream.  There is no CPU or
PyTorch fallback: without the library every call raises ``RuntimeError``.

Internal layout (the build's own; only ``out`` is contractual):

* ``qids [J, MAXR]``, ``kids [J, 1]`` (first physical token), ``qlen [J]``,
  ``klen [J]`` as in the reference (kernels.py:114-128), over execution jobs:
  the plan's physical jobs, small ones (<= 16 query rows) first as in the
  reference (kernels.py:109-110), with runs of jobs over one request group
  re-cut into chunks sized for the GPU (``_recut``).
* Partial outputs are compact: job ``j``'s requests own partial rows
  ``rowbase[j] .. rowbase[j] + qlen[j]`` of ``part [NSLOT, HQ, D]`` and
  ``lse [NSLOT, HQ]``; ``slots[r]`` lists request ``r``'s partial rows in job
  order (the reference instead indexes ``job * MAXR + local``, which allocates
  ``J * MAXR`` rows).
* Work items are ``(job, first row, KV head)`` triples: small jobs (<= 16
  query rows) get one per KV head, processed by one wave each; larger jobs
  are cut into 64/128/256-row tiles, one workgroup per (job, tile, KV head).
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass, field
from itertools import chain

import numpy as np
import torch

from . import _native
from .schedule import Job, Plan, physical_jobs
from .tree import id_run

_DTYPES = {torch.bfloat16: _native.TA_BF16, torch.float16: _native.TA_FP16}
SMALL_ROWS = 16  # rows of one MFMA block; same threshold as kernels.py:109-110


def _large_kind(rows: int, tile_rows: int = 256) -> int:
    """Row-tile kernel for a job with ``rows`` query rows (tiles of at most ``tile_rows``).

    Jobs of more than 64 rows take 256-row items (the pipelined kernel, which
    also attends attached private segments) unless ``tile_rows`` caps the tile
    at 128 rows.
    """
    if rows <= 64 or tile_rows <= 64:
        return _native.TA_LARGE64
    if tile_rows <= 128:
        return _native.TA_LARGE128
    return _native.TA_LARGE256


@dataclass
class PreparedPlan:
    """Device metadata and reusable scratch of one plan (reference kernels.py:86-100)."""
    jobs: list
    small_jobs: int
    contiguous_k: bool
    contiguous_q: bool
    qids: torch.Tensor
    kids: torch.Tensor
    qlen: torch.Tensor
    klen: torch.Tensor
    slots: torch.Tensor
    counts: torch.Tensor
    part: torch.Tensor
    lse: torch.Tensor
    out: torch.Tensor
    rowbase: torch.Tensor | None = None
    items: dict = field(default_factory=dict)
    abi: _native.TaPlan | None = None
    metadata: torch.Tensor | None = None
    rest: torch.Tensor | None = None  # requests the merge kernel covers (no TA_TAIL job)
    # private segments folded into TA_LARGE256 work items: {(job, first row): [(Job, first job row)]}
    attached: dict = field(default_factory=dict)
    xtail: torch.Tensor | None = None
    plan: Plan | None = None
    options: dict = field(default_factory=dict)  # prepare's tile_rows / fixed_from
    growing_len: int | None = None  # last CachedDecodePlan.update length of the growing jobs
    qbase_host: list = field(default_factory=list)  # per job: first request if consecutive, else -1
    _unattached: "PreparedPlan | None" = None
    # positions in ``metadata`` of every growing tail's length: klen of the growing
    # jobs, the token field of the records of the items the attached ones joined
    grow_offsets: torch.Tensor | None = None

    def fill_growing(self, length: int) -> None:
        """Set the length of every growing tail (tokens from ``fixed_from`` on) to
        ``length``, here and in the unattached variant (device-side, no sync)."""
        if self.grow_offsets is not None:
            self.metadata.index_fill_(0, self.grow_offsets, length)
        self.growing_len = length
        if self._unattached is not None:
            self._unattached.fill_growing(length)

    def for_pools(self, kp: torch.Tensor) -> "PreparedPlan":
        """The plan to launch on pools like ``kp``: this one, or, when it has
        attached segments and the pool capacity is not a multiple of 8 (the
        register-staged kernels, which take no attachments), the same plan
        prepared without attachments, writing into the same ``out``."""
        if not self.attached or kp.shape[-1] % 8 == 0:
            return self
        if self._unattached is None:
            alt = prepare(self.plan, self.out, attach_tails=False, **self.options)
            alt.out = self.out
            if self.growing_len is not None:
                alt.fill_growing(self.growing_len)
            self._unattached = alt
        return self._unattached


def _tail_jobs(jobs, small_jobs):
    """Indices of the small jobs that are the only small job of their one request.

    Their work items (kind TA_TAIL) also merge that request's partials, so the
    merge kernel covers only the other requests.
    """
    owners = {}
    for j in range(small_jobs):
        for r in jobs[j].requests:
            owners[r] = owners.get(r, 0) + 1
    return {j for j in range(small_jobs) if len(jobs[j].requests) == 1 and owners[jobs[j].requests[0]] == 1}


def _build_items(jobs, small_jobs, group, kvheads, tile_rows=256, tails=frozenset()):
    """Work-item triples ``(job, first row, KV head)`` per kernel kind as int32 arrays.

    Small jobs (<= 16 query rows) get one item per KV head, of kind TA_TAIL for
    the jobs in ``tails`` and TA_SMALL otherwise; larger jobs one per (row
    tile, KV head), the tile size chosen by ``_large_kind``; TA_LARGE256 items
    are ordered by KV head, then job, then first row.
    """
    def triples(job, row0, head):
        return np.stack([job, row0, head], axis=1).astype(np.int32).reshape(-1)

    heads = np.arange(kvheads)
    out = {}
    small = np.arange(small_jobs)
    is_tail = np.isin(small, np.fromiter(tails, dtype=np.int64, count=len(tails)))
    for kind, sel in ((_native.TA_SMALL, ~is_tail), (_native.TA_TAIL, is_tail)):
        js = small[sel]  # one item per (job, KV head), job-major
        out[kind] = triples(np.repeat(js, kvheads), np.zeros(js.size * kvheads, dtype=np.int64),
                            np.tile(heads, js.size))
    big = np.arange(small_jobs, len(jobs))
    rows = np.fromiter((len(jobs[j].requests) * group for j in big), dtype=np.int64, count=big.size)
    kinds = np.where((rows <= 64) | (tile_rows <= 64), _native.TA_LARGE64,
                     _native.TA_LARGE128 if tile_rows <= 128 else _native.TA_LARGE256)
    for kind, tile in _native.KIND_ROWS.items():
        js = big[kinds == kind]
        ntile = -(-rows[kinds == kind] // tile)
        if kind == _native.TA_LARGE256:
            # The 256-row kernel gives each XCD a contiguous range of items: in
            # head-major order an XCD works on one KV head, so its L2 holds that
            # head's Q rows and K/V.  Order: head, job, first row.
            n = int(ntile.sum())
            within = np.arange(n) - np.repeat(np.cumsum(ntile) - ntile, ntile)
            job = np.tile(np.repeat(js, ntile), kvheads)
            first = np.tile(within * tile, kvheads)
            head = np.repeat(heads, n)
        else:  # job, head, first row
            per_job = ntile * kvheads
            within = np.arange(int(per_job.sum())) - np.repeat(np.cumsum(per_job) - per_job, per_job)
            nt = np.repeat(ntile, per_job)
            job = np.repeat(js, per_job)
            head = within // np.maximum(nt, 1)
            first = within % np.maximum(nt, 1) * tile
        out[kind] = triples(job, first, head)
    return out


TOKEN_QUANTUM = 64  # tokens per LDS tile of the segment kernels
XTAIL_MAX = 4       # segments one TA_LARGE256 work item takes on (TA_XTAIL_MAX, tree_attn.h)
XTAIL_FIELDS = 4    # per segment: first token, tokens, first job row, rows (TA_XTAIL_STRIDE, tree_attn.h)
WAVE_ROWS = 32      # query rows of one wave of the TA_LARGE256 kernel
# attached tiles an item may take beyond its own count: the one-tile root items of
# decode-sized layers take their requests' private and growing tails
ATTACH_MIN_CAP = 2 * XTAIL_MAX
# large jobs run in the small-job kernel as 16-row request groups when the small-job
# kernel launches anyway and the groups stream at most this many (tile, KV head) work
# units: about 0.4 tile per resident small-job wave (8 per CU), less than the start-up
# of a launch of its own (measured over the 81-shape evaluation grid)
ROUTE_ITEMS = 768
# jobs over one token run execute as one job when together they fill a 256-row work item
FUSE_ROWS = 256
# tails (a request's only small job) stay whole, one merging work item each, when they fill
# the GPU; tails longer than one tile only with four items per CU, since each item streams
# its tail alone (measured on the six benchmark cases and the 81-shape grid: 0.92x over
# the 13 layers it changes, 0.78x at best)
TAIL_KEEP_TILES = 1
TAIL_KEEP_ITEMS_PER_CU = 4
# large chunks are at least this many tiles long when that keeps the lowering's kernel
# kinds and attachments and still gives half a work item per CU: a work item's time is
# mostly its start-up latency, and every chunk is one more partial slot to merge
# (measured: 0.986x on the 81-shape grid, 0.997x on the reference's 81 trees, 0.89x on
# the benchmark case "wide" of 32 requests over 2048 shared tokens)
LARGE_MIN_TILES = 2
# wider large jobs run as 64-row request groups when 64-row items run anyway and no wider
# job exceeds this many rows (prepare's consolidate_rows; 0: never)
CONSOLIDATE_ROWS = 128
# a launch of small-job items alone (2048 one-wave workgroups, 8 per CU) takes two-tile chunks
# instead of one-tile chunks when those would fill at least 45 % of its waves: a wave streams
# the second tile of an item while it computes the first, and every chunk is one more partial
# slot to merge.  Measured on the 81-shape grid, the reference's 81 trees and the calibration
# trees (graph replay): 0.80-0.97x on most of the 70 layers it changes; with fuller thresholds
# of 41-43 % of the waves two layers ran 1.11-1.15x.
SMALL_PAIRS = True


def _tiles(job) -> int:
    """LDS tiles the segment kernels stream for ``job``'s token run."""
    t0 = job.tokens[0]
    return -(-(t0 + len(job.tokens) - (t0 & ~7)) // TOKEN_QUANTUM)


def _attach_tails(small, large, group, tile_rows, is_fixed, min_cap=ATTACH_MIN_CAP):
    """``_attach_tails_py`` through the host library (``tp_attach_tails``) when it is built.
    ``small`` are the candidate jobs (any job whose rows fit one wave).

    Both give the same attachments in the same order.
    """
    from . import _planner
    if not small or not large or not _planner.available():
        return _attach_tails_py(small, large, group, tile_rows, is_fixed, min_cap)
    is256 = [_large_kind(len(j.requests) * group, tile_rows) == _native.TA_LARGE256 for j in large]
    if not any(is256):
        return small, {}
    nreq = 1 + max(max(j.requests) for j in (*large, *small))
    item, lrow, keys = _planner.attach_tails(
        large, small, group, is256, [_tiles(j) for j in large], [_tiles(j) for j in small],
        [bool(is_fixed(j)) for j in small], nreq, XTAIL_MAX, WAVE_ROWS, 256, min_cap)
    attached, left = {}, []
    for job, it, lr in zip(small, item, lrow):
        if it < 0:
            left.append(job)
        else:
            attached.setdefault(keys[it], []).append((job, lr))
    return left, attached


def _attach_tails_py(small, large, group, tile_rows, is_fixed, min_cap=ATTACH_MIN_CAP):
    """Fold jobs whose rows fit one wave into TA_LARGE256 work items of large jobs.

    A candidate job over requests ``r0 .. rn-1`` (a private tail, or a node of
    a few requests) can be attended by any 256-row work item of a large job
    that holds those requests at consecutive rows within one wave: that wave
    attends the job's tokens into the same online-softmax state, so the item's
    partials for ``r0 .. rn-1`` cover the large job's tokens and the job's, and
    the job needs no launch, work item or partial slot of its own.  Each job
    goes to the candidate item with the fewest attached tiles (then the fewest
    on the owning wave, then the first large job), up to ``XTAIL_MAX``
    segments per item and no more attached tiles than the item's own (at least
    ``min_cap``), so the large kernel's items stay balanced.  Jobs for
    which ``is_fixed`` holds are not attached.  A growing decode tail is
    balanced by its reserved length; its record reads the current length on
    the device.

    Returns the candidate jobs left and
    ``{(large job index, first row): [(job, first job row)]}``.
    """
    # the 256-row work items: their key (large job index, first row) and the
    # tiles their own job streams; holders[r]: (job, item, wave, first job row)
    # of every item whose rows include request r's within one wave
    keys, own = [], []
    holders = {}
    for J, job in enumerate(large):
        rows = len(job.requests) * group
        if _large_kind(rows, tile_rows) != _native.TA_LARGE256:
            continue
        first, n = len(keys), _tiles(job)
        for row0 in range(0, rows, 256):
            keys.append((J, row0))
            own.append(n)
        for pos, r in enumerate(job.requests):
            lrow = pos * group
            if lrow % WAVE_ROWS + group <= WAVE_ROWS:
                holders.setdefault(r, []).append((J, first + lrow // 256, lrow % 256 // WAVE_ROWS, lrow))

    def fits(J, lrow, reqs):  # reqs at consecutive rows of one wave of large[J], from lrow on
        held = large[J].requests
        pos = lrow // group
        return (lrow % WAVE_ROWS + len(reqs) * group <= WAVE_ROWS
                and tuple(held[pos:pos + len(reqs)]) == tuple(reqs))
    if not holders:
        return small, {}
    waves = 256 // WAVE_ROWS
    item_tiles, item_segs, wave_tiles = [0] * len(keys), [0] * len(keys), [0] * (len(keys) * waves)
    attached = {}
    left = []
    for job in small:
        cands = holders.get(job.requests[0])
        if not cands or is_fixed(job):
            left.append(job)
            continue
        n = _tiles(job)
        best = None
        for J, item, wave, lrow in cands:
            if len(job.requests) > 1 and not fits(J, lrow, job.requests):
                continue
            t = item_tiles[item]
            if item_segs[item] >= XTAIL_MAX or t + n > max(own[item], min_cap):
                continue
            score = (t, wave_tiles[item * waves + wave], J)
            if best is None or score < best[0]:
                best = (score, item, wave, lrow)
        if best is None:
            left.append(job)
            continue
        _, item, wave, lrow = best
        attached.setdefault(keys[item], []).append((job, lrow))
        item_tiles[item] += n
        item_segs[item] += 1
        wave_tiles[item * waves + wave] += n
    return left, attached


def _fuse_same_tokens(jobs, group, min_rows):
    """Large jobs (more than 16 query rows) over the same token run run as one job over the
    union of their requests when together they hold at least ``min_rows`` query rows and
    share no request.

    Each request keeps one partial over those tokens, so the attention is the same; the K/V
    run is streamed once per 256-row work item instead of once per job.  A plan that splits
    a wide node into request groups (a cost model with 64-row query tiles) then runs the node
    in the 256-row kernel.  Jobs of a few requests -- the per-request plan's among them --
    are left as planned.  The fused job takes the place of the first of its jobs.
    """
    runs = {}
    for j in jobs:
        if len(j.requests) * group > SMALL_ROWS:
            runs.setdefault((j.tokens[0], len(j.tokens)), []).append(j)
    fused = {}
    for key, grp in runs.items():
        if len(grp) < 2:
            continue
        reqs = [r for j in grp for r in j.requests]
        if len(reqs) * group >= min_rows and len(set(reqs)) == len(reqs):
            fused[key] = Job(tuple(sorted(reqs)), grp[0].tokens)
    if not fused:
        return jobs
    out = []
    for j in jobs:
        key = (j.tokens[0], len(j.tokens))
        if key not in fused or len(j.requests) * group <= SMALL_ROWS:
            out.append(j)
        elif fused[key] is not None:
            out.append(fused[key])
            fused[key] = None
    return out


def _recut(jobs, items_per_chunk, target_items, is_fixed, min_tiles=1, floor_items=0, one_round=False,
           pairs=False):
    """Execution jobs for one kernel kind: runs of consecutive jobs over the same
    requests and contiguous tokens are cut again into near-equal chunks, as long
    as possible while the kind still gets ``target_items`` work items (one
    workgroup per CU for the large kinds).  Fewer, longer chunks mean fewer
    partial outputs to write and merge; the result is the same attention.
    Jobs for which ``is_fixed(job)`` holds (growing decode tails, tails that
    merge their request) are left alone.  Chunks are at least ``min_tiles``
    tiles long whenever that still gives ``floor_items`` work items.
    ``one_round``: ``target_items`` items run at once (one per CU), so a cut that
    gives a few more than that runs a second round of items for them; the next
    longer cut, one round of longer chunks, is taken when its chunks are shorter
    than the rounds' chunks end to end.
    ``pairs``: chunks are two tiles long, not one, when one-tile chunks would give at
    least 45 % of ``target_items`` items.
    """
    runs = []  # [requests, first token, length, fixed]
    for job in jobs:
        t0, n = job.tokens[0], len(job.tokens)
        fixed = is_fixed(job)
        last = runs[-1] if runs else None
        if last and not fixed and not last[3] and last[0] == job.requests and last[1] + last[2] == t0:
            last[2] += n
        else:
            runs.append([job.requests, t0, n, fixed])

    weights = [(items_per_chunk(r), n, f) for r, _, n, f in runs]
    fixed_items = sum(w for w, _, f in weights if f)
    cut = [(w, n) for w, n, f in weights if not f]

    def count(limit):  # work items at a chunk limit; non-increasing in limit
        return fixed_items + sum(w * -(-n // limit) for w, n in cut)

    longest = max((n for _, n in cut), default=0)
    if longest == 0:
        return jobs
    # the longest limit (a multiple of TOKEN_QUANTUM, at most the longest run)
    # that still gives target_items, else TOKEN_QUANTUM: binary search over the
    # multiples, count being monotone
    lo, hi = 1, -(-longest // TOKEN_QUANTUM)
    if count(hi * TOKEN_QUANTUM) >= target_items:
        lo = hi
    while hi - lo > 1:  # count(lo) >= target_items or lo == 1; count(hi) < target_items
        mid = (lo + hi) // 2
        if count(mid * TOKEN_QUANTUM) >= target_items:
            lo = mid
        else:
            hi = mid
    if one_round and hi > lo:
        rounds = -(-count(lo * TOKEN_QUANTUM) // target_items)
        if rounds > 1 and hi < rounds * lo:  # count(hi) < target_items: one round
            lo = hi
    if pairs and lo == 1 and hi == 2 and 20 * count(TOKEN_QUANTUM) >= 9 * target_items:
        lo = 2
    if lo < min_tiles and count(min_tiles * TOKEN_QUANTUM) >= floor_items:
        lo = min_tiles
    limit = lo * TOKEN_QUANTUM
    out = []
    # chunks are built field by field (what the frozen dataclass's __init__
    # does) from slices of one id run: this loop makes most of prepare's jobs
    new, put = object.__new__, object.__setattr__
    for reqs, t0, n, fixed in runs:
        ids = id_run(t0, t0 + n)
        if fixed:
            out.append(Job(reqs, ids))
            continue
        pieces = -(-n // limit)
        size = -(-(-(-n // pieces)) // 8) * 8  # near-equal, 8-token aligned
        for a in range(0, n, size):
            job = new(Job)
            put(job, "requests", reqs)
            put(job, "tokens", ids[a:a + size])
            out.append(job)
    return out


def _cu_count(device) -> int:
    if device.type == "cuda":
        return torch.cuda.get_device_properties(device).multi_processor_count
    return 256  # MI355X


def _request_error(jobs, nreq):
    """ValueError naming the first job with a request outside [0, nreq)."""
    for i, job in enumerate(jobs):
        for r in job.requests:
            if not 0 <= r < nreq:
                return ValueError(f"Job {i} names request {r} outside q's {nreq} requests")
    return ValueError("a request is outside q's requests")


def _xtail_record(segs, group):
    """The attachment record of one TA_LARGE256 item: the segment count, then
    (first token, tokens, first job row, rows) of each segment."""
    return [len(segs)] + [x for job, lrow in segs for x in (job.tokens[0], len(job.tokens), lrow,
                                                             len(job.requests) * group)]


def _metadata_sections(njobs, maxr, nreq, maxs, n_rest, n_l256, attached, xstride, n_items):
    """Shapes of the int32 metadata sections, in upload order (tp_build_metadata's order)."""
    return ([(njobs, maxr), (njobs, 1), (njobs,), (njobs,), (nreq, maxs), (nreq,), (njobs,), (n_rest,),
             (n_l256 if attached else 0, xstride), (njobs,)] + [(3 * n_items[k],) for k in range(_native.TA_NKINDS)])


def _metadata_native(jobs, small_jobs, nreq, group, kvheads, tile_rows, attached, xstride):
    """The metadata sections through the host library (``tp_build_metadata``)."""
    from . import _planner
    qlen = np.fromiter((len(j.requests) for j in jobs), dtype=np.int32, count=len(jobs))
    req = np.fromiter(chain.from_iterable(j.requests for j in jobs), dtype=np.int32, count=int(qlen.sum()))
    kstart = np.fromiter((j.tokens[0] for j in jobs), dtype=np.int32, count=len(jobs))
    klen = np.fromiter((len(j.tokens) for j in jobs), dtype=np.int32, count=len(jobs))
    att_job = np.fromiter((j + small_jobs for j, _ in attached), dtype=np.int32, count=len(attached))
    att_row0 = np.fromiter((r0 for _, r0 in attached), dtype=np.int32, count=len(attached))
    att_rec = np.zeros((len(attached), xstride), dtype=np.int32)
    for i, segs in enumerate(attached.values()):
        att_rec[i, :1 + XTAIL_FIELDS * len(segs)] = _xtail_record(segs, group)
    try:
        sizes, buf = _planner.build_metadata(qlen, req, kstart, klen, small_jobs, nreq, group, kvheads, tile_rows,
                                             att_job, att_row0, att_rec, xstride)
    except ValueError:
        raise _request_error(jobs, nreq) from None
    maxr, maxs, nslot, n_rest = sizes[:4]
    n_items = sizes[4:9]
    shapes = _metadata_sections(len(jobs), maxr, nreq, maxs, n_rest, sizes[12], attached, xstride, n_items)
    qbase = buf[-3 * sum(n_items) - len(jobs):len(buf) - 3 * sum(n_items)]
    return {"buf": buf, "shapes": shapes, "maxr": maxr, "maxs": maxs, "nslot": nslot,
            "contiguous_q": bool(sizes[9]), "slot_stride": sizes[10], "qbase": qbase}


def _metadata_numpy(jobs, small_jobs, nreq, group, kvheads, tile_rows, attached, xstride):
    """The metadata sections with numpy (the same arrays as ``_metadata_native``)."""
    njobs = len(jobs)
    qlen = np.fromiter((len(j.requests) for j in jobs), dtype=np.int32, count=njobs)
    klen = np.fromiter((len(j.tokens) for j in jobs), dtype=np.int32, count=njobs)
    kids = np.fromiter((j.tokens[0] for j in jobs), dtype=np.int32, count=njobs).reshape(njobs, 1)
    ends = np.cumsum(qlen)
    rowbase = (ends - qlen).astype(np.int32)  # partial slot of each job's first request
    nslot = int(ends[-1])
    flat = np.fromiter(chain.from_iterable(j.requests for j in jobs), dtype=np.int64, count=nslot)
    if flat.size and (flat.min() < 0 or flat.max() >= nreq):
        raise _request_error(jobs, nreq)
    maxr = int(qlen.max())
    local = np.arange(nslot) - np.repeat(rowbase, qlen)  # request's row within its job
    qids = np.zeros((njobs, maxr), dtype=np.int32)
    qids[np.repeat(np.arange(njobs), qlen), local] = flat
    # each request's slots in job order: slot s holds request flat[s]
    counts = np.bincount(flat, minlength=nreq).astype(np.int32)
    maxs = max(1, int(counts.max()))
    order = np.argsort(flat, kind="stable")
    rank = np.arange(nslot) - np.repeat(np.cumsum(counts) - counts, counts)
    slot_array = np.zeros((nreq, maxs), dtype=np.int32)
    slot_array[flat[order], rank] = order
    tails = _tail_jobs(jobs, small_jobs)
    tail_list = sorted(tails)
    tail_req = np.array([jobs[j].requests[0] for j in tail_list], dtype=np.int64)
    if tail_req.size:
        # A tail job's slot goes last: its work item merges the request's other
        # slots first.  Small jobs come first, so it is the request's first slot.
        rows = slot_array[tail_req]
        assert (rows[:, 0] == rowbase[tail_list]).all()
        c = counts[tail_req][:, None]
        k = np.arange(maxs)[None, :]
        src = np.where(k < c - 1, k + 1, np.where(k == c - 1, 0, k))
        slot_array[tail_req] = np.take_along_axis(rows, src, 1)
    items = _build_items(jobs, small_jobs, group, kvheads, tile_rows, tails)
    rest = np.setdiff1d(np.arange(nreq, dtype=np.int32), tail_req.astype(np.int32))
    # affine slots (slot k of request r is r + k * stride, every request maxs of them):
    # the merge computes them instead of loading counts and slot lists
    slot_stride = 0
    if maxs > 1 and (counts == maxs).all():
        stride = int(slot_array[0, 1] - slot_array[0, 0])
        affine = np.arange(nreq)[:, None] + np.arange(maxs)[None, :] * stride
        if stride > 0 and np.array_equal(slot_array, affine):
            slot_stride = stride
    # attached segments of each TA_LARGE256 item: count, then (first token, tokens, first job row, rows)
    # (one record per (job, first row), shared by the item of every KV head)
    if attached:
        recs = np.zeros((len(attached), xstride), dtype=np.int32)
        codes = np.zeros(len(attached), dtype=np.int64)
        for i, ((j, row0), segs) in enumerate(attached.items()):
            recs[i, :1 + XTAIL_FIELDS * len(segs)] = _xtail_record(segs, group)
            codes[i] = (j + small_jobs) << 32 | row0
        big = items[_native.TA_LARGE256].reshape(-1, 3).astype(np.int64)
        item_codes = big[:, 0] << 32 | big[:, 1]
        order = np.argsort(codes)
        pos = np.minimum(np.searchsorted(codes[order], item_codes), len(codes) - 1)
        hit = codes[order][pos] == item_codes
        xtail = np.zeros((len(big), xstride), dtype=np.int32)
        xtail[hit] = recs[order[pos[hit]]]
    else:
        xtail = np.zeros((0, xstride), dtype=np.int32)

    # first request of each job over consecutive requests, else -1 (kernels.py:23-26, 138)
    breaks = np.zeros(nslot, dtype=np.int64)
    breaks[1:] = np.cumsum(np.diff(flat) != 1)  # steps other than +1 up to each slot
    consecutive = breaks[ends - 1] == breaks[rowbase]
    qbase = np.where(consecutive, flat[rowbase], -1).astype(np.int32)

    contiguous_q = bool((flat[ends - 1] - flat[rowbase] + 1 == qlen).all())
    arrays = ([qids, kids, qlen, klen, slot_array, counts, rowbase, rest, xtail, qbase]
              + [items[k] for k in range(_native.TA_NKINDS)])
    return {"buf": np.concatenate([a.ravel() for a in arrays]).astype(np.int32, copy=False),
            "shapes": [a.shape for a in arrays], "maxr": maxr, "maxs": maxs, "nslot": nslot,
            "contiguous_q": contiguous_q, "slot_stride": slot_stride, "qbase": qbase}


def prepare(plan: Plan, q: torch.Tensor, tile_rows: int = 256, fixed_from: int | None = None,
            attach_tails: bool = True, route_items: int = ROUTE_ITEMS, fuse_rows: int = FUSE_ROWS,
            consolidate_rows: int = CONSOLIDATE_ROWS, large_target: int | None = None,
            small_target: int | None = None, large_min_tiles: int = LARGE_MIN_TILES) -> PreparedPlan:
    """Lower ``plan`` to device metadata and scratch for queries shaped like ``q``.

    Mirrors kernels.py:103-141: physical jobs, stable small-first order, one
    host-to-device copy of all int32 metadata, scratch allocated once.
    ``tile_rows`` (64, 128 or 256) caps the query rows one workgroup of the
    large-job kernels handles; it changes the work split, not the result.
    Large jobs over the same token run that together hold at least ``fuse_rows``
    query rows (0: never) run as one (``_fuse_same_tokens``).  Runs of jobs over one request group are re-cut for the
    GPU (``_recut``), so ``jobs`` holds the execution jobs; ``fixed_from`` keeps jobs whose tokens
    start at or after it (decode tails whose length changes) as they are.
    ``attach_tails`` folds private single-request jobs into the 256-row work
    items of the large jobs holding their request (``_attach_tails``); those
    tails are then in ``attached``, not in ``jobs``.  When small jobs are left for
    the small-job kernel and the large jobs, cut into 16-row request groups, stream
    at most ``route_items`` (tile, KV head) units, the large jobs run as those
    groups in the small-job kernel instead (one segment launch less).
    ``large_target`` and ``small_target`` are the work items the re-cut aims at
    for the large kinds and the small-job kind (default: one and eight per CU);
    a large re-cut that would leave a few items for a second round takes the
    next longer chunks when one round of them is shorter.
    Large chunks of one tile are lengthened to ``large_min_tiles`` tiles when
    that keeps the kernel kinds and the attachments and gives at least half of
    ``large_target`` work items.  Jobs of at most ``consolidate_rows`` rows run
    as 64-row request groups when 64-row items run anyway, or when their
    256-row items would fill only a quarter to a half of the CUs and every
    small job is one tile long (0: never).  Raises
    ``ValueError`` for jobs without requests or tokens, request ids outside
    ``q`` and token runs that are not consecutive physical ids.
    """
    if q.dim() != 3:
        raise ValueError("q must be [requests, query heads, head dim]")
    nreq, hq, dim = q.shape
    kvheads = plan.settings["kvheads"]
    if hq % kvheads:
        raise ValueError("Query heads must be divisible by KV heads")
    group = hq // kvheads
    jobs = physical_jobs(plan.jobs)
    for i, job in enumerate(jobs):
        toks = job.tokens
        if not job.requests or not toks:
            raise ValueError("Every job needs requests and tokens")
        if toks[0] < 0 or (len(toks) > 1 and toks != id_run(toks[0], toks[0] + len(toks))):
            raise ValueError(f"Job {i} tokens are not one run of consecutive physical ids")
    if not jobs:
        raise ValueError("Plan has no jobs")
    if fuse_rows > 0:
        jobs = _fuse_same_tokens(jobs, group, fuse_rows)
    small = [j for j in jobs if len(j.requests) * group <= SMALL_ROWS]
    large = [j for j in jobs if len(j.requests) * group > SMALL_ROWS]
    per = SMALL_ROWS // group
    routed = [Job(j.requests[i:i + per], j.tokens) for j in large for i in range(0, len(j.requests), per)] \
        if per and small and large else []
    small0 = small
    n_cu = _cu_count(q.device)
    large_target = n_cu if large_target is None else large_target
    small_target = 8 * n_cu if small_target is None else small_target

    def growing(job):
        return fixed_from is not None and job.tokens[0] >= fixed_from

    def lower(small, large, min_tiles):
        """Re-cut, order and attach: (small jobs, large jobs, attachments)."""
        large = _recut(large, lambda r: -(-len(r) * group // _native.KIND_ROWS[_large_kind(len(r) * group, tile_rows)])
                       * kvheads, large_target, growing, min_tiles, large_target // 2, one_round=True)
        # chunks of one token range side by side: a root split into request groups then gives
        # request r its k-th slot at r + k * (requests of a chunk), the layout the merge computes
        large.sort(key=lambda j: (j.tokens[0], j.requests[0]))
        attached = {}
        if attach_tails:  # growing tails too: their records' token fields are rewritten by fill_growing
            # candidates: the small jobs, then the large ones whose rows fit one wave
            mids = [j for j in large if len(j.requests) * group <= WAVE_ROWS]
            left, attached = _attach_tails(small + mids, large, group, tile_rows, lambda job: False)
            if any(len(j.requests) * group <= SMALL_ROWS for j in left):
                # the small-job kernel launches anyway: items take no more attached tiles than
                # their own, so that the large kernel does not become the longer of the two
                left, attached = _attach_tails(small + mids, large, group, tile_rows, lambda job: False, 0)
            small = [j for j in left if len(j.requests) * group <= SMALL_ROWS]
            if mids:
                gone = {id(job) for segs in attached.values() for job, _ in segs}
                large = [j for j in large if id(j) not in gone]
        return small, large, attached

    def lowering(min_tiles, fill=None):
        """``lower``, then one large-job kind and routing: (small, large, attachments, fill).

        ``fill``: whether the wider jobs run as 64-row groups to fill the GPU (decided from
        one-tile chunks when None)."""
        small, large, attached = lower(small0, large0, min_tiles)
        # One large-job kind: when 64-row items run anyway and every wider job holds at most
        # consolidate_rows rows, the wider jobs run as 64-row request groups in the same kind
        # (one launch and its start-up less; their K/V is read once per group).
        per64 = 64 // group
        wide = [j for j in large0 if len(j.requests) * group > 64]
        # ... and also when the wider jobs' 256-row items, cut into one-tile chunks, fill more
        # than a quarter but at most half of the CUs and every small job is one tile long (the
        # private suffixes and growing tails of a decode step): two 64-row groups per job read
        # its K/V twice but fill up to all of them, and the one-tile small jobs run beside them
        # instead of in sequence on the 256-row items.  Longer small jobs stay with the
        # 256-row items, whose attachments and single merge they need.
        if fill is None:
            items256 = sum(-(-len(j.requests) * group // 256) for j in large
                           if _large_kind(len(j.requests) * group, tile_rows) == _native.TA_LARGE256) * kvheads
            fill = (min_tiles == 1 and n_cu // 4 < items256 <= n_cu // 2
                    and all(_tiles(j) <= 1 for j in small0))
        if (consolidate_rows and per64 and wide and all(len(j.requests) * group <= consolidate_rows for j in wide)
                and (any(_large_kind(len(j.requests) * group, tile_rows) == _native.TA_LARGE64 for j in large)
                     or fill)):
            split = []
            for j in large0:
                if len(j.requests) * group > 64:
                    split += [Job(j.requests[i:i + per64], j.tokens) for i in range(0, len(j.requests), per64)]
                else:
                    split.append(j)
            # a last group of at most 16 rows is a small job
            small, large, attached = lower(small0 + [j for j in split if len(j.requests) * group <= SMALL_ROWS],
                                           [j for j in split if len(j.requests) * group > SMALL_ROWS], min_tiles)
        if small and routed and sum(map(_tiles, routed)) * kvheads <= route_items:
            small, large, attached = small0 + routed, [], {}
        return small, large, attached, fill

    def kinds(small, large):
        return ({-1} if small else set()) | {_large_kind(len(j.requests) * group, tile_rows) for j in large}

    large0 = large
    small, large, attached, fill = lowering(1)
    if large_min_tiles > 1 and any(len(j.tokens) < large_min_tiles * TOKEN_QUANTUM for j in large):
        # A one-tile chunk costs a work item's start-up and a partial slot: chunks of
        # large_min_tiles tiles are taken when the lowering keeps its kernel kinds and
        # leaves no more small jobs (an item's latency, not its tiles, sets its time).
        alt = lowering(large_min_tiles, fill)
        if kinds(*alt[:2]) == kinds(small, large) and len(alt[0]) <= len(small):
            small, large, attached = alt[:3]
    # Tails (a request's only small job) stay whole when they alone fill the GPU,
    # so that their work items can merge their requests.
    owners = {}
    for j in small:
        for r in j.requests:
            owners[r] = owners.get(r, 0) + 1
    tails = [j for j in small if len(j.requests) == 1 and owners[j.requests[0]] == 1]
    # (a work item streams its tail alone: tails longer than TAIL_KEEP_TILES tiles are re-cut
    # unless there are enough of them for TAIL_KEEP_ITEMS_PER_CU items per CU)
    longest = max((_tiles(j) for j in tails), default=0)
    enough = len(tails) * kvheads >= n_cu * (1 if longest <= TAIL_KEEP_TILES else TAIL_KEEP_ITEMS_PER_CU)
    keep = {id(j) for j in tails} if enough else set()
    small = _recut(small, lambda r: kvheads, small_target, lambda j: growing(j) or id(j) in keep,
                   pairs=SMALL_PAIRS and not large)
    jobs = small + large
    small_jobs = len(small)
    njobs = len(jobs)
    xstride = 1 + XTAIL_FIELDS * XTAIL_MAX
    from . import _planner
    build = _metadata_native if _planner.available() else _metadata_numpy
    meta = build(jobs, small_jobs, nreq, group, kvheads, tile_rows, attached, xstride)
    maxr, maxs, nslot, slot_stride = meta["maxr"], meta["maxs"], meta["nslot"], meta["slot_stride"]
    dev = q.device
    metadata = torch.from_numpy(meta["buf"]).to(dev)
    sizes = [math.prod(shape) for shape in meta["shapes"]]
    views = [part if len(shape) == 1 else part.view(shape)
             for part, shape in zip(metadata[:sum(sizes)].split(sizes), meta["shapes"])]
    qids_t, kids_t, qlen_t, klen_t, slots_t, counts_t, rowbase_t, rest_t, xtail_t, qbase_t = views[:10]
    item_views = dict(zip(range(_native.TA_NKINDS), views[10:]))
    contiguous_q = meta["contiguous_q"]
    rest_size = meta["shapes"][7][0]
    # partial rows: fp16 scaled by 2^-e per row; lse holds (log-sum-exp, e) per row
    part = torch.empty((nslot, hq, dim), device=dev, dtype=torch.float16)
    lse = torch.empty((nslot, hq, 2), device=dev, dtype=torch.float32)
    out = torch.empty_like(q)

    abi = _native.TaPlan()
    abi.qids, abi.kstart, abi.qlen, abi.klen = (qids_t.data_ptr(), kids_t.data_ptr(),
                                                qlen_t.data_ptr(), klen_t.data_ptr())
    abi.rowbase, abi.slots, abi.counts = rowbase_t.data_ptr(), slots_t.data_ptr(), counts_t.data_ptr()
    for kind, view in item_views.items():
        abi.items[kind] = view.data_ptr() if view.numel() else None
        abi.n_items[kind] = view.numel() // 3
    # rest = every request: the merge takes requests 0..nreq-1 directly (one dependent load less)
    every = rest_size == nreq
    abi.rest, abi.n_rest = (rest_t.data_ptr() if rest_size and not every else None), int(rest_size)
    abi.part, abi.lse = part.data_ptr(), lse.data_ptr()
    abi.njobs, abi.maxr, abi.maxs, abi.nreq, abi.nslot = njobs, maxr, maxs, nreq, nslot
    abi.hq, abi.hk, abi.d = hq, kvheads, dim
    abi.dtype = _DTYPES.get(q.dtype, -1)
    abi.xtail, abi.xtail_stride = (xtail_t.data_ptr(), xstride) if attached else (None, 0)
    abi.qbase = qbase_t.data_ptr()
    abi.slot_stride = slot_stride
    keyed = {(j + small_jobs, row0): segs for (j, row0), segs in attached.items()}
    # Growing decode tails: the length of one lives in klen when it is a job, and in
    # the token field of the attachment record of every item holding it when it is
    # attached.  fill_growing writes all of them with one device-side fill.
    offs = np.cumsum([0] + sizes)
    grow = [int(offs[3]) + j for j, job in enumerate(jobs) if growing(job)]
    if attached and fixed_from is not None:
        slots_of = {key: [k for k, (job, _) in enumerate(segs) if growing(job)] for key, segs in keyed.items()}
        if any(slots_of.values()):
            k256 = 10 + _native.TA_LARGE256
            big = meta["buf"][offs[k256]:offs[k256 + 1]].reshape(-1, 3)
            for i, (j, row0, _) in enumerate(big.tolist()):
                for k in slots_of.get((j, row0), ()):
                    grow.append(int(offs[8]) + i * xstride + 2 + XTAIL_FIELDS * k)
    grow_offsets = torch.tensor(grow, dtype=torch.long, device=dev) if grow else None
    return PreparedPlan(jobs, small_jobs, True, contiguous_q, qids_t, kids_t, qlen_t, klen_t,
                        slots_t, counts_t, part, lse, out, rowbase_t, item_views, abi, metadata, rest_t,
                        keyed, xtail_t if attached else None, plan,
                        {"tile_rows": tile_rows, "fixed_from": fixed_from, "route_items": route_items, "fuse_rows": fuse_rows,
                         "consolidate_rows": consolidate_rows, "large_target": large_target,
                         "small_target": small_target, "large_min_tiles": large_min_tiles}, None,
                        meta["qbase"].tolist(),
                        grow_offsets=grow_offsets)


def pack_kv(k: torch.Tensor, v: torch.Tensor):
    """``k [T,HK,D] -> kp [HK,D,T]`` (token-minor) and ``v -> vp [HK,T,D]`` (kernels.py:144-145)."""
    return k.permute(1, 2, 0).contiguous(), v.permute(1, 0, 2).contiguous()


def attention(q, k, v, prepared):
    """``attention_matrix`` on pools packed from ``k, v [T,HK,D]`` (kernels.py:148-149)."""
    return attention_matrix(q, *pack_kv(k, v), prepared)


def _check_inputs(q, kp, vp, p):
    abi = p.abi
    if q.dtype not in _DTYPES or kp.dtype != q.dtype or vp.dtype != q.dtype:
        raise ValueError("q, kp and vp must share dtype bfloat16 or float16")
    if _DTYPES[q.dtype] != abi.dtype:
        raise ValueError("q dtype differs from the dtype the plan was prepared for")
    if not (q.is_cuda and kp.device == q.device and vp.device == q.device):
        raise ValueError("q, kp and vp must be on the same GPU")
    if tuple(q.shape) != (abi.nreq, abi.hq, abi.d):
        raise ValueError(f"q shape {tuple(q.shape)} differs from the prepared {(abi.nreq, abi.hq, abi.d)}")
    if kp.dim() != 3 or vp.dim() != 3 or kp.shape[0] != abi.hk or kp.shape[1] != abi.d:
        raise ValueError("kp must be [KV heads, head dim, tokens]")
    if tuple(vp.shape) != (abi.hk, kp.shape[2], abi.d):
        raise ValueError("vp must be [KV heads, tokens, head dim] with kp's token capacity")
    if not (kp.is_contiguous() and vp.is_contiguous()):
        raise ValueError("kp and vp must be contiguous")


def attention_matrix(q, kp, vp, prepared):
    """Attention on resident ``K [HK,D,T]`` / ``V [HK,T,D]`` pools (kernels.py:152-168).

    Returns ``prepared.out`` (``[R, HQ, D]`` in q's dtype), which every call
    overwrites, as in the reference.
    """
    _check_inputs(q, kp, vp, prepared)
    p = prepared.for_pools(kp)
    if not q.is_contiguous():
        q = q.contiguous()
    lib = _native.load()
    with torch.cuda.device(q.device):
        stream = torch.cuda.current_stream(q.device).cuda_stream
        rc = lib.ta_attention_matrix(q.data_ptr(), kp.data_ptr(), vp.data_ptr(), kp.shape[2],
                                     ctypes.byref(p.abi), p.out.data_ptr(), stream)
    _native.check(rc)
    return prepared.out


def segment(q, kp, vp, prepared, kind: int):
    """Launch one segment phase (``kind`` = TA_SMALL / TA_LARGE64/128/256 / TA_TAIL) of a plan.

    Every kind writes partials here, TA_TAIL included; ``merge`` then combines
    all requests.  TA_LARGE256 items attend their attached segments too.

    Counterpart of the direct ``_segment`` launches in the reference's
    scripts/calibrate_tiles.py:24-29 and scripts/profile_kernel.py:17-20.
    """
    _check_inputs(q, kp, vp, prepared)
    p = prepared.for_pools(kp)
    if p.abi.n_items[kind] == 0:
        return
    lib = _native.load()
    with torch.cuda.device(q.device):
        stream = torch.cuda.current_stream(q.device).cuda_stream
        rc = lib.ta_segment_plan(q.contiguous().data_ptr(), kp.data_ptr(), vp.data_ptr(), kp.shape[2],
                                 ctypes.byref(p.abi), kind, stream)
    _native.check(rc)


def tail_merge(q, kp, vp, prepared):
    """Launch the fused tail-and-merge kind of a plan (``ta_tail_merge``) into ``prepared.out``.

    Each TA_TAIL item attends its request's tail job and merges the request's
    other partial slots, which earlier ``segment`` launches on the stream wrote.
    """
    p = prepared
    _check_inputs(q, kp, vp, p)
    lib = _native.load()
    with torch.cuda.device(q.device):
        stream = torch.cuda.current_stream(q.device).cuda_stream
        rc = lib.ta_tail_merge(q.contiguous().data_ptr(), kp.data_ptr(), vp.data_ptr(), kp.shape[2],
                               ctypes.byref(p.abi), p.out.data_ptr(), stream)
    _native.check(rc)
    return p.out


def merge(prepared, kp=None):
    """Launch the log-sum-exp merge of a plan's partials into ``prepared.out`` (kernels.py:166-167).

    ``kp``: the pools the partials were computed on (selects the plan variant,
    see ``PreparedPlan.for_pools``); default: pools with a capacity multiple of 8.
    """
    p = prepared if kp is None else prepared.for_pools(kp)
    abi = p.abi
    lib = _native.load()
    with torch.cuda.device(p.out.device):
        stream = torch.cuda.current_stream(p.out.device).cuda_stream
        rc = lib.ta_merge_plan(ctypes.byref(abi), p.out.data_ptr(), stream)
    _native.check(rc)
    return p.out


def decode_append(q, k, v, cos, sin, slots, kp, vp, q_out=None):
    """One decode step's per-layer glue in one HIP launch (``ta_decode_append``).

    Replaces the reference adapter's ``apply_rotary_pos_emb`` (qwen.py:86),
    the two ``index_copy_`` scatters of the step's K and V into the pools
    (qwen.py:89-90) and the Q layout copy (qwen.py:91, kernels.py:157):
    ``q [R, HQ, D]``, ``k, v [R, HK, D]`` (any view that flattens to those
    rows, e.g. the ``[R, 1, H, D]`` projections), ``cos, sin`` with ``D``
    values per request (``[R, 1, D]``) or one row for all, ``slots [R]`` the
    step's pool positions, ``kp [HK, D, T]`` / ``vp [HK, T, D]``.  Returns the
    rotated Q ``[R, HQ, D]`` (``q_out`` if given).  The results are
    bit-identical to the eager ops in bf16 and fp16.

    ``slots`` given as host data (a sequence or a CPU tensor) are range-checked
    here: a position outside ``[0, T)`` raises ``ValueError``, as the eager
    ``index_copy_`` does.  Slots already on the GPU are not read back (that
    would synchronise the host); the kernel then skips a position outside the
    pool, writing nothing for it.
    """
    nreq = q.shape[0]
    d = q.shape[-1]
    q2, k2, v2 = q.reshape(nreq, -1, d), k.reshape(nreq, -1, d), v.reshape(nreq, -1, d)
    hq, hk = q2.shape[1], k2.shape[1]
    if q.dtype not in _DTYPES or any(t.dtype != q.dtype for t in (k, v, cos, sin, kp, vp)):
        raise ValueError("q, k, v, cos, sin and the pools must share dtype bfloat16 or float16")
    if tuple(v2.shape) != (nreq, hk, d) or kp.shape[:2] != (hk, d) or tuple(vp.shape) != (hk, kp.shape[2], d):
        raise ValueError("k/v must be [R, HK, D] and the pools [HK, D, T] / [HK, T, D]")
    if not (kp.is_contiguous() and vp.is_contiguous()):
        raise ValueError("kp and vp must be contiguous")
    cos2, sin2 = cos.reshape(-1, d), sin.reshape(-1, d)
    if cos2.shape != sin2.shape or cos2.shape[0] not in (1, nreq):
        raise ValueError("cos and sin need D values per request or one row for all")
    cs_stride = d if cos2.shape[0] == nreq else 0
    q2, k2, v2, cos2, sin2 = (t.contiguous() for t in (q2, k2, v2, cos2, sin2))
    if not isinstance(slots, torch.Tensor):
        slots = torch.tensor(list(slots), dtype=torch.int64)
    if slots.numel() != nreq:
        raise ValueError("slots needs one pool position per request")
    if not slots.is_cuda and nreq and not (0 <= int(slots.min()) and int(slots.max()) < kp.shape[2]):
        raise ValueError(f"slots must lie in [0, {kp.shape[2]}) (the pool capacity)")
    slots = slots.to(device=q.device, dtype=torch.int32).contiguous()
    if q_out is None:
        q_out = torch.empty((nreq, hq, d), device=q.device, dtype=q.dtype)
    lib = _native.load()
    with torch.cuda.device(q.device):
        stream = torch.cuda.current_stream(q.device).cuda_stream
        rc = lib.ta_decode_append(q2.data_ptr(), k2.data_ptr(), v2.data_ptr(), cos2.data_ptr(), sin2.data_ptr(),
                                  cs_stride, slots.data_ptr(), kp.data_ptr(), vp.data_ptr(), q_out.data_ptr(),
                                  nreq, hq, hk, d, kp.shape[2], _DTYPES[q.dtype], stream)
    _native.check(rc)
    return q_out


def launch_durations_us(fn, n: int, device=None) -> list:
    """Kernel durations of ``n`` eager calls ``fn(0..n-1)`` on the current stream, in microseconds.

    Each call's first kernel launch of this library is stamped at dispatch
    begin and end through ``ta_time_next_launch`` (hipExtLaunchKernel), so the
    figures are the kernel's own duration, without launch gaps -- the same
    quantity ``rocprofv3 --kernel-trace`` reports.  Not for use under capture.
    """
    device = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    stream = torch.cuda.current_stream(device)
    lib = _native.load()
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    for start, stop in events:  # a first record creates the underlying HIP events
        start.record(stream)
        stop.record(stream)
    torch.cuda.synchronize(device)
    try:
        for i, (start, stop) in enumerate(events):
            _native.check(lib.ta_time_next_launch(start.cuda_event, stop.cuda_event))
            fn(i)
    finally:
        lib.ta_time_next_launch(None, None)
    torch.cuda.synchronize(device)
    return [start.elapsed_time(stop) * 1e3 for start, stop in events]


class CachedDecodePlan:
    """A prompt schedule plus one contiguous growing KV tail per request (kernels.py:171-186)."""

    def __init__(self, prefix_plan, q, prefix_tokens, max_new_tokens):
        tails = [Job((r,), id_run(prefix_tokens + r * max_new_tokens, prefix_tokens + (r + 1) * max_new_tokens))
                 for r in range(q.shape[0])]
        plan = Plan(prefix_plan.jobs + tails, prefix_plan.method, prefix_plan.estimated_us,
                    prefix_plan.settings)
        self.max_new_tokens = max_new_tokens
        self.prepared = prepare(plan, q, fixed_from=prefix_tokens)
        ordered = self.prepared.jobs
        # the growing tails that stay jobs (the others are attached to root work items,
        # their lengths in the attachment records; update() sets both)
        self.tail_indices = torch.tensor([i for i, job in enumerate(ordered) if job.tokens[0] >= prefix_tokens],
                                         device=q.device, dtype=torch.long)

    def update(self, generated_tokens):
        """Set every tail's length to ``generated_tokens`` (device-side fill, no sync)."""
        if not 0 <= generated_tokens <= self.max_new_tokens:
            raise ValueError("generated_tokens must be within [0, max_new_tokens]")
        self.prepared.fill_growing(generated_tokens)
        return self.prepared
