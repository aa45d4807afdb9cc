"""Segment planner and analytical cost model for tree-shared decode attention.

Drop-in for the reference's ``src/tree_attention/schedule.py`` (``Job`` :7-10,
``physical_jobs`` :13-26, ``CostModel`` :29-52, ``Plan`` :55-69, ``schedule``
:72-151).  Plans are bit-exact with the reference planner for equal cost
parameters: same job tuples, same job order, same ``estimated_us`` float.

What has to stay identical, and why:

* ``CostModel.cost`` evaluates ``max(flops/F, reads/B) + task*qtiles*HK +
  partial/B + merge*nreq`` in exactly that association (schedule.py:41-52);
  any reassociation changes the last bits of ``estimated_us``.
* Every plan cost is a left-to-right float sum over ``physical_jobs`` in job
  order, starting from integer 0 (schedule.py:84-85).  The reference was
  measured on CPython 3.11, whose ``sum`` adds floats one by one; the sums here
  are explicit loops so the result does not depend on the interpreter's
  ``sum`` implementation (3.12+ compensates rounding).
* The subset DP keeps a table keyed by "requests removed" with strict ``<``
  updates and breaks final ties by comparing ``(cost, pushed_children)``
  tuples (schedule.py:116-131); greedy pushes a child only on strict
  ``split_q < split_k`` (schedule.py:103-112).

How it differs: costs of ``split(range(count), tokens)`` are evaluated from
the run-length structure of ``tokens`` (contiguous physical runs) without
building job tuples, DP states are memoised by ``(node, top of inherited
chain)`` instead of hashing token tuples, and both the DP and the plan
materialisation are iterative, so planning holds no reference cycles and the
input tree is freed as soon as the caller drops it (tests/test_semantics.py:56-67
in the reference).
"""
from __future__ import annotations

from dataclasses import asdict, dataclass
from itertools import chain
from math import ceil

from .tree import KVTree, id_run


@dataclass(frozen=True)
class Job:
    """Requests that attend together to one KV segment (reference schedule.py:7-10)."""
    requests: tuple[int, ...]
    tokens: tuple[int, ...]


def physical_jobs(jobs):
    """Split jobs at physical KV discontinuities (reference schedule.py:13-26).

    A job whose ids span exactly ``len(tokens)`` positions is kept as is;
    otherwise it becomes one job per maximal run of consecutive ids.
    """
    out = []
    for job in jobs:
        toks = job.tokens
        if toks[-1] - toks[0] + 1 == len(toks):
            out.append(job)
            continue
        begin = 0
        for i in range(1, len(toks)):
            if toks[i] != toks[i - 1] + 1:
                out.append(Job(job.requests, toks[begin:i]))
                begin = i
        out.append(Job(job.requests, toks[begin:]))
    return out


@dataclass
class CostModel:
    """Roofline parameters in bytes/us and FLOP/us (reference schedule.py:29-39).

    The defaults are the reference's Ascend 910B values; ``mi355x()`` returns
    the parameters fitted on MI355X.
    """
    bandwidth: float = 900_000.0
    cube_flops: float = 100_000_000.0
    task_us: float = 0.15
    merge_us: float = 0.03
    cube_rows: int = 16
    key_tile: int = 128
    kv_split: int = 512
    max_query_rows: int = 64

    def _cost_n(self, nreq: int, ntok: int, qheads: int, kvheads: int, dim: int):
        """Cost of one physical job with ``nreq`` requests and ``ntok`` tokens."""
        if not nreq or not ntok:
            return 0.0
        rows = nreq * (qheads // kvheads)
        small = rows <= self.cube_rows
        q_tile = self.cube_rows if small else self.max_query_rows
        k_tile = self.key_tile if small else self.key_tile // 2
        qtiles = ceil(rows / q_tile)
        ktiles = ceil(ntok / k_tile)
        flops = 4 * qtiles * q_tile * ktiles * k_tile * dim * kvheads
        reads = 4 * ntok * dim * kvheads * qtiles
        partial = 4 * nreq * qheads * (dim + 1)
        return (max(flops / self.cube_flops, reads / self.bandwidth)
                + self.task_us * qtiles * kvheads
                + partial / self.bandwidth
                + self.merge_us * nreq)

    def cost(self, requests, tokens, qheads, kvheads, dim):
        """Estimated microseconds of one job (reference schedule.py:41-52)."""
        return self._cost_n(len(requests), len(tokens), qheads, kvheads, dim)

    @classmethod
    def mi355x(cls) -> "CostModel":
        """Parameters fitted on one MI355X (see ``tree_attention.calibration``)."""
        from .calibration import mi355x_cost_model
        return mi355x_cost_model()


@dataclass
class Plan:
    """A schedule: jobs in execution order plus its estimate (reference schedule.py:55-69)."""
    jobs: list[Job]
    method: str
    estimated_us: float
    settings: dict

    def validate(self, tree):
        """Raise ``ValueError`` unless every request's context is covered exactly once."""
        seen = [[] for _ in tree.paths]
        for job in self.jobs:
            for r in job.requests:
                seen[r].extend(job.tokens)
        for r, path in enumerate(tree.paths):
            if sorted(seen[r]) != sorted(path):
                raise ValueError(f"Plan does not partition request {r}'s context")


def _is_range(toks) -> bool:
    """True if ``toks`` is exactly ``range(toks[0], toks[0] + len(toks))`` (C-speed compare)."""
    return bool(toks) and toks[-1] - toks[0] + 1 == len(toks) and toks == id_run(toks[0], toks[0] + len(toks))


def _runs_of(tokens) -> tuple:
    """Maximal runs of consecutive ids as ``((start, length), ...)``."""
    if _is_range(tokens):
        return ((tokens[0], len(tokens)),)
    runs = []
    for t in tokens:
        if runs and runs[-1][0] + runs[-1][1] == t:
            runs[-1][1] += 1
        else:
            runs.append([t, 1])
    return tuple((s, n) for s, n in runs)


def _join_runs(a: tuple, b: tuple) -> tuple:
    if a and b and a[-1][0] + a[-1][1] == b[0][0]:
        return a[:-1] + ((a[-1][0], a[-1][1] + b[0][1]),) + b[1:]
    return a + b


def _increasing(tree: KVTree, node_runs=None) -> bool:
    """True if every root-to-node id chain is strictly increasing.

    Under that condition a chunk passes the reference's span test
    (``last - first + 1 == len``) exactly when it is one consecutive run, so
    run-length costs equal the reference's per-job costs.  ``node_runs``
    (each node's ``_runs_of``) saves rescanning the tokens.
    """
    nodes = tree.nodes
    for v, node in enumerate(nodes):
        toks = node.tokens
        runs = node_runs[v] if node_runs is not None else _runs_of(toks)
        for i in range(1, len(runs)):
            if runs[i][0] <= runs[i - 1][0] + runs[i - 1][1] - 1:
                return False
        if toks and node.parent >= 0:
            # nearest ancestor with tokens must end below this node's first id
            p = node.parent
            while p >= 0 and not nodes[p].tokens:
                p = nodes[p].parent
            if p >= 0 and nodes[p].tokens[-1] >= toks[0]:
                return False
    return True


def schedule(tree: KVTree, qheads=32, kvheads=8, dim=128, method="cube", model=None, native=None) -> Plan:
    """Plan one decode step's attention over ``tree`` (reference schedule.py:72-151).

    Methods: ``request`` (each request alone), ``fixed`` (one group per tree
    node), ``greedy`` (per-child SplitQ/SplitK choice) and ``cube`` (subset DP
    over children with full descendant cost).

    ``native`` selects the implementation of the greedy / cube decisions:
    ``None`` uses the C++ planner (libtree_plan.so) when it is built and the
    case is one it covers (the reference's cost formula, increasing id chains),
    else this module's; ``True`` requires the C++ planner (``ValueError`` for
    a case it does not cover); ``False`` uses this module's.  Both give the
    same plan, bit for bit.
    """
    if qheads % kvheads:
        raise ValueError("Query heads must be divisible by KV heads")
    model = model or CostModel()
    group = qheads // kvheads
    req_tile = max(1, model.max_query_rows // group)
    kv_split = model.kv_split
    nodes = tree.nodes

    def split(requests, tokens):
        return [Job(tuple(requests[q:q + req_tile]), tuple(tokens[k:k + kv_split]))
                for q in range(0, len(requests), req_tile)
                for k in range(0, len(tokens), kv_split)]

    def plan_cost(jobs):
        total = 0
        for job in physical_jobs(jobs):
            total = total + model.cost(job.requests, job.tokens, qheads, kvheads, dim)
        return total

    if method == "request":
        jobs = [j for r, path in enumerate(tree.paths) for j in split((r,), path)]
    elif method == "fixed":
        jobs = [j for n in nodes for j in split(n.requests, n.tokens)]
    elif method in ("greedy", "cube"):
        jobs = _grouped_jobs(tree, method, model, split, plan_cost, qheads, kvheads, dim, req_tile, native)
    else:
        raise ValueError(f"Unknown scheduling method: {method}")
    settings = asdict(model)
    settings.update(qheads=qheads, kvheads=kvheads, head_dim=dim)
    return Plan(jobs, method, plan_cost(jobs), settings)


def _native_covers(model) -> bool:
    """The C++ planner evaluates the cost formula on int64 sizes and double rates."""
    ints = (model.cube_rows, model.key_tile, model.kv_split, model.max_query_rows)
    rates = (model.bandwidth, model.cube_flops, model.task_us, model.merge_us)
    return (type(model)._cost_n is CostModel._cost_n
            and all(type(x) is int and 0 < x < 2 ** 31 for x in ints)
            and all(type(x) in (int, float) for x in rates))


def _grouped_jobs(tree, method, model, split, plan_cost, qheads, kvheads, dim, req_tile, native=None):
    """Greedy / subset-DP grouping, then pre-order materialisation of jobs."""
    nodes = tree.nodes
    kv_split = model.kv_split
    all_runs = [_runs_of(nd.tokens) for nd in nodes] if type(model).cost is CostModel.cost else None
    fast = all_runs is not None and _increasing(tree, all_runs)
    if native is not False:
        from . import _planner
        covered = fast and _native_covers(model)
        if native and not covered:
            raise ValueError("the C++ planner covers the reference cost formula over increasing id chains only")
        if covered and (native or _planner.available()):
            pushed, _ = _planner.grouped_decisions(tree, method, model, qheads, kvheads, dim, all_runs)
            return _materialise(nodes, split, lambda v, top: {c for c in nodes[v].children if pushed[c]})

    # --- token chains ------------------------------------------------------
    # A DP state (v, top) means: node v plus the inherited tokens of the chain
    # top -> parent(v); top is None when nothing is inherited.
    node_runs = {}
    chain_runs = {}

    def own_runs(v):
        got = node_runs.get(v)
        if got is None:
            got = node_runs[v] = all_runs[v] if all_runs is not None else _runs_of(nodes[v].tokens)
        return got

    def runs(v, top):
        if top is None or top == v:
            return own_runs(v)
        got = chain_runs.get((v, top))
        if got is not None:
            return got
        # Walk up to ``top`` (or to a cached prefix), then join downwards.
        pending = []
        u = v
        while u != top and (u, top) not in chain_runs:
            pending.append(u)
            u = nodes[u].parent
        acc = own_runs(top) if u == top else chain_runs[(u, top)]
        for w in reversed(pending):
            acc = _join_runs(acc, own_runs(w))
            chain_runs[(w, top)] = acc
        return acc

    def chain_tokens(v, top):
        parts = []
        u = v
        while True:
            parts.append(nodes[u].tokens)
            if top is None or u == top:
                break
            u = nodes[u].parent
        return parts[0] if len(parts) == 1 else tuple(chain.from_iterable(reversed(parts)))

    # --- cost of split(range(count), tokens) -------------------------------
    count_memo = {}

    def count_cost(count, v, top):
        key = (count, v, top)
        got = count_memo.get(key)
        if got is not None:
            return got
        if fast:
            got = _count_cost_runs(model, count, runs(v, top), req_tile, kv_split, qheads, kvheads, dim)
        else:
            got = plan_cost(split(range(count), chain_tokens(v, top)))
        count_memo[key] = got
        return got

    def child_top(v, top):
        return v if top is None else top

    # --- memoised post-order evaluation -------------------------------------
    memo = {}
    greedy_push = {}

    def deps(key):
        v, top = key
        kids = nodes[v].children
        if not kids:
            return ()
        ct = child_top(v, top)
        if method == "cube":
            return tuple(d for c in kids for d in ((c, None), (c, ct)))
        choice = greedy_push.get(key)
        if choice is None:
            choice = greedy_push[key] = _greedy_choice(nodes, v, top, ct, count_cost)
        pushed = choice[0]
        return tuple((c, ct if c in pushed else None) for c in kids)

    def evaluate(key):
        v, top = key
        node = nodes[v]
        if not node.children:
            return count_cost(len(node.requests), v, top), ()
        ct = child_top(v, top)
        if method == "greedy":
            pushed, remaining = greedy_push[key]
            total = count_cost(remaining, v, top)
            kids_total = 0
            for c in node.children:
                kids_total = kids_total + memo[(c, ct if c in pushed else None)][0]
            return total + kids_total, tuple(pushed)
        table = {0: (0.0, ())}
        for c in node.children:
            count = len(nodes[c].requests)
            alone = memo[(c, None)][0]
            joined = memo[(c, ct)][0]
            nxt = {}
            for removed, (subtotal, pushed) in table.items():
                for extra, sub, chosen in ((0, alone, pushed), (count, joined, pushed + (c,))):
                    slot = removed + extra
                    value = subtotal + sub
                    if slot not in nxt or value < nxt[slot][0]:
                        nxt[slot] = value, chosen
            table = nxt
        best = None
        for removed, (subtotal, pushed) in table.items():
            cand = (subtotal + count_cost(len(node.requests) - removed, v, top), pushed)
            if best is None or cand < best:
                best = cand
        return best

    stack = [(0, None)]
    while stack:
        key = stack[-1]
        if key in memo:
            stack.pop()
            continue
        missing = [d for d in deps(key) if d not in memo]
        if missing:
            stack.extend(reversed(missing))
            continue
        memo[key] = evaluate(key)
        stack.pop()

    return _materialise(nodes, split, lambda v, top: memo[(v, top)][1])


def _materialise(nodes, split, pushed_of):
    """Jobs of the chosen states in pre-order (reference schedule.py:133-151).

    ``pushed_of(v, top)`` is the set of children that state (v, top) pushes;
    a pushed child's state inherits the chain top -> v.
    """
    def chain_tokens(v, top):
        parts = []
        u = v
        while True:
            parts.append(nodes[u].tokens)
            if top is None or u == top:
                break
            u = nodes[u].parent
        return parts[0] if len(parts) == 1 else tuple(chain.from_iterable(reversed(parts)))

    jobs = []
    todo = [(0, None)]
    while todo:
        v, top = todo.pop()
        node = nodes[v]
        pushed = pushed_of(v, top)
        detached = {r for c in pushed for r in nodes[c].requests}
        remaining = tuple(r for r in node.requests if r not in detached)
        jobs.extend(split(remaining, chain_tokens(v, top)))
        ct = v if top is None else top
        for c in reversed(node.children):
            todo.append((c, ct if c in pushed else None))
    return jobs


def _greedy_choice(nodes, v, top, ct, count_cost):
    """SplitQ/SplitK decision per child in child order (reference schedule.py:103-112).

    Returns ``(pushed_children_list, remaining_request_count)``.
    """
    remaining = len(nodes[v].requests)
    pushed = []
    for c in nodes[v].children:
        count = len(nodes[c].requests)
        split_k = count_cost(remaining, v, top) + count_cost(count, c, c)
        split_q = count_cost(remaining - count, v, top) + count_cost(count, c, ct)
        if split_q < split_k:
            pushed.append(c)
            remaining -= count
    return pushed, remaining


def _count_cost_runs(model, count, runs, req_tile, kv_split, qheads, kvheads, dim):
    """``sum(cost(j) for j in physical_jobs(split(range(count), tokens)))`` from runs.

    ``split`` emits request tiles (outer) times ``kv_split`` chunks (inner);
    ``physical_jobs`` cuts each chunk at run boundaries.  Costs are added in
    that order.
    """
    ntok = sum(n for _, n in runs)
    # Piece lengths of every kv_split chunk, in order, computed once.
    pieces = []
    edges = []
    pos = 0
    for _, n in runs:
        edges.append((pos, pos + n))
        pos += n
    ri = 0
    for k in range(0, ntok, kv_split):
        kend = min(k + kv_split, ntok)
        chunk = []
        while edges[ri][1] <= k:
            ri += 1
        j = ri
        while j < len(edges) and edges[j][0] < kend:
            lo = max(edges[j][0], k)
            hi = min(edges[j][1], kend)
            chunk.append(hi - lo)
            j += 1
        pieces.append(chunk)
    total = 0
    for q in range(0, count, req_tile):
        nq = min(req_tile, count - q)
        for chunk in pieces:
            for n in chunk:
                total = total + model._cost_n(nq, n, qheads, kvheads, dim)
    return total
