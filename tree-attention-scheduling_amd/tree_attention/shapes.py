"""Named tree shapes of the reference's benchmarks and of the evaluation configs.

Each function returns the ``(parents, lengths, terminals)`` triple accepted by
``KVTree.synthetic``; ``tree(spec)`` builds it.

* ``benchmark_cases`` -- scripts/benchmark.py:14-23 (``wide_long`` is the
  128-request x 8192-token, 8128-shared headline shape).
* ``reference_grid`` -- the reference's 81 evaluation trees,
  scripts/tree_shapes.py:5-19.
* ``config_grid`` -- the 81-shape factorial grid requests x context x shared
  fraction x depth.  ``shared = floor(fraction * context + 0.5)``; the shared
  region is cut into ``depth`` levels of a balanced binary tree (level ``i``
  has ``2**i`` nodes), level lengths ``shared // depth`` with the first
  ``shared % depth`` levels one token longer; requests are spread evenly over
  the last level's nodes (request ``r`` goes to leaf ``r * leaves // R``) and
  each gets a private tail of ``context - shared`` tokens.
* ``nested_unequal`` -- root 4096 -> 8 x 1024 -> 4 x 256 per child (32 leaf
  requests), plus one request ending at the first 1024-token node and two
  requests duplicating the first two leaf paths (35 requests, 20,480 tokens).
* ``calibration_grid`` -- shapes used only to fit the MI355X cost model; every
  length is disjoint from the evaluation shapes above.
* ``decode_calibration_grid`` -- decode-step layers (a prompt tree plus a
  growing tail per request) used only to fit the MI355X cost model, in the
  form of scripts/calibrate_tiles.py:13-14 (many requests over a short shared
  root, or private contexts only), at counts and lengths of their own.
* ``qwen3_4b_workload`` -- the token sequences of the Qwen3-4B-shaped decode
  workload (32 requests over a 2048-token prompt, 4 branches, 8 suffixes each).
* ``decode_layers`` -- the two decode-step evaluation layers: the protocol of
  scripts/benchmark_decode_plan.py:21-27 and the Qwen3-4B-shaped workload's.
"""
from __future__ import annotations

from itertools import product

from .tree import KVTree


def tree(spec) -> KVTree:
    parents, lengths, terminals = spec
    return KVTree.synthetic(list(parents), list(lengths), list(terminals))


def shared_prefix(requests: int, root: int, private) -> tuple:
    """One shared root of ``root`` tokens plus a private child per request."""
    tails = list(private) if isinstance(private, (list, tuple)) else [private] * requests
    return [-1] + [0] * requests, [root] + tails, list(range(1, requests + 1))


def benchmark_cases() -> dict:
    """The six representative shapes of scripts/benchmark.py:14-23."""
    return {
        "no_share": shared_prefix(32, 0, 1024),
        "wide": shared_prefix(32, 2048, 64),
        "unequal": shared_prefix(32, 1024, [32 + 31 * i for i in range(32)]),
        "deep": ([-1, 0, 1, 1, 2, 2, 3, 3] + list(range(4, 8)) * 4, [512] * 8 + [64] * 16,
                 list(range(8, 24))),
        "wide_long": shared_prefix(128, 8128, 64),
        "no_share_long": shared_prefix(128, 0, 8192),
    }


def headline() -> tuple:
    """128 requests x 8192 tokens, 8128 shared (16,320 physical tokens)."""
    return shared_prefix(128, 8128, 64)


def cpu_baseline_shape() -> tuple:
    """8 requests, 1024-token shared root plus 64 private tokens each."""
    return shared_prefix(8, 1024, 64)


def nested_unequal() -> tuple:
    parents, lengths = [-1], [4096]
    for _ in range(8):
        parents.append(0)
        lengths.append(1024)
    leaves = []
    for child in range(1, 9):
        for _ in range(4):
            leaves.append(len(parents))
            parents.append(child)
            lengths.append(256)
    terminals = leaves + [1, leaves[0], leaves[1]]
    return parents, lengths, terminals


def reference_grid():
    """Yield ``(params, spec)`` for scripts/tree_shapes.py:5-19's 81 trees."""
    for fanout, root, shared, private in product(((3, 1), (9, 3), (17, 7)), (32, 192, 768),
                                                (12, 96, 384), (24, 192, 768)):
        parents, lengths, terminals = [-1], [root], []
        for branch, width in enumerate(fanout):
            node = len(parents)
            parents.append(0)
            lengths.append(shared * (branch + 1) + 7 * branch)
            for leaf in range(width):
                terminals.append(len(parents))
                parents.append(node)
                lengths.append(private * (1 + leaf % 3) + 5 * branch)
        yield dict(fanout=list(fanout), root=root, shared=shared, private=private), (parents, lengths, terminals)


def grid_tree(requests: int, context: int, fraction: float, depth: int) -> tuple:
    shared = int(fraction * context + 0.5)
    private = context - shared
    level_len = [shared // depth + (1 if i < shared % depth else 0) for i in range(depth)]
    parents, lengths = [-1], [level_len[0]]
    level = [0]
    for i in range(1, depth):
        nxt = []
        for parent in level:
            for _ in range(2):
                nxt.append(len(parents))
                parents.append(parent)
                lengths.append(level_len[i])
        level = nxt
    terminals = []
    for r in range(requests):
        leaf = level[r * len(level) // requests]
        terminals.append(len(parents))
        parents.append(leaf)
        lengths.append(private)
    return parents, lengths, terminals


def config_grid():
    """Yield ``(params, spec)`` for the 81-shape requests x context x fraction x depth grid."""
    for requests, context, fraction, depth in product((16, 32, 128), (1024, 4096, 8192),
                                                      (0.25, 0.75, 0.99), (1, 2, 3)):
        yield (dict(requests=requests, context=context, fraction=fraction, depth=depth),
               grid_tree(requests, context, fraction, depth))


def calibration_grid():
    """Yield ``(name, spec)`` of cost-model calibration shapes (disjoint lengths and counts)."""
    for requests in (6, 20, 40, 96):
        for root, private in ((600, 40), (1500, 100), (3000, 300), (5000, 20)):
            yield f"shared_r{requests}_{root}_{private}", shared_prefix(requests, root, private)
    for requests in (6, 20, 40):
        for private in (700, 2000):
            yield f"private_r{requests}_{private}", shared_prefix(requests, 0, private)
    # short shared prefixes under long private contexts, where sharing saves little and
    # every shared job adds a partial slot per request to merge
    for requests, root, private in ((28, 300, 940), (44, 700, 2300), (60, 1100, 3900), (20, 180, 1300)):
        yield f"shared_r{requests}_{root}_{private}", shared_prefix(requests, root, private)
    # large shapes, where launch overheads are a small part of the layer
    for requests, root, private in ((112, 7000, 50), (80, 6000, 150), (72, 3500, 90)):
        yield f"shared_r{requests}_{root}_{private}", shared_prefix(requests, root, private)
    parents, lengths = [-1, 0, 0], [2500, 1800, 2200]
    for leaf in range(60):
        parents.append(1 + leaf % 2)
        lengths.append((73, 79, 91)[leaf % 3])
    yield "two_level_r60", (parents, lengths, list(range(3, 63)))
    # three levels with unequal branches, a request ending at an inner node and a duplicate
    # path: request counts whose rows are not a multiple of the 256-row tile
    for name, root, mids, leaves_per, mid_len, leaf_len in (("nested_r26", 3700, 3, 8, 905, 230),
                                                            ("nested_r54", 2600, 4, 13, 1300, 170)):
        parents, lengths, terminals = [-1], [root], []
        for m in range(mids):
            node = len(parents)
            parents.append(0)
            lengths.append(mid_len + 11 * m)
            for _ in range(leaves_per):
                terminals.append(len(parents))
                parents.append(node)
                lengths.append(leaf_len)
        yield name, (parents, lengths, terminals + [1, terminals[0]])
    # deeper trees in the evaluation grid's form (balanced binary splits of the shared part),
    # at request counts and lengths of their own
    for requests, context, fraction, depth in product((20, 40, 96), (1500, 6000), (0.5, 0.9), (2, 3)):
        yield (f"deep_r{requests}_{context}_{int(fraction * 100)}_d{depth}",
               grid_tree(requests, context, fraction, depth))


def decode_calibration_grid():
    """Yield ``(name, spec, reserved, generated)``: a prompt tree, the tail tokens reserved per
    request and the tokens generated so far (a ``CachedDecodePlan`` updated to that step)."""
    yield "dec_private_r28_736", shared_prefix(28, 0, 736), 15, 9
    yield "dec_shared_r28_736_44", shared_prefix(28, 736, 44), 15, 9
    yield "dec_shared_r44_1400_56", shared_prefix(44, 1400, 56), 19, 13
    yield "dec_shared_r60_480_30", shared_prefix(60, 480, 30), 9, 3
    yield "dec_shared_r20_2600_36", shared_prefix(20, 2600, 36), 21, 17
    # a branching prompt: 3 branches of 70 tokens, 12 suffixes of 100 tokens under each
    parents, lengths, terminals = [-1], [1800], []
    for _ in range(3):
        branch = len(parents)
        parents.append(0)
        lengths.append(70)
        for _ in range(12):
            terminals.append(len(parents))
            parents.append(branch)
            lengths.append(100)
    yield "dec_branch_r36_1800_70_100", (parents, lengths, terminals), 15, 5


def decode_layers():
    """Yield ``(name, tree, reserved, generated)`` of the two decode-step evaluation layers:
    32 requests over a 1024-token root with 64 private tokens each (the decode-plan protocol,
    scripts/benchmark_decode_plan.py:21-27) and the Qwen3-4B-shaped workload's prompt tree,
    each with 16 reserved tail tokens per request, at 8 generated."""
    yield "protocol_r32_1024_64", tree(shared_prefix(32, 1024, 64)), 16, 8
    yield "qwen3_4b", KVTree.from_sequences(qwen3_4b_workload()), 16, 8


def qwen3_4b_workload(seed: int = 5) -> list:
    """32 requests: a 2048-token prompt, a 4-way branch of 64-token nodes, 8 suffixes of 128 tokens each.

    Token ids are uniform over Qwen3's 151,936-entry vocabulary.  The branch
    nodes' length (64) is this workload's own choice; the resulting tree is
    checked (``ValueError`` otherwise), since random ids could merge nodes.
    """
    import random
    rng = random.Random(seed)
    ids = lambda n: [rng.randrange(151_936) for _ in range(n)]  # noqa: E731
    prompt = ids(2048)
    sequences = []
    for _ in range(4):
        branch = ids(64)
        for _ in range(8):
            sequences.append(prompt + branch + ids(128))
    t = KVTree.from_sequences(sequences)
    lengths = sorted(len(n.tokens) for n in t.nodes if n.tokens)  # the root node is empty
    if lengths != [64] * 4 + [128] * 32 + [2048] or t.storage_tokens != 2048 + 4 * 64 + 32 * 128:
        raise ValueError("random ids merged nodes of the workload tree")
    return sequences
