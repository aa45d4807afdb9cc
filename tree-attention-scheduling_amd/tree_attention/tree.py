"""Compressed radix tree over decode contexts and its physical KV storage order.

Drop-in for the reference's ``src/tree_attention/tree.py`` (``Node`` at :4-10,
``KVTree`` at :13-92).  The physical KV id of every token is fixed here: the
attention backend reads K/V pools in exactly this order, so node ids, token ids
and child order must match the reference bit for bit.

Storage order (tree.py:19-50): nodes are created depth-first; siblings appear in
the order their first token is first seen among the parent's requests; a node's
whole subtree receives ids before its next sibling.  This module builds the
tree with an explicit stack instead of recursion so that very deep trees (long
chains of single-token branches) do not hit Python's recursion limit.
"""
from __future__ import annotations

from dataclasses import dataclass, field

_IDS: tuple = ()
_IDS_MAX = 1 << 20


def id_run(start: int, stop: int) -> tuple:
    """``tuple(range(start, stop))``, sliced from one shared tuple of ids below 2**20.

    Slicing allocates no int objects, and tuples cut from the shared one hold
    the same objects, so comparing two of them is an identity check per
    element.  Token ids are compared and re-cut on every plan, which makes
    this the cheap way to build them.
    """
    global _IDS
    if start < 0 or stop > _IDS_MAX:
        return tuple(range(start, stop))
    if stop > len(_IDS):
        _IDS = tuple(range(min(_IDS_MAX, max(stop, 2 * len(_IDS), 1 << 14))))
    return _IDS[start:stop]


@dataclass
class Node:
    """One compressed edge of the tree (reference tree.py:4-10).

    ``tokens`` are physical KV ids, ``requests`` every request whose context
    passes through this node, ``terminal`` the requests whose context ends here.
    """
    parent: int
    tokens: tuple[int, ...]
    children: list[int] = field(default_factory=list)
    terminal: list[int] = field(default_factory=list)
    requests: tuple[int, ...] = ()


@dataclass
class KVTree:
    """Radix tree plus per-request physical paths (reference tree.py:13-17)."""
    nodes: list[Node]
    paths: list[tuple[int, ...]]
    token_ids: list[int] | None = None

    @classmethod
    def from_sequences(cls, sequences: list[list[int]]) -> "KVTree":
        """Build the compressed trie of ``sequences`` (reference tree.py:19-50).

        Each pending entry on the stack is a group of requests that agree on
        every token before ``offset`` and whose node must be created under
        ``parent``.  Popping order reproduces the reference's pre-order walk.
        """
        if not sequences or any(not seq for seq in sequences):
            raise ValueError("Every decode request needs a nonempty context")
        seqs = [list(s) for s in sequences]
        nodes = [Node(-1, ())]
        token_ids: list[int] = []
        paths: list[tuple[int, ...] | None] = [None] * len(seqs)

        def expand(node_id, group, offset, prefix):
            """Record requests ending at ``offset``; return child groups in first-seen order."""
            done = [r for r in group if len(seqs[r]) == offset]
            nodes[node_id].terminal.extend(done)
            for r in done:
                paths[r] = prefix
            by_token: dict[int, list[int]] = {}
            for r in group:
                if len(seqs[r]) > offset:
                    by_token.setdefault(seqs[r][offset], []).append(r)
            return list(by_token.values())

        # Stack entries: (parent, member requests, offset, prefix ids of parent).
        stack = [(0, grp, 0, ()) for grp in reversed(expand(0, list(range(len(seqs))), 0, ()))]
        while stack:
            parent, group, offset, prefix = stack.pop()
            # Longest common extension of the group, bounded by its shortest member.
            limit = min(len(seqs[r]) for r in group)
            end = offset + 1
            lead = seqs[group[0]]
            while end < limit and all(seqs[r][end] == lead[end] for r in group):
                end += 1
            first = len(token_ids)
            ids = id_run(first, first + end - offset)
            token_ids.extend(lead[offset:end])
            node_id = len(nodes)
            nodes.append(Node(parent, ids, requests=tuple(group)))
            nodes[parent].children.append(node_id)
            path = prefix + ids
            for grp in reversed(expand(node_id, group, end, path)):
                stack.append((node_id, grp, end, path))
        nodes[0].requests = tuple(range(len(seqs)))
        return cls(nodes, paths, token_ids)

    @classmethod
    def synthetic(cls, parents, lengths, terminal_nodes) -> "KVTree":
        """Topology-only tree (reference tree.py:52-73).

        Node ``i`` owns physical ids ``[sum(lengths[:i]), sum(lengths[:i+1]))``;
        request ``r`` ends at node ``terminal_nodes[r]`` and its path is the
        concatenation of its ancestors' ids, root first.
        """
        nodes: list[Node] = []
        base = 0
        for i, (parent, length) in enumerate(zip(parents, lengths)):
            valid = parent == -1 if i == 0 else 0 <= parent < i
            if not valid:
                raise ValueError("Parents must precede children")
            nodes.append(Node(parent, id_run(base, base + length)))
            base += length
            if parent >= 0:
                nodes[parent].children.append(i)
        paths = []
        for r, leaf in enumerate(terminal_nodes):
            nodes[leaf].terminal.append(r)
            chain = []
            node = leaf
            while node >= 0:
                nodes[node].requests += (r,)
                chain.append(nodes[node].tokens)
                node = nodes[node].parent
            path = tuple(t for part in reversed(chain) for t in part)
            if not path:
                raise ValueError("Every decode request needs a nonempty context")
            paths.append(path)
        return cls(nodes, paths)

    def extend_leaves(self, leaves, token_indices) -> None:
        """Append one physical KV position per request (reference tree.py:75-88).

        A request that alone owns a childless leaf grows that leaf in place;
        otherwise it moves to a new private child, so private paths stay one
        compressed node each.  ``leaves`` is updated in place.
        """
        for request, token in enumerate(token_indices):
            at = leaves[request]
            node = self.nodes[at]
            if not node.children and node.requests == (request,):
                node.tokens = node.tokens + (token,)
            else:
                node.terminal.remove(request)
                new_id = len(self.nodes)
                self.nodes.append(Node(at, (token,), terminal=[request], requests=(request,)))
                node.children.append(new_id)
                leaves[request] = new_id
            self.paths[request] = self.paths[request] + (token,)

    @property
    def storage_tokens(self) -> int:
        """Number of physical KV positions (reference tree.py:90-92)."""
        return sum(len(n.tokens) for n in self.nodes)
