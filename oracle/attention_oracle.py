"""CPU oracle for tree-shared decode attention -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only to check results against it (or
as the timed CPU baseline).  The product path (``tree_attention.kernels``) never
calls it and fails loudly when the HIP library is missing.

Restates the reference's FP32 oracle ``src/tree_attention/reference.py``:

* ``request_attention`` (reference.py:4-13): for every request, gather its
  path's K/V rows, expand KV heads to query heads (query head ``h`` reads KV
  head ``h // G``), FP32 softmax(q k^T / sqrt(D)) v, cast to ``q.dtype``.
* ``segmented_attention`` (reference.py:16-33): per job, FP32 attention of its
  requests over its tokens plus the row log-sum-exp; per request, weight the
  partial outputs by ``softmax(lse)`` over its jobs and sum; cast to ``q.dtype``.
* ``attention_f64`` is an independent float64 numpy restatement of the same
  textbook definition (max-shifted exponentials, explicit loops over heads),
  used to pin the two functions above on small inputs.

Pinning (what checks each function, all in ``tests/test_oracle.py``):

* ``request_attention``: float64 brute force (``attention_f64``) on the
  reference's own test trees; closed forms -- a one-token context returns that
  token's V row, equal scores return the mean of V over the path, a planted
  dominant key returns its V row.
* ``segmented_attention``: equality with ``request_attention`` for every valid
  plan of all four methods at atol = rtol = 2e-5 on the reference's test trees
  (tests/test_semantics.py:23-34), and a planted error (dropping one job)
  that the comparison catches.
* ``attention_f64``: closed forms above plus agreement with ``torch.softmax``
  attention written independently per head.
"""
from __future__ import annotations

import math

import numpy as np
import torch


def _paths(tree_or_paths):
    return tree_or_paths.paths if hasattr(tree_or_paths, "paths") else tree_or_paths


def request_attention(q, k, v, tree):
    """Per-request FP32 attention over each request's full path (reference.py:4-13).

    q: [R, HQ, D]; k, v: [T, HK, D] in physical token order; ``tree`` is a
    ``KVTree`` or any object with ``.paths`` (a list of physical id tuples).
    """
    paths = _paths(tree)
    hq, d = q.shape[1], q.shape[2]
    hk = k.shape[1]
    kv_of_head = torch.arange(hq) // (hq // hk)
    scale = 1.0 / math.sqrt(d)
    out = torch.empty((len(paths), hq, d), dtype=torch.float32)
    for r, path in enumerate(paths):
        ids = torch.as_tensor(path, dtype=torch.long)
        kr = k.index_select(0, ids).float()[:, kv_of_head, :]   # [L, HQ, D]
        vr = v.index_select(0, ids).float()[:, kv_of_head, :]
        s = torch.einsum("hd,lhd->hl", q[r].float(), kr) * scale
        out[r] = torch.einsum("hl,lhd->hd", torch.softmax(s, dim=-1), vr)
    return out.to(q.dtype)


def segmented_attention(q, k, v, plan):
    """Plan-driven FP32 attention with a global log-sum-exp merge (reference.py:16-33)."""
    hq, d = q.shape[1], q.shape[2]
    hk = k.shape[1]
    kv_of_head = torch.arange(hq) // (hq // hk)
    scale = 1.0 / math.sqrt(d)
    pieces = [[] for _ in range(q.shape[0])]
    for job in plan.jobs:
        reqs = torch.as_tensor(job.requests, dtype=torch.long)
        toks = torch.as_tensor(job.tokens, dtype=torch.long)
        qs = q.index_select(0, reqs).float()
        ks = k.index_select(0, toks).float()[:, kv_of_head, :]
        vs = v.index_select(0, toks).float()[:, kv_of_head, :]
        s = torch.einsum("rhd,lhd->rhl", qs, ks) * scale
        lse = torch.logsumexp(s, dim=-1)
        o = torch.einsum("rhl,lhd->rhd", torch.softmax(s, dim=-1), vs)
        for i, r in enumerate(job.requests):
            pieces[r].append((o[i], lse[i]))
    out = torch.empty((q.shape[0], hq, d), dtype=torch.float32)
    for r, parts in enumerate(pieces):
        o = torch.stack([p[0] for p in parts])        # [S, HQ, D]
        lse = torch.stack([p[1] for p in parts])      # [S, HQ]
        w = torch.softmax(lse, dim=0)
        out[r] = (o * w[..., None]).sum(0)
    return out.to(q.dtype)


def attention_f64(q, k, v, paths):
    """Float64 numpy attention, one (request, head) at a time; returns float64 [R, HQ, D]."""
    qn = np.asarray(q, dtype=np.float64)
    kn = np.asarray(k, dtype=np.float64)
    vn = np.asarray(v, dtype=np.float64)
    r_count, hq, d = qn.shape
    group = hq // kn.shape[1]
    out = np.zeros((r_count, hq, d))
    for r, path in enumerate(_paths(paths)):
        idx = np.asarray(path, dtype=np.int64)
        for h in range(hq):
            kk = kn[idx, h // group, :]
            vv = vn[idx, h // group, :]
            s = kk @ qn[r, h] / math.sqrt(d)
            e = np.exp(s - s.max())
            out[r, h] = (e / e.sum()) @ vv
    return out


def relative_l2(actual, expected) -> float:
    """||actual - expected||_2 / ||expected||_2 in float64 (scripts/model_checks.py:9-14)."""
    a = torch.as_tensor(actual).double()
    e = torch.as_tensor(expected).double()
    return float(torch.linalg.vector_norm(a - e) / torch.linalg.vector_norm(e))
