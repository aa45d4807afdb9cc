"""ctypes binding of ``libtree_plan.so``, the host planner library (include/tree_plan.h).

``grouped_decisions`` hands the tree to ``tp_grouped_plan`` in CSR form and
returns, per node, whether its parent pushes it (the subset-DP / greedy
decision of the reference's schedule.py:94-131).  ``attach_tails`` runs the
tail-attachment step of ``kernels.prepare`` (``tp_attach_tails``) and
``build_metadata`` its device metadata (``tp_build_metadata``).  The
library is a plain host library (g++), loaded on first use; ``TREE_PLAN_LIB``
selects another build.
"""
from __future__ import annotations

import ctypes
import os
import threading
from itertools import chain
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).with_name("libtree_plan.so")
EXPORTS = ("tp_grouped_plan", "tp_attach_tails", "tp_build_metadata")
METHODS = {"greedy": 0, "cube": 1}

_lib = None
_missing = False
_lock = threading.Lock()
_p = ctypes.c_void_p


def load(required: bool = True):
    """Return the loaded library; ``None`` if it is not built and not ``required``."""
    global _lib, _missing
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            target = Path(os.environ.get("TREE_PLAN_LIB", LIB_PATH))
            if not target.exists():
                _missing = True
                if required:
                    raise RuntimeError(f"planner library not found at {target}; build it with "
                                       "`python tree-attention-scheduling_amd/csrc/build.py`")
                return None
            lib = ctypes.CDLL(str(target))
            lib.tp_grouped_plan.restype = ctypes.c_int
            lib.tp_grouped_plan.argtypes = [ctypes.c_int32, ctypes.c_int32] + [_p] * 11
            i32 = ctypes.c_int32
            lib.tp_attach_tails.restype = ctypes.c_int
            lib.tp_attach_tails.argtypes = ([i32, _p, _p, _p, _p, i32, i32, _p, _p, _p, _p, i32, i32, i32, i32, i32]
                                            + [_p] * 5)
            lib.tp_build_metadata.restype = ctypes.c_int
            lib.tp_build_metadata.argtypes = [i32, i32, _p, _p, _p, _p, i32, i32, i32, i32, i32, _p, _p, _p, i32,
                                              _p, _p, ctypes.c_int64]
            _lib = lib
    return _lib


def available() -> bool:
    return load(required=False) is not None


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(_p)


def grouped_decisions(tree, method: str, model, qheads: int, kvheads: int, dim: int, node_runs):
    """Per-node push flags and the root estimate from the native planner.

    ``node_runs[v]`` are node v's tokens as ``((start, length), ...)`` runs.
    """
    lib = load()
    nodes = tree.nodes
    n = len(nodes)
    parent = np.fromiter((nd.parent for nd in nodes), dtype=np.int32, count=n)
    child_off = np.zeros(n + 1, dtype=np.int32)
    np.cumsum([len(nd.children) for nd in nodes], out=child_off[1:])
    child_idx = np.fromiter((c for nd in nodes for c in nd.children), dtype=np.int32, count=int(child_off[-1]))
    nreq = np.fromiter((len(nd.requests) for nd in nodes), dtype=np.int32, count=n)
    run_off = np.zeros(n + 1, dtype=np.int64)
    np.cumsum([len(r) for r in node_runs], out=run_off[1:])
    flat = np.array([x for r in node_runs for run in r for x in run], dtype=np.int64).reshape(-1, 2)
    run_start = np.ascontiguousarray(flat[:, 0]) if len(flat) else np.zeros(1, np.int64)
    run_len = np.ascontiguousarray(flat[:, 1]) if len(flat) else np.zeros(1, np.int64)
    fparams = np.array([model.bandwidth, model.cube_flops, model.task_us, model.merge_us], dtype=np.float64)
    iparams = np.array([model.cube_rows, model.key_tile, model.kv_split, model.max_query_rows,
                        qheads, kvheads, dim], dtype=np.int64)
    pushed = np.zeros(n, dtype=np.int8)
    total = np.zeros(1, dtype=np.float64)
    if len(child_idx) == 0:
        child_idx = np.zeros(1, dtype=np.int32)
    rc = lib.tp_grouped_plan(METHODS[method], n, _ptr(parent), _ptr(child_off), _ptr(child_idx), _ptr(nreq),
                             _ptr(run_off), _ptr(run_start), _ptr(run_len), _ptr(fparams), _ptr(iparams),
                             _ptr(pushed), _ptr(total))
    if rc != 0:
        raise ValueError(f"tp_grouped_plan rejected its arguments (code {rc})")
    return pushed, float(total[0])


def attach_tails(large, small, group, is256, large_tiles, small_tiles, fixed, nreq, xtail_max, wave_rows,
                 item_rows, min_cap):
    """``tp_attach_tails`` over job lists; returns (item per candidate job or -1, its first row, item keys)."""
    lib = load()
    nl, ns = len(large), len(small)
    req_off = np.zeros(nl + 1, dtype=np.int32)
    np.cumsum([len(j.requests) for j in large], out=req_off[1:])
    req = np.fromiter(chain.from_iterable(j.requests for j in large), dtype=np.int32, count=int(req_off[-1]))
    is256 = np.asarray(is256, dtype=np.int32)
    tiles = np.asarray(large_tiles, dtype=np.int32)
    sreq_off = np.zeros(ns + 1, dtype=np.int32)
    np.cumsum([len(j.requests) for j in small], out=sreq_off[1:])
    sreq = np.fromiter(chain.from_iterable(j.requests for j in small), dtype=np.int32, count=int(sreq_off[-1]))
    tiles_s = np.asarray(small_tiles, dtype=np.int32)
    fixed = np.asarray(fixed, dtype=np.int8)
    cap = int(sum(-(-len(j.requests) * group // item_rows) for j, b in zip(large, is256) if b))
    item = np.zeros(max(ns, 1), dtype=np.int32)
    lrow = np.zeros(max(ns, 1), dtype=np.int32)
    item_job = np.zeros(max(cap, 1), dtype=np.int32)
    item_row0 = np.zeros(max(cap, 1), dtype=np.int32)
    n_items = np.zeros(1, dtype=np.int32)
    one = np.zeros(1, dtype=np.int32)
    ptr = lambda a: _ptr(a if a.size else one)  # noqa: E731
    rc = lib.tp_attach_tails(nl, ptr(is256), ptr(tiles), _ptr(req_off), ptr(req), group, ns, _ptr(sreq_off), ptr(sreq),
                             ptr(tiles_s), _ptr(fixed if fixed.size else np.zeros(1, np.int8)), nreq, xtail_max,
                             wave_rows, item_rows, min_cap, _ptr(item), _ptr(lrow), _ptr(item_job), _ptr(item_row0),
                             _ptr(n_items))
    if rc != 0:
        raise ValueError(f"tp_attach_tails rejected its arguments (code {rc})")
    keys = list(zip(item_job[:n_items[0]].tolist(), item_row0[:n_items[0]].tolist()))
    return item[:ns].tolist(), lrow[:ns].tolist(), keys


def build_metadata(qlen, req, kstart, klen, small_jobs, nreq, group, kvheads, tile_rows, att_job, att_row0, att_rec,
                   xstride):
    """``tp_build_metadata``: (sizes, one int32 buffer of every metadata section)."""
    lib = load()
    one = np.zeros(1, dtype=np.int32)
    ptr = lambda a: _ptr(a if a.size else one)  # noqa: E731
    sizes = np.zeros(13, dtype=np.int32)
    args = (len(qlen), small_jobs, ptr(qlen), ptr(req), ptr(kstart), ptr(klen), nreq, group, kvheads, tile_rows,
            len(att_job), ptr(att_job), ptr(att_row0), ptr(np.ascontiguousarray(att_rec).reshape(-1)), xstride,
            _ptr(sizes))
    if lib.tp_build_metadata(*args, None, 0) != 0:
        raise ValueError("tp_build_metadata rejected its arguments")
    buf = np.empty(int(sizes[11]), dtype=np.int32)
    if lib.tp_build_metadata(*args, _ptr(buf), buf.size) != 0:
        raise ValueError("tp_build_metadata rejected its arguments")
    return sizes.tolist(), buf
