"""ctypes binding of ``libtree_plan.so``, the host grouped planner (include/tree_plan.h).

``grouped_decisions`` hands the tree to ``tp_grouped_plan`` in CSR form and
returns, per node, whether its parent pushes it (the subset-DP / greedy
decision of the reference's schedule.py:94-131).  The library is a plain host
library (g++), loaded on first use; ``TREE_PLAN_LIB`` selects another build.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).with_name("libtree_plan.so")
EXPORTS = ("tp_grouped_plan",)
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
