"""Tree-shared decode attention for MI355X (gfx950).

Public names match the reference package (``src/tree_attention/__init__.py:1-2``):
``KVTree``, ``CostModel``, ``Plan`` and ``schedule``.  The HIP backend lives in
``tree_attention.kernels`` and is loaded on first use, so importing this
package needs neither a GPU nor the native library.
"""
from .tree import KVTree
from .schedule import CostModel, Plan, schedule

__all__ = ["KVTree", "CostModel", "Plan", "schedule"]
