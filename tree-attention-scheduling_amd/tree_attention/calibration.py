"""MI355X cost-model parameters.

The reference fits its ``CostModel`` terms on Ascend 910B (schedule.py:31-39,
scripts/calibrate_tiles.py).  The values below are fitted on one MI355X by
``python -m tree_attention.calibrate`` on a calibration grid whose shapes are
disjoint from every evaluation shape; the fitted numbers are written to
``mi355x_cost_model.json`` beside this file.
"""
import json
from pathlib import Path

from .schedule import CostModel

_FITTED = Path(__file__).with_name("mi355x_cost_model.json")


def mi355x_cost_model() -> CostModel:
    """Return the fitted MI355X parameters (reference defaults if none are fitted)."""
    if _FITTED.exists():
        return CostModel(**json.loads(_FITTED.read_text())["params"])
    return CostModel()
