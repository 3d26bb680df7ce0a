"""Reproducible-backward switch for the Relation path (the interface of mote/determinism.py:41-62).

What varies between two identical backward passes here:
* the bf16 tile backward (every preset) never varies: it has no atomics, and dlam is summed in a fixed
  order by one workgroup;
* the fp32 and padded-head-dim backward adds dP1 with fp32 atomics unless `DETERMINISTIC` is set,
  which selects the query-stationary pass instead;
* library GEMMs around the path (projections, `wo`) follow torch's deterministic-algorithms mode.

`apply(reproducible)` sets all three the way the reference's switch does: the environment variable
MOTE_DETERMINISTIC_RELATION, the already-imported module flag, and torch's process-wide mode with
warn_only (an op without a deterministic implementation warns instead of failing). `state()` is the
record a run keeps of its mode.
"""

from __future__ import annotations

import os

import torch

WORKSPACE = ":4096:8"  # the fixed GEMM workspace torch asks for in deterministic mode


def apply(reproducible: bool = True) -> None:
    """Enter (or leave) the reproducible configuration for this process."""
    os.environ["CUBLAS_WORKSPACE_CONFIG"] = WORKSPACE
    os.environ["MOTE_DETERMINISTIC_RELATION"] = "1" if reproducible else "0"
    from . import flash_relation

    flash_relation.DETERMINISTIC = bool(reproducible)
    torch.use_deterministic_algorithms(bool(reproducible), warn_only=True)


def state() -> dict:
    """The mode a run should record: numbers are comparable only within one mode."""
    from . import flash_relation

    return {
        "reproducible": bool(torch.are_deterministic_algorithms_enabled()),
        "relation_backward": "two-pass" if flash_relation.DETERMINISTIC else "atomics",
        "relation_backward_bf16": "tiles (atomic-free)",
        "cublas_workspace": os.environ.get("CUBLAS_WORKSPACE_CONFIG"),
    }
