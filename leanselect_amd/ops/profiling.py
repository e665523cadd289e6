"""roctx ranges around the hot-path stages.

Same names as leanselect/ops/profiling.py:10-15 (``range_push``/``range_pop``).
The reference's ranges are no-ops on ROCm; here they are real roctx ranges when
torch exposes them, so rocprofv3 ``--marker-trace`` can attribute time per stage.
"""
from __future__ import annotations

import torch

__all__ = ["range_push", "range_pop"]

try:  # torch's ROCm build routes torch.cuda.nvtx to roctx
    _push = torch.cuda.nvtx.range_push
    _pop = torch.cuda.nvtx.range_pop
except Exception:  # pragma: no cover - torch without the marker bindings
    _push = _pop = None


def range_push(name: str) -> None:
    if _push is not None and torch.version.hip is not None:
        try:
            _push(name)
        except RuntimeError:
            pass


def range_pop() -> None:
    if _pop is not None and torch.version.hip is not None:
        try:
            _pop()
        except RuntimeError:
            pass
