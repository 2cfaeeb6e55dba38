"""Recurrent state container, the same NamedTuple the reference exposes
(causallsso/reference.py:14-16): predictor C [B,H,r,r] (prediction = C u) and
memory S [B,H,r,V], both FP32 on the native path."""
from __future__ import annotations

from typing import NamedTuple

import torch

RELATIVE_FRAME_RADIUS = 5.0 / 8.0


class SolveDeltaState(NamedTuple):
    predictor: torch.Tensor
    S: torch.Tensor


def solvedelta_zero_state(batch, heads, rank, value_dim, *, dtype, device) -> SolveDeltaState:
    """Zero continuation (reference.py:19-35)."""
    return SolveDeltaState(
        torch.zeros(batch, heads, rank, rank, dtype=dtype, device=device),
        torch.zeros(batch, heads, rank, value_dim, dtype=dtype, device=device),
    )
