"""Masks and resets without repacking or host synchronisation.

The reference runs masked / reset batches by compacting valid tokens into
reset-free segments, which needs the segment lengths on the host
(causallsso/ops/packing.py:43-150, the sync at :130-132; the operator at
ops/operator.py:96-193).  Here the dense [B,T] batch runs through the same
kernels unchanged in shape:

* an invalid token becomes neutral: u, h, q, keys, values = 0 and log-decay 0.
  Its erase read, write and readout vanish exactly (normalising a zero vector
  gives zero, so the predictor's write, the dual sources and the primal address
  are zero), so it emits 0 and keeps both states -- the reference's semantics
  (reference.py:156-227);
* a reset on a valid token zeroes both states before that token: its
  log-decay is replaced by RESET_LOG_DECAY (exp underflows to exactly 0 in
  FP32, so D C and D S vanish), and the token is flagged *fresh* for the
  kernels, which drops the predictor's erase read x = gamma u^ on it -- the
  predictor's residual is taken before forgetting (h - C_{t-1} u), so the
  decay alone would not reset it.

Gradients reach the masked operands through torch.where, so invalid tokens'
inputs and reset tokens' log-decay get zero gradient, as when the reference
leaves them out of its segments.  Everything is elementwise on the device and
capturable in a HIP graph.
"""
from __future__ import annotations

from typing import Optional

import torch

from .operator import _dispatch, _validate
from .state import SolveDeltaState

# log-decay of a reset token: exp(-200) underflows to 0 in FP32 (the smallest
# subnormal is exp(-103.3)); the kernels take any finite decay exactly
RESET_LOG_DECAY = -200.0


def _check_masks(valid_mask, reset_mask, B, T, device):
    if valid_mask is None:
        valid_mask = torch.ones(B, T, dtype=torch.bool, device=device)
    if reset_mask is None:
        reset_mask = torch.zeros(B, T, dtype=torch.bool, device=device)
    for name, m in (("valid_mask", valid_mask), ("reset_mask", reset_mask)):
        if m.shape != (B, T) or m.dtype != torch.bool:
            raise ValueError(f"{name} must be bool [B,T]")
        if m.device != device:
            raise ValueError(f"{name} must be on the activation device")
    return valid_mask, reset_mask


def solvedelta_masked_native(u, h, q, keys, values, associative_log_decay, erase_raw,
                             write_raw, geometry_write, valid_mask=None, reset_mask=None, *,
                             initial_state: Optional[SolveDeltaState] = None,
                             return_final_state: bool = False):
    """solvedelta_native with the reference's valid / reset masks
    (reference.py:156-227; the reference's segmented operator
    ops/operator.py:96-193), on the dense batch: no compaction, no host sync."""
    associative_log_decay = _validate(u, h, q, keys, values, associative_log_decay, erase_raw,
                                      write_raw, geometry_write, initial_state)
    B, T = u.shape[:2]
    valid_mask, reset_mask = _check_masks(valid_mask, reset_mask, B, T, u.device)
    reset = reset_mask & valid_mask
    m4 = valid_mask[:, :, None, None]
    m5 = valid_mask[:, :, None, None, None]
    zero = lambda x: torch.where(m4 if x.ndim == 4 else m5, x, torch.zeros((), dtype=x.dtype,
                                                                           device=x.device))
    u, h, q = zero(u), zero(h), zero(q)
    keys, values, erase_raw, write_raw = zero(keys), zero(values), zero(erase_raw), zero(write_raw)
    g = torch.where(reset[:, :, None, None],
                    torch.full((), RESET_LOG_DECAY, dtype=torch.float32, device=u.device),
                    zero(associative_log_decay))
    fresh = reset.to(torch.uint8)
    return _dispatch(u, h, q, keys, values, g, erase_raw, write_raw, geometry_write,
                     initial_state, return_final_state, fresh)


__all__ = ["RESET_LOG_DECAY", "solvedelta_masked_native"]
