"""Masks and resets without repacking or host synchronisation.

The reference runs masked / reset batches by compacting valid tokens into
reset-free segments, which needs the segment lengths on the host
(causallsso/ops/packing.py:43-150, the sync at :130-132; the operator at
ops/operator.py:96-193).  Here the dense [B,T] batch runs through the same
kernels unchanged in shape:

* an invalid token becomes neutral: its gamma, q, keys and log-decay are zeroed.
  gamma = 0 makes the predictor's write delta = gamma (h - C u) and its erase
  read x = gamma u^ vanish (so the dual sources' phi, and with keys = 0 the
  primal address d = k + C^T k and the erase source e, are zero: no memory
  write), q = 0 makes the readout vanish, and log-decay 0 keeps both states: the
  token emits 0 and leaves both states as they were -- the reference's
  semantics (reference.py:156-227).  u, h and the values need no masking: each
  of their effects passes through delta, x, d or the token's write, all zero,
  so their gradients on the token are exactly zero as well (they, like the
  gate logits, must be finite there: zero times a NaN is not zero);
* a reset on a valid token clears both states before that token: its
  log-decay is replaced by RESET_LOG_DECAY, so D C and D S keep exp(-20) ~
  2.1e-9 of the old states, where the reference keeps none (below FP32
  rounding, 6e-8, of the terms that follow while the old state is at most ~30x
  their size; a relative error of ~1e-3 with an old state 1e5x the later
  writes) -- while the chunk kernels keep the token on their factored
  (matrix-core) decay path: a 16-token block whose decay exceeds their wild
  threshold of 60 (an exact exp(-inf) kill would, and so would three such
  resets in one block) takes the exact per-coordinate fix-up, several times
  slower, and the slowest block sets each round's time.  The token is also flagged *fresh* for the
  kernels, which drops the predictor's erase read x = gamma u^ on it exactly --
  the predictor's residual is taken before forgetting (h - C_{t-1} u), so the
  decay alone would not reset it.

The masking is one HIP launch for the per-token flags (sd_mask_flags) and one
in the backward (sd_mask_rows).  The kernels read q, keys, the log-decay and
gamma through the token flags they take as their `fresh` input
(include/solvedelta.h: SD_TOK_INVALID reads the token's q, keys, gamma and
log-decay as 0, SD_TOK_RESET its log-decay as RESET_LOG_DECAY, SD_TOK_FRESH
drops its erase read), so the forward copies nothing; the backward zeroes the
same rows of those operands' gradients in place (one wave per token, writing
only the rows that change) and the reset tokens' log-decay gradient, so invalid
tokens' inputs and reset tokens' log-decay get zero gradient, as when the
reference leaves them out of its segments.  erase_raw and write_raw need no
masking either: their partners on an invalid token (the key, and the write
through d) are zero.  Everything stays on the device and is capturable in a
HIP graph.
"""
from __future__ import annotations

from typing import Optional

import ctypes

import torch

from . import _lib
from .operator import _dispatch, _stream, _validate
from .state import SolveDeltaState

# log-decay of a reset token: the old states survive as exp(-20) ~ 2.1e-9 of
# their value (the reference zeroes them); two resets and up
# to 20 of ordinary decay fit in one 16-token block before it leaves the
# kernels' factored path (see the module docstring for why not an exact kill)
RESET_LOG_DECAY = -20.0


def _check_masks(valid_mask, reset_mask, B, T, device):
    for name, m in (("valid_mask", valid_mask), ("reset_mask", reset_mask)):
        if m is None:
            continue
        if m.shape != (B, T) or m.dtype != torch.bool:
            raise ValueError(f"{name} must be bool [B,T]")
        if m.device != device:
            raise ValueError(f"{name} must be on the activation device")
    return valid_mask, reset_mask


def _flags(valid_mask, reset_mask, B, T, device):
    """uint8 [B,T] flags (bit 0 valid, bit 1 valid reset) and fresh flags (1 on
    valid resets) in one launch (sd_mask_flags); a None mask is all-valid / no-reset."""
    flags = torch.empty(B, T, dtype=torch.uint8, device=device)
    fresh = torch.empty(B, T, dtype=torch.uint8, device=device)
    args = []
    for m in (valid_mask, reset_mask):
        args += [0, 0, 0] if m is None else [m.data_ptr(), m.stride(0), m.stride(1)]
    rc = _lib.load().sd_mask_flags(B, T, *args, flags.data_ptr(), fresh.data_ptr(),
                                   _stream(device))
    _lib.check(rc, "sd_mask_flags")
    return flags, fresh


def _mask_tensor(src: torch.Tensor, dst: torch.Tensor, reset_fill: bool, reset_value: float):
    return _lib.SdMaskTensor(src.data_ptr(), src.stride(0), src.stride(1), src.stride(2),
                             dst.data_ptr(), src.shape[-1], int(src.dtype == torch.float32),
                             int(reset_fill), reset_value)


def _mask_rows(flags, srcs, decay_idx, reset_value: float, inplace: bool = False):
    """Masked contiguous copies of srcs ([B,T,H,...,w] views, unit inner stride),
    or, with inplace, srcs themselves masked in place (each must be contiguous);
    srcs[decay_idx] (if not None) is the log-decay or its gradient, whose reset
    rows take reset_value."""
    B, T, H = srcs[0].shape[:3]
    outs = list(srcs) if inplace else [torch.empty(x.shape, dtype=x.dtype, device=x.device)
                                       for x in srcs]
    arr = (_lib.SdMaskTensor * len(srcs))(*[
        _mask_tensor(x, o, i == decay_idx, reset_value)
        for i, (x, o) in enumerate(zip(srcs, outs))])
    rc = _lib.load().sd_mask_rows(B, T, H, flags.data_ptr(), flags.stride(0), flags.stride(1),
                                  arr, len(srcs), _stream(srcs[0].device))
    _lib.check(rc, "sd_mask_rows")
    return outs


_DECAY = 2  # position of the log-decay among the masked operands


class _MaskGrads(torch.autograd.Function):
    """q, keys, log-decay, gamma ([B,T,H,1]) pass through unchanged (views: the
    kernels read them masked through the token flags); the backward zeroes the
    gradients of invalid tokens' rows and reset tokens' log-decay rows."""

    @staticmethod
    def forward(ctx, flags, q, keys, log_decay, gamma):
        ctx.save_for_backward(flags)
        return q.view_as(q), keys.view_as(keys), log_decay.view_as(log_decay), gamma.view_as(gamma)

    @staticmethod
    def backward(ctx, *grads):
        (flags,) = ctx.saved_tensors
        live = [i for i, g in enumerate(grads) if g is not None]
        out = [None] * len(grads)
        if live:
            # The incoming gradients are this function's alone (its outputs feed
            # only the operator), so they are masked in place: only invalid rows
            # (and reset tokens' log-decay rows) are written.
            srcs = [grads[i].contiguous() for i in live]
            decay = live.index(_DECAY) if _DECAY in live else None
            masked = _mask_rows(flags, srcs, decay, 0.0, inplace=True)
            for i, m in zip(live, masked):
                out[i] = m
        return (None, *out)


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
    flags, fresh = _flags(valid_mask, reset_mask, B, T, u.device)
    H = u.shape[2]
    gamma = geometry_write if geometry_write.dim() == 3 else geometry_write.reshape(1, 1, H)
    gamma = gamma.expand(B, T, H).unsqueeze(-1)
    q, keys, g, gamma = _MaskGrads.apply(flags, q, keys, associative_log_decay, gamma)
    return _dispatch(u, h, q, keys, values, g, erase_raw, write_raw, gamma.squeeze(-1),
                     initial_state, return_final_state, fresh)


__all__ = ["RESET_LOG_DECAY", "solvedelta_masked_native"]
