"""Masks and resets: reset-free segment packing around the native operator.

Mirrors the reference's ``build_packed_segments`` / ``solvedelta_segmented_native``
(causallsso/ops/packing.py:43-150, causallsso/ops/operator.py:96-193): valid
tokens are compacted per batch row and split at valid resets into independent
segments; the segments run as one neutral-padded batch through
``solvedelta_native`` and the outputs are scattered back (invalid positions stay
zero).  The first segment of a row inherits the row's initial state unless it
starts with a reset; the final state of a row is that of its last segment (or
the initial state when the row has no valid token).

A reset cannot be folded into the kernels as an infinite decay: the predictor's
residual is taken against the state *before* forgetting, so a reset has to start
a new sequence.  Planning needs one small device-to-host copy (segment lengths),
as in the reference (packing.py:130-132).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from .operator import solvedelta_native
from .state import SolveDeltaState


@dataclass(frozen=True)
class PackedSegments:
    batch: int
    length: int
    indices: torch.Tensor        # flat [B*T] positions of valid tokens, row-major
    segment_ids: torch.Tensor    # segment of each valid token
    segment_batch: torch.Tensor  # batch row of each segment
    use_initial: torch.Tensor    # segment inherits the row's initial state
    segment_lengths: torch.Tensor
    cu_seqlens: torch.Tensor
    cu_seqlens_cpu: torch.Tensor
    last_segment: torch.Tensor   # last segment of each row, -1 if none

    @property
    def num_tokens(self) -> int:
        return int(self.indices.shape[0])

    @property
    def num_segments(self) -> int:
        return int(self.segment_batch.shape[0])

    @property
    def max_seqlen(self) -> int:
        if self.num_segments == 0:
            return 0
        return int(torch.diff(self.cu_seqlens_cpu).max().item())


def build_packed_segments(valid_mask: torch.Tensor, reset_mask: torch.Tensor) -> PackedSegments:
    """Reset-free segment plan (packing.py:43-150 semantics, own implementation)."""
    if valid_mask.ndim != 2 or valid_mask.dtype != torch.bool:
        raise ValueError("valid_mask must be bool [B,T]")
    if reset_mask.shape != valid_mask.shape or reset_mask.dtype != torch.bool:
        raise ValueError("reset_mask must be bool [B,T]")
    if reset_mask.device != valid_mask.device:
        raise ValueError("valid_mask and reset_mask must share one device")
    B, T = valid_mask.shape
    dev = valid_mask.device
    indices = torch.nonzero(valid_mask.reshape(-1), as_tuple=False).flatten()
    if indices.numel() == 0:
        cu = torch.zeros(1, dtype=torch.long)
        e = torch.empty(0, dtype=torch.long, device=dev)
        return PackedSegments(B, T, indices, e, e, torch.empty(0, dtype=torch.bool, device=dev),
                              torch.empty(0, dtype=torch.int32, device=dev), cu.to(dev), cu,
                              torch.full((B,), -1, dtype=torch.long, device=dev))
    row = indices // T
    reset_valid = reset_mask.reshape(-1)[indices]
    starts = torch.ones_like(reset_valid)
    starts[1:] = (row[1:] != row[:-1]) | reset_valid[1:]
    segment_ids = torch.cumsum(starts.long(), 0) - 1
    start_pos = torch.nonzero(starts, as_tuple=False).flatten()
    segment_batch = row[start_pos]
    end_pos = torch.cat((start_pos[1:], start_pos.new_full((1,), indices.numel())))
    lengths = (end_pos - start_pos).to(torch.int32)
    first_in_row = torch.ones_like(segment_batch, dtype=torch.bool)
    first_in_row[1:] = segment_batch[1:] != segment_batch[:-1]
    use_initial = first_in_row & ~reset_valid[start_pos]
    seg_no = torch.arange(segment_batch.numel(), device=dev)
    last_segment = torch.full((B,), -1, dtype=torch.long, device=dev).scatter_reduce(
        0, segment_batch, seg_no, reduce="amax", include_self=True)
    lengths_cpu = lengths.long().cpu()
    cu_cpu = torch.zeros(lengths_cpu.numel() + 1, dtype=torch.long)
    cu_cpu[1:] = torch.cumsum(lengths_cpu, 0)
    return PackedSegments(B, T, indices, segment_ids, segment_batch, use_initial, lengths,
                          cu_cpu.to(dev), cu_cpu, last_segment)


def _to_segments(x: torch.Tensor, plan: PackedSegments, padded: int) -> torch.Tensor:
    """[B,T,...] -> [S,padded,...] with valid tokens compacted, zeros elsewhere."""
    flat = x.reshape(plan.batch * plan.length, *x.shape[2:])
    actual = flat.index_select(0, plan.indices)
    pos = torch.arange(plan.num_tokens, device=x.device) - plan.cu_seqlens[plan.segment_ids]
    dest = plan.segment_ids * padded + pos
    out = actual.new_zeros(plan.num_segments * padded, *x.shape[2:])
    out = out.index_copy(0, dest, actual)
    return out.view(plan.num_segments, padded, *x.shape[2:])


def _from_segments(y: torch.Tensor, plan: PackedSegments) -> torch.Tensor:
    padded = y.shape[1]
    pos = torch.arange(plan.num_tokens, device=y.device) - plan.cu_seqlens[plan.segment_ids]
    src = plan.segment_ids * padded + pos
    actual = y.reshape(plan.num_segments * padded, *y.shape[2:]).index_select(0, src)
    out = actual.new_zeros(plan.batch * plan.length, *y.shape[2:])
    out = out.index_copy(0, plan.indices, actual)
    return out.view(plan.batch, plan.length, *y.shape[2:])


def solvedelta_segmented_native(u, h, q, keys, values, associative_log_decay, erase_raw, write_raw,
                                geometry_write, plan: PackedSegments, *,
                                initial_state: Optional[SolveDeltaState] = None,
                                return_final_state: bool = False):
    """Run reset-free packed segments as one neutral-padded native batch
    (ops/operator.py:96-193)."""
    B, T, H, r = u.shape
    V = values.shape[-1]
    if (plan.batch, plan.length) != (B, T):
        raise ValueError("packed segment plan does not match the operator input")
    if plan.num_tokens == 0:
        out = values.new_zeros(B, T, H, V)
        if not return_final_state:
            return out, None
        if initial_state is not None:
            return out, initial_state
        return out, SolveDeltaState(
            torch.zeros(B, H, r, r, dtype=torch.float32, device=u.device),
            torch.zeros(B, H, r, V, dtype=torch.float32, device=u.device))
    padded = plan.max_seqlen
    gw = geometry_write
    if gw.shape == (B, T, H):
        gw = _to_segments(gw, plan, padded)
    seg = [_to_segments(x, plan, padded) for x in (u, h, q, keys, values, associative_log_decay,
                                                   erase_raw, write_raw)]
    seg_init = None
    if initial_state is not None:
        initial_state = SolveDeltaState(*initial_state)
        keep = plan.use_initial[:, None, None, None]
        C0 = initial_state.predictor.index_select(0, plan.segment_batch)
        S0 = initial_state.S.index_select(0, plan.segment_batch)
        seg_init = SolveDeltaState(torch.where(keep, C0, torch.zeros_like(C0)),
                                   torch.where(keep, S0, torch.zeros_like(S0)))
    out_seg, fin = solvedelta_native(*seg, gw, initial_state=seg_init,
                                     return_final_state=return_final_state)
    out = _from_segments(out_seg, plan)
    if not return_final_state:
        return out, None
    has = (plan.last_segment >= 0)[:, None, None, None]
    sel = plan.last_segment.clamp_min(0)
    C = fin.predictor.index_select(0, sel)
    S = fin.S.index_select(0, sel)
    if initial_state is None:
        C0, S0 = torch.zeros_like(C), torch.zeros_like(S)
    else:
        C0, S0 = initial_state.predictor, initial_state.S
    return out, SolveDeltaState(torch.where(has, C, C0), torch.where(has, S, S0))


__all__ = ["PackedSegments", "build_packed_segments", "solvedelta_segmented_native"]
