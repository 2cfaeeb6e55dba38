"""The reference's packed-segment API for masks and resets, run on the dense
masked path.

The reference compacts each batch row's valid tokens into reset-free segments,
runs them as one padded native batch and scatters the outputs back
(causallsso/ops/packing.py:43-150, causallsso/ops/operator.py:96-193).  Its plan
object and the two entry points are kept here for their callers, but nothing is
compacted: ``solvedelta_segmented_native`` turns the plan back into the [B,T]
valid / reset flags it was built from and runs ``solvedelta_masked_native``, the
dense masked operator (invalid tokens neutral, resets as a killed decay plus a
fresh predictor read), so the operator itself needs no host sync and keeps
static shapes.  Only building the plan reads its segment lengths back to the
host, as the reference's does (packing.py:130-132), because the plan carries
``cu_seqlens_cpu``.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from .masks import solvedelta_masked_native
from .state import SolveDeltaState


@dataclass(frozen=True)
class PackedSegments:
    """Reset-free segments of a [batch, length] masked batch (packing.py:27-40).
    A segment is a maximal run of a row's valid tokens with a reset only on its
    first token; ``indices`` are the valid tokens' flat positions in row-major
    order, segment by segment."""
    batch: int
    length: int
    indices: torch.Tensor            # [N] flat positions b*length + t of valid tokens
    segment_ids: torch.Tensor        # [N] segment of each valid token
    segment_batch: torch.Tensor      # [S] batch row of each segment
    use_initial: torch.Tensor        # [S] segment starts from the row's initial state
    segment_lengths: torch.Tensor    # [S] int32
    cu_seqlens: torch.Tensor         # [S+1] cumulative lengths (device)
    cu_seqlens_cpu: torch.Tensor     # [S+1] the same on the host
    segment_batch_cpu: torch.Tensor  # [S] host copy of segment_batch
    use_initial_cpu: torch.Tensor    # [S] host copy of use_initial
    last_segment: torch.Tensor       # [batch] last segment of each row, -1 for none

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
        return int((self.cu_seqlens_cpu[1:] - self.cu_seqlens_cpu[:-1]).max())


def build_packed_segments(valid_mask: torch.Tensor, reset_mask: torch.Tensor) -> PackedSegments:
    """The segment plan of a masked batch (packing.py:43-150: same fields, same
    errors).  Worked out on the dense [B,T] grid: a valid token opens a segment
    when it is its row's first valid token or a valid reset; a segment inherits
    the row's initial state when it opens on the row's first valid token
    without a reset."""
    if valid_mask.ndim != 2 or valid_mask.dtype != torch.bool:
        raise ValueError("valid_mask must be bool [B,T]")
    if reset_mask.shape != valid_mask.shape or reset_mask.dtype != torch.bool:
        raise ValueError("reset_mask must be bool [B,T]")
    if reset_mask.device != valid_mask.device:
        raise ValueError("valid_mask and reset_mask must share one device")
    B, T = valid_mask.shape
    dev = valid_mask.device
    row_first = valid_mask & (valid_mask.long().cumsum(1) == 1)      # first valid token of its row
    opens = valid_mask & (row_first | reset_mask)                    # opens a segment
    inherits = row_first & ~reset_mask                               # ... from the initial state
    indices = valid_mask.reshape(-1).nonzero().flatten()
    opens_at = opens.reshape(-1).index_select(0, indices)
    segment_ids = opens_at.long().cumsum(0) - 1
    starts = opens.reshape(-1).nonzero().flatten()                  # flat positions of openings
    S = int(starts.numel())
    segment_batch = torch.div(starts, T, rounding_mode="floor")
    use_initial = inherits.reshape(-1).index_select(0, starts)
    lengths = torch.bincount(segment_ids, minlength=S).to(torch.int32) if S else \
        torch.empty(0, dtype=torch.int32, device=dev)
    per_row = opens.long().sum(1)
    last_segment = torch.where(per_row > 0, per_row.cumsum(0) - 1, torch.full_like(per_row, -1))
    host = torch.stack((lengths.long(), segment_batch, use_initial.long()), 0).cpu()
    cu_cpu = torch.zeros(S + 1, dtype=torch.long)
    cu_cpu[1:] = host[0].cumsum(0)
    return PackedSegments(B, T, indices, segment_ids, segment_batch, use_initial, lengths,
                          cu_cpu.to(dev), cu_cpu, host[1].clone(), host[2].bool(), last_segment)


def plan_masks(plan: PackedSegments, device) -> tuple[torch.Tensor, torch.Tensor]:
    """The [B,T] valid and reset flags a plan describes: valid on its tokens,
    reset on the first token of every segment that does not inherit the row's
    initial state."""
    n = plan.batch * plan.length
    valid = torch.zeros(n, dtype=torch.bool, device=device)
    valid.index_fill_(0, plan.indices.to(device), True)
    first_token = plan.indices.index_select(0, plan.cu_seqlens[:-1]).to(device) \
        if plan.num_segments else plan.indices.new_empty(0).to(device)
    fresh = ~plan.use_initial.to(device)
    reset = torch.zeros(n, dtype=torch.bool, device=device)
    reset.index_put_((first_token,), fresh)
    return valid.view(plan.batch, plan.length), reset.view(plan.batch, plan.length)


def solvedelta_segmented_native(u, h, q, keys, values, associative_log_decay, erase_raw, write_raw,
                                geometry_write, plan: PackedSegments, *,
                                initial_state: Optional[SolveDeltaState] = None,
                                return_final_state: bool = False):
    """The segmented operator (ops/operator.py:96-193): outputs are zero on
    invalid tokens, each segment runs from its row's initial state or from zero,
    and a row's final state is its last segment's (the initial state when the row
    has no valid token).  Runs as the dense masked operator on the plan's masks."""
    B, T = u.shape[:2]
    if (plan.batch, plan.length) != (B, T):
        raise ValueError("packed segment plan does not match the operator input")
    valid, reset = plan_masks(plan, u.device)
    return solvedelta_masked_native(u, h, q, keys, values, associative_log_decay, erase_raw,
                                    write_raw, geometry_write, valid, reset,
                                    initial_state=initial_state,
                                    return_final_state=return_final_state)


__all__ = ["PackedSegments", "build_packed_segments", "plan_masks", "solvedelta_segmented_native"]
