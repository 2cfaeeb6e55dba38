"""SolveDelta chunked recurrence on MI355X (gfx950): hand-written HIP kernels
behind the reference's ``solvedelta_native`` operator API."""
from .operator import solvedelta_native
from .segments import PackedSegments, build_packed_segments, solvedelta_segmented_native
from .state import RELATIVE_FRAME_RADIUS, SolveDeltaState, solvedelta_zero_state

__all__ = ["solvedelta_native", "solvedelta_segmented_native", "build_packed_segments",
           "PackedSegments", "SolveDeltaState", "solvedelta_zero_state",
           "RELATIVE_FRAME_RADIUS"]
