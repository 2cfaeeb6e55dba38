"""SolveDelta chunked recurrence on MI355X (gfx950): hand-written HIP kernels
behind the reference's ``solvedelta_native`` operator API, plus the mixer layer
around it (conv4 frontend, decay gate, gated-RMSNorm readout)."""
from .operator import solvedelta_native
from .segments import PackedSegments, build_packed_segments, solvedelta_segmented_native
from .state import RELATIVE_FRAME_RADIUS, SolveDeltaState, solvedelta_zero_state
from .mixer import (RMSNormGated, SolveDelta, SolveDeltaLayerState, SolveDeltaMixerConfig,
                    conv4_silu, kda_decay_gate)

__all__ = ["solvedelta_native", "solvedelta_segmented_native", "build_packed_segments",
           "PackedSegments", "SolveDeltaState", "solvedelta_zero_state",
           "RELATIVE_FRAME_RADIUS", "SolveDelta", "SolveDeltaLayerState",
           "SolveDeltaMixerConfig", "RMSNormGated", "conv4_silu", "kda_decay_gate"]
