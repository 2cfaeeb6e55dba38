"""SolveDelta chunked recurrence on MI355X (gfx950): hand-written HIP kernels
behind the reference's ``solvedelta_native`` operator API, plus the mixer layer
around it (conv4 frontend, decay gate, gated-RMSNorm readout), the
recurrent cache, a causal LM shell and the Hugging Face ``SolveDeltaConfig``."""
from .operator import solvedelta_native
from .segments import PackedSegments, build_packed_segments, solvedelta_segmented_native
from .masks import solvedelta_masked_native
from .state import RELATIVE_FRAME_RADIUS, SolveDeltaState, solvedelta_zero_state
from .mixer import (RMSNormGated, SolveDelta, SolveDeltaLayerState, SolveDeltaMixerConfig,
                    conv4_silu, kda_decay_gate)

_LAZY = {"SolveDeltaConfig": ".config", "SolveDeltaForCausalLM": ".lm",
         "SolveDeltaModel": ".lm", "SolveDeltaGraphedTrainingStep": ".graph"}


def __getattr__(name):
    # transformers (behind SolveDeltaConfig) is imported only when asked for
    if name in _LAZY:
        import importlib
        return getattr(importlib.import_module(_LAZY[name], __name__), name)
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")


__all__ = ["solvedelta_native", "solvedelta_segmented_native", "solvedelta_masked_native",
           "build_packed_segments",
           "PackedSegments", "SolveDeltaState", "solvedelta_zero_state",
           "RELATIVE_FRAME_RADIUS", "SolveDelta", "SolveDeltaLayerState",
           "SolveDeltaMixerConfig", "RMSNormGated", "conv4_silu", "kda_decay_gate",
           *_LAZY]
