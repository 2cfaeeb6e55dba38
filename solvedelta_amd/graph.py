"""Fixed-shape HIP-graph training step for the SolveDelta causal LM.

Counterpart of the reference's ``SolveDeltaGraphedTrainingStep``
(causallsso/cuda_graph.py:125-331): the loss forward and its backward are
captured once as two HIP graphs (torch's ``make_graphed_callables``, which on
ROCm records hipGraphs) and replayed per step; the optimizer stays outside
the graph.  The whole path is capturable because every HIP entry point runs on
torch's current stream, takes its scratch from torch-allocated workspaces,
never synchronises and issues no memset.

Limits, as in the reference: one fixed [B, T] shape, CUDA long token ids and
labels, no masks/resets, no recurrent cache, bf16 autocast; run backward
before replaying again (graph outputs are reused).  Multi-GPU capture (DDP
after capture) is not part of this single-GPU build.
"""
from __future__ import annotations

import threading
from typing import Any, Optional

import torch
from torch import nn

from .lm import SolveDeltaForCausalLM

_CAPTURE_LOCK = threading.Lock()
_PROBE = "solvedelta_graph_probe"


def _has_live_grad_accumulator(param: torch.Tensor) -> bool:
    """True when an autograd graph still alive elsewhere (an eager loss the
    caller holds) owns ``param``'s AccumulateGrad node.  A node created here
    dies as soon as it is dropped, so a tag set on it survives the next lookup
    only when someone else holds the node."""
    node = torch.autograd.graph.get_gradient_edge(param).node
    node.metadata[_PROBE] = True
    del node
    node = torch.autograd.graph.get_gradient_edge(param).node
    alive = node.metadata.pop(_PROBE, False)
    return alive


class _LossModule(nn.Module):
    def __init__(self, model: SolveDeltaForCausalLM) -> None:
        super().__init__()
        self.model = model

    def forward(self, input_ids, labels):
        loss, _, _ = self.model(input_ids, labels=labels, use_cache=False)
        return loss


class SolveDeltaGraphedTrainingStep:
    """Calling the object replays the forward graph and returns the scalar
    loss; ``loss.backward()`` replays the backward graph."""

    def __init__(self, model: SolveDeltaForCausalLM, sample_input_ids: torch.Tensor,
                 sample_labels: torch.Tensor, *, num_warmup_iters: int = 3,
                 pool: Optional[Any] = None) -> None:
        if not isinstance(model, SolveDeltaForCausalLM):
            raise TypeError("model must be a SolveDeltaForCausalLM")
        if not model.training:
            raise ValueError("graph training capture requires model.train()")
        if isinstance(num_warmup_iters, bool) or not isinstance(num_warmup_iters, int):
            raise TypeError("num_warmup_iters must be an int")
        if num_warmup_iters < 1:
            raise ValueError("num_warmup_iters must be positive")
        self._validate_pair(sample_input_ids, sample_labels)
        if {p.device for p in model.parameters()} != {sample_input_ids.device}:
            raise ValueError("all model parameters and samples must share one device")
        for m in model.modules():
            if m._forward_hooks or m._forward_pre_hooks or m._backward_hooks:
                raise ValueError("remove module hooks before graph capture")
        # An AccumulateGrad node records the stream current when it was created.
        # A node kept alive by an earlier eager graph belongs to that graph's
        # stream (normally the default stream), and the capture's backward,
        # which runs on make_graphed_callables' private stream, would make that
        # stream wait on an event of the capture: the default stream joins the
        # capture and is never rejoined.  The reference redirects such nodes with
        # torch's stale-capture-stream override (cuda_graph.py:75-122), which
        # this torch does not have, so the capture refuses them instead.
        if any(_has_live_grad_accumulator(p) for p in model.parameters() if p.requires_grad):
            raise ValueError("an autograd graph built on the model's parameters is still alive "
                             "(an eager loss or output that was not released): release it "
                             "before graph capture")
        self.model = model
        self.device = sample_input_ids.device
        self._replay_stream = torch.cuda.current_stream(self.device)
        self.batch_size, self.sequence_length = sample_input_ids.shape
        static_ids = sample_input_ids.detach().contiguous().clone()
        static_labels = sample_labels.detach().contiguous().clone()
        loss_module = _LossModule(model).train()
        with _CAPTURE_LOCK:
            with torch.autocast(device_type="cuda", dtype=torch.bfloat16, cache_enabled=False):
                self._graphed = torch.cuda.make_graphed_callables(
                    loss_module, (static_ids, static_labels), num_warmup_iters=num_warmup_iters,
                    allow_unused_input=False, pool=pool)

    @staticmethod
    def _validate_pair(input_ids, labels):
        if input_ids.device.type != "cuda" or labels.device != input_ids.device:
            raise ValueError("input_ids and labels must share one ROCm device")
        if input_ids.ndim != 2 or labels.shape != input_ids.shape:
            raise ValueError("input_ids and labels must have the same [B,T] shape")
        if input_ids.dtype != torch.long or labels.dtype != torch.long:
            raise TypeError("input_ids and labels must have torch.long dtype")
        if input_ids.requires_grad or labels.requires_grad:
            raise ValueError("token IDs and labels must not require gradients")

    def __call__(self, input_ids: torch.Tensor, labels: torch.Tensor) -> torch.Tensor:
        self._validate_pair(input_ids, labels)
        if input_ids.shape != (self.batch_size, self.sequence_length):
            raise ValueError(f"this graph requires input shape "
                             f"{(self.batch_size, self.sequence_length)}, "
                             f"got {tuple(input_ids.shape)}")
        if input_ids.device != self.device:
            raise ValueError("input device must match the captured device")
        if torch.cuda.current_stream(self.device).cuda_stream != self._replay_stream.cuda_stream:
            raise RuntimeError("graph replay must use the stream that built this helper")
        if not self.model.training:
            raise RuntimeError("the captured model must remain in training mode")
        return self._graphed(input_ids, labels)


__all__ = ["SolveDeltaGraphedTrainingStep"]
