"""Recurrent-cache wire format and the cache-owning layer adapter.

Mirrors the reference's cache ABI around the mixer
(causallsso/modeling_solvedelta.py:104-195): each SolveDelta layer's cache
entry is a dict

    {"recurrent_state": (C [B,H,r,r] fp32, S [B,H,r,V] fp32),
     "conv_state":      [B, 2*H*r + H*V, 3] (activation dtype) or None,
     ...}

and the layer adapter reads it into ``SolveDeltaLayerState``, runs the mixer
(T = 1 calls take the decode kernel) and writes the final state back with the
call's token count as offset.

The reference keeps these dicts in flash-linear-attention 0.6.0's
``fla.models.utils.Cache`` (its ``update(recurrent_state=, conv_state=,
layer_idx=, offset=)``, per-layer indexing and ``get_seq_length``), which is
not available on ROCm here; ``RecurrentCache`` restates that part of its
interface: the first layer's updates advance the seen-token count, and legacy
caches are lists of the per-layer dicts.
"""
from __future__ import annotations

from typing import Any, Iterator, Optional

import torch
from torch import nn

from .mixer import SolveDelta, SolveDeltaLayerState
from .state import SolveDeltaState


class RecurrentCache:
    """Per-layer recurrent state store with fla's Cache update / lookup API."""

    def __init__(self, seen_tokens: int = 0) -> None:
        self.states: list[dict[str, Any]] = []
        self._seen_tokens = seen_tokens

    def __getitem__(self, layer_idx: int) -> dict[str, Any]:
        if layer_idx < len(self.states):
            return self.states[layer_idx]
        raise KeyError(f"cache has {len(self.states)} layers, asked for layer {layer_idx}")

    def __iter__(self) -> Iterator[dict[str, Any]]:
        return iter(self.states)

    def __len__(self) -> int:
        return len(self.states)

    def update(self, recurrent_state=None, attn_state=None, conv_state=None, ffn_state=None,
               layer_idx: int = 0, offset: int = 1, **kwargs) -> dict[str, Any]:
        if layer_idx == 0:
            self._seen_tokens += offset
        entry = dict(recurrent_state=recurrent_state, attn_state=attn_state,
                     conv_state=conv_state, ffn_state=ffn_state)
        if layer_idx < len(self.states):
            self.states[layer_idx].update(
                {k: v for k, v in entry.items() if v is not None})
        elif layer_idx == len(self.states):
            self.states.append(entry)
        else:
            raise ValueError(f"layer {layer_idx} updated before layer {len(self.states)}")
        return self.states[layer_idx]

    def get_seq_length(self, layer_idx: int = 0) -> int:
        if len(self.states) <= layer_idx:
            return 0
        return self._seen_tokens

    def to_legacy_cache(self) -> list[dict[str, Any]]:
        return list(self.states)

    @classmethod
    def from_legacy_cache(cls, past_key_values=None, seen_tokens: int = 0) -> "RecurrentCache":
        cache = cls(seen_tokens)
        if past_key_values is not None:
            if isinstance(past_key_values, RecurrentCache):
                return past_key_values
            for layer_idx, entry in enumerate(past_key_values):
                cache.update(**dict(entry), layer_idx=layer_idx, offset=0)
        return cache


def state_from_cache(last_state: Optional[dict]) -> Optional[SolveDeltaLayerState]:
    """dict entry -> SolveDeltaLayerState (modeling_solvedelta.py:104-115)."""
    if last_state is None:
        return None
    recurrent_state = last_state.get("recurrent_state")
    if recurrent_state is None:
        return None
    if not isinstance(recurrent_state, (tuple, list)) or len(recurrent_state) != 2:
        raise ValueError("SolveDelta cache recurrent_state must contain (predictor,S)")
    return SolveDeltaLayerState(operator=SolveDeltaState(*recurrent_state),
                                conv=last_state.get("conv_state"))


def segment_reset_mask(hidden_states: torch.Tensor, cu_seqlens: torch.Tensor) -> torch.Tensor:
    """Packed [1,T,D] rows with cu_seqlens -> reset at every segment start
    (modeling_solvedelta.py:118-131)."""
    if hidden_states.shape[0] != 1:
        raise ValueError("explicit cu_seqlens require packed hidden states [1,T,D]")
    if cu_seqlens.ndim != 1 or cu_seqlens.numel() < 2:
        raise ValueError("cu_seqlens must be one-dimensional with at least two entries")
    if cu_seqlens.dtype not in (torch.int32, torch.int64):
        raise TypeError("cu_seqlens must have int32 or int64 dtype")
    starts = cu_seqlens[:-1].to(device=hidden_states.device, dtype=torch.long)
    mask = torch.zeros((1, hidden_states.shape[1]), dtype=torch.bool, device=hidden_states.device)
    return mask.scatter(1, starts.unsqueeze(0), True)


class SolveDeltaCacheAdapter(nn.Module):
    """Cache ABI around the mixer (modeling_solvedelta.py:134-195)."""

    def __init__(self, config, layer_idx: int) -> None:
        super().__init__()
        self.layer_idx = layer_idx
        self.mixer = SolveDelta(config)

    def forward(self, hidden_states, attention_mask=None, past_key_values=None,
                use_cache: Optional[bool] = False, output_attentions: Optional[bool] = False,
                **kwargs):
        del output_attentions
        batch, length, _ = hidden_states.shape
        last_state = None
        if past_key_values is not None and self.layer_idx < len(past_key_values):
            last_state = past_key_values[self.layer_idx]
        initial_state = state_from_cache(last_state)
        valid_mask = None
        if attention_mask is not None:
            if attention_mask.ndim != 2 or attention_mask.shape[0] != batch:
                raise ValueError("attention_mask must have shape [B,T]")
            if attention_mask.shape[1] < length:
                raise ValueError("attention_mask is shorter than the current input")
            valid_mask = attention_mask[:, -length:].to(torch.bool)
        reset_mask = kwargs.get("solvedelta_reset_mask")
        cu_seqlens = kwargs.get("cu_seqlens")
        if reset_mask is None and cu_seqlens is not None:
            reset_mask = segment_reset_mask(hidden_states, cu_seqlens)
        if reset_mask is not None:
            if reset_mask.shape != (batch, length) or reset_mask.dtype != torch.bool:
                raise ValueError("solvedelta_reset_mask must be bool [B,T]")
            if initial_state is not None and cu_seqlens is not None:
                # a packed continuation carries the cached state into its first segment
                reset_mask = reset_mask.clone()
                reset_mask[0, 0] = False
        cache_requested = bool(use_cache and past_key_values is not None)
        result = self.mixer(hidden_states, initial_state=initial_state, valid_mask=valid_mask,
                            reset_mask=reset_mask, return_final_state=cache_requested)
        if cache_requested:
            output, final_state = result
            past_key_values.update(recurrent_state=tuple(final_state.operator),
                                   conv_state=final_state.conv, layer_idx=self.layer_idx,
                                   offset=length)
        else:
            output = result
        return output, None, past_key_values


__all__ = ["RecurrentCache", "SolveDeltaCacheAdapter", "segment_reset_mask", "state_from_cache"]
