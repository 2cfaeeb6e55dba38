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

from typing import Any, Iterator, NamedTuple, Optional

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
    """A layer's cache entry as the mixer's initial state, or None when the entry
    is absent or holds no recurrent state yet.  Wire format
    (modeling_solvedelta.py:104-115): ``recurrent_state`` is the pair
    (predictor C, memory S); ``conv_state`` rides along unchanged (it may be None)."""
    pair = None if last_state is None else last_state.get("recurrent_state")
    if pair is None:
        return None
    if not isinstance(pair, (tuple, list)) or len(pair) != 2:
        raise ValueError("SolveDelta cache recurrent_state must contain (predictor,S)")
    return SolveDeltaLayerState(SolveDeltaState(*pair), last_state.get("conv_state"))


def segment_reset_mask(hidden_states: torch.Tensor, cu_seqlens: torch.Tensor) -> torch.Tensor:
    """Reset flags of a packed row: ``hidden_states`` is one [1,T,D] row holding
    several sequences back to back, ``cu_seqlens`` their cumulative boundaries;
    every sequence's first token starts from a zero state
    (modeling_solvedelta.py:118-131; the same errors for the same inputs)."""
    if hidden_states.shape[0] != 1:
        raise ValueError("explicit cu_seqlens require packed hidden states [1,T,D]")
    if cu_seqlens.ndim != 1 or cu_seqlens.numel() < 2:
        raise ValueError("cu_seqlens must be one-dimensional with at least two entries")
    if cu_seqlens.dtype not in (torch.int32, torch.int64):
        raise TypeError("cu_seqlens must have int32 or int64 dtype")
    device = hidden_states.device
    first_tokens = cu_seqlens.narrow(0, 0, cu_seqlens.numel() - 1).to(device, torch.long)
    flags = torch.zeros(hidden_states.shape[1], dtype=torch.bool, device=device)
    return flags.index_fill_(0, first_tokens, True).unsqueeze(0)


class _CallPlan(NamedTuple):
    """What one adapter call hands the mixer, derived from the HF-style arguments."""
    initial_state: Optional[SolveDeltaLayerState]
    valid_mask: Optional[torch.Tensor]
    reset_mask: Optional[torch.Tensor]
    write_back: bool


def _valid_from_attention(attention_mask, batch: int, length: int):
    """The last ``length`` columns of a [B, >=T] padding mask as valid flags."""
    if attention_mask is None:
        return None
    if attention_mask.ndim != 2 or attention_mask.shape[0] != batch:
        raise ValueError("attention_mask must have shape [B,T]")
    if attention_mask.shape[1] < length:
        raise ValueError("attention_mask is shorter than the current input")
    return attention_mask[:, attention_mask.shape[1] - length:].bool()


def _resets(hidden_states, explicit, cu_seqlens, continues_cache: bool):
    """Reset flags from an explicit mask, else from packed-sequence boundaries.
    When boundaries are given and the call continues a cached state, the row's
    first sequence is the cached one carried on, so its first token keeps the
    state (the reference clears that one flag, modeling_solvedelta.py:180-187)."""
    batch, length = hidden_states.shape[:2]
    flags = explicit
    if flags is None and cu_seqlens is not None:
        flags = segment_reset_mask(hidden_states, cu_seqlens)
    if flags is None:
        return None
    if flags.dtype != torch.bool or tuple(flags.shape) != (batch, length):
        raise ValueError("solvedelta_reset_mask must be bool [B,T]")
    if continues_cache and cu_seqlens is not None and bool(length):
        keep_first = torch.ones_like(flags)
        keep_first[0, 0] = False
        flags = flags & keep_first
    return flags


class SolveDeltaCacheAdapter(nn.Module):
    """The layer's cache boundary around the mixer (modeling_solvedelta.py:134-195):
    reads the layer's entry from ``past_key_values``, turns the padding mask,
    explicit resets or packed boundaries into the mixer's dense masks, and with
    ``use_cache`` writes the final (C, S) and conv state back, advancing the
    cache by the call's token count.  Returns (output, None, past_key_values)."""

    def __init__(self, config, layer_idx: int) -> None:
        super().__init__()
        self.layer_idx = layer_idx
        self.mixer = SolveDelta(config)

    def _plan(self, hidden_states, attention_mask, past_key_values, use_cache, extra) -> _CallPlan:
        batch, length = hidden_states.shape[:2]
        entry = None
        if past_key_values is not None and self.layer_idx < len(past_key_values):
            entry = past_key_values[self.layer_idx]
        initial = state_from_cache(entry)
        valid = _valid_from_attention(attention_mask, batch, length)
        resets = _resets(hidden_states, extra.get("solvedelta_reset_mask"),
                         extra.get("cu_seqlens"), initial is not None)
        return _CallPlan(initial, valid, resets, bool(use_cache) and past_key_values is not None)

    def forward(self, hidden_states, attention_mask=None, past_key_values=None,
                use_cache: Optional[bool] = False, output_attentions: Optional[bool] = False,
                **kwargs):
        plan = self._plan(hidden_states, attention_mask, past_key_values, use_cache, kwargs)
        result = self.mixer(hidden_states, initial_state=plan.initial_state,
                            valid_mask=plan.valid_mask, reset_mask=plan.reset_mask,
                            return_final_state=plan.write_back)
        if not plan.write_back:
            return result, None, past_key_values
        output, final = result
        past_key_values.update(recurrent_state=(final.operator.predictor, final.operator.S),
                               conv_state=final.conv, layer_idx=self.layer_idx,
                               offset=hidden_states.shape[1])
        return output, None, past_key_values


__all__ = ["RecurrentCache", "SolveDeltaCacheAdapter", "segment_reset_mask", "state_from_cache"]
