"""A minimal SolveDelta causal LM stack around the HIP mixer.

Just enough of the reference's model shell (causallsso/modeling_solvedelta.py:
31-100 MLP, :198-255 block, :283-395 model, :398-505 LM head and loss) to run
the CausalLM configuration end to end on MI355X and to capture its training
step in a HIP graph: token embedding, per layer pre-norm mixer + pre-norm
SwiGLU MLP with residuals, final norm, LM head and the shifted cross-entropy.
Module and parameter names follow the reference (``model.embeddings``,
``model.layers.{i}.mixer_norm / mixer.mixer / mlp_norm / mlp.gate_up_proj /
mlp.down_proj``, ``model.norm``, ``lm_head``) so its state dicts line up.
Everything but the mixer is plain PyTorch-ROCm (hipBLASLt GEMMs, torch norms
and loss); there is no HF ``generate`` or hybrid attention here.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn.functional as F
from torch import nn

from .cache import RecurrentCache, SolveDeltaCacheAdapter
from .mixer import SolveDeltaMixerConfig


@dataclass
class SolveDeltaLMConfig(SolveDeltaMixerConfig):
    """Mixer fields plus the shell's (config.py:10-90)."""
    num_hidden_layers: int = 24
    hidden_ratio: Optional[int] = 4
    intermediate_size: Optional[int] = None
    vocab_size: int = 32000
    initializer_range: float = 0.02


class SolveDeltaMLP(nn.Module):
    """SwiGLU MLP with one gate/up projection (modeling_solvedelta.py:31-100)."""

    def __init__(self, hidden_size: int, hidden_ratio: Optional[int] = None,
                 intermediate_size: Optional[int] = None) -> None:
        super().__init__()
        if hidden_ratio is None:
            hidden_ratio = 4
        if intermediate_size is None:
            intermediate_size = int(hidden_size * hidden_ratio * 2 / 3)
            intermediate_size = 256 * ((intermediate_size + 255) // 256)
        self.hidden_size = hidden_size
        self.intermediate_size = intermediate_size
        self.gate_up_proj = nn.Linear(hidden_size, 2 * intermediate_size, bias=False)
        self.down_proj = nn.Linear(intermediate_size, hidden_size, bias=False)

    def forward(self, x):
        gate, value = self.gate_up_proj(x).chunk(2, dim=-1)
        return self.down_proj(F.silu(gate) * value)


class SolveDeltaBlock(nn.Module):
    def __init__(self, config: SolveDeltaLMConfig, layer_idx: int) -> None:
        super().__init__()
        self.layer_idx = layer_idx
        self.mixer_norm = nn.RMSNorm(config.hidden_size, eps=config.norm_eps)
        self.mixer = SolveDeltaCacheAdapter(config, layer_idx)
        self.mlp_norm = nn.RMSNorm(config.hidden_size, eps=config.norm_eps)
        self.mlp = SolveDeltaMLP(config.hidden_size, config.hidden_ratio,
                                 config.intermediate_size)

    def forward(self, x, attention_mask=None, past_key_values=None, use_cache=False, **kw):
        y, _, past_key_values = self.mixer(self.mixer_norm(x), attention_mask=attention_mask,
                                           past_key_values=past_key_values, use_cache=use_cache,
                                           **kw)
        x = x + y
        return x + self.mlp(self.mlp_norm(x)), past_key_values


class SolveDeltaModel(nn.Module):
    def __init__(self, config: SolveDeltaLMConfig) -> None:
        super().__init__()
        self.config = config
        self.embeddings = nn.Embedding(config.vocab_size, config.hidden_size)
        self.layers = nn.ModuleList(SolveDeltaBlock(config, i)
                                    for i in range(config.num_hidden_layers))
        self.norm = nn.RMSNorm(config.hidden_size, eps=config.norm_eps)

    def forward(self, input_ids, attention_mask=None, past_key_values=None, use_cache=False,
                **kw):
        x = self.embeddings(input_ids)
        if use_cache and not isinstance(past_key_values, RecurrentCache):
            past_key_values = RecurrentCache.from_legacy_cache(past_key_values)
        elif not use_cache:
            past_key_values = None
        for layer in self.layers:
            x, past_key_values = layer(x, attention_mask=attention_mask,
                                       past_key_values=past_key_values, use_cache=use_cache, **kw)
        return self.norm(x), past_key_values


class SolveDeltaForCausalLM(nn.Module):
    def __init__(self, config: SolveDeltaLMConfig) -> None:
        super().__init__()
        self.config = config
        self.model = SolveDeltaModel(config)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        self.apply(self._init_weights)

    def _init_weights(self, module):
        """Linear and embedding weights ~ N(0, initializer_range), biases zero
        (modeling_solvedelta.py:268-280); the mixer's own gate parameters keep
        their initial values."""
        if isinstance(module, nn.Linear):
            nn.init.normal_(module.weight, mean=0.0, std=self.config.initializer_range)
            if module.bias is not None:
                nn.init.zeros_(module.bias)
        elif isinstance(module, nn.Embedding):
            nn.init.normal_(module.weight, mean=0.0, std=self.config.initializer_range)

    def forward(self, input_ids, labels=None, attention_mask=None, past_key_values=None,
                use_cache: bool = False, **kw):
        """Returns (loss or None, logits, cache or None); the loss is the mean
        cross-entropy of token t+1 given tokens <= t (the last position ignored)."""
        h, cache = self.model(input_ids, attention_mask=attention_mask,
                              past_key_values=past_key_values, use_cache=use_cache, **kw)
        logits = self.lm_head(h)
        loss = None
        if labels is not None:
            shifted = torch.cat((labels[..., 1:], torch.full_like(labels[:, :1], -100)), dim=1)
            loss = F.cross_entropy(logits.reshape(-1, logits.shape[-1]).float(),
                                   shifted.reshape(-1), ignore_index=-100)
        return loss, logits, cache


__all__ = ["SolveDeltaLMConfig", "SolveDeltaMLP", "SolveDeltaBlock", "SolveDeltaModel",
           "SolveDeltaForCausalLM"]
