"""``SolveDeltaConfig``: the Hugging Face configuration of the SolveDelta mixer
and its causal LM, as the reference declares it (causallsso/config.py:8-195).

Same constructor fields, defaults, validation order, messages and exception
types, same derived properties (``resolved_head_k_dim``, ``resolved_head_v_dim``,
``geometry_width``, ``key_dim``, ``value_dim``) and ``model_type``, so a
reference config dict (``config.json``) loads unchanged and builds
``solvedelta_amd.SolveDelta`` / ``SolveDeltaForCausalLM``.  Hybrid attention
layers need flash-linear-attention's normaliser (config.py:152-166); that
package does not exist on this stack, so a non-null ``attn`` raises the same
ImportError the reference raises without it.
"""
from __future__ import annotations

import math

from transformers import AutoConfig
from transformers.configuration_utils import PretrainedConfig

_POSITIVE_INTS = ("hidden_size", "num_heads", "num_edits", "num_hidden_layers", "vocab_size",
                  "max_position_embeddings")
_OPTIONAL_INTS = ("head_k_dim", "head_v_dim", "intermediate_size")
_POSITIVE_REALS = ("expand_k", "expand_v", "norm_eps", "initializer_range")
_FLAGS = ("use_short_conv", "bias", "use_cache", "fuse_norm", "fuse_swiglu",
          "fuse_cross_entropy", "fuse_linear_cross_entropy", "use_l2warp")


def _is_int(x) -> bool:
    return isinstance(x, int) and not isinstance(x, bool)


class SolveDeltaConfig(PretrainedConfig):
    """One configuration for the SolveDelta mixer and its causal LM."""

    model_type = "solvedelta"
    keys_to_ignore_at_inference = ["past_key_values"]

    def __init__(self, hidden_size: int = 2048, num_heads: int = 16,
                 head_k_dim: int | None = None, head_v_dim: int | None = None,
                 expand_k: float = 1.0, expand_v: float = 1.0, num_edits: int = 1,
                 use_short_conv: bool = True, bias: bool = False, *,
                 num_hidden_layers: int = 24, hidden_ratio: int | None = 4,
                 intermediate_size: int | None = None, hidden_act: str = "swish",
                 norm_eps: float = 1e-6, max_position_embeddings: int = 2048,
                 attn: dict | list | None = None, use_cache: bool = True,
                 fuse_norm: bool = True, fuse_swiglu: bool = True,
                 fuse_cross_entropy: bool = True, fuse_linear_cross_entropy: bool = False,
                 use_l2warp: bool = False, vocab_size: int = 32000,
                 initializer_range: float = 0.02, pad_token_id: int | None = None,
                 bos_token_id: int = 1, eos_token_id: int = 2,
                 tie_word_embeddings: bool = False, **kwargs) -> None:
        fields = dict(hidden_size=hidden_size, num_heads=num_heads, head_k_dim=head_k_dim,
                      head_v_dim=head_v_dim, expand_k=expand_k, expand_v=expand_v,
                      num_edits=num_edits, use_short_conv=use_short_conv, bias=bias,
                      num_hidden_layers=num_hidden_layers, hidden_ratio=hidden_ratio,
                      intermediate_size=intermediate_size, hidden_act=hidden_act,
                      norm_eps=norm_eps, max_position_embeddings=max_position_embeddings,
                      use_cache=use_cache, fuse_norm=fuse_norm, fuse_swiglu=fuse_swiglu,
                      fuse_cross_entropy=fuse_cross_entropy,
                      fuse_linear_cross_entropy=fuse_linear_cross_entropy,
                      use_l2warp=use_l2warp, vocab_size=vocab_size,
                      initializer_range=initializer_range)
        for name, value in fields.items():
            setattr(self, name, value)
        self._validate()
        if attn is not None:
            raise ImportError("hybrid attention requires flash-linear-attention")
        self.attn = None
        super().__init__(pad_token_id=pad_token_id, bos_token_id=bos_token_id,
                         eos_token_id=eos_token_id, tie_word_embeddings=tie_word_embeddings,
                         **kwargs)

    def _validate(self) -> None:
        for name in _POSITIVE_INTS:
            value = getattr(self, name)
            if not _is_int(value):
                raise TypeError(f"{name} must be an int, got {type(value).__name__}")
            if value <= 0:
                raise ValueError(f"{name} must be positive, got {value}")
        if self.num_edits != 1:
            raise ValueError("the current SolveDelta production contract requires num_edits=1")
        for name in _OPTIONAL_INTS:
            value = getattr(self, name)
            if value is None:
                continue
            if not _is_int(value):
                raise TypeError(f"{name} must be an int or None")
            if value <= 0:
                raise ValueError(f"{name} must be positive, got {value}")
        if self.hidden_ratio is not None:
            if not _is_int(self.hidden_ratio):
                raise TypeError("hidden_ratio must be an int or None")
            if self.hidden_ratio <= 0:
                raise ValueError("hidden_ratio must be positive")
        for name in _POSITIVE_REALS:
            value = getattr(self, name)
            if isinstance(value, bool) or not isinstance(value, (int, float)):
                raise TypeError(f"{name} must be a real number")
            if not math.isfinite(float(value)) or value <= 0:
                raise ValueError(f"{name} must be finite and positive")
        for name in _FLAGS:
            value = getattr(self, name)
            if not isinstance(value, bool):
                raise TypeError(f"{name} must be a bool, got {type(value).__name__}")
        if self.fuse_cross_entropy and self.fuse_linear_cross_entropy:
            raise ValueError("fuse_cross_entropy and fuse_linear_cross_entropy are mutually "
                             "exclusive")
        if not isinstance(self.hidden_act, str) or not self.hidden_act:
            raise TypeError("hidden_act must be a non-empty string")
        # resolve now so a bad expansion fails before any module allocates
        _ = self.resolved_head_k_dim, self.resolved_head_v_dim

    def _resolve_head_dim(self, explicit, expand, name) -> int:
        if explicit is not None:
            return explicit
        total_f = self.hidden_size * float(expand)
        total = round(total_f)
        if not math.isclose(total_f, total, rel_tol=0.0, abs_tol=1e-9):
            raise ValueError(f"hidden_size * {name} must be an integer, got {total_f}")
        if total % self.num_heads:
            raise ValueError(f"resolved total width {total} must be divisible by "
                             f"num_heads={self.num_heads}")
        return total // self.num_heads

    @property
    def resolved_head_k_dim(self) -> int:
        return self._resolve_head_dim(self.head_k_dim, self.expand_k, "expand_k")

    @property
    def resolved_head_v_dim(self) -> int:
        return self._resolve_head_dim(self.head_v_dim, self.expand_v, "expand_v")

    @property
    def geometry_width(self) -> int:
        return self.resolved_head_k_dim

    @property
    def key_dim(self) -> int:
        return self.num_heads * self.resolved_head_k_dim

    @property
    def value_dim(self) -> int:
        return self.num_heads * self.resolved_head_v_dim


try:  # AutoConfig.for_model("solvedelta", ...) as with the reference installed
    AutoConfig.register("solvedelta", SolveDeltaConfig)
except ValueError:  # already registered (the reference package in the same process)
    pass

__all__ = ["SolveDeltaConfig"]
