"""CPU checks of ``SolveDeltaConfig`` (solvedelta_amd/config.py) against the
reference's config contract (causallsso/config.py:8-195) and model tests
(tests/model/test_modeling_solvedelta.py:69-79, 187-202): a reference-shaped
config round-trips through its dict, is reachable through AutoConfig, builds
the mixer with the reference's projection layout and the causal LM, and
rejects what the reference rejects with the same exception types."""
import pytest
import torch
from transformers import AutoConfig

from solvedelta_amd import SolveDeltaConfig


def _tiny(**kw):
    values = dict(hidden_size=32, num_heads=2, head_k_dim=16, head_v_dim=16, num_hidden_layers=2,
                  hidden_ratio=2, vocab_size=97, max_position_embeddings=64, use_short_conv=True,
                  fuse_norm=False, fuse_swiglu=False, fuse_cross_entropy=False, use_cache=False)
    values.update(kw)
    return SolveDeltaConfig(**values)


def test_roundtrip_and_auto_registration():
    cfg = _tiny()
    again = SolveDeltaConfig.from_dict(cfg.to_dict())
    assert again.to_dict() == cfg.to_dict()
    auto = AutoConfig.for_model("solvedelta", hidden_size=32, num_heads=2)
    assert isinstance(auto, SolveDeltaConfig)
    assert auto.resolved_head_k_dim == 16 and auto.value_dim == 32


def test_config_builds_mixer_with_reference_layout():
    from solvedelta_amd import SolveDelta
    mixer = SolveDelta(_tiny(num_hidden_layers=1))
    assert mixer.projection_sizes == (32, 32, 32, 32, 32, 32, 32, 2, 16, 16)
    assert mixer.projection_width == 258 and mixer.projection_padding == 62
    assert mixer.in_proj.out_features == 320
    assert mixer.decay_proj.weight.shape == (32, 16)
    assert mixer.output_gate_proj.weight.shape == (32, 16)
    assert mixer.output_gate_proj.bias.shape == (32,)
    assert mixer.associative_log_rate.shape == (2,)
    assert mixer.associative_decay_bias.shape == (2, 16)
    assert mixer.output_norm.weight.shape == (16,)


def test_config_builds_causal_lm():
    from solvedelta_amd import SolveDeltaForCausalLM
    cfg = _tiny()
    model = SolveDeltaForCausalLM(cfg)
    names = dict(model.named_parameters())
    assert "model.embeddings.weight" in names and "lm_head.weight" in names
    assert "model.layers.1.mixer.mixer.in_proj.weight" in names
    assert names["model.layers.0.mlp.gate_up_proj.weight"].shape[1] == 32
    assert len(model.model.layers) == 2
    # head widths from expansion instead of explicit dims
    derived = SolveDeltaConfig(hidden_size=64, num_heads=4, expand_k=0.5, expand_v=1.0)
    assert derived.resolved_head_k_dim == 8 and derived.resolved_head_v_dim == 16
    assert derived.geometry_width == 8 and derived.key_dim == 32


@pytest.mark.parametrize("kw,exc", [
    (dict(hidden_size=0), ValueError),
    (dict(hidden_size=32.0), TypeError),
    (dict(num_heads=True), TypeError),
    (dict(num_edits=2), ValueError),
    (dict(head_k_dim=-1), ValueError),
    (dict(hidden_ratio=1.5), TypeError),
    (dict(norm_eps=float("inf")), ValueError),
    (dict(use_cache=1), TypeError),
    (dict(fuse_cross_entropy=True, fuse_linear_cross_entropy=True), ValueError),
    (dict(hidden_act=""), TypeError),
    (dict(head_k_dim=None, expand_k=0.3), ValueError),
    (dict(head_k_dim=None, num_heads=3, hidden_size=32), ValueError),
    (dict(attn={"layers": [0]}), ImportError),
])
def test_config_validation_errors(kw, exc):
    with pytest.raises(exc):
        _tiny(**kw)
