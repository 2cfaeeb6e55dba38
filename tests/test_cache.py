"""CPU checks of the recurrent-cache wire format (solvedelta_amd/cache.py):
the per-layer dict layout, seen-token accounting, legacy round trip, and the
reference's validation errors (modeling_solvedelta.py:104-131)."""
import pytest
import torch

from solvedelta_amd.cache import RecurrentCache, segment_reset_mask, state_from_cache


def test_cache_update_and_seq_length():
    cache = RecurrentCache()
    assert len(cache) == 0 and cache.get_seq_length() == 0
    C, S = torch.zeros(1, 2, 4, 4), torch.zeros(1, 2, 4, 3)
    conv = torch.zeros(1, 2 * 2 * 4 + 2 * 3, 3)
    for layer in range(3):
        cache.update(recurrent_state=(C, S), conv_state=conv, layer_idx=layer, offset=5)
    assert len(cache) == 3 and cache.get_seq_length() == 5      # first layer counts tokens
    cache.update(recurrent_state=(C + 1, S), layer_idx=0, offset=1)
    assert cache.get_seq_length() == 6
    assert torch.equal(cache[0]["recurrent_state"][0], C + 1)
    assert cache[0]["conv_state"] is conv                         # kept when not given
    legacy = cache.to_legacy_cache()
    again = RecurrentCache.from_legacy_cache(legacy, seen_tokens=6)
    assert len(again) == 3 and again.get_seq_length() == 6
    with pytest.raises(ValueError):
        cache.update(recurrent_state=(C, S), layer_idx=7)


def test_state_from_cache_layout_and_errors():
    assert state_from_cache(None) is None
    assert state_from_cache({"recurrent_state": None}) is None
    C, S = torch.zeros(1, 1, 2, 2), torch.zeros(1, 1, 2, 2)
    conv = torch.zeros(1, 6, 3)
    st = state_from_cache({"recurrent_state": (C, S), "conv_state": conv})
    assert st.operator.predictor is C and st.operator.S is S and st.conv is conv
    with pytest.raises(ValueError):
        state_from_cache({"recurrent_state": (C,)})


def test_segment_reset_mask():
    h = torch.zeros(1, 10, 4)
    m = segment_reset_mask(h, torch.tensor([0, 3, 7, 10], dtype=torch.int32))
    assert m.tolist() == [[True, False, False, True, False, False, False, True, False, False]]
    with pytest.raises(ValueError):
        segment_reset_mask(torch.zeros(2, 10, 4), torch.tensor([0, 10]))
    with pytest.raises(TypeError):
        segment_reset_mask(h, torch.tensor([0.0, 10.0]))
    with pytest.raises(ValueError):
        segment_reset_mask(h, torch.tensor([0]))


def test_graphed_step_validates_like_the_reference():
    from solvedelta_amd.graph import SolveDeltaGraphedTrainingStep
    from solvedelta_amd.lm import SolveDeltaForCausalLM, SolveDeltaLMConfig
    cfg = SolveDeltaLMConfig(hidden_size=32, num_heads=2, head_k_dim=16, head_v_dim=16,
                             num_hidden_layers=1, hidden_ratio=2, vocab_size=11)
    model = SolveDeltaForCausalLM(cfg)
    ids = torch.zeros(1, 4, dtype=torch.long)
    with pytest.raises(TypeError):
        SolveDeltaGraphedTrainingStep(torch.nn.Linear(2, 2), ids, ids)
    with pytest.raises(ValueError):
        SolveDeltaGraphedTrainingStep(model.eval(), ids, ids)
    with pytest.raises(ValueError):                     # host tensors
        SolveDeltaGraphedTrainingStep(model.train(), ids, ids)
    with pytest.raises(TypeError):
        SolveDeltaGraphedTrainingStep(model.train(), ids, ids, num_warmup_iters=True)
    # reference parameter names line up (modeling_solvedelta.py module tree)
    names = {n for n, _ in model.named_parameters()}
    for n in ("model.embeddings.weight", "model.layers.0.mixer_norm.weight",
              "model.layers.0.mixer.mixer.in_proj.weight", "model.layers.0.mlp.gate_up_proj.weight",
              "model.layers.0.mlp.down_proj.weight", "model.norm.weight", "lm_head.weight",
              "model.layers.0.mixer.mixer.associative_decay_bias"):
        assert n in names, n


def test_live_grad_accumulator_probe():
    """The capture guard's probe: True exactly while another autograd graph
    holds the parameter's AccumulateGrad node, and it leaves no tag behind."""
    import gc
    from solvedelta_amd.graph import _has_live_grad_accumulator
    p = torch.nn.Parameter(torch.randn(3))
    assert not _has_live_grad_accumulator(p)
    y = (p * 2).sum()
    assert _has_live_grad_accumulator(p)
    y.backward()
    assert _has_live_grad_accumulator(p)          # backward ran; the graph is still held
    node = torch.autograd.graph.get_gradient_edge(p).node
    assert not any(k.startswith("solvedelta") for k in node.metadata)
    del node, y
    gc.collect()
    assert not _has_live_grad_accumulator(p)
