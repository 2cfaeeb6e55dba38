"""HIP-graph training step (solvedelta_amd/graph.py) on a small causal LM:
every replay (with eager work and synchronisations between replays) gives the
eager loss and parameter gradients, and replays follow in-place parameter
updates.  The graph path runs the same kernels on the same inputs, so the
bound is tight (rel 1e-5); the only freedom is library GEMM algorithm choice
inside and outside capture."""
import pytest
import torch

from gpu_common import check_lm_against_oracle, rel

pytestmark = pytest.mark.gpu


def _model(seed=0):
    from solvedelta_amd.lm import SolveDeltaForCausalLM, SolveDeltaLMConfig
    torch.manual_seed(seed)
    cfg = SolveDeltaLMConfig(hidden_size=128, num_heads=2, head_k_dim=64, head_v_dim=64,
                             num_hidden_layers=2, hidden_ratio=2, vocab_size=97)
    return SolveDeltaForCausalLM(cfg).cuda().train()


def _eager(model, ids, labels):
    model.zero_grad(set_to_none=True)
    with torch.autocast("cuda", dtype=torch.bfloat16, cache_enabled=False):
        loss, _, _ = model(ids, labels=labels)
    loss.backward()
    return loss.detach().clone(), [p.grad.detach().clone() for p in model.parameters()]


def test_graphed_step_replays_match_eager():
    from solvedelta_amd.graph import SolveDeltaGraphedTrainingStep
    model = _model()
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, 97, (2, 64), generator=g).cuda()
    labels = ids.clone()
    ref_loss, ref_grads = _eager(model, ids, labels)
    step = SolveDeltaGraphedTrainingStep(model, ids, labels)
    for rep in range(3):
        model.zero_grad(set_to_none=True)
        loss = step(ids, labels)
        loss.backward()
        torch.cuda.synchronize()
        el = rel(loss.detach().float(), ref_loss.float())
        eg = max(rel(p.grad, r) for p, r in zip(model.parameters(), ref_grads))
        print(f"[graph replay {rep}] loss {loss.item():.6f} rel loss {el:.1e} worst grad {eg:.1e}",
              flush=True)
        assert el < 1e-5 and eg < 1e-4
        _ = (torch.randn(1000, device="cuda") ** 2).sum().item()   # eager work between replays
    # the graph reads parameters in place: an update is seen by the next replay
    with torch.no_grad():
        for p in model.parameters():
            if p.grad is not None:
                p.add_(p.grad, alpha=-0.5)
    new_loss, new_grads = _eager(model, ids, labels)
    model.zero_grad(set_to_none=True)
    loss = step(ids, labels)
    loss.backward()
    assert rel(loss.detach().float(), new_loss.float()) < 1e-5
    assert abs(new_loss.item() - ref_loss.item()) > 1e-4
    assert max(rel(p.grad, r) for p, r in zip(model.parameters(), new_grads)) < 1e-4


def test_graphed_step_matches_fp64_lm_oracle():
    """The captured training step against the FP64 LM oracle (not only against
    eager): loss and every parameter gradient of a replay."""
    from solvedelta_amd.graph import SolveDeltaGraphedTrainingStep
    model = _model(seed=4)
    with torch.no_grad():
        for n, p in model.named_parameters():
            if n.endswith("norm.weight"):
                p.uniform_(0.5, 1.5)
    ids = torch.randint(0, 97, (2, 64), generator=torch.Generator().manual_seed(5)).cuda()
    step = SolveDeltaGraphedTrainingStep(model, ids, ids)
    for _ in range(2):
        model.zero_grad(set_to_none=True)
        loss = step(ids, ids)
        loss.backward()
    torch.cuda.synchronize()
    check_lm_against_oracle(model, ids, loss, "graph vs oracle", layers=2, heads=2, rk=64, rv=64)


def test_capture_refuses_a_live_eager_graph():
    """A loss still holding its autograd graph pins the parameters'
    AccumulateGrad nodes to the stream it ran on; the helper refuses to capture
    then (before any capture starts) and captures once the loss is released."""
    from solvedelta_amd.graph import SolveDeltaGraphedTrainingStep
    model = _model(seed=2)
    ids = torch.randint(0, 97, (2, 64), generator=torch.Generator().manual_seed(3)).cuda()
    with torch.autocast("cuda", dtype=torch.bfloat16, cache_enabled=False):
        loss, _, _ = model(ids, labels=ids)
    loss.backward()
    with pytest.raises(ValueError, match="still alive"):
        SolveDeltaGraphedTrainingStep(model, ids, ids)
    del loss
    step = SolveDeltaGraphedTrainingStep(model, ids, ids)
    model.zero_grad(set_to_none=True)
    step(ids, ids).backward()
    torch.cuda.synchronize()
    assert all(torch.isfinite(p.grad).all() for p in model.parameters())
