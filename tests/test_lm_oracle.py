"""Pins the FP64 causal-LM oracle's shell (oracle/lm_oracle.py) on the CPU:
with every mixer and MLP output projection zeroed the model reduces to
embedding -> final RMSNorm -> head, whose shifted loss is recomputed here
token by token with an explicit log-sum-exp; the fused gate/up projection
equals two separate projections (reference test_modeling_solvedelta.py:81-134);
and gradcheck holds for the whole composition on a tiny model."""
import math

import torch
import torch.nn.functional as F

from oracle.lm_oracle import lm_oracle


def _params(hidden=16, H=2, r=4, layers=2, vocab=11, seed=0):
    from solvedelta_amd.lm import SolveDeltaForCausalLM, SolveDeltaLMConfig
    torch.manual_seed(seed)
    cfg = SolveDeltaLMConfig(hidden_size=hidden, num_heads=H, head_k_dim=r, head_v_dim=r,
                             num_hidden_layers=layers, hidden_ratio=2, vocab_size=vocab)
    model = SolveDeltaForCausalLM(cfg)
    p = {k: v.detach().double().clone() for k, v in model.named_parameters()}
    for k in p:
        if k.endswith("norm.weight"):
            p[k].uniform_(0.5, 1.5)
    return cfg, p


def test_zero_blocks_reduce_to_embedding_head_loss():
    cfg, p = _params()
    for k in p:
        if k.endswith("mixer.mixer.output_proj.weight") or k.endswith("mlp.down_proj.weight"):
            p[k].zero_()
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, 11, (2, 7), generator=g)
    loss, logits = lm_oracle(p, ids, ids, layers=2, heads=2, rk=4, rv=4)
    emb, wn, head = p["model.embeddings.weight"], p["model.norm.weight"], p["lm_head.weight"]
    total, count = 0.0, 0
    for b in range(2):
        for t in range(6):
            x = emb[ids[b, t]]
            n = x / math.sqrt(float((x * x).mean()) + 1e-6) * wn
            z = [float(n @ head[v]) for v in range(11)]
            m = max(z)
            lse = m + math.log(sum(math.exp(zz - m) for zz in z))
            total += lse - z[int(ids[b, t + 1])]
            count += 1
    assert abs(loss.item() - total / count) < 1e-10
    assert logits.shape == (2, 7, 11)


def test_fused_gate_up_matches_two_projections():
    cfg, p = _params(layers=1)
    ids = torch.randint(0, 11, (1, 5), generator=torch.Generator().manual_seed(2))
    loss, _ = lm_oracle(p, ids, ids, layers=1, heads=2, rk=4, rv=4)
    w = p["model.layers.0.mlp.gate_up_proj.weight"]
    gate_w, up_w = w.chunk(2, dim=0)
    # the same model with the MLP written as two projections
    x = F.embedding(ids, p["model.embeddings.weight"])
    from oracle.mixer_oracle import mixer_oracle
    pre = "model.layers.0."
    rms = lambda v, wt: v * torch.rsqrt(v.square().mean(-1, keepdim=True) + 1e-6) * wt
    mix = {k[len(pre + "mixer.mixer."):]: v for k, v in p.items() if k.startswith(pre + "mixer.mixer.")}
    x = x + mixer_oracle(mix, rms(x, p[pre + "mixer_norm.weight"]), heads=2, rk=4, rv=4)[0]
    n = rms(x, p[pre + "mlp_norm.weight"])
    x = x + F.linear(F.silu(n @ gate_w.T) * (n @ up_w.T), p[pre + "mlp.down_proj.weight"])
    logits = rms(x, p["model.norm.weight"]) @ p["lm_head.weight"].T
    ref = F.cross_entropy(logits[:, :-1].reshape(-1, 11), ids[:, 1:].reshape(-1))
    assert abs(loss.item() - ref.item()) < 1e-12


def test_lm_oracle_gradcheck():
    cfg, p = _params(hidden=8, H=1, r=4, layers=1, vocab=5)
    ids = torch.randint(0, 5, (1, 4), generator=torch.Generator().manual_seed(3))
    names = ["model.embeddings.weight", "model.layers.0.mixer.mixer.in_proj.weight",
             "model.layers.0.mlp.gate_up_proj.weight", "lm_head.weight"]
    leaves = [p[n].clone().requires_grad_() for n in names]

    def f(*xs):
        q = dict(p)
        q.update(zip(names, xs))
        return lm_oracle(q, ids, ids, layers=1, heads=1, rk=4, rv=4)[0]

    assert torch.autograd.gradcheck(f, leaves, eps=1e-6, atol=1e-6)
