"""FP64 oracle of the SolveDelta causal LM (test infrastructure only).

Composes ``mixer_oracle`` (the FP64 mixer layer, itself over the FP64 token
loop of ``sd_oracle``) with the reference's LM shell in plain torch
(causallsso/modeling_solvedelta.py:31-100 SwiGLU MLP, :198-255 pre-norm
block, :283-395 model, :398-505 head and loss):

    x   = embed(ids)
    x  += mixer(rmsnorm(x))            per layer
    x  += down(silu(gate(n)) * up(n)),  n = rmsnorm(x)
    loss = mean CE(head(rmsnorm(x))[t], ids[t+1])   (last position ignored)

``params`` maps the parameter names of ``solvedelta_amd.lm.SolveDeltaForCausalLM``
to tensors.  The product never imports this file.

Parity status: the mixer is pinned through ``mixer_oracle``; the shell is
pinned in ``tests/test_lm_oracle.py`` (zero-mixer / zero-MLP reduction to an
independently written logsumexp loss, the fused gate-up split against two
separate projections, and ``gradcheck``).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .mixer_oracle import mixer_oracle


def _rms(x, w, eps):
    return x * torch.rsqrt(x.square().mean(-1, keepdim=True) + eps) * w


def lm_oracle(params: dict, ids, labels, *, layers, heads, rk, rv, eps=1e-6,
              use_short_conv=True, taps=None):
    """Returns (loss, logits) in FP64; ``taps`` is passed to each layer's
    ``mixer_oracle``."""
    p = {k: v.double() for k, v in params.items()}
    x = F.embedding(ids, p["model.embeddings.weight"])
    for i in range(layers):
        pre = f"model.layers.{i}."
        mix = {k[len(pre) + len("mixer.mixer."):]: v for k, v in p.items()
               if k.startswith(pre + "mixer.mixer.")}
        y, _, _ = mixer_oracle(mix, _rms(x, p[pre + "mixer_norm.weight"], eps), heads=heads,
                               rk=rk, rv=rv, eps=eps, use_short_conv=use_short_conv, taps=taps)
        x = x + y
        n = _rms(x, p[pre + "mlp_norm.weight"], eps)
        gate, up = F.linear(n, p[pre + "mlp.gate_up_proj.weight"]).chunk(2, dim=-1)
        x = x + F.linear(F.silu(gate) * up, p[pre + "mlp.down_proj.weight"])
    logits = F.linear(_rms(x, p["model.norm.weight"], eps), p["lm_head.weight"])
    target = torch.cat((labels[:, 1:], torch.full_like(labels[:, :1], -100)), dim=1)
    loss = F.cross_entropy(logits.reshape(-1, logits.shape[-1]), target.reshape(-1),
                           ignore_index=-100)
    return loss, logits


__all__ = ["lm_oracle"]
