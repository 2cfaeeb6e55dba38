"""FP64 oracle for the SolveDelta mixer layer (test infrastructure only).

A restatement of the reference mixer's CPU path in our own code: the checker
for the HIP frontend/readout kernels and for ``solvedelta_amd.mixer``; the
product code never imports it.

  projection   in_proj, split into (q, k, v | u, h, erase, write, geometry,
               decay_hidden, gate_hidden)                (model.py:35-60, 342-367)
  conv4        causal depthwise conv of (q, k, v) + SiLU, with a [B, D, 3]
               state; invalid tokens emit 0 and keep the state, a valid reset
               clears it first                           (model.py:146-164)
  decay gate   log_decay = -exp(log_rate[h]) softplus(decay_proj(x) + bias[h, c])
                                                         (model.py:384-390)
  geometry     gamma = sigmoid(geometry_raw + geometry_write_bias[h])
                                                         (model.py:391-394)
  operator     the FP64 token loop of ``oracle.sd_oracle``  (reference.py:82-229)
  readout      y = x rsqrt(mean x^2 + eps) w sigmoid(gate), then output_proj
                                                         (ops/norm_gate.py:20-43)

Parity status: ``conv4_loop`` is pinned against ``torch.nn.functional.conv1d``
on the state-prefixed sequence and against brute force on masks;
``rms_norm_gated`` against the reference test's closed form
(test_rebuild_semantics.py:251-276) and ``gradcheck`` (:279-293);
``kda_decay`` against its limits (softplus -> identity above 20, -> exp(x)
far below 0) and its derivative; ``projection_layout`` against the reference
test's sizes (test_modeling_solvedelta.py:187-202).  All in
``tests/test_mixer_oracle.py``.
"""
from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn.functional as F

from .sd_oracle import OracleState, solvedelta_oracle


def projection_layout(hidden, heads, rk, rv, edits=1):
    """Sizes of the packed in_proj rows and the pad to a multiple of 64
    (model.py:35-60)."""
    sizes = (heads * rk, heads * edits * rk, heads * edits * rv, heads * rk, heads * rk,
             heads * edits * rk, heads * edits * rv, heads, rv, rv)
    width = sum(sizes)
    return sizes, width, (-width) % 64


def conv4_loop(x, weight, state=None, valid_mask=None, reset_mask=None):
    """x [B,T,D], weight [D,4], state [B,D,3] -> (silu(conv) [B,T,D], final [B,D,3])."""
    B, T, D = x.shape
    st = x.new_zeros(B, D, 3) if state is None else state
    outs = []
    for t in range(T):
        valid = torch.ones(B, dtype=torch.bool) if valid_mask is None else valid_mask[:, t]
        reset = torch.zeros(B, dtype=torch.bool) if reset_mask is None else reset_mask[:, t]
        reset = reset & valid
        st = torch.where(reset[:, None, None], torch.zeros_like(st), st)
        window = torch.cat((st, x[:, t, :, None]), dim=-1)         # [B,D,4]
        y = F.silu((window * weight[None]).sum(-1))
        outs.append(torch.where(valid[:, None], y, torch.zeros_like(y)))
        st = torch.where(valid[:, None, None], window[..., 1:], st)
    return torch.stack(outs, 1), st


def kda_decay(raw, log_rate, bias):
    """raw [B,T,H,r], log_rate [H], bias [H,r] -> log-decay [B,T,H,r]."""
    H = log_rate.shape[0]
    return -torch.exp(log_rate).view(1, 1, H, 1) * F.softplus(raw + bias.view(1, 1, H, -1))


def rms_norm_gated(x, gate, weight, eps):
    rstd = torch.rsqrt(x.square().mean(-1, keepdim=True) + eps)
    return x * rstd * weight * torch.sigmoid(gate)


def mixer_oracle(params: dict, hidden, *, heads, rk, rv, eps=1e-6, use_short_conv=True,
                 initial_state: Optional[tuple] = None, valid_mask=None, reset_mask=None,
                 geometry_enabled=True, decay_enabled=True, taps: Optional[list] = None,
                 act_round=None):
    """One mixer layer in FP64.  ``params`` maps the reference module's parameter
    names (in_proj.weight, conv_weight, decay_proj.weight, output_gate_proj.weight/
    .bias, output_norm.weight, output_proj.weight, geometry_write_bias,
    associative_log_rate, associative_decay_bias; optional in_proj.bias /
    output_proj.bias) to tensors.  ``initial_state`` = ((C, S), conv) or None.
    Returns (output [B,T,hidden], (C, S), conv_state).  If ``taps`` is a list,
    the log-decay tensor [B,T,H,r] is appended to it (for conditioning
    estimates of the decay-rate gradient in tests).  ``act_round`` (e.g. a
    round trip through bf16) is applied where a bf16 layer materialises its
    activations -- the in-projection, the conv4 + SiLU output, the decay and
    output-gate projections and the operator output -- so that the FP64
    recurrence runs on the operands the bf16 layer hands its operator; None
    keeps every activation exact."""
    p = {k: v.double() for k, v in params.items()}
    hidden = hidden.double()
    rnd = act_round if act_round is not None else (lambda x: x)
    B, T, _ = hidden.shape
    sizes, width, _ = projection_layout(hidden.shape[-1], heads, rk, rv)
    proj = rnd(F.linear(hidden, p["in_proj.weight"], p.get("in_proj.bias"))[..., :width])
    parts = proj.split(sizes, dim=-1)
    qkv = torch.cat(parts[:3], dim=-1)
    op_init, conv_init = (None, None) if initial_state is None else initial_state
    conv_state = None
    if use_short_conv:
        qkv, conv_state = conv4_loop(qkv, p["conv_weight"],
                                     None if conv_init is None else conv_init.double(),
                                     valid_mask, reset_mask)
    else:
        qkv = F.silu(qkv)
    qkv = rnd(qkv)
    q, k, v = qkv.split(sizes[:3], dim=-1)
    u, h, er, wr, geo, dec_h, gate_h = parts[3:]
    view = lambda x, n: x.reshape(B, T, heads, n)
    log_decay = kda_decay(view(rnd(F.linear(dec_h, p["decay_proj.weight"])), rk),
                          p["associative_log_rate"], p["associative_decay_bias"])
    if not decay_enabled:
        log_decay = torch.zeros_like(log_decay)
    if taps is not None:
        taps.append(log_decay)
    gamma = torch.sigmoid(geo + p["geometry_write_bias"].view(1, 1, heads))
    if not geometry_enabled:
        gamma = torch.zeros_like(gamma)
    gate = view(rnd(F.linear(gate_h, p["output_gate_proj.weight"], p["output_gate_proj.bias"])), rv)
    init = None if op_init is None else OracleState(*(s.double() for s in op_init))
    out, st = solvedelta_oracle(
        view(u, rk), view(h, rk), view(q, rk), k.reshape(B, T, heads, 1, rk),
        v.reshape(B, T, heads, 1, rv), log_decay, torch.sigmoid(er).reshape(B, T, heads, 1, rk),
        torch.sigmoid(wr).reshape(B, T, heads, 1, rv), gamma, initial_state=init,
        valid_mask=valid_mask, reset_mask=reset_mask)
    y = rms_norm_gated(rnd(out), gate, p["output_norm.weight"], eps)
    y = F.linear(y.reshape(B, T, heads * rv), p["output_proj.weight"], p.get("output_proj.bias"))
    return y, (st.predictor, st.S), conv_state


__all__ = ["projection_layout", "conv4_loop", "kda_decay", "rms_norm_gated", "mixer_oracle"]
