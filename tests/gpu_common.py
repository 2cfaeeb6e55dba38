"""Shared helpers for the GPU parity tests: seeded inputs in the reference's
conventions and error metrics against the FP64 oracle."""
from __future__ import annotations

import torch
import torch.nn.functional as F

from oracle.sd_oracle import OracleState, solvedelta_oracle_raw


def make_inputs(B, T, H, r, V, *, seed=0, device="cuda", decay="softplus", gamma=0.9,
                gamma_shape="BTH", requires_grad=False, gate_scale=1.0):
    """Config-1 style inputs: u,h,q,k,v ~ N(0,1) bf16 (q,k per-head L2-normalised),
    raw erase/write ~ N(0,1), log-decay = -softplus(N(0,1)), gamma constant.
    Other decays: "small" (near 1), "extreme" (-100, every block wild), "mixed"
    (wild and ordinary coordinates side by side), anything else zero."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    n = lambda *s: torch.randn(*s, generator=g)
    u, h = n(B, T, H, r), n(B, T, H, r)
    q = F.normalize(n(B, T, H, r), dim=-1)
    k = F.normalize(n(B, T, H, 1, r), dim=-1)
    v = n(B, T, H, 1, V)
    er, wr = gate_scale * n(B, T, H, 1, r), gate_scale * n(B, T, H, 1, V)
    if decay == "softplus":
        gd = -F.softplus(n(B, T, H, r))
    elif decay == "small":
        gd = -0.02 * torch.rand(B, T, H, r, generator=g)
    elif decay == "extreme":
        gd = torch.full((B, T, H, r), -100.0)
    elif decay == "mixed":
        # three tiers of coordinates: x8 (16-token block drops ~100, always past
        # the kernels' wild threshold of 60), x4.5 (drops ~58: wild in some
        # blocks only) and x1 (~13, never), so exact wild fix-ups and ordinary
        # coordinates meet in one block
        fast = torch.tensor([8.0, 4.5, 1.0]).repeat(r // 3 + 1)[:r]
        gd = -F.softplus(n(B, T, H, r)) * fast
    else:
        gd = torch.zeros(B, T, H, r)
    if gamma_shape == "BTH":
        gm = torch.full((B, T, H), float(gamma))
    elif gamma_shape == "H":
        gm = torch.full((H,), float(gamma))
    else:
        gm = torch.full((1, H), float(gamma))
    bf = lambda x: x.to(torch.bfloat16).to(device)
    args = [bf(u), bf(h), bf(q), bf(k), bf(v), gd.float().to(device), bf(er), bf(wr),
            gm.float().to(device)]
    if requires_grad:
        args = [a.requires_grad_() for a in args]
    return args


def make_state(B, H, r, V, *, seed=1, scale=0.02, device="cuda", requires_grad=False):
    g = torch.Generator(device="cpu").manual_seed(seed)
    C = (scale * torch.randn(B, H, r, r, generator=g)).to(device)
    S = (scale * torch.randn(B, H, r, V, generator=g)).to(device)
    if requires_grad:
        C.requires_grad_()
        S.requires_grad_()
    return C, S


def oracle_of(args, state=None, **kw):
    """FP64 oracle on the exact (bf16-quantised) inputs, on the CPU."""
    d = [a.detach().double().cpu() for a in args]
    st = None if state is None else OracleState(*(s.detach().double().cpu() for s in state))
    return solvedelta_oracle_raw(*d, initial_state=st, **kw)


def rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def max_rel(a, b):
    """max |a-b| / max |b| (max-norm relative error)."""
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).abs().max() / b.abs().max().clamp_min(1e-30)).item()


def c_token_loop():
    """The FP64/FP32 C token loop (oracle/sd_token_loop.c), built on demand."""
    import ctypes
    import os
    import subprocess
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    so = os.path.join(root, "oracle", "libsd_token_loop.so")
    if not os.path.exists(so):
        subprocess.run(["make", "-C", os.path.join(root, "oracle")], check=True)
    return ctypes.CDLL(so)


def c_forward_f64(ins, state):
    """Runs the C FP64 token loop on operator inputs (raw gates, any device) and an
    initial (C, S); returns (out [B,T,H,V], C_T, S_T) as fp32 CPU tensors."""
    import ctypes
    import numpy as np
    B, T, H, r = ins[0].shape
    V = ins[4].shape[-1]
    arr = lambda x: np.ascontiguousarray(
        x.detach().float().cpu().numpy().reshape(*x.shape[:3], -1) if x.dim() == 5
        else x.detach().float().cpu().numpy())
    a = [arr(x) for x in ins]
    C = np.ascontiguousarray(state[0].detach().float().cpu().numpy())
    S = np.ascontiguousarray(state[1].detach().float().cpu().numpy())
    o = np.zeros((B, T, H, V), np.float32)
    ptr = lambda z: z.ctypes.data_as(ctypes.c_void_p)
    rc = c_token_loop().sd_cpu_forward_f64(B, T, H, r, V, *(ptr(z) for z in a), ptr(C), ptr(S),
                                           ptr(o))
    assert rc == 0
    return torch.from_numpy(o), torch.from_numpy(C), torch.from_numpy(S)


def check_lm_against_oracle(model, ids, loss, tag, layers, heads, rk, rv):
    """Loss and every parameter gradient of a SolveDelta causal LM (grads already
    in p.grad) against the FP64 LM oracle on the same parameters.  Bounds: loss
    rel 5e-3; every gradient rel-Frobenius 5e-2, except the decay rates'
    d loss / d log_rate[h] = sum over (b, t, c) of dlog_decay * log_decay, whose
    terms cancel to ~1e-3 of their magnitude: it is bounded against the sum of
    the terms' magnitudes (what carries over is each term's bf16 rounding)."""
    from oracle.lm_oracle import lm_oracle
    params = {n: p.detach().double().cpu().requires_grad_() for n, p in model.named_parameters()}
    taps = []
    ref_loss, _ = lm_oracle(params, ids.cpu(), ids.cpu(), layers=layers, heads=heads, rk=rk,
                            rv=rv, taps=taps)
    for t in taps:
        t.retain_grad()
    ref_loss.backward()
    e_loss = abs(loss.item() - ref_loss.item()) / abs(ref_loss.item())
    errs = {n: rel(p.grad.float(), params[n].grad) for n, p in model.named_parameters()}
    print(f"[{tag}] loss {loss.item():.6f} oracle {ref_loss.item():.6f} rel {e_loss:.1e}",
          flush=True)
    for n, e in sorted(errs.items(), key=lambda kv: -kv[1])[:6]:
        print(f"  {n} {e:.2e}", flush=True)
    assert e_loss < 5e-3
    for n, e in errs.items():
        if not n.endswith("associative_log_rate"):
            assert e < 5e-2, (n, e)
    for i, ld in enumerate(taps):
        scale = (ld.grad * ld).abs().sum(dim=(0, 1, 3)).detach()
        n = f"model.layers.{i}.mixer.mixer.associative_log_rate"
        err = (model.get_parameter(n).grad.double().cpu() - params[n].grad).abs()
        print(f"  {n}: |err| {err.tolist()} vs sum|terms| {scale.tolist()}", flush=True)
        assert torch.all(err < 5e-3 * scale), n
