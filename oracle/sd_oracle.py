"""FP64 token-loop oracle for the SolveDelta recurrence (test infrastructure only).

This is a restatement of the reference's token loop
(``causallsso/reference.py:82-229``) in our own code.  It is the checker for the
HIP path: the product code never imports it.  Autograd through this loop gives
the FP64 VJP oracle (the reference gets its gradients the same way,
``tests/core/test_rebuild_semantics.py:540-597``).

Per token, with u, q, k L2-normalised, D = diag(exp(g)):

    r     = h - C u                 residual against the un-forgotten C
    delta = gamma r
    C'    = C D + delta u^T         right (source-axis) decay
    phi   = rho delta / sqrt(rho^2 + |u|^2 |delta|^2),  rho = 5/8
    den   = 1 + phi.u
    d     = k + C'^T k              primal address through I + C'
    e     = b - phi (u.b)/den       b = sigmoid(erase) * k  (dual, F^-T b)
    chi   = q - phi (u.q)/den       (query, F^-T q)
    S~    = D S
    S'    = S~ + d (z - S~^T e)^T   z = sigmoid(write) * v
    o     = S'^T chi

Invalid tokens (valid_mask False) emit zero and keep the state; a reset on a
valid token restarts from the zero state (``reference.py:156-227``).

Parity status: every function here is pinned by ``tests/test_oracle.py``
(closed-form known answers, the GDN2 reduction, the ``linalg.solve`` identity
for chi, denominator bounds, split/mask/reset invariants and ``gradcheck``).
"""

from __future__ import annotations

from typing import NamedTuple, Optional

import torch
import torch.nn.functional as F

RELATIVE_FRAME_RADIUS = 5.0 / 8.0


class OracleState(NamedTuple):
    predictor: torch.Tensor  # C  [B,H,r,r], prediction = C @ u
    S: torch.Tensor  # S  [B,H,r,V]


def zero_state(batch, heads, rank, value_dim, dtype=torch.float64, device="cpu"):
    return OracleState(
        torch.zeros(batch, heads, rank, rank, dtype=dtype, device=device),
        torch.zeros(batch, heads, rank, value_dim, dtype=dtype, device=device),
    )


def _check_shapes(u, h, q, keys, values, log_decay, erase, write, gamma):
    """Shape contract of ``reference.py:38-79`` (ValueError on mismatch)."""
    if u.ndim != 4:
        raise ValueError("u must have shape [B,T,H,r]")
    B, T, H, r = u.shape
    if h.shape != u.shape or q.shape != u.shape:
        raise ValueError("h and q must match u")
    if keys.ndim != 5 or keys.shape[:3] != (B, T, H):
        raise ValueError("keys must have shape [B,T,H,K,r]")
    K, kr = keys.shape[-2:]
    if kr != r:
        raise ValueError("key width must equal r")
    if values.ndim != 5 or values.shape[:4] != (B, T, H, K):
        raise ValueError("values must have shape [B,T,H,K,d_v]")
    if log_decay.shape != (B, T, H, r):
        raise ValueError("associative_log_decay must have shape [B,T,H,r]")
    if erase.shape != keys.shape:
        raise ValueError("erase must match keys")
    if write.shape != values.shape:
        raise ValueError("write must match values")
    if gamma.shape not in ((H,), (1, H), (B, T, H)):
        raise ValueError("geometry_write must have shape [H], [1,H], or [B,T,H]")
    if K != 1:
        raise ValueError("the current SolveDelta contract requires num_edits=1")
    return B, T, H, r, values.shape[-1]


def solvedelta_oracle(
    u, h, q, keys, values, log_decay, erase, write, gamma,
    *, initial_state: Optional[OracleState] = None,
    valid_mask: Optional[torch.Tensor] = None,
    reset_mask: Optional[torch.Tensor] = None,
):
    """Token loop with *activated* gates ``erase``/``write`` in [0,1].

    Follows ``reference.py:82-229`` step by step; batched over (B,H).
    Returns ``(output [B,T,H,V], OracleState)``.
    """
    B, T, H, r, V = _check_shapes(u, h, q, keys, values, log_decay, erase, write, gamma)
    dt, dev = u.dtype, u.device
    if valid_mask is None:
        valid_mask = torch.ones(B, T, dtype=torch.bool, device=dev)
    if reset_mask is None:
        reset_mask = torch.zeros(B, T, dtype=torch.bool, device=dev)
    zero = zero_state(B, H, r, V, dtype=dt, device=dev)
    C, S = (zero if initial_state is None else initial_state)
    if C.shape != zero.predictor.shape or S.shape != zero.S.shape:
        raise ValueError("initial_state shapes do not match inputs")
    u = F.normalize(u, p=2, dim=-1)
    q = F.normalize(q, p=2, dim=-1)
    k_all = F.normalize(keys[:, :, :, 0], p=2, dim=-1)
    erase = erase[:, :, :, 0]
    write = write[:, :, :, 0]
    values = values[:, :, :, 0]
    gamma = gamma.to(dt)
    if gamma.shape != (B, T, H):
        gamma = gamma.reshape(1, 1, H).expand(B, T, H)
    rho = RELATIVE_FRAME_RADIUS
    outs = []
    for t in range(T):
        valid = valid_mask[:, t]
        reset = reset_mask[:, t] & valid
        C = torch.where(reset[:, None, None, None], zero.predictor, C)
        S = torch.where(reset[:, None, None, None], zero.S, S)
        ut, kt, qt = u[:, t], k_all[:, t], q[:, t]
        decay = log_decay[:, t].exp()  # [B,H,r]
        delta = gamma[:, t, :, None] * (h[:, t] - torch.einsum("bhij,bhj->bhi", C, ut))
        C_new = C * decay[..., None, :] + delta[..., :, None] * ut[..., None, :]
        usq = (ut * ut).sum(-1, keepdim=True)
        dsq = (delta * delta).sum(-1, keepdim=True)
        phi = rho / torch.sqrt(rho * rho + usq * dsq) * delta
        den = 1.0 + (phi * ut).sum(-1, keepdim=True)
        d = kt + torch.einsum("bhij,bhi->bhj", C_new, kt)
        b = erase[:, t] * kt
        e = b - phi * ((ut * b).sum(-1, keepdim=True) / den)
        chi = qt - phi * ((ut * qt).sum(-1, keepdim=True) / den)
        S_dec = decay[..., :, None] * S
        pred = torch.einsum("bhrv,bhr->bhv", S_dec, e)
        z = write[:, t] * values[:, t]
        S_new = S_dec + d[..., :, None] * (z - pred)[..., None, :]
        o = torch.einsum("bhrv,bhr->bhv", S_new, chi)
        outs.append(torch.where(valid[:, None, None], o, torch.zeros_like(o)))
        C = torch.where(valid[:, None, None, None], C_new, C)
        S = torch.where(valid[:, None, None, None], S_new, S)
    return torch.stack(outs, dim=1), OracleState(C, S)


def solvedelta_oracle_raw(u, h, q, keys, values, log_decay, erase_raw, write_raw, gamma, **kw):
    """Oracle with *raw* gate logits, the convention of the native operator.

    The native entry applies the sigmoids itself (``sources.py:87-88,119-120``);
    the reference tests compare it to ``solvedelta_reference(..., sigmoid(erase_raw),
    sigmoid(write_raw), ...)`` (``test_rebuild_semantics.py:553-559``).
    """
    return solvedelta_oracle(u, h, q, keys, values, log_decay,
                             torch.sigmoid(erase_raw), torch.sigmoid(write_raw), gamma, **kw)


def gdn2_oracle(q, keys, values, log_decay, erase, write, initial_S=None):
    """Gated-DeltaNet-2 edit/read: the gamma = 0 limit of SolveDelta.

    Restates the expected loop of ``test_rebuild_semantics.py:296-316``:
    S <- D S ; S <- S + k (z - S^T (erase*k))^T ; o = S^T q.
    """
    q = F.normalize(q, dim=-1)
    k = F.normalize(keys[:, :, :, 0], dim=-1)
    B, T, H, r = q.shape
    V = values.shape[-1]
    S = torch.zeros(B, H, r, V, dtype=q.dtype) if initial_S is None else initial_S
    outs = []
    for t in range(T):
        S = log_decay[:, t].exp()[..., None] * S
        kt = k[:, t]
        pred = torch.einsum("bhrv,bhr->bhv", S, erase[:, t, :, 0] * kt)
        S = S + kt[..., :, None] * (write[:, t, :, 0] * values[:, t, :, 0] - pred)[..., None, :]
        outs.append(torch.einsum("bhrv,bhr->bhv", S, q[:, t]))
    return torch.stack(outs, 1), S


__all__ = ["RELATIVE_FRAME_RADIUS", "OracleState", "zero_state", "solvedelta_oracle",
           "solvedelta_oracle_raw", "gdn2_oracle"]
