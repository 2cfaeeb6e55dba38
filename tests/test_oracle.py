"""Pins the FP64 oracle (oracle/sd_oracle.py) without running the reference.

Each check is chosen so that a plausible slip (left instead of right decay,
residual after instead of before forgetting, C instead of C^T in the primal,
a dropped radial term, S decayed after the read) fails at least one of them.
The reference's own known-answer tests these restate are cited per test
(tests/core/test_rebuild_semantics.py in the reference).
"""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle.sd_oracle import (
    RELATIVE_FRAME_RADIUS,
    OracleState,
    gdn2_oracle,
    solvedelta_oracle,
    zero_state,
)



@pytest.fixture(autouse=True)
def _fp64_default():
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    yield
    torch.set_default_dtype(old)


def small_inputs(T=6, r=8, V=5, seed=7):
    # Same shapes/scales as test_rebuild_semantics.py:31-57 (own generator).
    g = torch.Generator().manual_seed(seed)
    B, H = 2, 2
    n = lambda *s: torch.randn(*s, generator=g)
    u, h, q = n(B, T, H, r), n(B, T, H, r), n(B, T, H, r)
    keys = n(B, T, H, 1, r)
    values = n(B, T, H, 1, V)
    decay = -0.02 * torch.rand(B, T, H, r, generator=g)
    erase = torch.rand(B, T, H, 1, r, generator=g)
    write = torch.rand(B, T, H, 1, V, generator=g)
    gamma = torch.full((H,), 0.25)
    return u, h, q, keys, values, decay, erase, write, gamma


def test_closed_form_two_tokens():
    """test_rebuild_semantics.py:135-167: token 1 writes C = e2 e1^T, and the
    token-2 output is all ones (primal (I+C)^T e2 = e1 + e2, local frame I)."""
    u = torch.tensor([[[[1.0, 0.0]], [[0.0, 1.0]]]])
    h = torch.tensor([[[[0.0, 1.0]], [[0.0, 0.0]]]])
    q = torch.tensor([[[[1.0, 0.0]], [[1.0, 0.0]]]])
    keys = torch.tensor([[[[[1.0, 0.0]]], [[[0.0, 1.0]]]]])
    values = torch.tensor([0.0, 1.0]).view(1, 2, 1, 1, 1)
    out, st = solvedelta_oracle(u, h, q, keys, values, torch.zeros(1, 2, 1, 2),
                                torch.zeros_like(keys), torch.ones_like(values), torch.ones(1))
    assert torch.allclose(out[:, 1], torch.ones_like(out[:, 1]), atol=1e-14)
    assert torch.allclose(st.predictor, torch.tensor([[[[0.0, 0.0], [1.0, 0.0]]]]), atol=1e-14)


def test_pre_decay_residual_and_right_channel_decay():
    """test_rebuild_semantics.py:170-228: with h = C0 u the write is zero and
    C is right-decayed (columns), S left-decayed (rows)."""
    u = torch.tensor([[[[1.0, 0.0]]]])
    C0 = torch.tensor([[[[2.0, 3.0], [4.0, 1.0]]]])
    h = torch.tensor([[[[2.0, 4.0]]]])
    g = torch.tensor([math.log(0.25), 0.0]).view(1, 1, 1, 2)
    S0 = torch.tensor([[[[5.0], [7.0]]]])
    keys = torch.tensor([[[[[1.0, 0.0]]]]])
    values = torch.zeros(1, 1, 1, 1, 1)
    _, st = solvedelta_oracle(u, h, torch.tensor([[[[1.0, 0.0]]]]), keys, values, g,
                              torch.zeros_like(keys), torch.zeros_like(values),
                              torch.tensor([0.75]), initial_state=OracleState(C0, S0))
    ret = g[:, 0].exp()
    assert torch.allclose(st.predictor, C0 * ret[..., None, :], atol=1e-14)
    assert not torch.allclose(st.predictor, ret[..., :, None] * C0)
    assert not torch.allclose(st.predictor, g.mean().exp() * C0)
    assert torch.allclose(st.S, ret[..., :, None] * S0, atol=1e-14)


def test_chi_is_inverse_transpose_solve_and_den_bounds():
    """test_rebuild_semantics.py:60-132: chi = solve(F^T, q) with F = I + u phi^T,
    and 3/8 < den < 13/8, for every token of a random run (explicit re-derivation
    of phi from the run's own C sequence)."""
    args = small_inputs()
    u, h, q, keys, values, decay, erase, write, gamma = args
    B, T, H, r = u.shape
    un, qn = F.normalize(u, dim=-1), F.normalize(q, dim=-1)
    C = torch.zeros(B, H, r, r)
    rho = RELATIVE_FRAME_RADIUS
    for t in range(T):
        delta = gamma.view(1, H, 1) * (h[:, t] - (C @ un[:, t, ..., None])[..., 0])
        C = C * decay[:, t].exp()[..., None, :] + delta[..., :, None] * un[:, t, ..., None, :]
        phi = rho * delta / torch.sqrt(rho ** 2 + delta.square().sum(-1, keepdim=True))
        den = 1 + (phi * un[:, t]).sum(-1)
        assert torch.all(den > 3 / 8) and torch.all(den < 13 / 8)
        Fm = torch.eye(r) + un[:, t, ..., :, None] * phi[..., None, :]
        chi_solve = torch.linalg.solve(Fm.transpose(-1, -2), qn[:, t, ..., None])[..., 0]
        chi_formula = qn[:, t] - phi * ((un[:, t] * qn[:, t]).sum(-1, keepdim=True) / den[..., None])
        assert torch.allclose(chi_solve, chi_formula, atol=1e-12)


def test_adversarial_radius_bound():
    """test_rebuild_semantics.py:231-249: |delta| = 1e6 keeps den inside (3/8, 13/8)."""
    rho = RELATIVE_FRAME_RADIUS
    d = F.normalize(torch.tensor([1.0, -2.0, 3.0]), dim=0)
    for sign in (-1.0, 1.0):
        upd = sign * 1e6 * d
        phi = rho / math.sqrt(rho ** 2 + float(upd.square().sum())) * upd
        den = 1 + float(phi @ d)
        assert 1 - rho < den < 1 + rho
        assert abs(den - (1 + sign * rho)) < 1e-6


def test_gamma_zero_is_gdn2():
    """test_rebuild_semantics.py:296-316: gamma = 0 reduces exactly to GDN2."""
    args = list(small_inputs())
    args[-1] = torch.zeros_like(args[-1])
    out, st = solvedelta_oracle(*args)
    _, _, q, keys, values, decay, erase, write, _ = args
    out_g, S_g = gdn2_oracle(q, keys, values, decay, erase, write)
    assert torch.allclose(out, out_g, atol=2e-12, rtol=2e-12)
    assert torch.allclose(st.S, S_g, atol=2e-12, rtol=2e-12)
    assert torch.count_nonzero(st.predictor) == 0


def test_independent_matrix_restatement():
    """An independent restatement with explicit matrices P = I + C and
    F^-T = inv(F)^T agrees to 2e-12 (test_rebuild_semantics.py:60-132)."""
    args = small_inputs(T=5, r=6, V=4, seed=3)
    u, h, q, keys, values, decay, erase, write, gamma = args
    out, st = solvedelta_oracle(*args)
    B, T, H, r = u.shape
    V = values.shape[-1]
    for b in range(B):
        for hh in range(H):
            C = torch.zeros(r, r)
            S = torch.zeros(r, V)
            for t in range(T):
                uu = F.normalize(u[b, t, hh], dim=0)
                kk = F.normalize(keys[b, t, hh, 0], dim=0)
                qq = F.normalize(q[b, t, hh], dim=0)
                D = torch.diag(decay[b, t, hh].exp())
                delta = gamma[hh] * (h[b, t, hh] - C @ uu)
                C = C @ D + torch.outer(delta, uu)
                phi = 0.625 * delta / torch.sqrt(0.625 ** 2 + uu.dot(uu) * delta.dot(delta))
                Fm = torch.eye(r) + torch.outer(uu, phi)
                Finv_T = torch.linalg.inv(Fm).T
                d = (torch.eye(r) + C).T @ kk
                e = Finv_T @ (erase[b, t, hh, 0] * kk)
                chi = Finv_T @ qq
                S = D @ S
                S = S + torch.outer(d, write[b, t, hh, 0] * values[b, t, hh, 0] - S.T @ e)
                assert torch.allclose(out[b, t, hh], S.T @ chi, atol=2e-12, rtol=2e-12)
            assert torch.allclose(st.predictor[b, hh], C, atol=2e-12)
            assert torch.allclose(st.S[b, hh], S, atol=2e-12)


def test_masks_resets_split_and_finite_vjp():
    """test_rebuild_semantics.py:319-360."""
    args = tuple(a.clone().requires_grad_() for a in small_inputs(T=8))
    valid = torch.tensor([[1, 1, 0, 1, 1, 1, 1, 1], [1, 0, 1, 1, 1, 0, 1, 1]], dtype=torch.bool)
    reset = torch.zeros_like(valid)
    reset[0, 4] = True
    reset[1, 2] = True
    out, st = solvedelta_oracle(*args, valid_mask=valid, reset_mask=reset)
    assert torch.equal(out[~valid], torch.zeros_like(out[~valid]))
    s = 4
    lo, ls = solvedelta_oracle(*(a[:, :s] for a in args[:-1]), args[-1],
                               valid_mask=valid[:, :s], reset_mask=reset[:, :s])
    ro, rs = solvedelta_oracle(*(a[:, s:] for a in args[:-1]), args[-1], initial_state=ls,
                               valid_mask=valid[:, s:], reset_mask=reset[:, s:])
    assert torch.allclose(out, torch.cat((lo, ro), 1), atol=2e-12, rtol=2e-12)
    for a, b in zip(rs, st):
        assert torch.allclose(a, b, atol=2e-12, rtol=2e-12)
    loss = out.square().sum() + st.predictor.sum() + st.S.sum()
    grads = torch.autograd.grad(loss, args)
    assert all(torch.isfinite(gr).all() for gr in grads)


def test_reset_equals_fresh_start():
    """A reset on a valid token restarts from the zero state: the suffix equals a
    fresh run on the suffix (reference.py:156-165)."""
    args = small_inputs(T=7)
    reset = torch.zeros(2, 7, dtype=torch.bool)
    reset[:, 3] = True
    out, st = solvedelta_oracle(*args, reset_mask=reset)
    out2, st2 = solvedelta_oracle(*(a[:, 3:] for a in args[:-1]), args[-1])
    assert torch.allclose(out[:, 3:], out2, atol=1e-13)
    assert torch.allclose(st.S, st2.S, atol=1e-13)


def test_rejects_multiple_edits():
    """test_rebuild_semantics.py:363-372."""
    args = list(small_inputs())
    for i in (3, 4, 6, 7):
        args[i] = args[i].expand(-1, -1, -1, 2, -1).clone()
    with pytest.raises(ValueError, match="num_edits=1"):
        solvedelta_oracle(*args)


def test_gradcheck_small():
    """The FP64 VJP is the autograd of the loop; gradcheck pins it against
    finite differences (all 9 inputs and both initial states)."""
    g = torch.Generator().manual_seed(5)
    B, T, H, r, V = 1, 3, 1, 3, 2
    n = lambda *s: torch.randn(*s, generator=g).requires_grad_()
    ins = (n(B, T, H, r), n(B, T, H, r), n(B, T, H, r), n(B, T, H, 1, r), n(B, T, H, 1, V),
           (-0.3 * torch.rand(B, T, H, r, generator=g)).requires_grad_(),
           torch.rand(B, T, H, 1, r, generator=g).requires_grad_(),
           torch.rand(B, T, H, 1, V, generator=g).requires_grad_(),
           torch.full((B, T, H), 0.6).requires_grad_(),
           (0.3 * torch.randn(B, H, r, r, generator=g)).requires_grad_(),
           (0.3 * torch.randn(B, H, r, V, generator=g)).requires_grad_())

    def f(*a):
        o, s = solvedelta_oracle(*a[:9], initial_state=OracleState(a[9], a[10]))
        return o, s.predictor, s.S

    assert torch.autograd.gradcheck(f, ins, eps=1e-6, atol=1e-6, rtol=1e-5)
