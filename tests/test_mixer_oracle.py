"""Pins the FP64 mixer oracle (oracle/mixer_oracle.py) with checks that do not
restate its formulas: an independent conv1d formulation, brute-force masks,
the reference test's closed forms and sizes, limits and gradcheck."""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle.mixer_oracle import conv4_loop, kda_decay, mixer_oracle, projection_layout, rms_norm_gated


def test_projection_layout_matches_reference_sizes():
    # test_modeling_solvedelta.py:187-202 (hidden 32, 2 heads, r = V = 16)
    sizes, width, pad = projection_layout(32, 2, 16, 16)
    assert sizes == (32, 32, 32, 32, 32, 32, 32, 2, 16, 16)
    assert width == 258 and pad == 62 and width + pad == 320
    # config 0 (hidden 256, H 4, r = V = 64): 1924 -> 1984
    _, width, pad = projection_layout(256, 4, 64, 64)
    assert width == 1924 and width + pad == 1984


def test_conv4_loop_equals_conv1d_on_state_prefixed_sequence():
    g = torch.Generator().manual_seed(0)
    B, T, D = 3, 11, 7
    x = torch.randn(B, T, D, generator=g, dtype=torch.float64)
    w = torch.randn(D, 4, generator=g, dtype=torch.float64)
    st = torch.randn(B, D, 3, generator=g, dtype=torch.float64)
    y, fin = conv4_loop(x, w, st)
    seq = torch.cat((st, x.transpose(1, 2)), dim=-1)          # [B, D, 3+T]
    ref = F.silu(F.conv1d(seq, w[:, None, :], groups=D)).transpose(1, 2)
    torch.testing.assert_close(y, ref, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(fin, seq[..., -3:], rtol=0, atol=0)
    # T < 3: the final state still holds the newest three of (state, tokens)
    y2, fin2 = conv4_loop(x[:, :2], w, st)
    torch.testing.assert_close(fin2, torch.cat((st, x[:, :2].transpose(1, 2)), -1)[..., -3:])


def test_conv4_loop_masks_equal_brute_force_segments():
    g = torch.Generator().manual_seed(1)
    B, T, D = 2, 12, 5
    x = torch.randn(B, T, D, generator=g, dtype=torch.float64)
    w = torch.randn(D, 4, generator=g, dtype=torch.float64)
    st = torch.randn(B, D, 3, generator=g, dtype=torch.float64)
    valid = torch.rand(B, T, generator=g) > 0.25
    reset = torch.rand(B, T, generator=g) > 0.8
    y, fin = conv4_loop(x, w, st, valid, reset)
    for b in range(B):
        hist = st[b].clone()                                    # [D, 3]
        for t in range(T):
            if not valid[b, t]:
                assert torch.all(y[b, t] == 0)
                continue
            if reset[b, t]:
                hist = torch.zeros_like(hist)
            window = torch.cat((hist, x[b, t][:, None]), -1)
            torch.testing.assert_close(y[b, t], F.silu((window * w).sum(-1)))
            hist = window[:, 1:]
        torch.testing.assert_close(fin[b], hist)


def test_rms_norm_gated_closed_form_and_vjp():
    # test_rebuild_semantics.py:251-276 closed form, :279-293 gradcheck
    torch.manual_seed(13)
    x = torch.randn(2, 5, 2, 12, dtype=torch.float64)
    gate = torch.randn_like(x)
    w = torch.linspace(0.5, 1.5, 12, dtype=torch.float64)
    ms = (x ** 2).sum(-1, keepdim=True) / 12
    expected = x / torch.sqrt(ms + 1e-6) * w / (1 + torch.exp(-gate))
    torch.testing.assert_close(rms_norm_gated(x, gate, w, 1e-6), expected, rtol=2e-12, atol=2e-12)
    xs = torch.randn(2, 3, 2, 5, dtype=torch.float64, requires_grad=True)
    gs = torch.randn_like(xs, requires_grad=True)
    ws = torch.rand(5, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(lambda a, b, c: rms_norm_gated(a, b, c, 1e-6), (xs, gs, ws),
                                    eps=1e-6, atol=1e-5, rtol=1e-4)


def test_kda_decay_limits_and_derivative():
    H, r = 3, 4
    lr = torch.tensor([0.0, math.log(2.0), math.log(16.0)], dtype=torch.float64)
    bias = torch.zeros(H, r, dtype=torch.float64)
    big = torch.full((1, 1, H, r), 40.0, dtype=torch.float64)
    # softplus(x) -> x far above 0: log-decay -> -rate * x
    torch.testing.assert_close(kda_decay(big, lr, bias),
                               -torch.exp(lr).view(1, 1, H, 1) * 40.0 * torch.ones_like(big))
    small = torch.full((1, 1, H, r), -30.0, dtype=torch.float64)
    # softplus(x) -> e^x far below 0
    torch.testing.assert_close(kda_decay(small, lr, bias),
                               -torch.exp(lr).view(1, 1, H, 1) * math.exp(-30.0) * torch.ones_like(small),
                               rtol=1e-10, atol=0)
    # at raw + bias = 0: -rate * log 2; derivative -rate * sigmoid(0) = -rate / 2
    raw = torch.zeros(1, 1, H, r, dtype=torch.float64, requires_grad=True)
    out = kda_decay(raw, lr, bias)
    torch.testing.assert_close(out.detach(), -torch.exp(lr).view(1, 1, H, 1) * math.log(2.0) * torch.ones_like(out))
    (g,) = torch.autograd.grad(out.sum(), raw)
    torch.testing.assert_close(g, -torch.exp(lr).view(1, 1, H, 1) / 2 * torch.ones_like(g))
    assert torch.all(kda_decay(torch.randn(2, 3, H, r, dtype=torch.float64), lr, bias) < 0)


def test_mixer_oracle_gamma_zero_no_conv_reduces_to_gdn2_layer():
    """With geometry off the operator is the GDN2 edit (reference.py), so the
    mixer's output only depends on (q, k, v, decay, gates): changing the u and h
    rows of in_proj must leave it unchanged."""
    g = torch.Generator().manual_seed(5)
    hidden, H, r = 16, 2, 8
    sizes, width, pad = projection_layout(hidden, H, r, r)
    p = {
        "in_proj.weight": 0.3 * torch.randn(width + pad, hidden, generator=g),
        "conv_weight": torch.randn(sum(sizes[:3]), 4, generator=g),
        "decay_proj.weight": 0.3 * torch.randn(H * r, r, generator=g),
        "output_gate_proj.weight": 0.3 * torch.randn(H * r, r, generator=g),
        "output_gate_proj.bias": torch.zeros(H * r),
        "output_norm.weight": torch.ones(r),
        "output_proj.weight": 0.3 * torch.randn(hidden, H * r, generator=g),
        "geometry_write_bias": torch.full((H,), math.log(9.0)),
        "associative_log_rate": torch.zeros(H),
        "associative_decay_bias": torch.zeros(H, r),
    }
    x = torch.randn(2, 7, hidden, generator=g, dtype=torch.float64)
    y1, _, _ = mixer_oracle(p, x, heads=H, rk=r, rv=r, geometry_enabled=False)
    p2 = dict(p)
    w = p["in_proj.weight"].clone()
    off = sum(sizes[:3])
    w[off:off + 2 * H * r] = torch.randn(2 * H * r, hidden, generator=g)
    p2["in_proj.weight"] = w
    y2, _, _ = mixer_oracle(p2, x, heads=H, rk=r, rv=r, geometry_enabled=False)
    torch.testing.assert_close(y1, y2, rtol=1e-12, atol=1e-12)
    y3, _, _ = mixer_oracle(p2, x, heads=H, rk=r, rv=r, geometry_enabled=True)
    assert (y3 - y1).abs().max() > 1e-6
