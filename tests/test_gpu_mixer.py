"""GPU parity of the mixer frontend / readout kernels and of the whole mixer
layer against the FP64 mixer oracle (oracle/mixer_oracle.py), on the same
bf16-quantised inputs and parameters.

Tolerances: elementwise kernels whose output is bf16 are held to the bf16
rounding (rel-Frobenius < 1e-2); FP32 outputs and parameter gradients to 1e-4
(gate) / 1e-3 (reductions over many tokens, done in FP32).  The full layer
compounds bf16 roundings of every projection, so it uses the reference's
operator gate (rel-Frobenius < 3e-2) on outputs, states and gradients."""
import math

import pytest
import torch

from gpu_common import rel
from oracle.mixer_oracle import conv4_loop, kda_decay, mixer_oracle, rms_norm_gated

BF16 = lambda t: t.to(torch.bfloat16).double()  # the oracle's bf16 activation points

pytestmark = pytest.mark.gpu


def _mx():
    from solvedelta_amd import mixer
    return mixer


def _d(t):
    return t.detach().double().cpu()


@pytest.mark.parametrize("B,T,D,with_init", [(2, 130, 300, True), (1, 2, 40, True),
                                             (3, 1, 64, False), (2, 67, 256, False)])
def test_conv4_silu_forward_backward(B, T, D, with_init):
    mx = _mx()
    g = torch.Generator().manual_seed(B * 1000 + T)
    wide = torch.randn(B, T, D + 24, generator=g).to(torch.bfloat16).cuda()
    x = wide[..., 8:8 + D].requires_grad_()  # strided view, as the projection slice
    w = (0.5 * torch.randn(D, 4, generator=g)).cuda().requires_grad_()
    init = (torch.randn(B, D, 3, generator=g).to(torch.bfloat16).cuda().requires_grad_()
            if with_init else None)
    y, fin = mx.conv4_silu(x, w, init, return_final_state=True)
    xo = _d(x).requires_grad_()
    wo = _d(w).requires_grad_()
    io = _d(init).requires_grad_() if with_init else None
    yo, fo = conv4_loop(xo, wo, io)
    print(f"[conv B{B} T{T} D{D}] rel y {rel(y.float(), yo):.2e}", flush=True)
    assert rel(y.float(), yo) < 1e-2
    assert torch.equal(fin.float().cpu(), fo.float())      # state is a copy of inputs
    dy = torch.randn(B, T, D, generator=g).to(torch.bfloat16).cuda()
    dfin = torch.randn(B, D, 3, generator=g).to(torch.bfloat16).cuda()
    leaves = [x, w] + ([init] if with_init else [])
    grads = torch.autograd.grad((y, fin), leaves, (dy, dfin))
    oleaves = [xo, wo] + ([io] if with_init else [])
    ogr = torch.autograd.grad((yo, fo), oleaves, (_d(dy), _d(dfin)))
    for name, a, b in zip(("dx", "dw", "dinit"), grads, ogr):
        e = rel(a.float(), b)
        print(f"  {name} {e:.2e}", flush=True)
        assert e < 1e-2, name


def test_kda_gate_forward_backward():
    mx = _mx()
    g = torch.Generator().manual_seed(7)
    B, T, H, r = 2, 100, 4, 64
    raw = torch.randn(B, T, H, r, generator=g).mul(3).to(torch.bfloat16).cuda().requires_grad_()
    raw.data[0, 0, 0, :4] = torch.tensor([30.0, 25.0, -40.0, 0.0])   # threshold and tails
    lr = torch.randn(H, generator=g).cuda().requires_grad_()
    bias = torch.randn(H, r, generator=g).cuda().requires_grad_()
    out = mx.kda_decay_gate(raw, lr, bias)
    ro, lo, bo = (_d(t).requires_grad_() for t in (raw, lr, bias))
    oo = kda_decay(ro, lo, bo)
    print(f"[kda] rel out {rel(out, oo):.2e}", flush=True)
    assert out.dtype == torch.float32 and rel(out, oo) < 1e-5
    dout = torch.randn(B, T, H, r, generator=g).cuda()
    ga = torch.autograd.grad(out, (raw, lr, bias), dout)
    gb = torch.autograd.grad(oo, (ro, lo, bo), _d(dout))
    for name, a, b, tol in zip(("draw", "dlog_rate", "dbias"), ga, gb, (1e-2, 1e-4, 1e-4)):
        e = rel(a.float(), b)
        print(f"  {name} {e:.2e}", flush=True)
        assert e < tol, name


def test_rmsnorm_gated_and_linear_owner():
    mx = _mx()
    g = torch.Generator().manual_seed(11)
    B, T, H, V, hidden = 2, 33, 4, 64, 96
    x = torch.randn(B, T, H, V, generator=g).to(torch.bfloat16).cuda().requires_grad_()
    gate = torch.randn(B, T, H, V, generator=g).to(torch.bfloat16).cuda().requires_grad_()
    norm = mx.RMSNormGated(V).cuda()
    with torch.no_grad():
        norm.weight.copy_(torch.linspace(0.5, 1.5, V))
    lin = torch.nn.Linear(H * V, hidden, bias=True).cuda().to(torch.bfloat16)
    y = norm(x, gate)
    xo, go, wo = _d(x).requires_grad_(), _d(gate).requires_grad_(), _d(norm.weight).requires_grad_()
    yo = rms_norm_gated(xo, go, wo, norm.eps)
    print(f"[rms] rel y {rel(y.float(), yo):.2e}", flush=True)
    assert rel(y.float(), yo) < 1e-2
    dy = torch.randn(B, T, H, V, generator=g).to(torch.bfloat16).cuda()
    ga = torch.autograd.grad(y, (x, gate, norm.weight), dy)
    gb = torch.autograd.grad(yo, (xo, go, wo), _d(dy))
    for name, a, b in zip(("dx", "dgate", "dweight"), ga, gb):
        e = rel(a.float(), b)
        print(f"  {name} {e:.2e}", flush=True)
        assert e < 1e-2, name
    # fused norm + projection owner (ops/norm_gate.py:46-150)
    out = norm.forward_linear(x, gate, lin)
    lw, lb = _d(lin.weight).requires_grad_(), _d(lin.bias).requires_grad_()
    oo = torch.nn.functional.linear(rms_norm_gated(xo, go, wo, norm.eps).reshape(B, T, -1), lw, lb)
    assert rel(out.float(), oo) < 1e-2
    do = torch.randn(B, T, hidden, generator=g).to(torch.bfloat16).cuda()
    ga = torch.autograd.grad(out, (x, gate, norm.weight, lin.weight, lin.bias), do)
    gb = torch.autograd.grad(oo, (xo, go, wo, lw, lb), _d(do))
    for name, a, b in zip(("dx", "dgate", "dnorm", "dlin_w", "dlin_b"), ga, gb):
        e = rel(a.float(), b)
        print(f"  linear {name} {e:.2e}", flush=True)
        assert e < 1.5e-2, name


def _layer(hidden=256, H=4, r=64, conv=True, seed=0):
    mx = _mx()
    torch.manual_seed(seed)
    cfg = mx.SolveDeltaMixerConfig(hidden_size=hidden, num_heads=H, head_k_dim=r, head_v_dim=r,
                                   use_short_conv=conv)
    layer = mx.SolveDelta(cfg)
    with torch.no_grad():   # non-trivial norm and gate parameters
        layer.output_norm.weight.uniform_(0.5, 1.5)
    return layer.cuda().to(torch.bfloat16)


def _params(layer):
    return {k: _d(v) for k, v in layer.named_parameters()}


def test_mixer_config0_forward_and_state():
    """hidden 256, H 4, r = V = 64, B 2, T 128."""
    layer = _layer()
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 128, 256, generator=g).to(torch.bfloat16).cuda()
    with torch.no_grad():
        y, st = layer(x, return_final_state=True)
    yo, (Co, So), conv_o = mixer_oracle(_params(layer), _d(x), heads=4, rk=64, rv=64)
    ey, eC, eS = rel(y.float(), yo), rel(st.operator.predictor, Co), rel(st.operator.S, So)
    ec = rel(st.conv.float(), conv_o)
    print(f"[mixer cfg0] rel y {ey:.2e} C {eC:.2e} S {eS:.2e} conv {ec:.2e}", flush=True)
    assert ey < 3e-2 and eC < 3e-2 and eS < 3e-2 and ec < 1e-2
    assert y.shape == x.shape and y.dtype == torch.bfloat16
    # the oracle on the bf16 layer's own activation points: what is left is the
    # kernels' arithmetic (and an occasional one-ulp difference in a rounded
    # activation), so the states meet the operator-level bound
    yb, (Cb, Sb), _ = mixer_oracle(_params(layer), _d(x), heads=4, rk=64, rv=64, act_round=BF16)
    eyb, eCb, eSb = rel(y.float(), yb), rel(st.operator.predictor, Cb), rel(st.operator.S, Sb)
    print(f"[mixer cfg0, bf16 activation points] rel y {eyb:.2e} C {eCb:.2e} S {eSb:.2e}",
          flush=True)
    assert eyb < 1e-2 and eCb < 1e-3 and eSb < 1e-3


def test_mixer_gradients_against_oracle():
    layer = _layer(hidden=128, H=2, r=64, seed=1)
    g = torch.Generator().manual_seed(4)
    x = torch.randn(2, 80, 128, generator=g).to(torch.bfloat16).cuda().requires_grad_()
    dy = torch.randn(2, 80, 128, generator=g).to(torch.bfloat16).cuda()
    y = layer(x)
    names = [n for n, _ in layer.named_parameters()]
    ga = torch.autograd.grad(y, [x] + list(layer.parameters()), dy)
    po = {k: v.requires_grad_() for k, v in _params(layer).items()}
    xo = _d(x).requires_grad_()
    yo, _, _ = mixer_oracle(po, xo, heads=2, rk=64, rv=64)
    gb = torch.autograd.grad(yo, [xo] + [po[n] for n in names], _d(dy))
    worst = 0.0
    for name, a, b in zip(["hidden"] + names, ga, gb):
        e = rel(a.float(), b)
        worst = max(worst, e)
        print(f"  d{name} {e:.2e}", flush=True)
        assert e < 3e-2, name
    print(f"[mixer grads] worst {worst:.2e}", flush=True)


def test_mixer_masks_resets_and_continuation():
    layer = _layer(hidden=128, H=2, r=32, seed=2)
    g = torch.Generator().manual_seed(5)
    B, T = 2, 48
    x = torch.randn(B, T, 128, generator=g).to(torch.bfloat16).cuda()
    valid = torch.rand(B, T, generator=g) > 0.2
    reset = torch.rand(B, T, generator=g) > 0.9
    valid[1, 40:] = False
    mx = _mx()
    C0 = 0.02 * torch.randn(B, 2, 32, 32, generator=g)
    S0 = 0.02 * torch.randn(B, 2, 32, 32, generator=g)
    conv0 = torch.randn(B, 3 * 64, 3, generator=g).to(torch.bfloat16)
    from solvedelta_amd import SolveDeltaState
    init = mx.SolveDeltaLayerState(SolveDeltaState(C0.cuda(), S0.cuda()), conv0.cuda())
    with torch.no_grad():
        y, st = layer(x, initial_state=init, valid_mask=valid.cuda(), reset_mask=reset.cuda(),
                      return_final_state=True)
    yo, (Co, So), conv_o = mixer_oracle(_params(layer), _d(x), heads=2, rk=32, rv=32,
                                        initial_state=((C0.double(), S0.double()), _d(conv0)),
                                        valid_mask=valid, reset_mask=reset)
    ey, eC, eS = rel(y.float(), yo), rel(st.operator.predictor, Co), rel(st.operator.S, So)
    print(f"[mixer masks] rel y {ey:.2e} C {eC:.2e} S {eS:.2e}", flush=True)
    assert torch.all(y[~valid.cuda()] == 0)
    assert ey < 3e-2 and eC < 3e-2 and eS < 3e-2
    assert rel(st.conv.float(), conv_o) < 1e-2   # projections differ by bf16 GEMM rounding
    # continuation: two calls with the carried layer state equal one call
    with torch.no_grad():
        yf, sf = layer(x, return_final_state=True)
        y1, s1 = layer(x[:, :20], return_final_state=True)
        y2, s2 = layer(x[:, 20:], initial_state=s1, return_final_state=True)
    assert rel(torch.cat((y1, y2), 1).float(), yf.float()) < 1e-2
    assert torch.equal(s2.conv, sf.conv)
    assert rel(s2.operator.S, sf.operator.S) < 1e-2


@pytest.mark.parametrize("with_init", [True, False])
def test_conv4_masked_matches_oracle_loop_with_grads(with_init):
    """conv4 + SiLU under valid / reset masks (no repacking) against the FP64
    CPU loop (oracle conv4_loop, model.py:146-164): output, final state and the
    gradients of x, the weight and the initial state."""
    from oracle.mixer_oracle import conv4_loop
    from solvedelta_amd.mixer import conv4_silu_masked
    g = torch.Generator().manual_seed(31)
    B, T, D = 3, 77, 200
    x = torch.randn(B, T, D, generator=g).to(torch.bfloat16)
    w = 0.5 * torch.randn(D, 4, generator=g)
    init = torch.randn(B, D, 3, generator=g).to(torch.bfloat16) if with_init else None
    valid = torch.rand(B, T, generator=g) > 0.25
    reset = torch.rand(B, T, generator=g) > 0.9
    reset[0, 0] = True
    valid[2, :] = False            # a row with no valid token keeps its initial state
    valid[1, 70:] = False
    xc = x.cuda().requires_grad_()
    wc = w.cuda().requires_grad_()
    ic = init.cuda().float().requires_grad_() if with_init else None
    y, fin = conv4_silu_masked(xc, wc, valid.cuda(), reset.cuda(), ic, True)
    xr = x.double().requires_grad_()
    wr = w.double().requires_grad_()
    ir = init.double().requires_grad_() if with_init else None
    yo, fo = conv4_loop(xr, wr, ir, valid_mask=valid, reset_mask=reset)
    assert torch.all(y[~valid.cuda()] == 0)
    cy = torch.randn(B, T, D, generator=g)
    cf = torch.randn(B, D, 3, generator=g)
    grads = torch.autograd.grad((y, fin), [xc, wc] + ([ic] if with_init else []),
                                (cy.to(torch.bfloat16).cuda(), cf.to(torch.bfloat16).cuda()))
    rg = torch.autograd.grad((yo, fo), [xr, wr] + ([ir] if with_init else []),
                             (cy.to(torch.bfloat16).double(), cf.to(torch.bfloat16).double()))
    errs = [rel(y.float(), yo), rel(fin.float(), fo)] + [rel(a.float(), b) for a, b in zip(grads, rg)]
    print(f"[conv masked init={with_init}] " + " ".join(f"{e:.1e}" for e in errs), flush=True)
    assert errs[1] == 0.0          # the final state is a copy of bf16 inputs
    assert max(errs) < 5e-3
    assert torch.all(grads[0][~valid.cuda()] == 0)


def test_mixer_masks_backward_matches_oracle():
    """The masked mixer (masked conv4 + masked operator, no repacking) forward and
    every parameter / input gradient against the FP64 mixer oracle."""
    mx = _mx()
    layer = _layer(hidden=128, H=2, r=32, seed=3)
    g = torch.Generator().manual_seed(7)
    B, T = 2, 70
    x = torch.randn(B, T, 128, generator=g).to(torch.bfloat16).cuda().requires_grad_()
    valid = torch.rand(B, T, generator=g) > 0.2
    reset = torch.rand(B, T, generator=g) > 0.93
    y = layer(x, valid_mask=valid.cuda(), reset_mask=reset.cuda())
    params = _params(layer)
    for p in params.values():
        p.requires_grad_()
    xd = _d(x).requires_grad_()
    yo, _, _ = mixer_oracle(params, xd, heads=2, rk=32, rv=32, valid_mask=valid, reset_mask=reset)
    cot = torch.randn(y.shape, generator=g)
    names = [n for n, _ in layer.named_parameters()]
    grads = torch.autograd.grad(y, [x] + [p for _, p in layer.named_parameters()],
                                cot.to(y.device, y.dtype))
    rg = torch.autograd.grad(yo, [xd] + [params[n] for n in names], cot.double())
    errs = {"y": rel(y.float(), yo), "x": rel(grads[0].float(), rg[0])}
    for n, a, b in zip(names, grads[1:], rg[1:]):
        errs[n] = rel(a.float(), b)
    print("[mixer masks bwd] " + " ".join(f"{k}={v:.1e}" for k, v in errs.items()), flush=True)
    for k, v in errs.items():
        assert v < 3e-2, (k, v)
