"""The chunked algorithm the HIP kernels implement (tests/chunk_model.py) equals
the FP64 token-loop oracle, forward and full VJP, to FP64 round-off.

This pins the kernel algebra (block-centred factorisation, wild-coordinate
fix-up, WY inverse, state passes, closed-form chunk VJP and the reverse-cumsum
decay closure) independently of any GPU."""
import pytest
import torch
import torch.nn.functional as F

import chunk_model as cm
from oracle.sd_oracle import OracleState, solvedelta_oracle_raw


def _case(T, r, V, seed, decay_scale=1.0, gam=0.9, extreme=False):
    g = torch.Generator().manual_seed(seed)
    n = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64)
    u, h, q, k = n(1, T, 1, r), n(1, T, 1, r), n(1, T, 1, r), n(1, T, 1, 1, r)
    v, er, wr = n(1, T, 1, 1, V), n(1, T, 1, 1, r), n(1, T, 1, 1, V)
    gd = -F.softplus(n(1, T, 1, r)) * decay_scale
    if extreme:
        gd[:, 20:40] = -100.0
    gm = torch.full((1, T, 1), gam, dtype=torch.float64)
    C0, S0 = 0.1 * n(1, 1, r, r), 0.1 * n(1, 1, r, V)
    return u, h, q, k, v, gd, er, wr, gm, C0, S0


@pytest.mark.parametrize("T,r,V,seed,scale,gam,extreme", [
    (128, 16, 12, 0, 1.0, 0.9, False),
    (192, 16, 16, 1, 1.0, 0.9, False),
    (128, 16, 12, 2, 1.0, 0.9, True),
    (128, 16, 12, 3, 4.0, 0.9, False),
    (64, 16, 12, 4, 1.0, 0.0, False),
])
def test_chunk_model_matches_oracle(T, r, V, seed, scale, gam, extreme):
    args = _case(T, r, V, seed, scale, gam, extreme)
    leaves = [a.clone().requires_grad_() for a in args]
    o, st = solvedelta_oracle_raw(*leaves[:9], initial_state=OracleState(leaves[9], leaves[10]))
    g = torch.Generator().manual_seed(100 + seed)
    do = torch.randn(o.shape, generator=g, dtype=torch.float64)
    dC = torch.randn(st.predictor.shape, generator=g, dtype=torch.float64)
    dS = torch.randn(st.S.shape, generator=g, dtype=torch.float64)
    grads = torch.autograd.grad((o * do).sum() + (st.predictor * dC).sum() + (st.S * dS).sum(), leaves)
    u, h, q, k, v, gd, er, wr, gm, C0, S0 = args
    seq = (u[0, :, 0], h[0, :, 0], q[0, :, 0], k[0, :, 0, 0], v[0, :, 0, 0], gd[0, :, 0],
           er[0, :, 0, 0], wr[0, :, 0, 0], gm[0, :, 0])
    fw = cm.forward_seq(*seq, C0[0, 0], S0[0, 0])

    def rel(a, b):
        return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()

    assert rel(fw["out"], o[0, :, 0]) < 1e-12
    assert rel(fw["C"], st.predictor[0, 0]) < 1e-12
    assert rel(fw["S"], st.S[0, 0]) < 1e-12
    bw = cm.backward_seq(fw, *seq, do[0, :, 0], dC[0, 0], dS[0, 0])
    expected = [grads[0][0, :, 0], grads[1][0, :, 0], grads[2][0, :, 0], grads[3][0, :, 0, 0],
                grads[4][0, :, 0, 0], grads[5][0, :, 0], grads[6][0, :, 0, 0], grads[7][0, :, 0, 0],
                grads[8][0, :, 0], grads[9][0, 0], grads[10][0, 0]]
    for i, (a, b) in enumerate(zip(bw, expected)):
        if b.norm() == 0:
            assert a.norm() < 1e-12, i
        else:
            assert rel(a, b) < 1e-11, i
