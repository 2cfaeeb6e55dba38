"""GPU parity of the HIP forward and T=1 decode against the FP64 oracle.

Tolerances are the reference's own native gates
(tests/core/test_rebuild_semantics.py:540-597, 870-929 in the reference):
output rtol = atol = 2e-2; C rtol 8e-3 / atol 1.5e-2; S rtol 1e-2 / atol 3e-2;
plus relative-Frobenius bounds stated per test."""
import pytest
import torch

from gpu_common import make_inputs, make_state, max_rel, oracle_of, rel

pytestmark = pytest.mark.gpu


def _native():
    from solvedelta_amd import solvedelta_native
    return solvedelta_native


def _check(out, st, eo, es, tag, frob=1e-2):
    e_out, e_C, e_S = rel(out.float(), eo), rel(st.predictor, es.predictor), rel(st.S, es.S)
    print(f"[{tag}] rel out {e_out:.2e} C {e_C:.2e} S {e_S:.2e} "
          f"max-rel out {max_rel(out.float(), eo):.2e} C {max_rel(st.predictor, es.predictor):.2e} "
          f"S {max_rel(st.S, es.S):.2e}", flush=True)
    torch.testing.assert_close(out.float().cpu(), eo.float(), rtol=2e-2, atol=2e-2)
    torch.testing.assert_close(st.predictor.cpu(), es.predictor.float(), rtol=8e-3, atol=1.5e-2)
    torch.testing.assert_close(st.S.cpu(), es.S.float(), rtol=1e-2, atol=3e-2)
    assert e_out < frob and e_C < frob and e_S < frob


@pytest.mark.parametrize("B,T,H,r,V,seed,decay,with_state", [
    (1, 16, 2, 16, 16, 23, "small", True),
    (1, 64, 2, 16, 16, 3, "softplus", False),
    (2, 130, 2, 32, 24, 4, "softplus", True),
    (1, 256, 1, 128, 128, 5, "softplus", True),
    (1, 19, 2, 16, 16, 6, "small", True),
    (1, 1, 2, 16, 16, 7, "small", True),
    (1, 70, 2, 20, 12, 8, "softplus", True),   # widths not a multiple of 8: element-wise row loads
    (1, 130, 2, 32, 24, 31, "mixed", True),    # wild and ordinary coordinates in one block
    (1, 128, 1, 128, 128, 32, "mixed", True),
])
def test_forward_matches_oracle(B, T, H, r, V, seed, decay, with_state):
    args = make_inputs(B, T, H, r, V, seed=seed, decay=decay)
    state = make_state(B, H, r, V, seed=seed + 100) if with_state else None
    print(f"case B{B} T{T} H{H} r{r} V{V} decay={decay}", flush=True)
    out, st = _native()(*args, initial_state=state, return_final_state=True)
    torch.cuda.synchronize()
    eo, es = oracle_of(args, state)
    _check(out, st, eo, es, f"fwd T{T} r{r}")


def test_forward_gamma_zero_is_gdn2():
    from oracle.sd_oracle import gdn2_oracle
    args = make_inputs(2, 128, 2, 64, 64, seed=11, gamma=0.0)
    out, st = _native()(*args, return_final_state=True)
    d = [a.detach().double().cpu() for a in args]
    eo, eS = gdn2_oracle(d[2], d[3], d[4], d[5], torch.sigmoid(d[6]), torch.sigmoid(d[7]))
    print(f"[gdn2] rel out {rel(out.float(), eo):.2e} S {rel(st.S, eS):.2e}", flush=True)
    assert rel(out.float(), eo) < 1e-2 and rel(st.S, eS) < 1e-2
    assert st.predictor.abs().max().item() == 0.0


def test_forward_extreme_decay_finite():
    args = make_inputs(1, 80, 1, 16, 16, seed=13, decay="extreme")
    state = make_state(1, 1, 16, 16, seed=14, scale=1.0)
    out, st = _native()(*args, initial_state=state, return_final_state=True)
    assert torch.isfinite(out.float()).all() and torch.isfinite(st.predictor).all()
    eo, es = oracle_of(args, state)
    _check(out, st, eo, es, "extreme")


def test_gamma_broadcast_shapes_agree():
    B, T, H, r, V = 1, 70, 2, 16, 16
    outs = []
    for shape in ("BTH", "H", "1H"):
        args = make_inputs(B, T, H, r, V, seed=17, gamma=0.7, gamma_shape=shape)
        outs.append(_native()(*args, return_final_state=True))
    for o, s in outs[1:]:
        assert torch.equal(o, outs[0][0])
        assert torch.equal(s.predictor, outs[0][1].predictor)


def test_strided_views_bitwise_equal_packed():
    """test_rebuild_semantics.py:487-537: strided inputs give bitwise the same result."""
    args = make_inputs(1, 40, 2, 16, 16, seed=19)
    strided = list(args)
    for i in (0, 1, 2, 3, 4, 6, 7):
        x = args[i]
        store = torch.empty(*x.shape[:-1], x.shape[-1] + 7, dtype=x.dtype, device=x.device)
        view = store[..., : x.shape[-1]]
        view.copy_(x)
        strided[i] = view
        assert not view.is_contiguous()
    o1, s1 = _native()(*args, return_final_state=True)
    o2, s2 = _native()(*strided, return_final_state=True)
    o3, s3 = _native()(*args, return_final_state=False)
    assert s3 is None and torch.equal(o1, o3)
    assert torch.equal(o1, o2)
    assert torch.equal(s1.predictor, s2.predictor) and torch.equal(s1.S, s2.S)


def test_aligned_split_continuation():
    """test_rebuild_semantics.py:850-867 (split at a chunk boundary and inside one)."""
    for split in (64, 40):
        args = make_inputs(1, 128, 2, 32, 32, seed=29)
        ow, sw = _native()(*args, return_final_state=True)
        first = [a[:, :split] if a.ndim >= 3 else a for a in args]
        second = [a[:, split:] if a.ndim >= 3 else a for a in args]
        ol, sl = _native()(*first, return_final_state=True)
        orr, sr = _native()(*second, initial_state=sl, return_final_state=True)
        torch.testing.assert_close(ow.float(), torch.cat((ol, orr), 1).float(), rtol=2e-2, atol=2e-2)
        torch.testing.assert_close(sr.predictor, sw.predictor, rtol=8e-3, atol=2e-2)
        torch.testing.assert_close(sr.S, sw.S, rtol=8e-3, atol=2e-2)


@pytest.mark.parametrize("B,H,r,V", [(1, 2, 16, 16), (4, 8, 128, 128), (3, 2, 40, 24)])
def test_decode_step_matches_oracle(B, H, r, V):
    """test_rebuild_semantics.py:900-929 tolerances: out rtol 8e-3 / atol 2e-3,
    states rtol 5e-3 / atol 3e-3."""
    args = make_inputs(B, 1, H, r, V, seed=31)
    state = make_state(B, H, r, V, seed=37)
    with torch.no_grad():
        out, st = _native()(*args, initial_state=state, return_final_state=True)
    torch.cuda.synchronize()
    eo, es = oracle_of(args, state)
    print(f"[decode r{r}] rel out {rel(out.float(), eo):.2e} C {rel(st.predictor, es.predictor):.2e} "
          f"S {rel(st.S, es.S):.2e}", flush=True)
    torch.testing.assert_close(out.float().cpu(), eo.float(), rtol=8e-3, atol=2e-3)
    torch.testing.assert_close(st.predictor.cpu(), es.predictor.float(), rtol=5e-3, atol=3e-3)
    torch.testing.assert_close(st.S.cpu(), es.S.float(), rtol=5e-3, atol=3e-3)


def test_decode_multi_step_matches_oracle():
    """Config-3 style: states advance over several T=1 calls."""
    B, H, r, V, steps = 2, 2, 64, 64, 12
    args = make_inputs(B, steps, H, r, V, seed=41)
    state = make_state(B, H, r, V, seed=43, scale=0.01)
    st = state
    outs = []
    with torch.no_grad():
        for t in range(steps):
            step = [a[:, t:t + 1] if a.ndim >= 3 else a for a in args]
            o, st = _native()(*step, initial_state=st, return_final_state=True)
            outs.append(o)
    eo, es = oracle_of(args, state)
    out = torch.cat(outs, 1)
    print(f"[decode x{steps}] rel out {rel(out.float(), eo):.2e} S {rel(st.S, es.S):.2e}", flush=True)
    assert rel(out.float(), eo) < 1e-2 and rel(st.S, es.S) < 1e-2 and rel(st.predictor, es.predictor) < 1e-2
