"""Masks / resets through the segmented native path vs the FP64 oracle with the
same valid/reset masks (reference test_rebuild_semantics.py:932-1039: outputs
2e-2, states rtol 1e-2 / atol 3e-2, gradients rel-Frobenius < 3e-2)."""
import pytest
import torch

from gpu_common import make_inputs, make_state, rel
from oracle.sd_oracle import OracleState, solvedelta_oracle_raw

pytestmark = pytest.mark.gpu


def _run(B, T, H, r, V, valid, reset, seed, gamma_shape="BTH"):
    from solvedelta_amd import build_packed_segments, solvedelta_segmented_native
    args = make_inputs(B, T, H, r, V, seed=seed, requires_grad=True, gamma_shape=gamma_shape)
    state = make_state(B, H, r, V, seed=seed + 1, requires_grad=True)
    valid, reset = valid.cuda(), reset.cuda()
    plan = build_packed_segments(valid, reset)
    out, st = solvedelta_segmented_native(*args, plan, initial_state=state, return_final_state=True)
    ref = [a.detach().double().cpu().requires_grad_() for a in list(args) + list(state)]
    ro, rs = solvedelta_oracle_raw(*ref[:9], initial_state=OracleState(ref[9], ref[10]),
                                   valid_mask=valid.cpu(), reset_mask=reset.cpu())
    print(f"[seg B{B} T{T}] rel out {rel(out.float(), ro):.2e} C {rel(st.predictor, rs.predictor):.2e} "
          f"S {rel(st.S, rs.S):.2e}", flush=True)
    torch.testing.assert_close(out.float().cpu(), ro.float(), rtol=2e-2, atol=2e-2)
    for a, b in zip(st, rs):
        torch.testing.assert_close(a.cpu(), b.float(), rtol=1e-2, atol=3e-2)
    assert torch.equal(out[~valid], torch.zeros_like(out[~valid]))
    g = torch.Generator().manual_seed(seed + 2)
    cot = [torch.randn(x.shape, generator=g) for x in (out, st.predictor, st.S)]
    grads = torch.autograd.grad((out, st.predictor, st.S), list(args) + list(state),
                                [c.to(x.device, x.dtype) for c, x in zip(cot, (out, st.predictor, st.S))])
    rg = torch.autograd.grad((ro, rs.predictor, rs.S), ref, [c.double() for c in cot])
    for i, (a, b) in enumerate(zip(grads, rg)):
        assert torch.isfinite(a).all()
        e = rel(a.float(), b)
        assert e < 3e-2, (i, e)


def test_segmented_masks_resets_and_vjp():
    valid = torch.tensor([[1, 1, 0, 1, 1, 1, 1, 0, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1],
                          [0] * 19], dtype=torch.bool)
    reset = torch.zeros_like(valid)
    reset[0, 8] = True
    _run(2, 19, 1, 16, 16, valid, reset, seed=149)


def test_segmented_long_rows_several_resets():
    g = torch.Generator().manual_seed(5)
    valid = torch.rand(3, 150, generator=g) > 0.2
    reset = torch.rand(3, 150, generator=g) > 0.97
    reset[1, 0] = True
    _run(3, 150, 2, 32, 32, valid, reset, seed=151, gamma_shape="H")
