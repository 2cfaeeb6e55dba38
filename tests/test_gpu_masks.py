"""Masks and resets on the dense batch (solvedelta_amd.masks: neutral invalid
tokens, reset = log-decay kill + fresh predictor read, no repacking and no host
sync) against the FP64 oracle with the same valid / reset masks (reference
tests/core/test_rebuild_semantics.py:932-1039: outputs 2e-2, states rtol 1e-2 /
atol 3e-2, gradients rel-Frobenius < 3e-2), and against the segmented path."""
import pytest
import torch

from gpu_common import make_inputs, make_state, rel
from oracle.sd_oracle import OracleState, solvedelta_oracle_raw

pytestmark = pytest.mark.gpu


def _masks(B, T, seed, p_valid=0.8, p_reset=0.03):
    g = torch.Generator().manual_seed(seed)
    valid = torch.rand(B, T, generator=g) < p_valid
    reset = torch.rand(B, T, generator=g) < p_reset
    return valid, reset


def _run(B, T, H, r, V, valid, reset, seed, gamma_shape="BTH", with_state=True, grad=True):
    from solvedelta_amd import solvedelta_masked_native
    print(f"case masked B{B} T{T} H{H} r{r} V{V} seed {seed}", flush=True)
    args = make_inputs(B, T, H, r, V, seed=seed, requires_grad=grad, gamma_shape=gamma_shape)
    state = make_state(B, H, r, V, seed=seed + 1, requires_grad=grad) if with_state else None
    valid, reset = valid.cuda(), reset.cuda()
    out, st = solvedelta_masked_native(*args, valid, reset, initial_state=state,
                                       return_final_state=True)
    leaves = list(args) + (list(state) if with_state else [])
    ref = [a.detach().double().cpu().requires_grad_(grad) for a in leaves]
    ro, rs = solvedelta_oracle_raw(*ref[:9], initial_state=OracleState(ref[9], ref[10])
                                   if with_state else None,
                                   valid_mask=valid.cpu(), reset_mask=reset.cpu())
    errs = {"out": rel(out.float(), ro), "C": rel(st.predictor, rs.predictor), "S": rel(st.S, rs.S)}
    torch.testing.assert_close(out.float().cpu(), ro.float(), rtol=2e-2, atol=2e-2)
    for a, b in zip(st, rs):
        torch.testing.assert_close(a.cpu(), b.float(), rtol=1e-2, atol=3e-2)
    assert torch.equal(out[~valid], torch.zeros_like(out[~valid]))   # invalid tokens emit 0
    if grad:
        g = torch.Generator().manual_seed(seed + 2)
        cot = [torch.randn(x.shape, generator=g) for x in (out, st.predictor, st.S)]
        grads = torch.autograd.grad((out, st.predictor, st.S), leaves,
                                    [c.to(x.device, x.dtype) for c, x in
                                     zip(cot, (out, st.predictor, st.S))])
        rg = torch.autograd.grad((ro, rs.predictor, rs.S), ref, [c.double() for c in cot])
        for i, (a, b) in enumerate(zip(grads, rg)):
            assert torch.isfinite(a).all(), i
            errs[f"g{i}"] = rel(a.float(), b)
        # invalid tokens' per-token inputs get exactly zero gradient, as when the
        # reference leaves them out (u, h and the values included: they are not
        # masked, every path from them through the token carries a zero factor)
        inv = (~valid).cuda()
        for i in range(9):
            if grads[i].dim() >= 3 and grads[i].shape[:2] == (B, T):
                assert grads[i][inv].abs().max().item() == 0.0 if inv.any() else True, i
    print("  " + " ".join(f"{k}={v:.1e}" for k, v in errs.items()), flush=True)
    for k, v in errs.items():
        assert v < 3e-2, (k, v)


def test_masked_short_rows():
    """An invalid token inside the first row, a reset at 8, a row with no valid
    token (its final state is the initial state)."""
    valid = torch.tensor([[1, 1, 0, 1, 1, 1, 1, 0, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1],
                          [0] * 19], dtype=torch.bool)
    reset = torch.zeros_like(valid)
    reset[0, 8] = True
    reset[1, 3] = True   # a reset on an invalid token is ignored
    _run(2, 19, 1, 16, 16, valid, reset, seed=149)


@pytest.mark.parametrize("B,T,H,r,V,seed", [
    (3, 150, 2, 32, 32, 151),
    (2, 200, 2, 128, 128, 153),   # resets inside and at the edges of 64-token chunks
    (1, 90, 2, 160, 96, 155),     # wide kernels
])
def test_masked_long_rows_several_resets(B, T, H, r, V, seed):
    valid, reset = _masks(B, T, seed)
    reset[0, 0] = True                      # a reset on the first token drops the initial state
    if T > 130:
        reset[-1, 64] = True                # on a chunk boundary
        reset[-1, 127] = True               # on a chunk's last token
        reset[-1, 128] = reset[-1, 129] = True   # consecutive resets
        valid[-1, 64] = valid[-1, 127:130] = True
    _run(B, T, H, r, V, valid, reset, seed, gamma_shape="H" if seed % 2 else "BTH")


def test_masked_without_initial_state_and_all_valid_equals_dense():
    """No masks set: the masked entry equals the dense operator bitwise."""
    from solvedelta_amd import solvedelta_masked_native, solvedelta_native
    args = make_inputs(2, 70, 2, 32, 24, seed=157)
    valid = torch.ones(2, 70, dtype=torch.bool, device="cuda")
    reset = torch.zeros_like(valid)
    with torch.no_grad():
        o1, s1 = solvedelta_masked_native(*args, valid, reset, return_final_state=True)
        o2, s2 = solvedelta_native(*args, return_final_state=True)
    assert torch.equal(o1, o2) and torch.equal(s1.S, s2.S) and torch.equal(s1.predictor, s2.predictor)
    _run(1, 40, 1, 16, 16, *_masks(1, 40, 158), seed=158, with_state=False)


def test_masked_decode_step():
    """T = 1 through the decode kernel: a reset row restarts from zero, an
    invalid row emits 0 and keeps its state."""
    valid = torch.tensor([[True], [False], [True], [True]])
    reset = torch.tensor([[True], [False], [False], [True]])
    with torch.no_grad():
        _run(4, 1, 2, 64, 64, valid, reset, seed=159, grad=False)


def test_masked_matches_segmented_path():
    from solvedelta_amd import (build_packed_segments, solvedelta_masked_native,
                                solvedelta_segmented_native)
    valid, reset = _masks(2, 130, 161, p_reset=0.05)
    valid, reset = valid.cuda(), reset.cuda()
    args = make_inputs(2, 130, 2, 64, 64, seed=161)
    state = make_state(2, 2, 64, 64, seed=162)
    with torch.no_grad():
        o1, s1 = solvedelta_masked_native(*args, valid, reset, initial_state=state,
                                          return_final_state=True)
        o2, s2 = solvedelta_segmented_native(*args, build_packed_segments(valid, reset),
                                             initial_state=state, return_final_state=True)
    # the segmented entry rebuilds the masks from the plan and runs the same path
    assert torch.equal(o1, o2) and torch.equal(s1.predictor, s2.predictor)
    assert torch.equal(s1.S, s2.S)


def test_reset_after_a_large_state():
    """A reset keeps exp(-20) ~ 2.1e-9 of the state before it (RESET_LOG_DECAY),
    where the reference zeroes it (reference.py:156-164).  A pre-reset memory S
    of magnitude ~300 per entry (Frobenius ~4e4 at r = V = 128; fp16 chunk slots
    hold up to 65504 per entry) against writes after the reset ~1e-3 (h and the
    values scaled down): the outputs and final states after the reset against
    the FP64 oracle with an exact reset.  Row 0 resets on its first token; row 1
    carries the large state for 40 tokens of weak decay and resets at token 40.
    (The predictor C stays at a moderate scale: C enters the memory's write
    address d = k + C^T k, and a large C makes the memory's transition
    I - d e^T expansive in the reference's own recurrence.)"""
    from solvedelta_amd import solvedelta_masked_native
    B, T, H, r, V = 2, 100, 2, 128, 128
    print(f"case large-state reset B{B} T{T} H{H} r{r} V{V}", flush=True)
    args = make_inputs(B, T, H, r, V, seed=171, decay="small")
    args[1] = (args[1].float() * 1e-3).to(torch.bfloat16)        # h: predictor writes
    args[4] = (args[4].float() * 1e-3).to(torch.bfloat16)        # values: memory writes
    g = torch.Generator().manual_seed(172)
    C0 = (0.05 * torch.randn(B, H, r, r, generator=g)).cuda()
    S0 = (300.0 * torch.randn(B, H, r, V, generator=g)).cuda()
    valid = torch.ones(B, T, dtype=torch.bool)
    reset = torch.zeros(B, T, dtype=torch.bool)
    reset[0, 0] = True
    reset[1, 40] = True
    with torch.no_grad():
        out, st = solvedelta_masked_native(*args, valid.cuda(), reset.cuda(),
                                           initial_state=(C0, S0), return_final_state=True)
    ref = [a.double().cpu() for a in args]
    ro, rs = solvedelta_oracle_raw(*ref, initial_state=OracleState(C0.double().cpu(),
                                                                   S0.double().cpu()),
                                   valid_mask=valid, reset_mask=reset)
    after = [(0, slice(0, T)), (1, slice(40, T))]
    e_out = max(rel(out[b, t].float(), ro[b, t]) for b, t in after)
    e_pre = rel(out[1, :40].float(), ro[1, :40])
    e_C, e_S = rel(st.predictor, rs.predictor), rel(st.S, rs.S)
    print(f"  after reset: out {e_out:.2e}  C {e_C:.2e}  S {e_S:.2e}; before: out {e_pre:.2e}; "
          f"|S0| {S0.norm().item():.1e} |S_T| {rs.S.norm().item():.1e}", flush=True)
    assert torch.isfinite(out.float()).all()
    assert e_out < 2e-2 and e_pre < 2e-2 and e_C < 1e-2 and e_S < 1e-2


def test_mask_flags_null_and_strided_masks():
    """sd_mask_flags: None masks mean all-valid / no reset (equal to the dense
    operator bitwise), and column-strided bool masks (every other column of a
    wider mask) give the same result as their contiguous copies."""
    from solvedelta_amd import solvedelta_masked_native, solvedelta_native
    args = make_inputs(2, 70, 2, 32, 24, seed=161)
    with torch.no_grad():
        o1, s1 = solvedelta_masked_native(*args, None, None, return_final_state=True)
        o2, s2 = solvedelta_native(*args, return_final_state=True)
    assert torch.equal(o1, o2) and torch.equal(s1.S, s2.S)
    valid, reset = _masks(2, 140, 162)
    valid, reset = valid.cuda()[:, ::2], reset.cuda()[:, ::2]
    assert not valid.is_contiguous()
    with torch.no_grad():
        o3, s3 = solvedelta_masked_native(*args, valid, reset, return_final_state=True)
        o4, s4 = solvedelta_masked_native(*args, valid.contiguous(), reset.contiguous(),
                                          return_final_state=True)
    assert torch.equal(o3, o4) and torch.equal(s3.S, s4.S) and torch.equal(s3.predictor, s4.predictor)
    assert torch.equal(o3[~valid], torch.zeros_like(o3[~valid]))


@pytest.mark.parametrize("B,T,H,r,V,seed", [(2, 150, 3, 64, 48, 171), (2, 130, 2, 128, 128, 172),
                                            (1, 96, 2, 160, 144, 173), (3, 1, 2, 32, 40, 174)])
def test_token_flags_equal_masked_operands(B, T, H, r, V, seed):
    """The kernels read q, keys, gamma and the log-decay through the token flags:
    outputs, final states and every gradient are bitwise those of the same
    operands masked beforehand in torch (invalid rows zeroed, reset rows'
    log-decay at RESET_LOG_DECAY) with only the fresh bit set -- chunked, wide
    (r = 160) and decode (T = 1) kernels."""
    from solvedelta_amd import solvedelta_masked_native, solvedelta_native
    from solvedelta_amd.masks import RESET_LOG_DECAY
    from solvedelta_amd.state import SolveDeltaState
    print(f"case token flags B{B} T{T} H{H} r{r} V{V} seed {seed}", flush=True)
    grad = T > 1
    args = make_inputs(B, T, H, r, V, seed=seed, requires_grad=grad,
                       gamma_shape="H" if seed % 2 else "BTH")
    C0, S0 = make_state(B, H, r, V, seed=seed + 1, requires_grad=grad)
    g = torch.Generator().manual_seed(seed + 2)
    valid = torch.rand(B, T, generator=g) < 0.75
    reset = valid & (torch.rand(B, T, generator=g) < 0.1)
    valid, reset = valid.cuda(), reset.cuda()

    def masked():
        return solvedelta_masked_native(*args, valid, reset,
                                        initial_state=SolveDeltaState(C0, S0),
                                        return_final_state=True)

    def manual():
        u, h, q, k, v, gd, er, wr, gm = args
        keep = valid[:, :, None]
        qm = q * keep[..., None].to(q.dtype)
        km = k * keep[..., None, None].to(k.dtype)
        gdm = torch.where(reset[:, :, None, None], torch.full_like(gd, RESET_LOG_DECAY),
                          gd * keep[..., None].to(gd.dtype))
        gme = gm if gm.dim() == 3 else gm.reshape(1, 1, H).expand(B, T, H)
        gmm = gme * keep.to(gme.dtype)
        fresh = reset.to(torch.uint8)  # bit 0 only: the erase read dropped
        from solvedelta_amd.operator import _dispatch
        return _dispatch(u, h, qm, km, v, gdm, er, wr, gmm, SolveDeltaState(C0, S0), True,
                         fresh)

    def run(fn):
        if not grad:
            with torch.no_grad():
                o, st = fn()
            return [o, st.predictor, st.S]
        o, st = fn()
        cg = torch.Generator().manual_seed(seed + 3)
        cots = [torch.randn(x.shape, generator=cg).to(x.device, x.dtype)
                for x in (o, st.predictor, st.S)]
        leaves = list(args) + [C0, S0]
        return [o, st.predictor, st.S] + list(torch.autograd.grad((o, st.predictor, st.S), leaves, cots))

    a, b = run(masked), run(manual)
    names = ["out", "C_T", "S_T", "du", "dh", "dq", "dk", "dv", "dlog_decay", "derase", "dwrite",
             "dgamma", "dC0", "dS0"]
    bad = [n for n, x, y in zip(names, a, b) if not torch.equal(x, y)]
    assert not bad, bad
