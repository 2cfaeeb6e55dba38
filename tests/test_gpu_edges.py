"""Edge shapes against the FP64 oracle: widths 1 and odd widths, T one short
of / at / one past a chunk boundary, odd batch and head counts, and a T = 1
call with gradients (which takes the chunked path).  Forward, final states and
all 11 gradients under the reference's gates (test_rebuild_semantics.py:540-597)."""
import pytest
import torch

from gpu_common import make_inputs, make_state, rel
from oracle.sd_oracle import OracleState, solvedelta_oracle_raw

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B,T,H,r,V,seed", [
    (1, 9, 1, 1, 1, 201),      # one-element heads
    (2, 63, 3, 1, 128, 203),   # one short of a chunk
    (1, 64, 5, 128, 1, 205),   # exactly one chunk
    (3, 65, 1, 7, 33, 207),    # one past a chunk, odd widths
    (1, 1, 2, 24, 40, 209),    # T = 1 with gradients
    (1, 40, 1, 129, 7, 211),   # just past the main kernels' key width
])
def test_edge_shapes_match_oracle(B, T, H, r, V, seed):
    print(f"case edge B{B} T{T} H{H} r{r} V{V}", flush=True)
    from solvedelta_amd import solvedelta_native
    args = make_inputs(B, T, H, r, V, seed=seed, requires_grad=True)
    state = make_state(B, H, r, V, seed=seed + 1, requires_grad=True)
    out, st = solvedelta_native(*args, initial_state=state, return_final_state=True)
    leaves = list(args) + list(state)
    ref = [a.detach().double().cpu().requires_grad_() for a in leaves]
    ro, rs = solvedelta_oracle_raw(*ref[:9], initial_state=OracleState(ref[9], ref[10]))
    g = torch.Generator().manual_seed(seed + 2)
    cot = [torch.randn(x.shape, generator=g) for x in (out, st.predictor, st.S)]
    grads = torch.autograd.grad((out, st.predictor, st.S), leaves,
                                [c.to(x.device, x.dtype) for c, x in zip(cot, (out, st.predictor, st.S))])
    rg = torch.autograd.grad((ro, rs.predictor, rs.S), ref, [c.double() for c in cot])
    errs = {"out": rel(out.float(), ro), "C": rel(st.predictor, rs.predictor), "S": rel(st.S, rs.S)}
    for i, (a, b) in enumerate(zip(grads, rg)):
        assert torch.isfinite(a).all(), i
        if r == 1 and i in (0, 2, 3):
            # a one-element vector normalises to +-1 whatever its value, so the
            # gradients of u, q and k are zero (up to rounding) on both sides
            assert a.abs().max().item() < 1e-3 and b.abs().max().item() < 1e-9, i
            continue
        errs[f"g{i}"] = rel(a.float(), b)
    print("  " + " ".join(f"{k}={v:.1e}" for k, v in errs.items()), flush=True)
    torch.testing.assert_close(out.float().cpu(), ro.float(), rtol=2e-2, atol=2e-2)
    for k, v in errs.items():
        assert v < 3e-2, (k, v)
