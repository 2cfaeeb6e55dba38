"""Seeded random sweep of shapes and options against the FP64 oracle: batch,
length (from 1 and across chunk boundaries), heads, key / value widths on both
sides of 128 (main and wide-width kernels), decay regimes, gamma layouts, with
and without an initial state, dense or masked (valid / reset masks).  Gates as
the reference's (tests/core/test_rebuild_semantics.py:540-597, 932-1039):
output and state relative errors below 2e-2 / 1e-2, every gradient below 3e-2.
The cases are drawn once from a fixed seed, so the sweep is the same on every
run; each prints its parameters before it runs."""
import random

import pytest
import torch

from gpu_common import make_inputs, make_state, rel
from oracle.sd_oracle import OracleState, solvedelta_oracle_raw

pytestmark = pytest.mark.gpu


def _cases(n=24, seed=20261202):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        wide = i % 3 == 2
        r = rng.randint(129, 256) if wide and i % 2 else rng.randint(3, 128)
        V = rng.randint(129, 256) if wide and not i % 2 else rng.randint(3, 128)
        B, H = rng.randint(1, 3), rng.randint(1, 3)
        u = rng.random()
        T = 1 if u < 0.15 else (rng.randint(2, 63) if u < 0.5 else rng.randint(64, 200))
        while B * T * H > 600:
            T = max(1, T // 2)
        out.append(dict(B=B, T=T, H=H, r=r, V=V, seed=100 + i,
                        decay=rng.choice(["softplus", "small", "mixed"]),
                        gamma_shape=rng.choice(["BTH", "H", "1H"]),
                        with_state=rng.random() < 0.7, masked=rng.random() < 0.3))
    return out


CASES = _cases()


@pytest.mark.parametrize("case", CASES, ids=[f"c{i}" for i in range(len(CASES))])
def test_random_case_matches_oracle(case):
    from solvedelta_amd import solvedelta_masked_native, solvedelta_native
    print(f"case {case}", flush=True)
    B, T, H, r, V, seed = (case[k] for k in ("B", "T", "H", "r", "V", "seed"))
    args = make_inputs(B, T, H, r, V, seed=seed, decay=case["decay"],
                       gamma_shape=case["gamma_shape"], requires_grad=True)
    state = make_state(B, H, r, V, seed=seed + 1, requires_grad=True) if case["with_state"] else None
    kw = {}
    if case["masked"]:
        g = torch.Generator().manual_seed(seed + 3)
        valid = torch.rand(B, T, generator=g) < 0.85
        reset = torch.rand(B, T, generator=g) < 0.05
        out, st = solvedelta_masked_native(*args, valid.cuda(), reset.cuda(), initial_state=state,
                                           return_final_state=True)
        kw = dict(valid_mask=valid, reset_mask=reset)
    else:
        out, st = solvedelta_native(*args, initial_state=state, return_final_state=True)
    leaves = list(args) + (list(state) if state is not None else [])
    ref = [a.detach().double().cpu().requires_grad_() for a in leaves]
    ro, rs = solvedelta_oracle_raw(*ref[:9], initial_state=OracleState(ref[9], ref[10])
                                   if state is not None else None, **kw)
    errs = {"out": rel(out.float(), ro), "C": rel(st.predictor, rs.predictor), "S": rel(st.S, rs.S)}
    g = torch.Generator().manual_seed(seed + 2)
    cot = [torch.randn(x.shape, generator=g) for x in (out, st.predictor, st.S)]
    grads = torch.autograd.grad((out, st.predictor, st.S), leaves,
                                [c.to(x.device, x.dtype) for c, x in zip(cot, (out, st.predictor, st.S))])
    rg = torch.autograd.grad((ro, rs.predictor, rs.S), ref, [c.double() for c in cot])
    for i, (a, b) in enumerate(zip(grads, rg)):
        assert torch.isfinite(a).all(), i
        if b.abs().max() > 0:  # exactly-zero references (e.g. fully masked) compare absolutely below
            errs[f"g{i}"] = rel(a.float(), b)
        else:
            assert a.abs().max().item() == 0.0, i
    print("  " + " ".join(f"{k}={v:.1e}" for k, v in errs.items()), flush=True)
    assert errs["out"] < 2e-2 and errs["C"] < 1e-2 and errs["S"] < 1e-2, errs
    for k, v in errs.items():
        assert v < 3e-2, (k, v)
