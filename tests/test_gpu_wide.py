"""GPU parity of the wide-width kernels (key width 128 < r <= 256, value
width up to 256 per call) against the FP64 oracle.

The reference's state pass takes head widths up to 256
(causallsso/ops/residual_frame/common_left_h.py:139-151); the main kernels
stop at 128, so these widths run on the library's wide-width kernels (32-token
chunks, FP32 token panels, 16-bit state pass).  Gates as for the main path (reference
tests/core/test_rebuild_semantics.py:540-597): output rtol/atol 2e-2, final
states and every gradient's relative Frobenius error well inside 3e-2; the
wide path is held to 1e-2."""
import pytest
import torch

from gpu_common import make_inputs, make_state, oracle_of, rel
from oracle.sd_oracle import OracleState, solvedelta_oracle_raw

pytestmark = pytest.mark.gpu

NAMES = ["du", "dh", "dq", "dk", "dv", "dlog_decay", "derase", "dwrite", "dgamma", "dC0", "dS0"]


def _native():
    from solvedelta_amd import solvedelta_native
    return solvedelta_native


def _check_fb(B, T, H, r, V, seed, decay="softplus", with_state=True, cot="all",
              bound=1e-2):
    print(f"case B{B} T{T} H{H} r{r} V{V} {decay} state={with_state} cot={cot}", flush=True)
    args = make_inputs(B, T, H, r, V, seed=seed, decay=decay, requires_grad=True)
    state = make_state(B, H, r, V, seed=seed + 1, requires_grad=True) if with_state else None
    out, st = _native()(*args, initial_state=state, return_final_state=True)
    ref = [a.detach().double().cpu().requires_grad_() for a in
           list(args) + (list(state) if with_state else [])]
    ro, rs = solvedelta_oracle_raw(*ref[:9], initial_state=OracleState(ref[9], ref[10])
                                   if with_state else None)
    errs = {"out": rel(out.float(), ro), "C": rel(st.predictor, rs.predictor), "S": rel(st.S, rs.S)}
    g = torch.Generator().manual_seed(seed + 2)
    do = torch.randn(out.shape, generator=g)
    dC = torch.randn(st.predictor.shape, generator=g)
    dS = torch.randn(st.S.shape, generator=g)
    if cot == "out":
        outs, cots, rcots = (out,), (do.to(out.device, out.dtype),), (do.double(),)
        routs = (ro,)
    else:
        outs = (out, st.predictor, st.S)
        cots = (do.to(out.device, out.dtype), dC.cuda(), dS.cuda())
        routs = (ro, rs.predictor, rs.S)
        rcots = (do.double(), dC.double(), dS.double())
    leaves = list(args) + (list(state) if with_state else [])
    grads = torch.autograd.grad(outs, leaves, cots)
    rgrads = torch.autograd.grad(routs, ref, rcots)
    for n, a, b in zip(NAMES, grads, rgrads):
        assert torch.isfinite(a).all(), n
        assert a.shape == b.shape, n
        errs[n] = rel(a.float(), b)
    print("  " + " ".join(f"{k}={v:.1e}" for k, v in errs.items()), flush=True)
    for k, v in errs.items():
        assert v < bound, (k, v)


@pytest.mark.parametrize("B,T,H,r,V,seed,decay", [
    (1, 70, 2, 256, 256, 51, "softplus"),   # three 32-token chunks, ragged tail
    (2, 33, 1, 200, 136, 53, "softplus"),   # widths not a multiple of 32
    (1, 100, 2, 160, 64, 55, "mixed"),      # wide keys, narrow values; strongly decaying coordinates
    (1, 64, 1, 144, 144, 57, "small"),
    (2, 70, 4, 160, 144, 59, "softplus"),  # B*H = 8: the XCD-grouped workgroup mapping
])
def test_wide_forward_backward_matches_oracle(B, T, H, r, V, seed, decay):
    _check_fb(B, T, H, r, V, seed, decay)


def test_wide_no_state_output_cotangent_only():
    _check_fb(1, 48, 2, 256, 128, 59, with_state=False, cot="out")


def test_wide_value_groups_above_256():
    """r > 128 with V > 256: value groups of 256 columns on the wide kernels."""
    _check_fb(1, 40, 1, 136, 300, 61)


def test_wide_extreme_decay_and_t1():
    """log-decay = -100 stays finite and exact; T = 1 at r = 256 takes the
    chunked path (the reference's decode dispatch needs r, V <= 128,
    residual_frame/operator.py:198-216)."""
    args = make_inputs(1, 40, 2, 192, 96, seed=63, decay="extreme")
    state = make_state(1, 2, 192, 96, seed=64, scale=1.0)
    one = [a[:, :1] if a.ndim >= 3 else a for a in make_inputs(2, 1, 2, 256, 256, seed=65)]
    st1 = make_state(2, 2, 256, 256, seed=66)
    with torch.no_grad():
        out, st = _native()(*args, initial_state=state, return_final_state=True)
        o1, s1 = _native()(*one, initial_state=st1, return_final_state=True)
    eo, es = oracle_of(args, state)
    eo1, es1 = oracle_of(one, st1)
    errs = [rel(out.float(), eo), rel(st.predictor, es.predictor), rel(st.S, es.S),
            rel(o1.float(), eo1), rel(s1.predictor, es1.predictor), rel(s1.S, es1.S)]
    print("[wide extreme / T1] " + " ".join(f"{e:.1e}" for e in errs), flush=True)
    assert all(torch.isfinite(x).all() for x in (out, st.predictor, st.S, o1))
    assert max(errs) < 1e-2


def test_wide_gamma_zero_is_gdn2():
    """gamma = 0 leaves C at its initial value (zero here) and the memory reduces
    to the GDN2 path (test_rebuild_semantics.py:296-316)."""
    from oracle.sd_oracle import gdn2_oracle
    args = make_inputs(1, 50, 2, 256, 160, seed=67, gamma=0.0)
    with torch.no_grad():
        out, st = _native()(*args, return_final_state=True)
    d = [a.detach().double().cpu() for a in args]
    eo, eS = gdn2_oracle(d[2], d[3], d[4], d[5], torch.sigmoid(d[6]), torch.sigmoid(d[7]))
    errs = [rel(out.float(), eo), rel(st.S, eS)]
    print("[wide gdn2] " + " ".join(f"{e:.1e}" for e in errs), flush=True)
    assert st.predictor.abs().max().item() == 0.0
    assert max(errs) < 1e-2


def test_wide_strided_bitwise_and_split_continuation():
    """Strided views equal packed inputs bitwise (ops/operator.py:36-40); a
    split at a chunk boundary with the carried state equals one call."""
    args = make_inputs(1, 64, 2, 160, 48, seed=69)
    strided = list(args)
    for i in (0, 1, 2, 3, 4, 6, 7):
        x = args[i]
        store = torch.empty(*x.shape[:-1], x.shape[-1] + 5, dtype=x.dtype, device=x.device)
        store[..., : x.shape[-1]].copy_(x)
        strided[i] = store[..., : x.shape[-1]]
    with torch.no_grad():
        o1, s1 = _native()(*args, return_final_state=True)
        o2, s2 = _native()(*strided, return_final_state=True)
        a = [x[:, :32] if x.ndim >= 3 else x for x in args]
        b = [x[:, 32:] if x.ndim >= 3 else x for x in args]
        oa, sa = _native()(*a, return_final_state=True)
        ob, sb = _native()(*b, initial_state=sa, return_final_state=True)
    assert torch.equal(o1, o2) and torch.equal(s1.S, s2.S) and torch.equal(s1.predictor, s2.predictor)
    split = torch.cat([oa, ob], dim=1)
    e = [rel(split.float(), o1.float()), rel(sb.S, s1.S), rel(sb.predictor, s1.predictor)]
    print("[wide split] " + " ".join(f"{x:.1e}" for x in e), flush=True)
    assert max(e) < 1e-5


def test_wide_larger_forward_matches_fp64_token_loop():
    """B=2, T=1024, H=4 at r = V = 256 against the FP64 C token loop
    (oracle/sd_token_loop.c), with the north-star's state bound 1e-3."""
    from gpu_common import c_forward_f64
    args = make_inputs(2, 1024, 4, 256, 256, seed=71)
    state = make_state(2, 4, 256, 256, seed=72)
    with torch.no_grad():
        out, st = _native()(*args, initial_state=state, return_final_state=True)
    torch.cuda.synchronize()
    eo, eC, eS = c_forward_f64(args, state)
    errs = [rel(out.float(), eo), rel(st.predictor, eC), rel(st.S, eS)]
    print("[wide B2 T1024 H4 r256] " + " ".join(f"{e:.1e}" for e in errs), flush=True)
    assert errs[0] < 5e-3 and errs[1] < 1e-3 and errs[2] < 1e-3
