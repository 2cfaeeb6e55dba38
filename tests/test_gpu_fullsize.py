"""Parity at the benchmark's own shape (B=4, T=2048, H=8, r=V=128): the HIP
forward against the FP64 C token loop (oracle/sd_token_loop.c, checked against
the torch oracle in test_cpu_lib.py), plus size-independent properties of the
recurrence at that size (split continuation, strided views).  Tolerances are
the reference's native gates (test_rebuild_semantics.py:540-597): output
rtol = atol = 2e-2, states rtol 8e-3 / 1e-2."""
import ctypes
import os
import subprocess

import numpy as np
import pytest
import torch

from gpu_common import rel

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
B, T, H, R, V = 4, 2048, 8, 128, 128


def _inputs(seed=11):
    import torch.nn.functional as F
    g = torch.Generator().manual_seed(seed)
    n = lambda *s: torch.randn(*s, generator=g)
    bf = lambda x: x.to(torch.bfloat16).cuda()
    ins = [bf(n(B, T, H, R)), bf(n(B, T, H, R)), bf(F.normalize(n(B, T, H, R), dim=-1)),
           bf(F.normalize(n(B, T, H, 1, R), dim=-1)), bf(n(B, T, H, 1, V)),
           (-F.softplus(n(B, T, H, R))).cuda(), bf(n(B, T, H, 1, R)), bf(n(B, T, H, 1, V)),
           torch.full((B, T, H), 0.9).cuda()]
    st = ((0.02 * n(B, H, R, R)).cuda(), (0.02 * n(B, H, R, V)).cuda())
    return ins, st


def _c_loop():
    so = os.path.join(ROOT, "oracle", "libsd_token_loop.so")
    if not os.path.exists(so):
        subprocess.run(["make", "-C", os.path.join(ROOT, "oracle")], check=True)
    return ctypes.CDLL(so)


def test_full_size_forward_matches_fp64_token_loop():
    from solvedelta_amd import solvedelta_native
    ins, st = _inputs()
    with torch.no_grad():
        out, fin = solvedelta_native(*ins, initial_state=st, return_final_state=True)
    torch.cuda.synchronize()
    lib = _c_loop()
    arr = lambda x: np.ascontiguousarray(x.detach().float().cpu().numpy().reshape(
        x.shape[0], x.shape[1], x.shape[2], -1) if x.dim() == 5 else x.detach().float().cpu().numpy())
    a = [arr(x) for x in ins]
    C = st[0].cpu().numpy().astype(np.float32).copy()
    S = st[1].cpu().numpy().astype(np.float32).copy()
    o = np.zeros((B, T, H, V), np.float32)
    ptr = lambda z: z.ctypes.data_as(ctypes.c_void_p)
    assert lib.sd_cpu_forward_f64(B, T, H, R, V, *(ptr(z) for z in a), ptr(C), ptr(S), ptr(o)) == 0
    eo = rel(out.float(), torch.from_numpy(o))
    eC = rel(fin.predictor, torch.from_numpy(C))
    eS = rel(fin.S, torch.from_numpy(S))
    print(f"[full size] rel out {eo:.2e} C {eC:.2e} S {eS:.2e}", flush=True)
    torch.testing.assert_close(out.float().cpu(), torch.from_numpy(o), rtol=2e-2, atol=2e-2)
    torch.testing.assert_close(fin.predictor.cpu(), torch.from_numpy(C), rtol=8e-3, atol=1e-2)
    torch.testing.assert_close(fin.S.cpu(), torch.from_numpy(S), rtol=8e-3, atol=1e-2)
    assert eo < 5e-3 and eC < 1e-3 and eS < 1e-3   # the north-star state bound


def test_full_size_split_continuation_and_strides():
    """Running the sequence as two calls with the carried state equals one call
    (test_rebuild_semantics.py:850-867 at the benchmark shape), and strided
    views give bitwise the packed result (ops/operator.py:36-40)."""
    from solvedelta_amd import solvedelta_native
    ins, st = _inputs(seed=12)
    with torch.no_grad():
        out, fin = solvedelta_native(*ins, initial_state=st, return_final_state=True)
        cut = 1000  # not a chunk multiple
        first = [x[:, :cut] if x.dim() >= 3 else x for x in ins]
        second = [x[:, cut:] if x.dim() >= 3 else x for x in ins]
        o1, s1 = solvedelta_native(*first, initial_state=st, return_final_state=True)
        o2, s2 = solvedelta_native(*second, initial_state=s1, return_final_state=True)
        e = rel(torch.cat((o1, o2), 1).float(), out.float())
        print(f"[full size split] rel out {e:.2e} C {rel(s2.predictor, fin.predictor):.2e} "
              f"S {rel(s2.S, fin.S):.2e}", flush=True)
        assert e < 1e-2
        assert rel(s2.predictor, fin.predictor) < 1e-3 and rel(s2.S, fin.S) < 1e-3
        # strided: the operands as column slices of one wide buffer
        wide = torch.zeros(B, T, H, 3 * R, dtype=torch.bfloat16, device="cuda")
        wide[..., :R] = ins[0]
        wide[..., R:2 * R] = ins[1]
        wide[..., 2 * R:] = ins[2]
        sv = [wide[..., :R], wide[..., R:2 * R], wide[..., 2 * R:]] + ins[3:]
        os_, fs = solvedelta_native(*sv, initial_state=st, return_final_state=True)
    assert torch.equal(os_, out) and torch.equal(fs.predictor, fin.predictor) and torch.equal(fs.S, fin.S)
