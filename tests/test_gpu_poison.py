"""Uninitialised-memory check of the HIP path: every buffer the operator takes
from torch.empty (outputs, gradients, the forward's saved and scratch regions,
the backward workspace) is filled with NaN bytes first.  A kernel that reads a
location nothing wrote -- even one it masks by multiplying with 0 -- then turns
the result NaN or changes it, so forward, final states and all gradients must
agree bitwise with the same call on unpoisoned buffers.  Shapes with padded
last chunks, widths that are not multiples of 16, the wide-width kernels and
the masked path are covered."""
import types

import pytest
import torch

from gpu_common import make_inputs, make_state

pytestmark = pytest.mark.gpu


class _PoisonTorch(types.ModuleType):
    """torch with empty() returning NaN-filled (0xFF-byte) tensors."""

    def __init__(self):
        super().__init__("torch")

    def __getattr__(self, name):
        return getattr(torch, name)

    @staticmethod
    def empty(*shape, **kw):
        t = torch.empty(*shape, **kw)
        if t.dtype == torch.uint8:
            t.fill_(255)
        else:
            t.view(torch.uint8).fill_(255)
        return t


def _run(poison, B, T, H, r, V, seed, masked=False, with_state=True):
    from solvedelta_amd import operator as op
    from solvedelta_amd import solvedelta_native, solvedelta_masked_native
    saved = op.torch
    if poison:
        op.torch = _PoisonTorch()
    try:
        args = make_inputs(B, T, H, r, V, seed=seed, requires_grad=True)
        state = make_state(B, H, r, V, seed=seed + 1, requires_grad=True) if with_state else None
        if masked:
            g = torch.Generator(device="cpu").manual_seed(seed + 5)
            valid = (torch.rand(B, T, generator=g) > 0.1).cuda()
            reset = (torch.rand(B, T, generator=g) < 0.05).cuda()
            out, st = solvedelta_masked_native(*args, valid, reset, initial_state=state,
                                               return_final_state=True)
        else:
            out, st = solvedelta_native(*args, initial_state=state, return_final_state=True)
        g = torch.Generator().manual_seed(seed + 2)
        cot = [torch.randn(out.shape, generator=g).to(out.device, out.dtype),
               torch.randn(st.predictor.shape, generator=g).cuda(),
               torch.randn(st.S.shape, generator=g).cuda()]
        leaves = list(args) + (list(state) if with_state else [])
        grads = torch.autograd.grad((out, st.predictor, st.S), leaves, cot)
        torch.cuda.synchronize()
        return [out, st.predictor, st.S, *grads]
    finally:
        op.torch = saved


@pytest.mark.parametrize("B,T,H,r,V,seed,masked,with_state", [
    (1, 100, 2, 128, 128, 23, False, True),   # padded last chunk, packed rows
    (1, 100, 2, 128, 128, 23, False, False),  # the same without an initial state
    (2, 40, 2, 16, 24, 19, False, True),      # one short chunk, narrow widths
    (2, 40, 2, 16, 24, 19, False, False),
    (1, 70, 2, 20, 12, 8, False, True),       # widths not a multiple of 8
    (1, 130, 2, 128, 128, 3, True, True),     # masked operator: invalid tokens and resets
    (1, 70, 1, 256, 200, 5, False, True),     # wide-width kernels
    (1, 70, 1, 256, 200, 5, False, False),
])
def test_no_read_of_unwritten_memory(B, T, H, r, V, seed, masked, with_state):
    print(f"case poison B{B} T{T} H{H} r{r} V{V} masked={masked} state={with_state}", flush=True)
    clean = _run(False, B, T, H, r, V, seed, masked, with_state)
    dirty = _run(True, B, T, H, r, V, seed, masked, with_state)
    names = ["out", "C_T", "S_T", "du", "dh", "dq", "dk", "dv", "dlog_decay", "derase",
             "dwrite", "dgamma", "dC0", "dS0"]
    bad = [(n, (a.float() - b.float()).abs().max().item()) for n, a, b in zip(names, clean, dirty)
           if not torch.equal(a, b)]
    assert not bad, bad


@pytest.mark.parametrize("T,r,seed", [(40, 16, 19), (100, 128, 23)])
def test_strided_views_with_nan_padding(T, r, seed):
    """Input rows with a stride of r + 7 whose seven padding columns hold NaN:
    no kernel may read past a row's r columns, so every output and gradient
    matches the packed inputs' bitwise."""
    from solvedelta_amd import solvedelta_native
    print(f"case nan-padded strided views T{T} r{r}", flush=True)
    args = make_inputs(1, T, 2, r, r, seed=seed, requires_grad=True)
    strided = list(a.detach().clone().requires_grad_() for a in args)
    for i in (0, 1, 2, 3, 4, 6, 7):
        x = args[i]
        store = torch.full((*x.shape[:-1], x.shape[-1] + 7), float("nan"), dtype=x.dtype,
                           device=x.device)
        view = store[..., : x.shape[-1]]
        view.copy_(x.detach())
        strided[i] = view.detach().requires_grad_()
    o1, s1 = solvedelta_native(*args, return_final_state=True)
    o2, s2 = solvedelta_native(*strided, return_final_state=True)
    cot = [torch.randn_like(o1), torch.randn_like(s1.predictor), torch.randn_like(s1.S)]
    g1 = torch.autograd.grad((o1, s1.predictor, s1.S), args, cot)
    g2 = torch.autograd.grad((o2, s2.predictor, s2.S), strided, cot)
    names = ["out", "C_T", "S_T", "du", "dh", "dq", "dk", "dv", "dlog_decay", "derase",
             "dwrite", "dgamma"]
    pairs = [(o1, o2), (s1.predictor, s2.predictor), (s1.S, s2.S), *zip(g1, g2)]
    bad = [n for n, (a, b) in zip(names, pairs) if not torch.equal(a, b)]
    assert not bad, bad
