"""The kernels read no workspace entry they have not written: forward and
backward through the C-ABI with both workspaces pre-filled with 0xFF bytes (a
NaN in every floating format) give bitwise the results of zero-filled
workspaces, at a length with a padded tail chunk and at full chunks."""
import ctypes

import pytest
import torch

from gpu_common import make_inputs, make_state

pytestmark = pytest.mark.gpu


def _run(B, T, H, r, V, fill, seed, split=False):
    from solvedelta_amd import _lib
    from solvedelta_amd.operator import _inputs
    lib = _lib.load()
    args = make_inputs(B, T, H, r, V, seed=seed)
    C0, S0 = make_state(B, H, r, V, seed=seed + 1)
    ins = _inputs(*args, C0, S0)
    dev = args[0].device
    st = torch.cuda.current_stream(dev).cuda_stream
    g = torch.Generator().manual_seed(seed + 2)
    dout = torch.randn(B, T, H, V, generator=g).to(torch.bfloat16).to(dev)
    dC = torch.randn(B, H, r, r, generator=g).to(dev)
    dS = torch.randn(B, H, r, V, generator=g).to(dev)
    nf, nb = lib.sd_fwd_workspace_bytes(B, T, H, r, V), lib.sd_bwd_workspace_bytes(B, T, H, r, V)
    fws = torch.full((nf,), fill, dtype=torch.uint8, device=dev)
    bws = torch.full((nb,), fill, dtype=torch.uint8, device=dev)
    out = torch.empty(B, T, H, V, dtype=torch.bfloat16, device=dev)
    C_T, S_T = torch.empty_like(C0), torch.empty_like(S0)
    if split:
        # saved and scratch regions as separate buffers; the backward gets an
        # exactly sized saved region, the scratch is released before it runs
        ns, nx = lib.sd_fwd_saved_bytes(B, T, H, r, V), lib.sd_fwd_scratch_bytes(B, T, H, r, V)
        fws = torch.full((ns,), fill, dtype=torch.uint8, device=dev)
        scratch = torch.full((nx,), fill, dtype=torch.uint8, device=dev)
        assert lib.sd_fwd_split(ctypes.byref(ins), out.data_ptr(), C_T.data_ptr(), S_T.data_ptr(),
                                fws.data_ptr(), ns, scratch.data_ptr(), nx, st) == 0
        scratch.fill_(0xFF)   # the backward reads nothing from it
    else:
        assert lib.sd_fwd(ctypes.byref(ins), out.data_ptr(), C_T.data_ptr(), S_T.data_ptr(),
                          fws.data_ptr(), nf, st) == 0
    bf = dict(dtype=torch.bfloat16, device=dev)
    grads = [torch.empty(B, T, H, r, **bf) for _ in range(4)] + \
            [torch.empty(B, T, H, V, **bf) for _ in range(2)] + [torch.empty(B, T, H, r, **bf)]
    du, dh, dq, dk, dv, dwr, der = grads
    dg = torch.empty(B, T, H, r, device=dev)
    dgam = torch.empty(B, T, H, device=dev)
    dC0, dS0 = torch.empty_like(C0), torch.empty_like(S0)
    assert lib.sd_bwd(ctypes.byref(ins), fws.data_ptr(), dout.data_ptr(), dC.data_ptr(),
                      dS.data_ptr(), du.data_ptr(), dh.data_ptr(), dq.data_ptr(), dk.data_ptr(),
                      dv.data_ptr(), der.data_ptr(), dwr.data_ptr(), dg.data_ptr(),
                      dgam.data_ptr(), dC0.data_ptr(), dS0.data_ptr(), bws.data_ptr(), nb, st) == 0
    torch.cuda.synchronize()
    return [out, C_T, S_T, du, dh, dq, dk, dv, der, dwr, dg, dgam, dC0, dS0]


@pytest.mark.parametrize("B,T,H,r,V", [(1, 200, 2, 128, 128), (2, 128, 1, 40, 24), (1, 19, 1, 16, 16),
                                       (1, 70, 2, 256, 200), (1, 33, 1, 136, 40)])  # last two: wide kernels
def test_results_do_not_depend_on_workspace_contents(B, T, H, r, V):
    print(f"case workspace fill B{B} T{T} H{H} r{r} V{V}", flush=True)
    a = _run(B, T, H, r, V, 0xFF, 61)
    z = _run(B, T, H, r, V, 0x00, 61)
    for i, (x, y) in enumerate(zip(a, z)):
        assert torch.isfinite(x.float()).all(), i
        assert torch.equal(x, y), i


@pytest.mark.parametrize("B,T,H,r,V", [(1, 200, 2, 128, 128), (1, 70, 2, 256, 200)])
def test_split_workspace_equals_single_workspace(B, T, H, r, V):
    """sd_fwd_split with separate saved / scratch buffers (the scratch overwritten
    before the backward) gives bitwise the single-workspace results."""
    print(f"case split workspace B{B} T{T} H{H} r{r} V{V}", flush=True)
    a = _run(B, T, H, r, V, 0x00, 63, split=True)
    z = _run(B, T, H, r, V, 0x00, 63)
    for i, (x, y) in enumerate(zip(a, z)):
        assert torch.equal(x, y), i


@pytest.mark.parametrize("B,T,H,r,V", [(1, 130, 2, 64, 64), (1, 70, 2, 32, 40)])
def test_unaligned_output_pointer_bitwise(B, T, H, r, V):
    """The S pass stores its readout as 16-byte pieces only when the output's
    rows allow it; an output base 2 bytes off a 16-byte boundary takes the
    element-wise path and must give bitwise the aligned result."""
    from solvedelta_amd import _lib
    from solvedelta_amd.operator import _inputs
    lib = _lib.load()
    args = make_inputs(B, T, H, r, V, seed=41)
    C0, S0 = make_state(B, H, r, V, seed=42)
    ins = _inputs(*args, C0, S0)
    dev = args[0].device
    st = torch.cuda.current_stream(dev).cuda_stream
    nf = lib.sd_fwd_workspace_bytes(B, T, H, r, V)
    fws = torch.empty(nf, dtype=torch.uint8, device=dev)
    n = B * T * H * V
    outs = []
    for off in (0, 1):
        buf = torch.full((n + 8,), float("nan"), dtype=torch.bfloat16, device=dev)
        out = buf[off:off + n]
        print(f"case B{B} T{T} H{H} r{r} V{V} output offset {off}", flush=True)
        assert lib.sd_fwd(ctypes.byref(ins), out.data_ptr(), None, None, fws.data_ptr(), nf,
                          st) == 0
        torch.cuda.synchronize()
        assert torch.isfinite(out.float()).all()
        outs.append(out.clone())
    assert torch.equal(outs[0], outs[1])
