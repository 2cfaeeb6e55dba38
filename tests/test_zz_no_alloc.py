"""sd_fwd_noalloc (include/solvedelta_noalloc.h): the forward with its workspace
in its library's static device array instead of a caller buffer.  Called through the
C-ABI twice in a row (the second call smaller, so it runs on what the first
left in the array) and checked bitwise against sd_fwd on the same inputs; a
shape whose workspace exceeds the array is rejected before any launch."""
import ctypes

import pytest
import torch

from gpu_common import make_inputs, make_state

pytestmark = pytest.mark.gpu


def _call_both(B, T, H, r, V, seed):
    from solvedelta_amd import _lib
    from solvedelta_amd.operator import _inputs
    lib = _lib.load()
    nlib = _lib.load_noalloc()
    args = make_inputs(B, T, H, r, V, seed=seed)
    C0, S0 = make_state(B, H, r, V, seed=seed + 1)
    ins = _inputs(*args, C0, S0)
    dev = args[0].device
    stream = torch.cuda.current_stream(dev).cuda_stream
    outs = []
    for mode in ("ws", "noalloc"):
        out = torch.empty(B, T, H, V, dtype=torch.bfloat16, device=dev)
        C_T = torch.empty(B, H, r, r, dtype=torch.float32, device=dev)
        S_T = torch.empty(B, H, r, V, dtype=torch.float32, device=dev)
        if mode == "ws":
            n = lib.sd_fwd_workspace_bytes(B, T, H, r, V)
            ws = torch.empty(n, dtype=torch.uint8, device=dev)
            rc = lib.sd_fwd(ctypes.byref(ins), out.data_ptr(), C_T.data_ptr(), S_T.data_ptr(),
                            ws.data_ptr(), n, stream)
        else:
            rc = nlib.sd_fwd_noalloc(ctypes.byref(ins), out.data_ptr(), C_T.data_ptr(),
                                    S_T.data_ptr(), stream)
        assert rc == 0, (mode, rc)
        outs.append((out, C_T, S_T))
    torch.cuda.synchronize()
    return outs


def test_noalloc_forward_equals_workspace_forward_twice():
    from solvedelta_amd import _lib
    lib = _lib.load()
    nlib = _lib.load_noalloc()
    assert nlib.sd_noalloc_scratch_bytes() == 96 << 20
    for B, T, H, r, V, seed in ((1, 1024, 8, 128, 128, 3), (2, 200, 3, 64, 48, 5)):
        print(f"case noalloc B{B} T{T} H{H} r{r} V{V}", flush=True)
        assert lib.sd_fwd_workspace_bytes(B, T, H, r, V) <= nlib.sd_noalloc_scratch_bytes()
        (o1, c1, s1), (o2, c2, s2) = _call_both(B, T, H, r, V, seed)
        assert torch.equal(o1, o2) and torch.equal(c1, c2) and torch.equal(s1, s2)


def test_noalloc_rejects_shapes_beyond_the_scratch():
    from solvedelta_amd import _lib
    from solvedelta_amd.operator import _inputs
    lib = _lib.load()
    nlib = _lib.load_noalloc()
    B, T, H, r, V = 1, 4096, 8, 128, 128
    assert lib.sd_fwd_workspace_bytes(B, T, H, r, V) > nlib.sd_noalloc_scratch_bytes()
    args = make_inputs(1, 1, 1, 16, 16, seed=1)      # valid pointers; the shape is what fails
    ins = _inputs(*args, None, None)
    ins.B, ins.T, ins.H, ins.r, ins.V = B, T, H, r, V
    out = torch.empty(1, device="cuda")
    rc = nlib.sd_fwd_noalloc(ctypes.byref(ins), out.data_ptr(), None, None,
                            torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.SD_ERR_WORKSPACE
