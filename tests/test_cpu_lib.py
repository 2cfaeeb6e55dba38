"""CPU-side checks of the native boundary: the C-ABI library loads and exports
every symbol include/*.h declares, the host-side validation raises the
reference's exception types, and the C token loop agrees with the FP64 oracle."""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared(headers):
    inc = os.path.join(ROOT, "include")
    text = "".join(open(os.path.join(inc, f)).read() for f in headers)
    return sorted(set(re.findall(r"\b(sd_[a-z_]+)\s*\(", text)))


def test_every_header_is_checked():
    inc = os.path.join(ROOT, "include")
    assert sorted(f for f in os.listdir(inc) if f.endswith(".h")) == [
        "solvedelta.h", "solvedelta_mixer.h", "solvedelta_noalloc.h"]


def test_library_exports_every_declared_symbol():
    from solvedelta_amd import _lib
    lib = _lib.load()
    names = _declared(["solvedelta.h", "solvedelta_mixer.h"])
    assert "sd_fwd" in names and "sd_bwd" in names and "sd_decode" in names
    for name in names:
        assert hasattr(lib, name), name
        assert name in _lib.EXPORTS, name
    assert lib.sd_version().startswith(b"solvedelta_amd")
    assert not hasattr(lib, "sd_fwd_noalloc")     # the static array stays out of this library


def test_noalloc_library_exports_its_declared_symbols():
    from solvedelta_amd import _lib
    lib = _lib.load_noalloc()
    names = _declared(["solvedelta_noalloc.h"])
    assert names == ["sd_fwd_noalloc", "sd_noalloc_scratch_bytes"]
    for name in names:
        assert hasattr(lib, name), name
        assert name in _lib.NOALLOC_EXPORTS, name
    assert lib.sd_noalloc_scratch_bytes() == 96 << 20


def test_workspace_queries_and_argument_rejection():
    from solvedelta_amd import _lib
    lib = _lib.load()
    small = lib.sd_fwd_workspace_bytes(1, 64, 1, 16, 16)
    big = lib.sd_fwd_workspace_bytes(4, 2048, 8, 128, 128)
    assert 0 < small < big
    assert lib.sd_bwd_workspace_bytes(4, 2048, 8, 128, 128) > 0
    # key widths 129..256 take the wide-width kernels' own (larger) layout
    wide = lib.sd_fwd_workspace_bytes(1, 64, 1, 200, 16)
    assert wide > small and lib.sd_bwd_workspace_bytes(1, 64, 1, 200, 256) > 0
    ins = _lib.SdInputs()
    ins.B, ins.T, ins.H, ins.r, ins.V = 1, 4, 1, 264, 16  # r > 256
    assert lib.sd_fwd(ctypes.byref(ins), None, None, None, None, 0, None) == _lib.SD_ERR_SHAPE
    ins.r, ins.V = 16, 300  # one call takes at most 256 value columns
    assert lib.sd_fwd(ctypes.byref(ins), None, None, None, None, 0, None) == _lib.SD_ERR_SHAPE
    ins.r, ins.V, ins.T = 200, 16, 1  # decode kernel: r, V <= 128
    assert lib.sd_decode(ctypes.byref(ins), None, None, None, None) == _lib.SD_ERR_SHAPE
    ins.T, ins.V = 4, 16
    ins.r = 16  # null operand pointers
    assert lib.sd_fwd(ctypes.byref(ins), None, None, None, None, 0, None) == _lib.SD_ERR_ARG


def test_operator_rejects_like_the_reference():
    from solvedelta_amd import solvedelta_native
    x = torch.zeros(1, 4, 1, 8, dtype=torch.bfloat16)
    k = torch.zeros(1, 4, 1, 1, 8, dtype=torch.bfloat16)
    g = torch.zeros(1, 4, 1, 8)
    gm = torch.zeros(1)
    with pytest.raises(TypeError):  # CPU tensors: ops/operator.py:28-29
        solvedelta_native(x, x, x, k, k, g, k, k, gm)


def test_c_token_loop_matches_oracle():
    from oracle.sd_oracle import OracleState, solvedelta_oracle_raw
    so = os.path.join(ROOT, "oracle", "libsd_token_loop.so")
    if not os.path.exists(so):
        import subprocess
        subprocess.run(["make", "-C", os.path.join(ROOT, "oracle")], check=True)
    lib = ctypes.CDLL(so)
    B, T, H, r, V = 2, 9, 2, 8, 6
    g = torch.Generator().manual_seed(3)
    n = lambda *s: torch.randn(*s, generator=g)
    u, h, q, k = n(B, T, H, r), n(B, T, H, r), n(B, T, H, r), n(B, T, H, r)
    v, er, wr = n(B, T, H, V), n(B, T, H, r), n(B, T, H, V)
    gd = -torch.nn.functional.softplus(n(B, T, H, r))
    gm = torch.full((B, T, H), 0.8)
    C0, S0 = 0.1 * n(B, H, r, r), 0.1 * n(B, H, r, V)
    o_ref, st = solvedelta_oracle_raw(*(x.double() for x in (u, h, q, k[:, :, :, None], v[:, :, :, None], gd,
                                      er[:, :, :, None], wr[:, :, :, None], gm)),
                                      initial_state=OracleState(C0.double(), S0.double()))
    arrs = [np.ascontiguousarray(x.numpy(), dtype=np.float32) for x in (u, h, q, k, v, gd, er, wr, gm)]
    C, S = C0.numpy().astype(np.float32).copy(), S0.numpy().astype(np.float32).copy()
    out = np.zeros((B, T, H, V), np.float32)
    ptr = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    assert lib.sd_cpu_forward_f64(B, T, H, r, V, *(ptr(a) for a in arrs), ptr(C), ptr(S), ptr(out)) == 0
    np.testing.assert_allclose(out, o_ref.numpy(), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(C, st.predictor.numpy(), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(S, st.S.numpy(), rtol=1e-5, atol=1e-5)


def test_packed_segment_plan_on_cpu():
    """Plan semantics of packing.py:43-150: compaction, reset splits, first
    segment inherits the initial state unless it starts with a reset."""
    from solvedelta_amd.segments import build_packed_segments
    valid = torch.tensor([[1, 1, 0, 1, 1, 1], [0, 0, 0, 0, 0, 0], [1, 1, 1, 1, 0, 1]], dtype=torch.bool)
    reset = torch.zeros_like(valid)
    reset[0, 4] = True
    reset[2, 0] = True
    reset[1, 2] = True  # on an invalid token: ignored
    plan = build_packed_segments(valid, reset)
    assert plan.num_tokens == 10 and plan.num_segments == 3
    assert plan.segment_batch.tolist() == [0, 0, 2]
    assert plan.segment_lengths.tolist() == [3, 2, 5]
    assert plan.use_initial.tolist() == [True, False, False]
    assert plan.last_segment.tolist() == [1, -1, 2]
    assert plan.max_seqlen == 5
    with pytest.raises(ValueError):
        build_packed_segments(valid.int(), reset)
    assert plan.cu_seqlens_cpu.tolist() == [0, 3, 5, 10]
    assert plan.segment_batch_cpu.tolist() == [0, 0, 2] and plan.use_initial_cpu.tolist() == [
        True, False, False]
    assert plan.indices.tolist() == [0, 1, 3, 4, 5, 12, 13, 14, 15, 17]
    assert plan.segment_ids.tolist() == [0, 0, 0, 1, 1, 2, 2, 2, 2, 2]


def test_packed_segment_plan_against_a_token_walk():
    """Random masks: the plan equals a plain walk over each row's tokens, and
    the masks the segmented operator rebuilds from it are the valid tokens and
    the valid resets."""
    from solvedelta_amd.segments import build_packed_segments, plan_masks
    g = torch.Generator().manual_seed(3)
    for B, T in ((1, 1), (3, 17), (4, 64)):
        valid = torch.rand(B, T, generator=g) > 0.3
        reset = torch.rand(B, T, generator=g) > 0.8
        plan = build_packed_segments(valid, reset)
        seg_rows, seg_len, seg_init, idx, ids, last = [], [], [], [], [], [-1] * B
        for b in range(B):
            first = True
            for t in range(T):
                if not valid[b, t]:
                    continue
                if first or reset[b, t]:
                    seg_rows.append(b)
                    seg_len.append(0)
                    seg_init.append(first and not bool(reset[b, t]))
                    last[b] = len(seg_rows) - 1
                first = False
                seg_len[-1] += 1
                idx.append(b * T + t)
                ids.append(len(seg_rows) - 1)
        assert plan.segment_batch.tolist() == seg_rows
        assert plan.segment_lengths.tolist() == seg_len
        assert plan.use_initial.tolist() == seg_init
        assert plan.indices.tolist() == idx and plan.segment_ids.tolist() == ids
        assert plan.last_segment.tolist() == last
        v2, r2 = plan_masks(plan, "cpu")
        assert torch.equal(v2, valid) and torch.equal(r2, valid & reset)


def test_mask_rows_argument_rejection():
    """sd_mask_rows checks its arguments before any launch: in-place masking
    (dst == src) needs a contiguous source, and at most eight tensors."""
    from solvedelta_amd import _lib
    lib = _lib.load()
    flags = ctypes.c_void_p(0x1000)  # never dereferenced: every call below fails its checks
    B, T, H, w = 2, 5, 3, 8
    fake = 0x2000

    def call(sb, st, sh, dst, n=1):
        arr = (_lib.SdMaskTensor * 9)(*[_lib.SdMaskTensor(fake, sb, st, sh, dst, w, 0, 0, 0.0)
                                        for _ in range(9)])
        return lib.sd_mask_rows(B, T, H, flags, T, 1, arr, n, None)

    # in place over a strided (non-contiguous) source
    assert call(2 * T * H * w, 2 * H * w, w, fake) == _lib.SD_ERR_ARG
    assert call(T * H * w, H * w, 2 * w, fake) == _lib.SD_ERR_ARG
    # null destination, too many tensors, empty shape
    assert call(T * H * w, H * w, w, 0) == _lib.SD_ERR_ARG
    assert call(T * H * w, H * w, w, 0x3000, n=9) == _lib.SD_ERR_SHAPE
    assert lib.sd_mask_rows(0, T, H, flags, T, 1, None, 1, None) == _lib.SD_ERR_SHAPE


def test_token_flag_constants_match_the_python_side():
    """The header's token flags and reset log-decay are the values the masked
    operator relies on (its RESET_LOG_DECAY)."""
    from solvedelta_amd.masks import RESET_LOG_DECAY
    text = open(os.path.join(ROOT, "include", "solvedelta.h")).read()
    consts = dict(re.findall(r"#define (SD_TOK_\w+) (\d+)u", text))
    assert consts == {"SD_TOK_FRESH": "1", "SD_TOK_INVALID": "2", "SD_TOK_RESET": "4"}
    m = re.search(r"#define SD_RESET_LOG_DECAY \(([-\d.]+)f\)", text)
    assert m and float(m.group(1)) == RESET_LOG_DECAY
