"""ctypes binding of libsolvedelta_hip.so (declared in include/solvedelta.h).

The product path needs the built HIP library: loading fails loudly when it is
missing; there is no CPU or PyTorch fallback.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsolvedelta_hip.so")

SD_OK, SD_ERR_SHAPE, SD_ERR_ARG, SD_ERR_WORKSPACE, SD_ERR_LAUNCH = 0, 1, 2, 3, 4


class SdView(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("sb", ctypes.c_int64), ("st", ctypes.c_int64),
                ("sh", ctypes.c_int64)]


class SdInputs(ctypes.Structure):
    _fields_ = [("B", ctypes.c_int), ("T", ctypes.c_int), ("H", ctypes.c_int),
                ("r", ctypes.c_int), ("V", ctypes.c_int),
                ("u", SdView), ("h", SdView), ("q", SdView), ("k", SdView), ("v", SdView),
                ("erase_raw", SdView), ("write_raw", SdView), ("log_decay", SdView),
                ("gamma", SdView), ("C0", ctypes.c_void_p), ("S0", ctypes.c_void_p),
                ("fresh", SdView)]


class SdMaskTensor(ctypes.Structure):
    _fields_ = [("src", ctypes.c_void_p), ("sb", ctypes.c_int64), ("st", ctypes.c_int64),
                ("sh", ctypes.c_int64), ("dst", ctypes.c_void_p), ("width", ctypes.c_int),
                ("is_fp32", ctypes.c_int), ("reset_fill", ctypes.c_int),
                ("reset_value", ctypes.c_float)]


EXPORTS = {
    "sd_version": (ctypes.c_char_p, []),
    "sd_fwd_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int] * 5),
    "sd_fwd_saved_bytes": (ctypes.c_size_t, [ctypes.c_int] * 5),
    "sd_fwd_scratch_bytes": (ctypes.c_size_t, [ctypes.c_int] * 5),
    "sd_fwd_split": (ctypes.c_int, [ctypes.POINTER(SdInputs), ctypes.c_void_p, ctypes.c_void_p,
                                    ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                    ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "sd_fwd": (ctypes.c_int, [ctypes.POINTER(SdInputs), ctypes.c_void_p, ctypes.c_void_p,
                              ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "sd_bwd_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int] * 5),
    "sd_bwd": (ctypes.c_int, [ctypes.POINTER(SdInputs), ctypes.c_void_p, ctypes.c_void_p,
                              ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_void_p] * 11
               + [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "sd_profile_enable": (ctypes.c_int, [ctypes.c_int]),
    "sd_profile_read": (ctypes.c_size_t, [ctypes.c_char_p, ctypes.c_size_t]),
    "sd_mask_rows": (ctypes.c_int, [ctypes.c_int] * 3 + [ctypes.c_void_p, ctypes.c_int64,
                                    ctypes.c_int64, ctypes.POINTER(SdMaskTensor), ctypes.c_int,
                                    ctypes.c_void_p]),
    "sd_mask_flags": (ctypes.c_int, [ctypes.c_int] * 2 + [ctypes.c_void_p, ctypes.c_int64,
                                     ctypes.c_int64] * 2 + [ctypes.c_void_p] * 3),
    "sd_decode": (ctypes.c_int, [ctypes.POINTER(SdInputs), ctypes.c_void_p, ctypes.c_void_p,
                                 ctypes.c_void_p, ctypes.c_void_p]),
    # mixer frontend / readout (include/solvedelta_mixer.h)
    "sd_conv4_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int] * 3),
    "sd_conv4_silu_fwd": (ctypes.c_int, [ctypes.c_int] * 3 + [ctypes.c_void_p, ctypes.c_int64,
                                         ctypes.c_int64] + [ctypes.c_void_p] * 5),
    "sd_conv4_silu_bwd": (ctypes.c_int, [ctypes.c_int] * 3 + [ctypes.c_void_p, ctypes.c_int64,
                                         ctypes.c_int64] + [ctypes.c_void_p] * 8
                          + [ctypes.c_size_t, ctypes.c_void_p]),
    "sd_conv4_masked_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int] * 2),
    "sd_conv4_silu_masked_fwd": (ctypes.c_int, [ctypes.c_int] * 3 + [ctypes.c_void_p, ctypes.c_int64,
                                 ctypes.c_int64] + [ctypes.c_void_p] * 4 + [ctypes.c_int64] * 2
                                 + [ctypes.c_void_p] * 3),
    "sd_conv4_silu_masked_bwd": (ctypes.c_int, [ctypes.c_int] * 3 + [ctypes.c_void_p, ctypes.c_int64,
                                 ctypes.c_int64] + [ctypes.c_void_p] * 4 + [ctypes.c_int64] * 2
                                 + [ctypes.c_void_p] * 6 + [ctypes.c_size_t, ctypes.c_void_p]),
    "sd_kda_gate_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int] * 3),
    "sd_kda_gate_fwd": (ctypes.c_int, [ctypes.c_int] * 3 + [ctypes.c_void_p, ctypes.c_int64]
                        + [ctypes.c_void_p] * 4),
    "sd_kda_gate_bwd": (ctypes.c_int, [ctypes.c_int] * 3 + [ctypes.c_void_p, ctypes.c_int64]
                        + [ctypes.c_void_p] * 7 + [ctypes.c_size_t, ctypes.c_void_p]),
    "sd_rmsnorm_gated_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int] * 2),
    "sd_rmsnorm_gated_fwd": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_float]
                             + [ctypes.c_void_p] * 6),
    "sd_rmsnorm_gated_bwd": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_float]
                             + [ctypes.c_void_p] * 9 + [ctypes.c_size_t, ctypes.c_void_p]),
}

# libsolvedelta_noalloc.so (include/solvedelta_noalloc.h): loaded only by its callers
NOALLOC_LIB_PATH = os.path.join(HERE, "libsolvedelta_noalloc.so")
NOALLOC_EXPORTS = {
    "sd_noalloc_scratch_bytes": (ctypes.c_size_t, []),
    "sd_fwd_noalloc": (ctypes.c_int, [ctypes.POINTER(SdInputs), ctypes.c_void_p, ctypes.c_void_p,
                                      ctypes.c_void_p, ctypes.c_void_p]),
}

_lib = None
_noalloc = None


def load(path: str = None) -> ctypes.CDLL:
    """Loads the HIP library once; raises if it has not been built.
    SD_LIBRARY overrides the path (used for instrumented builds)."""
    global _lib
    if _lib is not None:
        return _lib
    path = path or os.environ.get("SD_LIBRARY", LIB_PATH)
    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is missing: build the HIP extension first "
            "(python -m solvedelta_amd.build)")
    lib = ctypes.CDLL(path)
    for name, (res, args) in EXPORTS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def load_noalloc() -> ctypes.CDLL:
    """Loads libsolvedelta_noalloc.so (after the main library, which it links)."""
    global _noalloc
    if _noalloc is not None:
        return _noalloc
    load()
    if not os.path.exists(NOALLOC_LIB_PATH):
        raise RuntimeError(f"{NOALLOC_LIB_PATH} is missing: build the HIP extension first "
                           "(python -m solvedelta_amd.build)")
    lib = ctypes.CDLL(NOALLOC_LIB_PATH)
    for name, (res, args) in NOALLOC_EXPORTS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _noalloc = lib
    return lib


def check(rc: int, what: str) -> None:
    if rc == SD_OK:
        return
    if rc in (SD_ERR_SHAPE, SD_ERR_ARG, SD_ERR_WORKSPACE):
        raise ValueError(f"{what}: rejected by the HIP library (code {rc})")
    raise RuntimeError(f"{what}: HIP launch failed (code {rc})")


def profile_enable(on: bool) -> None:
    load().sd_profile_enable(1 if on else 0)


def profile_read() -> dict:
    """Per-kernel (total_ms, launches) recorded since profile_enable(True)."""
    lib = load()
    n = lib.sd_profile_read(None, 0)
    buf = ctypes.create_string_buffer(n + 16)
    lib.sd_profile_read(buf, len(buf))
    out = {}
    for line in buf.value.decode().splitlines():
        name, ms, cnt = line.split()
        out[name] = (float(ms), int(cnt))
    return out
