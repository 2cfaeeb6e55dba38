"""Public SolveDelta operator on MI355X: the drop-in for the reference's
``solvedelta_native`` (causallsso/ops/operator.py:13-55 and
causallsso/ops/residual_frame/operator.py:154-304).

Same positional order, keyword arguments, return type, dtype/shape/stride
checks and exception types as the reference; the arithmetic runs in the HIP
library (include/solvedelta.h) on the current stream with no host sync.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib
from .state import SolveDeltaState


# widest key and value widths of the main kernels; widths up to _WIDE_MAX run on
# the library's wide-width kernels (include/solvedelta.h), as the reference's
# state pass takes head widths up to 256 (residual_frame/common_left_h.py:139-140)
_MAX_WIDTH = 128
_WIDE_MAX = 256


def _view(t: torch.Tensor) -> _lib.SdView:
    return _lib.SdView(t.data_ptr(), t.stride(0), t.stride(1), t.stride(2))


def _gamma_view(g: torch.Tensor, B: int, T: int, H: int) -> _lib.SdView:
    if g.shape == (H,):
        return _lib.SdView(g.data_ptr(), 0, 0, g.stride(0))
    if g.shape == (1, H):
        return _lib.SdView(g.data_ptr(), 0, 0, g.stride(1))
    return _lib.SdView(g.data_ptr(), g.stride(0), g.stride(1), g.stride(2))


def _fresh_view(fresh: Optional[torch.Tensor]) -> _lib.SdView:
    if fresh is None:
        return _lib.SdView(None, 0, 0, 0)
    return _lib.SdView(fresh.data_ptr(), fresh.stride(0), fresh.stride(1), 0)


def _inputs(u, h, q, keys, values, log_decay, erase_raw, write_raw, gamma, C0, S0, fresh=None):
    B, T, H, r = u.shape
    V = values.shape[-1]
    return _lib.SdInputs(
        B, T, H, r, V, _view(u), _view(h), _view(q), _view(keys), _view(values),
        _view(erase_raw), _view(write_raw), _view(log_decay), _gamma_view(gamma, B, T, H),
        None if C0 is None else C0.data_ptr(), None if S0 is None else S0.data_ptr(),
        _fresh_view(fresh))


def _stream(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


class _SolveDeltaFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, u, h, q, keys, values, log_decay, erase_raw, write_raw, gamma, C0, S0,
                want_state: bool, fresh=None):
        lib = _lib.load()
        B, T, H, r = u.shape
        V = values.shape[-1]
        dev = u.device
        ins = _inputs(u, h, q, keys, values, log_decay, erase_raw, write_raw, gamma, C0, S0, fresh)
        out = torch.empty(B, T, H, V, dtype=torch.bfloat16, device=dev)
        C_T = torch.empty(B, H, r, r, dtype=torch.float32, device=dev) if want_state else None
        S_T = torch.empty(B, H, r, V, dtype=torch.float32, device=dev) if want_state else None
        # the saved region is held for the backward; the scratch region (panels
        # only the forward's state passes read) returns to the allocator here
        nsaved = lib.sd_fwd_saved_bytes(B, T, H, r, V)
        nscratch = lib.sd_fwd_scratch_bytes(B, T, H, r, V)
        ws = torch.empty(nsaved, dtype=torch.uint8, device=dev)
        scratch = torch.empty(nscratch, dtype=torch.uint8, device=dev)
        rc = lib.sd_fwd_split(ctypes.byref(ins), out.data_ptr(), _ptr(C_T), _ptr(S_T),
                              ws.data_ptr(), nsaved, scratch.data_ptr(), nscratch, _stream(dev))
        _lib.check(rc, "sd_fwd_split")
        del scratch
        ctx.set_materialize_grads(False)
        ctx.has_C0, ctx.has_S0 = C0 is not None, S0 is not None
        ctx.has_fresh = fresh is not None
        empty = u.new_empty(0)
        ctx.save_for_backward(u, h, q, keys, values, log_decay, erase_raw, write_raw, gamma,
                              C0 if C0 is not None else empty, S0 if S0 is not None else empty, ws,
                              fresh if fresh is not None else empty)
        if want_state:
            return out, C_T, S_T
        return out, None, None

    @staticmethod
    def backward(ctx, dout, dC, dS):
        lib = _lib.load()
        (u, h, q, keys, values, log_decay, erase_raw, write_raw, gamma, C0, S0,
         ws, fresh) = ctx.saved_tensors
        C0 = C0 if ctx.has_C0 else None
        S0 = S0 if ctx.has_S0 else None
        fresh = fresh if ctx.has_fresh else None
        B, T, H, r = u.shape
        V = values.shape[-1]
        dev = u.device
        ins = _inputs(u, h, q, keys, values, log_decay, erase_raw, write_raw, gamma, C0, S0, fresh)
        dout = None if dout is None else dout.to(torch.bfloat16).contiguous()
        dC = None if dC is None else dC.float().contiguous()
        dS = None if dS is None else dS.float().contiguous()
        bf = dict(dtype=torch.bfloat16, device=dev)
        du, dh, dq = (torch.empty(B, T, H, r, **bf) for _ in range(3))
        dk, der = (torch.empty(B, T, H, 1, r, **bf) for _ in range(2))
        dv, dwr = (torch.empty(B, T, H, 1, V, **bf) for _ in range(2))
        dg = torch.empty(B, T, H, r, dtype=torch.float32, device=dev)
        dgam = torch.empty(B, T, H, dtype=torch.float32, device=dev)
        dC0 = torch.empty(B, H, r, r, dtype=torch.float32, device=dev) if C0 is not None else None
        dS0 = torch.empty(B, H, r, V, dtype=torch.float32, device=dev) if S0 is not None else None
        nbytes = lib.sd_bwd_workspace_bytes(B, T, H, r, V)
        bws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        rc = lib.sd_bwd(ctypes.byref(ins), ws.data_ptr(), _ptr(dout), _ptr(dC), _ptr(dS),
                        du.data_ptr(), dh.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                        der.data_ptr(), dwr.data_ptr(), dg.data_ptr(), dgam.data_ptr(), _ptr(dC0),
                        _ptr(dS0), bws.data_ptr(), nbytes, _stream(dev))
        _lib.check(rc, "sd_bwd")
        if gamma.shape != (B, T, H):
            dgam = dgam.sum(dim=(0, 1)).reshape(gamma.shape)
        return (du.to(u.dtype), dh.to(h.dtype), dq.to(q.dtype), dk.to(keys.dtype),
                dv.to(values.dtype), dg.to(log_decay.dtype), der.to(erase_raw.dtype),
                dwr.to(write_raw.dtype), dgam.to(gamma.dtype), dC0, dS0, None, None)


def _decode(u, h, q, keys, values, log_decay, erase_raw, write_raw, gamma, initial_state,
            return_final_state, fresh=None):
    """T = 1 recurrent step (reference: residual_frame/recurrent.py:188-327)."""
    lib = _lib.load()
    B, T, H, r = u.shape
    V = values.shape[-1]
    dev = u.device
    C0 = S0 = None
    if initial_state is not None:
        C0, S0 = (s.contiguous() for s in initial_state)
    ins = _inputs(u, h, q, keys, values, log_decay, erase_raw, write_raw, gamma, C0, S0, fresh)
    out = torch.empty(B, 1, H, V, dtype=torch.bfloat16, device=dev)
    C_T = torch.empty(B, H, r, r, dtype=torch.float32, device=dev) if return_final_state else None
    S_T = torch.empty(B, H, r, V, dtype=torch.float32, device=dev) if return_final_state else None
    rc = lib.sd_decode(ctypes.byref(ins), out.data_ptr(), _ptr(C_T), _ptr(S_T), _stream(dev))
    _lib.check(rc, "sd_decode")
    if not return_final_state:
        return out, None
    return out, SolveDeltaState(C_T, S_T)


def _validate(u, h, q, keys, values, associative_log_decay, erase_raw, write_raw,
              geometry_write, initial_state):
    """The reference's operand checks (ops/operator.py:28-40, then
    residual_frame/operator.py:169-196 and :251-261, in that order); returns
    the log-decay with a unit inner stride."""
    if u.device.type != "cuda" or u.dtype != torch.bfloat16:
        raise TypeError("solvedelta_native requires BF16 CUDA activations")
    if keys.ndim != 5 or keys.shape[-2] != 1:
        raise ValueError("the current production path requires num_edits=1")
    if erase_raw.shape != keys.shape or erase_raw.dtype != torch.bfloat16:
        raise ValueError("erase_raw must be BF16 with the same shape as keys")
    if write_raw.shape != values.shape or write_raw.dtype != torch.bfloat16:
        raise ValueError("write_raw must be BF16 with the same shape as values")
    if any(x.stride(-1) != 1 for x in (u, h, q, keys, values, erase_raw, write_raw)):
        raise ValueError("native vector operands require unit innermost stride")
    if u.ndim != 4:
        raise ValueError("u must have shape [B,T,H,r]")
    B, T, H, r = u.shape
    if h.shape != u.shape or q.shape != u.shape:
        raise ValueError("h and q must match u")
    if keys.shape != (B, T, H, 1, r):
        raise ValueError("Residual-Frame SolveDelta requires keys [B,T,H,1,r]")
    if values.ndim != 5 or values.shape[:4] != (B, T, H, 1):
        raise ValueError("values must have shape [B,T,H,1,d_v]")
    V = values.shape[-1]
    if associative_log_decay.shape != (B, T, H, r):
        raise ValueError("associative_log_decay must have shape [B,T,H,r]")
    if geometry_write.shape not in ((H,), (1, H), (B, T, H)):
        raise ValueError("geometry_write must have shape [H], [1,H], or [B,T,H]")
    if any(x.dtype != u.dtype for x in (h, q, keys, values, erase_raw, write_raw)):
        raise TypeError("all public vector operands must be BF16")
    if associative_log_decay.dtype != torch.float32:
        raise TypeError("associative_log_decay must be FP32")
    if geometry_write.dtype != torch.float32:
        raise TypeError("geometry_write must be FP32")
    if r > _WIDE_MAX:
        # residual_frame/common_left_h.py:140 asserts the same bound
        raise AssertionError("current kernel does not support head dimension larger than 256.")
    if associative_log_decay.stride(-1) != 1:
        associative_log_decay = associative_log_decay.contiguous()
    if initial_state is not None:
        expected = ((B, H, r, r), (B, H, r, V))
        if any(s.shape != e for s, e in zip(initial_state, expected)):
            raise ValueError("initial_state shapes do not match the input geometry")
        if any(s.dtype != torch.float32 for s in initial_state):
            raise TypeError("all continuation states must be FP32")
    return associative_log_decay


def solvedelta_native(
    u: torch.Tensor,
    h: torch.Tensor,
    q: torch.Tensor,
    keys: torch.Tensor,
    values: torch.Tensor,
    associative_log_decay: torch.Tensor,
    erase_raw: torch.Tensor,
    write_raw: torch.Tensor,
    geometry_write: torch.Tensor,
    *,
    initial_state: Optional[SolveDeltaState] = None,
    return_final_state: bool = False,
) -> tuple[torch.Tensor, Optional[SolveDeltaState]]:
    """Dense K=1 SolveDelta from raw fused-projection views.

    Checks follow ops/operator.py:28-40 then residual_frame/operator.py:169-196
    and :251-261 in that order; raw erase/write logits are activated inside.
    """
    associative_log_decay = _validate(u, h, q, keys, values, associative_log_decay, erase_raw,
                                      write_raw, geometry_write, initial_state)
    return _dispatch(u, h, q, keys, values, associative_log_decay, erase_raw, write_raw,
                     geometry_write, initial_state, return_final_state)


def _dispatch(u, h, q, keys, values, log_decay, erase_raw, write_raw, gamma, initial_state,
              return_final_state, fresh=None):
    """Validated operands -> decode kernel (T = 1, no grad, r, V <= 128, as
    residual_frame/operator.py:198-216) or the chunked kernels, in value groups
    above the kernels' value width.  `fresh` is the optional uint8 [B,T] token
    flags the kernels read (fresh, invalid, reset: include/solvedelta.h)."""
    B, T, H, r = u.shape
    V = values.shape[-1]
    if T == 1 and r <= _MAX_WIDTH and V <= _MAX_WIDTH and not torch.is_grad_enabled():
        return _decode(u, h, q, keys, values, log_decay, erase_raw, write_raw, gamma,
                       initial_state, return_final_state, fresh)
    C0 = S0 = None
    if initial_state is not None:
        C0, S0 = (s.contiguous() for s in initial_state)
    group = _WIDE_MAX if value_route(r, V) == "wide" else _MAX_WIDTH
    if V <= group:
        out, C_T, S_T = _SolveDeltaFn.apply(u, h, q, keys, values, log_decay, erase_raw,
                                            write_raw, gamma, C0, S0, return_final_state, fresh)
    else:
        out, C_T, S_T = _value_groups(u, h, q, keys, values, log_decay, erase_raw, write_raw,
                                      gamma, C0, S0, return_final_state, group, fresh)
    if not return_final_state:
        return out, None
    return out, SolveDeltaState(C_T, S_T)


def value_route(r: int, V: int) -> str:
    """How a call of key width r and value width V runs: "main" (r, V <= 128:
    the 64-token kernels) or "wide" (the wide-width kernels, which take r, V <=
    256; V above 256 in groups of 256 columns).  For r <= 128 < V <= 256 one
    wide call (F+B 1.95 ms at B4 T2048 H8 r=128 V=256 on MI355X) beat two
    128-column groups on the main kernels, each recomputing the predictor
    (2.13 ms)."""
    if r <= _MAX_WIDTH and V <= _MAX_WIDTH:
        return "main"
    return "wide"


def _value_groups(u, h, q, keys, values, log_decay, erase_raw, write_raw, gamma, C0, S0,
                  want_state, group, fresh=None):
    """V above the kernels' value width (128, or 256 on the wide kernels): the
    columns of S (and of the output) evolve independently given the shared predictor C and the sources d, e, chi, so the value axis is cut
    into groups of at most `group` columns, each run by the HIP path with the same
    key-side inputs.  Every group recomputes the predictor identically; the
    output and S are the groups' concatenation and C_T comes from the first
    group, so autograd sums the shared inputs' gradients over the groups."""
    V = values.shape[-1]
    outs, S_parts, C_T = [], [], None
    for g0 in range(0, V, group):
        g1 = min(V, g0 + group)
        S0g = None if S0 is None else S0[..., g0:g1].contiguous()
        o, C, S = _SolveDeltaFn.apply(u, h, q, keys, values[..., g0:g1], log_decay, erase_raw,
                                      write_raw[..., g0:g1], gamma, C0, S0g, want_state, fresh)
        outs.append(o)
        S_parts.append(S)
        if g0 == 0:
            C_T = C
    out = torch.cat(outs, dim=-1)
    S_T = torch.cat(S_parts, dim=-1) if want_state else None
    return out, C_T, S_T


__all__ = ["solvedelta_native"]
