"""SolveDelta mixer layer on MI355X: projections, conv4 frontend, decay gate,
operator and gated-RMSNorm readout.

Mirrors the reference module ``causallsso.model.SolveDelta``
(causallsso/model.py:27-477): the same parameter names, shapes and initial
distributions (so a reference state dict loads unchanged), the same forward
signature, and ``SolveDeltaLayerState(operator, conv)``.  The pieces the
reference runs through third-party CUDA/Triton code run here through the HIP
library: conv4 + SiLU (``sd_conv4_silu_*``, replacing causal-conv1d,
model.py:119-136), the KDA decay gate (``sd_kda_gate_*``, replacing
fla.ops.kda.gate, model.py:375-383), the sigmoid-gated RMSNorm owner
(``sd_rmsnorm_gated_*``, replacing FLA's fused norm gate, ops/norm_gate.py:46-150)
and the recurrence itself (``solvedelta_native``).  The dense projections are
plain library GEMMs (torch / hipBLASLt).

Activations must be bf16 on a ROCm device (a bf16 module or autocast), as the
reference's native path requires (model.py:338-341); there is no CPU path.
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import NamedTuple, Optional

import torch
import torch.nn.functional as F
from torch import nn

from . import _lib
from .operator import _ptr, _stream, solvedelta_native
from .masks import solvedelta_masked_native
from .state import SolveDeltaState


class SolveDeltaLayerState(NamedTuple):
    """(operator state (C, S), conv state [B, D_qkv, 3]) (model.py:22-24)."""
    operator: SolveDeltaState
    conv: Optional[torch.Tensor]


@dataclass
class SolveDeltaMixerConfig:
    """The mixer fields of the reference's SolveDeltaConfig (config.py:10-200).
    Any object with these attributes (the reference config included) works."""
    hidden_size: int = 2048
    num_heads: int = 16
    head_k_dim: Optional[int] = None
    head_v_dim: Optional[int] = None
    expand_k: float = 1.0
    expand_v: float = 1.0
    num_edits: int = 1
    use_short_conv: bool = True
    bias: bool = False
    norm_eps: float = 1e-6

    def __post_init__(self):
        if self.num_edits != 1:
            raise ValueError("the current SolveDelta production contract requires num_edits=1")
        _ = self.resolved_head_k_dim, self.resolved_head_v_dim

    def _resolve(self, explicit, expand, name):
        if explicit is not None:
            return explicit
        total_f = self.hidden_size * float(expand)
        total = round(total_f)
        if not math.isclose(total_f, total, rel_tol=0.0, abs_tol=1e-9):
            raise ValueError(f"hidden_size * {name} must be an integer, got {total_f}")
        if total % self.num_heads:
            raise ValueError(f"resolved total width {total} must be divisible by "
                             f"num_heads={self.num_heads}")
        return total // self.num_heads

    @property
    def resolved_head_k_dim(self) -> int:
        return self._resolve(self.head_k_dim, self.expand_k, "expand_k")

    @property
    def resolved_head_v_dim(self) -> int:
        return self._resolve(self.head_v_dim, self.expand_v, "expand_v")


def _require_device(*ts):
    for t in ts:
        if t is not None and t.device.type != "cuda":
            raise TypeError("the SolveDelta mixer runs on a ROCm device only")


# --------------------------------------------------------------------------
# conv4 + SiLU
# --------------------------------------------------------------------------
class _Conv4SiluFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, init, want_final: bool):
        lib = _lib.load()
        B, T, D = x.shape
        if x.dtype != torch.bfloat16 or x.stride(2) != 1:
            raise ValueError("conv4 input must be bf16 [B,T,D] with unit channel stride")
        if weight.shape != (D, 4):
            raise ValueError("conv weight must have shape [D,4]")
        w32 = weight.detach().float().contiguous()
        init_dtype = None if init is None else init.dtype
        if init is not None:
            if init.shape != (B, D, 3):
                raise ValueError("conv initial state must have shape [B,D,3]")
            init = init.to(torch.bfloat16).contiguous()
        y = torch.empty(B, T, D, dtype=torch.bfloat16, device=x.device)
        fin = torch.empty(B, D, 3, dtype=torch.bfloat16, device=x.device) if want_final else None
        rc = lib.sd_conv4_silu_fwd(B, T, D, x.data_ptr(), x.stride(0), x.stride(1), w32.data_ptr(),
                                   _ptr(init), y.data_ptr(), _ptr(fin), _stream(x.device))
        _lib.check(rc, "sd_conv4_silu_fwd")
        ctx.save_for_backward(x, w32, init if init is not None else x.new_empty(0))
        ctx.has_init = init is not None
        ctx.wdtype = weight.dtype
        ctx.idtype = None if init is None else init_dtype
        ctx.set_materialize_grads(False)
        return y, fin

    @staticmethod
    def backward(ctx, dy, dfin):
        lib = _lib.load()
        x, w32, init = ctx.saved_tensors
        init = init if ctx.has_init else None
        B, T, D = x.shape
        if dy is None and dfin is None:
            return None, None, None, None
        dy = (torch.zeros(B, T, D, dtype=torch.bfloat16, device=x.device) if dy is None
              else dy.to(torch.bfloat16).contiguous())
        dfin = None if dfin is None else dfin.to(torch.bfloat16).contiguous()
        dx = torch.empty(B, T, D, dtype=torch.bfloat16, device=x.device)
        dw = torch.empty(D, 4, dtype=torch.float32, device=x.device)
        dinit = torch.empty(B, D, 3, dtype=torch.float32, device=x.device) if init is not None else None
        nb = lib.sd_conv4_workspace_bytes(B, T, D)
        ws = torch.empty(nb, dtype=torch.uint8, device=x.device)
        rc = lib.sd_conv4_silu_bwd(B, T, D, x.data_ptr(), x.stride(0), x.stride(1), w32.data_ptr(),
                                   _ptr(init), dy.data_ptr(), _ptr(dfin), dx.data_ptr(),
                                   dw.data_ptr(), _ptr(dinit), ws.data_ptr(), nb, _stream(x.device))
        _lib.check(rc, "sd_conv4_silu_bwd")
        return dx, dw.to(ctx.wdtype), None if dinit is None else dinit.to(ctx.idtype), None


class _Conv4SiluMaskedFn(torch.autograd.Function):
    """conv4 + SiLU under valid / reset masks on the dense batch (the CPU
    loop's semantics, model.py:146-164), without repacking."""

    @staticmethod
    def forward(ctx, x, weight, init, valid, reset, want_final: bool):
        lib = _lib.load()
        B, T, D = x.shape
        if x.dtype != torch.bfloat16 or x.stride(2) != 1:
            raise ValueError("conv4 input must be bf16 [B,T,D] with unit channel stride")
        if weight.shape != (D, 4):
            raise ValueError("conv weight must have shape [D,4]")
        w32 = weight.detach().float().contiguous()
        init_dtype = None if init is None else init.dtype
        if init is not None:
            if init.shape != (B, D, 3):
                raise ValueError("conv initial state must have shape [B,D,3]")
            init = init.to(torch.bfloat16).contiguous()
        valid = valid.to(torch.uint8).contiguous()
        reset = reset.to(torch.uint8).contiguous()
        y = torch.empty(B, T, D, dtype=torch.bfloat16, device=x.device)
        fin = torch.empty(B, D, 3, dtype=torch.bfloat16, device=x.device) if want_final else None
        rc = lib.sd_conv4_silu_masked_fwd(B, T, D, x.data_ptr(), x.stride(0), x.stride(1),
                                          w32.data_ptr(), _ptr(init), valid.data_ptr(),
                                          reset.data_ptr(), T, 1, y.data_ptr(), _ptr(fin),
                                          _stream(x.device))
        _lib.check(rc, "sd_conv4_silu_masked_fwd")
        ctx.save_for_backward(x, w32, init if init is not None else x.new_empty(0), valid, reset)
        ctx.has_init = init is not None
        ctx.wdtype = weight.dtype
        ctx.idtype = init_dtype
        ctx.set_materialize_grads(False)
        return y, fin

    @staticmethod
    def backward(ctx, dy, dfin):
        lib = _lib.load()
        x, w32, init, valid, reset = ctx.saved_tensors
        init = init if ctx.has_init else None
        B, T, D = x.shape
        if dy is None and dfin is None:
            return None, None, None, None, None, None
        dy = (torch.zeros(B, T, D, dtype=torch.bfloat16, device=x.device) if dy is None
              else dy.to(torch.bfloat16).contiguous())
        dfin = None if dfin is None else dfin.to(torch.bfloat16).contiguous()
        dx = torch.empty(B, T, D, dtype=torch.bfloat16, device=x.device)
        dw = torch.empty(D, 4, dtype=torch.float32, device=x.device)
        dinit = torch.empty(B, D, 3, dtype=torch.float32, device=x.device) if init is not None else None
        nb = lib.sd_conv4_masked_workspace_bytes(B, D)
        ws = torch.empty(nb, dtype=torch.uint8, device=x.device)
        rc = lib.sd_conv4_silu_masked_bwd(B, T, D, x.data_ptr(), x.stride(0), x.stride(1),
                                          w32.data_ptr(), _ptr(init), valid.data_ptr(),
                                          reset.data_ptr(), T, 1, dy.data_ptr(), _ptr(dfin),
                                          dx.data_ptr(), dw.data_ptr(), _ptr(dinit), ws.data_ptr(),
                                          nb, _stream(x.device))
        _lib.check(rc, "sd_conv4_silu_masked_bwd")
        return (dx, dw.to(ctx.wdtype), None if dinit is None else dinit.to(ctx.idtype), None,
                None, None)


def conv4_silu_masked(x, weight, valid_mask, reset_mask, initial_state=None,
                      return_final_state=False):
    """conv4 + SiLU under bool [B,T] valid / reset masks (model.py:146-164)."""
    _require_device(x, weight, initial_state, valid_mask, reset_mask)
    return _Conv4SiluMaskedFn.apply(x, weight, initial_state, valid_mask, reset_mask,
                                    return_final_state)


def conv4_silu(x, weight, initial_state=None, return_final_state=False):
    """causal_conv1d_fn(x^T, weight, initial_states, return_final_states,
    activation="silu") on [B,T,D] activations (model.py:119-136)."""
    _require_device(x, weight, initial_state)
    return _Conv4SiluFn.apply(x, weight, initial_state, return_final_state)


# --------------------------------------------------------------------------
# KDA decay gate
# --------------------------------------------------------------------------
class _KdaGateFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, raw, log_rate, bias):
        lib = _lib.load()
        B, T, H, r = raw.shape
        raw = raw.to(torch.bfloat16).contiguous()
        lr = log_rate.detach().float().contiguous()
        bs = bias.detach().float().contiguous().reshape(-1)
        out = torch.empty(B, T, H, r, dtype=torch.float32, device=raw.device)
        rc = lib.sd_kda_gate_fwd(B * T, H, r, raw.data_ptr(), H * r, lr.data_ptr(), bs.data_ptr(),
                                 out.data_ptr(), _stream(raw.device))
        _lib.check(rc, "sd_kda_gate_fwd")
        ctx.save_for_backward(raw, lr, bs)
        ctx.dtypes = (log_rate.dtype, bias.dtype, bias.shape)
        return out

    @staticmethod
    def backward(ctx, dout):
        lib = _lib.load()
        raw, lr, bs = ctx.saved_tensors
        B, T, H, r = raw.shape
        dout = dout.float().contiguous()
        draw = torch.empty_like(raw)
        dlr = torch.empty(H, dtype=torch.float32, device=raw.device)
        db = torch.empty(H * r, dtype=torch.float32, device=raw.device)
        nb = lib.sd_kda_gate_workspace_bytes(B * T, H, r)
        ws = torch.empty(nb, dtype=torch.uint8, device=raw.device)
        rc = lib.sd_kda_gate_bwd(B * T, H, r, raw.data_ptr(), H * r, lr.data_ptr(), bs.data_ptr(),
                                 dout.data_ptr(), draw.data_ptr(), dlr.data_ptr(), db.data_ptr(),
                                 ws.data_ptr(), nb, _stream(raw.device))
        _lib.check(rc, "sd_kda_gate_bwd")
        lr_dt, b_dt, b_shape = ctx.dtypes
        return draw, dlr.to(lr_dt), db.reshape(b_shape).to(b_dt)


def kda_decay_gate(raw, log_rate, bias):
    """log_decay = -exp(log_rate[h]) softplus(raw + bias[h,c]) in FP32
    (model.py:375-390); raw [B,T,H,r], log_rate [H], bias [H,r] or [H*r]."""
    _require_device(raw, log_rate, bias)
    return _KdaGateFn.apply(raw, log_rate, bias)


# --------------------------------------------------------------------------
# sigmoid-gated RMSNorm (+ output projection)
# --------------------------------------------------------------------------
def _rms_fwd(x2, g2, w32, eps):
    lib = _lib.load()
    N, D = x2.shape
    y = torch.empty_like(x2)
    rc = lib.sd_rmsnorm_gated_fwd(N, D, float(eps), x2.data_ptr(), g2.data_ptr(), w32.data_ptr(),
                                  y.data_ptr(), None, _stream(x2.device))
    _lib.check(rc, "sd_rmsnorm_gated_fwd")
    return y


def _rms_bwd(x2, g2, w32, dy2, eps, want_y):
    lib = _lib.load()
    N, D = x2.shape
    dx, dg = torch.empty_like(x2), torch.empty_like(x2)
    y = torch.empty_like(x2) if want_y else None
    dw = torch.empty(D, dtype=torch.float32, device=x2.device)
    nb = lib.sd_rmsnorm_gated_workspace_bytes(N, D)
    ws = torch.empty(nb, dtype=torch.uint8, device=x2.device)
    rc = lib.sd_rmsnorm_gated_bwd(N, D, float(eps), x2.data_ptr(), g2.data_ptr(), w32.data_ptr(),
                                  dy2.data_ptr(), dx.data_ptr(), dg.data_ptr(), dw.data_ptr(),
                                  _ptr(y), ws.data_ptr(), nb, _stream(x2.device))
    _lib.check(rc, "sd_rmsnorm_gated_bwd")
    return dx, dg, dw, y


class _RMSNormGatedFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, gate, weight, eps):
        D = x.shape[-1]
        x2 = x.to(torch.bfloat16).contiguous().reshape(-1, D)
        g2 = gate.to(torch.bfloat16).contiguous().reshape(-1, D)
        w32 = weight.detach().float().contiguous()
        y = _rms_fwd(x2, g2, w32, eps)
        ctx.save_for_backward(x2, g2, w32)
        ctx.eps, ctx.shape, ctx.wdt = eps, x.shape, weight.dtype
        ctx.xdt, ctx.gdt = x.dtype, gate.dtype
        return y.reshape(x.shape)

    @staticmethod
    def backward(ctx, dy):
        x2, g2, w32 = ctx.saved_tensors
        dy2 = dy.to(torch.bfloat16).contiguous().reshape(x2.shape)
        dx, dg, dw, _ = _rms_bwd(x2, g2, w32, dy2, ctx.eps, False)
        return (dx.reshape(ctx.shape).to(ctx.xdt), dg.reshape(ctx.shape).to(ctx.gdt),
                dw.to(ctx.wdt), None)


class _RMSNormGatedLinearFn(torch.autograd.Function):
    """Norm owner that recomputes its output for the projection's weight
    gradient instead of saving it (ops/norm_gate.py:46-150)."""

    @staticmethod
    def forward(ctx, x, gate, norm_weight, lin_weight, lin_bias, eps):
        D = x.shape[-1]
        lead = x.shape[:-2]
        x2 = x.to(torch.bfloat16).contiguous().reshape(-1, D)
        g2 = gate.to(torch.bfloat16).contiguous().reshape(-1, D)
        w32 = norm_weight.detach().float().contiguous()
        y = _rms_fwd(x2, g2, w32, eps)
        wl = lin_weight.detach().to(torch.bfloat16)
        bl = None if lin_bias is None else lin_bias.detach().to(torch.bfloat16)
        out = F.linear(y.reshape(*lead, -1), wl, bl)
        ctx.save_for_backward(x2, g2, w32, wl)
        ctx.eps, ctx.shape = eps, x.shape
        ctx.dtypes = (x.dtype, gate.dtype, norm_weight.dtype, lin_weight.dtype,
                      None if lin_bias is None else lin_bias.dtype)
        ctx.set_materialize_grads(False)
        return out

    @staticmethod
    def backward(ctx, dout):
        if dout is None:
            return (None,) * 6
        x2, g2, w32, wl = ctx.saved_tensors
        xdt, gdt, nwdt, lwdt, lbdt = ctx.dtypes
        d2 = dout.to(torch.bfloat16).contiguous().reshape(-1, dout.shape[-1])
        dy = F.linear(d2, wl.t()).reshape(x2.shape).contiguous()
        dx, dg, dw, y = _rms_bwd(x2, g2, w32, dy, ctx.eps, True)
        dlw = torch.mm(d2.t(), y.reshape(d2.shape[0], -1)).to(lwdt)
        dlb = None if lbdt is None else d2.float().sum(0).to(lbdt)
        return (dx.reshape(ctx.shape).to(xdt), dg.reshape(ctx.shape).to(gdt), dw.to(nwdt), dlw,
                dlb, None)


class RMSNormGated(nn.Module):
    """Sigmoid-gated RMSNorm (ops/norm_gate.py:153-212): same parameter and
    attributes; HIP kernels forward and backward."""

    def __init__(self, hidden_size: int, eps: float = 1e-6, *, device=None, dtype=None):
        super().__init__()
        self.hidden_size = hidden_size
        self.eps = eps
        self.activation = "sigmoid"
        self.weight = nn.Parameter(torch.ones(hidden_size, device=device, dtype=dtype))

    def forward(self, x, gate):
        _require_device(x, gate)
        if x.shape != gate.shape or x.ndim < 2:
            raise ValueError("x and gate must have the same [...,H,D] shape")
        return _RMSNormGatedFn.apply(x, gate, self.weight, self.eps)

    def forward_linear(self, x, gate, linear: nn.Linear):
        """Gated norm followed by ``linear`` without saving the normalised panel."""
        _require_device(x, gate)
        if x.shape != gate.shape or x.ndim < 2:
            raise ValueError("x and gate must have the same [...,H,D] shape")
        return _RMSNormGatedLinearFn.apply(x, gate, self.weight, linear.weight, linear.bias,
                                           self.eps)


# --------------------------------------------------------------------------
# projection split
# --------------------------------------------------------------------------
class _SplitColumns(torch.autograd.Function):
    """Column pieces of the packed projection as views; the backward joins the
    pieces' gradients with one concatenation (zeros only for absent pieces and
    the padding columns), instead of split backward's zero-filled buffer plus a
    copy per piece: at 24 layers the launches, not the bytes, are what cost."""

    @staticmethod
    def forward(ctx, x, sizes):
        ctx.sizes, ctx.shape, ctx.dtype = sizes, x.shape, x.dtype
        ctx.set_materialize_grads(False)
        return tuple(x[..., : sum(sizes)].split(sizes, dim=-1))

    @staticmethod
    def backward(ctx, *grads):
        dev = next(t for t in grads if t is not None).device
        lead = tuple(ctx.shape[:-1])
        parts = [gi.to(ctx.dtype) if gi is not None else
                 torch.zeros(lead + (n,), dtype=ctx.dtype, device=dev)
                 for n, gi in zip(ctx.sizes, grads)]
        pad = ctx.shape[-1] - sum(ctx.sizes)
        if pad:
            parts.append(torch.zeros(lead + (pad,), dtype=ctx.dtype, device=dev))
        return torch.cat(parts, dim=-1), None


# --------------------------------------------------------------------------
# the mixer
# --------------------------------------------------------------------------
class SolveDelta(nn.Module):
    """Projection, conv4, operator and output owner (model.py:27-474)."""

    def __init__(self, config) -> None:
        super().__init__()
        self.config = config
        heads = config.num_heads
        width = config.resolved_head_k_dim
        value_width = config.resolved_head_v_dim
        edits = config.num_edits
        if edits != 1:
            raise ValueError("the current SolveDelta production contract requires num_edits=1")
        gate_rank = value_width
        self.projection_sizes = (heads * width, heads * edits * width, heads * edits * value_width,
                                 heads * width, heads * width, heads * edits * width,
                                 heads * edits * value_width, heads, gate_rank, gate_rank)
        self.projection_width = sum(self.projection_sizes)
        # rows padded to a multiple of 64 for the GEMM; only the prefix is used
        self.projection_padding = (-self.projection_width) % 64
        self.in_proj = nn.Linear(config.hidden_size, self.projection_width + self.projection_padding,
                                 bias=config.bias)
        self.output_proj = nn.Linear(heads * value_width, config.hidden_size, bias=config.bias)
        self.decay_proj = nn.Linear(gate_rank, heads * width, bias=False)
        self.output_gate_proj = nn.Linear(gate_rank, heads * value_width, bias=True)
        self.output_norm = RMSNormGated(value_width, eps=config.norm_eps)
        if config.use_short_conv:
            conv_width = sum(self.projection_sizes[:3])
            self.conv_weight = nn.Parameter(torch.empty(conv_width, 4))
            nn.init.kaiming_uniform_(self.conv_weight, a=5 ** 0.5)
        # token-local normalised-LMS write rate: sigmoid(log 9) = 0.9 at init
        self.geometry_write_bias = nn.Parameter(torch.full((heads,), math.log(9.0),
                                                           dtype=torch.float32))
        # decay: rate ~ U(1, 16), step log-uniform in [1e-3, 1e-1], bias = softplus^-1(step)
        rate = torch.empty(heads, dtype=torch.float32).uniform_(1, 16)
        self.associative_log_rate = nn.Parameter(rate.log())
        step = torch.exp(torch.rand(heads, width, dtype=torch.float32)
                         * (math.log(0.1) - math.log(0.001)) + math.log(0.001)).clamp_min_(1e-4)
        self.associative_decay_bias = nn.Parameter(step + torch.log(-torch.expm1(-step)))
        for p in (self.geometry_write_bias, self.associative_log_rate,
                  self.associative_decay_bias):
            p._no_weight_decay = True

    def _gate_output(self, output, gate):
        return self.output_norm(output, gate)

    def forward(self, hidden_states, *, initial_state: Optional[SolveDeltaLayerState] = None,
                valid_mask=None, reset_mask=None, geometry_enabled: bool = True,
                associative_decay_enabled: bool = True, return_final_state: bool = False):
        if hidden_states.ndim != 3:
            raise ValueError("hidden_states must have shape [B,T,hidden_size]")
        B, T, hw = hidden_states.shape
        if hw != self.config.hidden_size:
            raise ValueError("hidden state width does not match the configuration")
        _require_device(hidden_states)
        H = self.config.num_heads
        rk = self.config.resolved_head_k_dim
        rv = self.config.resolved_head_v_dim
        proj = self.in_proj(hidden_states)
        if proj.dtype != torch.bfloat16:
            raise TypeError("the native SolveDelta mixer needs bf16 activations "
                            "(a bf16 module or autocast)")
        # masks run on the dense batch (conv4 under masks, then the operator with
        # neutral invalid tokens and reset tokens): no repacking, no host sync
        masked = valid_mask is not None or reset_mask is not None
        if masked:
            if valid_mask is None:
                valid_mask = torch.ones(B, T, dtype=torch.bool, device=hidden_states.device)
            if reset_mask is None:
                reset_mask = torch.zeros(B, T, dtype=torch.bool, device=hidden_states.device)
            if valid_mask.device != hidden_states.device or reset_mask.device != hidden_states.device:
                raise ValueError("masks must share the activation device")
            if (valid_mask.shape != (B, T) or reset_mask.shape != (B, T)
                    or valid_mask.dtype != torch.bool or reset_mask.dtype != torch.bool):
                raise ValueError("valid_mask and reset_mask must be bool [B,T]")
        conv_state = initial_state.conv if initial_state is not None else None
        sizes = self.projection_sizes
        final_conv = None
        if self.config.use_short_conv:
            qkv_w = sum(sizes[:3])
            qkv_proj, *rest = _SplitColumns.apply(proj, (qkv_w,) + tuple(sizes[3:]))
            if conv_state is not None and (conv_state.shape != (B, qkv_w, 3)):
                raise ValueError("conv initial state must have shape [B,D,3]")
            if not masked:
                qkv, final_conv = conv4_silu(qkv_proj, self.conv_weight, conv_state,
                                             return_final_state)
            else:
                qkv, final_conv = conv4_silu_masked(qkv_proj, self.conv_weight, valid_mask,
                                                    reset_mask, conv_state, return_final_state)
            q_raw, k_raw, v_raw = qkv.split(sizes[:3], dim=-1)
        else:
            parts = _SplitColumns.apply(proj, tuple(sizes))
            q_raw, k_raw, v_raw = (F.silu(t) for t in parts[:3])
            rest = parts[3:]
        u_raw, h_raw, erase_raw, write_raw, geometry_raw, decay_hidden, gate_hidden = rest
        u = u_raw.view(B, T, H, rk)
        h = h_raw.view(B, T, H, rk)
        q = q_raw.view(B, T, H, rk)
        keys = k_raw.view(B, T, H, 1, rk)
        values = v_raw.view(B, T, H, 1, rv)
        log_decay = kda_decay_gate(self.decay_proj(decay_hidden).view(B, T, H, rk),
                                   self.associative_log_rate, self.associative_decay_bias)
        # bf16 + fp32 promotes to fp32 exactly, in one kernel
        gamma = torch.sigmoid(geometry_raw + self.geometry_write_bias.float().view(1, 1, H))
        if not geometry_enabled:
            gamma = torch.zeros_like(gamma)
        if not associative_decay_enabled:
            log_decay = torch.zeros_like(log_decay)
        gate = self.output_gate_proj(gate_hidden).view(B, T, H, rv)
        op_init = initial_state.operator if initial_state is not None else None
        erase = erase_raw.view(B, T, H, 1, rk)
        write = write_raw.view(B, T, H, 1, rv)
        if masked:
            out, op_state = solvedelta_masked_native(
                u, h, q, keys, values, log_decay, erase, write, gamma, valid_mask, reset_mask,
                initial_state=op_init, return_final_state=return_final_state)
        else:
            out, op_state = solvedelta_native(
                u, h, q, keys, values, log_decay, erase, write, gamma,
                initial_state=op_init, return_final_state=return_final_state)
        y = self.output_norm.forward_linear(out, gate.to(out.dtype), self.output_proj)
        if not return_final_state:
            return y
        if op_state is None:
            raise RuntimeError("operator did not return the requested final state")
        return y, SolveDeltaLayerState(op_state, final_conv)


__all__ = ["SolveDelta", "SolveDeltaLayerState", "SolveDeltaMixerConfig", "RMSNormGated",
           "conv4_silu", "conv4_silu_masked", "kda_decay_gate"]
