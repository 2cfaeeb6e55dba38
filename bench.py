"""Benchmark: SolveDelta layer forward + full VJP on one MI355X.

Workload (timed at configs[1]'s shape): B=4, T=2048,
H=8, r=V=128, bf16 operands, FP32 state, chunk 64 inside the HIP kernels.
Synthetic seeded inputs: u,h,v ~ N(0,1); q,k per-head L2-normalised N(0,1);
raw erase/write ~ N(0,1) (gates sigmoid(N(0,1))); log-decay = -softplus(N(0,1));
gamma = 0.9 (the mixer's default sigmoid(log 9)); random FP32 initial (C,S) at
0.02 N(0,1); upstream dO ~ N(0,1).  One step = solvedelta_native forward plus
torch.autograd.grad for all 9 inputs and both initial states.

Prints ONE JSON line (rank 0).  Besides the throughput it reports:
  roofline      the step's dominant kernel, timed with HIP events on its launch
                stream inside a second pass over the same K steps, against HBM
                (its algorithmic bytes per launch: each tensor region of its
                interface once; its flops per byte sit far below the MFMA ridge,
                and the MFMA rate is reported beside it), with the HBM traffic
                the counters measured for it and the whole step's floor;
  cpu_baseline  the FP64 token-loop oracle (oracle/sd_oracle.py) forward+VJP on
                the host cores, on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import gc
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

B, T, H, R, V, CH = 4, 2048, 8, 128, 128, 64
PEAK_MFMA_BF16 = 2.5e15
PEAK_HBM = 8.0e12

# Algorithmic flops per (sequence, 64-token chunk) of each chunk kernel at
# r = V = 128: dense GEMM products 2*M*N*K, lower-triangular ones at half.
_G = 2 * 64 * 128 * 128      # (64 x 128) @ (128 x 128)
_T = 64 * 64 * 128           # triangular (64 x 64 x 128) product, halved
FLOPS_PER_CHUNK = {
    "k_prep_c": 3 * _T,                          # L, W, U
    "state_c_fwd": 2 * _G,                       # w = U - W X, X += K^T w
    "k_prep_s": 6 * _T + _G,                     # k.delta, apply, P, L, W, U; K X0^T
    "state_s_fwd": 3 * _G + _T,                  # w = U - W X, X += K^T w; o = Q X0 + P w
    "k_bprep_s": 2 * 64 ** 3 // 2 + 2 * _T * 2 // 2 + _T,  # N = P A, dU, Wk
    "state_s_bwd": 3 * _G,                       # dw, injection, lambda update
    "k_grad_s": 3 * _G + 6 * _T,                 # dw X0, dO X0, w lam; M1, M2, 2 apply, 2 apply_t
    "k_bprep_c": _T + 64 ** 3 + 2 * 2 * 64 * 64 * 128 // 2 + _T,
    "state_c_bwd": 3 * _G,
    "k_grad_c": 3 * _G + 7 * _T,
}


# Interface bytes per (sequence, 64-token chunk) of each kernel as built: every
# global tensor region it reads or writes, counted once (operator tensors and
# the workspace panels between kernels).  Units: a 2-byte token panel
# [64 x 128] (bf16 input / fp16 or bf16 workspace panel) 16 KiB; an FP32 token
# panel 32 KiB; a 2-byte chunk-state slot [128 x 128] 32 KiB; a 64 x 64 FP32
# block 16 KiB.  Reads + writes:
_H, _P, _S, _A = 16384, 32768, 32768, 16384
BYTES_PER_CHUNK = {
    "k_prep_c": (2 * _H + _P) + (_A + 2 * _H + _P),           # u,h,decay -> A,W,K (fp16),U
    "state_c_fwd": (2 * _H + _P) + (_S + _H),                # W,K,U -> slot, delta
    "k_prep_s": (7 * _H + _P + _S) + (3 * _H + _H + _A // 2 + _H + _A + _P + _H),
    # u,q,k,v,erase,write,delta,decay,C slot -> d,e,chi,K,P,Q,A,U,W
    "state_s_fwd": (3 * _H + _P + _A // 2) + (_S + 2 * _H),  # W,K,U,Q,P -> slot, w, out
    "k_bprep_s": (_A + _A // 2 + 3 * _H + _P + _H) + (_P + 4 * _H),
    # A,P,dO,K,e,decay,Q -> dU,Wk,Ant,At1,B1
    "state_s_bwd": (4 * _H + _P) + (_S + _H),                # Wk,Ant,At1,B1,dU -> slot, dw
    "state_c_bwd": (4 * _H + _P) + (_S + _H),
    "k_grad_s": (6 * _H + _P + 3 * _S) + (3 * _H + _P),      # dw,w,d,e,chi,dO,decay,X0,XC,lam -> de,dchi,dd,dg
    "k_src_bwd": (11 * _H) + (7 * _H),                       # 6 inputs,delta,de,dchi,dw,dd -> 4 grads,ddelta,du,dk
    "k_bprep_c": (_A + 5 * _H + _P) + (_P + 4 * _H + _A),    # A,u,k,K,dd,ddelta,decay -> dU,Wk,At1,B1,Ant,P'
    "k_grad_c": (6 * _H + _P + 3 * _S + _A + _P + 5 * _H) + (3 * _H + _P),
    # dw,delta,dd,u,k (raw, normalised in-kernel),d,decay,X0,XC,lam,P',dg,
    # tail: u,k,h and the partial du,dk (in the gradients) -> du,dk,dh,dg
}


# Algorithmic bytes per token-head of each kernel in the sense of the
# operator's own tensors (SURVEY-style accounting: the inputs it reads, the
# outputs and gradients it writes, each once; workspace panels between kernels
# are not algorithmic).  bf16 vector 2R = 256 B, fp32 log-decay / its gradient
# 4R = 512 B, gamma 4 B.  State kernels touch only the boundary states
# (64 KiB per sequence each), listed separately.
_VEC, _DEC, _GAM = 2 * R, 4 * R, 4
OP_BYTES_PER_TOKEN_HEAD = {
    "k_prep_c": 2 * _VEC + _DEC + _GAM,                    # u, h, log-decay, gamma
    "k_prep_s": 6 * _VEC + _DEC,                           # u, q, k, v, erase, write, log-decay
    "state_s_fwd": _VEC,                                   # out (plus the states below)
    "k_bprep_s": _VEC + _DEC,                              # dO, log-decay
    "k_grad_s": _VEC + 2 * _DEC,                           # dO, log-decay -> dlog_decay
    "k_src_bwd": 6 * _VEC + 4 * _VEC,                      # u, k, q, erase, v, write -> dq, derase, dv, dwrite
    "k_bprep_c": 2 * _VEC + _DEC + _GAM,                   # u, k, log-decay, gamma
    "k_grad_c": _DEC + _GAM + _DEC + 3 * _VEC + 3 * _VEC + _GAM,
    # log-decay, gamma, u, k, h -> dlog_decay (add), du, dk, dh, dgamma
}
STATE_BYTES_PER_SEQ = {"state_c_fwd": R * R * 4, "state_s_fwd": R * V * 4,  # C0 / S0 read
                       "state_c_bwd": R * R * 4, "state_s_bwd": R * V * 4}  # dC0 / dS0 write

PROFILE_DIR = os.path.join(ROOT, "profiles")
TRAFFIC_FILE = os.path.join(PROFILE_DIR, "fwd_bwd_B4_T2048_H8_d128_hbm_traffic.txt")
COUNTER_FILE = os.path.join(PROFILE_DIR, "fwd_bwd_B4_T2048_H8_d128_mfma_valu_counters.txt")


def profile_keys(path, key):
    """Machine-readable lines `<key> <kernel> <value>` of a committed rocprofv3
    summary (the counter runs of the current build that the file's header
    names); {} if the file is absent."""
    out = {}
    try:
        with open(path) as fh:
            for line in fh:
                parts = line.split()
                if len(parts) == 3 and parts[0] == key:
                    out[parts[1]] = float(parts[2])
    except OSError:
        pass
    return out


_NTH = B * T * H
STEP_FLOOR_BYTES = (_NTH * 2564 + B * H * 4 * R * R * 4          # forward
                    + _NTH * (7 * 2 * R + 4 * R + 4 + 2 * V)     # backward: inputs, dO
                    + _NTH * (7 * 2 * R + 4 * R + 4)             # backward: cotangents
                    + B * H * 4 * R * R * 4)                     # dC_T, dS_T, dC0, dS0


def make_inputs(device, seed=0, b=B, t=T):
    import torch.nn.functional as F
    g = torch.Generator().manual_seed(seed)
    n = lambda *s: torch.randn(*s, generator=g)
    bf = lambda x: x.to(torch.bfloat16).to(device).requires_grad_()
    u, h = bf(n(b, t, H, R)), bf(n(b, t, H, R))
    q = bf(F.normalize(n(b, t, H, R), dim=-1))
    k = bf(F.normalize(n(b, t, H, 1, R), dim=-1))
    v = bf(n(b, t, H, 1, V))
    gd = (-F.softplus(n(b, t, H, R))).to(device).requires_grad_()
    er, wr = bf(n(b, t, H, 1, R)), bf(n(b, t, H, 1, V))
    gm = torch.full((b, t, H), 0.9, device=device).requires_grad_()
    C0 = (0.02 * n(b, H, R, R)).to(device).requires_grad_()
    S0 = (0.02 * n(b, H, R, V)).to(device).requires_grad_()
    dO = n(b, t, H, V).to(torch.bfloat16).to(device)
    return [u, h, q, k, v, gd, er, wr, gm], (C0, S0), dO


def cpu_baseline(budget_s=24.0):
    """FP64 oracle forward + autograd VJP on the host, bounded sample: all 32
    (b,h) sequences, T tokens with T doubled (up to the full T) while the next
    pass is predicted to stay under budget_s."""
    from oracle.sd_oracle import OracleState, solvedelta_oracle_raw
    threads = min(16, os.cpu_count() or 1)
    torch.set_num_threads(threads)

    def run(tt):
        ins, st, dO = make_inputs("cpu", seed=1, t=tt)
        ins = [x.detach().double().requires_grad_() for x in ins]
        st = [x.detach().double().requires_grad_() for x in st]
        t0 = time.perf_counter()
        o, _ = solvedelta_oracle_raw(*ins, initial_state=OracleState(*st))
        torch.autograd.grad(o, ins + st, dO.double())
        return time.perf_counter() - t0

    # the next doubling is predicted from the last one's growth (autograd over a
    # token loop grows faster than linearly in T at the larger samples)
    tt, dt, grow = 64, run(64), 2.2
    while dt * grow < budget_s and tt < T:
        tt *= 2
        prev, dt = dt, run(tt)
        grow = max(2.2, dt / prev)
    return {"value": B * tt / dt, "unit": "tokens/s", "cores": threads, "kind": "port",
            "cpu": cpu_model(),
            "sample": f"FP64 torch token-loop oracle F+VJP, B={B} H={H} r=V={R}, T={tt} "
                      f"({dt:.1f} s)"}


def cpu_model() -> str:
    """The host CPU as lscpu names it (model name, family / model / stepping,
    sockets x cores x threads), falling back to /proc/cpuinfo."""
    import subprocess
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        f = {}
        for line in out.splitlines():
            k, _, v = line.partition(":")
            f.setdefault(k.strip(), v.strip())
        if f.get("Model name"):
            return (f"{f['Model name']} (family {f.get('CPU family', '?')} model "
                    f"{f.get('Model', '?')} stepping {f.get('Stepping', '?')}; "
                    f"{f.get('Socket(s)', '?')} socket(s) x {f.get('Core(s) per socket', '?')} "
                    f"cores x {f.get('Thread(s) per core', '?')} threads; "
                    f"{f.get('CPU(s)', '?')} CPUs listed)")
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_forward_baseline():
    """The C token loop (oracle/sd_token_loop.c, FP32, OpenMP over the 32 (b,h)
    sequences) on config 1's full forward: the reference's CPU recurrence
    (reference.py:156-227) as a compiled loop, timed on the host cores."""
    import ctypes
    import numpy as np
    so = os.path.join(ROOT, "oracle", "libsd_token_loop.so")
    if not os.path.exists(so):
        return None
    lib = ctypes.CDLL(so)
    ins, st, _ = make_inputs("cpu", seed=2)
    arr = lambda x: np.ascontiguousarray(x.detach().float().numpy().reshape(B, T, H, -1))
    a = [arr(x) for x in ins[:8]] + [np.ascontiguousarray(ins[8].detach().float().numpy())]
    C = np.ascontiguousarray(st[0].detach().numpy())
    S = np.ascontiguousarray(st[1].detach().numpy())
    o = np.zeros((B, T, H, V), np.float32)
    ptr = lambda z: z.ctypes.data_as(ctypes.c_void_p)
    t0 = time.perf_counter()
    rc = lib.sd_cpu_forward_f32(B, T, H, R, V, *(ptr(z) for z in a), ptr(C), ptr(S), ptr(o))
    dt = time.perf_counter() - t0
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {"value": round(B * T / dt, 1), "unit": "tokens/s", "cores": threads,
            "kind": "port", "ok": rc == 0, "cpu": cpu_model(),
            "sample": f"C FP32 token loop forward, full config 1 (B={B} T={T} H={H} r=V={R}), "
                      f"{dt:.2f} s"}


def forward_bench(ins, st, steps, warmup):
    """Config 1: the same layer forward only (no autograd), same inputs."""
    from solvedelta_amd import solvedelta_native
    with torch.no_grad():
        for _ in range(warmup):
            solvedelta_native(*ins, initial_state=st, return_final_state=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            solvedelta_native(*ins, initial_state=st, return_final_state=True)
        torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    return {"workload": "layer forward, B=4 T=2048 H=8 r=V=128, final states returned",
            "value": round(B * T / dt, 1), "unit": "tokens/s", "ms_per_step": round(dt * 1e3, 4)}


def variant_bench(dev, steps, warmup, *, r=R, v=V, masked=False):
    """F+B at the headline's B, T, H on a variant of the path: key / value widths
    above 128 (the wide-width kernels), or the masked operator with 10 % invalid
    tokens and 1 % resets on the dense batch.  Reported beside the headline."""
    import torch.nn.functional as F
    from solvedelta_amd import solvedelta_masked_native, solvedelta_native
    g = torch.Generator().manual_seed(7)
    n = lambda *sh: torch.randn(*sh, generator=g)
    bf = lambda x: x.to(torch.bfloat16).to(dev).requires_grad_()
    ins = [bf(n(B, T, H, r)), bf(n(B, T, H, r)), bf(F.normalize(n(B, T, H, r), dim=-1)),
           bf(F.normalize(n(B, T, H, 1, r), dim=-1)), bf(n(B, T, H, 1, v)),
           (-F.softplus(n(B, T, H, r))).to(dev).requires_grad_(), bf(n(B, T, H, 1, r)),
           bf(n(B, T, H, 1, v)), torch.full((B, T, H), 0.9, device=dev).requires_grad_()]
    dO = n(B, T, H, v).to(torch.bfloat16).to(dev)
    valid = (torch.rand(B, T, generator=g) > 0.1).to(dev)
    reset = (torch.rand(B, T, generator=g) < 0.01).to(dev)

    def step():
        if masked:
            out, _ = solvedelta_masked_native(*ins, valid, reset)
        else:
            out, _ = solvedelta_native(*ins)
        return torch.autograd.grad(out, ins, dO)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    what = ("masked operator, 10 % invalid tokens and 1 % resets" if masked
            else f"wide-width kernels, r={r} V={v}")
    res = {"workload": f"operator forward + full VJP, B={B} T={T} H={H}, {what}",
           "value": round(B * T / dt, 1), "unit": "tokens/s", "ms_per_step": round(dt * 1e3, 4)}
    if not masked and r <= R < v:
        # both routes for these widths, whichever the operator dispatches to:
        # value groups of the main kernels, and one call of the wide-width kernels
        from solvedelta_amd.operator import _SolveDeltaFn, _value_groups, value_route
        routes = {
            "value_groups_ms": lambda: _value_groups(*ins, None, None, False, R)[0],
            "one_wide_call_ms": lambda: _SolveDeltaFn.apply(*ins, None, None, False, None)[0],
        }
        for name, fwd in routes.items():
            fn = lambda: torch.autograd.grad(fwd(), ins, dO)
            for _ in range(warmup):
                fn()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                fn()
            torch.cuda.synchronize()
            res[name] = round((time.perf_counter() - t0) / steps * 1e3, 4)
        res["route"] = value_route(r, v)
    return res


def graph_time(fn, steps, warmup):
    """Captures fn (a forward + autograd.grad step on static inputs) once as a
    HIP graph on a side stream, after eager warm-up there, and returns the
    replay time per step (the reference's timing mode, docs/RESULTS.md:9-12)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        graph.replay()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    del graph
    return dt


def refshape_bench(dev, steps, warmup):
    """Forward + full VJP at the shape the reference's own README quotes its core
    F+B timing on (B=1 T=1024 H=8 r=V=128; 0.905 ms on an RTX 5070 Ti, reference
    README.md:270): a like-for-like point beside the headline, not the metric."""
    from solvedelta_amd import solvedelta_native
    ins, st, dO = make_inputs(dev, seed=5, b=1, t=1024)
    leaves = ins + list(st)

    def step():
        out, _ = solvedelta_native(*ins, initial_state=st, return_final_state=False)
        return torch.autograd.grad(out, leaves, dO)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    # memory one F+B step allocates on top of its resident inputs (workspaces,
    # output, the 11 gradients), against the reference's graph pool at this shape
    base = torch.cuda.memory_allocated(dev)
    torch.cuda.reset_peak_memory_stats(dev)
    grads = step()
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated(dev) - base
    del grads
    dt_graph = graph_time(step, 200, 10)
    return {"workload": "operator forward + full VJP, B=1 T=1024 H=8 r=V=128",
            "value": round(1024 / dt, 1), "unit": "tokens/s", "ms_per_step": round(dt * 1e3, 4),
            "graph_ms_per_step": round(dt_graph * 1e3, 4),
            "reference_published_ms": 0.905, "reference_hardware": "RTX 5070 Ti",
            "step_alloc_mib": round(peak / 2 ** 20, 1),
            "reference_graph_alloc_mib": 63.0}


def mixer_bench(dev, steps=20, warmup=5):
    """The projected mixer (in-projection, conv4 + SiLU, KDA decay gate, the
    operator, gated RMSNorm, out-projection) forward + backward at the shape the
    reference quotes it on (docs/RESULTS.md:9-18: B=1 T=1024 H=8 r=V=128, hidden
    1024, 8.99 M parameters; 1.760 ms F+B as a CUDA-graph replay on an RTX 5070 Ti,
    208.1 MiB graph allocation).  FP32 master parameters under bf16 autocast,
    hidden states ~ N(0,1) bf16, output cotangent ~ N(0,1); gradients of the input
    and every parameter.  Timed eagerly and as a HIP-graph replay."""
    from solvedelta_amd.mixer import SolveDelta, SolveDeltaMixerConfig
    torch.manual_seed(0)
    cfg = SolveDeltaMixerConfig(hidden_size=1024, num_heads=8, head_k_dim=128, head_v_dim=128)
    mixer = SolveDelta(cfg).to(dev).train()
    g = torch.Generator().manual_seed(11)
    x = torch.randn(1, 1024, 1024, generator=g).to(torch.bfloat16).to(dev).requires_grad_()
    dy = torch.randn(1, 1024, 1024, generator=g).to(torch.bfloat16).to(dev)
    leaves = [x] + list(mixer.parameters())

    def step():
        with torch.autocast("cuda", dtype=torch.bfloat16, cache_enabled=False):
            y = mixer(x)
        return torch.autograd.grad(y, leaves, dy)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    base = torch.cuda.memory_allocated(dev)
    torch.cuda.reset_peak_memory_stats(dev)
    grads = step()
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated(dev) - base
    del grads
    dt_graph = graph_time(step, 100, 5)
    return {"workload": "projected mixer forward + backward, B=1 T=1024 hidden 1024 H=8 "
                        "r=V=128, FP32 parameters + bf16 autocast",
            "params": sum(p.numel() for p in mixer.parameters()),
            "value": round(1024 / dt_graph, 1), "unit": "tokens/s",
            "graph_ms_per_step": round(dt_graph * 1e3, 4),
            "eager_ms_per_step": round(dt * 1e3, 4),
            "step_alloc_mib": round(peak / 2 ** 20, 1),
            "reference_published_ms": 1.760, "reference_hardware": "RTX 5070 Ti",
            "reference_graph_alloc_mib": 208.1}


def decode_bench(dev, steps=256, streams=64):
    """Config 3: 64 independent streams x H=8, r=V=128, FP32 states C,S ~ 0.01 N(0,1)
    advanced in place by `steps` T=1 calls of the C-ABI (inputs drawn as config 1).
    With 512 streams the 512 MiB state pool exceeds the 256 MB last-level cache, so
    that run shows the rate without cache residency."""
    import ctypes
    from solvedelta_amd import _lib
    lib = _lib.load()
    ins, _, _ = make_inputs(dev, seed=3, b=streams, t=steps)
    ins = [x.detach() for x in ins]
    g = torch.Generator().manual_seed(4)
    C = (0.01 * torch.randn(streams, H, R, R, generator=g)).to(dev)
    S = (0.01 * torch.randn(streams, H, R, V, generator=g)).to(dev)
    out = torch.empty(streams, 1, H, V, dtype=torch.bfloat16, device=dev)
    from solvedelta_amd.operator import _inputs
    calls = []
    for t in range(steps):
        step = [x[:, t:t + 1] for x in ins]
        calls.append(_inputs(*step, C, S))
    stream = torch.cuda.current_stream(dev).cuda_stream

    def run():
        for c in calls:
            rc = lib.sd_decode(ctypes.byref(c), out.data_ptr(), C.data_ptr(), S.data_ptr(), stream)
            if rc:
                raise RuntimeError(f"sd_decode failed ({rc})")

    run()
    torch.cuda.synchronize()
    _lib.profile_enable(True)
    t0 = time.perf_counter()
    run()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    prof = _lib.profile_read()
    _lib.profile_enable(False)
    ms, cnt = prof["k_decode"]
    per_step = ms / cnt / 1e3
    state_bytes = 2 * streams * H * (R * R + R * V) * 4      # read + write C and S
    in_bytes = streams * H * (7 * R * 2 + R * 4 + 4 + V * 2)  # bf16 vectors, fp32 decay, gamma, out
    gbs = (state_bytes + in_bytes) / per_step / 1e9
    return {"workload": f"decode {streams} streams x H={H} r=V={R}, {steps} T=1 steps, state in place",
            "value": round(streams * steps / dt, 1), "unit": "tokens/s",
            "kernel_us": round(per_step * 1e6, 2),
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM / 1e9,
                         "unit": "GB/s", "frac": round(gbs * 1e9 / PEAK_HBM, 4),
                         "bytes_per_launch": state_bytes + in_bytes,
                         "note": (f"the {state_bytes // 2 >> 20} MiB of state "
                                  + ("fits" if state_bytes // 2 < 256e6 else "exceeds")
                                  + " the 256 MB last-level cache")}}


def lm_bench(dev, steps=5, warmup=2, graph=False):
    """Config 4: SolveDelta causal LM forward + backward, hidden 1024, 24 layers,
    H=8, r=V=128, vocab 32000, conv4, FP32 master weights under bf16 autocast,
    B=2, T=1024 uniform-random token ids with labels = inputs; eager steps and
    the HIP-graph captured step (optimizer outside, as in the reference)."""
    from solvedelta_amd.graph import SolveDeltaGraphedTrainingStep
    from solvedelta_amd.lm import SolveDeltaForCausalLM, SolveDeltaLMConfig
    torch.manual_seed(0)
    cfg = SolveDeltaLMConfig(hidden_size=1024, num_heads=8, head_k_dim=128, head_v_dim=128,
                             num_hidden_layers=24, vocab_size=32000)
    model = SolveDeltaForCausalLM(cfg).to(dev).train()
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, 32000, (2, 1024), generator=g).to(dev)

    def eager():
        # a fresh step's gradients (as after an optimizer's zero_grad), not an
        # accumulation onto the previous step's
        model.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.bfloat16, cache_enabled=False):
            loss, _, _ = model(ids, labels=ids)
        loss.backward()

    def timed(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / steps

    t_eager = timed(eager)
    ntok = 2 * 1024
    res = {"workload": "causal LM F+B, hidden 1024 x 24 layers, H=8 r=V=128, vocab 32000, "
                       "B=2 T=1024, FP32 master weights + bf16 autocast",
           "params": sum(p.numel() for p in model.parameters()),
           "eager_ms_per_step": round(t_eager * 1e3, 3),
           "value": round(ntok / t_eager, 1), "unit": "tokens/s", "mode": "eager"}
    if graph:
        # eager() released its loss, so no autograd graph holds the parameters'
        # AccumulateGrad nodes when the capture starts
        print(json.dumps(res), flush=True)      # the eager figures, should capture fail
        model.zero_grad(set_to_none=True)
        step = SolveDeltaGraphedTrainingStep(model, ids, ids)

        def graphed():
            model.zero_grad(set_to_none=True)
            step(ids, ids).backward()

        t_graph = timed(graphed)
        res["graph_ms_per_step"] = round(t_graph * 1e3, 3)
        res.update(value=round(ntok / t_graph, 1), mode="hip_graph")
    return res


def lm_bench_child(timeout_s=600):
    """Runs the config-4 section in a child process (python bench.py --lm-only)
    and returns the last JSON line it printed, so that a failure there leaves
    the rest of this run's line intact; the error is reported in its place."""
    import subprocess
    cmd = [sys.executable, os.path.abspath(__file__), "--lm-only"]
    try:
        res = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout_s)
    except subprocess.TimeoutExpired:
        return {"error": f"causal LM section exceeded {timeout_s} s"}
    lines = [ln for ln in res.stdout.splitlines() if ln.startswith("{")]
    out = json.loads(lines[-1]) if lines else {}
    if res.returncode != 0:
        out["error"] = f"causal LM section exited with status {res.returncode}"
        out["stderr_tail"] = res.stderr[-800:]
    return out


def copy_calibration(dev, nbytes=1 << 30):
    """A plain device copy of `nbytes` (read nbytes, write nbytes), launched a few
    times: the FETCH_SIZE / WRITE_SIZE counters of these launches give the
    factor that turns the counters of the operator's kernels into bytes."""
    src = torch.empty(nbytes // 4, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": nbytes, "launches": 3}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-lm", action="store_true")
    ap.add_argument("--no-lm-graph", action="store_true",
                    help="time the causal LM step eagerly only (no HIP-graph capture)")
    ap.add_argument("--lm-only", action="store_true",
                    help="only the causal LM section (run as a child of the full bench)")
    ap.add_argument("--step-only", action="store_true",
                    help="only the headline forward+VJP steps (counter runs)")
    ap.add_argument("--variant", choices=["wide", "masked", "mixer", "wide_v"],
                    help="only that variant's F+B line (its kernel profiles)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 1 GiB device copy (HBM counter calibration)")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the per-(batch, head) recurrence shards over GPUs with no exchange)",
              file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    if a.copy_calibration:
        copy_calibration(dev)
        return
    if a.lm_only:
        print(json.dumps(lm_bench(dev, graph=not a.no_lm_graph)), flush=True)
        return
    if a.variant == "mixer":
        print(json.dumps({"mixer": mixer_bench(dev, a.steps, a.warmup)}), flush=True)
        return
    if a.variant:
        kw = {"wide": dict(r=256, v=256), "wide_v": dict(r=128, v=256),
              "masked": dict(masked=True)}[a.variant]
        print(json.dumps({a.variant: variant_bench(dev, a.steps, a.warmup, **kw)}), flush=True)
        return
    from solvedelta_amd import _lib, solvedelta_native
    ins, st, dO = make_inputs(dev)
    leaves = ins + list(st)

    def step():
        out, _ = solvedelta_native(*ins, initial_state=st, return_final_state=False)
        return torch.autograd.grad(out, leaves, dO)

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(a.steps):
        step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / a.steps

    # second pass: per-kernel HIP-event timing on the launch stream
    _lib.profile_enable(True)
    for _ in range(a.steps):
        step()
    torch.cuda.synchronize()
    prof = _lib.profile_read()
    _lib.profile_enable(False)
    nchunks = B * H * (T // CH)
    nth = B * T * H
    us = {k: v[0] / v[1] * 1e3 for k, v in prof.items()}
    dom = max(prof, key=lambda k: prof[k][0])
    avg_s = us[dom] / 1e6
    op_bytes = (OP_BYTES_PER_TOKEN_HEAD.get(dom, 0) * nth +
                STATE_BYTES_PER_SEQ.get(dom, 0) * B * H)
    flops = FLOPS_PER_CHUNK.get(dom, 0) * nchunks
    traffic = profile_keys(TRAFFIC_FILE, "traffic_bytes")
    mfma_busy = profile_keys(COUNTER_FILE, "mfma_busy")
    gbs = op_bytes / avg_s / 1e9
    # every kernel's flops per algorithmic byte is far below the MFMA/HBM ridge
    # (2.5e15 / 8e12 = 312 flop/B), so HBM is the roof that bounds it
    roof = {"kernel": dom, "bound": "hbm", "achieved": round(gbs, 1),
            "peak": PEAK_HBM / 1e9, "unit": "GB/s", "frac": round(gbs * 1e9 / PEAK_HBM, 4),
            "traffic": traffic.get(dom),
            "traffic_unit": "HBM bytes per launch (FETCH_SIZE/WRITE_SIZE counter runs, "
                            "profiles/fwd_bwd_B4_T2048_H8_d128_hbm_traffic.txt)",
            "algorithmic_bytes": op_bytes,
            "avg_us": round(avg_s * 1e6, 2),
            # the kernel's whole interface (operator tensors plus the workspace
            # panels it reads and writes), each once: what it must move as built
            "interface_bytes": BYTES_PER_CHUNK[dom] * nchunks if dom in BYTES_PER_CHUNK else None,
            "interface_GBs": (round(BYTES_PER_CHUNK[dom] * nchunks / avg_s / 1e9, 1)
                              if dom in BYTES_PER_CHUNK else None),
            "mfma_tflops": round(flops / avg_s / 1e12, 3),
            "mfma_frac": round(flops / avg_s / PEAK_MFMA_BF16, 5),
            "kernels_us": {k: round(v, 2) for k, v in sorted(us.items())},
            "kernels_mfma_busy": mfma_busy or None,
            "kernels_traffic": traffic or None,
            # each kernel's counter-measured HBM bytes over its event-timed duration
            # (the state passes' and per-token closures' bandwidth against 8 TB/s)
            "kernels_traffic_GBs": ({k: round(traffic[k] / (us[k] * 1e-6) / 1e9, 1)
                                     for k in sorted(us) if k in traffic} if traffic else None)}
    # every kernel runs once per step; the counter summary lists each by its event name
    step_bytes = sum(traffic.get(k, 0.0) for k in us) if traffic else None
    step = {"algorithmic_bytes": STEP_FLOOR_BYTES,
            "floor_us": round(STEP_FLOOR_BYTES / PEAK_HBM * 1e6, 1),
            "achieved_GBs": round(STEP_FLOOR_BYTES / dt / 1e9, 1),
            "frac": round(STEP_FLOOR_BYTES / PEAK_HBM / dt, 4),
            "traffic_bytes": step_bytes}
    res = {
        "metric": "SolveDelta layer fwd+bwd tokens/s @B4 T2048 H8 d128; % MFMA/HBM roofline",
        "value": round(B * T / dt, 1), "unit": "tokens/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(dt * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "SolveDelta core operator forward + full VJP (configs[2] timed "
                               "at configs[1] shape)", "global_batch": B, "seq_len": T,
                   "heads": H, "dk": R, "dv": V, "chunk": CH, "parallelism": "single-gpu"},
        "roofline": roof,
        "step_roofline": step,
    }
    if a.step_only:
        print(json.dumps(res), flush=True)
        return
    # each section starts from a collected heap: cyclic garbage left by the
    # previous sections (and the device memory it holds) otherwise slows the
    # launch-bound config-4 step by a third
    gc.collect()
    res["forward"] = forward_bench(ins, st, a.steps, a.warmup)
    gc.collect()
    res["reference_shape"] = refshape_bench(dev, a.steps, a.warmup)
    gc.collect()
    res["wide"] = variant_bench(dev, 5, 2, r=256, v=256)
    gc.collect()
    res["wide_v"] = variant_bench(dev, 5, 2, r=128, v=256)
    gc.collect()
    res["masked"] = variant_bench(dev, 10, 3, masked=True)
    gc.collect()
    res["mixer"] = mixer_bench(dev)
    if not a.no_decode:
        gc.collect()
        res["decode"] = decode_bench(dev)
        res["decode_uncached"] = decode_bench(dev, steps=32, streams=512)
    if not a.no_cpu:
        res["cpu_baseline"] = cpu_baseline()
        res["cpu_baseline_forward"] = cpu_forward_baseline()
    if not a.no_lm:
        # last: the child runs on the GPU after everything else here has finished
        gc.collect()
        torch.cuda.empty_cache()
        if a.no_lm_graph:
            res["causal_lm"] = lm_bench(dev, graph=False)
        else:
            res["causal_lm"] = lm_bench_child()
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
