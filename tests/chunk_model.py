"""FP64 model of the HIP kernels' chunked algorithm (test helper).

It states, in plain torch, exactly what the chunk kernels compute -- chunk 64,
16-token blocks, block-centred exponent factorisation with an exact fix-up for
coordinates whose in-block decay exceeds TAU, the (I+L)^-1 WY form, the
sequential state passes and the closed-form chunk VJP -- so the algebra can be
checked against the token-loop oracle on the CPU before any kernel runs.

Generic op (one (b,h) sequence), state X [r x V], per token i:
    w_i = v_i - X_{i-1}^T x_i^erase        (erase read before this token's decay;
                                            x~ = x e^{G_{i-1}} ('excl') or the
                                            S-memory form x e^{G_i} ('incl'))
    X_i = D_i X_{i-1} + k_i w_i^T
    o_i = X_i^T q_i ('col')   or   X_i q_i ('row')
The C predictor is (excl,row) with X = C^T, k = u, x = gamma u, v = gamma h,
q = key; the S memory is (incl,col) with k = d, x = e, v = z, q = chi.
"""
from __future__ import annotations

import torch

BT = 64
BS = 16
TAU = 60.0
RHO = 5.0 / 8.0


def block_refs(G):
    """R_J = G at the row before block J (0 for the first block); G [BT, r]."""
    R = torch.zeros(BT // BS, G.shape[1], dtype=G.dtype)
    for J in range(1, BT // BS):
        R[J] = G[J * BS - 1]
    return R


def gram(Xm, Ym, Gx, G, strict):
    """M_ij = sum_c X_ic Y_jc exp(Gx_ic - G_jc) for j < i (strict) or j <= i."""
    R = block_refs(G)
    M = torch.zeros(BT, BT, dtype=Xm.dtype)
    for J in range(BT // BS):
        js = slice(J * BS, (J + 1) * BS)
        drop = R[J] - G[J * BS + BS - 1]
        wild = drop > TAU
        Yh = Ym[js] * torch.exp(R[J] - G[js])
        Yh[:, wild] = 0
        for I in range(J, BT // BS):
            is_ = slice(I * BS, (I + 1) * BS)
            Xt = Xm[is_] * torch.exp(Gx[is_] - R[J])
            M[is_, js] = Xt @ Yh.T
            if wild.any():
                c = wild.nonzero()[:, 0]
                M[is_, js] += torch.einsum("ic,jc,ijc->ij", Xm[is_][:, c], Ym[js][:, c],
                                           torch.exp((Gx[is_][:, None, c] - G[js][None, :, c]).clamp(max=0)))
    mask = torch.tril(torch.ones(BT, BT, dtype=torch.bool), -1 if strict else 0)
    return torch.where(mask, M, torch.zeros_like(M))


def apply(M, Ym, Gx, G):
    """R_ic = sum_j M_ij Y_jc exp(Gx_ic - G_jc), M lower-triangular."""
    R = block_refs(G)
    out = torch.zeros(BT, Ym.shape[1], dtype=Ym.dtype)
    for J in range(BT // BS):
        js = slice(J * BS, (J + 1) * BS)
        wild = (R[J] - G[J * BS + BS - 1]) > TAU
        Yh = Ym[js] * torch.exp(R[J] - G[js])
        Yh[:, wild] = 0
        rows = slice(J * BS, BT)
        out[rows] += torch.exp(Gx[rows] - R[J]) * (M[rows, js] @ Yh)
        if wild.any():
            c = wild.nonzero()[:, 0]
            ex = torch.exp((Gx[rows][:, None, c] - G[js][None, :, c]).clamp(max=0))
            corr = torch.zeros_like(out[rows])
            corr[:, c] = torch.einsum("ij,jc,ijc->ic", M[rows, js], Ym[js][:, c], ex)
            out[rows] += corr
    return out


def apply_t(M, Xm, Gx, G):
    """R_jc = sum_i M_ij X_ic exp(Gx_ic - G_jc), M lower-triangular."""
    R = block_refs(G)
    out = torch.zeros(BT, Xm.shape[1], dtype=Xm.dtype)
    for J in range(BT // BS):
        js = slice(J * BS, (J + 1) * BS)
        wild = (R[J] - G[J * BS + BS - 1]) > TAU
        rows = slice(J * BS, BT)
        Xt = Xm[rows] * torch.exp(Gx[rows] - R[J])
        f = torch.exp(R[J] - G[js])
        f[:, wild] = 0
        out[js] += f * (M[rows, js].T @ Xt)
        if wild.any():
            c = wild.nonzero()[:, 0]
            ex = torch.exp((Gx[rows][:, None, c] - G[js][None, :, c]).clamp(max=0))
            corr = torch.zeros_like(out[js])
            corr[:, c] = torch.einsum("ij,ic,ijc->jc", M[rows, js], Xm[rows][:, c], ex)
            out[js] += corr
    return out


def tri_inverse(L):
    return torch.linalg.inv(torch.eye(BT, dtype=L.dtype) + L)


def chunk_cumsum(g):
    return torch.cumsum(g, 0)


class Op:
    """Generic chunked op for one sequence; all chunk quantities kept for the VJP."""

    def __init__(self, k, x, v, g, q, X0, erase_mode, out_mode):
        self.k, self.x, self.v, self.g, self.q = k, x, v, g, q
        self.em, self.om = erase_mode, out_mode
        T = k.shape[0]
        self.NT = T // BT
        self.X0s, self.ws, self.outs = [], [], []
        X = X0.clone()
        for n in range(self.NT):
            s = slice(n * BT, (n + 1) * BT)
            G = chunk_cumsum(g[s])
            Gx = G - g[s] if erase_mode == "excl" else G
            L = gram(x[s], k[s], Gx, G, strict=True)
            A = tri_inverse(L)
            xt = x[s] * torch.exp(Gx)
            W = A @ xt
            U = A @ v[s]
            Kh = k[s] * torch.exp(G[-1] - G)
            self.X0s.append(X.clone())
            w = U - W @ X
            if out_mode == "col":
                P = gram(q[s], k[s], G, G, strict=False)
                o = (q[s] * torch.exp(G)) @ X + P @ w
            else:
                M = torch.tril(q[s] @ w.T)
                o = torch.exp(G) * (q[s] @ X.T) + apply(M, k[s], G, G)
            X = torch.exp(G[-1])[:, None] * X + Kh.T @ w
            self.ws.append(w)
            self.outs.append(o)
        self.XT = X
        self.w = torch.cat(self.ws)
        self.o = torch.cat(self.outs)

    def backward(self, do, dW, dXT):
        """Returns dk, dx, dv, dg, dq, dX0 (dW may be None)."""
        k, x, v, g, q = self.k, self.x, self.v, self.g, self.q
        T = k.shape[0]
        dk, dx, dv, dg, dq = (torch.zeros_like(t) for t in (k, x, v, g, q))
        lam = dXT.clone()
        for n in reversed(range(self.NT)):
            s = slice(n * BT, (n + 1) * BT)
            G = chunk_cumsum(g[s])
            Gx = G - g[s] if self.em == "excl" else G
            L = gram(x[s], k[s], Gx, G, strict=True)
            A = tri_inverse(L)
            Kh = k[s] * torch.exp(G[-1] - G)
            xt = x[s] * torch.exp(Gx)
            X0, w = self.X0s[n], self.ws[n]
            dO = do[s]
            dWs = torch.zeros_like(w) if dW is None else dW[s]
            # reverse state step
            if self.om == "col":
                P = gram(q[s], k[s], G, G, strict=False)
                rhs = dWs + P.T @ dO
                inj = (q[s] * torch.exp(G)).T @ dO
            else:
                Pp = gram(dO, k[s], G, G, strict=False)
                rhs = dWs + Pp.T @ q[s]
                inj = (dO * torch.exp(G)).T @ q[s]
            lam_ext = lam
            dw = A.T @ (rhs + Kh @ lam_ext)
            lam = torch.exp(G[-1])[:, None] * lam_ext + inj - xt.T @ dw
            XC = torch.exp(G[-1])[:, None] * X0 + Kh.T @ w
            # chunk gradients
            M1 = torch.tril(dw @ w.T, -1)  # dw_i . w_j, j < i
            dxs = -(torch.exp(Gx) * (dw @ X0.T) + apply(M1, k[s], Gx, G))
            if self.om == "col":
                M2 = torch.tril(dO @ w.T)  # do_l . w_i, l >= i
                dks = torch.exp(G[-1] - G) * (w @ lam_ext.T) + apply_t(M2, q[s], G, G) - apply_t(M1, x[s], Gx, G)
                dqs = torch.exp(G) * (dO @ X0.T) + apply(M2, k[s], G, G)
                dG = q[s] * dqs - k[s] * dks
            else:
                M2 = torch.tril(q[s] @ w.T)  # q_l . w_i, l >= i
                dks = torch.exp(G[-1] - G) * (w @ lam_ext.T) + apply_t(M2, dO, G, G) - apply_t(M1, x[s], Gx, G)
                Pp = gram(dO, k[s], G, G, strict=False)
                dqs = (dO * torch.exp(G)) @ X0 + Pp @ w
                dG = self.outs[n] * dO - k[s] * dks
            xdx = x[s] * dxs
            if self.em == "excl":
                dG[:-1] += xdx[1:]
            else:
                dG += xdx
            dG[-1] += (XC * lam_ext).sum(1)
            dgs = torch.flip(torch.cumsum(torch.flip(dG, [0]), 0), [0])
            dk[s], dx[s], dv[s], dg[s], dq[s] = dks, dxs, dw, dgs, dqs
        return dk, dx, dv, dg, dq, lam


def l2n(x):
    rs = torch.rsqrt((x * x).sum(-1, keepdim=True) + 1e-24)
    return x * rs, rs


def l2n_bwd(y, rs, dy):
    return (dy - (dy * y).sum(-1, keepdim=True) * y) * rs


def sources(uh, delta, kh, qh, er, wr, v):
    usq = (uh * uh).sum(-1, keepdim=True)
    dsq = (delta * delta).sum(-1, keepdim=True)
    N = torch.sqrt(RHO * RHO + usq * dsq)
    phi = RHO / N * delta
    den = 1 + (phi * uh).sum(-1, keepdim=True)
    sig_e = torch.sigmoid(er)
    b = sig_e * kh
    ub = (uh * b).sum(-1, keepdim=True)
    uq = (uh * qh).sum(-1, keepdim=True)
    e = b - phi * (ub / den)
    chi = qh - phi * (uq / den)
    z = torch.sigmoid(wr) * v
    return e, chi, z


def sources_bwd(uh, delta, kh, qh, er, wr, v, de, dchi, dz):
    usq = (uh * uh).sum(-1, keepdim=True)
    dsq = (delta * delta).sum(-1, keepdim=True)
    N = torch.sqrt(RHO * RHO + usq * dsq)
    s = RHO / N
    phi = s * delta
    den = 1 + (phi * uh).sum(-1, keepdim=True)
    sig_e, sig_w = torch.sigmoid(er), torch.sigmoid(wr)
    b = sig_e * kh
    ub = (uh * b).sum(-1, keepdim=True)
    uq = (uh * qh).sum(-1, keepdim=True)
    sb, sq = ub / den, uq / den
    dv = sig_w * dz
    dwr = dz * v * sig_w * (1 - sig_w)
    db = de.clone()
    dphi = -sb * de - sq * dchi
    dsb = -(phi * de).sum(-1, keepdim=True)
    dsq_ = -(phi * dchi).sum(-1, keepdim=True)
    dub, duq = dsb / den, dsq_ / den
    dden = -(dsb * sb + dsq_ * sq) / den
    duh = dub * b + duq * qh + dden * phi
    db = db + dub * uh
    dqh = dchi + duq * uh
    dphi = dphi + dden * uh
    dkh = db * sig_e
    der = db * kh * sig_e * (1 - sig_e)
    ds = (dphi * delta).sum(-1, keepdim=True)
    ddelta = s * dphi
    dN = -RHO * ds / (N * N)
    dN2 = dN / (2 * N)
    duh = duh + 2 * dN2 * dsq * uh
    ddelta = ddelta + 2 * dN2 * usq * delta
    return duh, ddelta, dkh, dqh, der, dwr, dv


def forward_seq(u, h, q, k, v, g, er, wr, gam, C0, S0):
    """One (b,h) sequence, T a multiple of BT. Returns dict of all pieces."""
    uh, ru = l2n(u)
    kh, rk = l2n(k)
    qh, rq = l2n(q)
    opC = Op(uh, gam[:, None] * uh, gam[:, None] * h, g, kh, C0.T.clone(), "excl", "row")
    delta = opC.w
    d = kh + opC.o
    e, chi, z = sources(uh, delta, kh, qh, er, wr, v)
    opS = Op(d, e, z, g, chi, S0.clone(), "incl", "col")
    return dict(out=opS.o, C=opC.XT.T, S=opS.XT, opC=opC, opS=opS, uh=uh, ru=ru, kh=kh, rk=rk,
                qh=qh, rq=rq, delta=delta, d=d)


def backward_seq(fw, u, h, q, k, v, g, er, wr, gam, dout, dC, dS):
    opC, opS = fw["opC"], fw["opS"]
    uh, kh, qh, delta = fw["uh"], fw["kh"], fw["qh"], fw["delta"]
    dd, de, dz, dgS, dchi, dS0 = opS.backward(dout, None, dS)
    duh, ddelta, dkh, dqh, der, dwr, dv = sources_bwd(uh, delta, kh, qh, er, wr, v, de, dchi, dz)
    dkh = dkh + dd
    dk_c, dx_c, dv_c, dgC, dq_c, dX0 = opC.backward(dd, ddelta, dC.T.clone())
    duh = duh + dk_c + gam[:, None] * dx_c
    dgam = (uh * dx_c).sum(-1) + (h * dv_c).sum(-1)
    dh = gam[:, None] * dv_c
    dkh = dkh + dq_c
    du = l2n_bwd(uh, fw["ru"], duh)
    dk = l2n_bwd(kh, fw["rk"], dkh)
    dq = l2n_bwd(qh, fw["rq"], dqh)
    return du, dh, dq, dk, dv, dgS + dgC, der, dwr, dgam, dX0.T, dS0
