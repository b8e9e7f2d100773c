"""CPU oracle for the ALIF path — TEST INFRASTRUCTURE ONLY (see oracle/lif_oracle.py).

numpy fp32 restatement (own code) of the reference's adaptive-threshold LIF in
lifscan/triton_alif.py, with every `a*b + c` evaluated as two IEEE round-to-nearest
operations.  Step (triton_alif.py:26-31):
    v = beta*u + x;  s = v >= theta0 + w;  u' = s ? u_r : v;  w' = s ? rho*w + q : rho*w
Pins (tests/test_oracle_alif.py): exact rational recurrence with per-operation fp32 rounding,
dyadic exact cases, box-scan invariants (map evaluation == serial on in-box states, repair ==
serial), fp64 autograd for the adjoint.
"""
import math

import numpy as np

from oracle.lif_oracle import envelope_carry, envelope_chunks

f32 = np.float32
INF = f32(np.inf)


def _s(x):
    return f32(x)


def alif_step(u, w, x, beta, rho, q, theta0, u_r):
    """triton_alif.py:26-31."""
    b, r, qq, th, ur = _s(beta), _s(rho), _s(q), _s(theta0), _s(u_r)
    v = b * u + x
    s = v >= th + w
    u2 = np.where(s, ur, v).astype(f32)
    w2 = np.where(s, r * w + qq, r * w).astype(f32)
    return u2, w2, s


def serial_forward(I, beta, rho, q, theta0, u_r, u0, w0):
    """Serial ALIF (triton_alif.py:35-42, :46-71) -> (U, W, S)."""
    I = np.ascontiguousarray(I, dtype=f32)
    T, N = I.shape
    u = np.array(u0, dtype=f32).reshape(N).copy()
    w = np.array(w0, dtype=f32).reshape(N).copy()
    U = np.empty_like(I)
    W = np.empty_like(I)
    S = np.empty_like(I)
    for t in range(T):
        u, w, s = alif_step(u, w, I[t], beta, rho, q, theta0, u_r)
        U[t], W[t], S[t] = u, w, s
    return U, W, S


def serial_segment(I, beta, rho, q, theta0, u_r, u, w):
    u = np.array(u, dtype=f32).copy()
    w = np.array(w, dtype=f32).copy()
    for t in range(I.shape[0]):
        u, w, _ = alif_step(u, w, I[t], beta, rho, q, theta0, u_r)
    return u, w


def warm_predict(I, beta, rho, q, theta0, u_r, u0, w0, C, Wn=4, u_init=0.0, w_init=0.0,
                 UI=None, WI=None):
    """Predicted chunk-entry adaptation (triton_alif.py:75-92, :276-285): chunk m simulates
    chunks max(m-Wn, 0) .. m-1 from (u_init, w_init), from (UI, WI)[s0] when given, or from
    (u0, w0) when the warm-up reaches t = 0."""
    T, N = I.shape
    M = T // C
    WP = np.empty((M, N), f32)
    for m in range(M):
        s0 = max(m - Wn, 0)
        if s0 == 0:
            u, w = np.asarray(u0, f32), np.asarray(w0, f32)
        elif UI is not None:
            u, w = np.asarray(UI[s0], f32), np.asarray(WI[s0], f32)
        else:
            u, w = np.full(N, u_init, f32), np.full(N, w_init, f32)
        _, w = serial_segment(I[s0 * C:m * C], beta, rho, q, theta0, u_r, u, w)
        WP[m] = w
    return WP


def box_bounds(u0, w0, Wpred, dw, beta, rho, theta0, u_r, I, C):
    """Entry box of every chunk (triton_alif.py:310-318): lu from the hard-reset envelope,
    [lw, hw] = [max(Wp - dw, 0), Wp + dw] around the prediction (Wp[0] = w0),
    hu = max(theta0 + hw/rho, u_r) widened by 1e-5(|hu| + 1)."""
    EC, EA, EB = envelope_chunks(I, beta, u_r, C)
    Lu = envelope_carry(u0, EC, EA, EB)
    Wp = np.array(Wpred, dtype=f32).copy()
    Wp[0] = w0
    dw = _s(dw)
    Lw = np.maximum(Wp - dw, f32(0)).astype(f32)
    Hw = (Wp + dw).astype(f32)
    Hu = np.maximum(_s(theta0) + Hw / _s(rho), _s(u_r)).astype(f32)
    Hu = (Hu + f32(1e-5) * (np.abs(Hu) + f32(1.0))).astype(f32)
    return Lu, Hu, Lw, Hw


def build_maps(I, Lu, Hu, Lw, Hw, beta, rho, q, theta0, u_r, C, K1, K2, block=1):
    """Box-scan chunk maps (triton_alif.py:96-186): first-spike lines u0 >= ls*w0 + lc (K1)
    and post-spike x-pieces (K2) with constant final u and final w affine in x.  `block`
    neurons share the decision to split pieces in a step (the reference's Triton block BN:
    the split/compaction branch runs when any piece of any neuron of the block is cut)."""
    T, N = I.shape
    M = T // C
    b, r, qq, th, ur = _s(beta), _s(rho), _s(q), _s(theta0), _s(u_r)
    Ic = I.reshape(M, C, N)
    A = np.ones((M, N), f32)
    B = np.zeros((M, N), f32)
    R = np.ones((M, N), f32)
    wlo = Lw.astype(f32).copy()
    ls = np.zeros((M, K1, N), f32)
    lc = np.full((M, K1, N), INF, f32)
    lx = np.zeros((M, K1, N), f32)
    nl = np.zeros((M, N), np.int32)
    pown = np.full((M, K2, N), -1, np.int32)
    pxl = np.full((M, K2, N), INF, f32)
    pxr = np.full((M, K2, N), INF, f32)
    pu = np.zeros((M, K2, N), f32)
    pa = np.ones((M, K2, N), f32)
    pof = np.zeros((M, K2, N), f32)
    npc = np.zeros((M, N), np.int32)
    ovf = np.zeros((M, N), np.int32)
    k1 = np.arange(K1)[None, :, None]
    k2 = np.arange(K2)[None, :, None]
    nblk = -(-N // block)
    pad = nblk * block - N
    logk2 = int(math.log2(K2))

    def gather(a, idx):
        return np.take_along_axis(a, idx, axis=1)

    for j in range(C):
        x = Ic[:, j]
        valid = k2 < npc[:, None]
        v = b * pu + x[:, None]
        rr = (v - th) - pof
        es = valid & (rr > pa * pxl)
        en = valid & (rr < pa * pxr)
        cut = (es & en).any(1)
        cut = np.pad(cut, ((0, 0), (0, pad))).reshape(M, nblk, block).any(2)
        cut = np.repeat(cut, block, axis=1)[:, :N]
        if cut.any():
            with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
                z = (rr / pa).astype(f32)
            nout = es.astype(np.int32) + en.astype(np.int32)
            p = np.cumsum(nout, axis=1) - nout
            ntot = nout.sum(1)
            kk = np.broadcast_to(k2, (M, K2, N))
            lo_i = np.zeros((M, K2, N), np.int64)
            hi_i = np.full((M, K2, N), K2 - 1, np.int64)
            for _ in range(logk2):
                mid = (lo_i + hi_i + 1) // 2
                le = gather(p, mid) <= kk
                lo_i = np.where(le, mid, lo_i)
                hi_i = np.where(le, hi_i, mid - 1)
            idx = lo_i
            d = kk - gather(p, idx)
            is_s = (d == 0) & (gather(es, idx))
            g_xl, g_xr, g_z = gather(pxl, idx), gather(pxr, idx), gather(z, idx)
            g_v, g_pa, g_po, g_own = gather(v, idx), gather(pa, idx), gather(pof, idx), gather(pown, idx)
            n_new = np.minimum(ntot, K2)
            keep = k2 < n_new[:, None]
            c3 = cut[:, None, :]
            s_pxl = np.where(keep, np.where(is_s, g_xl, np.maximum(g_xl, g_z)), INF).astype(f32)
            s_pxr = np.where(keep, np.where(is_s, np.minimum(g_xr, g_z), g_xr), INF).astype(f32)
            s_pu = np.where(keep, np.where(is_s, ur, g_v), f32(0)).astype(f32)
            s_pa = np.where(keep, r * g_pa, f32(1)).astype(f32)
            s_pof = np.where(keep, np.where(is_s, r * g_po + qq, r * g_po), f32(0)).astype(f32)
            s_pown = np.where(keep, g_own, -1).astype(np.int32)
            u_pu = np.where(valid, np.where(es, ur, v), pu).astype(f32)
            u_pof = np.where(valid, np.where(es, r * pof + qq, r * pof), pof).astype(f32)
            u_pa = np.where(valid, r * pa, pa).astype(f32)
            ovf = np.where(cut & (ntot > K2), 1, ovf).astype(np.int32)
            pxl = np.where(c3, s_pxl, pxl)
            pxr = np.where(c3, s_pxr, pxr)
            pu = np.where(c3, s_pu, u_pu)
            pa = np.where(c3, s_pa, u_pa)
            pof = np.where(c3, s_pof, u_pof)
            pown = np.where(c3, s_pown, pown)
            npc = np.where(cut, n_new, npc).astype(np.int32)
        else:
            pu = np.where(valid, np.where(es, ur, v), pu).astype(f32)
            pof = np.where(valid, np.where(es, r * pof + qq, r * pof), pof).astype(f32)
            pa = np.where(valid, r * pa, pa).astype(f32)
        # first-spike line of step j
        A = b * A
        B = b * B + x
        with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
            sj = (R / A).astype(f32)
            cj = ((th - B) / A).astype(f32)
            whi = np.minimum(Hw, ((Hu - cj) / sj).astype(f32)).astype(f32)
        validl = k1 < nl[:, None]
        dom = (validl & (ls * wlo[:, None] + lc <= (sj * wlo + cj)[:, None])
               & (ls * whi[:, None] + lc <= (sj * whi + cj)[:, None])).any(1)
        newc = (wlo < whi) & ~dom
        cx = R * r
        put = newc[:, None] & (k1 == nl[:, None])
        ls = np.where(put, sj[:, None], ls)
        lc = np.where(put, cj[:, None], lc)
        lx = np.where(put, cx[:, None], lx)
        ovf = np.where(newc & (nl >= K1), 1, ovf).astype(np.int32)
        xlo = cx * wlo + qq
        xhi = cx * whi + qq
        pd = f32(4e-7) * (np.abs(xhi) + f32(1.0))
        putp = newc[:, None] & (k2 == npc[:, None])
        pxl = np.where(putp, (xlo - pd)[:, None], pxl)
        pxr = np.where(putp, (xhi + pd)[:, None], pxr)
        pu = np.where(putp, ur, pu).astype(f32)
        pa = np.where(putp, f32(1), pa).astype(f32)
        pof = np.where(putp, f32(0), pof).astype(f32)
        pown = np.where(putp, nl[:, None], pown)
        ovf = np.where(newc & (npc >= K2), 1, ovf).astype(np.int32)
        nl = np.where(newc, np.minimum(nl + 1, K1), nl).astype(np.int32)
        npc = np.where(newc, np.minimum(npc + 1, K2), npc).astype(np.int32)
        with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
            wlo = np.maximum(wlo, ((Lu - cj) / sj).astype(f32)).astype(f32)
        R = r * R
    return dict(A=A, B=B, ls=ls, lc=lc, lx=lx, nl=nl, pown=pown, pxl=pxl, pxr=pxr, pu=pu, pa=pa,
                pof=pof, npc=npc, ovf=ovf)


def carry(I, u0, w0, Lu, Hu, Lw, Hw, mp, beta, rho, q, theta0, u_r, C):
    """Verified carry (triton_alif.py:214-252): first firing line -> x = lx*w + q -> the
    unique piece of that line containing x; out of box, overflow or not exactly one piece ->
    the chunk is run serially.  Returns SU, SW, MISS."""
    M, K1, N = mp["ls"].shape
    K2 = mp["pxl"].shape[1]
    rhoC = _rho_pow(rho, C)
    u = np.asarray(u0, f32).copy()
    w = np.asarray(w0, f32).copy()
    SU = np.empty((M, N), f32)
    SW = np.empty((M, N), f32)
    MISS = np.empty((M, N), np.int32)
    k1 = np.arange(K1)[:, None]
    k2 = np.arange(K2)[:, None]
    for m in range(M):
        SU[m], SW[m] = u, w
        validl = k1 < mp["nl"][m][None]
        fire = validl & (u[None] >= mp["ls"][m] * w[None] + mp["lc"][m])
        first = np.where(fire, k1, K1).min(0)
        none_ = first == K1
        lxf = np.where(k1 == first[None], mp["lx"][m], f32(0)).sum(0, dtype=f32)
        xq = lxf * w + _s(q)
        validp = k2 < mp["npc"][m][None]
        hit = validp & (mp["pown"][m] == first[None]) & (mp["pxl"][m] <= xq[None]) & (xq[None] < mp["pxr"][m])
        nh = hit.sum(0)
        mu = np.where(hit, mp["pu"][m], f32(0)).sum(0, dtype=f32)
        mw = np.where(hit, mp["pa"][m] * xq[None] + mp["pof"][m], f32(0)).sum(0, dtype=f32)
        nu = np.where(none_, mp["A"][m] * u + mp["B"][m], mu).astype(f32)
        nw = np.where(none_, rhoC * w, mw).astype(f32)
        inbox = (u >= Lu[m]) & (u < Hu[m]) & (w >= Lw[m]) & (w <= Hw[m])
        bad = ~inbox | (mp["ovf"][m] > 0) | (~none_ & (nh != 1))
        MISS[m] = bad
        if bad.any():
            su, sw = serial_segment(I[m * C:(m + 1) * C], beta, rho, q, theta0, u_r, u, w)
            nu = np.where(bad, su, nu).astype(f32)
            nw = np.where(bad, sw, nw).astype(f32)
        u, w = nu, nw
    return SU, SW, MISS


def _rho_pow(rho, C):
    """rho^C as the reference computes it on the host: torch float32 pow (triton_alif.py:332)."""
    import torch
    return f32(float(torch.tensor(rho, dtype=torch.float32) ** C))


def replay(I, SU, SW, beta, rho, q, theta0, u_r, C):
    T, N = I.shape
    M = T // C
    Ic = I.reshape(M, C, N)
    u = SU.astype(f32).copy()
    w = SW.astype(f32).copy()
    U = np.empty((M, C, N), f32)
    W = np.empty((M, C, N), f32)
    S = np.empty((M, C, N), f32)
    for j in range(C):
        u, w, s = alif_step(u, w, Ic[:, j], beta, rho, q, theta0, u_r)
        U[:, j], W[:, j], S[:, j] = u, w, s
    return U.reshape(T, N), W.reshape(T, N), S.reshape(T, N), u, w


def scan_forward(I, beta, rho, q, theta0, u_r, u0, w0, Wpred, dw, C=128, K1=16, K2=32, block=1,
                 repair=0, stats=None, keep=None):
    """Box scan (triton_alif.py:301-358): box -> build -> verified carry -> replay -> repair."""
    I = np.ascontiguousarray(I, dtype=f32)
    T, N = I.shape
    u0 = np.asarray(u0, f32).reshape(N)
    w0 = np.asarray(w0, f32).reshape(N)
    Lu, Hu, Lw, Hw = box_bounds(u0, w0, Wpred, dw, beta, rho, theta0, u_r, I, C)
    mp = build_maps(I, Lu, Hu, Lw, Hw, beta, rho, q, theta0, u_r, C, K1, K2, block)
    SU, SW, MISS = carry(I, u0, w0, Lu, Hu, Lw, Hw, mp, beta, rho, q, theta0, u_r, C)
    U, W, S, EU, EW = replay(I, SU, SW, beta, rho, q, theta0, u_r, C)
    it = 0
    for it in range(1, repair + 1):
        nu_ = np.concatenate([u0[None], EU[:-1]], 0)
        nw_ = np.concatenate([w0[None], EW[:-1]], 0)
        if np.array_equal(nu_, SU) and np.array_equal(nw_, SW):
            it -= 1
            break
        SU, SW = nu_, nw_
        U, W, S, EU, EW = replay(I, SU, SW, beta, rho, q, theta0, u_r, C)
    if stats is not None:
        stats["repair_iters"] = it
        stats["miss_frac"] = float(MISS.astype(np.float64).mean())
        stats["overflow_frac"] = float(mp["ovf"].astype(np.float64).mean())
        stats["mean_lines"] = float(mp["nl"].astype(np.float64).mean())
        stats["mean_pieces"] = float(mp["npc"].astype(np.float64).mean())
        stats["max_pieces"] = int(mp["npc"].max())
    if keep is not None:
        keep.update(mp)
        keep.update(Lu=Lu, Hu=Hu, Lw=Lw, Hw=Hw, SU=SU, SW=SW, MISS=MISS)
    return U, W, S


# ----------------------------------------------------------------------------- backward
def surrogate(up, wp, x, beta, theta0, alpha, dtype=f32):
    """triton_alif.py:367-370: sg = alpha*sig*(1-sig), sig = sigmoid(alpha*(v - theta0 - w))."""
    dt = dtype
    v = dt(beta) * np.asarray(up, dt) + np.asarray(x, dt)
    sig = dt(1.0) / (dt(1.0) + np.exp(-(dt(alpha) * ((v - dt(theta0)) - np.asarray(wp, dt)))))
    return dt(alpha) * sig * (dt(1.0) - sig)


def backward(I, U, W, S, GS, beta, rho, q, theta0, u0, w0, alpha=4.0, dtype=f32):
    """Serial fused adjoint (triton_alif.py:444-487, PASS 4 of :374-440), reverse in t:
    d = g + q*lw; lv = (1-s)*beta*lv + sg*d; LW[t] = lw; LV[t] = lv; lw <- rho*lw - sg*d.
    Returns (LV, LW)."""
    dt = dtype
    T, N = I.shape
    Up = np.concatenate([np.asarray(u0, f32)[None], U[:-1]], 0)
    Wp = np.concatenate([np.asarray(w0, f32)[None], W[:-1]], 0)
    sg = surrogate(Up, Wp, I, beta, theta0, alpha, dt)
    b, r, qq = dt(beta), dt(rho), dt(q)
    lw = np.zeros(N, dt)
    lv = np.zeros(N, dt)
    LW = np.empty((T, N), dt)
    LV = np.empty((T, N), dt)
    GSd = np.asarray(GS, dt)
    Sd = np.asarray(S, dt)
    for t in range(T - 1, -1, -1):
        d = GSd[t] + qq * lw
        lv = ((dt(1.0) - Sd[t]) * b) * lv + sg[t] * d
        LW[t] = lw
        LV[t] = lv
        lw = r * lw - sg[t] * d
    return LV, LW


def param_grads(I, U, W, S, GS, LV, LW, beta, rho, q, theta0, u0, w0, alpha=4.0):
    """ALIFFn.backward gradient assembly (triton_alif.py:541-554), fp64:
    (dI, du0, dw0, dbeta, drho, dq, dtheta0)."""
    dt = np.float64
    Up = np.concatenate([np.asarray(u0, f32)[None], U[:-1]], 0).astype(dt)
    Wp = np.concatenate([np.asarray(w0, f32)[None], W[:-1]], 0).astype(dt)
    sg = surrogate(Up, Wp, I, beta, theta0, alpha, dt)
    d = np.asarray(GS, dt) + dt(q) * LW
    lw_m1 = dt(rho) * LW[0] - sg[0] * d[0]
    return (LV, dt(beta) * LV[0], lw_m1, float((LV * Up).sum()), float((LW * Wp).sum()),
            float((LW * np.asarray(S, dt)).sum()), float(-(sg * d).sum()))
