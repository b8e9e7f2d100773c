"""CPU oracle for the hard-reset LIF path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module,
and only as the checker (never as the thing measured or shipped).  The product path
(lifscan/*) runs HIP kernels and never calls into oracle/.

A numpy restatement (own code) of the reference's algorithm in fp32 with the rounding order
fixed explicitly: every `a*b + c` is two IEEE round-to-nearest operations (numpy evaluates
float32 array expressions one ufunc at a time, so nothing is fused).  Each function cites the
reference lines it restates.  Pins (tests/test_oracle_*.py): exact rational arithmetic with
correct fp32 rounding emulated per operation, Theorem-1 closed form (paper/main.tex:132-140),
brute-force map evaluation, fp64 autograd for the adjoint.
"""
import numpy as np

f32 = np.float32
INF = f32(np.inf)


def _s(x):
    return f32(x)


# ----------------------------------------------------------------------------- serial
def serial_forward(I, beta, theta, u_r, u0):
    """Serial hard-reset LIF (triton_lif.py:21-25 `_step`, :30-39; fast.py:70-81).
    v = fl(fl(beta*u) + x); s = v >= theta; u' = s ? u_r : v.  Returns (U, S) fp32 [T, N]."""
    I = np.ascontiguousarray(I, dtype=f32)
    T, N = I.shape
    b, th, ur = _s(beta), _s(theta), _s(u_r)
    u = np.array(u0, dtype=f32).reshape(N).copy()
    U = np.empty_like(I)
    S = np.empty_like(I)
    for t in range(T):
        v = b * u + I[t]
        s = v >= th
        u = np.where(s, ur, v).astype(f32)
        U[t] = u
        S[t] = s
    return U, S


def serial_segment(I, beta, theta, u_r, start):
    """State after len(I) serial steps from `start` (the chunk fallback, triton_lif.py:600-605)."""
    b, th, ur = _s(beta), _s(theta), _s(u_r)
    u = np.array(start, dtype=f32).copy()
    for t in range(I.shape[0]):
        v = b * u + I[t]
        u = np.where(v >= th, ur, v).astype(f32)
    return u


def coef(up, x, s, gs, gu, beta, theta, u_r, alpha, detach=True, dtype=f32):
    """Adjoint coefficients (triton_lif.py:43-50 `_coef`): returns (a, b) of
    lam_t = b_t + a_t * lam_{t+1}."""
    dt = dtype
    up, x, s, gs = (np.asarray(a, dtype=dt) for a in (up, x, s, gs))
    beta, theta, u_r, alpha = dt(beta), dt(theta), dt(u_r), dt(alpha)
    v = beta * up + x
    sig = dt(1.0) / (dt(1.0) + np.exp(-(alpha * (v - theta))))
    sg = alpha * sig * (dt(1.0) - sig)
    J = dt(1.0) - s
    if not detach:
        J = J + (u_r - v) * sg
    b = gs * sg
    if gu is not None:
        b = b + J * np.asarray(gu, dtype=dt)
    return beta * J, b


def serial_backward(I, u0, U, S, GS, GU, beta, theta, u_r, alpha=4.0, detach=True, dtype=f32):
    """Serial adjoint (triton_lif.py:54-72; fast.py:228-239): lam_t = b_t + a_t*lam_{t+1},
    lam_T = 0; dL/dI_t = lam_t.  dtype=np.float64 gives the reference-grade adjoint."""
    dt = dtype
    T, N = I.shape
    Uprev = np.concatenate([np.asarray(u0, dtype=f32).reshape(1, N), U[:-1]], 0)
    a, b = coef(Uprev, I, S, GS, GU, beta, theta, u_r, alpha, detach, dt)
    lam = np.zeros(N, dtype=dt)
    Lam = np.empty((T, N), dtype=dt)
    for t in range(T - 1, -1, -1):
        lam = b[t] + a[t] * lam
        Lam[t] = lam
    return Lam


def serial_backward_long(I, u0, U, S, GS, beta, theta, u_r, alpha=4.0, block=1024):
    """The fp64 adjoint of serial_backward (detached reset, no GU) for long sequences, where a
    Python loop over every step is slow: the same recurrence lam_t = b_t + a_t*lam_{t+1} (fp64
    coefficients of triton_lif.py:43-50) evaluated blockwise, i.e. each block of `block` steps
    composed to lam_start = P*lam_end + Q, the block ends carried from the last block, then each
    block replayed (the structure of triton_lif.py:512-526, in fp64).  Agrees with
    serial_backward(dtype=float64) to reassociation (~1e-13 relative; pinned in
    tests/test_oracle_lif.py).  T % block == 0."""
    dt = np.float64
    T, N = I.shape
    if T % block:
        raise ValueError("T must be a multiple of block")
    M = T // block
    Uprev = np.concatenate([np.asarray(u0, dtype=f32).reshape(1, N), U[:-1]], 0)
    a, b = coef(Uprev, I, S, GS, None, beta, theta, u_r, alpha, True, dt)
    a = a.reshape(M, block, N)
    b = b.reshape(M, block, N)
    P = np.ones((M, N), dt)
    Q = np.zeros((M, N), dt)
    for j in range(block - 1, -1, -1):
        Q = b[:, j] + a[:, j] * Q
        P = a[:, j] * P
    lam_end = np.zeros((M, N), dt)
    lam = np.zeros(N, dt)
    for m in range(M - 1, -1, -1):
        lam_end[m] = lam
        lam = Q[m] + P[m] * lam
    Lam = np.empty((M, block, N), dt)
    lam = lam_end
    for j in range(block - 1, -1, -1):
        lam = b[:, j] + a[:, j] * lam
        Lam[:, j] = lam
    return Lam.reshape(T, N)


def param_grads(I, u0, U, S, GS, Lam, beta, theta, u_r, alpha=4.0):
    """LIFParamFn.backward assembly (fit.py:36-48), fp64, detached reset:
    (dI, du0, dbeta, dtheta, du_r) = (Lam, beta*Lam[0], sum Lam_t u_{t-1},
    -sum gs_t sg(v_t - theta), sum s_t beta Lam_{t+1})."""
    dt = np.float64
    T, N = I.shape
    Lam = np.asarray(Lam, dt)
    Uprev = np.concatenate([np.asarray(u0, f32).reshape(1, N), U[:-1]], 0).astype(dt)
    v = dt(beta) * Uprev + np.asarray(I, dt)
    sig = 1.0 / (1.0 + np.exp(-(dt(alpha) * (v - dt(theta)))))
    sg = dt(alpha) * sig * (1.0 - sig)
    lam_next = np.concatenate([Lam[1:], np.zeros((1, N), dt)], 0)
    return (Lam, dt(beta) * Lam[0], float((Lam * Uprev).sum()), float(-(np.asarray(GS, dt) * sg).sum()),
            float((np.asarray(S, dt) * dt(beta) * lam_next).sum()))


# ----------------------------------------------------------------------------- two-level scan
def envelope_chunks(I, beta, u_r, C):
    """Per-chunk min-affine envelope map (c, a, b) (triton_lif.py:699-719)."""
    T, N = I.shape
    M = T // C
    b_, ur = _s(beta), _s(u_r)
    Ic = I.reshape(M, C, N)
    c = np.full((M, N), INF, dtype=f32)
    a = np.ones((M, N), dtype=f32)
    bb = np.zeros((M, N), dtype=f32)
    for j in range(C):
        x = Ic[:, j]
        c = np.minimum(ur, b_ * c + x)
        a = b_ * a
        bb = b_ * bb + x
    return c, a, bb


def envelope_carry(u0, EC, EA, EB, margin=1e-5):
    """Sequential envelope carry -> Lo[M, N] (triton_lif.py:723-733)."""
    M, N = EC.shape
    mg = _s(margin)
    l = np.array(u0, dtype=f32).reshape(N).copy()
    Lo = np.empty((M, N), dtype=f32)
    for m in range(M):
        Lo[m] = l - mg * (np.abs(l) + f32(1.0))
        l = np.minimum(EC[m], EA[m] * l + EB[m])
    return Lo


def _safe_div(num, den):
    """num/den with den == 0 -> +inf if num > 0 else -inf (fast.py:94-99, triton_lif.py:761); a
    quotient beyond the float32 range rounds to +-inf, as the IEEE division on the device does."""
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        q = num / den
    return np.where(den == 0, np.where(num > 0, INF, -INF), q).astype(f32)


def build_maps(I, beta, theta, u_r, lo, hi, C, K):
    """Capacity-K pruned chunk maps (triton_lif.py:737-779 build3_kernel; fast.py:148-183).
    lo: [M, N] per-chunk (v3) or [N] per-neuron (v1/v2) lower bound; hi: [N].
    Returns A, B [M,N], xd, cd [M,K,N] (breakpoints descending; slots >= n hold +inf / junk),
    n [M,N] int32, ovf [M,N] int32."""
    T, N = I.shape
    M = T // C
    b_, th, ur = _s(beta), _s(theta), _s(u_r)
    Ic = I.reshape(M, C, N)
    lo = np.broadcast_to(np.asarray(lo, dtype=f32), (M, N))
    hi = np.broadcast_to(np.asarray(hi, dtype=f32), (M, N))
    A = np.ones((M, N), dtype=f32)
    B = np.zeros((M, N), dtype=f32)
    xd = np.full((M, K, N), INF, dtype=f32)
    cd = np.zeros((M, K, N), dtype=f32)
    cnt = np.zeros((M, N), dtype=np.int32)
    xmin = np.full((M, N), INF, dtype=f32)
    ovf = np.zeros((M, N), dtype=np.int32)
    ks = np.arange(K, dtype=np.int32)[None, :, None]
    for j in range(C):
        x = Ic[:, j]
        vv = b_ * cd + x[:, None, :]
        cd = np.where(vv >= th, ur, vv).astype(f32)
        num = (th - x) - b_ * B
        den = b_ * A
        z = _safe_div(num, den)
        new = (z < xmin) & (z <= hi) & (xmin > lo)
        ovf = np.where(new & (cnt >= K), 1, ovf).astype(np.int32)
        new = new & (cnt < K)
        slot = (ks == cnt[:, None, :]) & new[:, None, :]
        xd = np.where(slot, z[:, None, :], xd)
        cd = np.where(slot, ur, cd).astype(f32)
        cnt = cnt + new.astype(np.int32)
        xmin = np.where(new, z, xmin)
        A = b_ * A
        B = b_ * B + x
    return A, B, xd, cd, cnt, ovf


def eval_map(A, B, xd, cd, n, u):
    """Map evaluation at states u (triton_lif.py:592-599; fast.py:243-251):
    k = #{i < n : xd[i] > u};  k == n -> A*u + B, else cd[k].  xd, cd: [K, N]."""
    K = xd.shape[0]
    valid = np.arange(K)[:, None] < n[None, :]
    k = ((xd > u[None, :]) & valid).sum(0)
    kc = np.minimum(k, K - 1)
    c = np.take_along_axis(cd, kc[None, :], 0)[0]
    return np.where(k == n, A * u + B, c).astype(f32)


def carry(I, u0, A, B, xd, cd, n, ovf, beta, theta, u_r, C):
    """Sequential carry with per-lane serial fallback on overflow (triton_lif.py:579-606)."""
    M, N = A.shape
    u = np.array(u0, dtype=f32).reshape(N).copy()
    starts = np.empty((M, N), dtype=f32)
    for m in range(M):
        starts[m] = u
        nu = eval_map(A[m], B[m], xd[m], cd[m], n[m], u)
        if ovf[m].any():
            w = serial_segment(I[m * C:(m + 1) * C], beta, theta, u_r, u)
            nu = np.where(ovf[m] > 0, w, nu).astype(f32)
        u = nu
    return starts


def replay(I, starts, beta, theta, u_r, C):
    """Replay every chunk from its start (triton_lif.py:152-165) -> U, S, Ends [M, N]."""
    T, N = I.shape
    M = T // C
    b_, th, ur = _s(beta), _s(theta), _s(u_r)
    Ic = I.reshape(M, C, N)
    u = starts.astype(f32).copy()
    U = np.empty((M, C, N), dtype=f32)
    S = np.empty((M, C, N), dtype=f32)
    for j in range(C):
        v = b_ * u + Ic[:, j]
        s = v >= th
        u = np.where(s, ur, v).astype(f32)
        U[:, j] = u
        S[:, j] = s
    return U.reshape(T, N), S.reshape(T, N), u


def scan_forward_v3(I, beta, theta, u_r, u0, C=64, K=16, repair=0, stats=None, lo=None,
                    keep=None):
    """Two-level scan (triton_lif.py:782-817): envelope -> build -> carry -> replay -> Jacobi
    repair (torch.equal on chunk starts), stats as :812-816.  lo: optional per-neuron bound
    (v1/v2 pruning) instead of the envelope.  keep: optional dict receiving intermediates."""
    I = np.ascontiguousarray(I, dtype=f32)
    T, N = I.shape
    assert T % C == 0
    M = T // C
    u0 = np.asarray(u0, dtype=f32).reshape(N)
    hi = np.maximum(u0, np.maximum(_s(theta), _s(u_r)))
    if lo is None:
        EC, EA, EB = envelope_chunks(I, beta, u_r, C)
        Lo = envelope_carry(u0, EC, EA, EB)
    else:
        Lo = np.broadcast_to(np.asarray(lo, dtype=f32), (M, N)).copy()
    A, B, xd, cd, n, ovf = build_maps(I, beta, theta, u_r, Lo, hi, C, K)
    starts = carry(I, u0, A, B, xd, cd, n, ovf, beta, theta, u_r, C)
    U, S, ends = replay(I, starts, beta, theta, u_r, C)
    it = 0
    for it in range(1, repair + 1):
        new = np.concatenate([u0[None], ends[:-1]], 0)
        if np.array_equal(new, starts):
            it -= 1
            break
        starts = new
        U, S, ends = replay(I, starts, beta, theta, u_r, C)
    if stats is not None:
        stats["repair_iters"] = it
        stats["overflow_frac"] = float(ovf.astype(np.float64).mean())
        stats["mean_pieces"] = float(n.astype(np.float64).mean()) + 1
        stats["max_pieces"] = int(n.max()) + 1
    if keep is not None:
        keep.update(Lo=Lo, A=A, B=B, xd=xd, cd=cd, n=n, ovf=ovf, starts=starts, ends=ends)
    return U, S


def state_bounds(I, beta, theta, u_r, u0):
    """Loose per-neuron bounds (triton_lif.py:238-243; fast.py:134-144), fp32."""
    I = np.asarray(I, dtype=f32)
    u0 = np.asarray(u0, dtype=f32)
    Imin = np.minimum(I.min(0), f32(0))
    base = np.minimum(np.minimum(u0, _s(u_r)), f32(0))
    if beta < 1:
        lo = base + Imin / f32(1 - beta)
    else:
        lo = base + np.minimum(I, f32(0)).sum(0, dtype=f32)
    hi = np.maximum(u0, f32(max(theta, u_r)))
    return lo.astype(f32), hi.astype(f32)


# ----------------------------------------------------------------------------- three-level scan
def compose_groups(A, B, xd, cd, n, ovf, Lo, u0, theta, u_r, G, K2):
    """Compose G consecutive chunk maps into super maps of capacity K2
    (triton_lif.py:829-899 compose_group_kernel): (1) push the left map's constants through
    the right map, (2) pull the right map's breakpoints back through the left map's affine
    part, appended iff z < xmin, z <= hi and xmin > lo (lo of the group's first chunk),
    overflow past K2, (3) compose the affine parts.  Returns SA, SB, SX, SC, SN, SOVF."""
    M, K, N = xd.shape
    M2 = M // G
    th, ur = _s(theta), _s(u_r)
    hi = np.maximum(np.asarray(u0, dtype=f32), np.maximum(th, ur))
    SA = np.empty((M2, N), f32)
    SB = np.empty((M2, N), f32)
    SX = np.full((M2, K2, N), INF, f32)
    SC = np.zeros((M2, K2, N), f32)
    SN = np.empty((M2, N), np.int32)
    SOVF = np.empty((M2, N), np.int32)
    k2 = np.arange(K2)[:, None]
    for s_ in range(M2):
        m0 = s_ * G
        lo = Lo[m0]
        Ah, Bh = A[m0].copy(), B[m0].copy()
        nH = n[m0].astype(np.int32).copy()
        ov = ovf[m0].astype(np.int32).copy()
        X = np.full((K2, N), INF, f32)
        Cc = np.zeros((K2, N), f32)
        kk = min(K, K2)
        X[:kk] = xd[m0, :kk]
        Cc[:kk] = cd[m0, :kk]
        xmin = np.where(k2 < nH[None], X, INF).min(0).astype(f32)
        for jj in range(1, G):
            m = m0 + jj
            Ag, Bg, ng = A[m], B[m], n[m]
            yd, dd = xd[m], cd[m]
            ov = ov | ovf[m]
            cnt = np.zeros((K2, N), np.int32)
            for j in range(K):
                cnt += ((yd[j][None] > Cc) & (j < ng)[None]).astype(np.int32)
            gc = np.zeros((K2, N), f32)
            for j in range(K):
                gc = np.where(cnt == j, dd[j][None], gc)
            Cc = np.where(cnt == ng[None], Ag[None] * Cc + Bg[None], gc).astype(f32)
            for j in range(K):
                num = yd[j] - Bh
                z = _safe_div(num, Ah)
                new = (j < ng) & (z < xmin) & (z <= hi) & (xmin > lo)
                ov = np.where(new & (nH >= K2), 1, ov).astype(np.int32)
                new = new & (nH < K2)
                slot = (k2 == nH[None]) & new[None]
                X = np.where(slot, z[None], X)
                Cc = np.where(slot, dd[j][None], Cc).astype(f32)
                nH = nH + new.astype(np.int32)
                xmin = np.where(new, z, xmin).astype(f32)
            Bh = Ag * Bh + Bg
            Ah = Ag * Ah
        SA[s_], SB[s_], SX[s_], SC[s_], SN[s_], SOVF[s_] = Ah, Bh, X, Cc, nH, ov
    return SA, SB, SX, SC, SN, SOVF


def carry_inner(I, sstarts, A, B, xd, cd, n, ovf, beta, theta, u_r, C, G):
    """Carry the G chunk maps of every super map in parallel from its start
    (triton_lif.py:903-932 carry_inner_kernel)."""
    M, N = A.shape
    M2 = M // G
    starts = np.empty((M, N), f32)
    u = sstarts.astype(f32).copy()  # [M2, N]
    for jj in range(G):
        ms = np.arange(M2) * G + jj
        starts[ms] = u
        nu = np.empty_like(u)
        for s_ in range(M2):
            m = s_ * G + jj
            v = eval_map(A[m], B[m], xd[m], cd[m], n[m], u[s_])
            if ovf[m].any():
                w = serial_segment(I[m * C:(m + 1) * C], beta, theta, u_r, u[s_])
                v = np.where(ovf[m] > 0, w, v).astype(f32)
            nu[s_] = v
        u = nu
    return starts


def carry_super(I, u0, SA, SB, SX, SC, SN, SOVF, A, B, xd, cd, n, ovf, beta, theta, u_r, C, G,
                fallback="chunks"):
    """Sequential carry over the super maps (triton_lif.py:958-963, carry2_kernel with fallback
    length C*G).  An overflowed super map is passed with fallback "serial" by its C*G serial steps
    (the reference), with "chunks" by evaluating its G chunk maps in turn from the super's start
    exactly as carry_inner does (an overflowed chunk map by its C serial steps), so that the
    next super's start is the value the inner carry reaches at the end of this one, and with
    "none" by evaluating it as stored (a start that may be wrong, for repair to convergence)."""
    if fallback == "serial":
        return carry(I, u0, SA, SB, SX, SC, SN, SOVF, beta, theta, u_r, C * G)
    if fallback == "none":
        return carry(I, u0, SA, SB, SX, SC, SN, np.zeros_like(SOVF), beta, theta, u_r, C * G)
    M2, N = SA.shape
    u = np.array(u0, dtype=f32).reshape(N).copy()
    sstarts = np.empty((M2, N), dtype=f32)
    for s_ in range(M2):
        sstarts[s_] = u
        nu = eval_map(SA[s_], SB[s_], SX[s_], SC[s_], SN[s_], u)
        bad = SOVF[s_] > 0
        if bad.any():
            w = u.copy()
            for jj in range(G):
                m = s_ * G + jj
                v = eval_map(A[m], B[m], xd[m], cd[m], n[m], w)
                if ovf[m].any():
                    v = np.where(ovf[m] > 0, serial_segment(I[m * C:(m + 1) * C], beta, theta, u_r, w),
                                 v).astype(f32)
                w = v
            nu = np.where(bad, w, nu).astype(f32)
        u = nu
    return sstarts


def scan_forward_v4(I, beta, theta, u_r, u0, C=64, G=16, K=16, K2=32, repair=0, stats=None,
                    keep=None, super_fallback="chunks"):
    """Three-level scan (triton_lif.py:935-983): envelope -> chunk maps -> group composition
    -> carry over super maps (an overflowed one passed as carry_super's `fallback`) -> inner
    carry -> replay -> repair; stats as :976-982."""
    I = np.ascontiguousarray(I, dtype=f32)
    T, N = I.shape
    M = T // C
    assert T % C == 0 and M % G == 0, "T must be divisible by C*G"
    u0 = np.asarray(u0, dtype=f32).reshape(N)
    hi = np.maximum(u0, np.maximum(_s(theta), _s(u_r)))
    EC, EA, EB = envelope_chunks(I, beta, u_r, C)
    Lo = envelope_carry(u0, EC, EA, EB)
    A, B, xd, cd, n, ovf = build_maps(I, beta, theta, u_r, Lo, hi, C, K)
    SA, SB, SX, SC, SN, SOVF = compose_groups(A, B, xd, cd, n, ovf, Lo, u0, theta, u_r, G, K2)
    sstarts = carry_super(I, u0, SA, SB, SX, SC, SN, SOVF, A, B, xd, cd, n, ovf, beta, theta, u_r,
                          C, G, super_fallback)
    starts = carry_inner(I, sstarts, A, B, xd, cd, n, ovf, beta, theta, u_r, C, G)
    U, S, ends = replay(I, starts, beta, theta, u_r, C)
    it = 0
    for it in range(1, repair + 1):
        new = np.concatenate([u0[None], ends[:-1]], 0)
        if np.array_equal(new, starts):
            it -= 1
            break
        starts = new
        U, S, ends = replay(I, starts, beta, theta, u_r, C)
    if stats is not None:
        stats["repair_iters"] = it
        stats["overflow_frac"] = float(ovf.astype(np.float64).mean())
        stats["super_overflow_frac"] = float(SOVF.astype(np.float64).mean())
        stats["mean_pieces"] = float(n.astype(np.float64).mean()) + 1
        stats["super_mean_pieces"] = float(SN.astype(np.float64).mean()) + 1
        stats["super_max_pieces"] = int(SN.max()) + 1
    if keep is not None:
        keep.update(Lo=Lo, A=A, B=B, xd=xd, cd=cd, n=n, ovf=ovf, SA=SA, SB=SB, SX=SX, SC=SC,
                    SN=SN, SOVF=SOVF, sstarts=sstarts, starts=starts)
    return U, S


# ----------------------------------------------------------------------------- scan backward
def scan_backward(I, u0, U, S, GS, GU, beta, theta, u_r, alpha=4.0, detach=True, C=64):
    """Two-level affine scan of the adjoint (triton_lif.py:422-457, :198-208, :383-418), fp32."""
    T, N = I.shape
    M = T // C
    Uprev = np.concatenate([np.asarray(u0, dtype=f32).reshape(1, N), U[:-1]], 0)
    a, b = coef(Uprev, I, S, GS, GU, beta, theta, u_r, alpha, detach, f32)
    a = a.reshape(M, C, N)
    b = b.reshape(M, C, N)
    P = np.ones((M, N), dtype=f32)
    Q = np.zeros((M, N), dtype=f32)
    for j in range(C - 1, -1, -1):
        Q = b[:, j] + a[:, j] * Q
        P = a[:, j] * P
    lam_end = np.empty((M, N), dtype=f32)
    lam = np.zeros(N, dtype=f32)
    for m in range(M - 1, -1, -1):
        lam_end[m] = lam
        lam = Q[m] + P[m] * lam
    Lam = np.empty((M, C, N), dtype=f32)
    lam = lam_end.copy()
    for j in range(C - 1, -1, -1):
        lam = b[:, j] + a[:, j] * lam
        Lam[:, j] = lam
    return Lam.reshape(T, N)


# ----------------------------------------------------------------------------- dispatch policy
def pick_C(T, D=8):
    """triton_lif.py:647-651."""
    for C in (256, 128, 64, 32, 16, 8):
        if T % C == 0 and C % D == 0 and C * C <= 4 * T:
            return C
    raise ValueError(f"T={T} needs a chunk length divisible by {D}")
