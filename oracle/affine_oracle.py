"""CPU oracle for the affine-reset LIF scan — TEST INFRASTRUCTURE ONLY (see oracle/lif_oracle.py).

numpy fp32 restatement (own code) of lifscan/triton_affine.py, with every `a*b + c` evaluated as
two IEEE round-to-nearest operations and every division correctly rounded.  Step
(triton_affine.py:19-23):
    v = beta*u + x;  s = v >= theta;  u' = s ? gamma*v + delta : v        (0 <= gamma <= 1)
hard reset: gamma = 0, delta = u_r; soft reset: gamma = 1, delta = -theta.

Chunk maps are unsorted lists of pieces [xl, xr) with value a*u + c (triton_affine.py:6-10).
Pins (tests/test_oracle_affine.py): the step against exact rationals rounded to fp32 per
operation; gamma = 0 against the hard-reset oracle; dyadic inputs on which every fp32 operation
is exact, where the map must hold every start of the reachable interval in exactly one piece
and give the serial chunk result bit for bit (breakpoint ties included); the piece bound of
Theorem 7(b) and the tiling of the line by the unpruned pieces; the envelopes against the
serial trajectory; repair == serial on the reference's own test grid (tests/test_affine.py:
7-18); the adjoint and parameter gradients against fp64 autograd of the serial recurrence
(tests/test_affine.py:19-35).
"""
import numpy as np

from oracle.lif_oracle import envelope_carry, envelope_chunks

f32 = np.float32
INF = f32(np.inf)


def _s(x):
    return f32(x)


def r_theta(gamma, theta, delta):
    """Lower envelope's reset value r(theta) = gamma*theta + delta, computed in double from the
    Python floats and then taken as fp32 by the kernels (triton_affine.py:171)."""
    return f32(float(gamma) * float(theta) + float(delta))


def aff_step(u, x, beta, theta, gamma, delta):
    """triton_affine.py:19-23 -> (u', s, v)."""
    b, th, g, d = _s(beta), _s(theta), _s(gamma), _s(delta)
    v = b * u + x
    s = v >= th
    return np.where(s, g * v + d, v).astype(f32), s, v


def serial_forward(I, beta, theta, gamma, delta, u0):
    """Serial affine-reset LIF (triton_affine.py:144-162) -> (U, S) fp32 [T, N]."""
    I = np.ascontiguousarray(I, dtype=f32)
    T, N = I.shape
    u = np.array(u0, dtype=f32).reshape(N).copy()
    U = np.empty_like(I)
    S = np.empty_like(I)
    for t in range(T):
        u, s, _ = aff_step(u, I[t], beta, theta, gamma, delta)
        U[t], S[t] = u, s
    return U, S


def serial_segment(I, beta, theta, gamma, delta, u):
    u = np.array(u, dtype=f32).copy()
    for t in range(I.shape[0]):
        u, _, _ = aff_step(u, I[t], beta, theta, gamma, delta)
    return u


# ----------------------------------------------------------------------------- envelopes
def env_hi_chunks(I, beta, theta, gamma, delta, C):
    """Per-chunk max-affine upper envelope (c, a, b) (triton_affine.py:26-36):
    c = max(theta, gamma*(beta*c + x) + delta) from c = -inf (np.fmax: a NaN from
    0*(-inf) at gamma = 0 yields theta, as the kernels' max does), a = (gamma*beta)*a,
    b = gamma*(beta*b + x) + delta."""
    T, N = I.shape
    M = T // C
    b_, th, g, d = _s(beta), _s(theta), _s(gamma), _s(delta)
    gb = g * b_
    Ic = I.reshape(M, C, N)
    c = np.full((M, N), -INF, dtype=f32)
    a = np.ones((M, N), dtype=f32)
    bb = np.zeros((M, N), dtype=f32)
    with np.errstate(invalid="ignore"):
        for j in range(C):
            x = Ic[:, j]
            c = np.fmax(th, g * (b_ * c + x) + d).astype(f32)
            a = gb * a
            bb = g * (b_ * bb + x) + d
    return c, a, bb


def env_hi_carry(u0, EC, EA, EB, margin=1e-5):
    """Sequential upper-envelope carry -> Hi[M, N] (triton_affine.py:39-48)."""
    M, N = EC.shape
    mg = _s(margin)
    h = np.array(u0, dtype=f32).reshape(N).copy()
    Hi = np.empty((M, N), dtype=f32)
    for m in range(M):
        Hi[m] = h + mg * (np.abs(h) + f32(1.0))
        h = np.fmax(EC[m], EA[m] * h + EB[m]).astype(f32)
    return Hi


def envelopes(I, beta, theta, gamma, delta, u0, C):
    """(Lo, Hi) [M, N]: the hard-reset lower envelope with u_r = r(theta)
    (triton_affine.py:171-174) and the max-affine upper envelope (:175-177)."""
    u0 = np.asarray(u0, dtype=f32).reshape(-1)
    EC, EA, EB = envelope_chunks(I, beta, r_theta(gamma, theta, delta), C)
    Lo = envelope_carry(u0, EC, EA, EB)
    HC, HA, HB = env_hi_chunks(I, beta, theta, gamma, delta, C)
    Hi = env_hi_carry(u0, HC, HA, HB)
    return Lo, Hi


# ----------------------------------------------------------------------------- chunk maps
def build_maps(I, Lo, Hi, beta, theta, gamma, delta, C, K):
    """Capacity-K chunk maps (triton_affine.py:51-111).  Per step every piece [xl, xr) with
    value a*u + c is advanced; the threshold cut z = (ct - c)/a with ct = (theta - x)/beta
    splits it into a left (no spike, or spike when z <= xl) and a right (spike) part; parts
    outside [lo, hi] are dropped and the list compacted in order, left before right.
    Output slot k takes the piece i with p_i <= k < p_i + nout_i (p the exclusive prefix sum
    of the output counts), which the reference finds by binary search over p and which is
    written here as a scatter of every part to its slot.
    Returns xl, xr, a, c [M, N, K] (slots >= n hold xl = xr = inf, a = 1, c = 0), n [M, N]
    int32 (min(count, K)), ovf [M, N] int32."""
    I = np.ascontiguousarray(I, dtype=f32)
    T, N = I.shape
    M = T // C
    R = M * N
    b_, th, g, d = _s(beta), _s(theta), _s(gamma), _s(delta)
    gb = g * b_
    Ic = I.reshape(M, C, N)
    lo = np.asarray(Lo, dtype=f32).reshape(R)[:, None]
    hi = np.asarray(Hi, dtype=f32).reshape(R)[:, None]
    ks = np.arange(K)[None, :]
    xl = np.where(ks == 0, -INF, INF).astype(f32) + np.zeros((R, K), f32)
    xr = np.full((R, K), INF, f32)
    aa = np.ones((R, K), f32)
    cc = np.zeros((R, K), f32)
    cnt = np.ones(R, np.int32)
    ovf = np.zeros(R, np.int32)
    rows = np.arange(R)[:, None]
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        for j in range(C):
            x = Ic[:, j].reshape(R)[:, None]
            ct = (th - x) / b_
            valid = ks < cnt[:, None]
            num = ct - cc
            z = np.where(aa == 0, np.where(num > 0, INF, -INF), num / aa).astype(f32)
            full = z <= xl
            split = (z > xl) & (z < xr) & valid
            vns = b_ * cc + x
            c_sp = g * vns + d
            a_no = b_ * aa
            a_sp = gb * aa
            cl = np.where(full, c_sp, vns).astype(f32)
            al = np.where(full, a_sp, a_no).astype(f32)
            xr_left = np.where(split, z, xr).astype(f32)
            vl = valid & (xr_left > lo) & (xl <= hi)
            vr = split & (xr > lo) & (z <= hi)
            nout = vl.astype(np.int32) + vr.astype(np.int32)
            p = np.cumsum(nout, axis=1) - nout
            ntot = nout.sum(1)
            ovf = np.where(ntot > K, 1, ovf).astype(np.int32)
            # scatter: left part to slot p, right part to slot p + vl (column K = dropped)
            nxl = np.full((R, K + 1), INF, f32)
            nxr = np.full((R, K + 1), INF, f32)
            na = np.ones((R, K + 1), f32)
            nc = np.zeros((R, K + 1), f32)
            dl = np.where(vl & (p < K), p, K)
            dr = np.where(vr & (p + vl < K), p + vl, K)
            nxl[rows, dl], nxr[rows, dl], na[rows, dl], nc[rows, dl] = xl, xr_left, al, cl
            # right parts are written second; a dropped part only ever lands in column K
            nxl[rows, dr] = np.where(dr < K, z, nxl[rows, dr])
            nxr[rows, dr] = np.where(dr < K, xr, nxr[rows, dr])
            na[rows, dr] = np.where(dr < K, a_sp, na[rows, dr])
            nc[rows, dr] = np.where(dr < K, c_sp, nc[rows, dr])
            cnt = np.minimum(ntot, K).astype(np.int32)
            keep = ks < cnt[:, None]
            xl = np.where(keep, nxl[:, :K], INF).astype(f32)
            xr = np.where(keep, nxr[:, :K], INF).astype(f32)
            aa = np.where(keep, na[:, :K], f32(1.0)).astype(f32)
            cc = np.where(keep, nc[:, :K], f32(0.0)).astype(f32)
    sh = (M, N, K)
    return (xl.reshape(sh), xr.reshape(sh), aa.reshape(sh), cc.reshape(sh),
            cnt.reshape(M, N), ovf.reshape(M, N))


def eval_map(xl, xr, a, c, n, u):
    """Map value at u (triton_affine.py:130-132): the pieces with xl <= u < xr among the first
    n; value a*u + c of the hit (plus 0.0: the reference sums the hit lanes, so -0.0 reads as
    +0.0) and whether exactly one piece was hit.  xl..c: [N, K]; n, u: [N]."""
    K = xl.shape[-1]
    u = np.asarray(u, dtype=f32)
    hit = (np.arange(K)[None, :] < n[:, None]) & (xl <= u[:, None]) & (u[:, None] < xr)
    val = (a * u[:, None] + c).astype(f32)
    k = np.argmax(hit, axis=1)
    v = np.take_along_axis(val, k[:, None], 1)[:, 0] + f32(0.0)
    found = hit.sum(1) == 1
    return np.where(found, v, f32(0.0)).astype(f32), found


def carry(I, u0, xl, xr, a, c, n, ovf, beta, theta, gamma, delta, C):
    """Sequential carry with per-neuron serial fallback (triton_affine.py:114-140): a chunk
    whose map overflowed or whose start is not in exactly one piece runs serially."""
    M, N = n.shape
    u = np.array(u0, dtype=f32).reshape(N).copy()
    starts = np.empty((M, N), dtype=f32)
    for m in range(M):
        starts[m] = u
        nu, found = eval_map(xl[m], xr[m], a[m], c[m], n[m], u)
        bad = (ovf[m] > 0) | ~found
        if bad.any():
            w = serial_segment(I[m * C:(m + 1) * C], beta, theta, gamma, delta, u)
            nu = np.where(bad, w, nu).astype(f32)
        u = nu
    return starts


def replay(I, starts, beta, theta, gamma, delta, C):
    """Replay every chunk from its start (triton_affine.py:143-155) -> U, S, Ends [M, N]."""
    T, N = I.shape
    M = T // C
    Ic = I.reshape(M, C, N)
    u = starts.astype(f32).copy()
    U = np.empty((M, C, N), dtype=f32)
    S = np.empty((M, C, N), dtype=f32)
    for j in range(C):
        u, s, _ = aff_step(u, Ic[:, j], beta, theta, gamma, delta)
        U[:, j] = u
        S[:, j] = s
    return U.reshape(T, N), S.reshape(T, N), u


def scan_forward(I, beta, theta, gamma, delta, u0, C=128, K=32, repair=0, stats=None, keep=None):
    """Two-level affine-reset scan (triton_affine.py:165-199): envelopes -> build -> carry ->
    replay -> Jacobi repair until the chunk starts stop changing; stats repair_iters,
    overflow_frac, mean_pieces (mean kept pieces, :195-198)."""
    I = np.ascontiguousarray(I, dtype=f32)
    T, N = I.shape
    assert T % C == 0 and 0.0 <= float(gamma) <= 1.0
    u0 = np.asarray(u0, dtype=f32).reshape(N)
    Lo, Hi = envelopes(I, beta, theta, gamma, delta, u0, C)
    xl, xr, a, c, n, ovf = build_maps(I, Lo, Hi, beta, theta, gamma, delta, C, K)
    starts = carry(I, u0, xl, xr, a, c, n, ovf, beta, theta, gamma, delta, C)
    U, S, ends = replay(I, starts, beta, theta, gamma, delta, C)
    it = 0
    for it in range(1, repair + 1):
        new = np.concatenate([u0[None], ends[:-1]], 0)
        if np.array_equal(new, starts):
            it -= 1
            break
        starts = new
        U, S, ends = replay(I, starts, beta, theta, gamma, delta, C)
    if stats is not None:
        stats["repair_iters"] = it
        stats["overflow_frac"] = float(ovf.astype(np.float64).mean())
        stats["mean_pieces"] = float(n.astype(np.float64).mean())
    if keep is not None:
        keep.update(Lo=Lo, Hi=Hi, xl=xl, xr=xr, a=a, c=c, n=n, ovf=ovf, starts=starts, ends=ends)
    return U, S


# ----------------------------------------------------------------------------- adjoint
def backward(I, u0, U, S, GS, beta, gamma, delta, theta=1.0, alpha=4.0, dtype=f32):
    """LIFAffineFn.backward (triton_affine.py:229-242) with the reverse recurrence solved
    serially: v_t = beta*u_{t-1} + x_t, sg = sigmoid(alpha*(v - theta)), sgd = alpha*sg*(1-sg),
    J_t = (1 - s_t) + s_t*gamma (detached spike), lam_t = gs_t*sgd_t + beta*J_t*lam_{t+1}
    (lam_T = 0).  Returns (dI = lam, du0 = beta*lam_0, dbeta = sum lam_t*u_{t-1},
    dgamma = sum s_t*v_t*beta*lam_{t+1}, ddelta = sum s_t*beta*lam_{t+1}); the sums in fp64.
    dtype f32 or f64 for the recurrence."""
    I, U, S, GS = (np.asarray(z, dtype=dtype) for z in (I, U, S, GS))
    T, N = I.shape
    # the parameters as the fp32 scalars the kernels and torch's fp32 ops use
    b, g, th, al = (dtype(_s(z)) for z in (beta, gamma, theta, alpha))
    up = np.concatenate([np.asarray(u0, dtype=dtype).reshape(1, N), U[:-1]], 0)
    V = b * up + I
    sig = (1.0 / (1.0 + np.exp(-(al * (V - th))))).astype(dtype)
    sgd = (al * sig * (1 - sig)).astype(dtype)
    J = ((1 - S) + S * g).astype(dtype)
    lam = np.zeros((T, N), dtype=dtype)
    nxt = np.zeros(N, dtype=dtype)
    for t in range(T - 1, -1, -1):
        nxt = (GS[t] * sgd[t] + (b * J[t]) * nxt).astype(dtype)
        lam[t] = nxt
    lam_next = np.concatenate([lam[1:], np.zeros((1, N), dtype)], 0).astype(np.float64)
    S64, V64, b64 = S.astype(np.float64), V.astype(np.float64), float(np.float64(b))
    dbeta = float((lam.astype(np.float64) * up.astype(np.float64)).sum())
    dgamma = float((S64 * V64 * b64 * lam_next).sum())
    ddelta = float((S64 * b64 * lam_next).sum())
    return lam, b * lam[0], dbeta, dgamma, ddelta
