"""CPU oracle for the soft-reset LIF scan — TEST INFRASTRUCTURE ONLY (see oracle/lif_oracle.py).

numpy fp32 restatement (own code) of lifscan/triton_soft.py and the soft-reset serial kernels
of lifscan/triton_lif.py:1034-1083, with every `a*b + c` evaluated as two IEEE
round-to-nearest operations.  Step (triton_soft.py:106-110):
    v = beta*u + x;  s = v >= theta;  u' = s ? v - theta : v
Chunk maps share one slope A = beta^j and keep only the piece offsets c (triton_soft.py:3-7).
The GPU path runs this model as the affine reset with gamma = 1, delta = -theta; the pins in
tests/test_oracle_soft.py show that the two restatements give the same bits (step, envelopes,
pieces, carried starts), and pin the adjoint's FFT convolution against the direct float64
recurrence and fp64 autograd.
"""
import numpy as np

from oracle.lif_oracle import envelope_carry, envelope_chunks

f32 = np.float32
INF = f32(np.inf)


def _s(x):
    return f32(x)


def soft_step(u, x, beta, theta):
    """triton_soft.py:106-110 -> (u', s)."""
    b, th = _s(beta), _s(theta)
    v = b * u + x
    s = v >= th
    return np.where(s, v - th, v).astype(f32), s


def serial_forward(I, beta, theta, u0):
    """Serial soft-reset LIF (triton_soft.py:157-172; triton_lif.py:1037-1076) -> (U, S)."""
    I = np.ascontiguousarray(I, dtype=f32)
    T, N = I.shape
    u = np.array(u0, dtype=f32).reshape(N).copy()
    U = np.empty_like(I)
    S = np.empty_like(I)
    for t in range(T):
        u, s = soft_step(u, I[t], beta, theta)
        U[t], S[t] = u, s
    return U, S


def serial_segment(I, beta, theta, u):
    u = np.array(u, dtype=f32).copy()
    for t in range(I.shape[0]):
        u, _ = soft_step(u, I[t], beta, theta)
    return u


def env_hi_chunks(I, beta, theta, C):
    """Upper envelope per chunk (triton_soft.py:20-31): c = max(theta, beta*c + x - theta) from
    -inf, a = beta*a, b = beta*b + x - theta (left to right: fl(fl(fl(beta*c) + x) - theta))."""
    T, N = I.shape
    M = T // C
    b_, th = _s(beta), _s(theta)
    Ic = I.reshape(M, C, N)
    c = np.full((M, N), -INF, f32)
    a = np.ones((M, N), f32)
    bb = np.zeros((M, N), f32)
    for j in range(C):
        x = Ic[:, j]
        c = np.maximum(th, (b_ * c + x) - th)
        a = b_ * a
        bb = (b_ * bb + x) - th
    return c, a, bb


def env_hi_carry(u0, EC, EA, EB, margin=1e-5):
    """triton_soft.py:34-43: Hi[m] = h + margin(|h| + 1); h = max(c, max(a*h + b, h*0 + c))."""
    M, N = EC.shape
    mg = _s(margin)
    h = np.array(u0, dtype=f32).reshape(N).copy()
    Hi = np.empty((M, N), f32)
    for m in range(M):
        Hi[m] = h + mg * (np.abs(h) + f32(1.0))
        h = np.maximum(EC[m], np.maximum(EA[m] * h + EB[m], h * f32(0.0) + EC[m]))
    return Hi


def envelopes(I, beta, theta, u0, C):
    """(Lo, Hi): the hard-reset lower envelope with u_r = 0 (triton_soft.py:181-184) and the
    upper envelope (:185-187)."""
    u0 = np.asarray(u0, dtype=f32).reshape(-1)
    EC, EA, EB = envelope_chunks(I, beta, 0.0, C)
    Lo = envelope_carry(u0, EC, EA, EB)
    HC, HA, HB = env_hi_chunks(I, beta, theta, C)
    return Lo, env_hi_carry(u0, HC, HA, HB)


def build_maps(I, Lo, Hi, beta, theta, C, K):
    """Chunk maps with a common slope (triton_soft.py:46-103): per step ct = (theta - x)/beta,
    z = (ct - c)/A (A == 0: all or nothing), the left part keeps c' = beta*c + x (minus theta
    when the whole piece spikes), the right part [z, xr) takes beta*c + x - theta; compaction in
    order with overflow beyond K; A <- beta*A after the step.
    Returns A [M, N], xl, xr, c [M, N, K], n [M, N], ovf [M, N]."""
    I = np.ascontiguousarray(I, dtype=f32)
    T, N = I.shape
    M = T // C
    R = M * N
    b_, th = _s(beta), _s(theta)
    Ic = I.reshape(M, C, N)
    lo = np.asarray(Lo, dtype=f32).reshape(R)[:, None]
    hi = np.asarray(Hi, dtype=f32).reshape(R)[:, None]
    ks = np.arange(K)[None, :]
    xl = np.where(ks == 0, -INF, INF).astype(f32) + np.zeros((R, K), f32)
    xr = np.full((R, K), INF, f32)
    cc = np.zeros((R, K), f32)
    cnt = np.ones(R, np.int32)
    ovf = np.zeros(R, np.int32)
    A = np.ones((R, 1), f32)
    rows = np.arange(R)[:, None]
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        for j in range(C):
            x = Ic[:, j].reshape(R)[:, None]
            ct = (th - x) / b_
            valid = ks < cnt[:, None]
            num = ct - cc
            z = np.where(A == 0, np.where(num > 0, INF, -INF), num / A).astype(f32)
            full = z <= xl
            split = (z > xl) & (z < xr) & valid
            cns = b_ * cc + x
            cr = cns - th
            cl = np.where(full, cr, cns).astype(f32)
            xr_left = np.where(split, z, xr).astype(f32)
            vl = valid & (xr_left > lo) & (xl <= hi)
            vr = split & (xr > lo) & (z <= hi)
            nout = vl.astype(np.int32) + vr.astype(np.int32)
            p = np.cumsum(nout, axis=1) - nout
            ntot = nout.sum(1)
            ovf = np.where(ntot > K, 1, ovf).astype(np.int32)
            nxl = np.full((R, K + 1), INF, f32)
            nxr = np.full((R, K + 1), INF, f32)
            nc = np.zeros((R, K + 1), f32)
            dl = np.where(vl & (p < K), p, K)
            dr = np.where(vr & (p + vl < K), p + vl, K)
            nxl[rows, dl], nxr[rows, dl], nc[rows, dl] = xl, xr_left, cl
            nxl[rows, dr] = np.where(dr < K, z, nxl[rows, dr])
            nxr[rows, dr] = np.where(dr < K, xr, nxr[rows, dr])
            nc[rows, dr] = np.where(dr < K, cr, nc[rows, dr])
            cnt = np.minimum(ntot, K).astype(np.int32)
            keep = ks < cnt[:, None]
            xl = np.where(keep, nxl[:, :K], INF).astype(f32)
            xr = np.where(keep, nxr[:, :K], INF).astype(f32)
            cc = np.where(keep, nc[:, :K], f32(0.0)).astype(f32)
            A = b_ * A
    sh = (M, N, K)
    return (A.reshape(M, N), xl.reshape(sh), xr.reshape(sh), cc.reshape(sh), cnt.reshape(M, N),
            ovf.reshape(M, N))


def carry(I, u0, A, xl, xr, c, n, ovf, beta, theta, C):
    """triton_soft.py:113-140: the hit piece's offset (summed over the hit lanes, so -0.0 reads
    +0.0), end = A*u + c; overflow or not exactly one hit runs the chunk serially."""
    M, N = n.shape
    K = xl.shape[-1]
    u = np.array(u0, dtype=f32).reshape(N).copy()
    starts = np.empty((M, N), f32)
    for m in range(M):
        starts[m] = u
        hit = (np.arange(K)[None, :] < n[m][:, None]) & (xl[m] <= u[:, None]) & (u[:, None] < xr[m])
        k = np.argmax(hit, axis=1)
        cs = np.take_along_axis(c[m], k[:, None], 1)[:, 0] + f32(0.0)
        cs = np.where(hit.any(1), cs, f32(0.0)).astype(f32)
        nu = (A[m] * u + cs).astype(f32)
        bad = (ovf[m] > 0) | (hit.sum(1) != 1)
        if bad.any():
            w = serial_segment(I[m * C:(m + 1) * C], beta, theta, u)
            nu = np.where(bad, w, nu).astype(f32)
        u = nu
    return starts


def scan_forward(I, beta, theta, u0, C=32, K=16, repair=0, stats=None, keep=None):
    """triton_soft.py:175-211: envelopes -> build -> carry -> replay -> Jacobi repair; stats
    repair_iters, overflow_frac, mean_pieces, max_pieces."""
    I = np.ascontiguousarray(I, dtype=f32)
    T, N = I.shape
    assert T % C == 0
    M = T // C
    u0 = np.asarray(u0, dtype=f32).reshape(N)
    Lo, Hi = envelopes(I, beta, theta, u0, C)
    A, xl, xr, c, n, ovf = build_maps(I, Lo, Hi, beta, theta, C, K)
    starts = carry(I, u0, A, xl, xr, c, n, ovf, beta, theta, C)

    def replay(st):
        Ic = I.reshape(M, C, N)
        u = st.astype(f32).copy()
        U = np.empty((M, C, N), f32)
        S = np.empty((M, C, N), f32)
        for j in range(C):
            u, s = soft_step(u, Ic[:, j], beta, theta)
            U[:, j], S[:, j] = u, s
        return U.reshape(T, N), S.reshape(T, N), u

    U, S, ends = replay(starts)
    it = 0
    for it in range(1, repair + 1):
        new = np.concatenate([u0[None], ends[:-1]], 0)
        if np.array_equal(new, starts):
            it -= 1
            break
        starts = new
        U, S, ends = replay(starts)
    if stats is not None:
        stats["repair_iters"] = it
        stats["overflow_frac"] = float(ovf.astype(np.float64).mean())
        stats["mean_pieces"] = float(n.astype(np.float64).mean())
        stats["max_pieces"] = int(n.max())
    if keep is not None:
        keep.update(Lo=Lo, Hi=Hi, A=A, xl=xl, xr=xr, c=c, n=n, ovf=ovf, starts=starts)
    return U, S


def adjoint_fft(V, gS, beta, theta, alpha=4.0):
    """soft_adjoint_fft (triton_soft.py:214-221): b = gS*alpha*sg*(1 - sg) in fp32, sg =
    sigmoid(alpha*(V - theta)), then lam_t = b_t + beta*lam_{t+1} by a float64 FFT convolution
    with beta^k, cast to fp32."""
    V = np.asarray(V, f32)
    T = V.shape[0]
    al, th = _s(alpha), _s(theta)
    sg = (f32(1.0) / (f32(1.0) + np.exp(-(al * (V - th))))).astype(f32)
    b = (np.asarray(gS, f32) * al * sg * (f32(1.0) - sg)).astype(np.float64)
    k = float(beta) ** np.arange(T, dtype=np.float64)
    n = 2 * T
    lam = np.fft.irfft(np.fft.rfft(b[::-1], n=n, axis=0) * np.fft.rfft(k, n=n)[:, None], n=n,
                       axis=0)[:T][::-1]
    return lam.astype(f32)


def adjoint_direct64(V, gS, beta, theta, alpha=4.0):
    """The same recurrence solved directly in float64 (the FFT's exact value)."""
    V = np.asarray(V, f32)
    T, N = V.shape
    al, th = _s(alpha), _s(theta)
    sg = (f32(1.0) / (f32(1.0) + np.exp(-(al * (V - th))))).astype(f32)
    b = (np.asarray(gS, f32) * al * sg * (f32(1.0) - sg)).astype(np.float64)
    lam = np.zeros((T, N))
    nxt = np.zeros(N)
    for t in range(T - 1, -1, -1):
        nxt = b[t] + float(beta) * nxt
        lam[t] = nxt
    return lam
