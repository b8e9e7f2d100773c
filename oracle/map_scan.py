"""CPU oracle of the associative carry of the two-level scan (k_map_scan) — TEST INFRASTRUCTURE
ONLY.  Only tests/ may import it, as the checker; the product never calls into oracle/.

The chunk maps of one neuron are composed with a parallel prefix in a fixed association order:
64 chunks per wave, an inclusive scan inside the wave in the order of the DPP moves
(row_shr 1, 2, 4, 8 within 16-lane rows, then the last lane of rows 0 / 2 into rows 1 / 3,
then lane 31 into rows 2 / 3; every lane reads its source's value from before the level), the
wave totals composed the same way, then every chunk's entry state is its prefix map evaluated
at the tile's entry state.  The composition is the reference's monoid (triton_lif.py:864-892,
compose_group_kernel; exact.py:108-131); the envelope maps compose as min-affine maps
(triton_lif.py:699-733).  fp32 arithmetic with every operation rounded (numpy float32 scalars),
in the kernel's order.  Per neuron, in Python: for small test sizes only.
"""
import numpy as np

from oracle.lif_oracle import serial_segment

f32 = np.float32
INF = f32(np.inf)
KS = 32          # breakpoint capacity of a composed map
HEAD, BAD = 1, 2
WAVE = 64


class Elem:
    """Map over a run of chunks: u -> A*u + B below the smallest breakpoint, else the constant
    of the piece (slots: (breakpoint, constant), breakpoints descending); lo: the domain's lower
    bound; flags HEAD (starts at an overflowed chunk's exit) / BAD (capacity exceeded)."""

    __slots__ = ("A", "B", "lo", "slots", "flags")

    def __init__(self, A, B, lo, slots, flags):
        self.A, self.B, self.lo, self.slots, self.flags = A, B, lo, slots, flags


def identity(lo=-INF):
    return Elem(f32(1.0), f32(0.0), f32(lo), [], 0)


def count_gt(slots, u):
    return sum(1 for x, _ in slots if x > u)


def evaluate(e, u):
    """Map evaluation (triton_lif.py:592-599): k = #{xd > u}; k == n -> A*u + B, else cd[k]."""
    k = count_gt(e.slots, u)
    if k == len(e.slots):
        return f32(f32(e.A * u) + e.B)
    return e.slots[k][1]


def compose(H, g, hi):
    """g after H (H first), or g itself when it starts at an overflowed chunk
    (triton_lif.py:864-892): H's constants pushed through g; g's breakpoints pulled back
    through H's affine part, kept iff below the current smallest breakpoint, <= hi, while that
    one is above H's lower bound, at most KS in all; A = Ag*A, B = Ag*B + Bg."""
    if g.flags & HEAD:
        return g
    out = []
    xmin = INF
    for hx, hc in H.slots:
        out.append((hx, evaluate(g, hc)))
        xmin = hx
    flags = H.flags | (g.flags & BAD)
    for gx, gc in g.slots:
        num = f32(gx - H.B)
        if H.A == 0:
            z = INF if num > 0 else -INF
        else:
            with np.errstate(over="ignore", divide="ignore", invalid="ignore"):
                z = f32(num / H.A)
        if z < xmin and z <= hi and xmin > H.lo:
            if len(out) >= KS:
                flags |= BAD
            else:
                out.append((z, gc))
                xmin = z
    return Elem(f32(g.A * H.A), f32(f32(g.A * H.B) + g.B), H.lo, out, flags)


def env_after(e1, e2):
    """Envelope map (c2, a2, b2) after (c1, a1, b1): l -> min(c, a*l + b)."""
    c1, a1, b1 = e1
    c2, a2, b2 = e2
    return (min(c2, f32(f32(a2 * c1) + b2)), f32(a2 * a1), f32(f32(a2 * b1) + b2))


def env_apply(e, l):
    c, a, b = e
    return min(c, f32(f32(a * l) + b))


def _sources(level, lane):
    """DPP source lane of `lane` at one level of the wave scan, or None."""
    kind, d = level
    row = lane // 16
    if kind == "shr":
        return lane - d if lane % 16 >= d else None
    if kind == "bcast15":
        return 16 * row - 1 if row in (1, 3) else None
    return 31 if row in (2, 3) else None


LEVELS = [("shr", 1), ("shr", 2), ("shr", 4), ("shr", 8), ("bcast15", 15), ("bcast31", 31)]


def wave_scan(vals, combine, active=None):
    """Inclusive scan of 64 lane values in the DPP order; combine(earlier, later)."""
    vals = list(vals)
    for lev in LEVELS:
        new = list(vals)
        for l in range(WAVE):
            src = _sources(lev, l)
            if src is None or (active is not None and not active[l]):
                continue
            new[l] = combine(vals[src], vals[l])
        vals = new
    return vals


def map_scan_carry(EC, EA, EB, MA, MB, CNT, OVFRAW, MX, MC, I, u0, beta, theta, u_r, C, WG,
                   margin=1e-5):
    """Chunk entry states of the associative carry -> (LO, MN, OVF, STARTS) [M, N], as
    k_map_scan computes them from the single-read build's arrays (EC/EA/EB envelope maps,
    MA/MB/CNT/OVFRAW/MX/MC hi-pruned maps, MX/MC [M, K, N])."""
    M, N = EC.shape
    K = MX.shape[1]
    th, ur, mg = f32(theta), f32(u_r), f32(margin)
    LO = np.zeros((M, N), f32)
    MN = np.zeros((M, N), np.int32)
    OVF = np.zeros((M, N), np.int32)
    STARTS = np.zeros((M, N), f32)
    tile = WAVE * WG
    for n in range(N):
        hi = max(f32(u0[n]), max(th, ur))
        s_state = f32(u0[n])
        env_in = f32(u0[n])
        for m0 in range(0, M, tile):
            ms = [m0 + t for t in range(tile)]
            valid = [m < M for m in ms]
            # 1. envelope bounds
            envs = [(EC[m, n], EA[m, n], EB[m, n]) if v else (INF, f32(1.0), f32(0.0))
                    for m, v in zip(ms, valid)]
            incl = []
            tot = []
            for w in range(WG):
                sc = wave_scan(envs[w * WAVE:(w + 1) * WAVE], env_after)
                incl += sc
                tot.append(sc[-1])
            lo = []
            l_exit = []
            for w in range(WG):
                lw = env_in
                for v in range(w):
                    lw = env_apply(tot[v], lw)
                for lane in range(WAVE):
                    le = env_apply(incl[w * WAVE + lane], lw)
                    lin = lw if lane == 0 else l_exit[w * WAVE + lane - 1]
                    l_exit.append(le)
                    lo.append(f32(lin - f32(mg * f32(abs(lin) + f32(1.0)))))
            # 2. truncated chunk maps
            elems = []
            ovfs = []
            for t, m in enumerate(ms):
                if not valid[m - m0]:
                    elems.append(identity(lo[t]))
                    ovfs.append(False)
                    continue
                cnt = int(CNT[m, n])
                sl = [(MX[m, i, n], MC[m, i, n]) for i in range(min(cnt, K))]
                gt = sum(1 for x, _ in sl if x > lo[t])
                ne = min(cnt, gt + 1)
                ov = bool(OVFRAW[m, n]) and gt == cnt
                LO[m, n], MN[m, n], OVF[m, n] = lo[t], ne, int(ov)
                if ov:
                    elems.append(Elem(f32(1.0), f32(0.0), -INF, [], HEAD))
                else:
                    elems.append(Elem(MA[m, n], MB[m, n], lo[t], sl[:ne], 0))
                ovfs.append(ov)
            # 3. wave scans, totals scan
            comb = lambda a, b: compose(a, b, hi)
            scanned = []
            tflags = 0
            for w in range(WG):
                sc = wave_scan(elems[w * WAVE:(w + 1) * WAVE], comb)
                scanned += sc
                for e in sc:
                    tflags |= e.flags
            prefix = [None] * WG
            if WG > 1:
                tv = [scanned[j * WAVE + WAVE - 1] if j < WG - 1 else identity()
                      for j in range(WAVE)]
                ts = wave_scan(tv, comb, active=[j < WG - 1 for j in range(WAVE)])
                for j in range(WG - 1):
                    prefix[j + 1] = ts[j]
                    tflags |= ts[j].flags
            # 4. entry states
            after = [f32(0.0)] * tile
            if tflags == 0:
                for w in range(WG):
                    s_w = s_state if w == 0 else evaluate(prefix[w], s_state)
                    for lane in range(WAVE):
                        t = w * WAVE + lane
                        if valid[t]:
                            after[t] = evaluate(scanned[t], s_w)
            elif not (tflags & BAD):
                for w in range(WG):
                    s_w = s_state if w == 0 else after[w * WAVE - 1]
                    wa = [f32(0.0) if scanned[w * WAVE + l].flags & HEAD
                          else evaluate(scanned[w * WAVE + l], s_w) for l in range(WAVE)]
                    heads = [l for l in range(WAVE) if valid[w * WAVE + l] and ovfs[w * WAVE + l]]
                    for hidx, h in enumerate(heads):
                        sh = s_w if h == 0 else wa[h - 1]
                        m = ms[w * WAVE + h]
                        xh = serial_segment(I[m * C:(m + 1) * C, n:n + 1], beta, theta, u_r,
                                            np.array([sh], f32))[0]
                        h2 = heads[hidx + 1] if hidx + 1 < len(heads) else WAVE
                        for l in range(h, h2):
                            wa[l] = evaluate(scanned[w * WAVE + l], xh)
                    for l in range(WAVE):
                        if valid[w * WAVE + l]:
                            after[w * WAVE + l] = wa[l]
            else:
                u = s_state
                for t, m in enumerate(ms):
                    if not valid[t]:
                        break
                    cnt = int(CNT[m, n])
                    sl = [(MX[m, i, n], MC[m, i, n]) for i in range(min(cnt, K))]
                    gt = sum(1 for x, _ in sl if x > lo[t])
                    ne = min(cnt, gt + 1)
                    if OVFRAW[m, n] and gt == cnt:
                        u = serial_segment(I[m * C:(m + 1) * C, n:n + 1], beta, theta, u_r,
                                           np.array([u], f32))[0]
                    else:
                        u = evaluate(Elem(MA[m, n], MB[m, n], lo[t], sl[:ne], 0), u)
                    after[t] = u
            for t, m in enumerate(ms):
                if valid[t]:
                    STARTS[m, n] = s_state if t == 0 else after[t - 1]
            last = min(M - m0, tile) - 1
            s_state = after[last]
            env_in = l_exit[last]
    return LO, MN, OVF, STARTS
