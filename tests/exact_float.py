"""An exact float GEMM in Python rationals, written independently of the C
oracle: the sum is a Fraction, and the rounding picks among IEEE neighbours
by exact comparison (round-half-even for Nearest; the largest magnitude not
above |v| for the directed modes) instead of reading a bit window.  Used to
pin oracle/uor_oracle.c's ora_gemm_float on small cases."""
from __future__ import annotations

import math
from fractions import Fraction

import numpy as np

FMT = {False: (np.float32, np.uint32, 23, 8), True: (np.float64, np.uint64, 52, 11)}


def _max_finite(is64):
    return Fraction(np.finfo(np.float64 if is64 else np.float32).max.item())


def round_fraction(v: Fraction, is64: bool, mode: str, negative_hint: bool = False):
    """Round the exact v to f32/f64 bits under `mode`."""
    ft, ut, mant, _ = FMT[is64]
    if v == 0:
        return ut(0)
    neg = v < 0
    av = -v if neg else v
    mx = _max_finite(is64)
    ulp_max = Fraction(2) ** ((1023 if is64 else 127) - mant)
    if av > mx:
        if mode == "nearest" and av >= mx + ulp_max / 2:
            out = np.array(np.inf, dtype=ft)
        elif mode == "nearest":
            out = np.array(mx, dtype=ft)
        else:
            out = np.array(mx, dtype=ft)
        return (-out if neg else out).view(ut)
    # A candidate close to |v|, then the exact neighbours around it.
    try:
        approx = float(av)
    except OverflowError:
        approx = float(mx)
    c = ft(approx)
    cands = {c}
    lo = hi = c
    for _ in range(3):
        lo = np.nextafter(lo, ft(0))
        hi = np.nextafter(hi, ft(np.inf))
        cands.update([lo, hi])
    cands = [x for x in cands if np.isfinite(x) and x >= 0]
    below = max((x for x in cands if Fraction(x.item()) <= av), key=lambda x: Fraction(x.item()))
    if mode != "nearest" or Fraction(below.item()) == av:
        pick = below
    else:
        above = np.nextafter(below, ft(np.inf))
        if not np.isfinite(above):
            pick = above  # past MAX: handled above, kept for completeness
        else:
            db = av - Fraction(below.item())
            da = Fraction(above.item()) - av
            if db < da:
                pick = below
            elif da < db:
                pick = above
            else:
                pick = below if (int(np.array(below).view(ut)) & 1) == 0 else above
    out = np.array(pick, dtype=ft)
    if neg:
        out = -out  # also gives -0.0 for a negative value that rounds to zero
    return out.view(ut)


def _cls(x: float):
    if math.isnan(x):
        return "nan"
    if math.isinf(x):
        return "+inf" if x > 0 else "-inf"
    return "fin"


def gemm_float(a, b, c0, m, k, n, alpha=1, beta=0, mode="nearest"):
    """a (m x k), b (k x n), c0 (m x n) row-major numpy float arrays of one
    dtype; returns the output bits (uint32/uint64) row-major."""
    is64 = a.dtype == np.float64
    ft, ut, _, _ = FMT[is64]
    nan_bits = ut(0x7FF8000000000000 if is64 else 0x7FC00000)
    inf = {"+": np.array(np.inf, dtype=ft).view(ut), "-": np.array(-np.inf, dtype=ft).view(ut)}
    A = a.reshape(m, k).astype(np.float64)
    B = b.reshape(k, n).astype(np.float64)
    C = c0.reshape(m, n).astype(np.float64)
    out = np.zeros((m, n), dtype=ut)
    for i in range(m):
        for j in range(n):
            s = Fraction(0)
            nan = pinf = ninf = False
            for p in range(k):
                x, y = A[i, p].item(), B[p, j].item()
                cx, cy = _cls(x), _cls(y)
                if cx == "nan" or cy == "nan":
                    nan = True
                elif cx != "fin" or cy != "fin":
                    if x == 0 or y == 0:
                        nan = True
                    elif (x < 0) != (y < 0):
                        ninf = True
                    else:
                        pinf = True
                else:
                    s += Fraction(x) * Fraction(y)

            def scale(val, nan, pinf, ninf, f):
                if nan or (pinf and ninf):
                    return val, True, False, False
                if f == 0:
                    return Fraction(0), (pinf or ninf), False, False
                if f < 0:
                    pinf, ninf = ninf, pinf
                return val * f, False, pinf, ninf

            s, nan, pinf, ninf = scale(s, nan, pinf, ninf, alpha)
            if beta != 0:
                cv = C[i, j].item()
                cc = _cls(cv)
                g = (Fraction(0), cc == "nan", cc == "+inf", cc == "-inf")
                if cc == "fin":
                    g = (Fraction(cv), False, False, False)
                gv, gn, gp, gm = scale(*g, beta)
                s += gv
                nan, pinf, ninf = nan or gn, pinf or gp, ninf or gm
            if nan or (pinf and ninf):
                out[i, j] = nan_bits
            elif pinf:
                out[i, j] = inf["+"]
            elif ninf:
                out[i, j] = inf["-"]
            else:
                out[i, j] = round_fraction(s, is64, mode)
    return out.reshape(-1)
