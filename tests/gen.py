"""Deterministic synthetic inputs shared by tests and bench.py.

`fill` is the reference corpus generator: xorshift64 (13, 7, 17) seeded with
0x243F6A8885A308D3 ^ salt, one draw per element, value (s >> 33)
(crates/uor-matmul-validate/tests/massive.rs:42-53).  `draws` produces that
exact sequence for any length, split over parallel lanes whose start states
come from GF(2) jump-ahead, so multi-GiB fills take seconds.
"""
from __future__ import annotations

import numpy as np

SEED = 0x243F6A8885A308D3
M64 = (1 << 64) - 1


def xorshift_draws(n: int, salt: int) -> np.ndarray:
    """The reference's exact sequence of (s >> 33) draws (uint64), n of them."""
    s = (SEED ^ salt) & M64
    out = np.empty(n, dtype=np.uint64)
    for i in range(n):
        s ^= (s << 13) & M64
        s ^= s >> 7
        s ^= (s << 17) & M64
        out[i] = s >> 33
    return out


def _step_columns() -> np.ndarray:
    """One xorshift step is linear over GF(2)^64: column b is the image of bit b."""
    cols = []
    for b in range(64):
        s = 1 << b
        s ^= (s << 13) & M64
        s ^= s >> 7
        s ^= (s << 17) & M64
        cols.append(s)
    return np.array(cols, dtype=np.uint64)


def _apply(cols: np.ndarray, v: np.ndarray) -> np.ndarray:
    """The GF(2) matrix with these 64 columns times every state in v."""
    out = np.zeros_like(v)
    one = np.uint64(1)
    for b in range(64):
        out ^= cols[b] * ((v >> np.uint64(b)) & one)
    return out


def _power(cols: np.ndarray, e: int) -> np.ndarray:
    """The columns of the e-th power (e >= 0) by repeated squaring."""
    result = np.array([1 << b for b in range(64)], dtype=np.uint64)
    base = cols.copy()
    while e:
        if e & 1:
            result = _apply(base, result)
        base = _apply(base, base)
        e >>= 1
    return result


def draws(n: int, salt: int, lanes: int = 1 << 16) -> np.ndarray:
    """xorshift_draws(n, salt) exactly, computed in parallel: lane i starts
    at state M^(i*L) s0 (M the step, L = ceil(n / lanes), the start states by
    GF(2) jump-ahead) and produces draws i*L .. i*L + L - 1."""
    if n <= 0:
        return np.empty(0, dtype=np.uint64)
    lanes = max(1, min(lanes, n))
    L = (n + lanes - 1) // lanes
    jump = _power(_step_columns(), L)
    starts = np.array([(SEED ^ salt) & M64], dtype=np.uint64)
    while starts.size < lanes:
        starts = np.concatenate([starts, _apply(jump, starts)])
        jump = _apply(jump, jump)
    s = starts[:lanes].copy()
    out = np.empty((L, lanes), dtype=np.uint64)
    sh13, sh7, sh17, sh33 = np.uint64(13), np.uint64(7), np.uint64(17), np.uint64(33)
    for r in range(L):
        s ^= s << sh13
        s ^= s >> sh7
        s ^= s << sh17
        out[r] = s >> sh33
    return np.ascontiguousarray(out.T).reshape(-1)[:n]


def i8_full(n: int, salt: int) -> np.ndarray:
    """Uniform over all 256 i8 values: (s >> 33) as u8 as i8."""
    return (draws(n, salt) & np.uint64(0xFF)).astype(np.uint8).view(np.int8)


def i32_pm2_20(n: int, salt: int) -> np.ndarray:
    """Uniform i32 in [-2^20, 2^20]: (s >> 33) mod (2^21 + 1) - 2^20."""
    d = draws(n, salt)
    return ((d % np.uint64((1 << 21) + 1)).astype(np.int64) - (1 << 20)).astype(np.int32)


# ------------------------------------------------------------ float inputs --

def float_config4(rows: int, cols: int, is64: bool, salt: int) -> np.ndarray:
    """BASELINE configs[3] entries: random sign x significand uniform in [1, 2)
    x 2^e, e uniform over [-40, 40] (f32) or [-300, 300] (f64), with 1% exact
    zeros.  Built from IEEE fields so no host rounding is involved."""
    n = rows * cols
    d1 = draws(n, salt)
    d2 = draws(n, salt + 0x5151)
    span = 300 if is64 else 40
    mant_bits, bias = (52, 1023) if is64 else (23, 127)
    e = (d1 % np.uint64(2 * span + 1)).astype(np.int64) - span
    sign = (d1 >> np.uint64(20)) & np.uint64(1)
    frac = ((d2 << np.uint64(31)) ^ d1) & np.uint64((1 << mant_bits) - 1)
    zero = (d2 >> np.uint64(9)) % np.uint64(100) == 0
    bits = (sign << np.uint64(63 if is64 else 31)) | (((e + bias).astype(np.uint64)) << np.uint64(mant_bits)) | frac
    bits[zero] = 0
    if is64:
        return bits.view(np.float64).reshape(rows, cols)
    return bits.astype(np.uint32).view(np.float32).reshape(rows, cols)


def cancel_pairs(a: np.ndarray, b: np.ndarray, salt: int, frac: float = 0.01):
    """Make 1% of the reduction index pairs cancel exactly: for a chosen
    disjoint pair (p, q), column q of A is minus column p and row q of B
    equals row p, so A[i,p]*B[p,j] + A[i,q]*B[q,j] = 0 for every i, j."""
    k = a.shape[1]
    npairs = max(1, int(k * frac)) if k >= 2 else 0
    perm = np.argsort(draws(k, salt), kind="stable")
    for t in range(npairs):
        p, q = int(perm[2 * t]), int(perm[2 * t + 1])
        a[:, q] = -a[:, p]
        b[q, :] = b[p, :]
    return a, b


# The reference's float corpus (crates/uor-matmul-validate/src/float_corpus.rs:
# 17-330): structural fills built from IEEE fields with a splitmix finaliser.
FILLS = ["OneGrade", "FewGrades", "InverseGauge", "FullFiniteRange", "Boundaries", "NonFinite",
         "SparseSignificand", "DenseSignificand"]
CORRECTNESS_CASES = [  # float_corpus.rs:53-117: (m, k, n, fill, seed)
    (0, 3, 2, "OneGrade", 1), (2, 0, 3, "Boundaries", 2), (1, 17, 1, "FullFiniteRange", 3),
    (3, 5, 7, "FewGrades", 4), (5, 33, 4, "InverseGauge", 5), (4, 19, 3, "Boundaries", 6),
    (3, 23, 4, "NonFinite", 7), (7, 31, 5, "SparseSignificand", 8),
    (7, 31, 5, "DenseSignificand", 9)]
PERFORMANCE_CASES = [  # float_corpus.rs:124-167
    (1, 1, 1, "OneGrade", 101), (32, 32, 32, "FewGrades", 102), (16, 128, 16, "InverseGauge", 103),
    (7, 31, 5, "FullFiniteRange", 104), (1, 65536, 1, "DenseSignificand", 105),
    (128, 8, 128, "SparseSignificand", 106)]


def _mix(x: int) -> int:
    x ^= x >> 30
    x = (x * 0xBF58476D1CE4E5B9) & M64
    x ^= x >> 27
    x = (x * 0x94D049BB133111EB) & M64
    return x ^ (x >> 31)


def _corpus_code(is64, fill, seed, side, outer, p):
    fb, eb = (52, 11) if is64 else (23, 8)
    salt = 0xA24BAED4963EE407 if side == "A" else 0x9FB21C651E98DF25
    r = _mix((seed ^ salt ^ ((outer * 0xD6E8FEB86659FD93) & M64)
              ^ ((p * 0xA5A3564E27F8862D) & M64)) & M64)
    frac_mask = (1 << fb) - 1
    emax = (1 << eb) - 1
    bias = emax >> 1
    sign = (r >> 63) << (fb + eb)
    if fill == "OneGrade":
        e, f = bias, r & frac_mask
    elif fill == "FewGrades":
        e, f = bias + (r % 7) - 3, r & frac_mask
    elif fill == "InverseGauge":
        radius = max(emax // 8, 1)
        delta = (p % (2 * radius + 1)) - radius
        e, f = bias + (delta if side == "A" else -delta), r & frac_mask
    elif fill == "FullFiniteRange":
        e, f = 1 + r % (emax - 1), r & frac_mask
    elif fill == "Boundaries":
        e, f = [(0, 0), (0, 1), (0, frac_mask), (1, 0), (bias, 0), (emax - 1, frac_mask)][min(r % 6, 5)]
    elif fill == "NonFinite":
        e, f = [(0, 0), (emax, 0), (emax, 1), (emax, frac_mask), (bias, r & frac_mask),
                (bias, r & frac_mask)][r % 6]
    elif fill == "SparseSignificand":
        e, f = bias, 1 << ((r & 0xFFFFFFFF) % fb)
    elif fill == "DenseSignificand":
        e, f = bias, frac_mask ^ (1 << (r % fb))
    else:
        raise ValueError(fill)
    return sign | (e << fb) | f


def corpus_operands(case, is64):
    """float_corpus::operands: row-major A (m x k) and B (k x n); B's code for
    (p, j) is drawn with outer = j."""
    m, k, n, fill, seed = case
    ut = np.uint64 if is64 else np.uint32
    ft = np.float64 if is64 else np.float32
    a = np.array([_corpus_code(is64, fill, seed, "A", i, p) for i in range(m) for p in range(k)],
                 dtype=ut).view(ft)
    b = np.array([_corpus_code(is64, fill, seed, "B", j, p) for p in range(k) for j in range(n)],
                 dtype=ut).view(ft)
    return a, b
