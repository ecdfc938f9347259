"""Pins the integer oracle (driver::gemm + Linear + encode) independently.

Witnesses: the reference's committed CX-10 fixtures (oracles/numpy: NumPy int64
matmul, Wrapping, sha256-checked), NumPy int64 matmul over i8 (exact), Python
integers for the encode rules, and the reference's inline known answers.
"""
import hashlib
import json

import numpy as np
import pytest
from numpy.lib.stride_tricks import as_strided

from conftest import GOLDEN

I32_MIN, I32_MAX = -(1 << 31), (1 << 31) - 1


def run(oracle, a, am, ak, ars, acs, b, bk, bn, brs, bcs, c, crs, ccs, **kw):
    st = oracle.gemm_int(a, (am, ak), (ars, acs), b, (bk, bn), (brs, bcs), c, (am, bn),
                         (crs, ccs), **kw)
    return st


def test_readme_example(oracle):
    a = np.array([1, 2, 3, 4], np.int8)
    b = np.array([5, 6, 7, 8], np.int8)
    c = np.zeros(4, np.int32)
    assert run(oracle, a, 2, 2, 2, 1, b, 2, 2, 2, 1, c, 2, 1) == "ok"
    assert c.tolist() == [19, 22, 43, 50]  # README.md:38-39


def test_alpha_beta_cs05(oracle):
    a = np.array([1, 2, 3, 4], np.int8)
    b = np.array([5, 6, 7, 8], np.int8)
    c = np.array([100, 200, 300, 400], np.int32)
    run(oracle, a, 2, 2, 2, 1, b, 2, 2, 2, 1, c, 2, 1, alpha=3, beta=-2)
    assert c.tolist() == [3 * 19 - 200, 3 * 22 - 400, 3 * 43 - 600, 3 * 50 - 800]


def test_transposed_strides_cs06(oracle):
    a = np.array([1, 2, 3, 4, 5, 6], np.int8)
    b = np.array([1, 2, 3, 4, 5, 6], np.int8)
    c = np.zeros(4, np.int32)
    run(oracle, a, 2, 3, 3, 1, b, 3, 2, 2, 1, c, 2, 1)
    assert c.tolist() == [22, 28, 49, 64]
    d = np.zeros(9, np.int32)
    run(oracle, a, 3, 2, 1, 3, b, 2, 3, 3, 1, d, 3, 1)
    assert d.tolist() == [17, 22, 27, 22, 29, 36, 27, 36, 45]


def test_encode_modes_cd05(oracle):
    # kernel.rs:2315-2386: 500*127^2 fits; 200000*127^2 wraps vs saturates.
    a = np.full(4 * 500, 127, np.int8)
    c = np.zeros(16, np.int32)
    run(oracle, a, 4, 500, 500, 1, a, 500, 4, 4, 1, c, 4, 1, encode="wrapping")
    assert c[0] == 500 * 127 * 127
    deep = 200_000
    a = np.full(deep, 127, np.int8)
    w = np.zeros(1, np.int32)
    s = np.zeros(1, np.int32)
    run(oracle, a, 1, deep, deep, 1, a, deep, 1, 1, 1, w, 1, 1, encode="wrapping")
    run(oracle, a, 1, deep, deep, 1, a, deep, 1, 1, 1, s, 1, 1, encode="saturating")
    assert w[0] == np.int64(deep * 127 * 127).astype(np.int32)
    assert s[0] == I32_MAX


@pytest.mark.parametrize("k", [150_000, 300_000])
def test_depth_past_every_lane_ct01(oracle, k):
    a = np.full(k, -128, np.int8)
    c64 = np.zeros(1, np.int64)
    run(oracle, a, 1, k, k, 1, a, k, 1, 1, 1, c64, 1, 1)
    assert c64[0] == k * 128 * 128
    c32 = np.zeros(1, np.int32)
    run(oracle, a, 1, k, k, 1, a, k, 1, 1, 1, c32, 1, 1, encode="wrapping")
    assert c32[0] == np.int64(k * 128 * 128).astype(np.int32)


def test_numpy_cx10_fixtures(oracle):
    d = GOLDEN / "numpy_cx10"
    man = json.loads((d / "manifest.json").read_text())
    assert man["id"] == "CX-10" and man["dtype"] == "int64"
    for case in man["cases"]:
        m, k, n = (case["shape"][x] for x in "mkn")
        blobs = {}
        for name in ("a", "b", "expected"):
            raw = (d / f"{case['stem']}.{name}.bin").read_bytes()
            assert "sha256:" + hashlib.sha256(raw).hexdigest() == case[f"{name}_sha256" if name != "expected" else "expected_sha256"]
            blobs[name] = np.frombuffer(raw, "<i8").copy()
        c = np.zeros(m * n, np.int64)
        if m and n:
            st = oracle.gemm_int(blobs["a"], (m, k), (k, 1), blobs["b"], (k, n), (n, 1), c,
                                 (m, n), (n, 1), encode="wrapping")
            assert st == "ok"
        assert np.array_equal(c, blobs["expected"]), case["stem"]


def strided(buf, rows, cols, rs, cs, origin):
    item = buf.itemsize
    return as_strided(buf[origin:], shape=(rows, cols), strides=(rs * item, cs * item))


def encode_py(v, bits, mode):
    mn, mx = -(1 << (bits - 1)), (1 << (bits - 1)) - 1
    if mode == "wrapping":
        return (v - mn) % (1 << bits) + mn
    return max(mn, min(mx, v))


@pytest.mark.parametrize("seed", range(6))
def test_random_views_match_numpy(oracle, seed):
    rng = np.random.default_rng(seed)
    for _ in range(25):
        m, k, n = (int(x) for x in rng.integers(0, 9, 3))
        def pick(rows, cols):
            rs = int(rng.choice([-1, 1])) * int(rng.integers(0, 3)) * max(cols, 1)
            cs = int(rng.choice([-1, 1])) * int(rng.integers(0, 2))
            if rng.random() < 0.3:
                rs, cs = cs, rs
            return rs, cs
        ars, acs = pick(m, k)
        brs, bcs = pick(k, n)
        a = rng.integers(-128, 128, size=3 * (m * k + 1) + 30).astype(np.int8)
        b = rng.integers(-128, 128, size=3 * (k * n + 1) + 30).astype(np.int8)
        ao = oracle.place(a.size, m, k, ars, acs)
        bo = oracle.place(b.size, k, n, brs, bcs)
        if ao is None or bo is None:
            continue
        c = rng.integers(-1000, 1000, size=m * n).astype(np.int32)
        alpha, beta = int(rng.integers(-5, 6)), int(rng.integers(-5, 6))
        A = strided(a, m, k, ars, acs, ao).astype(np.int64) if m and k else np.zeros((m, k), np.int64)
        B = strided(b, k, n, brs, bcs, bo).astype(np.int64) if k and n else np.zeros((k, n), np.int64)
        want = alpha * (A @ B) + (beta * c.reshape(m, n).astype(np.int64) if beta else 0)
        st = oracle.gemm_int(a, (m, k), (ars, acs), b, (k, n), (brs, bcs), c, (m, n), (n, 1),
                             alpha=alpha, beta=beta)
        assert st == "ok"
        assert np.array_equal(c.reshape(m, n), np.vectorize(lambda v: encode_py(int(v), 32, "nearest"))(want).astype(np.int32) if m and n else c.reshape(m, n))


@pytest.mark.parametrize("out,bits", [(np.int8, 8), (np.int16, 16), (np.int32, 32), (np.int64, 64)])
@pytest.mark.parametrize("mode", ["nearest", "saturating", "toward_zero", "wrapping"])
def test_encode_rules_against_python_ints(oracle, out, bits, mode):
    rng = np.random.default_rng(bits)
    m, k, n = 5, 300, 6
    a = rng.integers(-128, 128, m * k).astype(np.int8)
    b = rng.integers(-128, 128, k * n).astype(np.int8)
    c0 = rng.integers(np.iinfo(out).min, np.iinfo(out).max, m * n, dtype=out, endpoint=True)
    for alpha, beta in [(1, 0), (7, -3), (-(1 << 40), 1 << 33), (1 << 62, -(1 << 62))]:
        c = c0.copy()
        assert oracle.gemm_int(a, (m, k), (k, 1), b, (k, n), (n, 1), c, (m, n), (n, 1),
                               alpha=alpha, beta=beta, encode=mode) == "ok"
        S = a.reshape(m, k).astype(object) @ b.reshape(k, n).astype(object)
        for idx in range(m * n):
            v = alpha * int(S.flat[idx]) + (beta * int(c0[idx]) if beta else 0)
            assert int(c[idx]) == encode_py(v, bits, mode), (alpha, beta, idx)


def test_beta_zero_never_reads_c(oracle):
    rng = np.random.default_rng(1)
    a = rng.integers(-128, 128, 12).astype(np.int8)
    c1 = np.full(9, 0x5A5A5A5A, np.int32)
    c2 = np.full(9, -1, np.int32)
    for c in (c1, c2):
        oracle.gemm_int(a, (3, 4), (4, 1), a, (4, 3), (3, 1), c, (3, 3), (3, 1), alpha=2, beta=0)
    assert np.array_equal(c1, c2)


def test_errors(oracle):
    a = np.zeros(12, np.int8)
    c = np.zeros(16, np.int32)
    assert oracle.gemm_int(a, (3, 4), (4, 1), a, (3, 4), (4, 1), c, (3, 4), (4, 1)) == "nonconformant"
    assert oracle.gemm_int(a, (3, 4), (4, 1), a, (4, 3), (3, 1), c, (3, 3), (1, 1)) == "output_aliases_itself"
    assert oracle.gemm_int(a, (3, 5), (5, 1), a, (5, 3), (3, 1), c, (3, 3), (3, 1)) == "short_buffer"


def test_wrapping_narrow_output_is_the_modular_lane(oracle):
    """gemm_packed_impl (kernel.rs:566-607): Wrapping into at most 32 bits
    runs the Z/2^32 lane and scales the lane's value, so alpha * X never
    saturates; wider outputs, or other encodes, scale the exact X with
    saturating_mul.  Closed form: i32 elements all 2^31 - 1, k = 8, so
    X = 8 (2^31 - 1)^2 = 2^65 - 2^35 + 8 and X mod 2^32 = 8; alpha = 2^63 - 1:
      Wrapping -> i32, i16: 8 (2^63 - 1) = 2^66 - 8, which wraps to -8
      Wrapping -> i64: alpha * X >= 2^127 saturates to i128::MAX, wraps to -1
      Nearest  -> i32: saturates to i32::MAX.
    (Scaling the exact X would give -1 for the narrow outputs too.)"""
    k = 8
    a = np.full(k, (1 << 31) - 1, np.int32)
    cases = [("wrapping", np.int32, -8), ("wrapping", np.int64, -1),
             ("nearest", np.int32, (1 << 31) - 1), ("wrapping", np.int16, -8)]
    for mode, dt, want in cases:
        c = np.zeros(1, dt)
        assert oracle.gemm_int(a, (1, k), (k, 1), a, (k, 1), (1, 1), c, (1, 1), (1, 1),
                               alpha=(1 << 63) - 1, encode=mode) == "ok"
        assert int(c[0]) == want, (mode, dt)
    # beta scales C in the same way on both routes: C = 3, beta = 2^62.
    c = np.array([3], np.int32)
    assert oracle.gemm_int(a, (1, k), (k, 1), a, (k, 1), (1, 1), c, (1, 1), (1, 1),
                           alpha=1, beta=1 << 62, encode="wrapping") == "ok"
    assert int(c[0]) == 8  # 8 + 3 * 2^62 mod 2^32


# ---------------------------------------------------------------------------
# Python-integer witnesses: the reference's integer epilogue written with
# unbounded integers and explicit register widths, independent of the C
# oracle's limb arithmetic.

def _clamp(v, bits):
    lo, hi = -(1 << (bits - 1)), (1 << (bits - 1)) - 1
    return lo if v < lo else hi if v > hi else v


def _wrap(v, bits):
    v &= (1 << bits) - 1
    return v - (1 << bits) if v >> (bits - 1) else v


def py_finish(x, prior, alpha, beta, elem_bytes, out_bytes, mode):
    """Linear::finish (epilogue.rs:80-95) and the one encode, for one cell.
    i8/i16/i32 elements: the i128 register, saturating_mul then a wrapping
    add (epilogue.rs:280-289, acc.rs:101-105); Wrapping into at most 32 bits
    first reduces the sum to the Z/2^32 lane (kernel.rs:566-607).  i64
    elements: Limbs<3>, every step mod 2^192 (epilogue.rs:307-328,
    acc.rs:208-215).  Encode: Wrapping truncates, the other modes clamp
    (acc.rs:128-150, 405-442)."""
    ob = 8 * out_bytes
    if elem_bytes == 8:
        total = _wrap(x * alpha + (prior * beta if beta else 0), 192)
    else:
        if mode == "wrapping" and out_bytes <= 4:
            x = _wrap(x, 32)
        total = _clamp(x * alpha, 128)
        if beta:
            total = _wrap(total + _clamp(prior * beta, 128), 128)
    return _wrap(total, ob) if mode == "wrapping" else _clamp(total, ob)


def py_gemm(a, b, c0, alpha, beta, elem_bytes, out_bytes, mode):
    m, k = a.shape
    n = b.shape[1]
    out = []
    for i in range(m):
        for j in range(n):
            x = sum(int(a[i, p]) * int(b[p, j]) for p in range(k))
            out.append(py_finish(x, int(c0[i * n + j]), alpha, beta, elem_bytes, out_bytes, mode))
    return out


def _c_ints(c, out_bytes):
    if out_bytes == 16:
        v = c.view(np.uint64).reshape(-1, 2)
        return [_wrap(int(lo) | (int(hi) << 64), 128) for lo, hi in v]
    return [int(x) for x in c]


OUT_DT = {1: np.int8, 2: np.int16, 4: np.int32, 8: np.int64}


@pytest.mark.parametrize("elem_bytes", [2, 4, 8])
@pytest.mark.parametrize("out_bytes", [1, 2, 4, 8, 16])
@pytest.mark.parametrize("mode", ["nearest", "saturating", "toward_zero", "wrapping"])
def test_full_range_elements_against_python_ints(oracle, elem_bytes, out_bytes, mode):
    """ora_gemm_int at i16/i32/i64 elements over full-range operands (the
    extremes planted), every output width and encode, alpha/beta from 1/0 to
    the i64 extremes, against the Python-integer restatement above."""
    et = {2: np.int16, 4: np.int32, 8: np.int64}[elem_bytes]
    info = np.iinfo(et)
    rng = np.random.default_rng(1000 * elem_bytes + 10 * out_bytes + len(mode))
    m, k, n = 3, 5, 4
    a = rng.integers(info.min, info.max, (m, k), dtype=et, endpoint=True)
    b = rng.integers(info.min, info.max, (k, n), dtype=et, endpoint=True)
    a[0, :] = info.min
    b[:, 0] = info.min
    a[1, 0] = info.max
    for alpha, beta in [(1, 0), (3, -1), (-(1 << 63), (1 << 63) - 1), ((1 << 62) + 3, -(1 << 40)),
                        (0, 1), (-1, -(1 << 63))]:
        if out_bytes == 16:
            c0 = rng.integers(-(1 << 62), 1 << 62, 2 * m * n, dtype=np.int64)
            c0.view(np.uint64)[1::2] = np.where(rng.random(m * n) < 0.5, 0, ~np.uint64(0))
        else:
            oi = np.iinfo(OUT_DT[out_bytes])
            c0 = rng.integers(oi.min, oi.max, m * n, dtype=OUT_DT[out_bytes], endpoint=True)
        prior = _c_ints(c0, out_bytes)
        want = [py_finish(sum(int(a[i, p]) * int(b[p, j]) for p in range(k)), prior[i * n + j],
                          alpha, beta, elem_bytes, out_bytes, mode)
                for i in range(m) for j in range(n)]
        c = c0.copy()
        assert oracle.gemm_int(a.reshape(-1), (m, k), (k, 1), b.reshape(-1), (k, n), (n, 1), c,
                               (m, n), (n, 1), alpha=alpha, beta=beta, encode=mode,
                               out_bytes=out_bytes) == "ok"
        assert _c_ints(c, out_bytes) == want, (alpha, beta)


def test_i64_register_wraps_mod_2_192(oracle):
    """Limbs<3> holds 192 bits and does not grow (acc.rs:208-215): with every
    element i64::MIN and k = 2^20 the exact sum is 2^20 * 2^126 = 2^146, and
    scale_exact(alpha) works in that register.  alpha = 2^46 gives 2^192,
    which is 0; alpha = 2^45 gives 2^191, the register's most negative value,
    so every clamping encode gives O::MIN; alpha = 2^44 gives 2^190 (O::MAX);
    and beta * C adds mod 2^192 as well."""
    k = 1 << 20
    a = np.full(k, np.iinfo(np.int64).min, np.int64)
    for alpha, out_dt, mode, want in [
            (1 << 46, np.int64, "nearest", 0), (1 << 45, np.int64, "nearest", -(1 << 63)),
            (1 << 45, np.int32, "saturating", -(1 << 31)), (1 << 44, np.int64, "toward_zero", (1 << 63) - 1),
            (1 << 46, np.int16, "wrapping", 0), (3, np.int64, "wrapping", 0)]:
        c = np.zeros(1, out_dt)
        assert oracle.gemm_int(a, (1, k), (k, 1), a, (k, 1), (1, 1), c, (1, 1), (1, 1),
                               alpha=alpha, encode=mode) == "ok"
        assert int(c[0]) == want, (alpha, out_dt, mode)
    # 2^191 + C * beta with C = i64::MIN, beta = i64::MIN: 2^191 + 2^126, still
    # negative in the register; with beta = -i64::MAX instead: 2^191 - (2^63 - 1)
    # * (-2^63) = 2^191 + 2^126 - 2^63.  Both clamp to i64::MIN.
    for beta in (-(1 << 63), -((1 << 63) - 1)):
        c = np.array([np.iinfo(np.int64).min], np.int64)
        assert oracle.gemm_int(a, (1, k), (k, 1), a, (k, 1), (1, 1), c, (1, 1), (1, 1),
                               alpha=1 << 45, beta=beta) == "ok"
        assert int(c[0]) == -(1 << 63)
    # i128 output, Wrapping: the register's low 128 bits of 2^146 * 3 are 0.
    c = np.zeros(2, np.int64)
    assert oracle.gemm_int(a, (1, k), (k, 1), a, (k, 1), (1, 1), c, (1, 1), (1, 1), alpha=3,
                           encode="wrapping", out_bytes=16) == "ok"
    assert c.tolist() == [0, 0]
