"""Pins the oracle's exact float GEMM (ora_gemm_float) on the CPU: against an
independent rational implementation (tests/exact_float.py) over the
reference's float corpus (float_corpus.rs CORRECTNESS_CASES, every encode
mode, f32 and f64), and against closed forms the IEEE rules fix: exact
cancellation is +0, ties go to even, overflow is +-inf under Nearest and
+-MAX otherwise, a nonzero that rounds to zero keeps its sign, NaN is the
canonical quiet NaN, inf * 0 and +inf + -inf are NaN."""
import numpy as np
import pytest

import exact_float
import gen

MODES = ["nearest", "toward_zero", "saturating", "wrapping"]


pytestmark = pytest.mark.filterwarnings("ignore::RuntimeWarning")


def run_oracle(oracle, a, b, m, k, n, c0=None, alpha=1, beta=0, mode="nearest"):
    c = np.zeros(m * n, a.dtype) if c0 is None else c0.copy()
    st = oracle.gemm_float(a, (m, k), (k, 1), b, (k, n), (n, 1), c, (m, n), (n, 1), alpha=alpha,
                           beta=beta, encode=mode)
    assert st == "ok"
    return c.view(np.uint64 if a.dtype == np.float64 else np.uint32)


@pytest.mark.parametrize("is64", [False, True])
@pytest.mark.parametrize("case", gen.CORRECTNESS_CASES, ids=lambda c: f"{c[3]}-{c[4]}")
def test_corpus_against_rationals(oracle, is64, case):
    m, k, n = case[:3]
    a, b = gen.corpus_operands(case, is64)
    if k == 0:
        a = np.zeros(0, a.dtype)
        b = np.zeros(0, a.dtype)
    for mode in MODES:
        got = run_oracle(oracle, a, b, m, k, n, mode=mode)
        want = exact_float.gemm_float(a, b, np.zeros(m * n, a.dtype), m, k, n, mode=mode)
        assert np.array_equal(got, want), (case, mode)


@pytest.mark.parametrize("is64", [False, True])
def test_alpha_beta_against_rationals(oracle, is64):
    ft = np.float64 if is64 else np.float32
    rng = np.random.default_rng(7 + is64)
    m, k, n = 4, 9, 5
    case = (m, k, n, "FewGrades", 31)
    a, b = gen.corpus_operands(case, is64)
    c0 = (rng.standard_normal(m * n) * 2.0 ** rng.integers(-30, 30, m * n)).astype(ft)
    c0[3] = np.inf
    c0[7] = -np.inf
    c0[11] = np.nan
    c0[12] = 0.0
    for alpha, beta in [(1, 1), (3, -1), (0, 2), (-7, 0), (1 << 40, -(1 << 50)), (0, 0),
                        (-(1 << 63), 1)]:
        for mode in ("nearest", "toward_zero"):
            got = run_oracle(oracle, a, b, m, k, n, c0=c0, alpha=alpha, beta=beta, mode=mode)
            want = exact_float.gemm_float(a, b, c0, m, k, n, alpha=alpha, beta=beta, mode=mode)
            assert np.array_equal(got, want), (alpha, beta, mode)


@pytest.mark.parametrize("case", [c for c in gen.PERFORMANCE_CASES if c[0] * c[1] * c[2] <= 40000],
                         ids=lambda c: f"{c[3]}-{c[4]}")
def test_performance_corpus_nearest(oracle, case):
    m, k, n = case[:3]
    for is64 in (False, True):
        a, b = gen.corpus_operands(case, is64)
        got = run_oracle(oracle, a, b, m, k, n)
        want = exact_float.gemm_float(a, b, np.zeros(m * n, a.dtype), m, k, n)
        assert np.array_equal(got, want), case


def bits32(x):
    return int(np.array(x, np.float32).view(np.uint32))


def one(oracle, avals, bvals, mode="nearest", ft=np.float32, alpha=1, beta=0, c=0.0):
    a = np.array(avals, ft)
    b = np.array(bvals, ft)
    k = len(avals)
    return int(run_oracle(oracle, a, b, 1, k, 1, c0=np.array([c], ft), alpha=alpha, beta=beta,
                          mode=mode)[0])


def test_closed_forms(oracle):
    f = np.float32
    # Exact cancellation gives +0, whatever the signs.
    assert one(oracle, [-3.0, 3.0], [1.5, 1.5]) == 0
    assert one(oracle, [-1e-30, 1e-30], [1e-10, 1e-10]) == 0
    # Ties to even: 1 + 2^-24 is halfway between 1 and 1 + 2^-23.
    assert one(oracle, [1.0, 2.0 ** -24], [1.0, 1.0]) == bits32(1.0)
    assert one(oracle, [1.0 + 2.0 ** -23, 2.0 ** -24], [1.0, 1.0]) == bits32(1.0 + 2.0 ** -22)
    # Just above the tie rounds up; toward zero truncates.
    assert one(oracle, [1.0, 2.0 ** -24, 2.0 ** -60], [1.0, 1.0, 1.0]) == bits32(1.0 + 2.0 ** -23)
    assert one(oracle, [1.0, 2.0 ** -24, 2.0 ** -60], [1.0, 1.0, 1.0], mode="toward_zero") == bits32(1.0)
    # A sum below a representable value truncates to its predecessor.
    assert one(oracle, [1.0, -2.0 ** -60], [1.0, 1.0], mode="toward_zero") == bits32(np.nextafter(f(1), f(0)))
    assert one(oracle, [1.0, -2.0 ** -60], [1.0, 1.0]) == bits32(1.0)
    # Overflow: +-inf under Nearest, +-MAX otherwise.
    mx = np.finfo(f).max
    assert one(oracle, [mx, mx], [1.0, 1.0]) == bits32(np.inf)
    assert one(oracle, [-mx, -mx], [1.0, 1.0]) == bits32(-np.inf)
    assert one(oracle, [mx, mx], [1.0, 1.0], mode="saturating") == bits32(mx)
    assert one(oracle, [-mx, -mx], [1.0, 1.0], mode="wrapping") == bits32(-mx)
    assert one(oracle, [mx], [1.0], alpha=2) == bits32(np.inf)
    # Underflow keeps the sign: -2^-150 is a tie between -0 and -2^-149 -> -0.
    assert one(oracle, [-(2.0 ** -75)], [2.0 ** -75]) == bits32(-0.0)
    assert one(oracle, [-(2.0 ** -75)], [2.0 ** -74]) == bits32(-(2.0 ** -149))
    assert one(oracle, [2.0 ** -75, 2.0 ** -100], [2.0 ** -75, 2.0 ** -60]) == bits32(2.0 ** -149)
    # Non-finite rules; NaN is the canonical quiet NaN.
    nan = 0x7FC00000
    assert one(oracle, [np.inf], [0.0]) == nan
    assert one(oracle, [np.inf, -np.inf], [1.0, 1.0]) == nan
    assert one(oracle, [np.inf, 5.0], [-2.0, 1.0]) == bits32(-np.inf)
    assert one(oracle, [np.float32(np.nan)], [1.0]) == nan
    assert one(oracle, [np.inf], [1.0], alpha=0) == nan
    assert one(oracle, [np.inf], [1.0], alpha=-3) == bits32(-np.inf)
    assert one(oracle, [1.0], [1.0], beta=0, c=np.nan) == bits32(1.0)   # beta = 0 never reads C
    assert one(oracle, [1.0], [1.0], beta=2, c=np.nan) == nan
    assert one(oracle, [1.0], [1.0], beta=-1, c=np.inf) == bits32(-np.inf)
    # The reference's raw test (raw.rs:253-277): k = 0 gives beta * C.
    a = np.zeros(0, f)
    c = np.array([1, 2, 3, 4], f)
    assert oracle.gemm_float(a, (2, 0), (0, 1), a, (0, 2), (2, 1), c, (2, 2), (2, 1), alpha=1,
                             beta=3) == "ok"
    assert c.tolist() == [3.0, 6.0, 9.0, 12.0]


def test_f64_matches_python_float_rounding(oracle):
    """For f64 under Nearest, CPython's float(Fraction) is a correctly rounded
    conversion: a third, library-level witness."""
    from fractions import Fraction
    case = (3, 40, 3, "FullFiniteRange", 77)
    a, b = gen.corpus_operands(case, True)
    got = run_oracle(oracle, a, b, 3, 40, 3)
    A = a.reshape(3, 40)
    B = b.reshape(40, 3)
    for i in range(3):
        for j in range(3):
            s = sum(Fraction(A[i, p].item()) * Fraction(B[p, j].item()) for p in range(40))
            try:
                want = float(s)
            except OverflowError:
                want = float("inf") if s > 0 else float("-inf")
            w = np.array(want).view(np.uint64)
            if want == 0:
                w = np.uint64(0)
            assert int(got[i * 3 + j]) == int(w)
