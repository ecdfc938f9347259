"""GPU parity of the exact float GEMM (uor_gfx950_gemm_float and its slice /
raw faces) against the oracle, bit for bit: the reference's float corpus in
every encode mode, alpha/beta with non-finite priors, the raw face's stride
matrix and degenerate extents (raw.rs:167-311), and BASELINE configs[3]
distributions at reduced sizes."""
import numpy as np
import pytest
import torch

import gen

pytestmark = [pytest.mark.gpu, pytest.mark.filterwarnings("ignore::RuntimeWarning")]

MODES = ["nearest", "toward_zero", "saturating", "wrapping"]


def bits(x):
    return x.view(np.uint64 if x.dtype == np.float64 else np.uint32)


def offer_for(uor, dev, offer, is64, m, k, n):
    """The scratch offer: none (direct route), the suggested size (CRT with
    every modulus available) or an eighth of it (CRT with few moduli: wide
    cases fall back to the direct loop cell by cell)."""
    if offer == "none":
        return None
    want = uor.suggested_scratch_float(is64, m, k, n)
    if want == 0:
        return None
    if offer == "small":
        want //= 8
    return torch.empty(want + 64, dtype=torch.uint8, device=dev)[64:]  # misaligned on purpose


def check(oracle, uor, dev, a, b, m, k, n, c0=None, alpha=1, beta=0, mode="nearest",
          a_strides=None, c_strides=None, scratch=None, expect_route=None, offer=None):
    if offer is not None:
        scratch = offer_for(uor, dev, offer, a.dtype == np.float64, m, k, n)
    ars = a_strides or (k, 1)
    crs = c_strides or (n, 1)
    c0 = np.zeros(m * n, a.dtype) if c0 is None else c0
    want = c0.copy()
    st = oracle.gemm_float(a, (m, k), ars, b, (k, n), (n, 1), want, (m, n), crs, alpha=alpha,
                           beta=beta, encode=mode)
    gc = torch.from_numpy(c0.copy()).to(dev)
    gst, route = uor.gemm_float(torch.from_numpy(a).to(dev), (m, k), ars,
                                torch.from_numpy(b).to(dev), (k, n), (n, 1), gc, (m, n), crs,
                                alpha=alpha, beta=beta, encode=mode, scratch=scratch)
    torch.cuda.synchronize()
    assert uor.STATUS.get(gst, gst) == st
    got = gc.cpu().numpy()
    if not np.array_equal(bits(got), bits(want)):
        bad = np.nonzero(bits(got) != bits(want))[0][:5]
        raise AssertionError(f"{m}x{k}x{n} {mode} a={alpha} b={beta} route={route}: cells {bad.tolist()} "
                             f"got {got[bad].tolist()} want {want[bad].tolist()}")
    if expect_route:
        assert route["kind"] == expect_route, route
    return route


OFFERS = ["none", "full", "small"]


@pytest.mark.parametrize("offer", OFFERS)
@pytest.mark.parametrize("is64", [False, True])
@pytest.mark.parametrize("case", gen.CORRECTNESS_CASES + gen.PERFORMANCE_CASES,
                         ids=lambda c: f"{c[3]}-{c[4]}")
def test_corpus(oracle, uor, dev, is64, case, offer):
    m, k, n = case[:3]
    a, b = gen.corpus_operands(case, is64)
    modes = MODES if m * k * n <= 4096 else ["nearest", "toward_zero"]
    for mode in modes:
        check(oracle, uor, dev, a, b, m, k, n, mode=mode, offer=offer)


@pytest.mark.parametrize("offer", OFFERS)
@pytest.mark.parametrize("is64", [False, True])
def test_alpha_beta(oracle, uor, dev, is64, offer):
    ft = np.float64 if is64 else np.float32
    rng = np.random.default_rng(11 + is64)
    m, k, n = 9, 40, 11
    a, b = gen.corpus_operands((m, k, n, "FewGrades", 41), is64)
    c0 = (rng.standard_normal(m * n) * 2.0 ** rng.integers(-60, 60, m * n)).astype(ft)
    c0[[3, 7, 11, 12, 50]] = [np.inf, -np.inf, np.nan, 0.0, -0.0]
    for alpha, beta in [(1, 1), (3, -1), (0, 2), (-7, 0), (1 << 40, -(1 << 50)), (0, 0),
                        (-(1 << 63), 1), ((1 << 63) - 1, -(1 << 63)),
                        # beta = 0 with |alpha| at the register window's 32-bit
                        # limit and just past it (the LDS-register kernel).
                        ((1 << 32) - 1, 0), (-(1 << 32) + 1, 0), (1 << 32, 0), (70000, 0)]:
        for mode in ("nearest", "toward_zero"):
            check(oracle, uor, dev, a, b, m, k, n, c0=c0, alpha=alpha, beta=beta, mode=mode,
                  offer=offer)


@pytest.mark.parametrize("offer", OFFERS)
@pytest.mark.parametrize("is64", [False, True])
def test_nonfinite_rows_and_columns(oracle, uor, dev, is64, offer):
    ft = np.float64 if is64 else np.float32
    m, k, n = 6, 50, 7
    a, b = gen.corpus_operands((m, k, n, "FullFiniteRange", 5), is64)
    a = a.copy()
    b = b.copy()
    a[1 * k + 3] = np.inf          # row 1: inf against B[3, :]
    b[3 * n + 2] = 0.0             # ... which is NaN at column 2
    a[2 * k + 4] = -np.inf
    b[10 * n + 5] = np.nan         # column 5 is NaN everywhere
    a[4 * k + 7] = np.inf
    a[4 * k + 8] = -np.inf         # row 4: +inf and -inf -> NaN
    # Narrow the finite entries so that the CRT route keeps these lines.
    a2, b2 = gen.corpus_operands((m, k, n, "FewGrades", 6), is64)
    fin_a, fin_b = np.isfinite(a), np.isfinite(b)
    keep_a = np.zeros(a.shape, bool)
    keep_a[[1 * k + 3, 2 * k + 4, 4 * k + 7, 4 * k + 8]] = True
    keep_b = np.zeros(b.shape, bool)
    keep_b[[3 * n + 2, 10 * n + 5]] = True
    a = np.where(keep_a, a, a2)
    b = np.where(keep_b, b, b2)
    assert not fin_a.all() and not fin_b.all()
    for mode in MODES:
        check(oracle, uor, dev, a, b, m, k, n, mode=mode, offer=offer)
    check(oracle, uor, dev, a, b, m, k, n, alpha=0, offer=offer)
    check(oracle, uor, dev, a, b, m, k, n, alpha=-2, beta=1, c0=np.full(m * n, ft(1.5)), offer=offer)


def strided(rs, cs, rows, cols, f, ft):
    """raw.rs Strided::new: the window the strides reach, NaN elsewhere, and
    the offset of element (0, 0)."""
    offs = [i * rs + j * cs for i in range(rows) for j in range(cols)]
    lo = min(offs) if offs else 0
    span = (max(offs) - lo + 1) if offs else 0
    buf = np.full(span, np.nan, ft)
    for i in range(rows):
        for j in range(cols):
            buf[i * rs + j * cs - lo] = f(i, j)
    return buf, -lo


@pytest.mark.parametrize("shape", [(1, 1, 1), (3, 7, 5), (4, 16, 6), (13, 17, 19)])
def test_raw_stride_matrix(oracle, uor, dev, shape):
    """raw.rs:167-241: seven A stride pairs by three C stride pairs."""
    m, k, n = shape
    ft = np.float32
    checked = 0
    for rsa, csa in [(k, 1), (1, m), (-k, 1), (k, -1), (-k, -1), (2 * k, 2), (-2 * k, 2)]:
        for rsc, csc in [(n, 1), (-n, 1), (n, -1)]:
            abuf, aoff = strided(rsa, csa, m, k, lambda i, j: (i * k + j) * 0.5 - 3.0, ft)
            bbuf, boff = strided(n, 1, k, n, lambda i, j: (i * n + j) * -0.25 + 1.5, ft)
            cbuf, coff = strided(rsc, csc, m, n, lambda i, j: 0.0, ft)
            want = cbuf.copy()
            # The oracle takes buffer-start views; the raw face takes (0,0).
            st = oracle.gemm_float(abuf, (m, k), (rsa, csa), bbuf, (k, n), (n, 1), want, (m, n),
                                   (rsc, csc))
            assert st == "ok"
            ga, gb = torch.from_numpy(abuf).to(dev), torch.from_numpy(bbuf).to(dev)
            gc = torch.from_numpy(cbuf.copy()).to(dev)
            assert uor.raw_gemm(m, k, n, 1, ga, rsa, csa, gb, n, 1, 0, gc, rsc, csc, a_off=aoff,
                                b_off=boff, c_off=coff) == 0
            torch.cuda.synchronize()
            assert np.array_equal(bits(gc.cpu().numpy()), bits(want)), (rsa, csa, rsc, csc)
            checked += 1
    assert checked == 21


def test_raw_degenerate_and_invalid(uor, dev):
    # k = 0: beta * C (raw.rs:253-277).
    empty = torch.zeros(1, dtype=torch.float32, device=dev)
    c = torch.tensor([1.0, 2.0, 3.0, 4.0], device=dev)
    assert uor.raw_gemm(2, 0, 2, 1, empty, 0, 1, empty, 2, 1, 3, c, 2, 1) == 0
    torch.cuda.synchronize()
    assert c.cpu().tolist() == [3.0, 6.0, 9.0, 12.0]
    # m = 0 or n = 0 writes nothing (raw.rs:279-311).
    op = torch.ones(8, device=dev)
    for m, n in [(0, 2), (2, 0), (0, 0)]:
        u = torch.full((4,), 7.0, device=dev)
        assert uor.raw_gemm(m, 4, n, 1, op, 4, 1, op, n, 1, 0, u, n, 1) == 0
        torch.cuda.synchronize()
        assert u.cpu().tolist() == [7.0] * 4
    # A C view that maps two cells onto one is a silent no-op on the raw face.
    u = torch.full((4,), 7.0, device=dev)
    assert uor.raw_gemm(2, 4, 2, 1, op, 4, 1, op, 2, 1, 0, u, 0, 1) == 0
    torch.cuda.synchronize()
    assert u.cpu().tolist() == [7.0] * 4
    # ... and a status on the view API.
    st, _ = uor.gemm_float(op, (2, 4), (4, 1), op, (4, 2), (2, 1), u, (2, 2), (0, 1))
    assert uor.STATUS[st] == "output_aliases_itself"
    st, _ = uor.gemm_float(op, (2, 4), (4, 1), op, (3, 2), (2, 1), u, (2, 2), (2, 1))
    assert uor.STATUS[st] == "nonconformant"
    st, _ = uor.gemm_float(op, (2, 5), (5, 1), op, (5, 2), (2, 1), u, (2, 2), (2, 1))
    assert uor.STATUS[st] == "short_buffer"


def test_dgemm_and_slice_faces(oracle, uor, dev):
    """raw.rs:321-364 (the f64 face), and slice::gemm_float_ex with padded
    leading dimensions."""
    m, k, n = 5, 9, 4
    rsa, csa = -k, 1
    abuf, aoff = strided(rsa, csa, m, k, lambda i, j: (i * k + j) * 0.25 - 1.0, np.float64)
    b = np.array([i * -0.5 + 2.0 for i in range(k * n)], np.float64)
    want = np.zeros(m * n, np.float64)
    oracle.gemm_float(abuf, (m, k), (rsa, csa), b, (k, n), (n, 1), want, (m, n), (n, 1))
    gc = torch.zeros(m * n, dtype=torch.float64, device=dev)
    assert uor.raw_gemm(m, k, n, 1, torch.from_numpy(abuf).to(dev), rsa, csa,
                        torch.from_numpy(b).to(dev), n, 1, 0, gc, n, 1, a_off=aoff) == 0
    torch.cuda.synchronize()
    assert np.array_equal(bits(gc.cpu().numpy()), bits(want))
    # slice face: lda = k + 3, ldb = n + 1, ldc = n + 2, alpha 3, beta -1.
    for is64 in (False, True):
        ft = np.float64 if is64 else np.float32
        a2, b2 = gen.corpus_operands((m, k, n, "FewGrades", 9), is64)
        A = np.zeros((m, k + 3), ft)
        A[:, :k] = a2.reshape(m, k)
        B = np.zeros((k, n + 1), ft)
        B[:, :n] = b2.reshape(k, n)
        C = np.arange(m * (n + 2), dtype=ft) * ft(0.125)
        want = C.copy()
        oracle.gemm_float(A.reshape(-1), (m, k), (k + 3, 1), B.reshape(-1), (k, n), (n + 1, 1), want,
                          (m, n), (n + 2, 1), alpha=3, beta=-1)
        gc = torch.from_numpy(C.copy()).to(dev)
        assert uor.slice_gemm_float_ex(m, k, n, 3, torch.from_numpy(A.reshape(-1)).to(dev), k + 3,
                                       torch.from_numpy(B.reshape(-1)).to(dev), n + 1, -1, gc,
                                       n + 2) == 0
        torch.cuda.synchronize()
        assert np.array_equal(bits(gc.cpu().numpy()), bits(want))


@pytest.mark.parametrize("is64", [False, True])
def test_slice_gemm_float_every_offer(oracle, uor, dev, is64):
    """slice::gemm_float (slice.rs:405-421) against the oracle at alpha 1,
    beta 0, and the same bytes at every offer: none, a few bytes, an eighth of
    the suggestion, the suggestion and more (CD-19: the _full spellings' offers
    fold into this one buffer and never change the result)."""
    m, k, n = 37, 300, 29
    a, b = gen.corpus_operands((m, k, n, "FewGrades", 5), is64)
    want = np.zeros(m * n, a.dtype)
    oracle.gemm_float(a, (m, k), (k, 1), b, (k, n), (n, 1), want, (m, n), (n, 1))
    ga, gb = torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev)
    full = uor.suggested_scratch_float(is64, m, k, n)
    assert full > 0
    for nbytes in (0, 8, full // 8, full, full + 4096):
        scratch = torch.empty(nbytes + 64, dtype=torch.uint8, device=dev)[64:] if nbytes else None
        gc = torch.full((m * n,), 7.0, dtype=ga.dtype, device=dev)
        assert uor.slice_gemm_float(m, k, n, ga, gb, gc, scratch=scratch) == 0
        torch.cuda.synchronize()
        assert np.array_equal(bits(gc.cpu().numpy()), bits(want)), nbytes
    # A C slice shorter than m * n is refused before anything runs.
    short = torch.zeros(m * n - 1, dtype=ga.dtype, device=dev)
    assert uor.STATUS[uor.slice_gemm_float(m, k, n, ga, gb, short)] == "short_buffer"


@pytest.mark.parametrize("offer", OFFERS)
@pytest.mark.parametrize("is64,m,k,n", [(False, 48, 4096, 40), (True, 24, 2048, 20)])
def test_config4_distribution_reduced(oracle, uor, dev, is64, m, k, n, offer):
    """configs[3] entries (e in [-40, 40] f32 / [-300, 300] f64, 1% zeros, 1%
    cancelling pairs) at the full depth, on a reduced m x n."""
    a = gen.float_config4(m, k, is64, 9)
    b = gen.float_config4(k, n, is64, 10)
    a, b = gen.cancel_pairs(a, b, 99)
    route = check(oracle, uor, dev, a.reshape(-1).copy(), b.reshape(-1).copy(), m, k, n,
                  offer=offer)
    if offer == "full":
        assert route["kind"] == "float_crt", route
    check(oracle, uor, dev, a.reshape(-1).copy(), b.reshape(-1).copy(), m, k, n, mode="toward_zero",
          offer=offer)


@pytest.mark.parametrize("is64", [False, True])
def test_crt_narrow_and_strided(oracle, uor, dev, is64):
    """Moderate exponent spreads (every line within the CRT route), odd
    shapes, a transposed A and column-major B and C, alpha and beta."""
    ft = np.float64 if is64 else np.float32
    rng = np.random.default_rng(5 + is64)
    for m, k, n in [(1, 1, 1), (3, 70, 5), (130, 200, 129), (257, 64, 33), (64, 1000, 300)]:
        a = (rng.standard_normal(m * k) * 2.0 ** rng.integers(-20, 20, m * k)).astype(ft)
        b = (rng.standard_normal(k * n) * 2.0 ** rng.integers(-20, 20, k * n)).astype(ft)
        c0 = rng.standard_normal(m * n).astype(ft)
        sc = offer_for(uor, dev, "full", is64, m, k, n)
        want = c0.copy()
        oracle.gemm_float(a, (m, k), (1, m), b, (k, n), (1, k), want, (m, n), (1, m), alpha=-3,
                          beta=2)
        gc = torch.from_numpy(c0.copy()).to(dev)
        st, route = uor.gemm_float(torch.from_numpy(a).to(dev), (m, k), (1, m),
                                   torch.from_numpy(b).to(dev), (k, n), (1, k), gc, (m, n), (1, m),
                                   alpha=-3, beta=2, scratch=sc)
        torch.cuda.synchronize()
        assert st == 0 and route["kind"] == "float_crt", route
        assert np.array_equal(bits(gc.cpu().numpy()), bits(want)), (m, k, n)


def plan_of(scratch):
    """The CRT plan the device wrote at the start of the (256-aligned) offer:
    (moduli used, direct fallback for every cell, bound bits)."""
    off = (-scratch.data_ptr()) % 256
    return scratch[off:off + 12].cpu().view(torch.int32).tolist()


def test_crt_plan_is_tight(oracle, uor, dev):
    """configs[3] f32 rows (e in [-40, 40]) at the full depth use the residue
    route with the fewest moduli that cover the bound, and no fallback."""
    m, k, n = 64, 4096, 64
    a = gen.float_config4(m, k, False, 9)
    b = gen.float_config4(k, n, False, 10)
    sc = offer_for(uor, dev, "full", False, m, k, n)
    c = torch.zeros(m * n, dtype=torch.float32, device=dev)
    st, route = uor.gemm_float(torch.from_numpy(a.reshape(-1).copy()).to(dev), (m, k), (k, 1),
                               torch.from_numpy(b.reshape(-1).copy()).to(dev), (k, n), (n, 1), c,
                               (m, n), (n, 1), scratch=sc)
    torch.cuda.synchronize()
    nmod, off, need = plan_of(sc)
    assert st == 0 and off == 0, (nmod, off, need)
    # widths of about 104 bits per line and an L1 bound a few bits above the
    # top element: well under the 4096-term worst case of 104 + 104 + 12.
    assert 200 <= need <= 222 and 27 <= nmod <= 30, (nmod, need)
    want = np.zeros(m * n, np.float32)
    oracle.gemm_float(a.reshape(-1).copy(), (m, k), (k, 1), b.reshape(-1).copy(), (k, n), (n, 1),
                      want, (m, n), (n, 1))
    assert np.array_equal(bits(c.cpu().numpy()), bits(want))


@pytest.mark.parametrize("is64", [False, True])
def test_crt_all_lines_empty(oracle, uor, dev, is64):
    """Every row of A zero (a plan with no moduli, not the direct loop): the
    register finish still writes every cell, +0 over a nonzero C with beta =
    0, as the oracle does."""
    ft = np.float64 if is64 else np.float32
    m, k, n = 8, 32, 16
    rng = np.random.default_rng(7)
    a = np.zeros(m * k, ft)
    b = rng.standard_normal(k * n).astype(ft)
    c0 = rng.standard_normal(m * n).astype(ft)
    check(oracle, uor, dev, a, b, m, k, n, c0=c0, offer="full")


@pytest.mark.parametrize("spread", [40, 50])
def test_crt_fast_wide_unsliced(oracle, uor, dev, spread):
    """Unsliced lines close to the 160-bit slicing limit (f64 significands
    times 2^e, e in [-spread, spread]): bounds past 256 bits, so more than 33
    moduli and more than sixteen 16-bit digits on the register finish
    (crt_fast_kernel, beta = 0; alpha up to 65535 takes one more digit), bit
    for bit with the oracle."""
    rng = np.random.default_rng(spread)
    m, k, n = 16, 48, 24

    def mat(r, c):
        mant = rng.integers(1 << 52, 1 << 53, size=r * c).astype(np.float64)
        e = rng.integers(-spread, spread + 1, size=r * c)
        return rng.choice([-1.0, 1.0], size=r * c) * np.ldexp(mant, e - 52)

    a, b = mat(m, k), mat(k, n)
    for alpha in (1, -3, 65535):
        sc = offer_for(uor, dev, "full", True, m, k, n)
        check(oracle, uor, dev, a, b, m, k, n, alpha=alpha, scratch=sc, expect_route="float_crt")
        off = (-sc.data_ptr()) % 256
        nmod, crt_off, need, sa, sb = sc[off:off + 20].cpu().view(torch.int32).tolist()
        assert crt_off == 0 and sa == 1 and sb == 1 and nmod >= 34 and need > 252, (nmod, need, sa, sb)


@pytest.mark.parametrize("is64,N", [(False, 4096), (True, 2048)])
def test_config4_full_size_rows_and_columns(oracle, uor, dev, is64, N):
    """configs[3] at its full size: f32 4096^3 (e in [-40, 40]) and f64 2048^3
    (e in [-300, 300]), 1% zeros, 1% cancelling pairs, on the CRT route with
    the suggested offer (the full-size grid, modulus batching and finish
    choice).  Whole output rows and columns -- the first, the last and
    seeded others -- are compared bit for bit with the oracle (ora_gemm_float,
    the Complete-register restatement), and every cell with the direct route
    where that is cheap (f32: rows are independent, so the direct route runs
    on a 64-row slab)."""
    a = gen.float_config4(N, N, is64, 9)
    b = gen.float_config4(N, N, is64, 10)
    a, b = gen.cancel_pairs(a, b, 99)
    ft = np.float64 if is64 else np.float32
    ga = torch.from_numpy(a.reshape(-1).copy()).to(dev)
    gb = torch.from_numpy(b.reshape(-1).copy()).to(dev)
    sc = offer_for(uor, dev, "full", is64, N, N, N)
    gc = torch.full((N * N,), float("nan"), dtype=torch.float64 if is64 else torch.float32,
                    device=dev)
    st, route = uor.gemm_float(ga, (N, N), (N, 1), gb, (N, N), (N, 1), gc, (N, N), (N, 1),
                               scratch=sc)
    torch.cuda.synchronize()
    assert st == 0 and route["kind"] == "float_crt", route
    got = gc.cpu().numpy().reshape(N, N)
    del sc
    torch.cuda.empty_cache()
    rng = np.random.default_rng(4 + is64)
    rows = sorted({0, 1, N // 2, N - 1, *(int(x) for x in rng.integers(0, N, 4))})
    cols = sorted({0, N - 1, *(int(x) for x in rng.integers(0, N, 2))})
    bflat = b.reshape(-1).copy()
    for i in rows:
        want = np.zeros(N, ft)
        assert oracle.gemm_float(a[i].copy(), (1, N), (N, 1), bflat, (N, N), (N, 1), want,
                                 (1, N), (N, 1)) == "ok"
        bad = np.nonzero(bits(got[i].copy()) != bits(want))[0]
        assert bad.size == 0, f"row {i}: columns {bad[:5].tolist()}"
    aflat = a.reshape(-1).copy()
    for j in cols:
        want = np.zeros(N, ft)
        assert oracle.gemm_float(aflat, (N, N), (N, 1), b[:, j].copy(), (N, 1), (1, 1), want,
                                 (N, 1), (1, 1)) == "ok"
        bad = np.nonzero(bits(got[:, j].copy()) != bits(want))[0]
        assert bad.size == 0, f"column {j}: rows {bad[:5].tolist()}"
    # The cancelling pairs and exact zeros reach the checked cells: the rows
    # hold exact zeros of the inputs.
    assert (a[rows] == 0).any()
