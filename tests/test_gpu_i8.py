"""GPU parity of the exact i8 GEMM route (through the C ABI) against the oracle.

Bar: bit-exact.  Small and ragged cases compare with the CPU oracle
(oracle/uor_oracle.c); the full-size configurations compare with float64
matmul, which is exact here because every partial sum is an integer below
2^53, plus oracle rows and closed forms for the deep case.
"""
import zlib

import numpy as np
import pytest
import torch

import gen

pytestmark = pytest.mark.gpu

I32_MAX = (1 << 31) - 1


def to_dev(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def dev_i8(x, dev):
    return to_dev(np.asarray(x, dtype=np.int8), dev)


def check_case(oracle, uor, dev, a, ash, ast, b, bsh, bst, c0, csh, cst, out="i32", alpha=1,
               beta=0, encode="nearest", scratch=None, expect_route=None):
    dt = {"i8": np.int8, "i16": np.int16, "i32": np.int32, "i64": np.int64}[out]
    want = c0.copy()
    st = oracle.gemm_int(a, ash, ast, b, bsh, bst, want, csh, cst, alpha=alpha, beta=beta,
                         encode=encode)
    ga, gb, gc = to_dev(a, dev), to_dev(b, dev), to_dev(c0, dev)
    gst, route = uor.gemm_i8(ga, ash, ast, gb, bsh, bst, gc, csh, cst, out=out, alpha=alpha,
                             beta=beta, encode=encode, scratch=scratch)
    torch.cuda.synchronize()
    assert uor.STATUS.get(gst, gst) == st
    got = gc.cpu().numpy()
    assert got.dtype == dt
    assert np.array_equal(got, want), (ash, bsh, csh, out, alpha, beta, encode, route)
    if expect_route:
        assert route["kind"] == expect_route, route
    return route


def test_readme_and_cs05_cs06(oracle, uor, dev):
    a = np.array([1, 2, 3, 4], np.int8)
    b = np.array([5, 6, 7, 8], np.int8)
    c = torch.zeros(4, dtype=torch.int32, device=dev)
    assert uor.slice_gemm_i8(2, 2, 2, dev_i8(a, dev), dev_i8(b, dev), c) == 0
    torch.cuda.synchronize()
    assert c.cpu().tolist() == [19, 22, 43, 50]
    c = torch.tensor([100, 200, 300, 400], dtype=torch.int32, device=dev)
    assert uor.slice_gemm_ex_i8(2, 2, 2, 3, dev_i8(a, dev), 2, dev_i8(b, dev), 2, -2, c, 2) == 0
    torch.cuda.synchronize()
    assert c.cpu().tolist() == [3 * 19 - 200, 3 * 22 - 400, 3 * 43 - 600, 3 * 50 - 800]
    a6 = np.array([1, 2, 3, 4, 5, 6], np.int8)
    d = np.zeros(9, np.int32)
    check_case(oracle, uor, dev, a6, (3, 2), (1, 3), a6, (2, 3), (3, 1), d, (3, 3), (3, 1))


@pytest.mark.parametrize("shape", [(1, 1, 1), (13, 17, 19), (64, 64, 64), (65, 130, 67),
                                   (127, 255, 129), (200, 1000, 300), (31, 4099, 33)])
@pytest.mark.parametrize("layout", ["nn", "tn", "nt", "tt"])
def test_layouts_against_oracle(oracle, uor, dev, shape, layout):
    m, k, n = shape
    rng = np.random.default_rng(m * 7919 + k * 31 + n)
    a = rng.integers(-128, 128, m * k).astype(np.int8)
    b = rng.integers(-128, 128, k * n).astype(np.int8)
    ast = (k, 1) if layout[0] == "n" else (1, m)
    bst = (n, 1) if layout[1] == "n" else (1, k)
    c0 = np.zeros(m * n, np.int32)
    check_case(oracle, uor, dev, a, (m, k), ast, b, (k, n), bst, c0, (m, n), (n, 1))


@pytest.mark.parametrize("out", ["i8", "i16", "i32", "i64"])
@pytest.mark.parametrize("encode", ["nearest", "saturating", "toward_zero", "wrapping"])
def test_output_types_and_encodes(oracle, uor, dev, out, encode):
    dt = {"i8": np.int8, "i16": np.int16, "i32": np.int32, "i64": np.int64}[out]
    rng = np.random.default_rng(zlib.crc32(f"{out}-{encode}".encode()))
    m, k, n = 37, 300, 41
    a = rng.integers(-128, 128, m * k).astype(np.int8)
    b = rng.integers(-128, 128, k * n).astype(np.int8)
    c0 = rng.integers(np.iinfo(dt).min, np.iinfo(dt).max, m * n, dtype=dt, endpoint=True)
    for alpha, beta in [(1, 0), (3, -1), (-(1 << 40), 1 << 33), (1 << 62, -(1 << 62)),
                        (-(1 << 63), (1 << 63) - 1)]:
        check_case(oracle, uor, dev, a, (m, k), (k, 1), b, (k, n), (n, 1), c0, (m, n), (n, 1),
                   out=out, alpha=alpha, beta=beta, encode=encode)


def test_i128_output(oracle, uor, dev):
    rng = np.random.default_rng(5)
    m, k, n = 9, 70, 11
    a = rng.integers(-128, 128, m * k).astype(np.int8)
    b = rng.integers(-128, 128, k * n).astype(np.int8)
    c0 = rng.integers(-(1 << 62), 1 << 62, 2 * m * n, dtype=np.int64)
    for alpha, beta, enc in [(1, 0, "nearest"), (5, -7, "wrapping"),
                             ((1 << 63) - 1, -(1 << 63), "saturating")]:
        want = c0.copy()
        assert oracle.gemm_int(a, (m, k), (k, 1), b, (k, n), (n, 1), want, (m, n), (n, 1),
                               alpha=alpha, beta=beta, encode=enc, out_bytes=16) == "ok"
        gc = to_dev(c0, dev)
        st, _ = uor.gemm_i8(to_dev(a, dev), (m, k), (k, 1), to_dev(b, dev), (k, n), (n, 1), gc,
                            (m, n), (n, 1), out="i128", alpha=alpha, beta=beta, encode=enc)
        torch.cuda.synchronize()
        assert st == 0 and np.array_equal(gc.cpu().numpy(), want), (alpha, beta, enc)


@pytest.mark.parametrize("seed", range(8))
def test_random_strided_views(oracle, uor, dev, seed):
    """Negative, zero, transposed and misaligned strides (the view API's
    arbitrary strides, layout.rs:29-154) go through the gathering loaders."""
    rng = np.random.default_rng(100 + seed)
    for _ in range(12):
        m, k, n = (int(x) for x in rng.integers(1, 70, 3))
        def pick(rows, cols):
            choice = rng.integers(0, 5)
            if choice == 0:
                return cols, 1
            if choice == 1:
                return 1, rows
            if choice == 2:
                return -cols, 1
            if choice == 3:
                return 0, 1
            return int(rng.integers(-3, 4)) * cols + 1, int(rng.choice([-1, 1, 2]))
        ars, acs = pick(m, k)
        brs, bcs = pick(k, n)
        a = rng.integers(-128, 128, 4 * (m * k + 1) + 64).astype(np.int8)
        b = rng.integers(-128, 128, 4 * (k * n + 1) + 64).astype(np.int8)
        if oracle.place(a.size, m, k, ars, acs) is None or oracle.place(b.size, k, n, brs, bcs) is None:
            continue
        c0 = rng.integers(-1000, 1000, m * n).astype(np.int32)
        crs, ccs = (n, 1) if rng.random() < 0.5 else (1, m)
        check_case(oracle, uor, dev, a, (m, k), (ars, acs), b, (k, n), (brs, bcs), c0, (m, n),
                   (crs, ccs), alpha=int(rng.integers(-4, 5)), beta=int(rng.integers(-4, 5)))


def test_misaligned_and_offset_buffers(oracle, uor, dev):
    rng = np.random.default_rng(9)
    m, k, n = 100, 150, 90
    a_full = rng.integers(-128, 128, m * k + 3).astype(np.int8)
    b_full = rng.integers(-128, 128, k * n + 5).astype(np.int8)
    ga, gb = to_dev(a_full, dev), to_dev(b_full, dev)
    gc = torch.zeros(m * n, dtype=torch.int32, device=dev)
    st, route = uor.gemm_i8(ga[3:], (m, k), (k, 1), gb[5:], (k, n), (n, 1), gc, (m, n), (n, 1))
    torch.cuda.synchronize()
    want = np.zeros(m * n, np.int32)
    oracle.gemm_int(a_full[3:].copy(), (m, k), (k, 1), b_full[5:].copy(), (k, n), (n, 1), want,
                    (m, n), (n, 1))
    assert st == 0 and np.array_equal(gc.cpu().numpy(), want)
    assert route["operand_modes"] == 2 | (2 << 2)  # both gathered


def test_empty_and_k_zero(oracle, uor, dev):
    c0 = np.arange(12, dtype=np.int32)
    r = check_case(oracle, uor, dev, np.zeros(0, np.int8), (3, 0), (0, 1),
                   np.zeros(0, np.int8), (0, 4), (4, 1), c0, (3, 4), (4, 1), alpha=5, beta=-3)
    assert r["kind"] == "epilogue_only"
    r = check_case(oracle, uor, dev, np.zeros(0, np.int8), (0, 5), (5, 1),
                   np.zeros(35, np.int8), (5, 7), (7, 1), np.zeros(0, np.int32), (0, 7), (7, 1))
    assert r["kind"] == "none"


def test_errors_report_before_launch(uor, dev):
    a = torch.zeros(12, dtype=torch.int8, device=dev)
    c = torch.zeros(16, dtype=torch.int32, device=dev)
    assert uor.gemm_i8(a, (3, 4), (4, 1), a, (3, 4), (4, 1), c, (3, 4), (4, 1))[0] == 1
    assert uor.gemm_i8(a, (3, 4), (4, 1), a, (4, 3), (3, 1), c, (3, 3), (1, 1))[0] == 2
    assert uor.gemm_i8(a, (3, 5), (5, 1), a, (5, 3), (3, 1), c, (3, 3), (3, 1))[0] == 3


def test_offer_ladder_same_bytes_cd10(oracle, uor, dev):
    """Every scratch offer, from none to suggested, gives identical bytes;
    only the route changes (reference CD-10, CD-22)."""
    rng = np.random.default_rng(77)
    m, k, n = 96, 140_000, 80
    a = rng.integers(-128, 128, m * k).astype(np.int8)
    b = rng.integers(-128, 128, k * n).astype(np.int8)
    ga, gb = to_dev(a, dev), to_dev(b, dev)
    want = (a.reshape(m, k).astype(np.float64) @ b.reshape(k, n).astype(np.float64))
    want = np.clip(3 * want - 7, -(1 << 31), I32_MAX).astype(np.int32)
    kinds = set()
    for offer in [0, 100, uor.suggested_scratch_i8(m, k, n)]:
        scratch = torch.empty(max(offer, 1), dtype=torch.uint8, device=dev) if offer else None
        gc = torch.ones(m * n, dtype=torch.int32, device=dev) * 7
        st, route = uor.gemm_i8(ga, (m, k), (k, 1), gb, (k, n), (n, 1), gc, (m, n), (n, 1),
                                alpha=3, beta=-1, scratch=scratch)
        torch.cuda.synchronize()
        assert st == 0
        assert np.array_equal(gc.cpu().numpy().reshape(m, n), want), route
        kinds.add(route["kind"])
    assert kinds == {"mfma_wide", "mfma_splitk"}


@pytest.mark.parametrize("shift", [1, 4, 8, 12])
def test_unaligned_offer_same_bytes(uor, dev, shift):
    """An offer that starts off a 256-byte boundary (a sub-buffer) still
    takes the split-K route, its i64 partial sums carved from the first
    aligned byte, and gives the no-offer bytes."""
    rng = np.random.default_rng(4100 + shift)
    m, k, n = 72, 70_000, 40
    a = rng.integers(-128, 128, m * k).astype(np.int8)
    b = rng.integers(-128, 128, k * n).astype(np.int8)
    ga, gb = to_dev(a, dev), to_dev(b, dev)
    base = torch.empty(uor.suggested_scratch_i8(m, k, n) + shift, dtype=torch.uint8, device=dev)
    offer = base[shift:]
    assert offer.data_ptr() % 8 != 0 or shift % 8 == 0
    outs = []
    for scratch in (None, offer):
        gc = torch.full((m * n,), 5, dtype=torch.int64, device=dev)
        st, route = uor.gemm_i8(ga, (m, k), (k, 1), gb, (k, n), (n, 1), gc, (m, n), (n, 1),
                                out="i64", alpha=-3, beta=2, scratch=scratch)
        torch.cuda.synchronize()
        assert st == 0
        outs.append((gc.cpu().numpy(), route["kind"]))
    assert outs[1][1] == "mfma_splitk" and outs[0][1] == "mfma_wide"
    assert np.array_equal(outs[0][0], outs[1][0])
    want = a.reshape(m, k).astype(np.float64) @ b.reshape(k, n).astype(np.float64)
    assert np.array_equal(outs[0][0].reshape(m, n), (-3 * want + 10).astype(np.int64))


def test_config1_slice_gemm_1024(uor, dev):
    """slice::gemm i8 -> i32, 1024^3, xorshift fill (salts 1, 2),
    suggested scratch offer; the reference's exact generator sequence."""
    n = 1024
    a = gen.i8_full(n * n, 1)
    b = gen.i8_full(n * n, 2)
    want = (a.reshape(n, n).astype(np.float64) @ b.reshape(n, n).astype(np.float64)).astype(np.int32)
    scratch = torch.empty(uor.suggested_scratch_i8(n, n, n), dtype=torch.uint8, device=dev)
    gc = torch.full((n * n,), 0x7B7B7B7B, dtype=torch.int32, device=dev)
    assert uor.slice_gemm_i8(n, n, n, to_dev(a, dev), to_dev(b, dev), gc, scratch=scratch) == 0
    torch.cuda.synchronize()
    assert np.array_equal(gc.cpu().numpy().reshape(n, n), want)


def test_config2_gemm_ex_8192_padded(oracle, uor, dev):
    """gemm_ex 8192^3, lda=ldb=ldc=8256, alpha=3, beta=-1, C
    uniform in [-2^20, 2^20]; padding columns must be neither read into the
    result nor written."""
    N, LD = 8192, 8256
    a = gen.i8_full(N * LD, 3)
    b = gen.i8_full(N * LD, 4)
    c0 = gen.i32_pm2_20(N * LD, 5)
    ga, gb, gc = to_dev(a, dev), to_dev(b, dev), to_dev(c0, dev)
    pad_before = gc.view(N, LD)[:, N:].clone()
    assert uor.slice_gemm_ex_i8(N, N, N, 3, ga, LD, gb, LD, -1, gc, LD) == 0
    torch.cuda.synchronize()
    A = ga.view(N, LD)[:, :N].to(torch.float64)
    B = gb.view(N, LD)[:, :N].to(torch.float64)
    C0 = to_dev(c0, dev).view(N, LD)[:, :N].to(torch.float64)
    want = 3 * (A @ B) - C0  # exact: |values| < 2^30
    got = gc.view(N, LD)[:, :N].to(torch.float64)
    assert torch.equal(got, want)
    assert torch.equal(gc.view(N, LD)[:, N:], pad_before)
    del A, B, C0, want, got
    # Rows against the oracle itself.
    rows = [0, 1, 4095, 8191]
    for r in rows:
        ar = a.reshape(N, LD)[r, :N].copy()
        c = c0.reshape(N, LD)[r, :N].copy()
        oracle.gemm_int(ar, (1, N), (N, 1), b, (N, N), (LD, 1), c, (1, N), (N, 1), alpha=3, beta=-1)
        assert np.array_equal(gc.view(N, LD)[r, :N].cpu().numpy(), c), r


@pytest.mark.parametrize("out,alpha,beta,encode", [
    ("i32", 1, 0, "nearest"), ("i64", 1, 0, "nearest"), ("i64", 3, -1, "nearest"),
    ("i32", 1, 0, "wrapping"), ("i32", 3, -1, "nearest")])
def test_config2_deep_k_2_24(uor, dev, out, alpha, beta, encode):
    """configs[1] deep case: m=n=128, k=2^24, A=B=-128, so every exact sum is
    2^38: i32 Nearest saturates to i32::MAX, i64 holds 2^38 (or 3*2^38 - C),
    Wrapping gives 2^38 mod 2^32 = 0."""
    m = n = 128
    k = 1 << 24
    ga = torch.full((m * k,), -128, dtype=torch.int8, device=dev)
    gb = torch.full((k * n,), -128, dtype=torch.int8, device=dev)
    dt = torch.int32 if out == "i32" else torch.int64
    c0 = torch.arange(m * n, dtype=dt, device=dev) - 5000
    gc = c0.clone()
    scratch = torch.empty(uor.suggested_scratch_i8(m, k, n), dtype=torch.uint8, device=dev)
    st, route = uor.gemm_i8(ga, (m, k), (k, 1), gb, (k, n), (n, 1), gc, (m, n), (n, 1), out=out,
                            alpha=alpha, beta=beta, encode=encode, scratch=scratch)
    torch.cuda.synchronize()
    assert st == 0 and route["kind"] == "mfma_splitk"
    exact = alpha * (1 << 38)
    want = [exact + beta * int(v) for v in c0.cpu().tolist()]
    bits = 32 if out == "i32" else 64
    mn, mx = -(1 << (bits - 1)), (1 << (bits - 1)) - 1
    if encode == "wrapping":
        want = [(v - mn) % (1 << bits) + mn for v in want]
    else:
        want = [max(mn, min(mx, v)) for v in want]
    assert gc.cpu().tolist() == want


@pytest.mark.parametrize("case", ["vec", "ldc_odd", "c_offset", "beta0", "wrap_alpha", "sat_alpha",
                                  "i16", "i64", "identity", "i32_edges", "alpha_2p31"])
def test_fused_tile_epilogues(uor, dev, case):
    """The 256x256 direct-to-LDS tile (>= 256 output tiles, n a multiple of
    16) with each epilogue branch: 16-byte i32 rows (vec), an odd ldc or a C
    base off 16-byte alignment (per-element i32), beta = 0, alpha large
    enough to saturate or wrap, and i16 / i64 outputs; the i32 output's
    32-bit-scalar evaluation at its widest scalars and one past them, and
    alpha = 1, beta = 0 (the sum itself).  Expected values from
    an exact float64 product (|sum| <= 512 * 2^14) and a numpy encode."""
    m = n = 4096
    k = 512
    lda, ldb = k + 64, n + 32
    ldc = n + (1 if case == "ldc_odd" else 4)
    off = 1 if case == "c_offset" else 0
    out = {"i16": "i16", "i64": "i64"}.get(case, "i32")
    alpha, beta, encode = 3, -1, "nearest"
    if case == "beta0":
        beta = 0
    if case == "wrap_alpha":
        alpha, beta, encode = (1 << 12) + 7, 5, "wrapping"
    if case == "sat_alpha":
        alpha, beta, encode = (1 << 12) + 7, -5, "saturating"
    if case == "identity":  # the exact sum stored as it is
        alpha, beta = 1, 0
    if case == "i32_edges":  # the widest scalars of the 32-bit evaluation
        alpha, beta, encode = -(1 << 31), (1 << 31) - 1, "saturating"
    if case == "alpha_2p31":  # one past them: the 64-bit evaluation
        alpha, beta, encode = 1 << 31, -1, "wrapping"
    rng = np.random.default_rng(len(case))
    dt = {"i16": np.int16, "i32": np.int32, "i64": np.int64}[out]
    a = torch.from_numpy(rng.integers(-128, 128, m * lda).astype(np.int8)).to(dev)
    b = torch.from_numpy(rng.integers(-128, 128, k * ldb).astype(np.int8)).to(dev)
    c0 = rng.integers(-(1 << 14), 1 << 14, m * ldc + off).astype(dt)
    c = torch.from_numpy(c0.copy()).to(dev)
    cv = c[off:]
    st, route = uor.gemm_i8(a, (m, k), (lda, 1), b, (k, n), (ldb, 1), cv, (m, n), (ldc, 1), out=out,
                            alpha=alpha, beta=beta, encode=encode)
    torch.cuda.synchronize()
    assert st == 0 and route["kind"] == "mfma_tile" and route["tile_m"] == 256, route
    S = (a.view(m, lda)[:, :k].double() @ b.view(k, ldb)[:, :n].double()).cpu().numpy().astype(np.int64)
    C0 = c0[off:off + m * ldc].reshape(m, ldc)[:, :n].astype(np.int64)
    x = alpha * S + beta * C0
    bits = 8 * np.dtype(dt).itemsize
    if encode == "wrapping":
        want = x.astype(dt)  # two's complement truncation (numpy casts wrap)
    else:
        info = np.iinfo(dt)
        want = np.clip(x, info.min, info.max).astype(dt)
    got = c.cpu().numpy()[off:off + m * ldc].reshape(m, ldc)
    assert np.array_equal(got[:, :n], want), case
    # padding columns untouched
    assert np.array_equal(got[:, n:], c0[off:off + m * ldc].reshape(m, ldc)[:, n:])
    assert bits in (16, 32, 64)


@pytest.mark.parametrize("m,n,k", [(4096 + 36, 4096 + 48, 64), (4096, 4096 + 16, 192),
                                   (4300, 4112, 320), (4096, 4096, 896), (4352, 4096, 8192 + 64),
                                   (4096 + 36, 4096 + 48, 128), (4096, 4096 + 16, 256),
                                   (4300, 4112, 384), (4352, 4096, 8192 + 128)])
def test_tile256_ragged_edges_and_depths(uor, dev, m, n, k):
    """The 256x256 direct-to-LDS tile at ragged m and n (partial edge tiles,
    rows and columns past the edge computed and discarded) and depths of 1, 3,
    5, 14 and 129 steps of 64 and of 2, 4, 6 and 130 (each remainder of the
    four-stage loop, odd and even), with alpha = 3, beta = -1.  Expected values from an exact float64 product
    (|sum| <= k * 2^14 < 2^53)."""
    lda, ldb, ldc = k + 16, n + 16, n + 8
    rng = np.random.default_rng(m * 7 + n * 3 + k)
    a = torch.from_numpy(rng.integers(-128, 128, m * lda).astype(np.int8)).to(dev)
    b = torch.from_numpy(rng.integers(-128, 128, k * ldb).astype(np.int8)).to(dev)
    c0 = rng.integers(-(1 << 20), 1 << 20, m * ldc).astype(np.int32)
    c = torch.from_numpy(c0.copy()).to(dev)
    st, route = uor.gemm_i8(a, (m, k), (lda, 1), b, (k, n), (ldb, 1), c, (m, n), (ldc, 1), out="i32",
                            alpha=3, beta=-1)
    torch.cuda.synchronize()
    assert st == 0 and route["kind"] == "mfma_tile" and route["tile_m"] == 256, route
    S = (a.view(m, lda)[:, :k].double() @ b.view(k, ldb)[:, :n].double()).cpu().numpy().astype(np.int64)
    C0 = c0.reshape(m, ldc).astype(np.int64)
    want = 3 * S - C0[:, :n]
    got = c.cpu().numpy().reshape(m, ldc)
    assert np.array_equal(got[:, :n].astype(np.int64), want)
    assert np.array_equal(got[:, n:], c0.reshape(m, ldc)[:, n:])


@pytest.mark.parametrize("m,n,k", [(2048 + 40, 1024 + 48, 64), (2048, 2048 + 8, 192),
                                   (1024 + 3, 4096, 320), (2048, 2048, 4096 + 64)])
@pytest.mark.parametrize("out", ["i32", "i8"])
def test_tile256_column_major_b(uor, dev, m, n, k, out):
    """The 256x256 tile with B k-contiguous (column-major, ldb = k + 16): its
    stage half in A's layout.  Ragged m and n, depths of 1, 3, 5 and 65 steps,
    alpha = 3, beta = -1, against an exact float64 product; the i8 output
    saturates."""
    lda, ldb, ldc = k + 16, k + 16, n + 8
    rng = np.random.default_rng(m * 5 + n * 3 + k)
    a = torch.from_numpy(rng.integers(-128, 128, m * lda).astype(np.int8)).to(dev)
    bt = torch.from_numpy(rng.integers(-128, 128, n * ldb).astype(np.int8)).to(dev)
    dt, tdt = (np.int32, torch.int32) if out == "i32" else (np.int8, torch.int8)
    c0 = rng.integers(-(1 << 20), 1 << 20, m * ldc).astype(np.int32) if out == "i32" else \
        rng.integers(-128, 128, m * ldc).astype(np.int8)
    c = torch.from_numpy(c0.copy()).to(dev)
    st, route = uor.gemm_i8(a, (m, k), (lda, 1), bt, (k, n), (1, ldb), c, (m, n), (ldc, 1), out=out,
                            alpha=3, beta=-1, encode="saturating")
    torch.cuda.synchronize()
    assert st == 0 and route["kind"] == "mfma_tile" and route["tile_m"] == 256, route
    assert route["operand_modes"] >> 4 & 1, route  # the direct-to-LDS pipeline
    S = (a.view(m, lda)[:, :k].double() @ bt.view(n, ldb)[:, :k].double().t()).cpu().numpy()
    C0 = c0.reshape(m, ldc).astype(np.int64)
    want = 3 * S.astype(np.int64) - C0[:, :n]
    lo, hi = (-(1 << 31), (1 << 31) - 1) if out == "i32" else (-128, 127)
    want = np.clip(want, lo, hi)
    got = c.cpu().numpy().reshape(m, ldc)
    assert got.dtype == dt
    assert np.array_equal(got[:, :n].astype(np.int64), want)
    assert np.array_equal(got[:, n:], c0.reshape(m, ldc)[:, n:])


def check_small_tile(oracle, uor, dev, m, k, n, out, tile):
    """One call with ragged m and n, alpha = -3, beta = 2, saturating, on the
    route with `tile`-wide tiles.  Rows 0, 1, the last two and a middle one
    against the oracle, the rest against an exact float64 product."""
    rng = np.random.default_rng(m + 3 * k + 7 * n)
    lda, ldb, ldc = k + 16, n + 16, n + 4
    a = rng.integers(-128, 128, m * lda).astype(np.int8)
    b = rng.integers(-128, 128, k * ldb).astype(np.int8)
    ob = {"i8": 1, "i32": 4, "i64": 8, "i128": 16}[out]
    rec = 2 if out == "i128" else 1
    dt = {1: np.int8, 4: np.int32, 8: np.int64, 16: np.int64}[ob]
    info = np.iinfo(dt)
    c0 = rng.integers(max(info.min, -(1 << 40)), min(info.max, 1 << 40), m * ldc * rec, dtype=dt)
    gc = to_dev(c0, dev)
    st, route = uor.gemm_i8(to_dev(a, dev), (m, k), (lda, 1), to_dev(b, dev), (k, n), (ldb, 1), gc,
                            (m, n), (ldc, 1), out=out, alpha=-3, beta=2, encode="saturating")
    torch.cuda.synchronize()
    assert st == 0 and route["kind"] == "mfma_tile" and route["tile_m"] == tile, route
    assert route["operand_modes"] & (1 << 4), route  # the direct-to-LDS pipeline
    got = gc.cpu().numpy()
    rows = sorted({r for r in (0, 1, m // 2, m - 2, m - 1) if 0 <= r < m})
    for r in rows:
        want = c0.copy()
        sub_c = want[r * ldc * rec:(r * ldc + n) * rec].copy()
        assert oracle.gemm_int(a[r * lda:r * lda + k].copy(), (1, k), (k, 1), b, (k, n), (ldb, 1),
                               sub_c, (1, n), (1, 1), alpha=-3, beta=2, encode="saturating",
                               out_bytes=ob) == "ok"
        assert np.array_equal(got[r * ldc * rec:(r * ldc + n) * rec], sub_c), (r, route)
    if out in ("i32", "i64"):
        S = a.reshape(m, lda)[:, :k].astype(np.float64) @ b.reshape(k, ldb)[:, :n].astype(np.float64)
        want = np.clip(-3 * S.astype(np.int64) + 2 * c0.reshape(m, ldc)[:, :n].astype(np.int64),
                       info.min, info.max)
        assert np.array_equal(got.reshape(m, ldc)[:, :n].astype(np.int64), want)
    # the padding columns are untouched
    assert np.array_equal(got.reshape(m, ldc * rec)[:, n * rec:], c0.reshape(m, ldc * rec)[:, n * rec:])


@pytest.mark.parametrize("m,k,n", [(512 + 24, 2048 + 64, 2048 + 16), (260, 4096 + 64, 3840),
                                   (1024 + 64, 2048 + 128, 1024), (320, 2048 + 64, 3520)])
@pytest.mark.parametrize("out", ["i8", "i32", "i64", "i128"])
def test_tile128_below_one_round(oracle, uor, dev, m, k, n, out):
    """Fewer than 32 tiles of 256, more 64-wide tiles than CUs and k > 2048:
    the 128-wide direct-to-LDS tile with the fused epilogue, every output
    width (i128 through the parked full evaluation)."""
    check_small_tile(oracle, uor, dev, m, k, n, out, 128)


@pytest.mark.parametrize("m,k,n", [(1024, 1024, 1024), (256, 4096 + 64, 4096), (130, 64, 3008), (64, 8192, 4096),
                                   (1, 1024, 1024), (33, 192, 80), (200, 960, 1040), (16, 4096, 8192),
                                   (40, 4160, 8208), (1000, 2048, 2000)])
@pytest.mark.parametrize("out", ["i8", "i32", "i64", "i128"])
def test_ring64_one_round(oracle, uor, dev, m, k, n, out):
    """At most one 64-wide tile per CU (two at k <= 2048): the 64-wide
    direct-to-LDS tile with sixteen stages in flight; reductions shorter than
    the ring (1, 3 and 15 steps), as long as it (16), and longer (32, 64, 65,
    128), ragged m and n, skinny products the 256-wide tile took before."""
    check_small_tile(oracle, uor, dev, m, k, n, out, 64)


@pytest.mark.parametrize("m,k,n", [(128, 8192 + 64, 128), (200, 2 * 65536 + 192, 144),
                                   (64, 262144 + 64, 48)])
def test_splitk_interleaved_steps(uor, dev, m, k, n):
    """Split-K on the 128-wide direct-to-LDS tile (k % 64 == 0, n % 16 == 0):
    split z sums the units of four 64-deep steps z, z + splits, z + 2*splits,
    ...  The step counts (129, 2051, 4097) end in a short unit and leave some
    splits a unit short, and m, n leave partial edge tiles.  Random i8
    operands, i64 output with alpha = 3, beta = -1; expected values from an
    exact float64 product (|sum| <= k * 2^14 < 2^53)."""
    rng = np.random.default_rng(m + 3 * n + 5 * k)
    a = torch.from_numpy(rng.integers(-128, 128, m * k).astype(np.int8)).to(dev)
    b = torch.from_numpy(rng.integers(-128, 128, k * n).astype(np.int8)).to(dev)
    c0 = rng.integers(-(1 << 40), 1 << 40, m * n).astype(np.int64)
    c = torch.from_numpy(c0.copy()).to(dev)
    scratch = torch.empty(uor.suggested_scratch_i8(m, k, n), dtype=torch.uint8, device=dev)
    st, route = uor.gemm_i8(a, (m, k), (k, 1), b, (k, n), (n, 1), c, (m, n), (n, 1), out="i64",
                            alpha=3, beta=-1, scratch=scratch)
    torch.cuda.synchronize()
    assert st == 0 and route["kind"] == "mfma_splitk" and route["tile_m"] == 128, route
    S = (a.view(m, k).double() @ b.view(k, n).double()).cpu().numpy().astype(np.int64)
    want = 3 * S - c0.reshape(m, n)
    assert np.array_equal(c.cpu().numpy().reshape(m, n), want)


@pytest.mark.parametrize("m,k,n", [(40, (1 << 20) + 768, 144), (100, (1 << 20) + 256, 16)])
def test_splitk_narrow_tile_far_rows(uor, dev, m, k, n):
    """A rows 1 MiB or more apart take the 32x128 split-K tile (a CU touches
    32 row pages, not 128): ragged m and n, stage counts not a multiple of
    the split count.  Random i8 operands, i64 output with alpha = 3,
    beta = -1; expected values from an exact float64 product."""
    g = torch.Generator(device=dev).manual_seed(m + n)
    a = torch.randint(-128, 128, (m * k,), dtype=torch.int8, device=dev, generator=g)
    b = torch.randint(-128, 128, (k * n,), dtype=torch.int8, device=dev, generator=g)
    c0 = torch.randint(-(1 << 40), 1 << 40, (m * n,), dtype=torch.int64, device=dev, generator=g)
    c = c0.clone()
    scratch = torch.empty(uor.suggested_scratch_i8(m, k, n), dtype=torch.uint8, device=dev)
    st, route = uor.gemm_i8(a, (m, k), (k, 1), b, (k, n), (n, 1), c, (m, n), (n, 1), out="i64",
                            alpha=3, beta=-1, scratch=scratch)
    torch.cuda.synchronize()
    assert st == 0 and route["kind"] == "mfma_splitk" and route["tile_m"] == 32, route
    S = a.view(m, k).double() @ b.view(k, n).double()
    want = 3 * S.cpu().numpy().astype(np.int64) - c0.cpu().numpy().reshape(m, n)
    assert np.array_equal(c.cpu().numpy().reshape(m, n), want)


def test_splitk_narrow_tile_folds_segments(uor, dev):
    """The 32x128 split-K tile folds each split's i32 lanes into i64 every
    256 stages (65 536 terms): at k = 2^24 + 512 one tile takes one split per
    CU, and each split sums 256 or 257 stages (a fold, then for two of them
    one stage more).  Random operands against float64 (|sum| <= 2^38 <
    2^53)."""
    m, k, n = 32, (1 << 24) + 512, 16
    g = torch.Generator(device=dev).manual_seed(7)
    a = torch.randint(-128, 128, (m * k,), dtype=torch.int8, device=dev, generator=g)
    b = torch.randint(-128, 128, (k * n,), dtype=torch.int8, device=dev, generator=g)
    c = torch.zeros(m * n, dtype=torch.int64, device=dev)
    scratch = torch.empty(uor.suggested_scratch_i8(m, k, n), dtype=torch.uint8, device=dev)
    st, route = uor.gemm_i8(a, (m, k), (k, 1), b, (k, n), (n, 1), c, (m, n), (n, 1), out="i64",
                            scratch=scratch)
    torch.cuda.synchronize()
    assert st == 0 and route["tile_m"] == 32, route
    S = (a.view(m, k).double() @ b.view(k, n).double()).cpu().numpy().astype(np.int64)
    assert np.array_equal(c.cpu().numpy().reshape(m, n), S)


@pytest.mark.parametrize("m,k,n", [(512, 1024, 28672), (256, 2048, 28672), (300, 640, 20000),
                                   (16, 4096, 20480), (40, 4160, 16400), (100, 4096, 9008)])
@pytest.mark.parametrize("out", ["i32", "i64"])
def test_wide_tile_below_one_round(uor, dev, m, k, n, out):
    """Fewer 256-wide tiles than CUs, wide n (and from 16 rows at k >= 4096):
    the 256-wide tile (one round) rather than several rounds of narrower
    tiles; ragged edges included (rows past m read the last row).
    Checked in float64 on the device (|3 AB - C| < 2^53)."""
    g = torch.Generator(device=dev).manual_seed(m + n)
    a = torch.randint(-128, 128, (m * k,), dtype=torch.int8, device=dev, generator=g)
    b = torch.randint(-128, 128, (k * n,), dtype=torch.int8, device=dev, generator=g)
    dt = torch.int32 if out == "i32" else torch.int64
    c0 = torch.randint(-(1 << 20), 1 << 20, (m * n,), dtype=dt, device=dev, generator=g)
    c = c0.clone()
    st, route = uor.gemm_i8(a, (m, k), (k, 1), b, (k, n), (n, 1), c, (m, n), (n, 1), out=out,
                            alpha=3, beta=-1)
    torch.cuda.synchronize()
    assert st == 0 and route["kind"] == "mfma_tile" and route["tile_m"] == 256, route
    want = 3 * (a.view(m, k).double() @ b.view(k, n).double()) - c0.view(m, n).double()
    assert torch.equal(c.view(m, n).double(), want)
