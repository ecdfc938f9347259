"""GPU parity of the collapse traversal (uor_gfx950_gemm_collapsed_i8, through
the C ABI): the plain product's bytes (the reference's CD-12), checked against
both the oracle (ora_gemm_int, driver::gemm) and the plain GPU route, with
repeated rows of A (or columns of B), the cases that must run the plain route
(beta != 0, pairwise distinct lines, no offer, k = 0), strided views and every
output width.

Bar: bit-exact."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

OUTDT = {"i8": np.int8, "i16": np.int16, "i32": np.int32, "i64": np.int64}


def repeated(rng, lines, distinct, length):
    """`lines` lines of `length` bytes drawn from `distinct` random ones."""
    base = rng.integers(-128, 128, (distinct, length)).astype(np.int8)
    pick = rng.integers(0, distinct, lines)
    pick[:distinct] = np.arange(distinct)  # every class appears
    rng.shuffle(pick)
    return base[pick]


def run(oracle, uor, dev, a2, b2, out="i32", alpha=1, beta=0, encode="nearest", columns=False,
        offer=True, a_cm=False, c_cm=False, seed=0):
    rng = np.random.default_rng(seed)
    m, k = a2.shape
    n = b2.shape[1]
    a = np.ascontiguousarray(a2.T if a_cm else a2).reshape(-1)
    a_str = (1, m) if a_cm else (k, 1)
    b = np.ascontiguousarray(b2).reshape(-1)
    c_str = (1, m) if c_cm else (n, 1)
    c0 = rng.integers(-1000, 1000, max(m * n, 1)).astype(OUTDT[out])
    want = c0.copy()
    st = oracle.gemm_int(a if a.size else np.zeros(1, np.int8), (m, k), a_str,
                         b if b.size else np.zeros(1, np.int8), (k, n), (n, 1), want, (m, n), c_str,
                         alpha=alpha, beta=beta, encode=encode)
    assert st == "ok"
    ga = torch.from_numpy(a if a.size else np.zeros(1, np.int8)).to(dev)
    gb = torch.from_numpy(b if b.size else np.zeros(1, np.int8)).to(dev)
    gc = torch.from_numpy(c0.copy()).to(dev)
    gp = torch.from_numpy(c0.copy()).to(dev)
    scratch = None
    if offer:
        nb = uor.suggested_scratch_collapse(m, k, n)
        scratch = torch.empty(max(nb, 1), dtype=torch.uint8, device=dev)
    gst, route = uor.gemm_collapsed_i8(ga, (m, k), a_str, gb, (k, n), (n, 1), gc, (m, n), c_str,
                                       out=out, alpha=alpha, beta=beta, encode=encode,
                                       columns=columns, scratch=scratch)
    pst, _ = uor.gemm_i8(ga, (m, k), a_str, gb, (k, n), (n, 1), gp, (m, n), c_str, out=out,
                         alpha=alpha, beta=beta, encode=encode)
    torch.cuda.synchronize()
    assert gst == 0 and pst == 0
    assert np.array_equal(gc.cpu().numpy(), want), route
    assert torch.equal(gc, gp)
    return route


@pytest.mark.parametrize("m,k,n,distinct", [(300, 257, 70, 17), (64, 8, 33, 1), (1000, 96, 40, 999),
                                            (4100, 130, 20, 64)])
def test_rows(oracle, uor, dev, m, k, n, distinct):
    rng = np.random.default_rng(m + k)
    a = repeated(rng, m, distinct, k)
    b = rng.integers(-128, 128, (k, n)).astype(np.int8)
    route = run(oracle, uor, dev, a, b, alpha=3, seed=1)
    assert route["kind"] == "collapsed" and route["moduli"] == distinct, route


@pytest.mark.parametrize("k", [8, 130, 200])
def test_rows_aligned_padded(oracle, uor, dev, k):
    """Rows that start 16 bytes apart with a stride past k (random padding):
    the pass reads them 16 bytes at a time with a ragged tail, and the
    padding never enters a class (the distinct count is the data's)."""
    rng = np.random.default_rng(k)
    m, n, distinct = 300, 40, 23
    ld = (k + 15) // 16 * 16 + 16
    a2 = repeated(rng, m, distinct, k)
    buf = rng.integers(-128, 128, (m, ld)).astype(np.int8)
    buf[:, :k] = a2
    b = rng.integers(-128, 128, (k, n)).astype(np.int8).reshape(-1)
    want = np.zeros(m * n, np.int32)
    assert oracle.gemm_int(buf.reshape(-1), (m, k), (ld, 1), b, (k, n), (n, 1), want, (m, n), (n, 1),
                           alpha=3) == "ok"
    ga = torch.from_numpy(buf.reshape(-1).copy()).to(dev)
    gb = torch.from_numpy(b).to(dev)
    gc = torch.zeros(m * n, dtype=torch.int32, device=dev)
    sc = torch.empty(uor.suggested_scratch_collapse(m, k, n), dtype=torch.uint8, device=dev)
    st, route = uor.gemm_collapsed_i8(ga, (m, k), (ld, 1), gb, (k, n), (n, 1), gc, (m, n), (n, 1),
                                      out="i32", alpha=3, scratch=sc)
    torch.cuda.synchronize()
    assert st == 0 and route["kind"] == "collapsed" and route["moduli"] == distinct, route
    assert np.array_equal(gc.cpu().numpy(), want)


def test_columns(oracle, uor, dev):
    rng = np.random.default_rng(2)
    m, k, n = 50, 77, 400
    a = rng.integers(-128, 128, (m, k)).astype(np.int8)
    b = repeated(rng, n, 9, k).T.copy()
    route = run(oracle, uor, dev, a, b, alpha=-2, columns=True, seed=2)
    assert route["kind"] == "collapsed" and route["moduli"] == 9, route


@pytest.mark.parametrize("out", ["i8", "i16", "i32", "i64"])
@pytest.mark.parametrize("encode", ["nearest", "wrapping"])
def test_outputs_and_strides(oracle, uor, dev, out, encode):
    rng = np.random.default_rng(3)
    a = repeated(rng, 90, 7, 45)
    b = rng.integers(-128, 128, (45, 31)).astype(np.int8)
    for a_cm, c_cm, columns in ((False, False, False), (True, False, False), (False, True, False),
                                (True, True, True)):
        route = run(oracle, uor, dev, a, b, out=out, alpha=1 << 40, encode=encode, columns=columns,
                    a_cm=a_cm, c_cm=c_cm, seed=4)
        if not columns:
            assert route["kind"] == "collapsed" and route["moduli"] == 7, route


def test_plain_route_cases(oracle, uor, dev):
    """beta != 0 (the epilogue reads C), pairwise distinct rows, no offer:
    the plain route, the same bytes."""
    rng = np.random.default_rng(5)
    a = repeated(rng, 40, 5, 64)
    b = rng.integers(-128, 128, (64, 24)).astype(np.int8)
    assert run(oracle, uor, dev, a, b, beta=-1, seed=5)["kind"] != "collapsed"
    assert run(oracle, uor, dev, a, b, offer=False, seed=6)["kind"] != "collapsed"
    distinct = rng.integers(-128, 128, (40, 64)).astype(np.int8)
    assert run(oracle, uor, dev, distinct, b, seed=7)["kind"] != "collapsed"
    empty_k = np.zeros((40, 0), np.int8)
    assert run(oracle, uor, dev, empty_k, np.zeros((0, 24), np.int8), seed=8)["kind"] != "collapsed"
