"""The CPU baseline (oracle/fastroute.cpp, the reference's packed route
restated) computes the oracle's bytes, on both its VNNI and AVX2 tiles."""
import numpy as np
import pytest


@pytest.mark.parametrize("avx2", [False, True])
@pytest.mark.parametrize("shape", [(1, 1, 1), (13, 17, 19), (130, 260, 1030), (9, 4096, 33)])
def test_fastroute_i8_matches_oracle(oracle, shape, avx2):
    if not avx2 and not oracle.fast().fr_has_vnni():
        pytest.skip("no AVX-512 VNNI on this host")
    m, k, n = shape
    rng = np.random.default_rng(m + k + n)
    lda, ldb, ldc = k + 3, n + 5, n + 1
    a = rng.integers(-128, 128, m * lda).astype(np.int8)
    b = rng.integers(-128, 128, k * ldb).astype(np.int8)
    c0 = rng.integers(-(1 << 20), 1 << 20, m * ldc).astype(np.int32)
    want = c0.copy()
    assert oracle.gemm_int(a, (m, k), (lda, 1), b, (k, n), (ldb, 1), want, (m, n), (ldc, 1),
                           alpha=3, beta=-1) == "ok"
    got = c0.copy()
    assert oracle.fast_gemm_i8_i32(m, k, n, 3, a, lda, b, ldb, -1, got, ldc, threads=3,
                                   force_avx2=avx2) == 0
    assert np.array_equal(got, want)


def test_fastroute_slab(oracle):
    m, k, n = 300, 64, 50
    rng = np.random.default_rng(3)
    a = rng.integers(-128, 128, m * k).astype(np.int8)
    b = rng.integers(-128, 128, k * n).astype(np.int8)
    full = np.zeros(m * n, np.int32)
    oracle.fast_gemm_i8_i32(m, k, n, 1, a, k, b, n, 0, full, n, threads=2)
    slab = np.zeros(m * n, np.int32)
    oracle.fast_gemm_i8_i32(m, k, n, 1, a, k, b, n, 0, slab, n, row0=128, rows=64, threads=2)
    s = slice(128 * n, 192 * n)
    assert np.array_equal(slab[s], full[s]) and not slab[:128 * n].any()


@pytest.mark.parametrize("mode", ["tabulate", "decode_dense"])
@pytest.mark.parametrize("m", [1, 3, 8, 19])
def test_fastroute_lut4_matches_oracle(oracle, m, mode):
    k, n, group = 256, 96, 32
    rng = np.random.default_rng(m)
    a = rng.integers(-128, 128, m * k).astype(np.int8)
    codes = rng.integers(0, 256, n * k // 2).astype(np.uint8)
    books = rng.integers(-128, 128, (n // group) * 16).astype(np.int8)
    books[:16] = -128                       # the extreme pair sum, 2 * 128 * 128
    a[:k] = -128
    want = np.zeros(m * n, np.int32)
    assert oracle.gemm_lut4(a, m, k, (k, 1), codes, n, books, group, want, (n, 1)) == "ok"
    got = np.full(m * n, 7, np.int32)
    assert oracle.fast_lut4(m, k, n, a, codes, books, group, got, threads=2, mode=mode) == 0
    assert np.array_equal(got, want)
    # A bounded sample: the first group only.
    part = np.full(m * n, 7, np.int32)
    assert oracle.fast_lut4(m, k, n, a, codes, books, group, part, groups=1, mode=mode) == 0
    g = part.reshape(m, n)
    assert np.array_equal(g[:, :group], want.reshape(m, n)[:, :group]) and (g[:, group:] == 7).all()


@pytest.mark.parametrize("shape", [(1, 1, 16), (5, 37, 32), (33, 300, 64)])
def test_fastroute_trop_matches_oracle(oracle, shape):
    m, k, n = shape
    rng = np.random.default_rng(k)

    def recs(count):
        r = np.zeros((count, 2), np.uint8)
        r[:, 0] = rng.integers(0, 256, count)
        r[:, 1] = rng.random(count) > 0.3
        return r.reshape(-1)

    a, b = recs(m * k), recs(k * n)
    a[0:2] = [0x80, 1]                      # -128, the lane's lowest finite value
    b.reshape(k, n, 2)[:, 1, 1] = 0         # column 1 is -inf in every row
    want = np.zeros(m * n * 8, np.uint8)
    assert oracle.gemm_trop(a, (m, k), (k, 1), b, (k, n), (n, 1), want, (m, n), (n, 1)) == "ok"
    got = np.full(m * n * 8, 0xEE, np.uint8)
    assert oracle.fast_trop_i8(m, k, n, a, b, got, threads=3) == 0
    g, w = got.reshape(-1, 8), want.reshape(-1, 8)
    assert np.array_equal(g[:, :5], w[:, :5])
    assert not w[:, 4].all() and w[:, 4].any()


def test_fastroute_chunked_depth_matches_oracle(oracle):
    """Past one i32 lane (three 65536-deep chunks and a ragged one), extremes
    planted: every term -128 * -128 in row 0 / column 0."""
    m, k, n = 9, 3 * 65536 + 256, 20
    rng = np.random.default_rng(17)
    a = rng.integers(-128, 128, m * k).astype(np.int8)
    b = rng.integers(-128, 128, k * n).astype(np.int8)
    a[:k] = -128
    b.reshape(k, n)[:, 0] = -128
    want = np.zeros(m * n, np.int64)
    assert oracle.gemm_int(a, (m, k), (k, 1), b, (k, n), (n, 1), want, (m, n), (n, 1)) == "ok"
    assert want[0] == k * 128 * 128
    got = np.full(m * n, 7, np.int64)
    assert oracle.fast_gemm_i8_i64_chunked(m, k, n, a, k, b, n, got, n, threads=3) == 0
    assert np.array_equal(got, want)
