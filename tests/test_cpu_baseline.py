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
