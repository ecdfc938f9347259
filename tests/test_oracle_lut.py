"""Pins the LUT oracle (oracle/uor_oracle.c ora_gemm_lut4).

Witnesses: the reference's CK-03 nibble-order known answer (codec/tests/
codec.rs:84-110: byte 0x3A through the i - 8 table decodes low nibble first to
2, then -5), and decode-then-NumPy-matmul (the reference's own CD-13 argument:
the table route and the decode-then-dense route give the same bytes), with the
decode written here independently in NumPy.
"""
import numpy as np
import pytest


def decode_np(codes, n, k, books, group):
    c = codes.reshape(n, k // 2)
    lo = (c & 15).astype(np.int64)
    hi = (c >> 4).astype(np.int64)
    nib = np.empty((n, k), np.int64)
    nib[:, 0::2] = lo
    nib[:, 1::2] = hi
    g = (np.arange(n) // group)[:, None]
    return books.reshape(-1, 16)[g, nib].astype(np.int64)  # n x k


def test_nibble_order_ck03(oracle):
    table = np.arange(16, dtype=np.int8) - 8  # i4 table: i - 8
    a = np.array([1, 0], np.int8)            # picks weight k=0
    codes = np.array([0x3A], np.uint8)       # low nibble 0xA -> 2, high 0x3 -> -5
    c = np.zeros(1, np.int32)
    assert oracle.gemm_lut4(a, 1, 2, (2, 1), codes, 1, table, 1, c, (1, 1)) == "ok"
    assert c[0] == 2
    a = np.array([0, 1], np.int8)
    assert oracle.gemm_lut4(a, 1, 2, (2, 1), codes, 1, table, 1, c, (1, 1)) == "ok"
    assert c[0] == -5


@pytest.mark.parametrize("m,k,n,group", [(1, 2, 1, 1), (3, 64, 10, 4), (5, 256, 33, 16),
                                          (2, 1030, 7, 7), (4, 96, 130, 128)])
def test_decode_then_matmul(oracle, m, k, n, group):
    rng = np.random.default_rng(m * 1000 + k + n)
    a = rng.integers(-128, 128, m * k).astype(np.int8)
    codes = rng.integers(0, 256, n * k // 2).astype(np.uint8)
    books = rng.integers(-128, 128, ((n + group - 1) // group) * 16).astype(np.int8)
    c0 = rng.integers(-1000, 1000, m * n).astype(np.int32)
    W = decode_np(codes, n, k, books, group)
    want = 3 * (a.reshape(m, k).astype(np.int64) @ W.T) - 2 * c0.reshape(m, n)
    c = c0.copy()
    assert oracle.gemm_lut4(a, m, k, (k, 1), codes, n, books, group, c, (n, 1),
                            alpha=3, beta=-2) == "ok"
    assert np.array_equal(c.reshape(m, n), want)


def test_shape_errors(oracle):
    a = np.zeros(6, np.int8)
    books = np.zeros(16, np.int8)
    c = np.zeros(4, np.int32)
    # odd k: no Packed<_, 2> matrix of that width exists
    assert oracle.gemm_lut4(a, 2, 3, (3, 1), np.zeros(3, np.uint8), 2, books, 2, c, (2, 1)) == "short_buffer"
    # codes of the wrong length
    assert oracle.gemm_lut4(a, 2, 2, (2, 1), np.zeros(3, np.uint8), 2, books, 2, c, (2, 1)) == "short_buffer"
    # aliasing output
    assert oracle.gemm_lut4(a, 2, 2, (2, 1), np.zeros(2, np.uint8), 2, books, 2, c, (0, 1)) == "output_aliases_itself"
