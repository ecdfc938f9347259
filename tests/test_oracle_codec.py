"""The oracle's codec decode (oracle/uor_oracle.c ora_coded_decode) pinned by
the reference's own known answers (crates/uor-matmul-codec/tests/codec.rs):
CK-03 nibble and 2-bit order, CK-05 three tiers with one decode, CK-01 Offset
as asymmetric quantization, CK-11 Sign<8> = Packed<Grid<2>,8> and CK-12
Ternary<4> = Packed<Grid<4>,4> over all 256 codes, and the code-width guard
of Sign/Ternary.  Then gemm_coded against a NumPy matmul of the decode."""
import numpy as np
import pytest

I4 = np.arange(16, dtype=np.int8) - 8  # i4_table (codec.rs:21-23)


def test_ck03_low_sub_code_first(oracle):
    # codec.rs:91-116: 0x3A -> (2, -5) over the i4 grid; 0xE4 -> 0, 1, 2, 3.
    cd = oracle.codec("grid", packed=2, table=I4)
    st, w = oracle.coded_decode(cd, np.array([0x3A], np.uint8), 1, 2)
    assert st == "ok" and w.tolist() == [[2, -5]]
    quad = oracle.codec("grid", packed=4, table=np.arange(4, dtype=np.int8))
    st, w = oracle.coded_decode(quad, np.array([0xE4], np.uint8), 1, 4)
    assert st == "ok" and w.tolist() == [[0, 1, 2, 3]]


def test_ck05_three_tiers_one_decode(oracle):
    # codec.rs:147-181: Book<4, 8> codes [0,1,2,3], Identity over the dense
    # stream, Grid<32> codes 0..31: equal decodes and equal products.
    book_table = (np.arange(32) - 16).astype(np.int8)
    dense = (np.arange(32) - 16).astype(np.int8)
    st, wb = oracle.coded_decode(oracle.codec("book", table=book_table, block=8),
                                 np.array([0, 1, 2, 3], np.uint16), 4, 8)
    assert st == "ok"
    st, wi = oracle.coded_decode(oracle.codec("identity", code_bits=8),
                                 dense.view(np.uint8), 4, 8)
    assert st == "ok"
    st, wg = oracle.coded_decode(oracle.codec("grid", table=book_table),
                                 np.arange(32, dtype=np.uint16), 4, 8)
    assert st == "ok"
    assert np.array_equal(wb, wi) and np.array_equal(wg, wi)
    assert np.array_equal(wi.reshape(-1), dense)
    acts = (np.arange(8) * 7 - 20).astype(np.int8)
    for r in range(4):
        want = int(acts.astype(np.int64) @ wi[r].astype(np.int64))
        assert int(acts.astype(np.int64) @ wb[r].astype(np.int64)) == want
        assert int(acts.astype(np.int64) @ wg[r].astype(np.int64)) == want


def test_ck01_offset(oracle):
    # codec.rs:187-203: Grid<16> over 0..15 with zero point 8 decodes c - 8.
    cd = oracle.codec("grid", table=np.arange(16, dtype=np.int8), zero=8)
    st, w = oracle.coded_decode(cd, np.arange(16, dtype=np.uint16), 1, 16)
    assert st == "ok" and w.tolist() == [list(range(-8, 8))]


def test_ck11_sign_is_packed_grid2(oracle):
    # codec.rs:775-815: all 256 codes, block 8.
    codes = np.arange(256, dtype=np.uint16)
    st, ws = oracle.coded_decode(oracle.codec("sign", code_bits=16, block=8), codes, 256, 8)
    assert st == "ok"
    packed = oracle.codec("grid", packed=8, table=np.array([-1, 1], np.int8))
    st, wp = oracle.coded_decode(packed, codes.astype(np.uint8), 256, 8)
    assert st == "ok" and np.array_equal(ws, wp)
    # and the u8 spelling of the same tier
    st, w8 = oracle.coded_decode(oracle.codec("sign", code_bits=8, block=8),
                                 codes.astype(np.uint8), 256, 8)
    assert st == "ok" and np.array_equal(w8, ws)


def test_ck12_ternary_is_packed_grid4(oracle):
    # codec.rs:830-877: all 256 codes, block 4, table [-1, 0, 1, 0].
    codes = np.arange(256, dtype=np.uint16)
    st, wt = oracle.coded_decode(oracle.codec("ternary", code_bits=16, block=4), codes, 256, 4)
    assert st == "ok"
    packed = oracle.codec("grid", packed=4, table=np.array([-1, 0, 1, 0], np.int8))
    st, wp = oracle.coded_decode(packed, codes.astype(np.uint8), 256, 4)
    assert st == "ok" and np.array_equal(wt, wp)


def test_sign_ternary_past_the_code_width(oracle):
    # codecs.rs:387-400, 492-516: positions the code type has no bit (digit)
    # for decode like a clear bit (a zero digit): -1.
    st, w = oracle.coded_decode(oracle.codec("sign", code_bits=8, block=12),
                                np.array([0xFF], np.uint8), 1, 12)
    assert st == "ok" and w.tolist() == [[1] * 8 + [-1] * 4]
    st, w = oracle.coded_decode(oracle.codec("ternary", code_bits=8, block=6),
                                np.array([0b10101010], np.uint8), 1, 6)
    assert st == "ok" and w.tolist() == [[1, 1, 1, 1, -1, -1]]


def test_packed_book_and_shapes(oracle):
    # Packed<Book<4, 2, u8>, 2>: MAX_BLOCK 4; sub-code s of a byte names
    # Book row s % 4, positions 2p, 2p+1.
    table = np.array([10, 11, 20, 21, 30, 31, 40, 41], np.int8)
    cd = oracle.codec("book", code_bits=8, packed=2, table=table, block=2)
    st, w = oracle.coded_decode(cd, np.array([0x21, 0x0F], np.uint8), 2, 4)
    assert st == "ok" and w.tolist() == [[20, 21, 30, 31], [40, 41, 10, 11]]
    # CodedMatrix::new refusals (matrix.rs:36-55): width not a multiple of
    # MAX_BLOCK, wrong code count.
    assert oracle.coded_decode(cd, np.array([0x21], np.uint8), 1, 6)[0] == "short_buffer"
    assert oracle.coded_decode(cd, np.array([0x21], np.uint8), 2, 4)[0] == "short_buffer"
    # a table shorter than N * BLK, an unknown tier, P not dividing 8
    assert oracle.coded_decode(oracle.codec("book", table=table[:7], entries=4, block=2),
                               np.zeros(2, np.uint16), 1, 4)[0] == "short_buffer"
    bad = dict(cd, tier=9)
    assert oracle.coded_decode(bad, np.zeros(2, np.uint8), 1, 8)[0] == "invalid_argument"
    bad = dict(cd, packed=3)
    assert oracle.coded_decode(bad, np.zeros(2, np.uint8), 1, 8)[0] == "invalid_argument"


def test_offset_wraps_like_i8_sub(oracle):
    # Offset::decode_element is i8 wrapping_sub (alphabet.rs:605-607).
    cd = oracle.codec("grid", table=np.array([-128, 127, 0], np.int8), zero=-1)
    st, w = oracle.coded_decode(cd, np.array([0, 1, 2], np.uint16), 1, 3)
    assert st == "ok" and w.tolist() == [[-127, -128, 1]]


@pytest.mark.parametrize("transposed", [True, False])
def test_gemm_coded_is_decode_then_matmul(oracle, transposed):
    rng = np.random.default_rng(5)
    m, k = 7, 24
    n = 10 if transposed else 12  # the coded width is a multiple of MAX_BLOCK = 4
    cd = oracle.codec("ternary", code_bits=8, block=4)
    rows, cols = (n, k) if transposed else (k, n)
    codes = rng.integers(0, 256, rows * cols // 4).astype(np.uint8)
    st, w = oracle.coded_decode(cd, codes, rows, cols)
    assert st == "ok"
    a = rng.integers(-128, 128, m * k).astype(np.int8)
    c = rng.integers(-1000, 1000, m * n).astype(np.int32)
    want = c.astype(np.int64).reshape(m, n) * -2
    ww = w.T if transposed else w
    want += 3 * (a.astype(np.int64).reshape(m, k) @ ww.astype(np.int64))
    st = oracle.gemm_coded(a, (m, k), (k, 1), cd, codes, rows, cols, transposed, c, (m, n),
                           (n, 1), alpha=3, beta=-2)
    assert st == "ok"
    assert np.array_equal(c.astype(np.int64).reshape(m, n), want)
