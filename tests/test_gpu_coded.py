"""GPU parity of products with one coded operand (uor_gfx950_gemm_coded, through
the C ABI) against the oracle (oracle/uor_oracle.c ora_coded_decode, then
ora_gemm_int over the decoded operand -- the decode-then-multiply value the
reference's CD-13 names).

Every fixed-width tier over the i8 alphabet -- Identity, Grid<N> (power of two
and not, past u16), Book<N,BLK,K>, Sign<BLK,K>, Ternary<BLK,K>, inside Packed<_,
P> and Offset<_, zero> -- in both orientations (gemm_tabulated: W n x k;
coded_gemm: W k x n), both routes (decode into the scratch then the dense int8
route; no offer: the per-cell loop), output widths, alpha/beta, the
CodedMatrix/triple statuses, and the 4-bit codec against gemm_lut4.

Bar: bit-exact."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

OUTDT = {"i8": np.int8, "i16": np.int16, "i32": np.int32, "i64": np.int64}

I4 = np.arange(16, dtype=np.int8) - 8

SPECS = {
    "identity": dict(tier="identity", code_bits=8),
    "packed_grid16_p2": dict(tier="grid", packed=2, table=I4),
    "packed_grid4_p4": dict(tier="grid", packed=4, table=np.array([-1, 0, 1, 0], np.int8)),
    "grid300": dict(tier="grid", table=(np.arange(300) % 251 - 125).astype(np.int8)),
    "grid70000": dict(tier="grid", table=((np.arange(70000) * 7) % 255 - 127).astype(np.int8)),
    "book256x8": dict(tier="book", block=8, table=((np.arange(2048) * 13) % 256 - 128).astype(np.int8)),
    "book64x3_u8": dict(tier="book", code_bits=8, block=3,
                        table=((np.arange(192) * 5) % 256 - 128).astype(np.int8)),
    "packed_book4x2_p2": dict(tier="book", code_bits=8, packed=2, block=2,
                              table=np.array([10, 11, -20, 21, 30, -31, 40, 41], np.int8)),
    "sign8": dict(tier="sign", block=8),
    "sign8_u8": dict(tier="sign", code_bits=8, block=8),
    "sign12_u8": dict(tier="sign", code_bits=8, block=12),
    "sign16": dict(tier="sign", block=16),
    "ternary4_u8": dict(tier="ternary", code_bits=8, block=4),
    "ternary6_u8": dict(tier="ternary", code_bits=8, block=6),
    "ternary8": dict(tier="ternary", block=8),
    "packed_sign2_p4": dict(tier="sign", code_bits=8, packed=4, block=2),
    "offset_grid16": dict(tier="grid", table=np.arange(16, dtype=np.int8), zero=8),
    "offset_packed_grid16": dict(tier="grid", packed=2, table=np.arange(16, dtype=np.int8),
                                 zero=-3),
    "offset_ternary_wraps": dict(tier="ternary", code_bits=8, block=4, zero=-128),
}


def code_bytes(spec):
    return 1 if spec.get("packed") or spec.get("code_bits", 16) == 8 else 2


def table_variant(spec, m, k):
    """The few-rows code-table kernel's conditions at a row-major A of depth k."""
    mb, cb = max_block(spec), code_bytes(spec)
    win = k % 16 == 0 and (k // mb) * cb % 16 == 0 and (16 // cb) * mb % 16 == 0
    return win and cb == 1 and ((mb in (4, 8) and m <= 4) or (mb == 4 and m <= 8))


def max_block(spec):
    ib = spec.get("block", 1) if spec["tier"] in ("book", "sign", "ternary") else 1
    return (spec.get("packed") or 1) * ib


def run(oracle, uor, dev, spec, m, k, n, transposed, offer, out="i32", alpha=1, beta=0,
        encode="nearest", seed=0, codes_len_delta=0, c_strides=None, offer_shift=0):
    rng = np.random.default_rng(seed)
    rows, cols = (n, k) if transposed else (k, n)
    mb = max_block(spec)
    ncodes = rows * cols // mb + codes_len_delta
    wide = not spec.get("packed") and spec.get("code_bits", 16) == 16
    codes = rng.integers(0, 1 << 16 if wide else 1 << 8, max(ncodes, 0)).astype(
        np.uint16 if wide else np.uint8)
    a = rng.integers(-128, 128, max(m * k, 1)).astype(np.int8)
    cs = c_strides or (n, 1)
    clen = max(1 + (m - 1) * abs(cs[0]) + (n - 1) * abs(cs[1]), 1) if m and n else 1
    c0 = rng.integers(-1000, 1000, clen).astype(OUTDT[out])
    kw = {x: spec[x] for x in ("code_bits", "packed", "zero", "block") if x in spec}
    table = spec.get("table")
    ocd = oracle.codec(spec["tier"], table=table, **kw)
    want = c0.copy()
    st = oracle.gemm_coded(a, (m, k), (k, 1), ocd, codes, rows, cols, transposed, want, (m, n),
                           cs, alpha=alpha, beta=beta, encode=encode)
    gtable = None if table is None else torch.from_numpy(table).to(dev)
    gcd = uor.codec(spec["tier"], table=gtable, **kw)
    gcodes = torch.from_numpy(codes.view(np.int16) if wide else codes).to(dev)
    gc = torch.from_numpy(c0.copy()).to(dev)
    scratch = None
    if offer:
        nb = uor.suggested_scratch_coded(m, k, n)
        # offer_shift: a sub-buffer that starts off any aligned boundary.
        scratch = torch.empty(nb + offer_shift, dtype=torch.uint8, device=dev)[offer_shift:] if nb else None
    gst, route = uor.gemm_coded(torch.from_numpy(a).to(dev), (m, k), (k, 1), gcd, gcodes, rows,
                                cols, transposed, gc, (m, n), cs, out=out, alpha=alpha,
                                beta=beta, encode=encode, scratch=scratch)
    torch.cuda.synchronize()
    assert uor.STATUS.get(gst, gst) == st, (gst, st, route)
    assert np.array_equal(gc.cpu().numpy(), want), (spec, m, k, n, transposed, route)
    return st, route


@pytest.mark.parametrize("name", sorted(SPECS))
@pytest.mark.parametrize("transposed", [True, False])
@pytest.mark.parametrize("offer", [True, False])
@pytest.mark.parametrize("m", [5, 9])
def test_tiers_against_oracle(oracle, uor, dev, name, transposed, offer, m):
    """k and n multiples of 48 (every MAX_BLOCK here divides 48).  W n x k
    with m <= 8 decodes in registers whatever the offer."""
    k, n = 96, 48
    st, route = run(oracle, uor, dev, SPECS[name], m, k, n, transposed, offer, alpha=3, beta=-2,
                    seed=len(name) + m)
    assert st == "ok"
    # Past four rows the register route keeps only the code-table variant
    # when the offer would hold the decode-into-scratch route.
    few = transposed and m <= 8 and (m <= 4 or table_variant(SPECS[name], m, k) or not offer)
    want = "coded_gemv" if few else "coded_dense" if offer else "coded_direct"
    assert route["kind"] == want, route


@pytest.mark.parametrize("name", ["packed_grid16_p2", "sign12_u8", "ternary6_u8", "book64x3_u8",
                                  "grid300", "offset_ternary_wraps"])
@pytest.mark.parametrize("m", [1, 2, 3, 8])
def test_few_rows_ragged_depth(oracle, uor, dev, name, m):
    """The register-decode route: depths that leave lane slices ragged (k not
    a multiple of 16 or of 64 x 16, and shorter than 64 lanes' worth) and a
    depth of several thousand, 1 to 8 rows."""
    mb = max_block(SPECS[name])
    for k in (mb * 7, mb * 40, mb * 1000):
        st, route = run(oracle, uor, dev, SPECS[name], m, k, 37, True, False, alpha=-2, beta=1,
                        seed=k + m)
        assert st == "ok" and route["kind"] == "coded_gemv", route


@pytest.mark.parametrize("name", sorted(SPECS))
@pytest.mark.parametrize("m", [1, 3, 8])
def test_few_rows_code_windows(oracle, uor, dev, name, m):
    """Rows of W that are whole 16-byte code windows: the windowed variant of
    the register-decode route (one window per lane and step), and for
    one-byte codes of 4 or 8 elements at m <= 4 its table variant; fewer
    windows than lanes and several steps per row, n not a multiple of the 4
    columns a wave takes."""
    spec = SPECS[name]
    mb = max_block(spec)
    cb = 1 if spec.get("packed") or spec.get("code_bits", 16) == 8 else 2
    for wins in (5, 150):
        k = 16 * wins * mb // cb
        st, route = run(oracle, uor, dev, spec, m, k, 37, True, False, alpha=3, beta=-1,
                        seed=k + m + len(name))
        assert st == "ok" and route["kind"] == "coded_gemv", route
        a_vec = k % 16 == 0
        win = a_vec and (16 // cb) * mb % 16 == 0
        lut = table_variant(spec, m, k)
        assert route["operand_modes"] == (3 if lut else 2 if win else 1 if a_vec else 0), route


def test_few_rows_strided_a(oracle, uor, dev):
    """A read element by element (column-major and padded rows) on the
    register-decode route."""
    rng = np.random.default_rng(4)
    m, k, n = 3, 200, 40
    spec = SPECS["ternary4_u8"]
    codes = rng.integers(0, 256, n * k // 4).astype(np.uint8)
    for a_str, alen in (((1, m), m * k), ((k + 5, 1), m * (k + 5))):
        a = rng.integers(-128, 128, alen).astype(np.int8)
        want = np.zeros(m * n, np.int32)
        ocd = oracle.codec("ternary", code_bits=8, block=4)
        assert oracle.gemm_coded(a, (m, k), a_str, ocd, codes, n, k, True, want, (m, n),
                                 (n, 1)) == "ok"
        gc = torch.zeros(m * n, dtype=torch.int32, device=dev)
        st, route = uor.gemm_coded(torch.from_numpy(a).to(dev), (m, k), a_str,
                                   uor.codec("ternary", code_bits=8, block=4),
                                   torch.from_numpy(codes).to(dev), n, k, True, gc, (m, n),
                                   (n, 1))
        torch.cuda.synchronize()
        assert st == 0 and route["kind"] == "coded_gemv" and route["operand_modes"] == 0, route
        assert np.array_equal(gc.cpu().numpy(), want), a_str


@pytest.mark.parametrize("name", ["packed_grid16_p2", "sign8", "ternary4_u8", "book256x8",
                                  "offset_packed_grid16"])
@pytest.mark.parametrize("transposed", [True, False])
def test_larger_shapes_dense_route(oracle, uor, dev, name, transposed):
    """Ragged tiles on both edges of the decode (n, k not multiples of 128)
    and a dense route of several tiles."""
    m, k, n = 130, 432, 288
    st, route = run(oracle, uor, dev, SPECS[name], m, k, n, transposed, True, seed=7)
    assert st == "ok" and route["kind"] == "coded_dense", route


@pytest.mark.parametrize("shift", [1, 4, 12])
@pytest.mark.parametrize("transposed", [True, False])
def test_dense_route_unaligned_offer(oracle, uor, dev, shift, transposed):
    """The decoded operand (16-byte stores) and the dense route's offer are
    carved from the offer's first aligned byte, so a suggested offer that
    starts anywhere still takes the dense route, with the oracle's bytes."""
    st, route = run(oracle, uor, dev, SPECS["ternary4_u8"], 130, 256, 200, transposed, True,
                    alpha=3, beta=-2, seed=shift, offer_shift=shift)
    assert st == "ok" and route["kind"] == "coded_dense", route


@pytest.mark.parametrize("name", ["ternary4_u8", "sign8_u8", "packed_sign2_p4", "packed_grid4_p4",
                                  "packed_book4x2_p2", "offset_ternary_wraps"])
def test_dense_route_code_table_decode(oracle, uor, dev, name):
    """W n x k with one-byte codes of 4 or 8 elements in whole 16-byte row
    runs (k a multiple of 128): the decode into the scratch expands codes
    through a per-workgroup table; n ragged against the 128-column tile."""
    for k in (128, 640):
        st, route = run(oracle, uor, dev, SPECS[name], 40, k, 200, True, True, alpha=-3, beta=2,
                        seed=k + len(name))
        assert st == "ok" and route["kind"] == "coded_dense", route


@pytest.mark.parametrize("out", ["i8", "i16", "i32", "i64"])
@pytest.mark.parametrize("encode", ["nearest", "wrapping"])
@pytest.mark.parametrize("offer", [True, False])
def test_outputs_and_encodes(oracle, uor, dev, out, encode, offer):
    for m in (4, 9):  # the register-decode route, then dense / per-cell
        for alpha, beta in [(1, 0), (7, -3), (1 << 40, 5)]:
            run(oracle, uor, dev, SPECS["ternary8"], m, 48, 96, True, offer, out=out, alpha=alpha,
                beta=beta, encode=encode, seed=3)


def test_strided_output_and_empty(oracle, uor, dev):
    spec = SPECS["sign8"]
    run(oracle, uor, dev, spec, 6, 48, 16, True, True, c_strides=(1, 6))      # column-major C
    run(oracle, uor, dev, spec, 6, 48, 16, False, False, c_strides=(-16, 1))  # reversed rows
    st, route = run(oracle, uor, dev, spec, 6, 0, 16, True, True, alpha=2, beta=-1)  # k = 0
    assert st == "ok" and route["kind"] == "epilogue_only", route
    run(oracle, uor, dev, spec, 0, 48, 16, True, True)                        # m = 0


def test_statuses(oracle, uor, dev):
    spec = SPECS["ternary4_u8"]
    # a code count CodedMatrix::new refuses
    st, _ = run(oracle, uor, dev, spec, 4, 48, 16, True, True, codes_len_delta=1)
    assert st == "short_buffer"
    st, _ = run(oracle, uor, dev, spec, 4, 48, 16, False, False, codes_len_delta=-1)
    assert st == "short_buffer"
    # a width that is not a multiple of MAX_BLOCK (k = 50 along W's rows)
    st, _ = run(oracle, uor, dev, spec, 4, 50, 16, True, True)
    assert st == "short_buffer"
    # an aliasing output
    st, _ = run(oracle, uor, dev, spec, 4, 48, 16, True, True, c_strides=(0, 1))
    assert st == "output_aliases_itself"
    # nonconformant: A's depth differs from W's
    a = torch.zeros(4 * 40, dtype=torch.int8, device=dev)
    codes = torch.zeros(16 * 48 // 4, dtype=torch.uint8, device=dev)
    c = torch.zeros(4 * 16, dtype=torch.int32, device=dev)
    gst, _ = uor.gemm_coded(a, (4, 40), (40, 1), uor.codec("ternary", code_bits=8, block=4),
                            codes, 16, 48, True, c, (4, 16), (16, 1))
    assert uor.STATUS[gst] == "nonconformant"
    # a tier the library does not know, and P not dividing 8
    for bad in (uor.codec(9, code_bits=8), uor.codec("sign", code_bits=8, packed=3, block=2)):
        gst, _ = uor.gemm_coded(a, (4, 40), (40, 1), bad, codes, 16, 48, True, c, (4, 16),
                                (16, 1))
        assert uor.STATUS[gst] == "invalid_argument"


def test_four_bit_codec_equals_lut4(uor, dev):
    """Packed<Grid<16>,2> through gemm_coded (one codebook) and through
    gemm_lut4 (group = n): the same bytes."""
    rng = np.random.default_rng(9)
    for m, offer in ((33, True), (33, False), (1, False), (8, False)):
        k, n = 512, 200
        a = torch.from_numpy(rng.integers(-128, 128, m * k).astype(np.int8)).to(dev)
        codes = torch.from_numpy(rng.integers(0, 256, n * k // 2).astype(np.uint8)).to(dev)
        book = torch.from_numpy((rng.integers(-128, 128, 16)).astype(np.int8)).to(dev)
        c1 = torch.zeros(m * n, dtype=torch.int32, device=dev)
        c2 = torch.zeros(m * n, dtype=torch.int32, device=dev)
        nb = uor.suggested_scratch_coded(m, k, n) if offer else 0
        scratch = torch.empty(nb, dtype=torch.uint8, device=dev) if nb else None
        st, _ = uor.gemm_coded(a, (m, k), (k, 1), uor.codec("grid", packed=2, table=book), codes,
                               n, k, True, c1, (m, n), (n, 1), scratch=scratch)
        assert st == 0
        st, _ = uor.gemm_lut4(a, m, k, (k, 1), codes, n, book, n, c2, (n, 1))
        assert st == 0
        torch.cuda.synchronize()
        assert torch.equal(c1, c2), offer


@pytest.mark.parametrize("name", ["ternary4_u8", "packed_grid16_p2", "book256x8", "sign12_u8"])
@pytest.mark.parametrize("transposed", [True, False])
@pytest.mark.parametrize("m,distinct", [(40, 4), (300, 20)])
def test_row_collapse(oracle, uor, dev, name, transposed, m, distinct):
    """gemm_coded_collapsed: A's rows drawn from a few distinct ones share
    product rows (the inner product then runs on d rows: the register route
    at d <= 8 for W n x k); the bytes are the oracle's and the plain coded
    route's.  beta != 0 and no offer run the plain routes."""
    spec = SPECS[name]
    rng = np.random.default_rng(m + len(name))
    k, n = 96, 48
    rows, cols = (n, k) if transposed else (k, n)
    mb = max_block(spec)
    wide = not spec.get("packed") and spec.get("code_bits", 16) == 16
    codes = rng.integers(0, 1 << 16 if wide else 1 << 8, rows * cols // mb).astype(
        np.uint16 if wide else np.uint8)
    base = rng.integers(-128, 128, (distinct, k)).astype(np.int8)
    pick = rng.integers(0, distinct, m)
    pick[:distinct] = np.arange(distinct)
    a = base[pick].reshape(-1).copy()
    kw = {x: spec[x] for x in ("code_bits", "packed", "zero", "block") if x in spec}
    table = spec.get("table")
    gtable = None if table is None else torch.from_numpy(table).to(dev)
    gcd = uor.codec(spec["tier"], table=gtable, **kw)
    gcodes = torch.from_numpy(codes.view(np.int16) if wide else codes).to(dev)
    ga = torch.from_numpy(a).to(dev)
    for beta, offer, want_kind in ((0, True, "collapsed"), (2, True, None), (0, False, None)):
        c0 = rng.integers(-1000, 1000, m * n).astype(np.int32)
        want = c0.copy()
        ocd = oracle.codec(spec["tier"], table=table, **kw)
        assert oracle.gemm_coded(a, (m, k), (k, 1), ocd, codes, rows, cols, transposed, want,
                                 (m, n), (n, 1), alpha=-3, beta=beta) == "ok"
        gc = torch.from_numpy(c0.copy()).to(dev)
        nb = uor.suggested_scratch_coded_collapse(m, k, n) if offer else 0
        scratch = torch.empty(nb, dtype=torch.uint8, device=dev) if nb else None
        st, route = uor.gemm_coded(ga, (m, k), (k, 1), gcd, gcodes, rows, cols, transposed, gc,
                                   (m, n), (n, 1), alpha=-3, beta=beta, scratch=scratch,
                                   collapse=True)
        torch.cuda.synchronize()
        assert st == 0
        assert np.array_equal(gc.cpu().numpy(), want), (beta, offer, route)
        if want_kind:
            assert route["kind"] == want_kind and route["moduli"] == distinct, route
        else:
            assert route["kind"] != "collapsed", route


@pytest.mark.parametrize("transposed", [True, False])
def test_dense_route_strided_a(oracle, uor, dev, transposed):
    """The decode-into-scratch route hands the caller's A view to the dense
    int8 route as it is: column-major, padded and reversed rows."""
    spec = SPECS["ternary4_u8"]
    rng = np.random.default_rng(17)
    m, k, n = 20, 128, 64
    rows, cols = (n, k) if transposed else (k, n)
    codes = rng.integers(0, 256, rows * cols // 4).astype(np.uint8)
    ocd = oracle.codec("ternary", code_bits=8, block=4)
    gcd = uor.codec("ternary", code_bits=8, block=4)
    for a_str, alen in (((1, m), m * k), ((k + 8, 1), m * (k + 8)), ((-k, 1), m * k)):
        a = rng.integers(-128, 128, alen).astype(np.int8)
        c0 = rng.integers(-1000, 1000, m * n).astype(np.int32)
        want = c0.copy()
        assert oracle.gemm_coded(a, (m, k), a_str, ocd, codes, rows, cols, transposed, want,
                                 (m, n), (n, 1), alpha=5, beta=-1) == "ok"
        gc = torch.from_numpy(c0.copy()).to(dev)
        sc = torch.empty(uor.suggested_scratch_coded(m, k, n), dtype=torch.uint8, device=dev)
        st, route = uor.gemm_coded(torch.from_numpy(a).to(dev), (m, k), a_str, gcd,
                                   torch.from_numpy(codes).to(dev), rows, cols, transposed, gc,
                                   (m, n), (n, 1), alpha=5, beta=-1, scratch=sc)
        torch.cuda.synchronize()
        assert st == 0 and route["kind"] == "coded_dense", route
        assert np.array_equal(gc.cpu().numpy(), want), a_str
