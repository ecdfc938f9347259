"""GPU parity of float products with an Arena-coded operand
(uor_gfx950_gemm_coded_float, through the C ABI): the CK-14 artifact's codes
and codebook against the exact float route on its committed dense spelling
(bit-exact) and against the CPU oracle (ora_gemm_float); both orientations,
u16 codes over a table that is not a power of two (code % N), f64, and the
refusal of an offer below the decoded operand."""
import json

import numpy as np
import pytest
import torch

from conftest import GOLDEN

pytestmark = pytest.mark.gpu

D = GOLDEN / "symbols_ck14"


def acts(rng, count, dtype):
    """Random signs and significands over a modest exponent range."""
    e = rng.integers(-20, 21, count)
    v = (rng.random(count) + 1.0) * np.exp2(e) * rng.choice([-1.0, 1.0], count)
    v[rng.random(count) < 0.05] = 0.0
    return v.astype(dtype)


def run(oracle, uor, dev, a, m, k, table, codes, w_rows, w_cols, transposed, alpha=1, beta=0,
        seed=0):
    rng = np.random.default_rng(seed)
    dt = table.dtype
    n = w_rows if transposed else w_cols
    c0 = acts(rng, m * n, dt)
    dense = table[codes.astype(np.int64) % len(table)].reshape(w_rows, w_cols)
    b = np.ascontiguousarray(dense.T if transposed else dense).reshape(-1)
    want = c0.copy()
    assert oracle.gemm_float(a, (m, k), (k, 1), b, (k, n), (n, 1), want, (m, n), (n, 1),
                             alpha=alpha, beta=beta) == "ok"
    ga = torch.from_numpy(a).to(dev)
    gc = torch.from_numpy(c0.copy()).to(dev)
    gd = torch.from_numpy(c0.copy()).to(dev)
    is64 = dt == np.float64
    sc = torch.empty(uor.suggested_scratch_coded_float(is64, m, k, n), dtype=torch.uint8,
                     device=dev)
    gcodes = torch.from_numpy(codes.view(np.int16) if codes.dtype == np.uint16 else codes).to(dev)
    st, route = uor.gemm_coded_float(ga, (m, k), (k, 1), torch.from_numpy(table).to(dev), gcodes,
                                     w_rows, w_cols, transposed, gc, (m, n), (n, 1), alpha=alpha,
                                     beta=beta, scratch=sc)
    sf = torch.empty(uor.suggested_scratch_float(is64, m, k, n), dtype=torch.uint8, device=dev)
    st2, _ = uor.gemm_float(ga, (m, k), (k, 1), torch.from_numpy(b).to(dev), (k, n), (n, 1), gd,
                            (m, n), (n, 1), alpha=alpha, beta=beta, scratch=sf)
    torch.cuda.synchronize()
    assert st == 0 and st2 == 0, (st, st2)
    got = gc.cpu().numpy()
    assert np.array_equal(got.view(np.uint64 if is64 else np.uint32),
                          gd.cpu().numpy().view(np.uint64 if is64 else np.uint32)), route
    assert np.array_equal(got.view(np.uint64 if is64 else np.uint32),
                          want.view(np.uint64 if is64 else np.uint32)), route
    return route


def fixture():
    book = np.frombuffer((D / "codebook.f32.bin").read_bytes(), "<f4").copy()
    codes = np.frombuffer((D / "13x257.codes.bin").read_bytes(), np.uint8).copy()
    return book, codes


@pytest.mark.parametrize("m", [1, 9, 40])
def test_ck14_artifact(oracle, uor, dev, m):
    """W is the 13 x 257 artifact (n = 13 output columns, k = 257)."""
    book, codes = fixture()
    rng = np.random.default_rng(m)
    a = acts(rng, m * 257, np.float32)
    run(oracle, uor, dev, a, m, 257, book, codes, 13, 257, True, alpha=3, beta=-1, seed=m)


def test_ck14_as_k_by_n(oracle, uor, dev):
    """The same codes read as a 257 x 13 operand (coded_gemm orientation)."""
    book, codes = fixture()
    rng = np.random.default_rng(5)
    a = acts(rng, 7 * 13, np.float32)
    run(oracle, uor, dev, a, 7, 13, book, codes, 13, 257, False, seed=5)


def test_large_artifact(oracle, uor, dev):
    """The 1024 x 1024 artifact at m = 4 (oracle on the dense spelling)."""
    book = np.frombuffer((D / "codebook.f32.bin").read_bytes(), "<f4").copy()
    codes = np.frombuffer((D / "1024x1024.codes.bin").read_bytes(), np.uint8).copy()
    rng = np.random.default_rng(6)
    a = acts(rng, 4 * 1024, np.float32)
    run(oracle, uor, dev, a, 4, 1024, book, codes, 1024, 1024, True, seed=6)


def test_u16_codes_table_mod_and_f64(oracle, uor, dev):
    rng = np.random.default_rng(7)
    for dt in (np.float32, np.float64):
        table = acts(rng, 300, dt)
        codes = rng.integers(0, 1 << 16, 24 * 50).astype(np.uint16)
        a = acts(rng, 6 * 50, dt)
        run(oracle, uor, dev, a, 6, 50, table, codes, 24, 50, True, alpha=-2, beta=1, seed=8)


def test_offer_below_the_decoded_operand(uor, dev):
    book, codes = fixture()
    a = torch.zeros(2 * 257, dtype=torch.float32, device=dev)
    c = torch.zeros(2 * 13, dtype=torch.float32, device=dev)
    for sc in (None, torch.empty(1024, dtype=torch.uint8, device=dev)):
        st, _ = uor.gemm_coded_float(a, (2, 257), (257, 1), torch.from_numpy(book).to(dev),
                                     torch.from_numpy(codes).to(dev), 13, 257, True, c, (2, 13),
                                     (13, 1), scratch=sc)
        assert uor.STATUS[st] == "invalid_argument"
