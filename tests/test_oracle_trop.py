"""Pins the tropical oracle (ora_gemm_trop) against the reference's committed
CX-11 fixtures (oracles/tropical: NumPy broadcast max-plus, -2^63 spelling
-inf, sha256-checked) and the reference's inline known answers."""
import hashlib
import json

import numpy as np
import pytest

from conftest import GOLDEN

NEG_INF = -(1 << 63)


def records(vals):
    """i64 artifact spelling -> Trop<i8> record bytes."""
    fin = vals != NEG_INF
    return __import__("oracle").oracle.trop_i8(np.where(fin, vals, 0).astype(np.int8), fin)


def test_cx11_fixtures(oracle):
    d = GOLDEN / "tropical_cx11"
    man = json.loads((d / "manifest.json").read_text())
    assert man["id"] == "CX-11" and man["neg_inf"] == NEG_INF
    for case in man["cases"]:
        m, k, n = (case["shape"][x] for x in "mkn")
        blobs = {}
        for name, key in (("a", "a_sha256"), ("b", "b_sha256"), ("expected", "expected_sha256")):
            raw = (d / f"{case['stem']}.{name}.bin").read_bytes()
            assert "sha256:" + hashlib.sha256(raw).hexdigest() == case[key]
            blobs[name] = np.frombuffer(raw, "<i8").copy()
        a = oracle.trop_bytes(records(blobs["a"]))
        b = oracle.trop_bytes(records(blobs["b"]))
        c = np.zeros(m * n, dtype=oracle.TROP_I32)
        cb = oracle.trop_bytes(c) if m * n else np.zeros(0, np.uint8)
        st = oracle.gemm_trop(a, (m, k), (k, 1), b, (k, n), (n, 1), cb, (m, n), (n, 1))
        assert st == "ok"
        got = cb.view(oracle.TROP_I32) if m * n else c
        want = blobs["expected"]
        fin = want != NEG_INF
        assert np.array_equal(got["finite"].astype(bool), fin), case["stem"]
        assert np.array_equal(got["value"][fin], want[fin]), case["stem"]
        assert not got["value"][~fin].any()  # NEG_INF writes value 0


def test_readme_known_answer(oracle):
    # driver.rs CD-29: A=[[1,2],[3,4]], B=[[5,6],[7,8]] -> [[9,10],[11,12]].
    a = oracle.trop_bytes(oracle.trop_i8(np.array([1, 2, 3, 4]), np.ones(4, bool)))
    b = oracle.trop_bytes(oracle.trop_i8(np.array([5, 6, 7, 8]), np.ones(4, bool)))
    c = oracle.trop_bytes(np.zeros(4, dtype=oracle.TROP_I32))
    assert oracle.gemm_trop(a, (2, 2), (2, 1), b, (2, 2), (2, 1), c, (2, 2), (2, 1)) == "ok"
    r = c.view(oracle.TROP_I32)
    assert r["value"].tolist() == [9, 10, 11, 12] and r["finite"].all()


def test_alpha_beta_and_absorption(oracle):
    # MaxPlus (epilogue.rs:137-192): (alpha (x) P) (+) (beta (x) C); -inf absorbs.
    a = oracle.trop_bytes(oracle.trop_i8(np.array([1, 2]), np.array([True, False])))
    b = oracle.trop_bytes(oracle.trop_i8(np.array([5, 7]), np.array([True, True])))
    c0 = np.zeros(1, dtype=oracle.TROP_I32)
    c0["value"] = 20
    c0["finite"] = 1
    c = oracle.trop_bytes(c0.copy())
    # P = max(1+5, -inf) = 6; alpha=3 -> 9; beta=-15 -> 20-15 = 5; max = 9
    oracle.gemm_trop(a, (1, 2), (2, 1), b, (2, 1), (1, 1), c, (1, 1), (1, 1),
                     alpha=(3, True), beta=(-15, True))
    assert c.view(oracle.TROP_I32)["value"][0] == 9
    c = oracle.trop_bytes(c0.copy())
    oracle.gemm_trop(a, (1, 2), (2, 1), b, (2, 1), (1, 1), c, (1, 1), (1, 1),
                     alpha=(0, False), beta=(-15, True))
    assert c.view(oracle.TROP_I32)["value"][0] == 5
    c = oracle.trop_bytes(c0.copy())
    oracle.gemm_trop(a, (1, 2), (2, 1), b, (2, 1), (1, 1), c, (1, 1), (1, 1),
                     alpha=(0, False), beta=(0, False))
    assert c.view(oracle.TROP_I32)["finite"][0] == 0


def test_encode_clamps_to_min_plus_one(oracle):
    # tropical.rs:336-350: finite values encode through [MIN+1, MAX-1].
    a = oracle.trop_bytes(oracle.trop_i8(np.array([100]), np.array([True])))
    b = oracle.trop_bytes(oracle.trop_i8(np.array([100]), np.array([True])))
    c = np.zeros(2, np.uint8)  # one Trop<i8> output record
    oracle.gemm_trop(a, (1, 1), (1, 1), b, (1, 1), (1, 1), c, (1, 1), (1, 1), out_bytes=1)
    assert c.view(np.int8)[0] == 126 and c[1] == 1  # 200 -> i8::MAX - 1
    oracle.gemm_trop(a, (1, 1), (1, 1), b, (1, 1), (1, 1), c, (1, 1), (1, 1), out_bytes=1,
                     encode="wrapping")
    # 200 wraps over span 254 starting at -127: (200 + 127) % 254 - 127 = -54
    assert c.view(np.int8)[0] == -54


# ------------------------------------------------------ gemm_selected witness

def sel(oracle, av, af, bv, bf, m, k, n, alpha=(0, True), beta=(0, False), c0=None):
    a = oracle.trop_bytes(oracle.trop_i8(np.asarray(av), np.asarray(af, bool)))
    b = oracle.trop_bytes(oracle.trop_i8(np.asarray(bv), np.asarray(bf, bool)))
    c = np.zeros(m * n, dtype=oracle.TROP_I32) if c0 is None else c0.copy()
    cb = oracle.trop_bytes(c) if m * n else np.zeros(0, np.uint8)
    w = np.full(m * n, 7777, np.uint64)
    st = oracle.gemm_trop_selected(a if a.size else np.zeros(0, np.uint8), (m, k), (k, 1),
                                   b if b.size else np.zeros(0, np.uint8), (k, n), (n, 1),
                                   cb, (m, n), (n, 1), w, (n, 1), alpha=alpha, beta=beta)
    return st, (cb.view(oracle.TROP_I32) if m * n else c), w


def test_selected_doc_example(oracle):
    # selection.rs:186-211 and its tie test: 1+9 and 9+1 both give 10; D-6
    # takes the smaller index.
    st, c, w = sel(oracle, [1, 9], [1, 1], [9, 1], [1, 1], 1, 2, 1)
    assert st == "ok" and c["finite"][0] and c["value"][0] == 10 and w[0] == 0


def test_selected_degenerate_ct04(oracle):
    # selection.rs the_degenerate_selections_are_answers_ct_04: every term
    # masked -> NEG_INF with witness 0; depth zero -> NEG_INF with witness 0.
    st, c, w = sel(oracle, [0] * 4, [0] * 4, [0] * 4, [0] * 4, 1, 4, 1)
    assert st == "ok" and not c["finite"][0] and w[0] == 0
    st, c, w = sel(oracle, [], [], [], [], 1, 0, 1)
    assert st == "ok" and not c["finite"][0] and w[0] == 0


def test_selected_nonconformant_and_aliasing_ct05(oracle):
    a = oracle.trop_bytes(oracle.trop_i8(np.array([1, 2]), np.ones(2, bool)))
    b = oracle.trop_bytes(oracle.trop_i8(np.array([3, 4]), np.ones(2, bool)))
    cb = oracle.trop_bytes(np.zeros(1, dtype=oracle.TROP_I32))
    w = np.zeros(4, np.uint64)
    # A 2x2 witness for a 1x1 product (selection.rs:236-250).
    st = oracle.lib().ora_gemm_trop_selected(
        1, *oracle._view(a, 1, 2, 2, 1, rec=2), *oracle._view(b, 2, 1, 1, 1, rec=2),
        *oracle._view(cb, 1, 1, 1, 1, rec=8), *oracle._view(w, 2, 2, 2, 1), 4, 0, 1, 0, 0, 0)
    assert oracle.STATUS[st] == "nonconformant"
    c4 = oracle.trop_bytes(np.zeros(4, dtype=oracle.TROP_I32))
    st = oracle.lib().ora_gemm_trop_selected(
        1, *oracle._view(a, 2, 1, 1, 1, rec=2), *oracle._view(b, 1, 2, 2, 1, rec=2),
        *oracle._view(c4, 2, 2, 2, 1, rec=8), *oracle._view(w, 2, 2, 0, 1), 4, 0, 1, 0, 0, 0)
    assert oracle.STATUS[st] == "output_aliases_itself"


@pytest.mark.parametrize("seed", range(4))
def test_selected_brute_force_with_ties(oracle, seed):
    """Values from a small range force ties; the witness is the least p whose
    term attains the maximum (every term masked: 0), and C is gemm_trop's."""
    rng = np.random.default_rng(seed)
    m, k, n = 5, 23, 6
    av, bv = rng.integers(-3, 4, m * k), rng.integers(-3, 4, k * n)
    af, bf = rng.random(m * k) > 0.25, rng.random(k * n) > 0.25
    af[:k] = False  # row 0 fully masked
    st, c, w = sel(oracle, av, af, bv, bf, m, k, n)
    assert st == "ok"
    A, B = av.reshape(m, k), bv.reshape(k, n)
    AF, BF = af.reshape(m, k), bf.reshape(k, n)
    for i in range(m):
        for j in range(n):
            terms = [A[i, p] + B[p, j] if AF[i, p] and BF[p, j] else None for p in range(k)]
            fin = [t for t in terms if t is not None]
            if fin:
                best = max(fin)
                assert c["finite"][i * n + j] and c["value"][i * n + j] == best
                assert w[i * n + j] == terms.index(best)
            else:
                assert not c["finite"][i * n + j] and w[i * n + j] == 0
    plain = oracle.trop_bytes(np.zeros(m * n, dtype=oracle.TROP_I32))
    a = oracle.trop_bytes(oracle.trop_i8(av, af))
    b = oracle.trop_bytes(oracle.trop_i8(bv, bf))
    oracle.gemm_trop(a, (m, k), (k, 1), b, (k, n), (n, 1), plain, (m, n), (n, 1))
    assert np.array_equal(plain.view(oracle.TROP_I32), c)
