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
