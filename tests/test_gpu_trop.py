"""GPU parity of the (max, +) GEMM over Trop<i8> (uor_gfx950_gemm_trop_i8)
against the oracle: random shapes with masked entries, every output width,
alpha/beta at finite and -inf values, both encode families, and the full
configs[4] shape (4096^3, 5% -inf) against a chunked torch max-plus plus
oracle rows."""
import numpy as np
import pytest
import torch

import gen

pytestmark = pytest.mark.gpu

REC = {1: np.dtype([("value", "i1"), ("finite", "u1")]),
       2: np.dtype([("value", "<i2"), ("finite", "u1"), ("_p", "V1")]),
       4: np.dtype([("value", "<i4"), ("finite", "u1"), ("_p", "V3")]),
       8: np.dtype([("value", "<i8"), ("finite", "u1"), ("_p", "V7")])}


def rand_trop(rng, count, p_inf=0.05, lo=-128, hi=128):
    vals = rng.integers(lo, hi, count)
    fin = rng.random(count) >= p_inf
    rec = np.zeros(count, REC[1])
    rec["value"] = np.where(fin, vals, 0)
    rec["finite"] = fin
    return rec.view(np.uint8).copy()


def check(oracle, uor, dev, a, ash, ast, b, bsh, bst, c0, csh, cst, ob=4, alpha=(0, True),
          beta=(0, False), encode="nearest"):
    want = c0.copy()
    st = oracle.gemm_trop(a, ash, ast, b, bsh, bst, want, csh, cst, alpha=alpha, beta=beta,
                          encode=encode, out_bytes=ob)
    gc = torch.from_numpy(c0.copy()).to(dev)
    gst, route = uor.gemm_trop_i8(torch.from_numpy(a).to(dev), ash, ast,
                                  torch.from_numpy(b).to(dev), bsh, bst, gc, csh, cst, out=ob,
                                  alpha=alpha, beta=beta, encode=encode)
    torch.cuda.synchronize()
    assert uor.STATUS.get(gst, gst) == st
    got = gc.cpu().numpy().view(REC[ob])
    w = want.view(REC[ob])
    assert np.array_equal(got["finite"], w["finite"]), (ash, bsh, route)
    assert np.array_equal(got["value"], w["value"]), (ash, bsh, route)


@pytest.mark.parametrize("shape", [(1, 1, 1), (3, 7, 11), (13, 17, 19), (128, 3, 128),
                                   (129, 200, 130), (64, 1000, 33), (300, 64, 257)])
def test_shapes(oracle, uor, dev, shape):
    m, k, n = shape
    rng = np.random.default_rng(m + 3 * k + 7 * n)
    a = rand_trop(rng, m * k)
    b = rand_trop(rng, k * n)
    c0 = np.zeros(m * n, REC[4]).view(np.uint8).copy()
    check(oracle, uor, dev, a, (m, k), (k, 1), b, (k, n), (n, 1), c0, (m, n), (n, 1))


@pytest.mark.parametrize("ob", [1, 2, 4, 8])
@pytest.mark.parametrize("encode", ["nearest", "wrapping"])
def test_outputs_and_epilogue(oracle, uor, dev, ob, encode):
    rng = np.random.default_rng(ob * 10 + len(encode))
    m, k, n = 40, 50, 37
    a = rand_trop(rng, m * k, p_inf=0.3)
    b = rand_trop(rng, k * n, p_inf=0.3)
    prior = np.zeros(m * n, REC[ob])
    prior["value"] = rng.integers(-100, 100, m * n)
    prior["finite"] = rng.random(m * n) < 0.7
    prior["value"] = np.where(prior["finite"], prior["value"], 0)
    c0 = prior.view(np.uint8).copy()
    for alpha, beta in [((0, True), (0, False)), ((5, True), (-3, True)), ((0, False), (7, True)),
                        ((120, True), (0, False)), ((1 << 40, True), (-(1 << 41), True))]:
        check(oracle, uor, dev, a, (m, k), (k, 1), b, (k, n), (n, 1), c0, (m, n), (n, 1), ob=ob,
              alpha=alpha, beta=beta, encode=encode)


def test_strides_masks_and_empty(oracle, uor, dev):
    rng = np.random.default_rng(3)
    m, k, n = 21, 30, 19
    a = rand_trop(rng, m * k)
    b = rand_trop(rng, k * n)
    c0 = np.zeros(m * n, REC[4]).view(np.uint8).copy()
    # transposed A, column-major C
    check(oracle, uor, dev, a, (m, k), (1, m), b, (k, n), (n, 1), c0, (m, n), (1, m))
    # reversed B rows
    check(oracle, uor, dev, a, (m, k), (k, 1), b, (k, n), (-n, 1), c0, (m, n), (n, 1))
    # a fully masked row of A gives -inf across its row
    a2 = a.view(REC[1]).copy()
    a2["finite"][:k] = 0
    a2["value"][:k] = 0
    check(oracle, uor, dev, a2.view(np.uint8).copy(), (m, k), (k, 1), b, (k, n), (n, 1), c0,
          (m, n), (n, 1))
    # k = 0: every cell is the semiring zero (or beta (x) C)
    check(oracle, uor, dev, np.zeros(0, np.uint8), (m, 0), (0, 1), np.zeros(0, np.uint8),
          (0, n), (n, 1), c0, (m, n), (n, 1), beta=(2, True))


def test_config5_4096(oracle, uor, dev):
    """m = n = k = 4096, uniform i8, 5% -inf (salts 11, 12)."""
    N = 4096
    va = gen.i8_full(N * N, 11).astype(np.int64)
    vb = gen.i8_full(N * N, 12).astype(np.int64)
    fa = (gen.draws(N * N, 111) % np.uint64(20)) != 0
    fb = (gen.draws(N * N, 112) % np.uint64(20)) != 0
    def recs(v, f):
        r = np.zeros(v.size, REC[1])
        r["value"] = np.where(f, v, 0)
        r["finite"] = f
        return r.view(np.uint8)
    a, b = recs(va, fa), recs(vb, fb)
    c = torch.zeros(N * N * 8, dtype=torch.uint8, device=dev)
    st, route = uor.gemm_trop_i8(torch.from_numpy(a).to(dev), (N, N), (N, 1),
                                 torch.from_numpy(b).to(dev), (N, N), (N, 1), c, (N, N), (N, 1))
    torch.cuda.synchronize()
    assert st == 0
    got = c.cpu().numpy().view(REC[4])
    # Independent check in torch: chunked broadcast max with a -2^20 sentinel.
    A = torch.from_numpy(np.where(fa, va, -(1 << 20)).reshape(N, N)).to(dev, torch.int32)
    B = torch.from_numpy(np.where(fb, vb, -(1 << 20)).reshape(N, N)).to(dev, torch.int32)
    acc = torch.full((N, N), -(1 << 30), dtype=torch.int32, device=dev)
    for p in range(0, N, 8):
        acc = torch.maximum(acc, (A[:, p:p + 8, None] + B[None, p:p + 8, :]).amax(1))
    want = acc.cpu().numpy().reshape(-1)
    fin = want > -(1 << 19)
    assert np.array_equal(got["finite"].astype(bool), fin)
    assert np.array_equal(got["value"][fin], want[fin])
    # and four rows against the oracle
    for r in (0, 1, 2047, 4095):
        cr = np.zeros(N, REC[4]).view(np.uint8)
        oracle.gemm_trop(a[2 * r * N:2 * (r + 1) * N].copy(), (1, N), (N, 1), b, (N, N), (N, 1),
                         cr, (1, N), (N, 1))
        assert np.array_equal(cr.view(REC[4])["value"], got["value"][r * N:(r + 1) * N])


@pytest.mark.parametrize("shape", [(8, 8, 8), (136, 200, 264), (1000, 96, 136), (129, 1000, 520),
                                   (5, 4104, 16)])
@pytest.mark.parametrize("ob", [1, 4])
def test_record_vector_loads(oracle, uor, dev, shape, ob):
    """Unit record strides, k and n multiples of 8: the 16-byte record loads
    (ragged m and n tiles, k tails shorter than a 32-deep step), against the
    oracle, with alpha/beta finite and a prior C."""
    m, k, n = shape
    rng = np.random.default_rng(m * 5 + k * 3 + n + ob)
    a = rand_trop(rng, m * k, p_inf=0.1)
    b = rand_trop(rng, k * n, p_inf=0.1)
    c0 = np.zeros(m * n, REC[ob])
    c0["value"] = rng.integers(-100, 100, m * n)
    c0["finite"] = rng.random(m * n) < 0.5
    check(oracle, uor, dev, a, (m, k), (k, 1), b, (k, n), (n, 1), c0.view(np.uint8).copy(), (m, n), (n, 1),
          ob=ob, alpha=(3, True), beta=(-2, True), encode="nearest" if ob == 4 else "wrapping")
