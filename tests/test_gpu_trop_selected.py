"""GPU parity of the witness GEMM over Trop<i8> (uor_gfx950_gemm_trop_i8_selected,
through the C ABI) against the oracle's restatement of gemm_selected
(oracle/uor_oracle.c ora_gemm_trop_selected): ties planted by a narrow value
range, masked entries, all-masked rows, k = 0, alpha/beta, every output width,
strided and transposed witnesses, both mechanisms, the status order of
SelectedTriple::new, the per-cell route past 2^21 terms, and the full
configs[4] shape against the unselected product plus oracle rows.

Bar: bit-exact, values and witnesses."""
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


def check(oracle, uor, dev, a, ash, ast, b, bsh, bst, c0, csh, cst, wst=None, wlen=None, ob=4,
          alpha=(0, True), beta=(0, False), encode="nearest", mechanism="lexicographic",
          route_kind=None):
    m, n = csh
    wst = wst or (n, 1)
    wlen = wlen or max(m * n, 1)
    want = c0.copy()
    w_want = np.full(wlen, 0xDEAD, np.uint64)
    st = oracle.gemm_trop_selected(a, ash, ast, b, bsh, bst, want, csh, cst, w_want, wst,
                                   alpha=alpha, beta=beta, encode=encode, out_bytes=ob)
    gc = torch.from_numpy(c0.copy()).to(dev)
    gw = torch.full((wlen,), 0xDEAD, dtype=torch.int64, device=dev)
    gst, route = uor.gemm_trop_i8_selected(torch.from_numpy(a).to(dev), ash, ast,
                                           torch.from_numpy(b).to(dev), bsh, bst, gc, csh, cst,
                                           gw, wst, out=ob, alpha=alpha, beta=beta, encode=encode,
                                           mechanism=mechanism)
    torch.cuda.synchronize()
    assert uor.STATUS.get(gst, gst) == st, (gst, st)
    got = gc.cpu().numpy().view(REC[ob])
    w = want.view(REC[ob])
    assert np.array_equal(got["finite"], w["finite"]), (ash, bsh, route)
    assert np.array_equal(got["value"], w["value"]), (ash, bsh, route)
    assert np.array_equal(gw.cpu().numpy().view(np.uint64), w_want), (ash, bsh, route)
    if route_kind is not None:
        assert route["kind"] == route_kind, route
    return route


@pytest.mark.parametrize("shape", [(1, 1, 1), (3, 7, 11), (13, 17, 19), (128, 3, 128),
                                   (129, 200, 130), (64, 1000, 33), (300, 64, 257)])
@pytest.mark.parametrize("mechanism", ["lexicographic", "compare_pass"])
def test_shapes_with_ties(oracle, uor, dev, shape, mechanism):
    """Values in [-3, 3] make most cells' maxima tie across many p: the
    witness must be the least of them (D-6)."""
    m, k, n = shape
    rng = np.random.default_rng(m + 3 * k + 7 * n)
    a = rand_trop(rng, m * k, p_inf=0.2, lo=-3, hi=4)
    b = rand_trop(rng, k * n, p_inf=0.2, lo=-3, hi=4)
    c0 = np.zeros(m * n, REC[4]).view(np.uint8).copy()
    check(oracle, uor, dev, a, (m, k), (k, 1), b, (k, n), (n, 1), c0, (m, n), (n, 1),
          mechanism=mechanism, route_kind="trop_selected")


@pytest.mark.parametrize("shape", [(40, 300, 37), (256, 128, 256)])
def test_full_range_values(oracle, uor, dev, shape):
    """Full i8 range, extremes included (sums from -256 to 254)."""
    m, k, n = shape
    rng = np.random.default_rng(k)
    a = rand_trop(rng, m * k, p_inf=0.1)
    b = rand_trop(rng, k * n, p_inf=0.1)
    av, bv = a.view(REC[1]), b.view(REC[1])
    av["value"][::7] = np.where(av["finite"][::7], -128, 0)
    bv["value"][::5] = np.where(bv["finite"][::5], 127, 0)
    c0 = np.zeros(m * n, REC[4]).view(np.uint8).copy()
    check(oracle, uor, dev, a, (m, k), (k, 1), b, (k, n), (n, 1), c0, (m, n), (n, 1))


@pytest.mark.parametrize("ob", [1, 2, 4, 8])
@pytest.mark.parametrize("encode", ["nearest", "wrapping"])
def test_outputs_and_epilogue(oracle, uor, dev, ob, encode):
    """alpha/beta at finite and -inf values: the witness is the product's,
    whatever the epilogue does to C."""
    rng = np.random.default_rng(ob * 10 + len(encode))
    m, k, n = 40, 50, 37
    a = rand_trop(rng, m * k, p_inf=0.3, lo=-8, hi=8)
    b = rand_trop(rng, k * n, p_inf=0.3, lo=-8, hi=8)
    prior = np.zeros(m * n, REC[ob])
    prior["value"] = rng.integers(-100, 100, m * n)
    prior["finite"] = rng.random(m * n) < 0.7
    prior["value"] = np.where(prior["finite"], prior["value"], 0)
    c0 = prior.view(np.uint8).copy()
    for alpha, beta in [((0, True), (0, False)), ((5, True), (-3, True)), ((0, False), (7, True)),
                        ((120, True), (0, False)), ((1 << 40, True), (-(1 << 41), True))]:
        check(oracle, uor, dev, a, (m, k), (k, 1), b, (k, n), (n, 1), c0, (m, n), (n, 1), ob=ob,
              alpha=alpha, beta=beta, encode=encode)


def test_strided_witness_masks_and_empty(oracle, uor, dev):
    rng = np.random.default_rng(3)
    m, k, n = 21, 30, 19
    a = rand_trop(rng, m * k, lo=-4, hi=4)
    b = rand_trop(rng, k * n, lo=-4, hi=4)
    c0 = np.zeros(m * n, REC[4]).view(np.uint8).copy()
    # transposed A, column-major C and witness
    check(oracle, uor, dev, a, (m, k), (1, m), b, (k, n), (n, 1), c0, (m, n), (1, m), wst=(1, m))
    # reversed B rows, reversed witness rows in a padded buffer
    check(oracle, uor, dev, a, (m, k), (k, 1), b, (k, n), (-n, 1), c0, (m, n), (n, 1),
          wst=(-(n + 3), 1), wlen=m * (n + 3))
    # a fully masked row of A: -inf across its row, witness 0 (the least p
    # whose term is the semiring zero)
    a2 = a.view(REC[1]).copy()
    a2["finite"][:k] = 0
    a2["value"][:k] = 0
    check(oracle, uor, dev, a2.view(np.uint8).copy(), (m, k), (k, 1), b, (k, n), (n, 1), c0,
          (m, n), (n, 1))
    # k = 0: witness 0, C is beta (x) C
    check(oracle, uor, dev, np.zeros(0, np.uint8), (m, 0), (0, 1), np.zeros(0, np.uint8),
          (0, n), (n, 1), c0, (m, n), (n, 1), beta=(2, True))
    # m = 0: nothing written
    check(oracle, uor, dev, np.zeros(0, np.uint8), (0, k), (k, 1), b, (k, n), (n, 1),
          np.zeros(0, np.uint8), (0, n), (n, 1))


def test_witness_status_order(oracle, uor, dev):
    """SelectedTriple::new: the product's own checks first, then the witness's
    shape, then its aliasing; the oracle agrees on every case."""
    m, k, n = 4, 5, 6
    a = torch.zeros(2 * m * k, dtype=torch.uint8, device=dev)
    b = torch.zeros(2 * k * n, dtype=torch.uint8, device=dev)
    c = torch.zeros(8 * m * n, dtype=torch.uint8, device=dev)
    w = torch.zeros(m * n, dtype=torch.int64, device=dev)
    call = lambda **kw: uor.STATUS[uor.gemm_trop_i8_selected(
        a, (m, k), (k, 1), b, (k, n), (n, 1), c, (m, n), kw.get("cst", (n, 1)), w,
        kw.get("wst", (n, 1)), w_shape=kw.get("wsh"), mechanism=kw.get("mech", 0))[0]]
    assert call() == "ok"
    assert call(mech="compare_pass") == "ok"
    assert call(wsh=(m, n - 1)) == "nonconformant"
    assert call(wsh=(m + 1, n), wst=(n, 1)) == "short_buffer"
    assert call(wst=(0, 1)) == "output_aliases_itself"
    assert call(wst=(1, 1)) == "output_aliases_itself"
    # the product's own failure is named before the witness's
    assert call(cst=(0, 1), wsh=(m, n - 1)) == "output_aliases_itself"
    assert call(mech=2) == "invalid_argument"
    # the oracle names the same statuses
    an, bn = np.zeros(2 * m * k, np.uint8), np.zeros(2 * k * n, np.uint8)
    cn = np.zeros(8 * m * n, np.uint8)
    wn = np.zeros(m * n, np.uint64)
    assert oracle.gemm_trop_selected(an, (m, k), (k, 1), bn, (k, n), (n, 1), cn, (m, n), (n, 1),
                                     wn, (0, 1)) == "output_aliases_itself"


def test_depth_at_key_limit(oracle, uor, dev):
    """k = 2^21, the deepest product the (value, index) keys hold: the
    maximum planted at the last p and tied at an earlier one."""
    m, n, k = 2, 3, 1 << 21
    rng = np.random.default_rng(21)
    a = rand_trop(rng, m * k, lo=-100, hi=0)
    b = rand_trop(rng, k * n, lo=-100, hi=0)
    av, bv = a.view(REC[1]), b.view(REC[1])
    av["value"][k - 1], av["finite"][k - 1] = 100, 1        # row 0, p = k - 1
    bv["value"][(k - 1) * n:k * n], bv["finite"][(k - 1) * n:k * n] = 27, 1
    av["value"][k + 5], av["finite"][k + 5] = 90, 1         # row 1, p = 5 ties p = k - 1
    av["value"][2 * k - 1], av["finite"][2 * k - 1] = 90, 1
    bv["value"][5 * n:6 * n], bv["finite"][5 * n:6 * n] = 27, 1
    c0 = np.zeros(m * n, REC[4]).view(np.uint8).copy()
    check(oracle, uor, dev, a, (m, k), (k, 1), b, (k, n), (n, 1), c0, (m, n), (n, 1),
          route_kind="trop_selected")


def test_depth_past_key_limit(oracle, uor, dev):
    """k = 2^21 + 9 takes the per-cell route; the maximum sits past 2^21."""
    m, n, k = 2, 3, (1 << 21) + 9
    rng = np.random.default_rng(22)
    a = rand_trop(rng, m * k, lo=-100, hi=0)
    b = rand_trop(rng, k * n, lo=-100, hi=0)
    av, bv = a.view(REC[1]), b.view(REC[1])
    p = (1 << 21) + 4
    av["value"][p], av["finite"][p] = 100, 1
    bv["value"][p * n:(p + 1) * n], bv["finite"][p * n:(p + 1) * n] = 27, 1
    c0 = np.zeros(m * n, REC[4]).view(np.uint8).copy()
    check(oracle, uor, dev, a, (m, k), (k, 1), b, (k, n), (n, 1), c0, (m, n), (n, 1),
          route_kind="trop_selected_direct")


def test_config5_4096(oracle, uor, dev):
    """configs[4] shape (4096^3, 5% -inf, salts 11, 12): C equals the
    unselected product's bytes, every witness attains its cell's maximum
    (checked by gather over all 16.7M cells), and eight rows match the
    oracle, least index included."""
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
    ga, gb = torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev)
    c = torch.zeros(N * N * 8, dtype=torch.uint8, device=dev)
    c_plain = torch.zeros(N * N * 8, dtype=torch.uint8, device=dev)
    w = torch.full((N * N,), -1, dtype=torch.int64, device=dev)
    st, route = uor.gemm_trop_i8_selected(ga, (N, N), (N, 1), gb, (N, N), (N, 1), c, (N, N),
                                          (N, 1), w, (N, 1))
    assert st == 0 and route["kind"] == "trop_selected", route
    st2, _ = uor.gemm_trop_i8(ga, (N, N), (N, 1), gb, (N, N), (N, 1), c_plain, (N, N), (N, 1))
    torch.cuda.synchronize()
    assert st2 == 0
    assert torch.equal(c, c_plain)
    # Every witness attains the value: A[i, w] + B[w, j] == C[i, j].
    A = torch.from_numpy(np.where(fa, va, -(1 << 20)).reshape(N, N)).to(dev, torch.int32)
    B = torch.from_numpy(np.where(fb, vb, -(1 << 20)).reshape(N, N)).to(dev, torch.int32)
    W = w.view(N, N)
    assert int(W.min()) >= 0 and int(W.max()) < N
    rows = torch.arange(N, device=dev)[:, None].expand(N, N)
    cols = torch.arange(N, device=dev)[None, :].expand(N, N)
    term = A[rows, W] + B[W, cols]
    got = c.cpu().numpy().view(REC[4])
    assert got["finite"].all()
    assert torch.equal(term.cpu(), torch.from_numpy(got["value"].reshape(N, N).astype(np.int32)))
    # Least index: eight rows against the oracle.
    pick = [0, 1, 777, 2048, 3000, 4000, 4094, 4095]
    wn = W.cpu().numpy()
    for i in pick:
        ar = a.reshape(N, 2 * N)[i].copy()
        cw = np.zeros(N * 8, np.uint8)
        ww = np.zeros(N, np.uint64)
        assert oracle.gemm_trop_selected(ar, (1, N), (N, 1), b, (N, N), (N, 1), cw, (1, N),
                                         (N, 1), ww, (N, 1)) == "ok"
        assert np.array_equal(wn[i].astype(np.uint64), ww), i
