"""GPU parity of the i16/i32/i64 element GEMMs (uor_gfx950_gemm_int, through
the C ABI) against the CPU oracle (oracle/uor_oracle.c ora_gemm_int, the
restatement of driver::gemm at E = i16/i32/i64) and the reference's CX-10
int64 fixtures.

Bar: bit-exact.  Both routes are checked: the int8 residue route (an offer of
uor_gfx950_suggested_scratch_int bytes) and the per-cell loop (no offer).
"""
import hashlib
import json

import numpy as np
import pytest
import torch

from conftest import GOLDEN

pytestmark = pytest.mark.gpu

DT = {2: np.int16, 4: np.int32, 8: np.int64}
OUTDT = {"i8": np.int8, "i16": np.int16, "i32": np.int32, "i64": np.int64, "i128": np.int64}


def full_range(rng, n, eb):
    info = np.iinfo(DT[eb])
    x = rng.integers(info.min, info.max, n, dtype=DT[eb], endpoint=True)
    # Every tenth element at an extreme or zero.
    pick = rng.integers(0, 10, n)
    x[pick == 0] = info.min
    x[pick == 1] = info.max
    x[pick == 2] = 0
    return x


def run(oracle, uor, dev, eb, m, k, n, a_str=None, b_str=None, out="i64", alpha=1, beta=0,
        encode="nearest", offer=True, seed=0, a=None, b=None):
    rng = np.random.default_rng(seed)
    ars, acs = a_str or (k, 1)
    brs, bcs = b_str or (n, 1)
    alen = 1 + max(0, (m - 1) * abs(ars) + (k - 1) * abs(acs)) if m and k else 1
    blen = 1 + max(0, (k - 1) * abs(brs) + (n - 1) * abs(bcs)) if k and n else 1
    a = full_range(rng, alen, eb) if a is None else a
    b = full_range(rng, blen, eb) if b is None else b
    ob = 16 if out == "i128" else np.dtype(OUTDT[out]).itemsize
    rec = 2 if out == "i128" else 1
    c0 = rng.integers(-(1 << 40), 1 << 40, m * n * rec).astype(OUTDT[out])
    want = c0.copy()
    w = want.reshape(-1, 2) if rec == 2 else want
    st = oracle.gemm_int(a, (m, k), (ars, acs), b, (k, n), (brs, bcs), w, (m, n), (n, 1),
                         alpha=alpha, beta=beta, encode=encode, out_bytes=ob)
    gc = torch.from_numpy(c0.copy()).to(dev)
    scratch = None
    if offer:
        nbytes = uor.suggested_scratch_int(eb, m, k, n)
        scratch = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev) if nbytes else None
    gst, route = uor.gemm_int(torch.from_numpy(a).to(dev), (m, k), (ars, acs),
                              torch.from_numpy(b).to(dev), (k, n), (brs, bcs), gc, (m, n), (n, 1),
                              out=out, alpha=alpha, beta=beta, encode=encode, scratch=scratch)
    torch.cuda.synchronize()
    assert uor.STATUS.get(gst, gst) == st, (gst, st)
    assert np.array_equal(gc.cpu().numpy(), want), (eb, m, k, n, out, alpha, beta, encode, route)
    return route


@pytest.mark.parametrize("eb", [2, 4, 8])
@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (3, 7, 11), (13, 17, 19), (64, 300, 70),
                                   (129, 257, 130), (5, 1000, 7), (260, 64, 300)])
@pytest.mark.parametrize("offer", [True, False])
def test_shapes_against_oracle(oracle, uor, dev, eb, m, k, n, offer):
    """Full-range operands (extremes and zeros included); i64 output, with
    alpha = 3, beta = -1."""
    alpha, beta = 3, -1
    route = run(oracle, uor, dev, eb, m, k, n, alpha=alpha, beta=beta, offer=offer,
                seed=eb * 1000 + m + k + n)
    want = ("int_limb" if eb < 8 else "int_crt") if offer else "int_direct"
    assert route["kind"] == want, route


@pytest.mark.parametrize("out", ["i8", "i16", "i32", "i64", "i128"])
@pytest.mark.parametrize("encode", ["nearest", "wrapping"])
@pytest.mark.parametrize("eb", [2, 4, 8])
def test_output_types_and_encodes(oracle, uor, dev, out, encode, eb):
    """Every output width under both integer encodes: sums far outside the
    narrow outputs saturate or wrap exactly as encode_i128_into /
    impl_encode_from_limbs do."""
    scalars = [(1, 0), (3, -1), (1 << 40, -(1 << 35)), (-(1 << 63), (1 << 63) - 1)]
    for alpha, beta in scalars:
        run(oracle, uor, dev, eb, 9, 33, 21, out=out, alpha=alpha, beta=beta, encode=encode,
            seed=eb + 7)


@pytest.mark.parametrize("eb", [2, 4, 8])
def test_strided_and_transposed_views(oracle, uor, dev, eb):
    """Column-major A, row-strided B, negative strides: the same bytes."""
    m, k, n = 37, 45, 29
    run(oracle, uor, dev, eb, m, k, n, a_str=(1, m), b_str=(1, k), seed=3)
    run(oracle, uor, dev, eb, m, k, n, a_str=(k + 3, 1), b_str=(n + 5, 1), seed=4)
    run(oracle, uor, dev, eb, m, k, n, a_str=(-k, -1), b_str=(n, -1), seed=5)


def test_i64_limbs_past_i128(oracle, uor, dev):
    """i64::MIN squared four times is 2^128, past i128: Limbs<3> saturates
    every output width under Nearest and wraps to 0 under Wrapping."""
    m, k, n = 3, 4, 5
    a = np.full(m * k, np.iinfo(np.int64).min, np.int64)
    b = np.full(k * n, np.iinfo(np.int64).min, np.int64)
    for out in ["i32", "i64", "i128"]:
        for encode in ["nearest", "wrapping"]:
            for offer in [True, False]:
                run(oracle, uor, dev, 8, m, k, n, out=out, encode=encode, offer=offer, a=a, b=b)


@pytest.mark.parametrize("eb", [2, 4])
def test_depth_chunks(oracle, uor, dev, eb):
    """Past 2^17 terms the residue GEMMs run in chunks whose residues add
    mod p: k = 2^17 + 192 is two chunks (the second short)."""
    route = run(oracle, uor, dev, eb, 16, (1 << 17) + 192, 24, alpha=3, beta=-1, seed=11)
    assert route["kind"] == "int_crt" and route["split_k"] == 2, route


def test_residue_route_past_the_limb_depth(oracle, uor, dev):
    """i32 elements at L k >= 2^17 (k = 2^15 + 40) under Nearest: the limb
    planes would not be exact in i32, so the residue route runs."""
    route = run(oracle, uor, dev, 4, 9, (1 << 15) + 40, 11, alpha=3, beta=-1, seed=12)
    assert route["kind"] == "int_crt" and route["split_k"] == 1, route


@pytest.mark.parametrize("out", ["i8", "i16", "i32"])
def test_limb_route_modular_depth(oracle, uor, dev, out):
    """Wrapping into at most 32 bits: the limb planes are only needed mod
    2^32, so the limb route takes any depth and drops the shifts past 32 bits
    (i32 elements: 4 of 7 plane GEMMs)."""
    route = run(oracle, uor, dev, 4, 9, (1 << 15) + 40, 11, out=out, alpha=(1 << 63) - 1,
                beta=-(1 << 62), encode="wrapping", seed=13)
    assert route["kind"] == "int_limb" and route["split_k"] == 4, route
    route = run(oracle, uor, dev, 2, 9, (1 << 16) + 40, 11, out=out, alpha=5, beta=3,
                encode="wrapping", seed=14)
    assert route["kind"] == "int_limb" and route["split_k"] == 3, route


@pytest.mark.parametrize("eb", [2, 4])
def test_limb_route_extremes(oracle, uor, dev, eb):
    """Every element at MIN (or MAX) at the deepest exact limb depth (L k just
    below 2^17): each plane GEMM sums L k products of magnitude 2^14."""
    info = np.iinfo(DT[eb])
    k = (1 << 17) // eb - 1
    for v in (info.min, info.max):
        a = np.full(3 * k, v, DT[eb])
        b = np.full(k * 2, info.min, DT[eb])
        route = run(oracle, uor, dev, eb, 3, k, 2, out="i128", a=a, b=b, seed=15)
        assert route["kind"] == "int_limb" and route["split_k"] == 2 * eb - 1, route


def test_k_zero_and_empty(oracle, uor, dev):
    """k = 0: C := enc(beta * C); m = 0 or n = 0: nothing written."""
    route = run(oracle, uor, dev, 4, 6, 0, 5, alpha=3, beta=-1)
    assert route["kind"] == "epilogue_only", route
    run(oracle, uor, dev, 2, 0, 5, 7)
    run(oracle, uor, dev, 8, 4, 5, 0)


@pytest.mark.parametrize("offer", [True, False])
def test_i64_register_wraps_mod_2_192(oracle, uor, dev, offer):
    """Limbs<3>'s epilogue works in its fixed 192-bit register (epilogue.rs:
    307-328, acc.rs:208-215): every element i64::MIN, k = 2^12, so the sum is
    2^138; alpha = 2^54 gives 2^192 = 0, alpha = 2^53 gives 2^191 (the most
    negative value: O::MIN), and beta * C adds mod 2^192 -- on the residue
    route and on the per-cell loop, against the oracle."""
    m, k, n = 2, 1 << 12, 3
    a = np.full(m * k, np.iinfo(np.int64).min, np.int64)
    b = np.full(k * n, np.iinfo(np.int64).min, np.int64)
    for alpha, beta, out, encode in [(1 << 54, 0, "i64", "nearest"), (1 << 53, 0, "i32", "nearest"),
                                     (1 << 53, -(1 << 63), "i64", "nearest"),
                                     (1 << 52, 7, "i128", "nearest"), (3, -5, "i128", "wrapping"),
                                     (-(1 << 63), (1 << 63) - 1, "i16", "wrapping")]:
        run(oracle, uor, dev, 8, m, k, n, out=out, alpha=alpha, beta=beta, encode=encode,
            offer=offer, a=a, b=b)


def test_numpy_cx10_fixtures(uor, dev):
    """The reference's CX-10 cases (oracles/numpy, int64 elements, int64
    output, Wrapping): both routes reproduce the committed expected bytes."""
    d = GOLDEN / "numpy_cx10"
    man = json.loads((d / "manifest.json").read_text())
    for case in man["cases"]:
        m, k, n = (case["shape"][x] for x in "mkn")
        blobs = {}
        for name in ("a", "b", "expected"):
            raw = (d / f"{case['stem']}.{name}.bin").read_bytes()
            assert "sha256:" + hashlib.sha256(raw).hexdigest() == case[f"{name}_sha256"]
            blobs[name] = np.frombuffer(raw, "<i8").copy()
        if not (m and n):
            continue
        for offer in [True, False]:
            c = torch.zeros(m * n, dtype=torch.int64, device=dev)
            nbytes = uor.suggested_scratch_int(8, m, k, n) if offer else 0
            scratch = torch.empty(nbytes, dtype=torch.uint8, device=dev) if nbytes else None
            st, route = uor.gemm_int(torch.from_numpy(blobs["a"]).to(dev), (m, k), (k, 1),
                                     torch.from_numpy(blobs["b"]).to(dev), (k, n), (n, 1), c,
                                     (m, n), (n, 1), out="i64", encode="wrapping",
                                     scratch=scratch)
            torch.cuda.synchronize()
            assert st == 0
            assert np.array_equal(c.cpu().numpy(), blobs["expected"]), (case["stem"], route)


@pytest.mark.parametrize("offer", [True, False])
def test_wrapping_narrow_output_is_the_modular_lane(oracle, uor, dev, offer):
    """Wrapping into at most 32 bits scales the sum in Z/2^32 (the public
    route's modular lane), so alpha = 2^63 - 1 on i32 elements near their
    extremes wraps instead of saturating; wider outputs saturate first.  The
    closed form (all 2^31 - 1, k = 8): -8 for i32/i16 outputs, -1 for i64."""
    k = 8
    a = np.full(k, (1 << 31) - 1, np.int32)
    for out, want in (("i32", -8), ("i16", -8), ("i64", -1)):
        run(oracle, uor, dev, 4, 1, k, 1, out=out, alpha=(1 << 63) - 1, encode="wrapping",
            offer=offer, a=a, b=a.copy())
        c = torch.zeros(1, dtype={"i32": torch.int32, "i16": torch.int16, "i64": torch.int64}[out],
                        device=dev)
        st, _ = uor.gemm_int(torch.from_numpy(a).to(dev), (1, k), (k, 1),
                             torch.from_numpy(a).to(dev), (k, 1), (1, 1), c, (1, 1), (1, 1),
                             out=out, alpha=(1 << 63) - 1, encode="wrapping")
        torch.cuda.synchronize()
        assert st == 0 and int(c.cpu()[0]) == want, out
    # full-range operands, large scalars, every narrow output
    for out in ("i8", "i16", "i32"):
        run(oracle, uor, dev, 4, 17, 300, 23, out=out, alpha=(1 << 63) - 1, beta=-(1 << 62),
            encode="wrapping", offer=offer, seed=31)
