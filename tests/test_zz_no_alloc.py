"""The no-alloc entry point (uor_gfx950_gemm_i8_noalloc, through the C ABI):
the same bytes as uor_gfx950_gemm_i8 with the suggested offer, on two calls
in a row whose second is smaller (the static scratch keeps the first call's
partial sums, which the route clears), on routes with and without scratch,
and the refusal of a request beyond the static maximum.  Bar: bit-exact."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def to_dev(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def both(uor, dev, m, k, n, seed, out="i64", alpha=3, beta=-2):
    rng = np.random.default_rng(seed)
    a = to_dev(rng.integers(-128, 128, m * k).astype(np.int8), dev)
    b = to_dev(rng.integers(-128, 128, k * n).astype(np.int8), dev)
    dt = {"i32": np.int32, "i64": np.int64}[out]
    c0 = rng.integers(-1000, 1000, m * n).astype(dt)
    ref = to_dev(c0, dev)
    got = to_dev(c0, dev)
    scratch = torch.empty(uor.suggested_scratch_i8(m, k, n), dtype=torch.uint8, device=dev)
    st, r_ref = uor.gemm_i8(a, (m, k), (k, 1), b, (k, n), (n, 1), ref, (m, n), (n, 1), out=out,
                            alpha=alpha, beta=beta, scratch=scratch)
    assert st == 0
    st, r_got = uor.gemm_i8_noalloc(a, (m, k), (k, 1), b, (k, n), (n, 1), got, (m, n), (n, 1),
                                    out=out, alpha=alpha, beta=beta)
    torch.cuda.synchronize()
    assert st == 0, st
    assert r_got["kind"] == r_ref["kind"], (r_got, r_ref)
    assert torch.equal(got, ref), (m, k, n, r_got)
    return r_got


def test_two_calls_second_smaller(uor, dev):
    """Split-K (k past one i32 lane): 200 x 70000 x 160, then 72 x 66000 x 40
    (its partials land in the first call's leftover scratch)."""
    r1 = both(uor, dev, 200, 70_000, 160, seed=1)
    r2 = both(uor, dev, 72, 66_000, 40, seed=2)
    assert r1["kind"] == r2["kind"] == "mfma_splitk", (r1, r2)


def test_small_output_deep_and_fused(uor, dev):
    """Split-K for a small output at k >= 8192, then the fused tile (no
    scratch), then split-K again: each equals gemm_i8's bytes."""
    assert both(uor, dev, 64, 9000, 48, seed=3, out="i32", alpha=1, beta=0)["kind"] == "mfma_splitk"
    assert both(uor, dev, 300, 500, 260, seed=4, out="i32")["kind"] == "mfma_tile"
    assert both(uor, dev, 16, 131_072 + 5, 24, seed=5)["kind"] == "mfma_splitk"


def test_beyond_static_scratch_refused(uor, dev):
    """A split-K request whose partial sums exceed the static array returns
    UOR_SCRATCH_LIMIT before anything runs; C is untouched."""
    m, k, n = 1536, 70_000, 1536  # m*n*8 = 18 MiB > 16 MiB
    assert m * n * 8 > uor.NOALLOC_SCRATCH_BYTES
    a = torch.zeros(m * k, dtype=torch.int8, device=dev)
    b = torch.zeros(k * n, dtype=torch.int8, device=dev)
    c = torch.full((m * n,), 7, dtype=torch.int32, device=dev)
    st, _ = uor.gemm_i8_noalloc(a, (m, k), (k, 1), b, (k, n), (n, 1), c, (m, n), (n, 1))
    torch.cuda.synchronize()
    assert uor.STATUS[st] == "scratch_limit"
    assert bool((c == 7).all())
