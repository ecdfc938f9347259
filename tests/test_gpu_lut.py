"""GPU parity of the 4-bit table-lookup GEMM (uor_gfx950_gemm_lut4) against the
oracle; full decode shapes (m in {1, 8, 32}, k = 8192,
n = 28672, one codebook per 128 coded rows) against a decode in torch plus a
float64 matmul, exact because every sum is an integer below 2^53."""
import numpy as np
import pytest
import torch

import gen

pytestmark = pytest.mark.gpu


def to_dev(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def run_case(oracle, uor, dev, m, k, n, group, seed, out=np.int32, alpha=1, beta=0,
             encode="nearest", a_strides=None, code_offset=0, expect=None, offer=False):
    rng = np.random.default_rng(seed)
    ars, acs = a_strides or (k, 1)
    alen = 1 + max(0, (m - 1) * abs(ars) + (k - 1) * abs(acs)) if m and k else 0
    a = rng.integers(-128, 128, alen + 7).astype(np.int8)
    codes = rng.integers(0, 256, n * k // 2 + code_offset).astype(np.uint8)
    books = rng.integers(-128, 128, ((n + group - 1) // group) * 16).astype(np.int8)
    c0 = rng.integers(np.iinfo(out).min // 2, np.iinfo(out).max // 2, m * n).astype(out)
    want = c0.copy()
    st = oracle.gemm_lut4(a, m, k, (ars, acs), codes[code_offset:].copy(), n, books, group, want,
                          (n, 1), alpha=alpha, beta=beta, encode=encode)
    gc = to_dev(c0, dev)
    gcodes = to_dev(codes, dev)[code_offset:]
    ost = {np.int8: "i8", np.int16: "i16", np.int32: "i32", np.int64: "i64"}[out]
    scratch = None
    if offer:
        nbytes = uor.suggested_scratch_lut4(m, k, n)
        scratch = torch.empty(nbytes, dtype=torch.uint8, device=dev) if nbytes else None
    gst, route = uor.gemm_lut4(to_dev(a, dev), m, k, (ars, acs), gcodes, n, to_dev(books, dev),
                               group, gc, (n, 1), out=ost, alpha=alpha, beta=beta, encode=encode,
                               scratch=scratch)
    torch.cuda.synchronize()
    assert uor.STATUS.get(gst, gst) == st
    assert np.array_equal(gc.cpu().numpy(), want), (m, k, n, group, route)
    if expect:
        assert route["tile_n"] == expect, route
    return route


@pytest.mark.parametrize("m,k,n,group", [
    (1, 2, 1, 1), (1, 64, 37, 5), (1, 8192, 300, 128), (2, 512, 70, 16), (3, 8192, 129, 128),
    (4, 1000, 64, 64), (5, 256, 33, 7), (8, 8192, 96, 128), (17, 640, 65, 32), (32, 2048, 64, 128),
    (33, 130, 31, 3), (64, 4096, 40, 128)])
def test_shapes_against_oracle(oracle, uor, dev, m, k, n, group):
    run_case(oracle, uor, dev, m, k, n, group, seed=m * 7 + k + n)


@pytest.mark.parametrize("m", [1, 3, 8])
def test_unaligned_and_strided(oracle, uor, dev, m):
    """Odd code offsets and column-strided activations take the gathering
    loads; the bytes are the same."""
    k, n = 256, 45
    run_case(oracle, uor, dev, m, k, n, 4, seed=5 + m, code_offset=3)
    run_case(oracle, uor, dev, m, k, n, 4, seed=9 + m, a_strides=(1, m + 2))


@pytest.mark.parametrize("out", [np.int8, np.int16, np.int32, np.int64])
@pytest.mark.parametrize("encode", ["nearest", "wrapping"])
@pytest.mark.parametrize("m", [1, 9])
def test_epilogue(oracle, uor, dev, out, encode, m):
    for alpha, beta in [(1, 0), (3, -1), (1 << 40, -(1 << 35))]:
        run_case(oracle, uor, dev, m, 128, 40, 8, seed=11, out=out, alpha=alpha, beta=beta,
                 encode=encode)


TILE = (8, 16)  # route["split_k"] of the 16-column tile kernel (its waves per workgroup)


@pytest.mark.parametrize("out", [np.int8, np.int16, np.int32, np.int64])
@pytest.mark.parametrize("encode", ["nearest", "wrapping"])
@pytest.mark.parametrize("k", [2048, 16384])
def test_lds_and_tile_kernel_epilogue(oracle, uor, dev, out, encode, k):
    """The output paths of the 16-column tile kernel (k = 2048: a multiple of
    2048 up to 8192, m <= 16) and of the LDS-activation kernel (k = 16384,
    2 <= m <= 32): i32 rows in 16-byte stores except the ragged last columns (n = 45),
    the per-cell finish for the other widths, each with plain, scaled and
    saturating alpha/beta."""
    for alpha, beta in [(1, 0), (3, -1), (1 << 40, -(1 << 35))]:
        route = run_case(oracle, uor, dev, 9, k, 45, 8, seed=13, out=out, alpha=alpha,
                         beta=beta, encode=encode)
        assert route["kind"] == "lut4_mfma", route
        assert (route["split_k"] in TILE) == (k <= 8192), route


@pytest.mark.parametrize("m", [1, 2, 5, 7, 8, 9, 16, 17, 32])
@pytest.mark.parametrize("k", [2048, 4096, 6144, 8192])
def test_tile_kernel_against_oracle(oracle, uor, dev, m, k):
    """The tile kernels at every depth they take: 8-column tiles at one row,
    16-column tiles (one or two row blocks) beyond; ragged n (a last
    tile of 3 or 2 columns), codebook groups that are not a multiple of the
    tile (7) or are single columns, alpha/beta and the i64 epilogue, against
    the oracle."""
    for n, group, out, alpha, beta in [(35, 7, np.int32, 1, 0), (50, 1, np.int64, -3, 2),
                                       (64, 128, np.int32, 5, -1)]:
        route = run_case(oracle, uor, dev, m, k, n, group, seed=m * 31 + k + n, out=out,
                         alpha=alpha, beta=beta)
        assert route["kind"] == "lut4_mfma" and route["split_k"] in TILE, route
        assert route["tile_n"] == (8 if m == 1 else 16), route


@pytest.mark.parametrize("m,k,n,group", [(1, 8192, 28672, 128), (8, 8192, 40000 + 9, 64),
                                         (32, 8192, 28672, 128), (24, 4096, 12 * 256 * 16, 128),
                                         (3, 2048, 16 * 100 + 1, 16), (12, 8192, 256 * 16, 3),
                                         (16, 4096, 12 * 256 * 16 + 16, 128),
                                         (1, 4096, 12 * 512 * 8, 128), (1, 2048, 12 * 512 * 8 + 8, 128)])
def test_tile_kernel_tiles_per_workgroup(uor, dev, m, k, n, group):
    """The tile kernels with 7, 10 and 12 tiles per workgroup (the most whose
    sums they hold), fewer tiles than CUs, one tile per CU, and one tile past
    the limit (another kernel then); against a decode in torch plus a float64
    matmul (exact: every sum is an integer below 2^53)."""
    rng = np.random.default_rng(m + k + n)
    a = to_dev(rng.integers(-128, 128, m * k).astype(np.int8), dev)
    codes = to_dev(rng.integers(0, 256, n * k // 2).astype(np.uint8), dev)
    books = to_dev(rng.integers(-128, 128, ((n + group - 1) // group) * 16).astype(np.int8), dev)
    c = torch.full((m * n,), 7, dtype=torch.int32, device=dev)
    st, route = uor.gemm_lut4(a, m, k, (k, 1), codes, n, books, group, c, (n, 1))
    torch.cuda.synchronize()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    tiled8 = m == 1 and (n + 7) // 8 <= 12 * 2 * cus
    tiled = tiled8 or (n + 15) // 16 <= 12 * cus
    assert st == 0 and route["kind"] == ("lut4_mfma" if tiled or m > 4 else "lut4_dot4"), route
    assert (route["split_k"] in TILE) == tiled, route
    if tiled:
        assert route["tile_n"] == (8 if tiled8 else 16), route
    W = decode_torch(codes, n, k, books, group).to(torch.float64)
    want = a.view(m, k).to(torch.float64) @ W.T
    assert torch.equal(c.view(m, n).to(torch.float64), want), route


def test_deep_rows_fold_exactly(oracle, uor, dev):
    """k past one i32 lane's reach (2^17 weights of |w*a| = 2^14) folds into
    i64: all -128 activations against a codebook of -128 give k * 2^14."""
    m, n, k = 2, 3, 1 << 18
    a = torch.full((m * k,), -128, dtype=torch.int8, device=dev)
    codes = torch.zeros(n * k // 2, dtype=torch.uint8, device=dev)
    books = torch.full((16,), -128, dtype=torch.int8, device=dev)
    c = torch.zeros(m * n, dtype=torch.int64, device=dev)
    st, _ = uor.gemm_lut4(a, m, k, (k, 1), codes, n, books, n, c, (n, 1), out="i64")
    torch.cuda.synchronize()
    assert st == 0 and c.cpu().tolist() == [k << 14] * (m * n)
    c32 = torch.zeros(m * n, dtype=torch.int32, device=dev)
    st, _ = uor.gemm_lut4(a, m, k, (k, 1), codes, n, books, n, c32, (n, 1), out="i32")
    torch.cuda.synchronize()
    assert st == 0 and c32.cpu().tolist() == [(1 << 31) - 1] * (m * n)


def decode_torch(codes, n, k, books, group):
    c = codes.view(n, k // 2).to(torch.int64)
    nib = torch.empty((n, k), dtype=torch.int64, device=codes.device)
    nib[:, 0::2] = c & 15
    nib[:, 1::2] = c >> 4
    g = (torch.arange(n, device=codes.device) // group)[:, None]
    return books.view(-1, 16).to(torch.int64)[g, nib]


@pytest.mark.parametrize("m", [1, 8, 32])
def test_config3_decode_shape(uor, dev, m):
    """A uniform i8 (salt 6), codes uniform 0..15 two per byte
    (salt 7), 224 codebooks uniform i8 (salt 8), k = 8192, n = 28672."""
    k, n, group = 8192, 28672, 128
    a = to_dev(gen.i8_full(m * k, 6), dev)
    codes = to_dev(gen.i8_full(n * k // 2, 7).view(np.uint8), dev)
    books = to_dev(gen.i8_full((n // group) * 16, 8), dev)
    c = torch.zeros(m * n, dtype=torch.int32, device=dev)
    st, route = uor.gemm_lut4(a, m, k, (k, 1), codes, n, books, group, c, (n, 1))
    torch.cuda.synchronize()
    assert st == 0
    W = decode_torch(codes, n, k, books, group).to(torch.float64)
    want = a.view(m, k).to(torch.float64) @ W.T
    assert torch.equal(c.view(m, n).to(torch.float64), want), route
    if m > 4:
        assert route["kind"] == "lut4_mfma" and route["tile_n"] == 16, route


@pytest.mark.parametrize("k", [1 << 18, (1 << 18) + 128])
def test_mfma16_quarters_at_depth_limit(uor, dev, k):
    """The 16-column MFMA tiles split k in four quarters of at most 65536
    weights, each exact in i32 (2^16 * 2^14 = 2^30); at k = 2^18 every quarter
    is at that limit, and one step more takes the other kernel.  All -128
    against a codebook of -128: every cell is k * 2^14 (past i32 in total)."""
    m, n = 8, 40
    a = torch.full((m * k,), -128, dtype=torch.int8, device=dev)
    codes = torch.zeros(n * k // 2, dtype=torch.uint8, device=dev)
    books = torch.full((16 * 3,), -128, dtype=torch.int8, device=dev)
    c = torch.zeros(m * n, dtype=torch.int64, device=dev)
    st, route = uor.gemm_lut4(a, m, k, (k, 1), codes, n, books, 16, c, (n, 1), out="i64")
    torch.cuda.synchronize()
    assert st == 0 and c.cpu().tolist() == [k << 14] * (m * n), route
    assert route["tile_n"] == (16 if k <= (1 << 18) else 32), route



@pytest.mark.parametrize("m,k,n", [(8, 4096, 8192 - 5), (20, 2048, 12288 + 3), (13, 2048, 32768),
                                   (32, 2048, 28672), (5, 6144, 16 * 256 * 5 + 9), (32, 2048, 64),
                                   (2, 8192, 28672), (4, 2048, 1000), (8, 16384, 8192 - 5),
                                   (32, 10240, 4096 + 3)])
def test_tiles_per_cu(uor, dev, m, k, n):
    """2 <= m <= 32 with 2, 4, 8, 7, 6, 1, 7 and 1 sixteen-column tiles per
    CU (ragged n, one row block or two): the code-stream kernel up to
    k = 8192, the LDS-activation kernel beyond (one to five activation
    chunks), against a decode in torch plus a float64 matmul (exact: every
    sum is an integer below 2^53)."""
    group = 128
    rng = np.random.default_rng(m + k + n)
    a = to_dev(rng.integers(-128, 128, m * k).astype(np.int8), dev)
    codes = to_dev(rng.integers(0, 256, n * k // 2).astype(np.uint8), dev)
    books = to_dev(rng.integers(-128, 128, ((n + group - 1) // group) * 16).astype(np.int8), dev)
    c = torch.zeros(m * n, dtype=torch.int32, device=dev)
    st, route = uor.gemm_lut4(a, m, k, (k, 1), codes, n, books, group, c, (n, 1))
    torch.cuda.synchronize()
    assert st == 0 and route["kind"] == "lut4_mfma", route
    assert (route["split_k"] in TILE) == (k <= 8192), route
    W = decode_torch(codes, n, k, books, group).to(torch.float64)
    want = a.view(m, k).to(torch.float64) @ W.T
    assert torch.equal(c.view(m, n).to(torch.float64), want), route


@pytest.mark.parametrize("m,k,n,group,out,alpha,beta,code_offset", [
    (128, 2048, 96, 32, np.int32, 1, 0, 0), (200, 1000, 333, 7, np.int64, 3, -1, 0),
    (130, 256, 45, 4, np.int16, 1 << 40, -(1 << 35), 3), (300, 130, 1000, 128, np.int8, 3, -1, 0),
    (96, 4096, 300, 128, np.int32, 3, -1, 0), (80, 4352, 260, 32, np.int64, -2, 5, 0)])
def test_prefill_decode_then_dense(oracle, uor, dev, m, k, n, group, out, alpha, beta, code_offset):
    """m >= 128 (m >= 80 at k >= 4096) with the suggested offer: W^T decoded
    once into the offer, then the dense int8 route (ragged n, k not a
    multiple of the 32-weight
    decode chunk, unaligned code rows, every output width's epilogue).  The
    same bytes as the oracle; without the offer the table-lookup kernels."""
    route = run_case(oracle, uor, dev, m, k, n, group, seed=m + n, out=out, alpha=alpha, beta=beta,
                     code_offset=code_offset, offer=True)
    assert route["kind"] == "lut4_prefill", route
    route = run_case(oracle, uor, dev, m, k, n, group, seed=m + n, out=out, alpha=alpha, beta=beta,
                     code_offset=code_offset)
    assert route["kind"] != "lut4_prefill", route


def test_prefill_config_shape(uor, dev):
    """The config 3 weights (k = 8192, n = 28672, 224 codebooks) at m = 512 on
    the decode-then-dense route, against a decode in torch and a float64
    matmul (exact: every sum is an integer below 2^53)."""
    m, k, n, group = 512, 8192, 28672, 128
    a = to_dev(gen.i8_full(m * k, 6), dev)
    codes = to_dev(gen.i8_full(n * k // 2, 7).view(np.uint8), dev)
    books = to_dev(gen.i8_full((n // group) * 16, 8), dev)
    c = torch.zeros(m * n, dtype=torch.int32, device=dev)
    scratch = torch.empty(uor.suggested_scratch_lut4(m, k, n), dtype=torch.uint8, device=dev)
    st, route = uor.gemm_lut4(a, m, k, (k, 1), codes, n, books, group, c, (n, 1), scratch=scratch)
    torch.cuda.synchronize()
    assert st == 0 and route["kind"] == "lut4_prefill", route
    W = decode_torch(codes, n, k, books, group).to(torch.float64)
    want = a.view(m, k).to(torch.float64) @ W.T
    assert torch.equal(c.view(m, n).to(torch.float64), want), route
