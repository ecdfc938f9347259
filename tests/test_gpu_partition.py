"""The partition of the output run on several HIP streams of one GPU
(crates/uor-matmul-gemm/src/partition.rs; CD-02 / CD-08): for every tile
shape and stream count, and for tiles claimed in reverse order, the bytes of C
equal the single call's, which equal the oracle's."""
import numpy as np
import pytest
import torch

import gen

pytestmark = pytest.mark.gpu

OUT_NP = {"i8": np.int8, "i16": np.int16, "i32": np.int32, "i64": np.int64}


def streams(count):
    return [torch.cuda.Stream() for _ in range(count)]  # default priority


def join(ss):
    for s in ss:
        s.synchronize()
    torch.cuda.synchronize()


@pytest.mark.parametrize("m,k,n", [(67, 200, 45), (96, 8192, 70)])
@pytest.mark.parametrize("out,alpha,beta,encode", [("i32", 1, 0, "nearest"),
                                                  ("i8", 3, -2, "saturating"),
                                                  ("i16", -5, 7, "wrapping")])
def test_i8_tiles_on_streams_equal_the_single_call(oracle, uor, dev, m, k, n, out, alpha, beta,
                                                   encode):
    rng = np.random.default_rng(m * 7 + k + n)
    a = rng.integers(-128, 128, m * k, dtype=np.int8)
    b = rng.integers(-128, 128, k * n, dtype=np.int8)
    c0 = rng.integers(-100, 100, m * n).astype(OUT_NP[out])
    want = c0.copy()
    assert oracle.gemm_int(a, (m, k), (k, 1), b, (k, n), (n, 1), want, (m, n), (n, 1),
                           alpha=alpha, beta=beta, encode=encode) == "ok"
    ga, gb = torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev)
    offer = uor.suggested_scratch_i8(m, k, n)
    scratch = torch.empty(4 * offer + 4096, dtype=torch.uint8, device=dev)
    single = torch.from_numpy(c0.copy()).to(dev)
    st, _ = uor.gemm_i8(ga, (m, k), (k, 1), gb, (k, n), (n, 1), single, (m, n), (n, 1), out=out,
                        alpha=alpha, beta=beta, encode=encode, scratch=scratch)
    torch.cuda.synchronize()
    assert st == 0
    assert np.array_equal(single.cpu().numpy(), want)
    for (tr, tc), ns in [((0, 0), 1), ((32, 32), 2), ((17, 13), 4), ((m, 1), 3), ((1, n), 4),
                         ((64, 16), 0)]:
        ss = streams(ns)
        gc = torch.from_numpy(c0.copy()).to(dev)
        torch.cuda.synchronize()
        st, ran = uor.gemm_i8_tiled(ga, (m, k), (k, 1), gb, (k, n), (n, 1), gc, (m, n), (n, 1),
                                    tr, tc, streams=ss, out=out, alpha=alpha, beta=beta,
                                    encode=encode, scratch=scratch)
        join(ss)
        assert st == 0 and ran == uor.partition_len(m, n, tr, tc)
        assert torch.equal(gc, single), (tr, tc, ns)


def test_i8_tiles_claimed_in_reverse_on_four_streams(uor, dev):
    """partition.rs:150-158, environment.rs:221-249: a caller-side executor
    claims tiles out of order through Partition::tile and MatView::subview and
    runs each on its own stream; the bytes do not move."""
    m, k, n = 150, 1000, 90
    rng = np.random.default_rng(5)
    ga = torch.from_numpy(rng.integers(-128, 128, m * k, dtype=np.int8)).to(dev)
    gb = torch.from_numpy(rng.integers(-128, 128, k * n, dtype=np.int8)).to(dev)
    single = torch.zeros(m * n, dtype=torch.int32, device=dev)
    assert uor.gemm_i8(ga, (m, k), (k, 1), gb, (k, n), (n, 1), single, (m, n), (n, 1))[0] == 0
    torch.cuda.synchronize()
    av = uor.view(ga, m, k, k, 1)
    bv = uor.view(gb, k, n, n, 1)
    gc = torch.full((m * n,), -1, dtype=torch.int32, device=dev)
    cv = uor.view(gc, m, n, n, 1, elem=4)
    ss = streams(4)
    torch.cuda.synchronize()
    count = uor.partition_len(m, n, 40, 25)
    for idx in reversed(range(count)):
        row, col, rows, cols = uor.partition_tile(m, n, 40, 25, idx)
        sts = [uor.subview(av, 1, row, 0, rows, k), uor.subview(bv, 1, 0, col, k, cols),
               uor.subview(cv, 4, row, col, rows, cols)]
        assert all(s == 0 for s, _ in sts)
        (_, sa), (_, sb), (_, sc) = sts
        st = uor.lib().uor_gfx950_gemm_i8(*(uor.ctypes.byref(x) for x in (sa, sb, sc)), 4, 1, 0,
                                          0, None, 0, ss[idx % 4].cuda_stream, None)
        assert st == 0
    join(ss)
    assert torch.equal(gc, single)


@pytest.mark.parametrize("is64", [False, True])
def test_float_tiles_on_streams_equal_the_single_call(oracle, uor, dev, is64):
    m, k, n = 37, 300, 29
    a, b = gen.corpus_operands((m, k, n, "FewGrades", 5), is64)
    ft = a.dtype
    c0 = (np.arange(m * n) * 0.25 - 3).astype(ft)
    want = c0.copy()
    assert oracle.gemm_float(a, (m, k), (k, 1), b, (k, n), (n, 1), want, (m, n), (n, 1), alpha=3,
                             beta=-1) == "ok"
    ga, gb = torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev)
    offer = uor.suggested_scratch_float(is64, m, k, n)
    for (tr, tc), ns, share in [((0, 0), 1, 1), ((8, 8), 3, 3), ((16, 5), 4, 0), ((1, 29), 2, 2)]:
        ss = streams(ns)
        scratch = torch.empty(share * offer + 4096, dtype=torch.uint8, device=dev) if share else None
        gc = torch.from_numpy(c0.copy()).to(dev)
        torch.cuda.synchronize()
        st, ran = uor.gemm_float_tiled(ga, (m, k), (k, 1), gb, (k, n), (n, 1), gc, (m, n), (n, 1),
                                       tr, tc, streams=ss, alpha=3, beta=-1, scratch=scratch)
        join(ss)
        assert st == 0 and ran == uor.partition_len(m, n, tr, tc)
        got = gc.cpu().numpy()
        assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), (tr, tc, ns)
