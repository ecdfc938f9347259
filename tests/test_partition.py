"""The partition of the output (crates/uor-matmul-gemm/src/partition.rs) and
MatView::subview (layout.rs:633-646) through the C ABI, host side only: no
call here enqueues device work."""
import ctypes
import itertools

import pytest


@pytest.fixture(scope="module")
def U():
    import uor_gfx950
    uor_gfx950.lib()
    return uor_gfx950


SHAPES = [(0, 0), (1, 1), (5, 7), (13, 17), (64, 64), (97, 3)]
TILES = [(0, 0), (1, 1), (2, 3), (8, 8), (64, 64), (1000, 1000)]


@pytest.mark.parametrize("m,n", SHAPES)
def test_partition_covers_the_output_exactly_once(U, m, n):
    """partition.rs:122-146 (CD-02): every cell of C in exactly one tile, for
    the reference's own shapes and tile extents."""
    for tr, tc in TILES:
        tiles = list(U.partition(m, n, tr, tc))
        assert len(tiles) == U.partition_len(m, n, tr, tc)
        seen = [0] * (m * n)
        for row, col, rows, cols in tiles:
            assert rows >= 1 and cols >= 1
            assert rows <= (tr or max(m, 1)) and cols <= (tc or max(n, 1))
            for i in range(row, row + rows):
                for j in range(col, col + cols):
                    seen[i * n + j] += 1
        assert all(s == 1 for s in seen), (m, n, tr, tc)


def test_partition_len_and_order(U):
    """partition.rs:150-158: indexing and iterating agree, tile(len) is None,
    tiles run row-major, and len is zero exactly when the output is empty."""
    m, n = 13, 17
    tiles = list(U.partition(m, n, 4, 6))
    assert len(tiles) == 4 * 3
    assert tiles == [U.partition_tile(m, n, 4, 6, i) for i in range(12)]
    assert U.partition_tile(m, n, 4, 6, 12) is None
    assert U.partition_tile(m, n, 4, 6, 1 << 60) is None
    assert tiles[0] == (0, 0, 4, 6) and tiles[1] == (0, 6, 4, 6) and tiles[2] == (0, 12, 4, 5)
    assert tiles[-1] == (12, 12, 1, 5)
    assert U.partition_len(0, 5, 2, 2) == 0 and U.partition_len(5, 0, 2, 2) == 0
    assert U.partition_len(5, 5, 0, 0) == 1
    assert U.partition_tile(5, 5, 0, 0, 0) == (0, 0, 5, 5)
    # A count past 64 bits saturates, and every index below it still names
    # its tile: (2^64 - 2) = (2^24 - 1) * 2^40 + (2^40 - 2).
    big = 1 << 40
    assert U.partition_len(big, big, 1, 1) == (1 << 64) - 1
    assert U.partition_tile(big, big, 1, 1, (1 << 64) - 2) == ((1 << 24) - 1, big - 2, 1, 1)


def window(rows, cols, rs, cs):
    offs = [i * rs + j * cs for i in range(rows) for j in range(cols)]
    return min(offs), max(offs)


@pytest.mark.parametrize("rs,cs", [(9, 1), (1, 7), (-9, 1), (9, -1), (-9, -1), (20, 2), (-20, 3)])
def test_subview_names_the_same_cells(U, rs, cs):
    """Every cell of a block addresses the byte the parent view gives it, and
    the block's buffer is exactly the window it reaches (lowest offset at its
    start, highest at its end)."""
    rows, cols, elem = 7, 6, 4
    lo, hi = window(rows, cols, rs, cs)
    base = 0x10000
    v = U.View(base, hi - lo + 1, rows, cols, rs, cs)
    origin = -lo

    def addr(view, r, c):
        vlo, _ = window(view.rows, view.cols, view.rs, view.cs)
        return view.data + (-vlo + r * view.rs + c * view.cs) * elem

    for i, j, br, bc in itertools.product(range(0, 7, 2), range(0, 6, 3), (1, 2, 5), (1, 3)):
        st, s = U.subview(v, elem, i, j, br, bc)
        if i + br > rows or j + bc > cols:
            assert U.STATUS[st] == "invalid_argument"
            continue
        assert st == 0
        assert (s.rows, s.cols, s.rs, s.cs) == (br, bc, rs, cs)
        slo, shi = window(br, bc, rs, cs)
        assert s.len == shi - slo + 1
        for r in range(br):
            for c in range(bc):
                want = base + (origin + (i + r) * rs + (j + c) * cs) * elem
                assert addr(s, r, c) == want
        # The block's window lies inside the parent's buffer.
        assert s.data >= base and s.data + s.len * elem <= base + v.len * elem


def test_subview_edges(U):
    v = U.View(0x1000, 12, 3, 4, 4, 1)
    st, s = U.subview(v, 1, 3, 0, 0, 4)   # empty block at the end: allowed
    assert st == 0 and s.rows == 0 and s.len == 0
    st, s = U.subview(v, 1, 0, 4, 3, 0)
    assert st == 0 and s.cols == 0 and s.len == 0
    assert U.STATUS[U.subview(v, 1, 1, 0, 3, 4)[0]] == "invalid_argument"
    assert U.STATUS[U.subview(v, 1, 0, 0, 1 << 63, 1 << 63)[0]] == "invalid_argument"
    short = U.View(0x1000, 11, 3, 4, 4, 1)   # the parent itself does not fit
    assert U.STATUS[U.subview(short, 1, 0, 0, 1, 1)[0]] == "short_buffer"
    assert U.STATUS[U.subview(v, 0, 0, 0, 1, 1)[0]] == "invalid_argument"


def test_tiled_validation_without_a_gpu(U):
    """The tiled executors check the whole call first, as the single call
    would, and enqueue nothing when it fails (fake addresses, never read)."""
    L = U.lib()
    P = 0x1000
    a = U.View(P, 6, 2, 3, 3, 1)
    b = U.View(P, 8, 4, 2, 2, 1)       # 4 x 2: A's 3 columns do not conform
    c = U.View(P, 4, 2, 2, 2, 1)
    ran = ctypes.c_uint64(99)
    st = L.uor_gfx950_gemm_i8_tiled(ctypes.byref(a), ctypes.byref(b), ctypes.byref(c), 4, 1, 0,
                                    0, 1, 1, None, 0, None, 0, ctypes.byref(ran))
    assert U.STATUS[st] == "nonconformant" and ran.value == 0
    b = U.View(P, 6, 3, 2, 2, 1)
    c = U.View(P, 4, 2, 2, 1, 1)       # rs 1 = cs 1: aliases itself
    st = L.uor_gfx950_gemm_float_tiled(0, ctypes.byref(a), ctypes.byref(b), ctypes.byref(c), 1,
                                       0, 0, 1, 1, None, 0, None, 0, ctypes.byref(ran))
    assert U.STATUS[st] == "output_aliases_itself" and ran.value == 0
    c = U.View(P, 3, 2, 2, 2, 1)       # too short for 2 x 2
    st = L.uor_gfx950_gemm_i8_tiled(ctypes.byref(a), ctypes.byref(b), ctypes.byref(c), 4, 1, 0,
                                    0, 1, 1, None, 0, None, 0, ctypes.byref(ran))
    assert U.STATUS[st] == "short_buffer"
    c = U.View(P, 4, 2, 2, 2, 1)
    st = L.uor_gfx950_gemm_i8_tiled(ctypes.byref(a), ctypes.byref(b), ctypes.byref(c), 3, 1, 0,
                                    0, 1, 1, None, 0, None, 0, ctypes.byref(ran))
    assert U.STATUS[st] == "invalid_argument"   # no 3-byte output type
    st = L.uor_gfx950_gemm_i8_tiled(ctypes.byref(a), ctypes.byref(b), ctypes.byref(c), 4, 1, 0,
                                    0, 1, 1, None, 2, None, 0, ctypes.byref(ran))
    assert U.STATUS[st] == "invalid_argument"   # two streams named, no array
    # An empty output is a valid call with no tiles.
    e = U.View(P, 0, 0, 2, 2, 1)
    a0 = U.View(P, 0, 0, 3, 3, 1)
    st = L.uor_gfx950_gemm_i8_tiled(ctypes.byref(a0), ctypes.byref(b), ctypes.byref(e), 4, 1, 0,
                                    0, 1, 1, None, 0, None, 0, ctypes.byref(ran))
    assert st == 0 and ran.value == 0
