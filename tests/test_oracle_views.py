"""Pins the oracle's view placement and self-alias predicate by brute force.

The reference's MatView::new (crates/uor-matmul-core/src/layout.rs:161-212)
accepts a view iff every coordinate lands in the buffer after placing the
lowest reached offset at element 0; Strides::self_aliases (layout.rs:116-143)
is exact: two distinct coordinates share a cell.  Both are checked here by
enumerating every coordinate, which shares no code with the gcd formula.
"""
import itertools

import pytest


def brute_place(length, rows, cols, rs, cs):
    if rows == 0 or cols == 0:
        return 0
    offs = [i * rs + j * cs for i in range(rows) for j in range(cols)]
    lo, hi = min(offs), max(offs)
    origin = -lo
    return origin if origin + hi < length else None


def brute_alias(rows, cols, rs, cs):
    seen = set()
    for i in range(rows):
        for j in range(cols):
            o = i * rs + j * cs
            if o in seen:
                return True
            seen.add(o)
    return False


STRIDES = [-7, -4, -3, -1, 0, 1, 2, 3, 4, 5, 6, 9]


def test_place_matches_enumeration(oracle):
    for rows, cols in [(0, 3), (3, 0), (1, 1), (1, 5), (5, 1), (3, 4), (4, 3)]:
        for rs, cs in itertools.product(STRIDES, STRIDES):
            need = brute_place(10 ** 6, rows, cols, rs, cs)
            for length in (0, 1, 11, 12, 13, 40, 10 ** 6):
                want = brute_place(length, rows, cols, rs, cs)
                got = oracle.place(length, rows, cols, rs, cs)
                assert got == want, (rows, cols, rs, cs, length, need)


def test_self_aliases_matches_enumeration(oracle):
    for rows, cols in [(0, 5), (5, 0), (1, 1), (1, 7), (7, 1), (2, 2), (3, 5), (5, 3), (6, 4)]:
        for rs, cs in itertools.product(STRIDES, STRIDES):
            assert oracle.self_aliases(rows, cols, rs, cs) == brute_alias(rows, cols, rs, cs), \
                (rows, cols, rs, cs)


def test_overflowing_reach_names_no_view(oracle):
    # layout.rs:62-68: 5 x 1 at rs = 1 << 62 must be rejected, not wrapped.
    assert oracle.place(100, 5, 1, 1 << 62, 1) is None
    assert oracle.place(100, 2, 1, -(1 << 63), 1) is None
