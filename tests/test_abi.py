"""The C ABI library: it loads, it exports every function include/uor_gfx950.h
declares, and its host-side validation (the reference's MatView::new and
Triple::new, which run before anything is enqueued) answers without a GPU."""
import ctypes
import re

import pytest

from conftest import ROOT

HEADER = ROOT / "include" / "uor_gfx950.h"


def declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(uor_gfx950_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    import uor_gfx950
    lib = uor_gfx950.lib()
    names = declared()
    assert names, "the header declares entry points"
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # The Python face binds exactly what the header declares.
    assert set(names) == set(uor_gfx950.SYMBOLS) | {"uor_gfx950_status_string"}, \
        set(names) ^ set(uor_gfx950.SYMBOLS)


def test_status_strings():
    import uor_gfx950
    lib = uor_gfx950.lib()
    assert lib.uor_gfx950_status_string(0) == b"ok"
    assert lib.uor_gfx950_status_string(1) == b"nonconformant"
    assert lib.uor_gfx950_status_string(2) == b"output_aliases_itself"
    assert lib.uor_gfx950_status_string(3) == b"short_buffer"


def _v(ptr, length, rows, cols, rs, cs):
    import uor_gfx950
    return uor_gfx950.View(ptr, length, rows, cols, rs, cs)


def test_validation_statuses_without_a_gpu():
    """Non-existence is reported before any device work (error.rs:28-53).
    Fake non-null addresses are never dereferenced: every request here fails
    validation."""
    import uor_gfx950
    lib = uor_gfx950.lib()
    P = 0x1000
    call = lambda a, b, c, ob=4, enc=0: lib.uor_gfx950_gemm_i8(
        ctypes.byref(a), ctypes.byref(b), ctypes.byref(c), ob, 1, 0, enc, None, 0, None, None)
    assert call(_v(P, 12, 3, 4, 4, 1), _v(P, 12, 3, 4, 4, 1), _v(P, 16, 3, 4, 4, 1)) == 1
    assert call(_v(P, 12, 3, 4, 4, 1), _v(P, 12, 4, 3, 3, 1), _v(P, 9, 3, 4, 4, 1)) == 3
    assert call(_v(P, 12, 3, 4, 4, 1), _v(P, 12, 4, 3, 3, 1), _v(P, 9, 3, 3, 1, 1)) == 2
    assert call(_v(P, 12, 3, 4, 4, 1), _v(P, 12, 4, 3, 3, 1), _v(P, 9, 3, 3, 3, 1), ob=3) == 4
    assert call(_v(P, 12, 3, 4, 4, 1), _v(P, 12, 4, 3, 3, 1), _v(P, 9, 3, 3, 3, 1), enc=7) == 4
    # 5 x 1 at rs = 1 << 62: the reach overflows, so no such view exists.
    assert call(_v(P, 100, 5, 1, 1 << 62, 1), _v(P, 1, 1, 1, 1, 1), _v(P, 5, 5, 1, 1, 1)) == 3
    # The slice face: a short slice is status 3 (does_not_fit, slice.rs:104-116).
    assert lib.uor_gfx950_slice_gemm_i8(4, 4, 4, P, 15, P, 16, P, 16, 4, None, 0, None) == 3


def test_coded_and_witness_validation_without_a_gpu():
    """gemm_coded and gemm_trop_i8_selected decide every refusal on the host:
    CodedMatrix::new's shape rule, the codec fields the decode needs, the
    triple, and SelectedTriple::new's witness rules.  Fake addresses, never
    dereferenced."""
    import uor_gfx950 as u
    lib = u.lib()
    P = 0x1000
    a, c = _v(P, 4 * 48, 4, 48, 48, 1), _v(P, 4 * 16, 4, 16, 16, 1)
    tern = u.Codec(u.TIER["ternary"], 8, 0, 0, 0, 0, 4, None, 0)  # Ternary<4, u8>

    def coded(cd, codes_len, w_rows=16, w_cols=48, a=a, c=c):
        return lib.uor_gfx950_gemm_coded(ctypes.byref(a), ctypes.byref(cd), P, codes_len, w_rows,
                                         w_cols, 1, ctypes.byref(c), 4, 1, 0, 0, None, 0, None, None)
    assert coded(tern, 16 * 48 // 4 + 1) == 3                       # code count
    assert coded(tern, 16 * 50 // 4, w_cols=50) == 3                 # width % MAX_BLOCK
    assert coded(u.Codec(9, 8, 0, 0, 0, 0, 4, None, 0), 192) == 4    # unknown tier
    assert coded(u.Codec(4, 8, 3, 0, 0, 0, 4, None, 0), 192) == 4    # P = 3
    assert coded(u.Codec(1, 16, 0, 0, 0, 16, 1, None, 0), 768) == 3  # Grid without its table
    assert coded(tern, 16 * 40 // 4, w_cols=40) == 1                 # A is 48 deep, W 40
    assert coded(tern, 192, c=_v(P, 16, 4, 16, 0, 1)) == 2           # aliasing C

    def sel(w, mech=0):
        av, bv = _v(P, 20, 4, 5, 5, 1), _v(P, 30, 5, 6, 6, 1)
        cv = _v(P, 24, 4, 6, 6, 1)
        return lib.uor_gfx950_gemm_trop_i8_selected(ctypes.byref(av), ctypes.byref(bv),
                                                    ctypes.byref(cv), ctypes.byref(w), 4, 0, 1,
                                                    0, 0, 0, mech, None, 0, None, None)
    assert sel(_v(P, 24, 4, 5, 5, 1)) == 1     # witness not m x n
    assert sel(_v(P, 24, 4, 6, 0, 1)) == 2     # witness aliases itself
    assert sel(_v(P, 20, 4, 6, 6, 1)) == 3     # witness buffer too short
    assert sel(_v(P, 24, 4, 6, 6, 1), mech=7) == 4


def test_coded_float_validation_without_a_gpu():
    """gemm_coded_float's refusals, all on the host (fake addresses)."""
    import uor_gfx950 as u
    lib = u.lib()
    P = 0x1000
    a, c = _v(P, 2 * 257, 2, 257, 257, 1), _v(P, 2 * 13, 2, 13, 13, 1)

    def call(is64=0, bits=8, codes_len=13 * 257, w_rows=13, w_cols=257, entries=256, c=c, sc=0):
        return lib.uor_gfx950_gemm_coded_float(is64, ctypes.byref(a), P, entries, bits, P, codes_len,
                                               w_rows, w_cols, 1, ctypes.byref(c), 1, 0, 0,
                                               P if sc else None, sc, None, None)
    assert call(is64=2) == 4
    assert call(bits=12) == 4
    assert call(entries=0) == 4
    assert call(codes_len=13 * 257 - 1) == 3                    # CodedMatrix::new
    assert call(w_rows=14, codes_len=14 * 257) == 1             # C is 2 x 13
    assert call(c=_v(P, 26, 2, 13, 0, 1)) == 2                  # aliasing C
    assert call(sc=16) == 4                                     # offer below the decoded operand
