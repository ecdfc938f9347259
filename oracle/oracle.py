"""ctypes face of the CPU oracle (oracle/uor_oracle.c) -- TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module. It restates the reference library's semantics on the host so the
GPU route has something independent to be compared against; the product
library never calls it.

Views follow the reference's MatView::new (crates/uor-matmul-core/src/layout.rs:212):
a buffer, a shape and two element strides; the origin is placed so that the
lowest offset reached is element 0.
"""
from __future__ import annotations

import ctypes
import os
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
# UOR_ORACLE_VARIANT=asan selects the AddressSanitizer/UBSan builds that
# `make -C oracle asan` makes and runs the CPU suite against.
_VARIANT = "_asan" if os.environ.get("UOR_ORACLE_VARIANT") == "asan" else ""
LIB = HERE / f"liboracle{_VARIANT}.so"

ENCODE = {"nearest": 0, "toward_zero": 1, "saturating": 2, "wrapping": 3}
STATUS = {0: "ok", 1: "nonconformant", 2: "output_aliases_itself",
          3: "short_buffer", 4: "invalid_argument"}

_u64, _i64, _i32, _vp = ctypes.c_uint64, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p
_VIEW = [_vp, _u64, _u64, _u64, _i64, _i64]

_lib = None


def build() -> None:
    target = "asan-libs" if _VARIANT else "all"
    subprocess.run(["make", "-s", "-C", str(HERE), "-B", target], check=True)


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = ctypes.CDLL(str(LIB))
        L.ora_place.argtypes = [_u64, _u64, _u64, _i64, _i64, ctypes.POINTER(_u64)]
        L.ora_place.restype = _i32
        L.ora_self_aliases.argtypes = [_u64, _u64, _i64, _i64]
        L.ora_self_aliases.restype = _i32
        L.ora_gemm_int.argtypes = [_i32] + _VIEW * 3 + [_i32, _i64, _i64, _i32]
        L.ora_gemm_int.restype = _i32
        L.ora_gemm_lut4.argtypes = [_vp, _u64, _u64, _u64, _i64, _i64, _vp, _u64, _u64,
                                    _vp, _u64, _u64, _vp, _u64, _i64, _i64,
                                    _i32, _i64, _i64, _i32]
        L.ora_gemm_lut4.restype = _i32
        L.ora_gemm_float.argtypes = [_i32] + _VIEW * 3 + [_i64, _i64, _i32]
        L.ora_gemm_float.restype = _i32
        L.ora_gemm_trop.argtypes = [_i32] + _VIEW * 3 + [_i32, _i64, _i32, _i64, _i32, _i32]
        L.ora_gemm_trop.restype = _i32
        L.ora_gemm_trop_selected.argtypes = [_i32] + _VIEW * 4 + [_i32, _i64, _i32, _i64, _i32, _i32]
        L.ora_gemm_trop_selected.restype = _i32
        L.ora_coded_decode.argtypes = [_i32, _i32, _i32, _i32, _i64, _u64, _u64, _vp, _u64,
                                       _vp, _u64, _u64, _u64, _vp]
        L.ora_coded_decode.restype = _i32
        _lib = L
    return _lib


def place(length, rows, cols, rs, cs):
    """The origin of an rows x cols view in `length` elements, or None."""
    o = _u64(0)
    ok = lib().ora_place(length, rows, cols, rs, cs, ctypes.byref(o))
    return o.value if ok else None


def self_aliases(rows, cols, rs, cs) -> bool:
    return bool(lib().ora_self_aliases(rows, cols, rs, cs))


def _ptr(arr):
    return arr.ctypes.data_as(_vp) if arr.size else None


def _view(arr, rows, cols, rs, cs, rec=1):
    return [_ptr(arr), arr.size // rec, rows, cols, rs, cs]


def row_major(rows, cols, ld=None):
    return (cols if ld is None else ld, 1)


_OUT_BYTES = {np.dtype(np.int8): 1, np.dtype(np.int16): 2, np.dtype(np.int32): 4,
              np.dtype(np.int64): 8}


def gemm_int(a, a_shape, a_strides, b, b_shape, b_strides, c, c_shape, c_strides,
             alpha=1, beta=0, encode="nearest", out_bytes=None):
    """driver::gemm with Linear{alpha,beta} over ring elements (i8/i16/i32/i64).

    `c` is updated in place; an i128 output is a (len, 2) int64 array / 16-byte
    records with out_bytes=16. Returns the status name.
    """
    eb = a.dtype.itemsize
    assert b.dtype == a.dtype
    ob = out_bytes or _OUT_BYTES[c.dtype]
    rec = 2 if ob == 16 else 1
    st = lib().ora_gemm_int(eb, *_view(a, *a_shape, *a_strides), *_view(b, *b_shape, *b_strides),
                            *_view(c, *c_shape, *c_strides, rec=rec), ob, int(alpha), int(beta),
                            ENCODE[encode])
    return STATUS[st]


def gemm_lut4(a, m, k, a_strides, codes, n, books, group, c, c_strides,
              alpha=1, beta=0, encode="nearest"):
    ob = _OUT_BYTES[c.dtype]
    st = lib().ora_gemm_lut4(_ptr(a), a.size, m, k, *a_strides, _ptr(codes), codes.size, n,
                             _ptr(books), books.size, group, _ptr(c), c.size, *c_strides,
                             ob, int(alpha), int(beta), ENCODE[encode])
    return STATUS[st]


def gemm_float(a, a_shape, a_strides, b, b_shape, b_strides, c, c_shape, c_strides,
               alpha=1, beta=0, encode="nearest"):
    is64 = a.dtype == np.float64
    assert b.dtype == a.dtype == c.dtype
    st = lib().ora_gemm_float(int(is64), *_view(a, *a_shape, *a_strides),
                              *_view(b, *b_shape, *b_strides), *_view(c, *c_shape, *c_strides),
                              int(alpha), int(beta), ENCODE[encode])
    return STATUS[st]


def gemm_trop(a, a_shape, a_strides, b, b_shape, b_strides, c, c_shape, c_strides,
              alpha=(0, True), beta=(0, False), encode="nearest", elem_bytes=1, out_bytes=4):
    """MaxPlus over Trop records: `a`/`b`/`c` are uint8 byte buffers of
    2*elem_bytes / 2*out_bytes-byte records. alpha/beta are (value, finite)."""
    st = lib().ora_gemm_trop(elem_bytes,
                             *_view(a, *a_shape, *a_strides, rec=2 * elem_bytes),
                             *_view(b, *b_shape, *b_strides, rec=2 * elem_bytes),
                             *_view(c, *c_shape, *c_strides, rec=2 * out_bytes),
                             out_bytes, int(alpha[0]), int(bool(alpha[1])),
                             int(beta[0]), int(bool(beta[1])), ENCODE[encode])
    return STATUS[st]


def gemm_trop_selected(a, a_shape, a_strides, b, b_shape, b_strides, c, c_shape, c_strides,
                       w, w_strides, alpha=(0, True), beta=(0, False), encode="nearest",
                       elem_bytes=1, out_bytes=4):
    """gemm_selected (Lexicographic) over Trop records: as gemm_trop, plus the
    witness `w`, a uint64 array viewed as an m x n matrix with w_strides."""
    m, n = c_shape
    st = lib().ora_gemm_trop_selected(elem_bytes,
                                      *_view(a, *a_shape, *a_strides, rec=2 * elem_bytes),
                                      *_view(b, *b_shape, *b_strides, rec=2 * elem_bytes),
                                      *_view(c, *c_shape, *c_strides, rec=2 * out_bytes),
                                      *_view(w, m, n, *w_strides),
                                      out_bytes, int(alpha[0]), int(bool(alpha[1])),
                                      int(beta[0]), int(bool(beta[1])), ENCODE[encode])
    return STATUS[st]


# ---------------------------------------------------------------- Trop records
TROP_I8 = np.dtype([("value", "i1"), ("finite", "u1")])
TROP_I32 = np.dtype([("value", "<i4"), ("finite", "u1"), ("_pad", "V3")])


def trop_i8(values, finite):
    out = np.zeros(np.shape(values), dtype=TROP_I8)
    out["value"] = np.where(finite, values, 0)
    out["finite"] = np.asarray(finite, dtype=np.uint8)
    return out


def trop_bytes(rec):
    return np.ascontiguousarray(rec).view(np.uint8).reshape(-1)


# ------------------------------------------------------------ CPU baseline
FAST = HERE / f"libfastroute{_VARIANT}.so"
_fast = None


def fast():
    """The CPU baseline (oracle/fastroute.cpp): the reference's fast routes
    restated in C++, timed beside the GPU by bench.py."""
    global _fast
    if _fast is None:
        if not FAST.exists():
            build()
        F = ctypes.CDLL(str(FAST))
        F.fr_has_vnni.restype = _i32
        F.fr_hw_threads.restype = _i32
        F.fr_gemm_i8_i32.argtypes = [_i32, _i32, _i32, _i64, _vp, _i64, _vp, _i64, _i64, _vp,
                                     _i64, _i32, _i32, _i32, _i32]
        F.fr_gemm_i8_i32.restype = _i32
        F.fr_lut4.argtypes = [_i32, _i32, _i32, _vp, _i64, _vp, _vp, _i32, _vp, _i64, _i32,
                              _i32, _i32]
        F.fr_lut4.restype = _i32
        F.fr_trop_i8.argtypes = [_i32, _i32, _i32, _vp, _vp, _vp, _i32, _i32, _i32]
        F.fr_trop_i8.restype = _i32
        F.fr_gemm_i8_i64_chunked.argtypes = [_i32, _i64, _i32, _vp, _i64, _vp, _i64, _vp, _i64,
                                             _i32]
        F.fr_gemm_i8_i64_chunked.restype = _i32
        _fast = F
    return _fast


def fast_gemm_i8_i32(m, k, n, alpha, a, lda, b, ldb, beta, c, ldc, row0=0, rows=None,
                     threads=1, force_avx2=False):
    rows = m if rows is None else rows
    return fast().fr_gemm_i8_i32(m, k, n, int(alpha), _ptr(a), lda, _ptr(b), ldb, int(beta),
                                 _ptr(c), ldc, row0, rows, threads, int(force_avx2))


def fast_lut4(m, k, n, a, codes, books, group, c, groups=None, threads=1, mode="tabulate"):
    """The table-lookup product on the CPU baseline: A (m x k i8, row-major),
    codes (n x k/2 bytes), one 16-entry book per `group` rows of W, C (m x n
    i32).  `groups` limits the run to the first groups (a bounded sample)."""
    groups = n // group if groups is None else groups
    return fast().fr_lut4(m, k, n, _ptr(a), k, _ptr(codes), _ptr(books), group, _ptr(c), n,
                          groups, threads, {"tabulate": 0, "decode_dense": 1}[mode])


def fast_gemm_i8_i64_chunked(m, k, n, a, lda, b, ldb, c, ldc, threads=1):
    """The chunked route on the CPU baseline: C (int64) := A B over any depth."""
    return fast().fr_gemm_i8_i64_chunked(m, k, n, _ptr(a), lda, _ptr(b), ldb, _ptr(c), ldc,
                                         threads)


def fast_trop_i8(m, k, n, a, b, c, row0=0, rows=None, threads=1):
    """Max-plus on the CPU baseline: Trop<i8> records in, Trop<i32> out
    (default MaxPlus), rows [row0, row0 + rows)."""
    rows = m if rows is None else rows
    return fast().fr_trop_i8(m, k, n, _ptr(a), _ptr(b), _ptr(c), row0, rows, threads)


# ------------------------------------------------------------------- codecs
TIER = {"identity": 0, "grid": 1, "book": 2, "sign": 3, "ternary": 4}


def codec(tier, code_bits=16, packed=0, zero=None, table=None, entries=None, block=1):
    """A fixed-width codec over the i8 alphabet (codecs.rs): the base tier,
    its code width, Packed<_, P> when packed > 0, Offset<_, zero> when zero is
    not None.  `table` is an int8 array (Grid: N entries, Book: N*BLK)."""
    t = None if table is None else np.ascontiguousarray(table, dtype=np.int8)
    if entries is None:
        entries = 0 if t is None else (t.size if tier == "grid" else t.size // max(block, 1))
    return {"tier": TIER[tier], "code_bits": code_bits, "packed": packed,
            "has_zero": int(zero is not None), "zero": 0 if zero is None else int(zero),
            "entries": entries, "block": block, "table": t}


def coded_decode(cd, codes, rows, cols):
    """CodedMatrix::new + every CodedMatrix::at, as (status, rows x cols int8)."""
    out = np.zeros(rows * cols, np.int8)
    t = cd["table"]
    codes = np.ascontiguousarray(codes)
    st = lib().ora_coded_decode(cd["tier"], cd["code_bits"], cd["packed"], cd["has_zero"],
                                cd["zero"], cd["entries"], cd["block"],
                                None if t is None or t.size == 0 else _ptr(t),
                                0 if t is None else t.size, _ptr(codes), codes.size, rows, cols,
                                _ptr(out))
    return STATUS[st], out.reshape(rows, cols)


def gemm_coded(a, a_shape, a_strides, cd, codes, w_rows, w_cols, transposed, c, c_shape,
               c_strides, alpha=1, beta=0, encode="nearest", out_bytes=None):
    """gemm_tabulated (transposed: W is n x k) or coded_gemm (W is k x n) over
    a fixed-width codec: the decode (CodedMatrix::at), then driver::gemm over
    the decoded operand -- the decode-then-multiply value (CD-13)."""
    st, w = coded_decode(cd, codes, w_rows, w_cols)
    if st != "ok":
        return st
    w = np.ascontiguousarray(w).reshape(-1)
    if transposed:
        b_shape, b_strides = (w_cols, w_rows), (1, w_cols)
    else:
        b_shape, b_strides = (w_rows, w_cols), (w_cols, 1)
    if w.size == 0:
        w = np.zeros(1, np.int8)
    return gemm_int(a, a_shape, a_strides, w, b_shape, b_strides, c, c_shape, c_strides,
                    alpha=alpha, beta=beta, encode=encode, out_bytes=out_bytes)
