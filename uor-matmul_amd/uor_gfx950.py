"""ctypes binding of libuor_gfx950.so (the C ABI in include/uor_gfx950.h).

Buffers are device tensors from PyTorch (used only for device memory and
streams); every computation runs in the library's HIP kernels.  Loading fails
loudly when the library has not been built: there is no other route.

Import torch before this module so the library binds to the HIP runtime torch
already loaded (both carry the SONAME libamdhip64.so.7).
"""
from __future__ import annotations

import ctypes
import os
import pathlib

HERE = pathlib.Path(__file__).resolve().parent
# UOR_GFX950_LIB points the binding at another build of the same ABI.
LIB_PATH = pathlib.Path(os.environ.get("UOR_GFX950_LIB", HERE / "libuor_gfx950.so"))

OUT = {"i8": 1, "i16": 2, "i32": 4, "i64": 8, "i128": 16}
ENCODE = {"nearest": 0, "toward_zero": 1, "saturating": 2, "wrapping": 3}
STATUS = {0: "ok", 1: "nonconformant", 2: "output_aliases_itself", 3: "short_buffer",
          4: "invalid_argument", 5: "scratch_limit"}
ROUTES = {0: "none", 1: "epilogue_only", 2: "mfma_tile", 3: "mfma_splitk", 4: "mfma_wide",
          5: "collapsed",
          10: "lut4_dot4", 11: "lut4_mfma", 12: "lut4_prefill",
          13: "coded_dense", 14: "coded_direct", 15: "coded_gemv", 20: "float_crt", 21: "float_direct", 30: "trop_valu",
          31: "trop_selected", 32: "trop_selected_direct", 40: "int_crt", 41: "int_direct", 42: "int_limb"}
WITNESS = {"lexicographic": 0, "compare_pass": 1}

# Every symbol include/uor_gfx950.h declares.
SYMBOLS = [
    "uor_gfx950_status_string",
    "uor_gfx950_gemm_i8",
    "uor_gfx950_slice_gemm_ex_i8",
    "uor_gfx950_slice_gemm_i8",
    "uor_gfx950_suggested_scratch_i8",
    "uor_gfx950_gemm_i8_noalloc",
    "uor_gfx950_gemm_int",
    "uor_gfx950_suggested_scratch_int",
    "uor_gfx950_gemm_lut4",
    "uor_gfx950_suggested_scratch_lut4",
    "uor_gfx950_gemm_coded",
    "uor_gfx950_suggested_scratch_coded",
    "uor_gfx950_gemm_coded_collapsed",
    "uor_gfx950_suggested_scratch_coded_collapse",
    "uor_gfx950_gemm_coded_float",
    "uor_gfx950_suggested_scratch_coded_float",
    "uor_gfx950_manifest_json",
    "uor_gfx950_gemm_float",
    "uor_gfx950_slice_gemm_float_ex",
    "uor_gfx950_slice_gemm_float",
    "uor_gfx950_sgemm",
    "uor_gfx950_dgemm",
    "uor_gfx950_suggested_scratch_float",
    "uor_gfx950_gemm_trop_i8",
    "uor_gfx950_gemm_trop_i8_selected",
    "uor_gfx950_gemm_collapsed_i8",
    "uor_gfx950_suggested_scratch_collapse",
    "uor_gfx950_partition_len",
    "uor_gfx950_partition_tile",
    "uor_gfx950_subview",
    "uor_gfx950_gemm_i8_tiled",
    "uor_gfx950_gemm_float_tiled",
]


class View(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("len", ctypes.c_uint64), ("rows", ctypes.c_uint64),
                ("cols", ctypes.c_uint64), ("rs", ctypes.c_int64), ("cs", ctypes.c_int64)]


class Tile(ctypes.Structure):
    _fields_ = [("row", ctypes.c_uint64), ("col", ctypes.c_uint64), ("rows", ctypes.c_uint64),
                ("cols", ctypes.c_uint64)]

    def as_tuple(self):
        return (self.row, self.col, self.rows, self.cols)


class Codec(ctypes.Structure):
    _fields_ = [("tier", ctypes.c_int32), ("code_bits", ctypes.c_int32),
                ("packed", ctypes.c_int32), ("has_zero", ctypes.c_int32),
                ("zero", ctypes.c_int64), ("entries", ctypes.c_uint64),
                ("block", ctypes.c_uint64), ("table", ctypes.c_void_p),
                ("table_len", ctypes.c_uint64)]


TIER = {"identity": 0, "grid": 1, "book": 2, "sign": 3, "ternary": 4, "packed": 5, "offset": 6,
        "runs": 7, "transcode": 8, "arena": 9}


class Route(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int32), ("tile_m", ctypes.c_int32), ("tile_n", ctypes.c_int32),
                ("tile_k", ctypes.c_int32), ("split_k", ctypes.c_int32),
                ("launches", ctypes.c_int32), ("operand_modes", ctypes.c_int32),
                ("moduli", ctypes.c_int32), ("scratch_used", ctypes.c_uint64)]

    def as_dict(self):
        d = {f: getattr(self, f) for f, _ in self._fields_}
        d["kind"] = ROUTES.get(self.kind, self.kind)
        return d


_u64, _i64, _i32, _vp = ctypes.c_uint64, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p
_PV = ctypes.POINTER(View)
_PR = ctypes.POINTER(Route)
_lib = None


class UorError(RuntimeError):
    def __init__(self, status):
        self.status = status
        super().__init__(f"uor_gfx950 status {status} ({STATUS.get(status, 'hip_error')})")


def lib():
    """The loaded C ABI.  Raises if libuor_gfx950.so is missing."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise FileNotFoundError(
                f"{LIB_PATH} is not built; run `python uor-matmul_amd/build.py` "
                "(or __graft_entry__.build()) first")
        L = ctypes.CDLL(str(LIB_PATH))
        L.uor_gfx950_status_string.argtypes = [_i32]
        L.uor_gfx950_status_string.restype = ctypes.c_char_p
        L.uor_gfx950_gemm_i8.argtypes = [_PV, _PV, _PV, _i32, _i64, _i64, _i32, _vp, _u64, _vp, _PR]
        L.uor_gfx950_gemm_i8.restype = _i32
        L.uor_gfx950_slice_gemm_ex_i8.argtypes = [_u64, _u64, _u64, _i64, _vp, _u64, _u64, _vp,
                                                  _u64, _u64, _i64, _vp, _u64, _u64, _i32, _vp,
                                                  _u64, _vp]
        L.uor_gfx950_slice_gemm_ex_i8.restype = _i32
        L.uor_gfx950_slice_gemm_i8.argtypes = [_u64, _u64, _u64, _vp, _u64, _vp, _u64, _vp, _u64,
                                               _i32, _vp, _u64, _vp]
        L.uor_gfx950_slice_gemm_i8.restype = _i32
        L.uor_gfx950_suggested_scratch_i8.argtypes = [_u64, _u64, _u64]
        L.uor_gfx950_suggested_scratch_i8.restype = _u64
        if hasattr(L, "uor_gfx950_partition_len"):
            L.uor_gfx950_partition_len.argtypes = [_u64, _u64, _u64, _u64]
            L.uor_gfx950_partition_len.restype = _u64
            L.uor_gfx950_partition_tile.argtypes = [_u64, _u64, _u64, _u64, _u64,
                                                    ctypes.POINTER(Tile)]
            L.uor_gfx950_partition_tile.restype = _i32
            L.uor_gfx950_subview.argtypes = [_PV, _i32, _u64, _u64, _u64, _u64, _PV]
            L.uor_gfx950_subview.restype = _i32
            L.uor_gfx950_gemm_i8_tiled.argtypes = [_PV, _PV, _PV, _i32, _i64, _i64, _i32, _u64,
                                                   _u64, ctypes.POINTER(_vp), ctypes.c_uint32,
                                                   _vp, _u64, ctypes.POINTER(_u64)]
            L.uor_gfx950_gemm_i8_tiled.restype = _i32
            L.uor_gfx950_gemm_float_tiled.argtypes = [_i32, _PV, _PV, _PV, _i64, _i64, _i32,
                                                      _u64, _u64, ctypes.POINTER(_vp),
                                                      ctypes.c_uint32, _vp, _u64,
                                                      ctypes.POINTER(_u64)]
            L.uor_gfx950_gemm_float_tiled.restype = _i32
        if hasattr(L, "uor_gfx950_gemm_int"):
            L.uor_gfx950_gemm_int.argtypes = [_i32, _PV, _PV, _PV, _i32, _i64, _i64, _i32, _vp,
                                              _u64, _vp, _PR]
            L.uor_gfx950_gemm_int.restype = _i32
            L.uor_gfx950_suggested_scratch_int.argtypes = [_i32, _u64, _u64, _u64]
            L.uor_gfx950_suggested_scratch_int.restype = _u64
        if hasattr(L, "uor_gfx950_gemm_lut4"):
            L.uor_gfx950_gemm_lut4.argtypes = [_PV, _vp, _u64, _u64, _vp, _u64, _u64, _PV, _i32,
                                               _i64, _i64, _i32, _vp, _u64, _vp, _PR]
            L.uor_gfx950_gemm_lut4.restype = _i32
            L.uor_gfx950_suggested_scratch_lut4.argtypes = [_u64, _u64, _u64]
            L.uor_gfx950_suggested_scratch_lut4.restype = _u64
        if hasattr(L, "uor_gfx950_gemm_collapsed_i8"):
            L.uor_gfx950_gemm_collapsed_i8.argtypes = [_PV, _PV, _PV, _i32, _i64, _i64, _i32, _i32,
                                                       _vp, _u64, _vp, _PR]
            L.uor_gfx950_gemm_collapsed_i8.restype = _i32
            L.uor_gfx950_suggested_scratch_collapse.argtypes = [_u64, _u64, _u64]
            L.uor_gfx950_suggested_scratch_collapse.restype = _u64
        if hasattr(L, "uor_gfx950_gemm_coded"):
            L.uor_gfx950_gemm_coded.argtypes = [_PV, ctypes.POINTER(Codec), _vp, _u64, _u64, _u64,
                                                _i32, _PV, _i32, _i64, _i64, _i32, _vp, _u64, _vp,
                                                _PR]
            L.uor_gfx950_gemm_coded.restype = _i32
            L.uor_gfx950_suggested_scratch_coded.argtypes = [_u64, _u64, _u64]
            L.uor_gfx950_suggested_scratch_coded.restype = _u64
            L.uor_gfx950_gemm_coded_collapsed.argtypes = L.uor_gfx950_gemm_coded.argtypes
            L.uor_gfx950_gemm_coded_collapsed.restype = _i32
            L.uor_gfx950_suggested_scratch_coded_collapse.argtypes = [_u64, _u64, _u64]
            L.uor_gfx950_suggested_scratch_coded_collapse.restype = _u64
            L.uor_gfx950_gemm_coded_float.argtypes = [_i32, _PV, _vp, _u64, _i32, _vp, _u64, _u64,
                                                      _u64, _i32, _PV, _i64, _i64, _i32, _vp, _u64,
                                                      _vp, _PR]
            L.uor_gfx950_gemm_coded_float.restype = _i32
            L.uor_gfx950_suggested_scratch_coded_float.argtypes = [_i32, _u64, _u64, _u64]
            L.uor_gfx950_suggested_scratch_coded_float.restype = _u64
        if hasattr(L, "uor_gfx950_manifest_json"):
            L.uor_gfx950_manifest_json.argtypes = [_i32, _u64, _u64, _u64, _u64, _u64,
                                                   ctypes.c_char_p, ctypes.c_char_p,
                                                   ctypes.c_char_p, ctypes.c_char_p, _u64,
                                                   ctypes.POINTER(_u64)]
            L.uor_gfx950_manifest_json.restype = _i32
        if hasattr(L, "uor_gfx950_gemm_float"):
            L.uor_gfx950_gemm_float.argtypes = [_i32, _PV, _PV, _PV, _i64, _i64, _i32, _vp, _u64,
                                                _vp, _PR]
            L.uor_gfx950_gemm_float.restype = _i32
            L.uor_gfx950_slice_gemm_float_ex.argtypes = [_i32, _u64, _u64, _u64, _i64, _vp, _u64,
                                                         _u64, _vp, _u64, _u64, _i64, _vp, _u64,
                                                         _u64, _vp, _u64, _vp]
            L.uor_gfx950_slice_gemm_float_ex.restype = _i32
            L.uor_gfx950_slice_gemm_float.argtypes = [_i32, _u64, _u64, _u64, _vp, _u64, _vp,
                                                      _u64, _vp, _u64, _vp, _u64, _vp]
            L.uor_gfx950_slice_gemm_float.restype = _i32
            for name in ("uor_gfx950_sgemm", "uor_gfx950_dgemm"):
                f = getattr(L, name)
                f.argtypes = [_u64, _u64, _u64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _i64,
                              _vp, _i64, _i64, _vp, _u64, _vp]
                f.restype = _i32
            L.uor_gfx950_suggested_scratch_float.argtypes = [_i32, _u64, _u64, _u64]
            L.uor_gfx950_suggested_scratch_float.restype = _u64
        if hasattr(L, "uor_gfx950_gemm_trop_i8"):
            L.uor_gfx950_gemm_trop_i8.argtypes = [_PV, _PV, _PV, _i32, _i64, _i32, _i64, _i32,
                                                  _i32, _vp, _u64, _vp, _PR]
            L.uor_gfx950_gemm_trop_i8.restype = _i32
            L.uor_gfx950_gemm_trop_i8_selected.argtypes = [_PV, _PV, _PV, _PV, _i32, _i64, _i32,
                                                           _i64, _i32, _i32, _i32, _vp, _u64, _vp,
                                                           _PR]
            L.uor_gfx950_gemm_trop_i8_selected.restype = _i32
        _lib = L
    return _lib


def _ptr(t):
    return None if t is None or t.numel() == 0 else t.data_ptr()


def _stream(stream):
    if stream is not None:
        return stream
    import torch
    return torch.cuda.current_stream().cuda_stream


def _dev(buf):
    """A buffer handed to the library must be device memory, contiguous."""
    if buf is None:
        return None
    if not buf.is_cuda:
        raise ValueError("uor_gfx950 buffers are device tensors")
    if not buf.is_contiguous():
        raise ValueError("uor_gfx950 buffers are contiguous tensors (strides go in the view)")
    return buf


def _len(buf, elem):
    """The buffer's length in elements of `elem` bytes (the C side's element
    type), whatever the tensor's own dtype: an int8 tensor passed as an i32
    output holds a quarter as many elements as it has bytes."""
    if buf is None:
        return 0
    return buf.numel() * buf.element_size() // elem


def _nbytes(buf):
    return 0 if buf is None else _dev(buf).numel() * buf.element_size()


def view(buf, rows, cols, rs, cs, elem=1):
    """A uor_view over the flat device tensor `buf` whose elements, as the
    library reads them, are `elem` bytes (1 for i8, the output width for C, 2
    for a Trop<i8> record, ...)."""
    _dev(buf)
    return View(_ptr(buf), _len(buf, elem), rows, cols, rs, cs)


def gemm_i8(a, a_shape, a_strides, b, b_shape, b_strides, c, c_shape, c_strides,
            out="i32", alpha=1, beta=0, encode="nearest", scratch=None, stream=None):
    """The view API at E = i8.  Returns (status, route dict).  `c` is a flat
    device tensor of the output type (int8/16/32/64, or int64 pairs for i128)."""
    ob = OUT[out]
    av = view(a, *a_shape, *a_strides)
    bv = view(b, *b_shape, *b_strides)
    cv = view(c, *c_shape, *c_strides, elem=ob)
    r = Route()
    st = lib().uor_gfx950_gemm_i8(ctypes.byref(av), ctypes.byref(bv), ctypes.byref(cv), ob,
                                  int(alpha), int(beta), ENCODE[encode], _ptr(scratch),
                                  _nbytes(scratch), _stream(stream), ctypes.byref(r))
    return st, r.as_dict()


def partition_len(m, n, tile_rows, tile_cols):
    """Partition::new(..).len(): tiles of at most tile_rows x tile_cols (0 = whole extent)."""
    return lib().uor_gfx950_partition_len(m, n, tile_rows, tile_cols)


def partition_tile(m, n, tile_rows, tile_cols, index):
    """Partition::tile: (row, col, rows, cols) of tile `index`, or None past the end."""
    t = Tile()
    if not lib().uor_gfx950_partition_tile(m, n, tile_rows, tile_cols, index, ctypes.byref(t)):
        return None
    return t.as_tuple()


def partition(m, n, tile_rows, tile_cols):
    """The Partition iterator: every tile in the stable order."""
    for i in range(partition_len(m, n, tile_rows, tile_cols)):
        yield partition_tile(m, n, tile_rows, tile_cols, i)


def subview(v, elem, i, j, rows, cols):
    """MatView::subview over a View: (status, View)."""
    out = View()
    st = lib().uor_gfx950_subview(ctypes.byref(v), elem, i, j, rows, cols, ctypes.byref(out))
    return st, out


def _streams(streams):
    if not streams:
        return None, 0
    arr = (_vp * len(streams))(*[s.cuda_stream if hasattr(s, "cuda_stream") else s
                                 for s in streams])
    return arr, len(streams)


def gemm_i8_tiled(a, a_shape, a_strides, b, b_shape, b_strides, c, c_shape, c_strides,
                  tile_rows, tile_cols, streams=(), out="i32", alpha=1, beta=0,
                  encode="nearest", scratch=None):
    """The partition run on streams (tile t on streams[t % len]): (status, tiles enqueued)."""
    ob = OUT[out]
    av = view(a, *a_shape, *a_strides)
    bv = view(b, *b_shape, *b_strides)
    cv = view(c, *c_shape, *c_strides, elem=ob)
    arr, ns = _streams(streams)
    ran = _u64(0)
    st = lib().uor_gfx950_gemm_i8_tiled(ctypes.byref(av), ctypes.byref(bv), ctypes.byref(cv), ob,
                                        int(alpha), int(beta), ENCODE[encode], tile_rows,
                                        tile_cols, arr, ns, _ptr(scratch), _nbytes(scratch),
                                        ctypes.byref(ran))
    return st, ran.value


def gemm_float_tiled(a, a_shape, a_strides, b, b_shape, b_strides, c, c_shape, c_strides,
                     tile_rows, tile_cols, streams=(), alpha=1, beta=0, encode="nearest",
                     scratch=None):
    import torch
    is64 = int(a.dtype == torch.float64)
    es = 8 if is64 else 4
    av = view(a, *a_shape, *a_strides, elem=es)
    bv = view(b, *b_shape, *b_strides, elem=es)
    cv = view(c, *c_shape, *c_strides, elem=es)
    arr, ns = _streams(streams)
    ran = _u64(0)
    st = lib().uor_gfx950_gemm_float_tiled(is64, ctypes.byref(av), ctypes.byref(bv),
                                           ctypes.byref(cv), int(alpha), int(beta),
                                           ENCODE[encode], tile_rows, tile_cols, arr, ns,
                                           _ptr(scratch), _nbytes(scratch), ctypes.byref(ran))
    return st, ran.value


def slice_gemm_ex_i8(m, k, n, alpha, a, lda, b, ldb, beta, c, ldc, out="i32", scratch=None,
                     stream=None):
    ob = OUT[out]
    a, b, c = _dev(a), _dev(b), _dev(c)
    return lib().uor_gfx950_slice_gemm_ex_i8(
        m, k, n, int(alpha), _ptr(a), _len(a, 1), lda, _ptr(b), _len(b, 1), ldb, int(beta),
        _ptr(c), _len(c, ob), ldc, ob, _ptr(scratch), _nbytes(scratch), _stream(stream))


def slice_gemm_i8(m, k, n, a, b, c, out="i32", scratch=None, stream=None):
    ob = OUT[out]
    a, b, c = _dev(a), _dev(b), _dev(c)
    return lib().uor_gfx950_slice_gemm_i8(
        m, k, n, _ptr(a), _len(a, 1), _ptr(b), _len(b, 1), _ptr(c), _len(c, ob), ob,
        _ptr(scratch), _nbytes(scratch), _stream(stream))


def suggested_scratch_i8(m, k, n):
    return lib().uor_gfx950_suggested_scratch_i8(m, k, n)


NOALLOC_SCRATCH_BYTES = 16 << 20  # UOR_NOALLOC_SCRATCH_BYTES


def gemm_i8_noalloc(a, a_shape, a_strides, b, b_shape, b_strides, c, c_shape, c_strides,
                    out="i32", alpha=1, beta=0, encode="nearest", stream=None):
    """gemm_i8 with the library's static per-GPU scratch (no offer, no
    allocation).  Returns (status, route dict)."""
    ob = OUT[out]
    av = view(a, *a_shape, *a_strides)
    bv = view(b, *b_shape, *b_strides)
    cv = view(c, *c_shape, *c_strides, elem=ob)
    r = Route()
    L = lib()
    L.uor_gfx950_gemm_i8_noalloc.argtypes = [_PV, _PV, _PV, _i32, _i64, _i64, _i32, _vp, _PR]
    L.uor_gfx950_gemm_i8_noalloc.restype = _i32
    st = L.uor_gfx950_gemm_i8_noalloc(ctypes.byref(av), ctypes.byref(bv), ctypes.byref(cv), ob,
                                      int(alpha), int(beta), ENCODE[encode], _stream(stream),
                                      ctypes.byref(r))
    return st, r.as_dict()


def gemm_int(a, a_shape, a_strides, b, b_shape, b_strides, c, c_shape, c_strides,
             out="i64", alpha=1, beta=0, encode="nearest", scratch=None, stream=None):
    """The view API at E = i8/i16/i32/i64 (the element width from a's dtype).
    Returns (status, route dict).  `c` is a flat device tensor of the output
    type (int8/16/32/64, or int64 pairs for i128)."""
    eb = a.element_size()
    ob = OUT[out]
    av = view(a, *a_shape, *a_strides, elem=eb)
    bv = view(b, *b_shape, *b_strides, elem=eb)
    cv = view(c, *c_shape, *c_strides, elem=ob)
    r = Route()
    st = lib().uor_gfx950_gemm_int(eb, ctypes.byref(av), ctypes.byref(bv), ctypes.byref(cv), ob,
                                   int(alpha), int(beta), ENCODE[encode], _ptr(scratch),
                                   _nbytes(scratch), _stream(stream), ctypes.byref(r))
    return st, r.as_dict()


def suggested_scratch_int(elem_bytes, m, k, n):
    return lib().uor_gfx950_suggested_scratch_int(elem_bytes, m, k, n)


def gemm_lut4(a, m, k, a_strides, codes, n, books, group, c, c_strides, out="i32", alpha=1,
              beta=0, encode="nearest", scratch=None, stream=None):
    ob = OUT[out]
    av = view(a, m, k, *a_strides)
    cv = view(c, m, n, *c_strides, elem=ob)
    codes, books = _dev(codes), _dev(books)
    r = Route()
    st = lib().uor_gfx950_gemm_lut4(
        ctypes.byref(av), _ptr(codes), _len(codes, 1), n, _ptr(books), _len(books, 1), group,
        ctypes.byref(cv), ob, int(alpha), int(beta), ENCODE[encode], _ptr(scratch),
        _nbytes(scratch), _stream(stream), ctypes.byref(r))
    return st, r.as_dict()


def suggested_scratch_lut4(m, k, n):
    return lib().uor_gfx950_suggested_scratch_lut4(m, k, n)


def gemm_float(a, a_shape, a_strides, b, b_shape, b_strides, c, c_shape, c_strides, alpha=1,
               beta=0, encode="nearest", scratch=None, stream=None):
    import torch
    is64 = int(a.dtype == torch.float64)
    es = 8 if is64 else 4
    av = view(a, *a_shape, *a_strides, elem=es)
    bv = view(b, *b_shape, *b_strides, elem=es)
    cv = view(c, *c_shape, *c_strides, elem=es)
    r = Route()
    st = lib().uor_gfx950_gemm_float(
        is64, ctypes.byref(av), ctypes.byref(bv), ctypes.byref(cv), int(alpha), int(beta),
        ENCODE[encode], _ptr(scratch), _nbytes(scratch), _stream(stream), ctypes.byref(r))
    return st, r.as_dict()


def slice_gemm_float_ex(m, k, n, alpha, a, lda, b, ldb, beta, c, ldc, scratch=None, stream=None):
    import torch
    is64 = int(a.dtype == torch.float64)
    es = 8 if is64 else 4
    a, b, c = _dev(a), _dev(b), _dev(c)
    return lib().uor_gfx950_slice_gemm_float_ex(
        is64, m, k, n, int(alpha), _ptr(a), _len(a, es), lda, _ptr(b), _len(b, es), ldb,
        int(beta), _ptr(c), _len(c, es), ldc, _ptr(scratch), _nbytes(scratch), _stream(stream))


def slice_gemm_float(m, k, n, a, b, c, scratch=None, stream=None):
    """slice::gemm_float: contiguous row-major, alpha 1, beta 0."""
    import torch
    is64 = int(a.dtype == torch.float64)
    es = 8 if is64 else 4
    a, b, c = _dev(a), _dev(b), _dev(c)
    return lib().uor_gfx950_slice_gemm_float(
        is64, m, k, n, _ptr(a), _len(a, es), _ptr(b), _len(b, es), _ptr(c), _len(c, es),
        _ptr(scratch), _nbytes(scratch), _stream(stream))


def raw_gemm(m, k, n, alpha, a, rsa, csa, b, rsb, csb, beta, c, rsc, csc, a_off=0, b_off=0,
             c_off=0, scratch=None, stream=None):
    """raw::sgemm / dgemm: a, b, c are device tensors and *_off the element
    index of element (0, 0) inside each (strides may be negative)."""
    import torch
    is64 = a.dtype == torch.float64
    es = 8 if is64 else 4
    f = lib().uor_gfx950_dgemm if is64 else lib().uor_gfx950_sgemm
    return f(m, k, n, int(alpha), a.data_ptr() + a_off * es, rsa, csa, b.data_ptr() + b_off * es,
             rsb, csb, int(beta), c.data_ptr() + c_off * es, rsc, csc, _ptr(scratch),
             _nbytes(scratch), _stream(stream))


def suggested_scratch_float(is64, m, k, n):
    return lib().uor_gfx950_suggested_scratch_float(int(is64), m, k, n)


def gemm_trop_i8(a, a_shape, a_strides, b, b_shape, b_strides, c, c_shape, c_strides, out=4,
                 alpha=(0, True), beta=(0, False), encode="nearest", scratch=None, stream=None):
    """a, b: uint8 device tensors of 2-byte Trop<i8> records; c: uint8 tensor of
    2*out-byte Trop<out> records."""
    av = view(a, *a_shape, *a_strides, elem=2)
    bv = view(b, *b_shape, *b_strides, elem=2)
    cv = view(c, *c_shape, *c_strides, elem=2 * out)
    r = Route()
    st = lib().uor_gfx950_gemm_trop_i8(
        ctypes.byref(av), ctypes.byref(bv), ctypes.byref(cv), out, int(alpha[0]),
        int(bool(alpha[1])), int(beta[0]), int(bool(beta[1])), ENCODE[encode], _ptr(scratch),
        _nbytes(scratch), _stream(stream), ctypes.byref(r))
    return st, r.as_dict()


def gemm_trop_i8_selected(a, a_shape, a_strides, b, b_shape, b_strides, c, c_shape, c_strides,
                          w, w_strides, out=4, alpha=(0, True), beta=(0, False), encode="nearest",
                          mechanism="lexicographic", w_shape=None, scratch=None, stream=None):
    """gemm_selected at E = Trop<i8>: as gemm_trop_i8, plus the witness `w`, a
    flat int64/uint64 device tensor viewed as w_shape (default c_shape) with
    w_strides."""
    av = view(a, *a_shape, *a_strides, elem=2)
    bv = view(b, *b_shape, *b_strides, elem=2)
    cv = view(c, *c_shape, *c_strides, elem=2 * out)
    wv = view(w, *(w_shape or c_shape), *w_strides, elem=8)
    r = Route()
    st = lib().uor_gfx950_gemm_trop_i8_selected(
        ctypes.byref(av), ctypes.byref(bv), ctypes.byref(cv), ctypes.byref(wv), out,
        int(alpha[0]), int(bool(alpha[1])), int(beta[0]), int(bool(beta[1])), ENCODE[encode],
        WITNESS.get(mechanism, mechanism), _ptr(scratch), _nbytes(scratch), _stream(stream),
        ctypes.byref(r))
    return st, r.as_dict()


def codec(tier, code_bits=16, packed=0, zero=None, table=None, entries=None, block=1):
    """A uor_codec: the base tier (identity/grid/book/sign/ternary), its code
    width in bits, Packed<_, P> when packed > 0, Offset<_, zero> when zero is
    not None.  `table` is an int8 device tensor (Grid: N entries, Book: N*BLK);
    keep it alive for the call."""
    n = 0 if table is None else table.numel()
    if entries is None:
        entries = n if tier == "grid" else (n // max(block, 1) if tier == "book" else 0)
    return Codec(TIER.get(tier, tier), code_bits, packed, int(zero is not None),
                 0 if zero is None else int(zero), entries, block, _ptr(table), n)


def gemm_coded(a, a_shape, a_strides, cd, codes, w_rows, w_cols, transposed, c, c_shape,
               c_strides, out="i32", alpha=1, beta=0, encode="nearest", scratch=None,
               stream=None, collapse=False):
    """gemm_tabulated (transposed: W is n x k) or coded_gemm (W is k x n) with
    W a fixed-width coded operand: `codes` is a device tensor of the stored
    codes (uint8, or int16/uint16 for 16-bit codes)."""
    ob = OUT[out]
    av = view(a, *a_shape, *a_strides)
    cv = view(c, *c_shape, *c_strides, elem=ob)
    # Stored codes are bytes when packed, else code_bits / 8 bytes each.
    celem = 1 if cd.packed else max(1, cd.code_bits // 8)
    codes = _dev(codes)
    r = Route()
    f = lib().uor_gfx950_gemm_coded_collapsed if collapse else lib().uor_gfx950_gemm_coded
    st = f(
        ctypes.byref(av), ctypes.byref(cd), _ptr(codes), _len(codes, celem), w_rows, w_cols,
        int(bool(transposed)), ctypes.byref(cv), ob, int(alpha), int(beta), ENCODE[encode],
        _ptr(scratch), _nbytes(scratch), _stream(stream), ctypes.byref(r))
    return st, r.as_dict()


def suggested_scratch_coded(m, k, n):
    return lib().uor_gfx950_suggested_scratch_coded(m, k, n)


def gemm_collapsed_i8(a, a_shape, a_strides, b, b_shape, b_strides, c, c_shape, c_strides,
                      out="i32", alpha=1, beta=0, encode="nearest", columns=False, scratch=None,
                      stream=None):
    """gemm_collapsed at E = i8: the bytes of gemm_i8, one product line per
    distinct row of A (columns=True: per distinct column of B)."""
    ob = OUT[out]
    av = view(a, *a_shape, *a_strides)
    bv = view(b, *b_shape, *b_strides)
    cv = view(c, *c_shape, *c_strides, elem=ob)
    r = Route()
    st = lib().uor_gfx950_gemm_collapsed_i8(
        ctypes.byref(av), ctypes.byref(bv), ctypes.byref(cv), ob, int(alpha), int(beta),
        ENCODE[encode], int(bool(columns)), _ptr(scratch), _nbytes(scratch), _stream(stream),
        ctypes.byref(r))
    return st, r.as_dict()


def suggested_scratch_collapse(m, k, n):
    return lib().uor_gfx950_suggested_scratch_collapse(m, k, n)


def suggested_scratch_coded_collapse(m, k, n):
    return lib().uor_gfx950_suggested_scratch_coded_collapse(m, k, n)


def gemm_coded_float(a, a_shape, a_strides, table, codes, w_rows, w_cols, transposed, c, c_shape,
                     c_strides, alpha=1, beta=0, encode="nearest", scratch=None, stream=None):
    """A float product with an Arena-coded operand: `table` is a float32 /
    float64 device tensor (the codebook), `codes` uint8 or int16 (u16 codes)."""
    import torch
    is64 = int(a.dtype == torch.float64)
    es = 8 if is64 else 4
    av = view(a, *a_shape, *a_strides, elem=es)
    cv = view(c, *c_shape, *c_strides, elem=es)
    bits = 8 if codes.element_size() == 1 else 16
    table, codes = _dev(table), _dev(codes)
    r = Route()
    st = lib().uor_gfx950_gemm_coded_float(
        is64, ctypes.byref(av), _ptr(table), _len(table, es), bits, _ptr(codes),
        _len(codes, bits // 8), w_rows, w_cols, int(bool(transposed)), ctypes.byref(cv),
        int(alpha), int(beta), ENCODE[encode], _ptr(scratch), _nbytes(scratch), _stream(stream),
        ctypes.byref(r))
    return st, r.as_dict()


def suggested_scratch_coded_float(is64, m, k, n):
    return lib().uor_gfx950_suggested_scratch_coded_float(int(is64), m, k, n)


def manifest_json(tier, bound, rows, cols, block, codebook_sha256, codes_sha256,
                  spec="uor-matmul/1", out_len=512):
    """Manifest::write_canonical_json: (status, text or the length needed)."""
    buf = ctypes.create_string_buffer(max(out_len, 1))
    n = _u64(0)
    st = lib().uor_gfx950_manifest_json(
        TIER.get(tier, tier), bound & ((1 << 64) - 1), bound >> 64, rows, cols, block,
        codebook_sha256.encode(), codes_sha256.encode(), spec.encode(),
        buf if out_len else None, out_len, ctypes.byref(n))
    if st == 0:
        return st, buf.raw[:n.value].decode()
    return st, n.value
