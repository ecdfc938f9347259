// Caller-driven partition of the output (crates/uor-matmul-gemm/src/
// partition.rs:34-110) and the executor that drives it on HIP streams.
//
// The reference declares the tiles and leaves the running to the caller's
// executor.  On one MI355X the executor is a set of streams: tile t of the
// partition is enqueued on stream t mod S as its own GEMM over the three
// sub-views (layout.rs:633-646 MatView::subview) of A's rows, B's columns and
// C's block.  The tiles write disjoint blocks of C and read only A and B, and
// each output cell is one exact sum, so the bytes are those of the single
// call whatever the tile shape, the stream count or the completion order
// (CD-02, CD-08).

#include "common.hpp"

using namespace uor;

namespace {

uint64_t div_ceil(uint64_t a, uint64_t b) { return a / b + (a % b != 0); }

// Partition::new: a zero tile extent means the whole extent (at least 1).
void tile_extents(uint64_t m, uint64_t n, uint64_t *tr, uint64_t *tc) {
    if (*tr == 0) *tr = m > 1 ? m : 1;
    if (*tc == 0) *tc = n > 1 ? n : 1;
}

// The window [lo, hi] of buffer offsets a rows x cols block with strides
// (rs, cs) anchored at offset `at` reaches; false when it overflows.
bool block_window(int64_t at, uint64_t rows, uint64_t cols, int64_t rs, int64_t cs,
                  int64_t *lo, int64_t *hi) {
    int64_t r, c;
    if (__builtin_mul_overflow((int64_t)(rows - 1), rs, &r)) return false;
    if (__builtin_mul_overflow((int64_t)(cols - 1), cs, &c)) return false;
    int64_t l = at, h = at;
    if (__builtin_add_overflow(l, r < 0 ? r : 0, &l)) return false;
    if (__builtin_add_overflow(l, c < 0 ? c : 0, &l)) return false;
    if (__builtin_add_overflow(h, r > 0 ? r : 0, &h)) return false;
    if (__builtin_add_overflow(h, c > 0 ? c : 0, &h)) return false;
    *lo = l;
    *hi = h;
    return true;
}

// The GEMM each tile runs: the integer (i8) or the exact float family.
enum class Family { I8, F32, F64 };

int run_one(Family f, const uor_view *a, const uor_view *b, const uor_view *c, int out_type,
            int64_t alpha, int64_t beta, int encode, void *scratch, uint64_t scratch_bytes,
            void *stream) {
    if (f == Family::I8)
        return uor_gfx950_gemm_i8(a, b, c, out_type, alpha, beta, encode, scratch, scratch_bytes,
                                  stream, nullptr);
    return uor_gfx950_gemm_float(f == Family::F64, a, b, c, alpha, beta, encode, scratch,
                                 scratch_bytes, stream, nullptr);
}

int run_tiled(Family f, const uor_view *a, const uor_view *b, const uor_view *c, int out_type,
              int64_t alpha, int64_t beta, int encode, uint64_t tile_rows, uint64_t tile_cols,
              void *const *streams, uint32_t nstreams, void *scratch, uint64_t scratch_bytes,
              uint64_t *tiles_run) {
    if (tiles_run) *tiles_run = 0;
    const int ea = f == Family::I8 ? 1 : f == Family::F32 ? 4 : 8;
    const int ec = f == Family::I8 ? out_type : ea;
    if (f == Family::I8 && !valid_out_type(out_type)) return UOR_INVALID_ARGUMENT;
    if (!valid_encode(encode)) return UOR_INVALID_ARGUMENT;
    if (nstreams > 0 && !streams) return UOR_INVALID_ARGUMENT;
    // The whole call is checked as the single GEMM would check it, so a tiled
    // call fails exactly where the untiled one does and before any tile runs.
    Placed A, B, C;
    int st = make_triple(a, ea, b, ea, c, ec, &A, &B, &C);
    if (st) return st;
    const uint64_t m = C.rows, n = C.cols, k = A.cols;
    const uint64_t tiles = uor_gfx950_partition_len(m, n, tile_rows, tile_cols);
    const uint32_t S = nstreams ? nstreams : 1;
    // Each stream owns an equal, 256-byte aligned share of the offer; its
    // tiles run one after another in stream order, so the share is reused.
    uint64_t have = 0;
    char *base = offer_align(scratch, scratch_bytes, &have);
    const uint64_t share = (have / S) & ~(uint64_t)255;
    for (uint64_t t = 0; t < tiles; ++t) {
        uor_tile tile;
        uor_gfx950_partition_tile(m, n, tile_rows, tile_cols, t, &tile);
        uor_view sa, sb, sc;
        if ((st = uor_gfx950_subview(a, ea, tile.row, 0, tile.rows, k, &sa))) return st;
        if ((st = uor_gfx950_subview(b, ea, 0, tile.col, k, tile.cols, &sb))) return st;
        if ((st = uor_gfx950_subview(c, ec, tile.row, tile.col, tile.rows, tile.cols, &sc)))
            return st;
        const uint32_t s = (uint32_t)(t % S);
        void *stream = nstreams ? streams[s] : nullptr;
        st = run_one(f, &sa, &sb, &sc, out_type, alpha, beta, encode,
                     share ? base + (uint64_t)s * share : nullptr, share, stream);
        if (st) return st;
        if (tiles_run) *tiles_run = t + 1;
    }
    return UOR_OK;
}

}  // namespace

// Partition::len (partition.rs:64-66): rows of tiles x columns of tiles;
// zero exactly when the output is empty.
extern "C" uint64_t uor_gfx950_partition_len(uint64_t m, uint64_t n, uint64_t tile_rows,
                                             uint64_t tile_cols) {
    tile_extents(m, n, &tile_rows, &tile_cols);
    uint64_t len;
    if (__builtin_mul_overflow(div_ceil(m, tile_rows), div_ceil(n, tile_cols), &len)) return UINT64_MAX;
    return len;
}

// Partition::tile (partition.rs:83-98): tile `index` in row-major tile order,
// clipped at the last row and column; 0 (None) past the end.
extern "C" int uor_gfx950_partition_tile(uint64_t m, uint64_t n, uint64_t tile_rows,
                                         uint64_t tile_cols, uint64_t index, uor_tile *out) {
    if (!out || index >= uor_gfx950_partition_len(m, n, tile_rows, tile_cols)) return 0;
    tile_extents(m, n, &tile_rows, &tile_cols);
    const uint64_t per_row = div_ceil(n, tile_cols);
    const uint64_t row = index / per_row * tile_rows, col = index % per_row * tile_cols;
    out->row = row;
    out->col = col;
    out->rows = tile_rows < m - row ? tile_rows : m - row;
    out->cols = tile_cols < n - col ? tile_cols : n - col;
    return 1;
}

// MatView::subview (layout.rs:633-646) over a uor_view of elem_bytes-byte
// elements: the block is re-expressed as a view of its own whose buffer
// starts at the lowest offset the block reaches, with the same strides, so
// that placing it anchors element (0, 0) at the block's (i, j).
extern "C" int uor_gfx950_subview(const uor_view *v, int elem_bytes, uint64_t i, uint64_t j,
                                  uint64_t rows, uint64_t cols, uor_view *out) {
    if (!v || !out || elem_bytes <= 0) return UOR_INVALID_ARGUMENT;
    Placed P;
    int st = place(v, elem_bytes, &P);
    if (st) return st;
    uint64_t ie, je;
    if (__builtin_add_overflow(i, rows, &ie) || ie > v->rows) return UOR_INVALID_ARGUMENT;
    if (__builtin_add_overflow(j, cols, &je) || je > v->cols) return UOR_INVALID_ARGUMENT;
    const int64_t origin = (int64_t)(((char *)P.base - (char *)v->data) / elem_bytes);
    *out = uor_view{v->data, 0, rows, cols, v->rs, v->cs};
    if (rows == 0 || cols == 0) return UOR_OK;
    // (i, j) lies inside the placed window, so these cannot overflow.
    const int64_t at = origin + (int64_t)i * v->rs + (int64_t)j * v->cs;
    int64_t lo, hi;
    if (!block_window(at, rows, cols, v->rs, v->cs, &lo, &hi)) return UOR_SHORT_BUFFER;
    out->data = (char *)v->data + lo * (int64_t)elem_bytes;
    out->len = (uint64_t)(hi - lo) + 1;
    return UOR_OK;
}

// The partition run on streams, integer family: uor_gfx950_gemm_i8 per tile.
extern "C" int uor_gfx950_gemm_i8_tiled(const uor_view *a, const uor_view *b, const uor_view *c,
                                        int out_type, int64_t alpha, int64_t beta, int encode,
                                        uint64_t tile_rows, uint64_t tile_cols,
                                        void *const *streams, uint32_t nstreams, void *scratch,
                                        uint64_t scratch_bytes, uint64_t *tiles_run) {
    return run_tiled(Family::I8, a, b, c, out_type, alpha, beta, encode, tile_rows, tile_cols,
                     streams, nstreams, scratch, scratch_bytes, tiles_run);
}

// The partition run on streams, exact float family: uor_gfx950_gemm_float
// per tile.
extern "C" int uor_gfx950_gemm_float_tiled(int is_f64, const uor_view *a, const uor_view *b,
                                           const uor_view *c, int64_t alpha, int64_t beta,
                                           int encode, uint64_t tile_rows, uint64_t tile_cols,
                                           void *const *streams, uint32_t nstreams,
                                           void *scratch, uint64_t scratch_bytes,
                                           uint64_t *tiles_run) {
    return run_tiled(is_f64 ? Family::F64 : Family::F32, a, b, c, 0, alpha, beta, encode,
                     tile_rows, tile_cols, streams, nstreams, scratch, scratch_bytes, tiles_run);
}
