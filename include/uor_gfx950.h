/*
 * uor_gfx950.h -- the C ABI of the MI355X (gfx950) route for the
 * exact-accumulation GEMM hot path of UOR-Foundation/uor-matmul.
 *
 * Every entry point computes exactly what the reference's CPU routes compute,
 * byte for byte: the exact sum, scaled and combined in the accumulator's width,
 * encoded once into the requested output type.
 *
 * Conventions (all entry points):
 *   - Every operand, output and scratch pointer is a DEVICE pointer owned by
 *     the caller.  The library never allocates device or pinned memory on the
 *     call path; `scratch` is an offer of any size, including 0, and changes
 *     only which kernels run, never the bytes written (reference CD-10,
 *     crates/uor-matmul-gemm/src/scratch.rs:50-120).
 *   - Work is enqueued on `stream` (a hipStream_t; NULL is the default
 *     stream) and the call returns without synchronising.  Shape validation
 *     happens on the host before anything is enqueued.
 *   - Strides are in elements and may be negative or zero on inputs, exactly
 *     as the reference's Strides (crates/uor-matmul-core/src/layout.rs:29-154).
 *   - Status: 0 ok; the reference's two NotAProduct variants
 *     (crates/uor-matmul-core/src/error.rs:28-53) as 1 and 2; a buffer that
 *     does not hold the view its caller described (MatView::new -> None,
 *     layout.rs:212; the slice face's does_not_fit panic, slice.rs:104-116)
 *     as 3; an argument outside the enums below as 4; a request beyond the
 *     no-alloc entry's static scratch as 5; a HIP runtime failure as
 *     100 + hipError_t (device-only; the reference has no such state).
 *     Values, depth and magnitude never produce an error (reference CT-01,
 *     CT-05).
 */
#ifndef UOR_GFX950_H
#define UOR_GFX950_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- status */
#define UOR_OK 0
#define UOR_NONCONFORMANT 1          /* NotAProduct::Nonconformant */
#define UOR_OUTPUT_ALIASES_ITSELF 2  /* NotAProduct::OutputAliasesItself */
#define UOR_SHORT_BUFFER 3           /* a view does not fit its buffer */
#define UOR_INVALID_ARGUMENT 4       /* unknown enum value */
#define UOR_SCRATCH_LIMIT 5          /* uor_gfx950_gemm_i8_noalloc: the call needs more
                                        scratch than UOR_NOALLOC_SCRATCH_BYTES */
#define UOR_HIP_ERROR 100            /* + hipError_t */

/* EncodeMode, crates/uor-matmul-core/src/policy.rs:19-43.  The slice face
 * always uses UOR_ENCODE_NEAREST (GemmOptions::default()). */
#define UOR_ENCODE_NEAREST 0
#define UOR_ENCODE_TOWARD_ZERO 1
#define UOR_ENCODE_SATURATING 2
#define UOR_ENCODE_WRAPPING 3

/* Integer output element type O, named by its width in bytes
 * (EncodeFrom<i128> for i8, i16, i32, i64, i128: acc.rs:115-123).  An i128
 * output is 16 bytes, little-endian two's complement. */
#define UOR_OUT_I8 1
#define UOR_OUT_I16 2
#define UOR_OUT_I32 4
#define UOR_OUT_I64 8
#define UOR_OUT_I128 16

/* A strided matrix view over a device buffer: the reference's
 * MatView::new(data[..len], rows, cols, Strides{rs, cs}) (layout.rs:212) and
 * MatViewMut::new (layout.rs:384).  `data` is the START of the buffer, not
 * element (0,0): the view's origin is placed so that the lowest offset it
 * reaches is element 0, which is how a negative stride walks backwards
 * through the buffer rather than reading before it. */
typedef struct uor_view {
    void *data;
    uint64_t len; /* buffer length, in elements */
    uint64_t rows;
    uint64_t cols;
    int64_t rs; /* elements between consecutive rows */
    int64_t cs; /* elements between consecutive columns */
} uor_view;

/* Which kernels ran: the analogue of the reference's RouteCensus
 * (crates/uor-matmul-gemm/src/kernel.rs:419-484), which observes the route
 * without changing it.  May be NULL. */
#define UOR_ROUTE_NONE 0          /* m == 0 or n == 0: nothing to write */
#define UOR_ROUTE_EPILOGUE_ONLY 1 /* k == 0: C := enc(beta * C) */
#define UOR_ROUTE_MFMA_TILE 2     /* int8 MFMA tile, fused epilogue */
#define UOR_ROUTE_MFMA_SPLITK 3   /* int8 MFMA split-K, exact i64 partials */
#define UOR_ROUTE_MFMA_WIDE 4     /* int8 MFMA, i64 register widening */
#define UOR_ROUTE_COLLAPSED 5     /* one product line per distinct line of A (or column of B) */
#define UOR_ROUTE_LUT4_DOT4 10    /* 4-bit table-lookup, v_perm decode, dot4 (small m) */
#define UOR_ROUTE_LUT4_MFMA 11    /* 4-bit table-lookup, v_perm decode into int8 MFMA */
#define UOR_ROUTE_LUT4_PREFILL 12 /* 4-bit table-lookup, many rows: decode W^T, dense int8 MFMA */
#define UOR_ROUTE_CODED_DENSE 13  /* any fixed-width codec: decode W into scratch, dense int8 route */
#define UOR_ROUTE_CODED_DIRECT 14 /* any fixed-width codec, no offer: per-cell decode and sum */
#define UOR_ROUTE_CODED_GEMV 15   /* any fixed-width codec, W n x k, m <= 8: decode in registers, one wave per column */
#define UOR_ROUTE_FLOAT_CRT 20    /* exact float: int8 residue MFMA + CRT */
#define UOR_ROUTE_FLOAT_DIRECT 21 /* exact float: per-cell exact register */
#define UOR_ROUTE_TROP_VALU 30    /* max-plus, packed i16 VALU */
#define UOR_ROUTE_TROP_SELECTED 31        /* max-plus + witness, (value, index) keys, VALU */
#define UOR_ROUTE_TROP_SELECTED_DIRECT 32 /* max-plus + witness, per-cell loop (k > 2^21) */
#define UOR_ROUTE_INT_CRT 40      /* i16/i32/i64 elements: int8 residue MFMA + CRT */
#define UOR_ROUTE_INT_DIRECT 41   /* i16/i32/i64 elements: per-cell exact loop */
#define UOR_ROUTE_INT_LIMB 42     /* i16/i32 elements: int8 limb planes on the dense int8 route */
typedef struct uor_route {
    int32_t kind;
    int32_t tile_m, tile_n, tile_k;
    int32_t split_k;
    int32_t launches;
    int32_t operand_modes; /* bit 0..1 A load mode, 2..3 B load mode */
    int32_t moduli;        /* float CRT route: residue moduli used */
    uint64_t scratch_used; /* bytes of the offer used */
} uor_route;

/* Returns a static string naming a status code. */
const char *uor_gfx950_status_string(int status);

/* ===================================================== integer (i8 x i8) */

/*
 * View API: gemm(&mut Triple, &Linear{alpha,beta}, GemmOptions{encode}, &mut
 * Scratch) at E = i8 (crates/uor-matmul-gemm/src/kernel.rs:523 gemm_auto,
 * re-exported as uor_matmul::gemm, crates/uor-matmul/src/lib.rs:135), with
 * Triple::new's checks (layout.rs:534-575).
 *
 *   C := enc(alpha * sum_p A[i,p]*B[p,j] + beta * C[i,j])
 *
 * The sum is exact at any depth.  alpha scales it with i128 saturating_mul,
 * beta*C is added with a wrapping i128 add, and the result is encoded once
 * (Linear::finish, epilogue.rs:67-95; ScaleExact for i128, epilogue.rs:280-289;
 * encode_i128_into, acc.rs:128-150).  beta == 0 never reads C (CS-04).
 * a, b: int8 views; c: a view of `out_type` elements.
 */
int uor_gfx950_gemm_i8(const uor_view *a, const uor_view *b, const uor_view *c,
                       int out_type, int64_t alpha, int64_t beta, int encode,
                       void *scratch, uint64_t scratch_bytes, void *stream,
                       uor_route *route);

/*
 * slice::gemm_ex::<i8, O> (crates/uor-matmul/src/slice.rs:144-178): row-major
 * with leading dimensions, lengths in elements, encode Nearest.  `scratch` is
 * a device buffer offer of `scratch_bytes` bytes.
 */
int uor_gfx950_slice_gemm_ex_i8(uint64_t m, uint64_t k, uint64_t n, int64_t alpha,
                                const int8_t *a, uint64_t a_len, uint64_t lda,
                                const int8_t *b, uint64_t b_len, uint64_t ldb,
                                int64_t beta, void *c, uint64_t c_len, uint64_t ldc,
                                int out_type, void *scratch, uint64_t scratch_bytes,
                                void *stream);

/* slice::gemm::<i8, O> (slice.rs:184-199): gemm_ex(m,k,n,1,a,k,b,n,0,c,n). */
int uor_gfx950_slice_gemm_i8(uint64_t m, uint64_t k, uint64_t n,
                             const int8_t *a, uint64_t a_len,
                             const int8_t *b, uint64_t b_len,
                             void *c, uint64_t c_len, int out_type,
                             void *scratch, uint64_t scratch_bytes, void *stream);

/*
 * The device-route offer that lets every gemm_i8 shape take its fastest route
 * (split-K partial sums).  Replaces suggested_scratch / suggested_accumulators
 * (crates/uor-matmul-gemm/src/scratch.rs:183-240) for this backend: the
 * reference's figure sizes CPU panels, which this route does not use.
 */
uint64_t uor_gfx950_suggested_scratch_i8(uint64_t m, uint64_t k, uint64_t n);

/*
 * uor_gfx950_gemm_i8 without a scratch offer and without any allocation: no
 * counterpart in the reference.  It is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The scratch is a static device array of
 * UOR_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends; a call
 * whose fastest route needs more (the split-K partial sums, m*n*8 bytes, taken
 * when k > 65536 or the output is small at k >= 8192) returns
 * UOR_SCRATCH_LIMIT.  Same bytes as uor_gfx950_gemm_i8.  Calls that overlap on
 * one GPU share its array and race: order them on one stream.  The first call
 * on a device looks the array's device address up (hipGetSymbolAddress).
 */
#define UOR_NOALLOC_SCRATCH_BYTES (16u << 20)
int uor_gfx950_gemm_i8_noalloc(const uor_view *a, const uor_view *b, const uor_view *c,
                               int out_type, int64_t alpha, int64_t beta, int encode,
                               void *stream, uor_route *route);

/*
 * The view API at E = i16, i32, i64 (elem_bytes 2, 4, 8; 1 forwards to
 * uor_gfx950_gemm_i8): the reference's Kernelized integer families
 * (crates/uor-matmul-gemm/src/kernel.rs:132-399, gemm_auto kernel.rs:523),
 * AccOf = i128 for i16/i32 and Limbs<3> for i64 (alphabet.rs:559-616,
 * acc.rs:215), Linear::finish and encode_i128_into / impl_encode_from_limbs
 * (epilogue.rs:67-95, acc.rs:128-150, 405-442).  The sum is exact at any
 * depth.  i64 elements scale and add in Limbs<3>'s 192-bit register, mod
 * 2^192 (ScaleExact for Limbs, epilogue.rs:307-328).  a, b: views of
 * elem_bytes-byte integers; c: a view
 * of `out_type` elements.  With an offer of uor_gfx950_suggested_scratch_int
 * bytes the int8 residue route runs; with none, a per-cell loop.
 */
int uor_gfx950_gemm_int(int elem_bytes, const uor_view *a, const uor_view *b,
                        const uor_view *c, int out_type, int64_t alpha, int64_t beta,
                        int encode, void *scratch, uint64_t scratch_bytes, void *stream,
                        uor_route *route);

/* The offer that lets gemm_int take the residue route at this shape. */
uint64_t uor_gfx950_suggested_scratch_int(int elem_bytes, uint64_t m, uint64_t k, uint64_t n);

/* ============================================ 4-bit table-lookup GEMM */

/*
 * gemm_tabulated over a TabulatedTriple (crates/uor-matmul-gemm/src/
 * tabulated.rs:607-658, 2555) with W a CodedMatrix<Packed<Grid<i8,16>,2>>
 * (crates/uor-matmul-codec/src/codecs.rs:80-259, matrix.rs:36-75):
 *
 *   C[i,j] := enc(alpha * sum_p A[i,p] * book_g(j)[code(j,p)] + beta * C[i,j])
 *
 * A: m x k int8 view.  codes: n x k/2 bytes, row-major contiguous (one coded
 * row per output column, k-major); byte q of row j holds k-position 2q in its
 * LOW nibble and 2q+1 in its high nibble (CK-03).  k must be even and
 * codes_len == n*k/2 (CodedMatrix::new), else status 3.
 * books: ceil(n/group) codebooks of 16 int8 entries; coded row j decodes
 * through book j/group.  The reference spells one codebook per CodedMatrix, so
 * a per-group codebook is ceil(n/group) reference calls over 128-row
 * CodedMatrix slices and MatViewMut column windows of C; group == n is one.
 * c: m x n view of `out_type` elements.  Epilogue and encode as gemm_i8.
 * For m >= 128 (m >= 80 at k >= 4096), an offer of
 * uor_gfx950_suggested_scratch_lut4 bytes decodes
 * W^T once into it and runs the dense int8 route (the reference's
 * decode-then-multiply spelling of the same value, coded.rs:98-140, CD-13);
 * any smaller offer, the table-lookup kernels.  The bytes are the same.
 */
int uor_gfx950_gemm_lut4(const uor_view *a, const uint8_t *codes, uint64_t codes_len,
                         uint64_t n, const int8_t *books, uint64_t books_len,
                         uint64_t group, const uor_view *c, int out_type,
                         int64_t alpha, int64_t beta, int encode, void *scratch,
                         uint64_t scratch_bytes, void *stream, uor_route *route);

/* The offer that lets gemm_lut4 take the decode-then-dense route (0 below m = 128). */
uint64_t uor_gfx950_suggested_scratch_lut4(uint64_t m, uint64_t k, uint64_t n);

/* ======================================== coded operands, any fixed-width tier */

/* Codec tiers over the i8 alphabet (crates/uor-matmul-codec/src/codecs.rs). */
#define UOR_TIER_IDENTITY 0 /* code = the value (int8)                     :42-57   */
#define UOR_TIER_GRID 1     /* table[code % entries], u16 codes            :80-104  */
#define UOR_TIER_BOOK 2     /* table[(code % entries) * block + i % block]  :268-309 */
#define UOR_TIER_SIGN 3     /* bit i % block of the code: 1 -> +1, else -1  :362-401 */
#define UOR_TIER_TERNARY 4  /* digit i % block: 0 -> -1, 2 -> +1, 1/3 -> 0  :466-517 */
/* Tiers that only name a manifest here (TierId, tier.rs:265-278): the
 * composing tiers of a uor_codec (Packed, Offset) and those with no GPU
 * descriptor (Runs, Transcode) or a float one (Arena). */
#define UOR_TIER_PACKED 5
#define UOR_TIER_OFFSET 6
#define UOR_TIER_RUNS 7
#define UOR_TIER_TRANSCODE 8
#define UOR_TIER_ARENA 9

/*
 * A constructed codec (Codec<i8, Bd>, codecs.rs), as the GPU reads it:
 *
 *   base tier   tier, entries (N), block (BLK), code_bits (the code type K:
 *               8 for u8, 16 for u16; Identity 8, Grid 16), table (device,
 *               int8: N entries for Grid, N * BLK for Book; NULL otherwise)
 *   packed      P in {1, 2, 4, 8}: Packed<base, P> (codecs.rs:150-200):
 *               stored codes are u8 holding P sub-codes of 8/P bits, the low
 *               sub-code first (CK-03); 0: the base codes are stored as is
 *   has_zero    Offset<.., zero> over the above (codecs.rs:566-620): the
 *               decoded value minus zero, i8 wrapping_sub
 *
 * The codec constructors' own checks (Sign/Ternary/Offset::new bounds) are
 * the caller's; the library checks only what the decode needs.
 */
typedef struct uor_codec {
    int32_t tier;
    int32_t code_bits;
    int32_t packed;
    int32_t has_zero;
    int64_t zero;
    uint64_t entries;
    uint64_t block;
    const int8_t *table;
    uint64_t table_len;
} uor_codec;

/*
 * A product with one coded operand, W a fixed-width CodedMatrix<i8, Bd, C>
 * (crates/uor-matmul-codec/src/matrix.rs:36-75, at :202-207) of w_rows x
 * w_cols over `codec`, its codes row-major (w_rows * w_cols / MAX_BLOCK codes
 * of code_bits / 8 bytes, 1 byte when packed):
 *
 *   transposed = 1: gemm_tabulated over TabulatedTriple (tabulated.rs:
 *                   624-650, 2555): W is n x k, C := enc(alpha * A W^T + beta C)
 *   transposed = 0: coded_gemm over CodedTriple (coded.rs:50-78, 98-140):
 *                   W is k x n, C := enc(alpha * A W + beta C)
 *
 * A: m x k int8 view; c: m x n view of out_type elements; Linear epilogue and
 * encode as gemm_i8.  A codes_len or shape that CodedMatrix::new refuses
 * (MAX_BLOCK = 0, w_cols % MAX_BLOCK != 0, wrong code count) is status 3; then
 * Nonconformant / OutputAliasesItself as the triples report them.  For
 * transposed = 1, m <= 8 and k <= 2^22, the codes are decoded in registers as
 * they are multiplied (no scratch).  Otherwise, with an offer of
 * uor_gfx950_suggested_scratch_coded bytes, W is decoded once into the
 * scratch as a k x n int8 matrix and the dense int8 route runs (the
 * decode-then-multiply spelling of the same value, CD-13); with less, a
 * per-cell loop.  The bytes are the same.
 */
int uor_gfx950_gemm_coded(const uor_view *a, const uor_codec *codec, const void *codes,
                          uint64_t codes_len, uint64_t w_rows, uint64_t w_cols,
                          int transposed, const uor_view *c, int out_type, int64_t alpha,
                          int64_t beta, int encode, void *scratch, uint64_t scratch_bytes,
                          void *stream, uor_route *route);

/* The offer that lets gemm_coded take the decode-then-dense route. */
uint64_t uor_gfx950_suggested_scratch_coded(uint64_t m, uint64_t k, uint64_t n);

/*
 * The same product with the row collapse gemm_tabulated takes as its
 * `collapse` argument (tabulated.rs:2555-2660, collapse.rs:71-120): with
 * beta = 0 and an offer of uor_gfx950_suggested_scratch_coded_collapse
 * bytes, equal rows of A share one product row (the pass reads back the
 * distinct count: a stream synchronisation; route->kind is
 * UOR_ROUTE_COLLAPSED and route->moduli the count).  Otherwise, or when
 * every row is distinct, it is uor_gfx950_gemm_coded.  The bytes are the
 * same (CD-15).
 */
int uor_gfx950_gemm_coded_collapsed(const uor_view *a, const uor_codec *codec,
                                    const void *codes, uint64_t codes_len, uint64_t w_rows,
                                    uint64_t w_cols, int transposed, const uor_view *c,
                                    int out_type, int64_t alpha, int64_t beta, int encode,
                                    void *scratch, uint64_t scratch_bytes, void *stream,
                                    uor_route *route);

/* The offer that lets gemm_coded_collapsed collapse. */
uint64_t uor_gfx950_suggested_scratch_coded_collapse(uint64_t m, uint64_t k, uint64_t n);

/*
 * A float product with an Arena-coded operand (Arena<f32|f64, N, u8|u16>,
 * crates/uor-matmul-codec/src/codecs.rs:894-960, CK-14): element (r, q) of
 * the w_rows x w_cols coded matrix is table[code(r, q) % entries], the codes
 * row-major, one per element (MAX_BLOCK 1).  transposed = 1: W is n x k
 * (C := A W^T); 0: W is k x n.  a, c: views of f32 (is_f64 = 0) or f64;
 * table: `entries` device values of that type.  The operand is decoded once
 * into the scratch, then multiplied by uor_gfx950_gemm_float (exact, one
 * rounding), so the bytes are those of the dense spelling's product.  There
 * is no decode-free route: an offer below the decoded operand's k*n*size
 * bytes is UOR_INVALID_ARGUMENT; uor_gfx950_suggested_scratch_coded_float
 * adds the float route's own offer.
 */
int uor_gfx950_gemm_coded_float(int is_f64, const uor_view *a, const void *table,
                                uint64_t entries, int code_bits, const void *codes,
                                uint64_t codes_len, uint64_t w_rows, uint64_t w_cols,
                                int transposed, const uor_view *c, int64_t alpha, int64_t beta,
                                int encode, void *scratch, uint64_t scratch_bytes, void *stream,
                                uor_route *route);

uint64_t uor_gfx950_suggested_scratch_coded_float(int is_f64, uint64_t m, uint64_t k, uint64_t n);

/* =================================================== exact float GEMM */

/*
 * gemm_float_packed through the view API (crates/uor-matmul-gemm/src/
 * float.rs:1824-1855), E = O = f32 (is_f64 = 0) or f64 (is_f64 = 1):
 *
 *   C := round_once(alpha * sum_p A[i,p]*B[p,j] + beta * C[i,j])
 *
 * computed exactly (Element::mac for floats, crates/uor-matmul-core/src/
 * alphabet.rs:856-902; Complete::scale, acc.rs:1028; Linear::finish) and
 * rounded once by the float encode (acc.rs:1734-1868): Nearest is
 * round-half-even with overflow to +-inf; the other modes truncate toward
 * zero and clamp to +-MAX.  An exact zero gives +0; NaN anywhere, inf*0 or
 * +inf with -inf give the canonical NaN.  alpha and beta are exact int64.
 */
int uor_gfx950_gemm_float(int is_f64, const uor_view *a, const uor_view *b,
                          const uor_view *c, int64_t alpha, int64_t beta, int encode,
                          void *scratch, uint64_t scratch_bytes, void *stream,
                          uor_route *route);

/* slice::gemm_float_ex (crates/uor-matmul/src/slice.rs:304-340), encode
 * Nearest, row-major with leading dimensions. */
int uor_gfx950_slice_gemm_float_ex(int is_f64, uint64_t m, uint64_t k, uint64_t n,
                                   int64_t alpha, const void *a, uint64_t a_len,
                                   uint64_t lda, const void *b, uint64_t b_len,
                                   uint64_t ldb, int64_t beta, void *c, uint64_t c_len,
                                   uint64_t ldc, void *scratch, uint64_t scratch_bytes,
                                   void *stream);

/* slice::gemm_float (slice.rs:405-421): gemm_float_ex(m,k,n,1,a,k,b,n,0,c,n).
 *
 * The reference's _full spellings take their working memory as several
 * offers: gemm_float_ex_full / gemm_float_full (slice.rs:357-398, :428-465)
 * as pa, pb, scaled, panels and accumulators, gemm_ex_full / gemm_full
 * (slice.rs:221-279) as panels and accumulators.  Here they are the same call
 * with ONE device offer: bind them to uor_gfx950_slice_gemm_float_ex /
 * _float / uor_gfx950_slice_gemm_ex_i8 / _i8 with a single buffer of at most
 * the offers' summed bytes.  As in the reference (CD-04, CD-10, CD-19) the
 * bytes written to C are the same at every offer, empty included; the offer
 * only selects the route, never the result. */
int uor_gfx950_slice_gemm_float(int is_f64, uint64_t m, uint64_t k, uint64_t n,
                                const void *a, uint64_t a_len, const void *b, uint64_t b_len,
                                void *c, uint64_t c_len, void *scratch, uint64_t scratch_bytes,
                                void *stream);

/*
 * raw::sgemm / raw::dgemm (crates/uor-matmul/src/raw.rs:45-90, raw_gemm
 * :98-158): matrixmultiply's signature.  a, b, c point at element (0,0);
 * strides may be negative.  Like the reference, an invalid request is a silent
 * no-op (status 0, nothing enqueued); a HIP failure still reports 100+.
 */
int uor_gfx950_sgemm(uint64_t m, uint64_t k, uint64_t n, int64_t alpha,
                     const float *a, int64_t rsa, int64_t csa,
                     const float *b, int64_t rsb, int64_t csb, int64_t beta,
                     float *c, int64_t rsc, int64_t csc, void *scratch,
                     uint64_t scratch_bytes, void *stream);
int uor_gfx950_dgemm(uint64_t m, uint64_t k, uint64_t n, int64_t alpha,
                     const double *a, int64_t rsa, int64_t csa,
                     const double *b, int64_t rsb, int64_t csb, int64_t beta,
                     double *c, int64_t rsc, int64_t csc, void *scratch,
                     uint64_t scratch_bytes, void *stream);

/* The offer that lets gemm_float take its fastest route at this shape
 * (replaces suggested_float_panels, float.rs:1876-1882, for this backend). */
uint64_t uor_gfx950_suggested_scratch_float(int is_f64, uint64_t m, uint64_t k,
                                            uint64_t n);

/*
 * gemm_collapsed(&mut Triple, &Linear{alpha,beta}, GemmOptions{encode},
 * &mut Scratch, &mut Collapse) at E = i8 (crates/uor-matmul-gemm/src/
 * collapse.rs:169-220): the bytes of uor_gfx950_gemm_i8, computing one
 * output row per distinct row of A (columns = 1: one output column per
 * distinct column of B, the transposed triple).  beta != 0 (the epilogue
 * reads C), k = 0, pairwise distinct lines, or an offer smaller than
 * uor_gfx950_suggested_scratch_collapse bytes run the plain route.  The
 * route reads back the distinct count (one 4-byte copy, a stream
 * synchronisation) before the product; route->moduli reports it.
 */
int uor_gfx950_gemm_collapsed_i8(const uor_view *a, const uor_view *b, const uor_view *c,
                                 int out_type, int64_t alpha, int64_t beta, int encode,
                                 int columns, void *scratch, uint64_t scratch_bytes,
                                 void *stream, uor_route *route);

/* The offer that lets gemm_collapsed_i8 collapse (suggested_collapse_index
 * plus suggested_collapse_rows, collapse.rs:103-120, and the product's). */
uint64_t uor_gfx950_suggested_scratch_collapse(uint64_t m, uint64_t k, uint64_t n);

/*
 * Manifest::write_canonical_json (crates/uor-matmul-codec/src/kappa.rs:
 * 321-360, CK-08): the canonical manifest of a coded artifact -- block,
 * bound (a u128 as two halves), both digests, cols, rows, spec, tier, keys in
 * that order -- into out[0..out_len).  *written gets the length (or, with
 * UOR_SHORT_BUFFER, the length needed: BufferTooSmall).  A digest that is not
 * `sha256:` + 64 lowercase hex, or an unknown tier, is UOR_INVALID_ARGUMENT
 * (MalformedDigest).  Host code: no device, no stream.
 */
int uor_gfx950_manifest_json(int tier, uint64_t bound_lo, uint64_t bound_hi, uint64_t rows,
                             uint64_t cols, uint64_t block, const char *codebook_sha256,
                             const char *codes_sha256, const char *spec, char *out,
                             uint64_t out_len, uint64_t *written);

/* ================================================ (max, +) over Trop<i8> */

/*
 * gemm(&mut Triple, &MaxPlus{alpha,beta}, GemmOptions{encode}, ..) at
 * E = Trop<i8>, O = Trop<out> (the reference traversal driver::gemm,
 * crates/uor-matmul-gemm/src/driver.rs:67-182, the public route for Trop):
 *
 *   C[i,j] := enc((alpha (x) max_p (A[i,p] + B[p,j])) (+) (beta (x) C[i,j]))
 *
 * over finite pairs only; -inf absorbs (tropical.rs:311-318).
 * a, b: views of 2-byte Trop<i8> records {int8 value; uint8 finite}
 * (#[repr(C)], tropical.rs:63-70).  c: view of Trop<O> records {O value;
 * uint8 finite; padding}, O = out_type in {1,2,4,8} bytes, record size
 * 2*out_type.  Finite values encode through [O::MIN+1, O::MAX-1]
 * (tropical.rs:336-350); -inf writes {0, 0}.  alpha/beta are Trop<i64>
 * (value, finite); beta = -inf never reads C (CS-11).
 */
int uor_gfx950_gemm_trop_i8(const uor_view *a, const uor_view *b, const uor_view *c,
                            int out_type, int64_t alpha, int alpha_finite,
                            int64_t beta, int beta_finite, int encode,
                            void *scratch, uint64_t scratch_bytes, void *stream,
                            uor_route *route);

/* Witness mechanisms (uor_matmul_gemm::Witness, selection.rs:45-56); both
 * give identical bytes (CD-25): the least index attaining the maximum. */
#define UOR_WITNESS_LEXICOGRAPHIC 0
#define UOR_WITNESS_COMPARE_PASS 1

/*
 * gemm_selected(&mut SelectedTriple, &MaxPlus{alpha,beta}, GemmOptions{encode},
 * mechanism, ..) at E = Trop<i8>, O = Trop<out>
 * (crates/uor-matmul-gemm/src/selection.rs:212-320): C as
 * uor_gfx950_gemm_trop_i8 writes it, and
 *
 *   W[i,j] := the least p with A[i,p] + B[p,j] equal to the maximum
 *
 * over the same terms, a term touching -inf counting as -inf (so a cell whose
 * every term is -inf has witness 0), and 0 at k == 0 (selection.rs:264-268).
 * w: view of uint64 elements (usize on a 64-bit target), 8-byte aligned.
 * Status order: the a, b, c checks of uor_gfx950_gemm_trop_i8, then the
 * witness (SelectedTriple::new, selection.rs:76-98): SHORT_BUFFER,
 * NONCONFORMANT when it is not m x n, OUTPUT_ALIASES_ITSELF.
 */
int uor_gfx950_gemm_trop_i8_selected(const uor_view *a, const uor_view *b,
                                     const uor_view *c, const uor_view *w,
                                     int out_type, int64_t alpha, int alpha_finite,
                                     int64_t beta, int beta_finite, int encode,
                                     int mechanism, void *scratch,
                                     uint64_t scratch_bytes, void *stream,
                                     uor_route *route);

/* ========================================= partition of the output (S12) */

/* One independently computable block of C (partition.rs:16-27 Tile). */
typedef struct uor_tile {
    uint64_t row, col;   /* first row and column of C */
    uint64_t rows, cols; /* extent, clipped at C's last row and column */
} uor_tile;

/* Partition::new + len (crates/uor-matmul-gemm/src/partition.rs:44-66): the
 * number of tiles of at most tile_rows x tile_cols covering an m x n output;
 * a zero tile extent means the whole extent.  0 exactly when m or n is 0;
 * UINT64_MAX when the count does not fit 64 bits. */
uint64_t uor_gfx950_partition_len(uint64_t m, uint64_t n, uint64_t tile_rows,
                                  uint64_t tile_cols);

/* Partition::tile (partition.rs:83-98): tile `index` in the stable row-major
 * tile order.  Returns 1 and fills *out, or 0 (None) when index >= len. */
int uor_gfx950_partition_tile(uint64_t m, uint64_t n, uint64_t tile_rows,
                              uint64_t tile_cols, uint64_t index, uor_tile *out);

/* MatView::subview (crates/uor-matmul-core/src/layout.rs:633-646): the
 * rows x cols block of *v at (i, j), as a view of its own into the same
 * buffer (same strides; data and len narrowed to the block's window).
 * UOR_INVALID_ARGUMENT where the reference returns None (the block reaches
 * outside the view), UOR_SHORT_BUFFER when *v itself does not fit. */
int uor_gfx950_subview(const uor_view *v, int elem_bytes, uint64_t i, uint64_t j,
                       uint64_t rows, uint64_t cols, uor_view *out);

/*
 * The partition driven on streams (the caller-side executor the reference
 * leaves to rayon and the like, partition.rs:1-11): tile t runs as its own
 * uor_gfx950_gemm_i8 / _gemm_float over the sub-views A[row.., :],
 * B[:, col..], C[row.., col..] on streams[t % nstreams] (nstreams 0: the null
 * stream).  The offer is split into nstreams equal 256-aligned shares, one
 * per stream.  The bytes of C equal the single call's for every tile shape and
 * stream count (CD-02): the tiles are disjoint and each cell is one exact sum.
 * The whole call is checked as the single call checks it before any tile is
 * enqueued; *tiles_run (may be NULL) counts the tiles enqueued.  The caller
 * orders the streams after its own work on A, B and C and joins them after;
 * streams must have the default priority.
 */
int uor_gfx950_gemm_i8_tiled(const uor_view *a, const uor_view *b, const uor_view *c,
                             int out_type, int64_t alpha, int64_t beta, int encode,
                             uint64_t tile_rows, uint64_t tile_cols, void *const *streams,
                             uint32_t nstreams, void *scratch, uint64_t scratch_bytes,
                             uint64_t *tiles_run);
int uor_gfx950_gemm_float_tiled(int is_f64, const uor_view *a, const uor_view *b,
                                const uor_view *c, int64_t alpha, int64_t beta, int encode,
                                uint64_t tile_rows, uint64_t tile_cols, void *const *streams,
                                uint32_t nstreams, void *scratch, uint64_t scratch_bytes,
                                uint64_t *tiles_run);

#ifdef __cplusplus
}
#endif

#endif /* UOR_GFX950_H */
