/*
 * uor_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C, single-threaded CPU restatement of the reference library's
 * semantics for the exact-accumulation GEMM hot path
 * (UOR-Foundation/uor-matmul, Rust; cannot be compiled here: no cargo/rustc).
 * It is the checker the GPU route is compared against. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the
 * product library (uor-matmul_amd/) never links, calls or falls back to it.
 *
 * Every function cites the reference file:line it restates
 * (paths relative to the reference repository root).
 *
 * Pinning (how each function is checked independently of this file):
 *   ora_place / ora_self_aliases  -- brute-force enumeration of every
 *       coordinate on small shapes (tests/test_oracle_views.py).
 *   ora_gemm_int                  -- NumPy int64 matmul (exact for i8), the
 *       reference's committed CX-10 fixtures (oracles/numpy, i64 elements,
 *       Wrapping), and the reference's inline known answers (CS-05, CS-06,
 *       CD-05, CT-01, README [19,22,43,50]).
 *   ora_gemm_lut4                 -- decode-then-NumPy-matmul, the CK-03
 *       nibble-order known answer (0x3A -> (2,-5)).
 *   ora_gemm_float                -- an independent exact rational oracle in
 *       Python (fractions.Fraction + a separate integer RNE), IEEE special
 *       cases (NaN, inf*0, +inf + -inf, exact cancellation -> +0, ties to
 *       even, overflow, gradual underflow).
 *   ora_gemm_trop                 -- the reference's committed CX-11 fixtures
 *       (oracles/tropical) and a NumPy broadcast max-plus.
 *   ora_gemm_trop_selected        -- the reference's doc example (1+9 / 9+1
 *       -> witness 0), CT-04/CT-05 cases, brute force with ties.
 *   ora_coded_decode              -- the reference's codec known answers:
 *       CK-03 (0x3A -> 2, -5; 0xE4 -> 0,1,2,3), CK-05 (Book = Identity =
 *       Grid decodes), CK-01 (Offset = c - 8), and the exhaustive
 *       cross-spellings CK-11 (Sign<8> = Packed<Grid<2>,8>) and CK-12
 *       (Ternary<4> = Packed<Grid<4>,4>) over all 256 codes.
 *   Parity unpinned (documented, no independent witness): the i128 epilogue's
 *   saturating_mul-then-wrapping-add behaviour at |alpha*sum| >= 2^127, which
 *   no input of the GPU route can reach (|sum| < 2^63 there).
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef __int128 i128;
typedef unsigned __int128 u128;

/* Status codes: identical numbering to include/uor_gfx950.h. */
enum {
    ORA_OK = 0,
    ORA_NONCONFORMANT = 1,        /* error.rs:33-39 */
    ORA_OUTPUT_ALIASES_ITSELF = 2,/* error.rs:40-52 */
    ORA_SHORT_BUFFER = 3,         /* MatView::new -> None, slice.rs:104-116 */
    ORA_INVALID_ARGUMENT = 4
};

/* EncodeMode, policy.rs:19-43. */
enum { ENC_NEAREST = 0, ENC_TOWARD_ZERO = 1, ENC_SATURATING = 2, ENC_WRAPPING = 3 };

/* ------------------------------------------------------------------------ */
/* Views: Strides::extent (layout.rs:69-98), place (layout.rs:161-182),     */
/* Strides::self_aliases (layout.rs:116-143), Triple::new (layout.rs:534).  */
/* ------------------------------------------------------------------------ */

static int extent(int64_t rs, int64_t cs, uint64_t rows, uint64_t cols,
                  int64_t *lo, int64_t *hi) {
    if (rows == 0 || cols == 0) { *lo = 0; *hi = 0; return 1; }
    int64_t last_r = (int64_t)(rows - 1);
    int64_t last_c = (int64_t)(cols - 1);
    int64_t r, c;
    if (__builtin_mul_overflow(last_r, rs, &r)) return 0;
    if (__builtin_mul_overflow(last_c, cs, &c)) return 0;
    int64_t r_lo = rs < 0 ? r : 0, r_hi = rs < 0 ? 0 : r;
    int64_t c_lo = cs < 0 ? c : 0, c_hi = cs < 0 ? 0 : c;
    if (__builtin_add_overflow(r_lo, c_lo, lo)) return 0;
    if (__builtin_add_overflow(r_hi, c_hi, hi)) return 0;
    return 1;
}

/* Returns 1 and the origin when an rows x cols view with these strides fits
 * in len elements; 0 when no such view exists. layout.rs:161-182. */
int ora_place(uint64_t len, uint64_t rows, uint64_t cols, int64_t rs, int64_t cs,
              uint64_t *origin) {
    if (rows == 0 || cols == 0) { *origin = 0; return 1; }
    int64_t lo, hi;
    if (!extent(rs, cs, rows, cols, &lo, &hi)) return 0;
    if (lo > 0) return 0;
    uint64_t o = (uint64_t)0 - (uint64_t)lo; /* unsigned_abs */
    uint64_t h = hi < 0 ? (uint64_t)0 - (uint64_t)hi : (uint64_t)hi;
    uint64_t top;
    if (__builtin_add_overflow(o, h, &top)) return 0;
    if (top < len) { *origin = o; return 1; }
    return 0;
}

static uint64_t gcd_u64(uint64_t a, uint64_t b) {
    while (b) { uint64_t t = a % b; a = b; b = t; }
    return a;
}

/* layout.rs:116-143 */
int ora_self_aliases(uint64_t rows, uint64_t cols, int64_t rs, int64_t cs) {
    if (rows == 0 || cols == 0) return 0;
    if (rows <= 1 && cols <= 1) return 0;
    if (rows > 1 && rs == 0) return 1;
    if (cols > 1 && cs == 0) return 1;
    if (rows <= 1 || cols <= 1) return 0;
    uint64_t a = rs < 0 ? (uint64_t)0 - (uint64_t)rs : (uint64_t)rs;
    uint64_t b = cs < 0 ? (uint64_t)0 - (uint64_t)cs : (uint64_t)cs;
    uint64_t g = gcd_u64(a, b);
    return (b / g) < rows && (a / g) < cols;
}

typedef struct {
    const void *data;
    uint64_t len, rows, cols;
    int64_t rs, cs;
    uint64_t origin;
} view_t;

/* MatView::new for the three operands, then Triple::new's two checks, in the
 * reference's order (slice.rs:164-170, layout.rs:534-575). */
static int make_triple(view_t *a, view_t *b, view_t *c) {
    if (!ora_place(a->len, a->rows, a->cols, a->rs, a->cs, &a->origin)) return ORA_SHORT_BUFFER;
    if (!ora_place(b->len, b->rows, b->cols, b->rs, b->cs, &b->origin)) return ORA_SHORT_BUFFER;
    if (!ora_place(c->len, c->rows, c->cols, c->rs, c->cs, &c->origin)) return ORA_SHORT_BUFFER;
    if (a->cols != b->rows) return ORA_NONCONFORMANT;
    if (c->rows != a->rows || c->cols != b->cols) return ORA_NONCONFORMANT;
    if (ora_self_aliases(c->rows, c->cols, c->rs, c->cs)) return ORA_OUTPUT_ALIASES_ITSELF;
    return ORA_OK;
}

static inline uint64_t at(const view_t *v, uint64_t i, uint64_t j) {
    /* Strides::offset wraps (layout.rs:53-57); origin+offset is in bounds by
     * construction. */
    return v->origin + (uint64_t)((int64_t)i * v->rs + (int64_t)j * v->cs);
}

/* ------------------------------------------------------------------------ */
/* Integer encode and the Linear epilogue.                                  */
/* ------------------------------------------------------------------------ */

static const i128 I128_MAX = (i128)(((u128)1 << 127) - 1);
static const i128 I128_MIN = (i128)((u128)1 << 127);

/* acc.rs:128-150 encode_i128_into */
static i128 encode_i128_into(i128 acc, i128 min, i128 max, int mode) {
    if (mode == ENC_WRAPPING) {
        if (min == I128_MIN && max == I128_MAX) return acc;
        u128 span = (u128)max - (u128)min + 1;
        u128 offset = (u128)acc - (u128)min;
        return (i128)((offset % span) + (u128)min);
    }
    if (acc < min) return min;
    if (acc > max) return max;
    return acc;
}

/* i128::saturating_mul, epilogue.rs:280-283 (ScaleExact for i128). */
static i128 sat_mul_i128(i128 x, int64_t f) {
    i128 r;
    if (__builtin_mul_overflow(x, (i128)f, &r))
        return ((x < 0) != (f < 0)) ? I128_MIN : I128_MAX;
    return r;
}

static void int_range(int out_bytes, i128 *min, i128 *max) {
    switch (out_bytes) {
    case 1: *min = INT8_MIN; *max = INT8_MAX; break;
    case 2: *min = INT16_MIN; *max = INT16_MAX; break;
    case 4: *min = INT32_MIN; *max = INT32_MAX; break;
    case 8: *min = INT64_MIN; *max = INT64_MAX; break;
    default: *min = I128_MIN; *max = I128_MAX; break;
    }
}

static i128 load_int(const void *p, uint64_t idx, int bytes) {
    switch (bytes) {
    case 1: return ((const int8_t *)p)[idx];
    case 2: return ((const int16_t *)p)[idx];
    case 4: return ((const int32_t *)p)[idx];
    case 8: return ((const int64_t *)p)[idx];
    default: { i128 v; memcpy(&v, (const char *)p + idx * 16, 16); return v; }
    }
}

static void store_int(void *p, uint64_t idx, int bytes, i128 v) {
    switch (bytes) {
    case 1: ((int8_t *)p)[idx] = (int8_t)v; break;
    case 2: ((int16_t *)p)[idx] = (int16_t)v; break;
    case 4: ((int32_t *)p)[idx] = (int32_t)v; break;
    case 8: ((int64_t *)p)[idx] = (int64_t)v; break;
    default: memcpy((char *)p + idx * 16, &v, 16); break;
    }
}

/* Linear::finish for the i128 accumulator (epilogue.rs:67-95):
 *   scaled = sat_mul(acc, alpha);
 *   total  = beta == 0 ? scaled : scaled + sat_mul(C, beta)   (wrapping add,
 *            acc.rs:101-105 in a release build, Cargo.toml overflow-checks=false)
 *   encode_i128_into(total, O::MIN, O::MAX, mode). */
static i128 linear_finish_i128(i128 acc, int has_prior, i128 prior, int64_t alpha,
                               int64_t beta, int out_bytes, int mode) {
    i128 total = sat_mul_i128(acc, alpha);
    if (has_prior && beta != 0)
        total = (i128)((u128)total + (u128)sat_mul_i128(prior, beta));
    i128 mn, mx;
    int_range(out_bytes, &mn, &mx);
    return encode_i128_into(total, mn, mx, mode);
}

/* 192-bit two's complement accumulator for i64 elements (Limbs<3>,
 * acc.rs:215, generated.rs:86-111). */
typedef struct { uint64_t w[3]; } l192;

static void l192_add_i128(l192 *x, i128 v) {
    u128 lo = (u128)x->w[0] + (uint64_t)(u128)v;
    x->w[0] = (uint64_t)lo;
    u128 mid = (u128)x->w[1] + (uint64_t)((u128)v >> 64) + (uint64_t)(lo >> 64);
    x->w[1] = (uint64_t)mid;
    uint64_t ext = v < 0 ? ~(uint64_t)0 : 0;
    x->w[2] = x->w[2] + ext + (uint64_t)(mid >> 64);
}

/* Two's complement negation over 192 bits (Limbs::neg, acc.rs:345-357). */
static l192 l192_neg(l192 x) {
    l192 r;
    uint64_t carry = 1;
    for (int i = 0; i < 3; i++) {
        u128 t = (u128)(~x.w[i]) + carry;
        r.w[i] = (uint64_t)t;
        carry = (uint64_t)(t >> 64);
    }
    return r;
}

/* Limbs::combine (acc.rs:391-402): the sum mod 2^192. */
static l192 l192_combine(l192 x, l192 y) {
    l192 r;
    uint64_t carry = 0;
    for (int i = 0; i < 3; i++) {
        u128 t = (u128)x.w[i] + y.w[i] + carry;
        r.w[i] = (uint64_t)t;
        carry = (uint64_t)(t >> 64);
    }
    return r;
}

/* ScaleExact for Limbs<L> (epilogue.rs:307-328): factor * x in the fixed
 * 192-bit register, wrapping past it ("no growth", acc.rs:208-215).  The
 * reference sums doublings of x (negated for a negative factor) over the bits
 * of |factor|; that is the product mod 2^192, computed here directly. */
static l192 l192_scale(l192 x, int64_t factor) {
    const uint64_t f = factor < 0 ? (uint64_t)0 - (uint64_t)factor : (uint64_t)factor;
    const u128 p0 = (u128)x.w[0] * f, p1 = (u128)x.w[1] * f;
    l192 r;
    r.w[0] = (uint64_t)p0;
    const u128 s1 = (u128)(uint64_t)p1 + (uint64_t)(p0 >> 64);
    r.w[1] = (uint64_t)s1;
    r.w[2] = x.w[2] * f + (uint64_t)(p1 >> 64) + (uint64_t)(s1 >> 64);
    return factor < 0 ? l192_neg(r) : r;
}

/* impl_encode_from_limbs (acc.rs:405-442). */
static i128 encode_l192(const l192 *x, int out_bytes, int mode) {
    i128 low = (i128)(((u128)x->w[1] << 64) | x->w[0]);
    if (mode == ENC_WRAPPING) {
        i128 mn, mx;
        int_range(out_bytes, &mn, &mx);
        return encode_i128_into(low, mn, mx, ENC_WRAPPING);
    }
    int negative = (int64_t)x->w[2] < 0;
    /* magnitude */
    uint64_t m0 = x->w[0], m1 = x->w[1], m2 = x->w[2];
    if (negative) {
        m0 = ~m0; m1 = ~m1; m2 = ~m2;
        u128 t = (u128)m0 + 1; m0 = (uint64_t)t;
        t = (u128)m1 + (uint64_t)(t >> 64); m1 = (uint64_t)t;
        m2 += (uint64_t)(t >> 64);
    }
    i128 mn, mx;
    int_range(out_bytes, &mn, &mx);
    if (m2 != 0) return negative ? mn : mx;
    u128 mag = ((u128)m1 << 64) | m0;
    u128 limit = negative ? (u128)0 - (u128)mn : (u128)mx;
    if (mag > limit) return negative ? mn : mx;
    return negative ? (i128)((u128)0 - mag) : (i128)mag;
}

/*
 * driver::gemm for a ring element (driver.rs:67-182): for every output cell,
 * the exact sum of E::mac products (alphabet.rs:559-616, acc i128 for
 * i8/i16/i32, Limbs<3> for i64), then Linear::finish.  beta == 0 never reads C
 * (epilogue.rs:73-77, CS-04).
 *
 * elem_bytes in {1,2,4,8}; out_bytes in {1,2,4,8,16}.  i64 elements: the
 * Limbs<3> register (acc.rs:215), Linear::finish as scale_exact(alpha) +
 * of_prior(C).scale_exact(beta), both mod 2^192 (epilogue.rs:80-95, 249-253,
 * 307-328), then impl_encode_from_limbs.  Their modular lane (Wrapping into
 * at most 64 bits, kernel.rs:371-398) is the same ring, so it gives the same
 * bytes and is not restated separately.
 */
int ora_gemm_int(int elem_bytes,
                 const void *a, uint64_t a_len, uint64_t a_rows, uint64_t a_cols, int64_t a_rs, int64_t a_cs,
                 const void *b, uint64_t b_len, uint64_t b_rows, uint64_t b_cols, int64_t b_rs, int64_t b_cs,
                 void *c, uint64_t c_len, uint64_t c_rows, uint64_t c_cols, int64_t c_rs, int64_t c_cs,
                 int out_bytes, int64_t alpha, int64_t beta, int mode) {
    if (!(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4 || elem_bytes == 8)) return ORA_INVALID_ARGUMENT;
    if (!(out_bytes == 1 || out_bytes == 2 || out_bytes == 4 || out_bytes == 8 || out_bytes == 16)) return ORA_INVALID_ARGUMENT;
    if (mode < 0 || mode > 3) return ORA_INVALID_ARGUMENT;
    view_t A = {a, a_len, a_rows, a_cols, a_rs, a_cs, 0};
    view_t B = {b, b_len, b_rows, b_cols, b_rs, b_cs, 0};
    view_t C = {c, c_len, c_rows, c_cols, c_rs, c_cs, 0};
    int st = make_triple(&A, &B, &C);
    if (st) return st;
    uint64_t m = A.rows, k = A.cols, n = B.cols;
    for (uint64_t i = 0; i < m; i++) {
        for (uint64_t j = 0; j < n; j++) {
            uint64_t ci = at(&C, i, j);
            if (elem_bytes == 8) {
                l192 acc = {{0, 0, 0}};
                for (uint64_t p = 0; p < k; p++) {
                    i128 x = load_int(a, at(&A, i, p), 8), y = load_int(b, at(&B, p, j), 8);
                    l192_add_i128(&acc, x * y);
                }
                l192 total = l192_scale(acc, alpha);
                if (beta != 0) {
                    l192 prior = {{0, 0, 0}};
                    l192_add_i128(&prior, load_int(c, ci, out_bytes));
                    total = l192_combine(total, l192_scale(prior, beta));
                }
                store_int(c, ci, out_bytes, encode_l192(&total, out_bytes, mode));
                continue;
            }
            i128 acc = 0;
            for (uint64_t p = 0; p < k; p++)
                acc += load_int(a, at(&A, i, p), elem_bytes) * load_int(b, at(&B, p, j), elem_bytes);
            /* gemm_packed_impl's modular route (kernel.rs:566-607): Wrapping
             * into an output of at most 32 bits adds in Z/2^32 and hands
             * Linear::finish the lane sign-extended (modular_spec and
             * modular_as_acc for i8/i16/i32, kernel.rs:185-221, 250-279,
             * 308-330).  Only the scaling can tell the two apart: alpha * X
             * saturates at 2^127 where alpha * (X mod 2^32) does not. */
            if (mode == 3 && out_bytes <= 4) acc = (i128)(int32_t)(uint32_t)(u128)acc;
            int reads = beta != 0;
            i128 prior = reads ? load_int(c, ci, out_bytes) : 0;
            store_int(c, ci, out_bytes, linear_finish_i128(acc, reads, prior, alpha, beta, out_bytes, mode));
        }
    }
    return ORA_OK;
}

/* ------------------------------------------------------------------------ */
/* Table-lookup GEMM over Packed<Grid<i8,16>,2> codes.                      */
/* TabulatedTriple (tabulated.rs:607-658): C = A * W^T, W is n x k coded    */
/* k-major, one coded row per output column; CodedMatrix::new               */
/* (matrix.rs:36-75): k even, codes.len == n * k/2.  Packed decodes the     */
/* low nibble first (codecs.rs:181-195, CK-03); Grid indexes code % 16      */
/* (codecs.rs:101-103).  The reference spells a per-group codebook as one   */
/* call per group of `group` coded rows; this restates all groups at once:  */
/* coded row r uses books[(r / group) * 16 + nibble].                       */
/* ------------------------------------------------------------------------ */
int ora_gemm_lut4(const int8_t *a, uint64_t a_len, uint64_t m, uint64_t k, int64_t a_rs, int64_t a_cs,
                  const uint8_t *codes, uint64_t codes_len, uint64_t n,
                  const int8_t *books, uint64_t books_len, uint64_t group,
                  void *c, uint64_t c_len, int64_t c_rs, int64_t c_cs,
                  int out_bytes, int64_t alpha, int64_t beta, int mode) {
    if (!(out_bytes == 1 || out_bytes == 2 || out_bytes == 4 || out_bytes == 8 || out_bytes == 16)) return ORA_INVALID_ARGUMENT;
    if (mode < 0 || mode > 3) return ORA_INVALID_ARGUMENT;
    /* CodedMatrix::new: a fixed-width tier with MAX_BLOCK 2. */
    if (k % 2 != 0) return ORA_SHORT_BUFFER;
    if (codes_len != n * (k / 2)) return ORA_SHORT_BUFFER;
    if (group == 0) return ORA_INVALID_ARGUMENT;
    uint64_t ngroups = n == 0 ? 0 : (n + group - 1) / group;
    if (books_len < ngroups * 16) return ORA_SHORT_BUFFER;
    view_t A = {a, a_len, m, k, a_rs, a_cs, 0};
    view_t C = {c, c_len, m, n, c_rs, c_cs, 0};
    if (!ora_place(A.len, A.rows, A.cols, A.rs, A.cs, &A.origin)) return ORA_SHORT_BUFFER;
    if (!ora_place(C.len, C.rows, C.cols, C.rs, C.cs, &C.origin)) return ORA_SHORT_BUFFER;
    if (ora_self_aliases(m, n, c_rs, c_cs)) return ORA_OUTPUT_ALIASES_ITSELF;
    uint64_t half = k / 2;
    for (uint64_t i = 0; i < m; i++) {
        for (uint64_t j = 0; j < n; j++) {
            const int8_t *book = books + (j / group) * 16;
            i128 acc = 0;
            for (uint64_t p = 0; p < k; p++) {
                uint8_t byte = codes[j * half + p / 2];
                uint8_t sub = (p % 2 == 0) ? (byte & 15) : (byte >> 4);
                acc += (i128)a[at(&A, i, p)] * (i128)book[sub % 16];
            }
            uint64_t ci = at(&C, i, j);
            int reads = beta != 0;
            i128 prior = reads ? load_int(c, ci, out_bytes) : 0;
            store_int(c, ci, out_bytes, linear_finish_i128(acc, reads, prior, alpha, beta, out_bytes, mode));
        }
    }
    return ORA_OK;
}

/* ------------------------------------------------------------------------ */
/* Exact float GEMM.                                                         */
/* Element::mac for floats (alphabet.rs:856-890) + FloatElement::decode      */
/* (alphabet.rs:905-957) + Complete accumulation (acc.rs:469-1243) +         */
/* Complete::scale (acc.rs:1028-1060) + Linear::finish + the round-once      */
/* encode (acc.rs:1734-1868).                                                */
/*                                                                           */
/* The exact value is held as sign-separated magnitudes (pos - neg) in a     */
/* fixed-point register whose bit 0 has exponent MIN_EXP: -298 for f32,      */
/* -2148 for f64 (generated.rs:114-127).  Non-finite state is a NaN/+inf/    */
/* -inf flag union as in Complete (set_nan / set_infinity / combine).        */
/* ------------------------------------------------------------------------ */

#define FL_NAN 1
#define FL_PINF 2
#define FL_NINF 4

typedef struct {
    int limbs;
    uint64_t *pos, *neg;
} bigreg;

static void big_add_shifted(uint64_t *r, int limbs, u128 mag, int64_t shift) {
    /* r += mag << shift; shift >= 0, mag < 2^128 */
    if (mag == 0) return;
    int64_t w = shift / 64, b = shift % 64;
    uint64_t parts[3];
    parts[0] = (uint64_t)(mag << b);
    parts[1] = (uint64_t)((b ? (mag >> (64 - b)) : (mag >> 64)));
    parts[2] = b ? (uint64_t)((mag >> 64) >> (64 - b)) : 0;
    uint64_t carry = 0;
    for (int64_t i = w, q = 0; i < limbs && (q < 3 || carry); i++, q++) {
        u128 s = (u128)r[i] + (q < 3 ? parts[q] : 0) + carry;
        r[i] = (uint64_t)s;
        carry = (uint64_t)(s >> 64);
    }
}

/* decode: alphabet.rs:905-957.  Returns class 0 finite, 1 inf, 2 NaN. */
static int decode_f(int is64, uint64_t bits, int *sign, uint64_t *mant, int *exp) {
    int mant_bits = is64 ? 52 : 23, exp_bits = is64 ? 11 : 8;
    int bias = (1 << (exp_bits - 1)) - 1;
    uint64_t fraction = bits & (((uint64_t)1 << mant_bits) - 1);
    uint64_t biased = (bits >> mant_bits) & (((uint64_t)1 << exp_bits) - 1);
    *sign = (int)((bits >> (mant_bits + exp_bits)) & 1);
    if (biased == ((uint64_t)1 << exp_bits) - 1) return fraction == 0 ? 1 : 2;
    if (biased == 0) { *mant = fraction; *exp = 1 - bias - mant_bits; return 0; }
    *mant = fraction | ((uint64_t)1 << mant_bits);
    *exp = (int)biased - bias - mant_bits;
    return 0;
}

/* Magnitude/sign of pos - neg into out (limbs), returns sign. */
static int big_sub_abs(const uint64_t *p, const uint64_t *q, uint64_t *out, int limbs) {
    int cmp = 0;
    for (int i = limbs - 1; i >= 0; i--) {
        if (p[i] != q[i]) { cmp = p[i] > q[i] ? 1 : -1; break; }
    }
    const uint64_t *x = cmp >= 0 ? p : q, *y = cmp >= 0 ? q : p;
    uint64_t borrow = 0;
    for (int i = 0; i < limbs; i++) {
        u128 d = (u128)x[i] - y[i] - borrow;
        out[i] = (uint64_t)d;
        borrow = (uint64_t)(d >> 64) ? 1 : 0;
    }
    return cmp < 0;
}

static void big_mul_small(uint64_t *r, int limbs, uint64_t f) {
    uint64_t carry = 0;
    for (int i = 0; i < limbs; i++) {
        u128 t = (u128)r[i] * f + carry;
        r[i] = (uint64_t)t;
        carry = (uint64_t)(t >> 64);
    }
}

/* The round-once encode, acc.rs:1734-1868, from a magnitude with bit 0 at
 * exponent min_exp. */
static uint64_t encode_float(int is64, int flags, int negative, const uint64_t *mag, int limbs,
                             int min_exp, int mode) {
    const int MANT = is64 ? 52 : 23, EXPO = is64 ? 11 : 8, P = MANT + 1;
    const int BIAS = (1 << (EXPO - 1)) - 1;
    const int SUB_LSB_EXP = 1 - BIAS - MANT;
    const uint64_t expmask = ((uint64_t)1 << EXPO) - 1;
    int nan = (flags & FL_NAN) || ((flags & FL_PINF) && (flags & FL_NINF));
    if (nan) return is64 ? 0x7ff8000000000000ull : 0x7fc00000ull; /* canonical NaN */
    if (flags & (FL_PINF | FL_NINF)) {
        uint64_t s = (flags & FL_NINF) ? 1 : 0;
        return (s << (MANT + EXPO)) | (expmask << MANT);
    }
    int high = -1;
    for (int i = limbs - 1; i >= 0; i--)
        if (mag[i]) { high = i * 64 + 63 - __builtin_clzll(mag[i]); break; }
    if (high < 0) return 0; /* exact zero -> +0 (acc.rs:1760-1766) */
    int exp = min_exp + high;
    int lsb_exp = exp - (P - 1) < SUB_LSB_EXP ? SUB_LSB_EXP : exp - (P - 1);
    int lsb = lsb_exp - min_exp;
    if (lsb < 0) return 0;
#define BIT(i) ((i) / 64 < limbs ? ((mag[(i) / 64] >> ((i) % 64)) & 1) : 0)
    uint64_t sig = 0;
    for (int t = 0; t < P; t++) sig |= (uint64_t)BIT(lsb + t) << t;
    int round_bit = 0, sticky = 0;
    if (lsb > 0) {
        round_bit = (int)BIT(lsb - 1);
        int below = lsb - 1;
        for (int i = 0; i < below / 64 && i < limbs; i++) if (mag[i]) sticky = 1;
        if (!sticky && below / 64 < limbs) {
            uint64_t msk = (below % 64) ? ((((uint64_t)1) << (below % 64)) - 1) : 0;
            if (mag[below / 64] & msk) sticky = 1;
        }
    }
#undef BIT
    int inc = (mode == ENC_NEAREST) ? (round_bit && (sticky || (sig & 1))) : 0;
    sig += (uint64_t)inc;
    if (sig >> P) { sig >>= 1; lsb_exp += 1; }
    uint64_t sbit = (uint64_t)(negative ? 1 : 0) << (MANT + EXPO);
    if (sig == 0) return sbit; /* underflow keeps the sign */
    int top = 63 - __builtin_clzll(sig);
    int value_exp = lsb_exp + top;
    if ((sig >> (P - 1)) == 1) {
        int biased = value_exp + BIAS;
        if (biased >= (int)expmask) {
            if (mode == ENC_NEAREST) return sbit | (expmask << MANT);
            return sbit | ((expmask - 1) << MANT) | (((uint64_t)1 << MANT) - 1);
        }
        return sbit | ((uint64_t)biased << MANT) | (sig & (((uint64_t)1 << MANT) - 1));
    }
    return sbit | sig;
}

static uint64_t load_fbits(const void *p, uint64_t idx, int is64) {
    return is64 ? ((const uint64_t *)p)[idx] : ((const uint32_t *)p)[idx];
}

/* One output cell: the value alpha * sum + beta * C, exactly, then encoded. */
typedef struct {
    int is64, limbs, min_exp;
    uint64_t *pos, *neg, *tmp;
} fctx;

static void fctx_clear(fctx *f) {
    memset(f->pos, 0, sizeof(uint64_t) * f->limbs);
    memset(f->neg, 0, sizeof(uint64_t) * f->limbs);
}

/* Complete::scale (acc.rs:1028-1060) applied to a (pos,neg,flags) value. */
static int scale_value(fctx *f, int flags, int64_t factor) {
    int nan = (flags & FL_NAN) || ((flags & FL_PINF) && (flags & FL_NINF));
    if (nan) return flags;
    if (factor == 1) return flags;
    if (factor == 0) {
        if (flags & (FL_PINF | FL_NINF)) { fctx_clear(f); return FL_NAN; }
        fctx_clear(f);
        return 0;
    }
    uint64_t mag = factor < 0 ? (uint64_t)0 - (uint64_t)factor : (uint64_t)factor;
    big_mul_small(f->pos, f->limbs, mag);
    big_mul_small(f->neg, f->limbs, mag);
    if (factor < 0) {
        uint64_t *t = f->pos; f->pos = f->neg; f->neg = t;
        int nf = flags & FL_NAN;
        if (flags & FL_PINF) nf |= FL_NINF;
        if (flags & FL_NINF) nf |= FL_PINF;
        flags = nf;
    }
    return flags;
}

int ora_gemm_float(int is64,
                   const void *a, uint64_t a_len, uint64_t a_rows, uint64_t a_cols, int64_t a_rs, int64_t a_cs,
                   const void *b, uint64_t b_len, uint64_t b_rows, uint64_t b_cols, int64_t b_rs, int64_t b_cs,
                   void *c, uint64_t c_len, uint64_t c_rows, uint64_t c_cols, int64_t c_rs, int64_t c_cs,
                   int64_t alpha, int64_t beta, int mode) {
    if (mode < 0 || mode > 3) return ORA_INVALID_ARGUMENT;
    view_t A = {a, a_len, a_rows, a_cols, a_rs, a_cs, 0};
    view_t B = {b, b_len, b_rows, b_cols, b_rs, b_cs, 0};
    view_t C = {c, c_len, c_rows, c_cols, c_rs, c_cs, 0};
    int st = make_triple(&A, &B, &C);
    if (st) return st;
    fctx f;
    f.is64 = is64;
    f.min_exp = is64 ? -2148 : -298;
    /* Register width: products reach 2^(2*max_exp) = 2^2048 (f64) / 2^256
     * (f32) above 2^min_exp, then depth (< 2^64), alpha (2^63), beta*C and a
     * sign: 4480 bits for f64, 768 for f32. */
    f.limbs = is64 ? 70 : 12;
    f.pos = calloc(f.limbs, 8);
    f.neg = calloc(f.limbs, 8);
    f.tmp = calloc(f.limbs, 8);
    uint64_t *cpos = calloc(f.limbs, 8), *cneg = calloc(f.limbs, 8);
    if (!f.pos || !f.neg || !f.tmp || !cpos || !cneg) return ORA_INVALID_ARGUMENT;
    uint64_t m = A.rows, k = A.cols, n = B.cols;
    for (uint64_t i = 0; i < m; i++) {
        for (uint64_t j = 0; j < n; j++) {
            fctx_clear(&f);
            int flags = 0;
            for (uint64_t p = 0; p < k; p++) {
                int sa, sb, ea, eb;
                uint64_t ma, mb;
                int ca = decode_f(is64, load_fbits(a, at(&A, i, p), is64), &sa, &ma, &ea);
                int cb = decode_f(is64, load_fbits(b, at(&B, p, j), is64), &sb, &mb, &eb);
                if (ca == 2 || cb == 2) { flags |= FL_NAN; continue; }
                if (ca == 1 || cb == 1) {
                    /* inf * 0 is NaN; otherwise an infinity of the product sign */
                    if ((ca == 0 && ma == 0) || (cb == 0 && mb == 0)) { flags |= FL_NAN; continue; }
                    flags |= (sa != sb) ? FL_NINF : FL_PINF;
                    continue;
                }
                u128 prod = (u128)ma * mb;
                if (!prod) continue;
                int64_t shift = (int64_t)ea + eb - f.min_exp;
                big_add_shifted((sa != sb) ? f.neg : f.pos, f.limbs, prod, shift);
            }
            flags = scale_value(&f, flags, alpha);
            uint64_t ci = at(&C, i, j);
            if (beta != 0) {
                /* AbsorbPrior: Complete::of(C) (acc.rs:1003-1020), scaled by beta. */
                int sc, ec;
                uint64_t mc;
                int cc = decode_f(is64, load_fbits(c, ci, is64), &sc, &mc, &ec);
                fctx g = f;
                g.pos = cpos; g.neg = cneg;
                fctx_clear(&g);
                int gflags = 0;
                if (cc == 2) gflags = FL_NAN;
                else if (cc == 1) gflags = sc ? FL_NINF : FL_PINF;
                else big_add_shifted(sc ? g.neg : g.pos, g.limbs, mc, (int64_t)ec - g.min_exp);
                gflags = scale_value(&g, gflags, beta);
                /* combine */
                uint64_t carry = 0;
                for (int t = 0; t < f.limbs; t++) {
                    u128 s = (u128)f.pos[t] + g.pos[t] + carry;
                    f.pos[t] = (uint64_t)s; carry = (uint64_t)(s >> 64);
                }
                carry = 0;
                for (int t = 0; t < f.limbs; t++) {
                    u128 s = (u128)f.neg[t] + g.neg[t] + carry;
                    f.neg[t] = (uint64_t)s; carry = (uint64_t)(s >> 64);
                }
                flags |= gflags;
                cpos = g.pos; cneg = g.neg;
            }
            int negative = big_sub_abs(f.pos, f.neg, f.tmp, f.limbs);
            uint64_t bits = encode_float(is64, flags, negative, f.tmp, f.limbs, f.min_exp, mode);
            if (is64) ((uint64_t *)c)[ci] = bits;
            else ((uint32_t *)c)[ci] = (uint32_t)bits;
        }
    }
    free(f.pos); free(f.neg); free(f.tmp); free(cpos); free(cneg);
    return ORA_OK;
}

/* ------------------------------------------------------------------------ */
/* Tropical (max, +) GEMM over Trop<i8> (tropical.rs:63-110, #[repr(C)]      */
/* {value: i8, finite: bool}, 2 bytes).  Trop::mac offers x + y only when    */
/* both are finite (tropical.rs:311-318); TropAcc's combine is max with      */
/* NEG_INF = i128::MIN (tropical.rs:150-215).  MaxPlus epilogue              */
/* (epilogue.rs:137-192): (alpha (x) P) (+) (beta (x) C), beta = -inf never   */
/* reads C (CS-11).  Encode (tropical.rs:336-350): -inf -> {0,false}; finite */
/* v -> encode_i128_into(v, O::MIN+1, O::MAX-1, mode).  Output record        */
/* Trop<O> is {O value; u8 finite} padded to alignof(O): 2, 4, 8, 16 bytes.  */
/* ------------------------------------------------------------------------ */

static i128 trop_load(const void *p, uint64_t idx, int vbytes, int *finite) {
    int rec = vbytes * 2;
    const unsigned char *r = (const unsigned char *)p + idx * rec;
    *finite = r[vbytes] != 0;
    return load_int(r, 0, vbytes);
}

static void trop_store(void *p, uint64_t idx, int vbytes, int finite, i128 v) {
    int rec = vbytes * 2;
    unsigned char *r = (unsigned char *)p + idx * rec;
    store_int(r, 0, vbytes, finite ? v : 0);
    r[vbytes] = (unsigned char)(finite ? 1 : 0);
}

int ora_gemm_trop(int elem_bytes,
                  const void *a, uint64_t a_len, uint64_t a_rows, uint64_t a_cols, int64_t a_rs, int64_t a_cs,
                  const void *b, uint64_t b_len, uint64_t b_rows, uint64_t b_cols, int64_t b_rs, int64_t b_cs,
                  void *c, uint64_t c_len, uint64_t c_rows, uint64_t c_cols, int64_t c_rs, int64_t c_cs,
                  int out_bytes, int64_t alpha, int alpha_finite, int64_t beta, int beta_finite, int mode) {
    if (!(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4 || elem_bytes == 8)) return ORA_INVALID_ARGUMENT;
    if (!(out_bytes == 1 || out_bytes == 2 || out_bytes == 4 || out_bytes == 8)) return ORA_INVALID_ARGUMENT;
    if (mode < 0 || mode > 3) return ORA_INVALID_ARGUMENT;
    view_t A = {a, a_len, a_rows, a_cols, a_rs, a_cs, 0};
    view_t B = {b, b_len, b_rows, b_cols, b_rs, b_cs, 0};
    view_t C = {c, c_len, c_rows, c_cols, c_rs, c_cs, 0};
    int st = make_triple(&A, &B, &C);
    if (st) return st;
    uint64_t m = A.rows, k = A.cols, n = B.cols;
    i128 mn, mx;
    int_range(out_bytes, &mn, &mx);
    for (uint64_t i = 0; i < m; i++) {
        for (uint64_t j = 0; j < n; j++) {
            i128 acc = I128_MIN;
            for (uint64_t p = 0; p < k; p++) {
                int fa, fb;
                i128 x = trop_load(a, at(&A, i, p), elem_bytes, &fa);
                i128 y = trop_load(b, at(&B, p, j), elem_bytes, &fb);
                if (fa && fb && x + y > acc) acc = x + y;
            }
            /* shift_exact by alpha (epilogue.rs:203-216) */
            i128 total = (acc != I128_MIN && alpha_finite) ? acc + alpha : I128_MIN;
            uint64_t ci = at(&C, i, j);
            if (beta_finite) {
                int fc;
                i128 cv = trop_load(c, ci, out_bytes, &fc);
                i128 prior = fc ? cv + beta : I128_MIN;
                if (prior > total) total = prior;
            }
            if (total == I128_MIN) trop_store(c, ci, out_bytes, 0, 0);
            else trop_store(c, ci, out_bytes, 1, encode_i128_into(total, mn + 1, mx - 1, mode));
        }
    }
    return ORA_OK;
}

/*
 * gemm_selected (crates/uor-matmul-gemm/src/selection.rs:170-320), the
 * Lexicographic mechanism: per cell, the maximum of the (value, index) pairs
 * under the order "greater value, then smaller index" (Lex::combine,
 * selection.rs:115-153), a term at the semiring zero standing at i128::MIN;
 * C gets MaxPlus::finish of the value, W the index, min(index, k) (an empty
 * reduction's index is k = 0).  The witness view has 8-byte (usize) cells and
 * is checked like C (SelectedTriple::new, selection.rs:72-97).
 */
int ora_gemm_trop_selected(int elem_bytes,
                           const void *a, uint64_t a_len, uint64_t a_rows, uint64_t a_cols, int64_t a_rs, int64_t a_cs,
                           const void *b, uint64_t b_len, uint64_t b_rows, uint64_t b_cols, int64_t b_rs, int64_t b_cs,
                           void *c, uint64_t c_len, uint64_t c_rows, uint64_t c_cols, int64_t c_rs, int64_t c_cs,
                           uint64_t *w, uint64_t w_len, uint64_t w_rows, uint64_t w_cols, int64_t w_rs, int64_t w_cs,
                           int out_bytes, int64_t alpha, int alpha_finite, int64_t beta, int beta_finite, int mode) {
    if (!(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4 || elem_bytes == 8)) return ORA_INVALID_ARGUMENT;
    if (!(out_bytes == 1 || out_bytes == 2 || out_bytes == 4 || out_bytes == 8)) return ORA_INVALID_ARGUMENT;
    if (mode < 0 || mode > 3) return ORA_INVALID_ARGUMENT;
    view_t A = {a, a_len, a_rows, a_cols, a_rs, a_cs, 0};
    view_t B = {b, b_len, b_rows, b_cols, b_rs, b_cs, 0};
    view_t C = {c, c_len, c_rows, c_cols, c_rs, c_cs, 0};
    int st = make_triple(&A, &B, &C);
    if (st) return st;
    view_t W = {w, w_len, w_rows, w_cols, w_rs, w_cs, 0};
    if (!ora_place(W.len, W.rows, W.cols, W.rs, W.cs, &W.origin)) return ORA_SHORT_BUFFER;
    if (W.rows != A.rows || W.cols != B.cols) return ORA_NONCONFORMANT;
    if (ora_self_aliases(W.rows, W.cols, W.rs, W.cs)) return ORA_OUTPUT_ALIASES_ITSELF;
    uint64_t m = A.rows, k = A.cols, n = B.cols;
    i128 mn, mx;
    int_range(out_bytes, &mn, &mx);
    for (uint64_t i = 0; i < m; i++) {
        for (uint64_t j = 0; j < n; j++) {
            i128 v = I128_MIN;
            uint64_t idx = UINT64_MAX;  /* Lex::EMPTY */
            for (uint64_t p = 0; p < k; p++) {
                int fa, fb;
                i128 x = trop_load(a, at(&A, i, p), elem_bytes, &fa);
                i128 y = trop_load(b, at(&B, p, j), elem_bytes, &fb);
                i128 t = (fa && fb) ? x + y : I128_MIN;
                if (t > v || (t == v && p < idx)) { v = t; idx = p; }
            }
            i128 total = (v != I128_MIN && alpha_finite) ? v + alpha : I128_MIN;
            uint64_t ci = at(&C, i, j);
            if (beta_finite) {
                int fc;
                i128 cv = trop_load(c, ci, out_bytes, &fc);
                i128 prior = fc ? cv + beta : I128_MIN;
                if (prior > total) total = prior;
            }
            if (total == I128_MIN) trop_store(c, ci, out_bytes, 0, 0);
            else trop_store(c, ci, out_bytes, 1, encode_i128_into(total, mn + 1, mx - 1, mode));
            w[at(&W, i, j)] = idx < k ? idx : k;
        }
    }
    return ORA_OK;
}

/* ------------------------------------------------------------------ codecs
 * Codec<i8, Bd>::decode_element for the fixed-width tiers
 * (crates/uor-matmul-codec/src/codecs.rs) and CodedMatrix::at
 * (crates/uor-matmul-codec/src/matrix.rs:202-207).
 */
enum { TIER_IDENTITY = 0, TIER_GRID = 1, TIER_BOOK = 2, TIER_SIGN = 3, TIER_TERNARY = 4 };

typedef struct {
    int tier, code_bits, packed, has_zero;
    int64_t zero;
    uint64_t entries, block;
    const int8_t *table;
    uint64_t table_len;
} ora_codec;

/* MAX_BLOCK of the base tier: Identity and Grid decode one element per code
 * (codecs.rs:46, 99); Book, Sign and Ternary BLK (:303, 384, 489). */
static uint64_t codec_inner_block(const ora_codec *c) {
    return (c->tier == TIER_IDENTITY || c->tier == TIER_GRID) ? 1 : c->block;
}

/* Packed: P * C::MAX_BLOCK (codecs.rs:177). */
static uint64_t codec_max_block(const ora_codec *c) {
    return (c->packed ? (uint64_t)c->packed : 1) * codec_inner_block(c);
}

static int8_t codec_base(const ora_codec *c, uint32_t code, uint64_t i) {
    switch (c->tier) {
    case TIER_IDENTITY: /* codecs.rs:49-51 */
        return (int8_t)(uint8_t)code;
    case TIER_GRID: /* codecs.rs:102-104 */
        return c->table[code % c->entries];
    case TIER_BOOK: /* codecs.rs:306-308 */
        return c->table[(code % c->entries) * c->block + i % c->block];
    case TIER_SIGN: { /* codecs.rs:387-400 */
        uint64_t bit = i % c->block;
        return (bit < (uint64_t)c->code_bits && ((code >> bit) & 1u)) ? 1 : -1;
    }
    default: { /* TIER_TERNARY, codecs.rs:492-516 */
        uint64_t shift = 2 * (i % c->block);
        uint32_t digit = shift < (uint64_t)c->code_bits ? (code >> shift) & 3u : 0u;
        return digit == 0 ? -1 : digit == 2 ? 1 : 0;
    }
    }
}

static int8_t codec_decode(const ora_codec *c, uint32_t code, uint64_t i) {
    int8_t v;
    if (c->packed) {
        /* Packed::decode_element (codecs.rs:181-199): the low sub-code first. */
        uint32_t bits = 8u / (uint32_t)c->packed;
        uint32_t mask = bits >= 8 ? 0xFFu : ((1u << bits) - 1u);
        uint64_t ib = codec_inner_block(c);
        uint64_t p = i / ib;
        uint32_t sub = (code >> (bits * (uint32_t)p)) & mask;
        v = codec_base(c, sub, i % ib);
    } else {
        v = codec_base(c, code, i);
    }
    /* Offset::decode_element (codecs.rs:608-616): i8 wrapping_sub. */
    if (c->has_zero) v = (int8_t)(uint8_t)((uint32_t)(uint8_t)v - (uint32_t)(uint8_t)(int8_t)c->zero);
    return v;
}

/* What the decode needs of a codec: a known tier, P dividing 8, code widths
 * the tier's code type has, a table of N (x BLK) entries. */
static int codec_check(const ora_codec *c) {
    if (c->tier < TIER_IDENTITY || c->tier > TIER_TERNARY) return ORA_INVALID_ARGUMENT;
    if (!(c->packed == 0 || c->packed == 1 || c->packed == 2 || c->packed == 4 || c->packed == 8))
        return ORA_INVALID_ARGUMENT;
    if (c->tier == TIER_IDENTITY && (c->packed || c->code_bits != 8)) return ORA_INVALID_ARGUMENT;
    if (c->tier == TIER_GRID && c->code_bits != 16) return ORA_INVALID_ARGUMENT;
    if (c->code_bits != 8 && c->code_bits != 16) return ORA_INVALID_ARGUMENT;
    if (c->has_zero && (c->zero < -128 || c->zero > 127)) return ORA_INVALID_ARGUMENT;
    if (c->tier == TIER_GRID || c->tier == TIER_BOOK) {
        if (c->entries == 0) return ORA_INVALID_ARGUMENT;
        uint64_t need = c->entries * (c->tier == TIER_BOOK ? c->block : 1);
        if (c->tier == TIER_BOOK && c->block && need / c->block != c->entries) return ORA_INVALID_ARGUMENT;
        if (!c->table || c->table_len < need) return ORA_SHORT_BUFFER;
    }
    /* The GPU cursor keeps positions inside a block in 32 bits; the oracle
     * refuses the same codecs so both name one status. */
    if (c->tier >= TIER_BOOK && c->block >= (1ull << 31)) return ORA_INVALID_ARGUMENT;
    return ORA_OK;
}

/* CodedMatrix::new for a fixed-width tier (matrix.rs:36-55) and the decode of
 * every element, row-major into out (rows x cols). */
int ora_coded_decode(int tier, int code_bits, int packed, int has_zero, int64_t zero,
                     uint64_t entries, uint64_t block, const int8_t *table, uint64_t table_len,
                     const void *codes, uint64_t codes_len, uint64_t rows, uint64_t cols,
                     int8_t *out) {
    ora_codec c = {tier, code_bits, packed, has_zero, zero, entries, block, table, table_len};
    int st = codec_check(&c);
    if (st) return st;
    uint64_t mb = codec_max_block(&c);
    if (mb == 0 || cols % mb != 0) return ORA_SHORT_BUFFER;
    uint64_t per_row = cols / mb;
    if (per_row && rows > UINT64_MAX / per_row) return ORA_SHORT_BUFFER;
    if (rows * per_row != codes_len) return ORA_SHORT_BUFFER;
    int cb = packed ? 1 : code_bits / 8;
    for (uint64_t r = 0; r < rows; r++)
        for (uint64_t q = 0; q < cols; q++) {
            uint64_t at = r * per_row + q / mb;
            uint32_t code = cb == 1 ? ((const uint8_t *)codes)[at] : ((const uint16_t *)codes)[at];
            out[r * cols + q] = codec_decode(&c, code, q % mb);
        }
    return ORA_OK;
}
