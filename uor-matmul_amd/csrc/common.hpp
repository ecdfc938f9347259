// Shared host and device pieces of the gfx950 route: view validation (the
// reference's MatView::new / Triple::new), the integer encode, and launch
// helpers.  Host code here runs before anything is enqueued, so a request the
// reference would reject never reaches a kernel.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/uor_gfx950.h"

namespace uor {

typedef __int128 i128;
typedef unsigned __int128 u128;

// ----------------------------------------------------------------- views --

// A view whose placement has been decided: the device address of element
// (0, 0) and its strides, plus the placement facts the loaders specialise on.
struct Placed {
    char *base;      // device address of element (0,0), in bytes
    uint64_t rows, cols;
    int64_t rs, cs;  // element strides
    int elem;        // element size in bytes
};

// Strides::extent + place (crates/uor-matmul-core/src/layout.rs:69-98,
// 161-182): the origin that puts the lowest reached offset at element 0, or
// false when the view does not fit in `len` elements or its reach overflows.
static inline bool place_view(uint64_t len, uint64_t rows, uint64_t cols, int64_t rs,
                              int64_t cs, uint64_t *origin) {
    if (rows == 0 || cols == 0) {
        *origin = 0;
        return true;
    }
    int64_t r, c, lo, hi;
    if (__builtin_mul_overflow((int64_t)(rows - 1), rs, &r)) return false;
    if (__builtin_mul_overflow((int64_t)(cols - 1), cs, &c)) return false;
    if (__builtin_add_overflow(rs < 0 ? r : (int64_t)0, cs < 0 ? c : (int64_t)0, &lo)) return false;
    if (__builtin_add_overflow(rs < 0 ? (int64_t)0 : r, cs < 0 ? (int64_t)0 : c, &hi)) return false;
    if (lo > 0) return false;
    uint64_t o = (uint64_t)0 - (uint64_t)lo;
    uint64_t h = (uint64_t)hi;  // hi >= 0 here
    uint64_t top;
    if (__builtin_add_overflow(o, h, &top)) return false;
    if (top >= len) return false;
    *origin = o;
    return true;
}

// Strides::self_aliases (layout.rs:116-143): two distinct coordinates of an
// rows x cols view share a cell iff (cs/g, -rs/g) fits the shape.
static inline bool self_aliases(uint64_t rows, uint64_t cols, int64_t rs, int64_t cs) {
    if (rows == 0 || cols == 0) return false;
    if (rows <= 1 && cols <= 1) return false;
    if (rows > 1 && rs == 0) return true;
    if (cols > 1 && cs == 0) return true;
    if (rows <= 1 || cols <= 1) return false;
    uint64_t a = rs < 0 ? (uint64_t)0 - (uint64_t)rs : (uint64_t)rs;
    uint64_t b = cs < 0 ? (uint64_t)0 - (uint64_t)cs : (uint64_t)cs;
    uint64_t x = a, y = b;
    while (y) {
        uint64_t t = x % y;
        x = y;
        y = t;
    }
    return (b / x) < rows && (a / x) < cols;
}

static inline int place(const uor_view *v, int elem, Placed *out) {
    if (!v) return UOR_INVALID_ARGUMENT;
    uint64_t origin;
    if (!place_view(v->len, v->rows, v->cols, v->rs, v->cs, &origin)) return UOR_SHORT_BUFFER;
    if (v->rows != 0 && v->cols != 0 && v->data == nullptr) return UOR_SHORT_BUFFER;
    out->base = (char *)v->data + origin * (uint64_t)elem;
    out->rows = v->rows;
    out->cols = v->cols;
    out->rs = v->rs;
    out->cs = v->cs;
    out->elem = elem;
    return UOR_OK;
}

// MatView::new x3 then Triple::new (crates/uor-matmul/src/slice.rs:164-170,
// layout.rs:534-575), in the reference's order.
static inline int make_triple(const uor_view *a, int ea, const uor_view *b, int eb,
                              const uor_view *c, int ec, Placed *A, Placed *B, Placed *C) {
    int st;
    if ((st = place(a, ea, A))) return st;
    if ((st = place(b, eb, B))) return st;
    if ((st = place(c, ec, C))) return st;
    if (A->cols != B->rows) return UOR_NONCONFORMANT;
    if (C->rows != A->rows || C->cols != B->cols) return UOR_NONCONFORMANT;
    if (self_aliases(C->rows, C->cols, C->rs, C->cs)) return UOR_OUTPUT_ALIASES_ITSELF;
    return UOR_OK;
}

static inline bool valid_out_type(int t) {
    return t == UOR_OUT_I8 || t == UOR_OUT_I16 || t == UOR_OUT_I32 || t == UOR_OUT_I64 ||
           t == UOR_OUT_I128;
}

static inline bool valid_encode(int e) { return e >= UOR_ENCODE_NEAREST && e <= UOR_ENCODE_WRAPPING; }

#define UOR_HIP(expr)                                   \
    do {                                                \
        hipError_t e_ = (expr);                         \
        if (e_ != hipSuccess) return UOR_HIP_ERROR + (int)e_; \
    } while (0)

static inline void route_set(uor_route *r, int kind) {
    if (!r) return;
    *r = uor_route{};
    r->kind = kind;
}

// A scratch offer may start anywhere.  Every route carves it from its first
// 256-byte aligned byte (so 8-byte atomics and 16-byte stores into it are
// aligned); *have gets what is left of the offer from there (0 for none).
static inline char *offer_align(void *scratch, uint64_t bytes, uint64_t *have) {
    if (!scratch) {
        *have = 0;
        return nullptr;
    }
    const uintptr_t p0 = (uintptr_t)scratch, p1 = (p0 + 255) & ~(uintptr_t)255;
    *have = bytes > (uint64_t)(p1 - p0) ? bytes - (uint64_t)(p1 - p0) : 0;
    return (char *)p1;
}

// ------------------------------------------------------ integer epilogue --

// The value range of an integer output of `bytes` bytes.
__host__ __device__ static inline void out_range(int bytes, i128 *mn, i128 *mx) {
    switch (bytes) {
    case 1: *mn = -128; *mx = 127; break;
    case 2: *mn = -32768; *mx = 32767; break;
    case 4: *mn = -(i128)2147483648LL; *mx = 2147483647; break;
    case 8: *mn = (i128)INT64_MIN; *mx = (i128)INT64_MAX; break;
    default:
        *mn = (i128)((u128)1 << 127);
        *mx = (i128)(((u128)1 << 127) - 1);
        break;
    }
}

// encode_i128_into (crates/uor-matmul-core/src/acc.rs:128-150): Wrapping is
// two's-complement truncation to the output width; every other mode clamps.
__device__ static inline i128 encode_int(i128 v, int bytes, int mode) {
    if (mode == UOR_ENCODE_WRAPPING) {
        if (bytes >= 16) return v;
        int sh = 128 - 8 * bytes;
        return (i128)((u128)v << sh) >> sh;
    }
    i128 mn, mx;
    out_range(bytes, &mn, &mx);
    return v < mn ? mn : (v > mx ? mx : v);
}

// i128::saturating_mul (ScaleExact for i128, crates/uor-matmul-gemm/src/
// epilogue.rs:280-289).
__device__ static inline i128 sat_mul(i128 x, int64_t f) {
    const i128 MX = (i128)(((u128)1 << 127) - 1), MN = (i128)((u128)1 << 127);
    if (x == 0 || f == 0) return 0;
    const bool neg = (x < 0) != (f < 0);
    const u128 ax = x < 0 ? (u128)0 - (u128)x : (u128)x;
    const uint64_t af = f < 0 ? (uint64_t)0 - (uint64_t)f : (uint64_t)f;
    // |x| * |f| as a 192-bit product (top : p), without a 128-bit division.
    const uint64_t a0 = (uint64_t)ax, a1 = (uint64_t)(ax >> 64);
    const uint64_t lo = a0 * af, c0 = __umul64hi(a0, af);
    const uint64_t m1 = a1 * af, h1 = __umul64hi(a1, af);
    const uint64_t mid = m1 + c0;
    const uint64_t top = h1 + (mid < m1 ? 1 : 0);
    const u128 p = ((u128)mid << 64) | lo;
    // It overflows i128 iff it exceeds the bound for its sign.
    const u128 limit = neg ? ((u128)1 << 127) : (((u128)1 << 127) - 1);
    if (top != 0 || p > limit) return neg ? MN : MX;
    return neg ? (i128)((u128)0 - p) : (i128)p;
}

template <int OB>
__device__ static inline i128 load_out(const char *p) {
    if constexpr (OB == 1) return *(const int8_t *)p;
    else if constexpr (OB == 2) return *(const int16_t *)p;
    else if constexpr (OB == 4) return *(const int32_t *)p;
    else if constexpr (OB == 8) return *(const int64_t *)p;
    else {
        const uint64_t *q = (const uint64_t *)p;
        return (i128)(((u128)q[1] << 64) | q[0]);
    }
}

template <int OB>
__device__ static inline void store_out(char *p, i128 v) {
    if constexpr (OB == 1) *(int8_t *)p = (int8_t)v;
    else if constexpr (OB == 2) *(int16_t *)p = (int16_t)v;
    else if constexpr (OB == 4) *(int32_t *)p = (int32_t)v;
    else if constexpr (OB == 8) *(int64_t *)p = (int64_t)v;
    else {
        uint64_t *q = (uint64_t *)p;
        q[0] = (uint64_t)(u128)v;
        q[1] = (uint64_t)((u128)v >> 64);
    }
}

// Linear::finish for an i128 accumulator (epilogue.rs:67-95): scale by alpha
// with saturating_mul, add sat_mul(C, beta) with a wrapping add (acc.rs:
// 101-105 in a release build), encode once.  `sum` is the exact sum.
// FAST is chosen by the host only when |alpha*sum| + |beta*C| < 2^63 for every
// reachable input, so that the int64 evaluation is the same integer.
template <int OB, bool FAST>
__device__ static inline void linear_finish(char *cp, int64_t sum, int64_t alpha, int64_t beta,
                                            int mode) {
    if constexpr (FAST) {
        int64_t t = sum * alpha;
        if (beta != 0) t += (int64_t)load_out<OB>(cp) * beta;
        store_out<OB>(cp, encode_int((i128)t, OB, mode));
    } else {
        i128 t = sat_mul((i128)sum, alpha);
        if (beta != 0) t = (i128)((u128)t + (u128)sat_mul(load_out<OB>(cp), beta));
        store_out<OB>(cp, encode_int(t, OB, mode));
    }
}

}  // namespace uor
