// Exact float GEMM on gfx950: C := round_once(alpha * sum_p A[i,p]*B[p,j] + beta * C[i,j])
// over f32 or f64 codes, for the reference's gemm_float_packed (crates/
// uor-matmul-gemm/src/float.rs:1824-1855) and its facades slice::gemm_float*
// (crates/uor-matmul/src/slice.rs:304-421) and raw::sgemm / dgemm
// (crates/uor-matmul/src/raw.rs:45-158).
//
// Semantics (the reference's, restated):
//  * every code decodes to an exact dyadic m * 2^x (FloatElement::decode,
//    crates/uor-matmul-core/src/alphabet.rs:905-957); a product is exact
//    (Element::mac, alphabet.rs:856-902): NaN in either operand, or an
//    infinity times a zero, gives NaN; an infinity times a nonzero gives an
//    infinity of the product's sign;
//  * the sum is exact, in a fixed-point register whose bit 0 has exponent
//    2 * (least subnormal exponent): -298 (f32), -2148 (f64)
//    (Complete<L, MIN_EXP>, acc.rs:469; complete_width, generated.rs:114-127);
//    +inf together with -inf is NaN;
//  * alpha and beta are exact i64 factors (Complete::scale, acc.rs:1028-1068):
//    0 times an infinity is NaN, a negative factor swaps the infinities; beta
//    = 0 never reads C (Linear::finish, epilogue.rs:67-95);
//  * one rounding at the end (impl_encode_into_float, acc.rs:1734-1868):
//    Nearest is round-half-even with overflow to +-inf, the other modes
//    truncate toward zero and clamp to +-MAX; an exact zero is +0; a nonzero
//    that rounds to zero keeps its sign; NaN is the canonical quiet NaN.
//
// Routes.  FLOAT_DIRECT needs no scratch and takes any input: one thread per
// output cell accumulates signed 32-bit digits into int64 slots of its own LDS
// register (carry-save; a digit slot absorbs 2^31 products before it could
// overflow), then normalises, scales, adds beta * C and encodes.  It is the
// exact fallback, not the fast route.

#include "common.hpp"

namespace uor {

// ------------------------------------------------------------ formats --

template <bool F64>
struct Fmt;
template <>
struct Fmt<false> {
    typedef uint32_t bits_t;
    static constexpr int MANT = 23, EXPO = 8, BIAS = 127;
    static constexpr int SUB_LSB = -149;  // exponent of the least subnormal
    static constexpr int RB = -298;       // register bit 0
    static constexpr int DIGITS = 24;     // 768 bits
    static constexpr uint64_t NAN_BITS = 0x7fc00000ull;
};
template <>
struct Fmt<true> {
    typedef uint64_t bits_t;
    static constexpr int MANT = 52, EXPO = 11, BIAS = 1023;
    static constexpr int SUB_LSB = -1074;
    static constexpr int RB = -2148;
    static constexpr int DIGITS = 140;  // 4480 bits
    static constexpr uint64_t NAN_BITS = 0x7ff8000000000000ull;
};

enum : int { FL_NAN = 1, FL_PINF = 2, FL_NINF = 4 };
enum : int { CLS_FINITE = 0, CLS_INF = 1, CLS_NAN = 2 };

struct Dec {
    int cls;
    int neg;
    uint64_t mant;  // finite: the integer significand (0 for a zero)
    int exp;        // finite: value = mant * 2^exp
};

// FloatElement::decode (alphabet.rs:905-957).
template <bool F64>
__host__ __device__ inline Dec decode(uint64_t bits) {
    using F = Fmt<F64>;
    const uint64_t frac = bits & ((1ull << F::MANT) - 1);
    const int be = (int)((bits >> F::MANT) & ((1u << F::EXPO) - 1));
    Dec d;
    d.neg = (int)((bits >> (F::MANT + F::EXPO)) & 1);
    if (be == (1 << F::EXPO) - 1) {
        d.cls = frac ? CLS_NAN : CLS_INF;
        d.mant = 0;
        d.exp = 0;
        return d;
    }
    d.cls = CLS_FINITE;
    if (be == 0) {
        d.mant = frac;
        d.exp = F::SUB_LSB;
    } else {
        d.mant = frac | (1ull << F::MANT);
        d.exp = be - F::BIAS - F::MANT;
    }
    return d;
}

// The flags of one product (Element::mac's non-finite cases).
__device__ inline int product_flags(const Dec &a, const Dec &b) {
    if (a.cls == CLS_NAN || b.cls == CLS_NAN) return FL_NAN;
    if (a.cls == CLS_INF || b.cls == CLS_INF) {
        if ((a.cls == CLS_FINITE && a.mant == 0) || (b.cls == CLS_FINITE && b.mant == 0)) return FL_NAN;
        return (a.neg != b.neg) ? FL_NINF : FL_PINF;
    }
    return 0;
}

// Complete::scale on the non-finite part (acc.rs:1028-1068).
__device__ inline int scale_flags(int flags, int64_t f) {
    const bool nan = (flags & FL_NAN) || ((flags & FL_PINF) && (flags & FL_NINF));
    if (nan) return flags;
    if (f == 1) return flags;
    if (f == 0) return (flags & (FL_PINF | FL_NINF)) ? FL_NAN : 0;
    if (f < 0) {
        int g = 0;
        if (flags & FL_PINF) g |= FL_NINF;
        if (flags & FL_NINF) g |= FL_PINF;
        return g;
    }
    return flags;
}

// ----------------------------------------------------- digit register --

// A register of S 32-bit digits held in int64 slots, slot q at p[q * st]
// (interleaved so that the threads of a workgroup use distinct words).
struct Reg {
    int64_t *p;
    int st;
    __device__ int64_t &operator[](int q) const { return p[q * st]; }
};

constexpr int64_t M32 = 0xffffffffll;

// R += (neg ? -1 : 1) * (hi:lo) * 2^pos, hi:lo below 2^106 (f64) or lo
// below 2^48 (f32, hi = 0).  Touches the 5 (3) digits from pos / 32.
template <bool F64>
__device__ inline void add_product(const Reg &R, uint64_t lo, uint64_t hi, int pos, bool neg) {
    const int q = pos >> 5, r = pos & 31;
    const uint64_t w0 = lo << r;
    const uint64_t w1 = r ? ((hi << r) | (lo >> (64 - r))) : hi;
    const int64_t d0 = (int64_t)(w0 & M32), d1 = (int64_t)(w0 >> 32);
    const int64_t d2 = (int64_t)(w1 & M32);
    if (neg) {
        R[q] -= d0;
        R[q + 1] -= d1;
        R[q + 2] -= d2;
    } else {
        R[q] += d0;
        R[q + 1] += d1;
        R[q + 2] += d2;
    }
    if constexpr (F64) {
        const uint64_t w2 = r ? (hi >> (64 - r)) : 0;
        const int64_t d3 = (int64_t)(w1 >> 32), d4 = (int64_t)w2;
        if (neg) {
            R[q + 3] -= d3;
            R[q + 4] -= d4;
        } else {
            R[q + 3] += d3;
            R[q + 4] += d4;
        }
    }
}

// Carry-propagate so that digits 0..S-2 lie in [0, 2^32); the top slot keeps
// the signed remainder.
template <int S>
__device__ inline void carry_mid(const Reg &R) {
    int64_t carry = 0;
    for (int q = 0; q < S - 1; ++q) {
        const int64_t v = R[q] + carry;
        R[q] = v & M32;
        carry = v >> 32;  // arithmetic shift: floor division
    }
    R[S - 1] += carry;
}

// Normalise to a magnitude in [0, 2^(32S)) with digits in [0, 2^32); returns
// true when the value is negative.  The register's headroom keeps the top
// slot's remainder at 0 or -1.
template <int S>
__device__ inline bool normalise(const Reg &R) {
    carry_mid<S>(R);
    const int64_t top = R[S - 1];
    const bool neg = top < 0;
    R[S - 1] = top & M32;
    if (neg) {
        // Two's complement over S digits: invert and add one.
        uint64_t c = 1;
        for (int q = 0; q < S; ++q) {
            const uint64_t v = (uint64_t)(~R[q] & M32) + c;
            R[q] = (int64_t)(v & M32);
            c = v >> 32;
        }
    }
    return neg;
}

template <int S>
__device__ inline void mul_small(const Reg &R, uint64_t f) {
    uint64_t carry = 0;  // below 2^64: digit * f + carry < 2^96
    for (int q = 0; q < S; ++q) {
        const u128 t = (u128)(uint64_t)R[q] * f + carry;
        R[q] = (int64_t)((uint64_t)t & M32);
        carry = (uint64_t)(t >> 32);
    }
}

// |R| (sign *neg) += (m_neg ? -1 : 1) * mag * 2^pos, exactly; mag < 2^117.
template <int S>
__device__ inline void add_signed(const Reg &R, bool *neg, u128 mag, int pos, bool m_neg) {
    if (mag == 0) return;
    const int q0 = pos >> 5, r = pos & 31;
    // mag << r as five digits.
    uint64_t dg[5];
    const u128 lo = mag << r;
    const uint64_t spill = r ? (uint64_t)((mag >> 64) >> (64 - r)) : 0;
    dg[0] = (uint64_t)lo & M32;
    dg[1] = (uint64_t)lo >> 32;
    dg[2] = (uint64_t)(lo >> 64) & M32;
    dg[3] = (uint64_t)(lo >> 96);
    dg[4] = spill;
    if (*neg == m_neg) {
        uint64_t c = 0;
        for (int q = q0; q < S; ++q) {
            const int t = q - q0;
            if (t >= 5 && c == 0) break;
            const uint64_t v = (uint64_t)R[q] + (t < 5 ? dg[t] : 0) + c;
            R[q] = (int64_t)(v & M32);
            c = v >> 32;
        }
        return;
    }
    // Opposite signs: R - M, then fix the sign if it went below zero.
    int64_t b = 0;
    for (int q = q0; q < S; ++q) {
        const int t = q - q0;
        if (t >= 5 && b == 0) break;
        const int64_t v = R[q] - (int64_t)(t < 5 ? dg[t] : 0) - b;
        R[q] = v & M32;
        b = v < 0 ? 1 : 0;
    }
    if (b) {
        uint64_t c = 1;
        for (int q = 0; q < S; ++q) {
            const uint64_t v = (uint64_t)(~R[q] & M32) + c;
            R[q] = (int64_t)(v & M32);
            c = v >> 32;
        }
        *neg = !*neg;
    }
}

__device__ inline int reg_bit(const Reg &R, int S, int i) {
    if (i < 0 || (i >> 5) >= S) return 0;
    return (int)((R[i >> 5] >> (i & 31)) & 1);
}

// impl_encode_into_float (acc.rs:1734-1868) from a magnitude register whose
// bit 0 has exponent RB.
template <bool F64, int S>
__device__ inline uint64_t encode_reg(const Reg &R, bool neg, int flags, int mode) {
    using F = Fmt<F64>;
    constexpr int MANT = F::MANT, EXPO = F::EXPO, P = MANT + 1;
    constexpr uint64_t EXPMASK = (1ull << EXPO) - 1;
    if ((flags & FL_NAN) || ((flags & FL_PINF) && (flags & FL_NINF))) return F::NAN_BITS;
    if (flags & (FL_PINF | FL_NINF)) {
        const uint64_t s = (flags & FL_NINF) ? 1 : 0;
        return (s << (MANT + EXPO)) | (EXPMASK << MANT);
    }
    int top = -1;
    for (int q = S - 1; q >= 0; --q) {
        const uint32_t d = (uint32_t)R[q];
        if (d) {
            top = 32 * q + 31 - __builtin_clz(d);
            break;
        }
    }
    if (top < 0) return 0;  // an exact zero is +0
    const int exp = F::RB + top;
    int lsb_exp = exp - (P - 1) < F::SUB_LSB ? F::SUB_LSB : exp - (P - 1);
    const int lsb = lsb_exp - F::RB;  // >= 0: RB lies below the subnormal floor
    // The P-bit window at lsb, read from three digits.
    const int q = lsb >> 5, r = lsb & 31;
    u128 w = 0;
    for (int t = 2; t >= 0; --t) w = (w << 32) | (uint64_t)(q + t < S ? (uint32_t)R[q + t] : 0u);
    uint64_t sig = (uint64_t)(w >> r) & ((1ull << P) - 1);
    int round_bit = 0, sticky = 0;
    if (lsb > 0) {
        round_bit = reg_bit(R, S, lsb - 1);
        const int below = lsb - 1;  // bits [0, below) feed the sticky bit
        const int qb = below >> 5;
        for (int t = 0; t < qb && t < S; ++t)
            if ((uint32_t)R[t]) sticky = 1;
        if (!sticky && qb < S && (below & 31)) {
            const uint32_t msk = (1u << (below & 31)) - 1;
            if ((uint32_t)R[qb] & msk) sticky = 1;
        }
    }
    const int inc = (mode == UOR_ENCODE_NEAREST) ? (round_bit && (sticky || (sig & 1))) : 0;
    sig += (uint64_t)inc;
    if (sig >> P) {
        sig >>= 1;
        lsb_exp += 1;
    }
    const uint64_t sbit = (uint64_t)(neg ? 1 : 0) << (MANT + EXPO);
    if (sig == 0) return sbit;  // rounded to zero: keeps the sign
    if ((sig >> (P - 1)) == 1) {
        const int value_exp = lsb_exp + (P - 1);
        const int biased = value_exp + F::BIAS;
        if (biased >= (int)EXPMASK) {
            if (mode == UOR_ENCODE_NEAREST) return sbit | (EXPMASK << MANT);
            return sbit | ((EXPMASK - 1) << MANT) | ((1ull << MANT) - 1);
        }
        return sbit | ((uint64_t)biased << MANT) | (sig & ((1ull << MANT) - 1));
    }
    return sbit | sig;  // subnormal
}

// ---------------------------------------------------------- arguments --

struct FArgs {
    const char *a;  // element (0,0)
    int64_t ars, acs;
    const char *b;
    int64_t brs, bcs;
    char *c;
    int64_t crs, ccs;
    uint64_t m, k, n;
    int64_t alpha, beta;
    int mode;
};

template <bool F64>
__device__ inline uint64_t load_bits(const char *base, int64_t idx) {
    if constexpr (F64) return ((const uint64_t *)base)[idx];
    else return ((const uint32_t *)base)[idx];
}

template <bool F64>
__device__ inline void store_bits(char *base, int64_t idx, uint64_t v) {
    if constexpr (F64) ((uint64_t *)base)[idx] = v;
    else ((uint32_t *)base)[idx] = (uint32_t)v;
}

// The epilogue of one cell from its normalised register: alpha, beta * C,
// encode, store.  `neg` is the sign of the register's value.
template <bool F64>
__device__ inline void finish_cell(const FArgs &F, const Reg &R, bool neg, int flags, uint64_t i,
                                   uint64_t j) {
    using Fm = Fmt<F64>;
    constexpr int S = Fm::DIGITS;
    flags = scale_flags(flags, F.alpha);
    if (F.alpha == 0) {
        for (int q = 0; q < S; ++q) R[q] = 0;
        neg = false;
    } else if (F.alpha != 1) {
        const uint64_t fa = F.alpha < 0 ? (uint64_t)0 - (uint64_t)F.alpha : (uint64_t)F.alpha;
        mul_small<S>(R, fa);
        if (F.alpha < 0) neg = !neg;
    }
    const int64_t ci = (int64_t)i * F.crs + (int64_t)j * F.ccs;
    if (F.beta != 0) {
        // AbsorbPrior: Complete::of(C) scaled by beta (acc.rs:1003-1020).
        const Dec d = decode<F64>(load_bits<F64>(F.c, ci));
        int g = 0;
        if (d.cls == CLS_NAN) g = FL_NAN;
        else if (d.cls == CLS_INF) g = d.neg ? FL_NINF : FL_PINF;
        else if (d.mant) {
            const uint64_t fb = F.beta < 0 ? (uint64_t)0 - (uint64_t)F.beta : (uint64_t)F.beta;
            add_signed<S>(R, &neg, (u128)d.mant * fb, d.exp - Fm::RB, (d.neg != 0) != (F.beta < 0));
        }
        flags |= scale_flags(g, F.beta);
    }
    store_bits<F64>(F.c, ci, encode_reg<F64, S>(R, neg, flags, F.mode));
}

// ------------------------------------------------------- direct route --

// One thread per cell of a TM x TN tile; each thread's register lives in LDS
// (S slots of 8 bytes, interleaved across the workgroup).  No thread reads
// another's register, so the kernel has no barrier.
template <bool F64, int TM, int TN>
__global__ void __launch_bounds__(TM * TN) float_direct_kernel(FArgs F, int gn) {
    using Fm = Fmt<F64>;
    constexpr int S = Fm::DIGITS, NT = TM * TN;
    __shared__ int64_t regs[S * NT];
    const int t = threadIdx.x;
    const uint64_t i = (uint64_t)(blockIdx.x / gn) * TM + t / TN;
    const uint64_t j = (uint64_t)(blockIdx.x % gn) * TN + t % TN;
    if (i >= F.m || j >= F.n) return;
    const Reg R{regs + t, NT};
    for (int q = 0; q < S; ++q) R[q] = 0;
    int flags = 0;
    const int64_t abase = (int64_t)i * F.ars, bbase = (int64_t)j * F.bcs;
    for (uint64_t p = 0; p < F.k; ++p) {
        const Dec a = decode<F64>(load_bits<F64>(F.a, abase + (int64_t)p * F.acs));
        const Dec b = decode<F64>(load_bits<F64>(F.b, (int64_t)p * F.brs + bbase));
        if (a.cls != CLS_FINITE || b.cls != CLS_FINITE) {
            flags |= product_flags(a, b);
            continue;
        }
        if (a.mant == 0 || b.mant == 0) continue;
        uint64_t lo, hi;
        if constexpr (F64) {
            lo = a.mant * b.mant;
            hi = __umul64hi(a.mant, b.mant);
        } else {
            lo = a.mant * b.mant;
            hi = 0;
        }
        add_product<F64>(R, lo, hi, a.exp + b.exp - Fm::RB, a.neg != b.neg);
        // A slot moves by below 2^32 per product: fold before 2^31 of them.
        if ((p & ((1ull << 30) - 1)) == (1ull << 30) - 1) carry_mid<S>(R);
    }
    const bool neg = normalise<S>(R);
    finish_cell<F64>(F, R, neg, flags, i, j);
}

template <bool F64>
static hipError_t launch_direct(const FArgs &F, hipStream_t s) {
    constexpr int TM = F64 ? 8 : 16, TN = F64 ? 8 : 16;
    const uint64_t gm = (F.m + TM - 1) / TM, gn = (F.n + TN - 1) / TN;
    if (gm * gn > 0x7fffffffull) return hipErrorInvalidValue;
    hipLaunchKernelGGL((float_direct_kernel<F64, TM, TN>), dim3((unsigned)(gm * gn)), dim3(TM * TN), 0, s,
                       F, (int)gn);
    return hipGetLastError();
}

}  // namespace uor

using namespace uor;

extern "C" uint64_t uor_gfx950_suggested_scratch_float(int is_f64, uint64_t m, uint64_t k,
                                                       uint64_t n) {
    (void)is_f64;
    (void)m;
    (void)k;
    (void)n;
    return 0;
}

extern "C" int uor_gfx950_gemm_float(int is_f64, const uor_view *a, const uor_view *b,
                                     const uor_view *c, int64_t alpha, int64_t beta, int encode,
                                     void *scratch, uint64_t scratch_bytes, void *stream,
                                     uor_route *route) {
    (void)scratch;
    (void)scratch_bytes;
    route_set(route, UOR_ROUTE_NONE);
    if (!valid_encode(encode)) return UOR_INVALID_ARGUMENT;
    const int elem = is_f64 ? 8 : 4;
    Placed A, B, C;
    int st = make_triple(a, elem, b, elem, c, elem, &A, &B, &C);
    if (st) return st;
    if (C.rows == 0 || C.cols == 0) return UOR_OK;
    if (((uintptr_t)A.base | (uintptr_t)B.base | (uintptr_t)C.base) & (uintptr_t)(elem - 1))
        return UOR_INVALID_ARGUMENT;
    FArgs F{A.base, A.rs, A.cs, B.base, B.rs, B.cs, C.base, C.rs, C.cs,
            A.rows, A.cols, B.cols, alpha, beta, encode};
    hipStream_t s = (hipStream_t)stream;
    UOR_HIP(is_f64 ? launch_direct<true>(F, s) : launch_direct<false>(F, s));
    if (route) {
        route->kind = A.cols == 0 ? UOR_ROUTE_EPILOGUE_ONLY : UOR_ROUTE_FLOAT_DIRECT;
        route->tile_m = route->tile_n = is_f64 ? 8 : 16;
        route->split_k = 1;
        route->launches = 1;
    }
    return UOR_OK;
}

extern "C" int uor_gfx950_slice_gemm_float_ex(int is_f64, uint64_t m, uint64_t k, uint64_t n,
                                              int64_t alpha, const void *a, uint64_t a_len,
                                              uint64_t lda, const void *b, uint64_t b_len,
                                              uint64_t ldb, int64_t beta, void *c, uint64_t c_len,
                                              uint64_t ldc, void *scratch, uint64_t scratch_bytes,
                                              void *stream) {
    // slice.rs:87 ld(): row-major strides {rs: ld, cs: 1}; encode Nearest.
    uor_view av{(void *)a, a_len, m, k, (int64_t)lda, 1};
    uor_view bv{(void *)b, b_len, k, n, (int64_t)ldb, 1};
    uor_view cv{c, c_len, m, n, (int64_t)ldc, 1};
    return uor_gfx950_gemm_float(is_f64, &av, &bv, &cv, alpha, beta, UOR_ENCODE_NEAREST, scratch,
                                 scratch_bytes, stream, nullptr);
}

// raw.rs low() / span(): the lowest offset a view reaches and its extent, or
// false when they overflow.
static bool raw_window(uint64_t rows, uint64_t cols, int64_t rs, int64_t cs, int64_t *low,
                       uint64_t *span) {
    if (rows == 0 || cols == 0) {
        *low = 0;
        *span = 0;
        return true;
    }
    int64_t r, cc, lo, hi;
    if (__builtin_mul_overflow((int64_t)(rows - 1), rs, &r)) return false;
    if (__builtin_mul_overflow((int64_t)(cols - 1), cs, &cc)) return false;
    if (__builtin_add_overflow(r < 0 ? r : 0, cc < 0 ? cc : 0, &lo)) return false;
    if (__builtin_add_overflow(r > 0 ? r : 0, cc > 0 ? cc : 0, &hi)) return false;
    int64_t ext;
    if (__builtin_sub_overflow(hi, lo, &ext)) return false;
    *low = lo;
    *span = (uint64_t)ext + 1;
    return true;
}

static int raw_gemm(int is_f64, uint64_t m, uint64_t k, uint64_t n, int64_t alpha, const void *a,
                    int64_t rsa, int64_t csa, const void *b, int64_t rsb, int64_t csb, int64_t beta,
                    void *c, int64_t rsc, int64_t csc, void *scratch, uint64_t scratch_bytes,
                    void *stream) {
    // raw_gemm (raw.rs:98-158): m == 0 or n == 0 returns; a view or triple
    // the safe API would reject is a silent no-op.
    if (m == 0 || n == 0) return UOR_OK;
    const int64_t elem = is_f64 ? 8 : 4;
    int64_t la, lb, lc;
    uint64_t sa, sb, sc;
    if (!raw_window(m, k, rsa, csa, &la, &sa) || !raw_window(k, n, rsb, csb, &lb, &sb) ||
        !raw_window(m, n, rsc, csc, &lc, &sc))
        return UOR_OK;
    uor_view av{(void *)((const char *)a + la * elem), sa, m, k, rsa, csa};
    uor_view bv{(void *)((const char *)b + lb * elem), sb, k, n, rsb, csb};
    uor_view cv{(void *)((char *)c + lc * elem), sc, m, n, rsc, csc};
    const int st = uor_gfx950_gemm_float(is_f64, &av, &bv, &cv, alpha, beta, UOR_ENCODE_NEAREST,
                                         scratch, scratch_bytes, stream, nullptr);
    return st >= UOR_HIP_ERROR ? st : UOR_OK;
}

extern "C" int uor_gfx950_sgemm(uint64_t m, uint64_t k, uint64_t n, int64_t alpha, const float *a,
                                int64_t rsa, int64_t csa, const float *b, int64_t rsb, int64_t csb,
                                int64_t beta, float *c, int64_t rsc, int64_t csc, void *scratch,
                                uint64_t scratch_bytes, void *stream) {
    return raw_gemm(0, m, k, n, alpha, a, rsa, csa, b, rsb, csb, beta, c, rsc, csc, scratch,
                    scratch_bytes, stream);
}

extern "C" int uor_gfx950_dgemm(uint64_t m, uint64_t k, uint64_t n, int64_t alpha, const double *a,
                                int64_t rsa, int64_t csa, const double *b, int64_t rsb, int64_t csb,
                                int64_t beta, double *c, int64_t rsc, int64_t csc, void *scratch,
                                uint64_t scratch_bytes, void *stream) {
    return raw_gemm(1, m, k, n, alpha, a, rsa, csa, b, rsb, csb, beta, c, rsc, csc, scratch,
                    scratch_bytes, stream);
}
