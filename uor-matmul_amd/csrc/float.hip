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
//
// FLOAT_CRT (when the scratch offer holds its planes and k <= 2^17) runs the
// products on int8 MFMA through a residue number system:
//  1. line statistics: for every row of A and column of B, the exponent of
//     its lowest set bit (lo), its width in bits (top - lo), an upper bound
//     of log2 of its L1 norm at that scale, and whether it holds a
//     non-finite code.  Row i of A is then the integer vector
//     alpha_ip = +-m_ip * 2^(x_ip - lo_i) of at most `width` bits;
//  2. a plan kernel picks, on the device, the fewest moduli whose product M
//     bounds every reconstructed sum X_ij = sum_p alpha_ip * beta_pj with
//     |X| < M / 2 (|X| <= ||alpha_i||_1 * max|beta_j| and symmetrically);
//  3. residue planes: balanced int8 residues of alpha and beta per modulus;
//  4. one batched int8 MFMA GEMM (grid z = modulus) on the direct-to-LDS
//     pipeline; its epilogue reduces each exact i32 sum mod p to a byte;
//  5. the finish kernel reconstructs X_ij by the CRT with a rounded quotient
//     (exact: |X| stays 2^-21 M away from M / 2), places X * 2^(lo_i + lo_j)
//     into the same digit register as the direct route, and runs the same
//     alpha / beta / encode epilogue.  Rows or columns wider than WIDE_BITS
//     and non-finite lines take the direct loop inside this kernel, cell by
//     cell, so every input is exact on either route and the bytes never
//     depend on the offer.

#include <algorithm>

#include "mfma_dl.hpp"
#include "crt_tables.hpp"

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

// Normalise to a magnitude with digits in [0, 2^32); returns true when the
// value is negative.  Only slots [lo, hi] may be nonzero (the others stay
// zero); slot hi's headroom keeps its remainder at 0 or -1.
template <int S>
__device__ inline bool normalise(const Reg &R, int lo = 0, int hi = S - 1) {
    int64_t carry = 0;
    for (int q = lo; q < hi; ++q) {
        const int64_t v = R[q] + carry;
        R[q] = v & M32;
        carry = v >> 32;  // arithmetic shift: floor division
    }
    const int64_t top = R[hi] + carry;
    const bool neg = top < 0;
    R[hi] = top & M32;
    if (neg) {
        // Two's complement over [lo, hi] (the zero digits below lo pass the
        // +1 through unchanged): invert and add one.
        uint64_t c = 1;
        for (int q = lo; q <= hi; ++q) {
            const uint64_t v = (uint64_t)(~R[q] & M32) + c;
            R[q] = (int64_t)(v & M32);
            c = v >> 32;
        }
    }
    return neg;
}

// R *= f over slots [lo, hi]; the caller leaves 64 bits of headroom above
// the value inside the window.
template <int S>
__device__ inline void mul_small(const Reg &R, uint64_t f, int lo = 0, int hi = S - 1) {
    uint64_t carry = 0;  // below 2^64: digit * f + carry < 2^96
    for (int q = lo; q <= hi; ++q) {
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
__device__ inline uint64_t encode_reg(const Reg &R, bool neg, int flags, int mode, int lo = 0,
                                      int hi = S - 1) {
    using F = Fmt<F64>;
    constexpr int MANT = F::MANT, EXPO = F::EXPO, P = MANT + 1;
    constexpr uint64_t EXPMASK = (1ull << EXPO) - 1;
    if ((flags & FL_NAN) || ((flags & FL_PINF) && (flags & FL_NINF))) return F::NAN_BITS;
    if (flags & (FL_PINF | FL_NINF)) {
        const uint64_t s = (flags & FL_NINF) ? 1 : 0;
        return (s << (MANT + EXPO)) | (EXPMASK << MANT);
    }
    int top = -1;
    for (int q = hi; q >= lo; --q) {
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
        for (int t = lo; t < qb && t < S; ++t)
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
// Slots outside [lo, hi] are zero and stay so until beta * C is added
// (which then widens the window to the whole register).
template <bool F64>
__device__ inline void finish_cell(const FArgs &F, const Reg &R, bool neg, int flags, uint64_t i,
                                   uint64_t j, int lo = 0, int hi = Fmt<F64>::DIGITS - 1) {
    using Fm = Fmt<F64>;
    constexpr int S = Fm::DIGITS;
    flags = scale_flags(flags, F.alpha);
    if (F.alpha == 0) {
        for (int q = lo; q <= hi; ++q) R[q] = 0;
        neg = false;
    } else if (F.alpha != 1) {
        const uint64_t fa = F.alpha < 0 ? (uint64_t)0 - (uint64_t)F.alpha : (uint64_t)F.alpha;
        mul_small<S>(R, fa, lo, hi);
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
        lo = 0;
        hi = S - 1;
    }
    store_bits<F64>(F.c, ci, encode_reg<F64, S>(R, neg, flags, F.mode, lo, hi));
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


// --------------------------------------------------------- CRT route --

constexpr int WIDE_BITS = 160;  // the widest slice (2W + log2(k S) fits 49 moduli)
constexpr int CRT_BK_MAX = 1 << 17;  // i32 MFMA sums stay exact: 2^14 * k < 2^31

enum : int32_t { LS_DIRTY = 1, LS_WIDE = 2, LS_EMPTY = 4 };

struct LineStat {
    int32_t lo;     // exponent of the lowest set bit over the line's finite nonzeros
    int32_t width;  // top - lo (bits of the largest aligned integer)
    float l1;       // upper bound of log2(sum |aligned integers|); -1e30 when empty
    int32_t flags;
};

struct CrtHdr {
    int32_t nmod;     // moduli in use (0: no residue work)
    int32_t crt_off;  // 1: every cell takes the direct loop
    int32_t need;     // the bound B used: |X| < 2^B (per diagonal when sliced)
    int32_t sa, sb;   // slices per A row / B column (1: unsliced)
    int32_t w;        // slice width in bits (sliced plans)
    int32_t pad[58];
};

// The trimmed significand and exponent of a finite nonzero: m odd.
__device__ inline void trim(const Dec &d, uint64_t *m, int *x) {
    const int tz = __builtin_ctzll(d.mant);
    *m = d.mant >> tz;
    *x = d.exp + tz;
}

__device__ inline int bitlen64(uint64_t v) { return 64 - __builtin_clzll(v); }

// Statistics of `lines` lines of `len` elements: element e of line t at
// base + t * s_line + e * s_elem.  LPB lines per workgroup, thread t on line
// t % LPB at elements t / LPB, + NT / LPB, ...: LPB = 1 (s_elem == 1) puts
// the threads along one line; LPB = 64, 16 or 4 (s_line == 1) puts a wave
// across LPB neighbouring lines, one LPB-element row segment per lane group;
// LPB = 16 with 256 threads is for the other strides.  One pass: each thread
// keeps its top bit hi and the sum of its |aligned integers| scaled by
// 2^-hi (every term at most 1), rescaled by a power of two when hi rises,
// and the threads' pairs combine the same way.
template <bool F64, int LPB, int NT = 256>
__global__ void __launch_bounds__(NT) line_stats_kernel(const char *base, int64_t s_line,
                                                        int64_t s_elem, uint64_t lines,
                                                        uint64_t len, LineStat *out) {
    constexpr int TPL = NT / LPB;  // threads per line
    constexpr int U = 4;           // loads in flight per thread
    __shared__ int s_lo[NT], s_hi[NT], s_fl[NT];
    __shared__ double s_sum[NT];
    const int t = threadIdx.x;
    const int tl = t % LPB, te = t / LPB;
    const uint64_t line = (uint64_t)blockIdx.x * LPB + tl;
    const bool live = line < lines;
    int lo = 1 << 30, hi = -(1 << 30), fl = 0;
    double sum = 0;
    if (live) {
        for (uint64_t e0 = te; e0 < len; e0 += (uint64_t)TPL * U) {
            uint64_t v[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint64_t e = e0 + (uint64_t)u * TPL;
                v[u] = e < len ? load_bits<F64>(base, (int64_t)line * s_line + (int64_t)e * s_elem) : 0;
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const Dec d = decode<F64>(v[u]);
                if (d.cls != CLS_FINITE) {
                    fl |= LS_DIRTY;
                    continue;
                }
                if (!d.mant) continue;
                uint64_t m;
                int x;
                trim(d, &m, &x);
                const int top = x + bitlen64(m);
                lo = min(lo, x);
                if (top > hi) {
                    sum = ldexp(sum, hi - top);
                    hi = top;
                }
                sum += ldexp((double)m, x - hi);
            }
        }
    }
    s_lo[t] = lo;
    s_hi[t] = hi;
    s_fl[t] = fl;
    s_sum[t] = sum;
    __syncthreads();
    for (int w = TPL / 2; w >= 1; w >>= 1) {
        if (te < w) {
            const int o = t + LPB * w;
            const int h0 = s_hi[t], h1 = s_hi[o], h = max(h0, h1);
            s_sum[t] = ldexp(s_sum[t], h0 - h) + ldexp(s_sum[o], h1 - h);
            s_hi[t] = h;
            s_lo[t] = min(s_lo[t], s_lo[o]);
            s_fl[t] |= s_fl[o];
        }
        __syncthreads();
    }
    lo = s_lo[tl];
    hi = s_hi[tl];
    fl = s_fl[tl];
    if (te == 0 && live) {
        LineStat st;
        if (hi <= lo) {
            st.lo = 0;
            st.width = 0;
            st.l1 = -1e30f;
            st.flags = fl | LS_EMPTY;
        } else {
            st.lo = lo;
            st.width = hi - lo;
            // Rounding of the double sum is below 2^-30 relative for any
            // reachable length (the rescalings are exact); terms that
            // underflowed are below 2^-900 each.
            const double s = s_sum[tl] * (1.0 + 0x1p-28) + (double)len * 0x1p-900;
            st.l1 = (float)(log2(s) + (double)(hi - lo) + 1e-6);
            st.flags = fl | (st.width > WIDE_BITS ? LS_WIDE : 0);
        }
        out[line] = st;
    }
}

// The plan, on the device.  Unsliced (every line at most WIDE_BITS wide): the
// bound B (|X_ij| < 2^B for every cell) from the line widths and L1 bounds.
// Sliced: every aligned integer is cut into S slices of W bits, X =
// sum_{s,t} 2^{W(s+t)} alpha^(s) beta^(t), and the slice pairs of one diagonal
// d = s + t form one GEMM, whose sum is below min(S_A, S_B) * k * 2^(2W).
// Then the fewest moduli whose capacity covers B; crt_off when the offer
// holds fewer planes or slices than the data needs.
__global__ void __launch_bounds__(256) crt_plan_kernel(const LineStat *ra, uint64_t m,
                                                       const LineStat *cb, uint64_t n, uint64_t k,
                                                       int nm_alloc, int sa_cap, int sb_cap,
                                                       CrtHdr *h) {
    __shared__ float s_w[4][256];
    const int t = threadIdx.x;
    float wa = -1e30f, la = -1e30f, wb = -1e30f, lb = -1e30f;
    for (uint64_t i = t; i < m; i += 256) {
        const LineStat s = ra[i];
        if (s.flags & LS_EMPTY) continue;
        wa = fmaxf(wa, (float)s.width);
        la = fmaxf(la, s.l1);
    }
    for (uint64_t j = t; j < n; j += 256) {
        const LineStat s = cb[j];
        if (s.flags & LS_EMPTY) continue;
        wb = fmaxf(wb, (float)s.width);
        lb = fmaxf(lb, s.l1);
    }
    s_w[0][t] = wa;
    s_w[1][t] = la;
    s_w[2][t] = wb;
    s_w[3][t] = lb;
    __syncthreads();
    for (int w = 128; w >= 1; w >>= 1) {
        if (t < w)
            for (int q = 0; q < 4; ++q) s_w[q][t] = fmaxf(s_w[q][t], s_w[q][t + w]);
        __syncthreads();
    }
    if (t != 0) return;
    wa = s_w[0][0];
    la = s_w[1][0];
    wb = s_w[2][0];
    lb = s_w[3][0];
    CrtHdr r{};
    r.sa = r.sb = 1;
    if (wa < 0 || wb < 0) {  // no cell has a nonzero product
        *h = r;
        return;
    }
    int lk = 0;
    while ((1ull << lk) < k) ++lk;
    int need;
    if (wa <= WIDE_BITS && wb <= WIDE_BITS) {
        const double b = fmin(fmin((double)la + wb, (double)wa + lb), (double)wa + wb + lk);
        need = (int)ceil(b + 1e-5);
    } else {
        const int iwa = (int)wa, iwb = (int)wb;
        int sa = (iwa + WIDE_BITS - 1) / WIDE_BITS, sb = (iwb + WIDE_BITS - 1) / WIDE_BITS;
        if (sa < 1) sa = 1;
        if (sb < 1) sb = 1;
        const int w = max((iwa + sa - 1) / sa, (iwb + sb - 1) / sb);
        sa = max(1, (iwa + w - 1) / w);
        sb = max(1, (iwb + w - 1) / w);
        int ls = 0;
        while ((1 << ls) < min(sa, sb)) ++ls;
        need = 2 * w + lk + ls;
        r.sa = sa;
        r.sb = sb;
        r.w = w;
    }
    int nm = 0;
    while (nm < CRT_NMAX && crt_cap[nm] < need) ++nm;
    r.need = need;
    if (crt_cap[nm] < need || nm > nm_alloc || r.sa > sa_cap || r.sb > sb_cap) {
        r.crt_off = 1;
        r.nmod = 0;
    } else {
        r.nmod = nm;
    }
    *h = r;
}

// Balanced int8 residue of +-m * 2^s modulo crt_mod[l] (s < 256); md is
// +-m as a double (exact: m < 2^53).  Every modulus but crt_mod[0] = 256 is
// odd, so a quotient x / p is never a half-integer: its distance from one is
// at least 1 / (2p) >= 2^-9, and rint of x * (1/p) is the nearest integer q
// whenever the product's error is below that; x - q p, an integer in
// [-(p-1)/2, (p-1)/2], is then the balanced residue, exact out of one fma.
// An f32 significand (< 2^24) keeps x = +-m (2^s mod p) below 2^32 (error of
// x * (1/p) below 2^-24); an f64 one is first reduced to r = +-m - q' p with
// q' = rint(md * (1/p)) off by at most one (error below 2^-3), so |r| < 3p/2,
// and x = r (2^s mod p), below 2^17, is then reduced in single precision
// (error below 2^-10).
template <bool F64>
__device__ inline int residue(uint64_t m, double md, int s, bool neg, int l, const uint8_t *pow2) {
    const uint32_t w = pow2[l * 256 + s];
    if (l == 0) {
        int b = (int)(((uint32_t)m * w) & 255);
        b = b >= 128 ? b - 256 : b;
        if (neg) b = -b;
        return b == 128 ? -128 : b;  // p = 256: 128 and -128 are one residue
    }
    const int p = crt_mod[l];
    if constexpr (!F64) {
        const double x = md * (double)w;
        return (int)fma(-rint(x * crt_invp[l]), (double)p, x);
    } else {
        const double r = fma(-rint(md * crt_invp[l]), (double)p, md);
        const float x = (float)r * (float)w;
        return (int)fmaf(-rintf(x * crt_invpf[l]), (float)p, x);
    }
}

// Residue planes.  A (ROWS_A): plane l holds m rows of S_A max * kp bytes,
// slice s of row i at columns [s * kp, s * kp + k).  B: plane l holds
// S_B max * kp rows of np bytes, slice t at rows [(S_B max - 1 - t) * kp, ...)
// (reversed, so that the slice pairs of one diagonal are one contiguous k
// range of both operands).  Padding (k <= p < kp, j >= n) is zero.  Element
// (r, c) of the source is at src + r * s_r + c * s_c, its line statistics at
// st[ROWS_A ? r : c].  Each thread writes 4 consecutive plane bytes per step
// of a grid-stride loop over the slices the plan uses.
template <bool F64, bool ROWS_A>
__global__ void __launch_bounds__(256) residue_kernel(const char *src, int64_t s_r, int64_t s_c,
                                                      uint64_t rows, uint64_t cols, uint64_t kp,
                                                      uint64_t np, int s_max, const LineStat *st,
                                                      const CrtHdr *h, int8_t *planes,
                                                      uint64_t plane_bytes) {
    __shared__ uint32_t pow2w[CRT_NMAX * 64];
    const int nmod = h->nmod;
    const int ns = ROWS_A ? h->sa : h->sb;
    const int w = (h->sa > 1 || h->sb > 1) ? h->w : 0;  // 0: unsliced
    const uint32_t *tab = (const uint32_t *)&crt_pow2[0][0];
    for (int q = threadIdx.x; q < nmod * 64; q += 256) pow2w[q] = tab[q];
    __syncthreads();
    if (nmod == 0) return;
    const uint8_t *pow2 = (const uint8_t *)pow2w;
    // Logical chunk space: (slice, R, C / 4) with (R, C) = (m, kp) for A and
    // (kp, np) for B; source coordinates (row, col) follow.
    const uint64_t R = ROWS_A ? rows : kp, C = ROWS_A ? kp : np;
    const uint64_t chunks = C / 4, per_slice = R * chunks, total = (uint64_t)ns * per_slice;
    for (uint64_t idx = (uint64_t)blockIdx.x * 256 + threadIdx.x; idx < total;
         idx += (uint64_t)gridDim.x * 256) {
        const int sl = (int)(idx / per_slice);
        const uint64_t rem = idx % per_slice;
        const uint64_t r = rem / chunks, c0 = (rem % chunks) * 4;
        uint64_t mm[4];
        int ss[4];
        bool ok[4], ng[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            // Source element: A (r, c0 + e), B (p = r, j = c0 + e).
            const uint64_t sr = r, sc = c0 + e;
            ok[e] = false;
            ng[e] = false;
            mm[e] = 0;
            ss[e] = 0;
            if (sr >= rows || sc >= cols) continue;
            const LineStat ls = st[ROWS_A ? sr : sc];
            if (ls.flags & LS_EMPTY) continue;
            const Dec d = decode<F64>(load_bits<F64>(src, (int64_t)sr * s_r + (int64_t)sc * s_c));
            if (d.cls != CLS_FINITE || !d.mant) continue;
            uint64_t m;
            int x;
            trim(d, &m, &x);
            const int sh = x - ls.lo;  // the aligned integer is m * 2^sh
            if (w == 0) {
                mm[e] = m;
                ss[e] = sh;
            } else {
                // Bits [w * sl, w * (sl + 1)) of m * 2^sh.
                const int lo_bit = w * sl, hi_bit = lo_bit + w, bl = bitlen64(m);
                if (sh >= hi_bit || sh + bl <= lo_bit) continue;
                if (sh >= lo_bit) {
                    const int keep = hi_bit - sh;  // bits of m inside the slice
                    mm[e] = keep >= 64 ? m : (m & ((1ull << keep) - 1));
                    ss[e] = sh - lo_bit;
                } else {
                    mm[e] = m >> (lo_bit - sh);  // below 2^53 <= 2^w: no upper mask
                    ss[e] = 0;
                }
                if (!mm[e]) continue;
            }
            ng[e] = d.neg;
            ok[e] = true;
        }
        int8_t *dst = ROWS_A ? planes + r * ((uint64_t)s_max * kp) + (uint64_t)sl * kp + c0
                             : planes + ((uint64_t)(s_max - 1 - sl) * kp + r) * np + c0;
        double md[4];  // +-m (0 for a cell with no residue: every residue 0)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if (!ok[e]) mm[e] = 0, ng[e] = false;
            md[e] = ng[e] ? -(double)mm[e] : (double)mm[e];
        }
        for (int l = 0; l < nmod; ++l) {
            uint32_t wd = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int v = residue<F64>(mm[e], md[e], ss[e], ng[e], l, pow2);
                wd |= (uint32_t)(uint8_t)(int8_t)v << (8 * e);
            }
            *(uint32_t *)(dst + (uint64_t)l * plane_bytes) = wd;
        }
    }
}

struct ResOut {
    uint8_t *y;  // diagonal d, modulus l at y + (d * nm + l) * y_plane: m x n bytes
    uint64_t y_plane;
    int nm;      // moduli the planes are laid out for
    int8_t *ap, *bp;  // residue planes: A [l][m][sa_max * kp], B [l][sb_max * kp][np]
    uint64_t a_plane, b_plane;
    uint64_t kp, np;
    int sa_max, sb_max;
    const CrtHdr *h;
    int accumulate;  // 1: add the planes' residues to y's (a later k chunk)
};

// One (diagonal, modulus) per grid (y, z): the exact i32 sum over the
// diagonal's slice pairs -- one contiguous k range of both operands -- reduced
// mod p into a byte per cell.
template <int BM, int BN, int WM, int WN, bool PF>
__global__ void __launch_bounds__(64 * WM * WN, 1)
residue_gemm_kernel(uint64_t m, uint64_t n, int gm, int gn, ResOut R) {
    constexpr int FM = BM / WM / 32, FN = BN / WN / 32;
    using L = DlLayout<BM, BN>;
    const int d = blockIdx.y, l = blockIdx.z;
    const CrtHdr hd = *R.h;
    if (l >= hd.nmod || d >= hd.sa + hd.sb - 1) return;
    const int a0 = max(0, d - hd.sb + 1), a1 = min(d, hd.sa - 1);
    const uint64_t K = (uint64_t)(a1 - a0 + 1) * R.kp;
    Opnd A{R.ap + (uint64_t)l * R.a_plane + (uint64_t)a0 * R.kp, (int64_t)((uint64_t)R.sa_max * R.kp), 1, m};
    Opnd B{R.bp + (uint64_t)l * R.b_plane + (uint64_t)(R.sb_max - 1 - d + a0) * R.kp * R.np, 1,
           (int64_t)R.np, n};
    __shared__ __attribute__((aligned(16))) char lds[L::BYTES];
    char *st0 = lds, *st1 = lds + L::A_BYTES, *st2 = lds + 2 * L::A_BYTES, *st3 = lds + 3 * L::A_BYTES;
    int tm, tn;
    tile_of(gm, gn, &tm, &tn);
    const uint64_t m0 = (uint64_t)tm * BM, n0 = (uint64_t)tn * BN;
    const int nk = (int)(K / DL_BK);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int half = lane >> 5, l32 = lane & 31;
    v16i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = v16i{};
    if constexpr (PF) dl_mainloop_pf<BM, BN, WM, WN>(A, B, m0, n0, 0, nk, st0, st1, st2, st3, acc);
    else dl_mainloop<BM, BN, WM, WN>(A, B, m0, n0, 0, nk, st0, st1, st2, st3, acc);
    const int p = crt_mod[l];
    const double invp = crt_invp[l];
    uint8_t *y = R.y + ((uint64_t)d * R.nm + l) * R.y_plane;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const uint64_t col = n0 + wn * (BN / WN) + 32 * j + l32;
            const uint64_t rbase = m0 + wm * (BM / WM) + 32 * i;
            if (col >= n) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint64_t row = rbase + 8 * (r >> 2) + 4 * half + (r & 3);
                if (row >= m) continue;
                const int v = acc[i][j][r];
                int q;
                if (l == 0) {
                    q = v & 255;
                } else {
                    q = v - p * (int)floor((double)v * invp);
                    if (q < 0) q += p;
                    if (q >= p) q -= p;
                }
                if (R.accumulate) {
                    q += y[row * n + col];
                    if (q >= p) q -= p;
                }
                y[row * n + col] = (uint8_t)q;
            }
        }
    }
}

// The CRT reconstruction of X_ij in ND 16-bit digits: |X| into D[] (each in
// [0, 2^16)), returns true when X < 0.  The sum over the moduli runs in
// 32-bit digits held in doubles: each slot adds a residue (|c| <= 129) times
// a 32-bit digit of M / p_l by one fma, and 49 such products stay below
// 2^46 in magnitude, so every partial sum is an exact integer.  The quotient round(sum c_l /
// p_l) is exact in a double because |X| / M stays 2^-21 away from 1/2.
// Digits past the tables' CRT_ND (a 16-bit digit count of ND = 2 CRT_ND - 1
// or 2 CRT_ND, room for an alpha) are zero in M and every M / p_l.
// A chain of reconstructions over several plane sets (the window finish's
// diagonals) passes `pre`: on entry (have_pre) the first G plane bytes of this
// set, already loaded; on exit those of `ynext` (if not null), loaded while
// this set's last group is summed instead of re-reading its own last plane.
template <int ND, int G = 8>
__device__ inline bool crt16(const uint8_t *y, uint64_t y_plane, uint64_t cell, int nmod,
                             uint32_t (&D)[ND], const uint8_t *ynext = nullptr, int *pre = nullptr,
                             bool have_pre = false) {
    constexpr int NW = (ND + 1) / 2;                   // 32-bit digits
    constexpr int NT = NW < CRT_ND ? NW : CRT_ND;      // those the tables hold
    double sl[NT];
#pragma unroll
    for (int e = 0; e < NT; ++e) sl[e] = 0;
    double f = 0;
    const double(*Ml)[CRT_ND] = crt_Ml[nmod - 1];
    const uint32_t *inv = crt_inv[nmod - 1];
    // G planes' bytes at a time, the next group's loads issued before this
    // group's arithmetic (clamped to the last plane, so every load is in
    // bounds and none is conditional).  The groups stay a loop: unrolled, the
    // compiler keeps every group's residues and table rows live at once (over
    // 200 VGPRs).
    // Plane l of the cell at y + l * y_plane + cell: the plane offset is
    // uniform and formed on the scalar unit (readfirstlane), so a load costs
    // one 64-bit add per lane instead of a 64-bit multiply-add.
    auto plane_byte = [&](const uint8_t *base, int l) -> int {
        const uint64_t off = (uint64_t)__builtin_amdgcn_readfirstlane(l) * y_plane;
        return base[off + cell];
    };
    int nxt[G];
#pragma unroll
    for (int u = 0; u < G; ++u) nxt[u] = have_pre ? pre[u] : plane_byte(y, min(u, nmod - 1));
#pragma unroll 1
    for (int l0 = 0; l0 < nmod; l0 += G) {
        int yb[G];
#pragma unroll
        for (int u = 0; u < G; ++u) yb[u] = nxt[u];
        if (l0 + G < nmod || !ynext) {
#pragma unroll
            for (int u = 0; u < G; ++u) nxt[u] = plane_byte(y, min(l0 + G + u, nmod - 1));
        } else {
#pragma unroll
            for (int u = 0; u < G; ++u) nxt[u] = plane_byte(ynext, min(u, nmod - 1));
        }
#pragma unroll
        for (int u = 0; u < G; ++u) {
            const int l = l0 + u;
            if (l < CRT_NMAX && l < nmod) {
                // c = yb * (M / p_l)^-1 mod p_l, any representative: x - p
                // rint(x / p), |c| <= p / 2 + 1 (x < 2^16, so x * (1/p) errs
                // far below the rounding's half), exact out of one fma.
                const double x = (double)(int)__umul24((uint32_t)yb[u], inv[l]);
                const double cd = fma(-rint(x * crt_invp[l]), crt_modd[l], x);
                f += cd * crt_invp[l];
#pragma unroll
                for (int e = 0; e < NT; ++e) sl[e] = fma(cd, Ml[l][e], sl[e]);
            }
        }
    }
    if (pre) {
#pragma unroll
        for (int u = 0; u < G; ++u) pre[u] = nxt[u];
    }
    // X = sum - q M in two's complement over NW 32-bit digits (q of either
    // sign): v below 2^47 in magnitude, its floor division by 2^32 and
    // remainder exact.
    const double q = floor(f + 0.5);
    double carry = 0;
    uint32_t W[NW];
#pragma unroll
    for (int e = 0; e < NW; ++e) {
        const double v = (e < NT ? fma(-q, crt_M[nmod][e < NT ? e : 0], sl[e < NT ? e : 0]) : 0.0) + carry;
        const double hi = floor(v * 0x1p-32);
        W[e] = (uint32_t)fma(-hi, 0x1p32, v);
        carry = hi;
    }
#pragma unroll
    for (int d = 0; d < ND; ++d) D[d] = (W[d / 2] >> (16 * (d % 2))) & 0xffff;
    const bool neg = carry < 0;
    if (neg) {
        uint32_t c = 1;
#pragma unroll
        for (int d = 0; d < ND; ++d) {
            const uint32_t v = (~D[d] & 0xffff) + c;
            D[d] = v & 0xffff;
            c = v >> 16;
        }
    }
    return neg;
}

// impl_encode_into_float (acc.rs:1734-1868) from a magnitude in N 16-bit
// digits D[] whose bit 0 has exponent E, all in registers: the same rounding
// as encode_reg, with every digit picked by comparison instead of indexing.
template <bool F64, int N>
__device__ inline uint64_t encode16(const uint32_t (&D)[N], int E, bool neg, int mode) {
    using F = Fmt<F64>;
    constexpr int MANT = F::MANT, EXPO = F::EXPO, P = MANT + 1;
    constexpr uint64_t EXPMASK = (1ull << EXPO) - 1;
    int top = -1;
#pragma unroll
    for (int t = 0; t < N; ++t)
        if (D[t]) top = 16 * t + 31 - __builtin_clz(D[t]);
    if (top < 0) return 0;  // an exact zero is +0
    const int exp = E + top;
    int lsb_exp = exp - (P - 1) < F::SUB_LSB ? F::SUB_LSB : exp - (P - 1);
    const int lsb = lsb_exp - E;
    uint64_t sig;
    int round_bit = 0, sticky = 0;
    if (lsb <= 0) {
        // Every bit of X lies at or above the output's LSB: X < 2^P.
        uint64_t x = 0;
#pragma unroll
        for (int t = 0; t < N && t < 4; ++t) x |= (uint64_t)D[t] << (16 * t);
        sig = x << (-lsb);
    } else {
        const int q = lsb >> 4, r = lsb & 15;
        uint64_t d0 = 0, d1 = 0, d2 = 0, d3 = 0, d4 = 0;
        const int rb = lsb - 1, qb = rb >> 4;
        const uint32_t below = (1u << (rb & 15)) - 1;
#pragma unroll
        for (int t = 0; t < N; ++t) {
            const uint64_t v = D[t];
            d0 = t == q ? v : d0;
            d1 = t == q + 1 ? v : d1;
            d2 = t == q + 2 ? v : d2;
            d3 = t == q + 3 ? v : d3;
            d4 = t == q + 4 ? v : d4;
            if (t == qb) {
                round_bit = (int)((v >> (rb & 15)) & 1);
                if (v & below) sticky = 1;
            }
            if (t < qb && v) sticky = 1;
        }
        const uint64_t lo = d0 | (d1 << 16) | (d2 << 32) | (d3 << 48);
        sig = ((lo >> r) | (r ? (d4 << (64 - r)) : 0)) & ((1ull << P) - 1);
    }
    const int inc = (mode == UOR_ENCODE_NEAREST) ? (round_bit && (sticky || (sig & 1))) : 0;
    sig += (uint64_t)inc;
    if (sig >> P) {
        sig >>= 1;
        lsb_exp += 1;
    }
    const uint64_t sbit = (uint64_t)(neg ? 1 : 0) << (MANT + EXPO);
    if (sig == 0) return sbit;
    if ((sig >> (P - 1)) == 1) {
        const int biased = lsb_exp + (P - 1) + F::BIAS;
        if (biased >= (int)EXPMASK) {
            if (mode == UOR_ENCODE_NEAREST) return sbit | (EXPMASK << MANT);
            return sbit | ((EXPMASK - 1) << MANT) | ((1ull << MANT) - 1);
        }
        return sbit | ((uint64_t)biased << MANT) | (sig & ((1ull << MANT) - 1));
    }
    return sbit | sig;
}

// The direct loop of one cell (any input), into the zeroed register R.
template <bool F64>
__device__ inline int direct_cell(const FArgs &F, const Reg &R, uint64_t i, uint64_t j) {
    using Fm = Fmt<F64>;
    constexpr int S = Fm::DIGITS;
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
        if ((p & ((1ull << 30) - 1)) == (1ull << 30) - 1) carry_mid<S>(R);
    }
    return flags;
}

// The flags of one cell: only the non-finite pairs matter.
template <bool F64>
__device__ inline int flags_cell(const FArgs &F, uint64_t i, uint64_t j) {
    int flags = 0;
    const int64_t abase = (int64_t)i * F.ars, bbase = (int64_t)j * F.bcs;
    for (uint64_t p = 0; p < F.k; ++p) {
        const Dec a = decode<F64>(load_bits<F64>(F.a, abase + (int64_t)p * F.acs));
        const Dec b = decode<F64>(load_bits<F64>(F.b, (int64_t)p * F.brs + bbase));
        if (a.cls != CLS_FINITE || b.cls != CLS_FINITE) flags |= product_flags(a, b);
    }
    return flags;
}

// The cells the register epilogue takes: an unsliced plan, no non-finite
// code on the cell's lines, beta = 0 and 0 < |alpha| < 2^16.  Decided from
// the plan and the line statistics only (never from C, which the fast kernel
// overwrites), so the two finish kernels split the cells exactly.
__device__ inline bool fast_cell(const FArgs &F, const CrtHdr &hd, const LineStat &sa,
                                 const LineStat &sb) {
    const uint64_t fa = F.alpha < 0 ? (uint64_t)0 - (uint64_t)F.alpha : (uint64_t)F.alpha;
    return !hd.crt_off && hd.sa == 1 && hd.sb == 1 && !((sa.flags | sb.flags) & LS_DIRTY) &&
           F.beta == 0 && fa != 0 && fa < 65536;
}

// The register epilogue of one fast cell: reconstruct, scale by alpha,
// encode, store.
template <bool F64, int ND>
__device__ inline void crt_fast_cell(const FArgs &F, const LineStat &sa, const LineStat &sb,
                                     int nmod, const uint8_t *y, uint64_t y_plane, uint64_t i,
                                     uint64_t j) {
    uint32_t D[ND + 1];
    bool neg = false;
    if (nmod > 0 && !((sa.flags | sb.flags) & LS_EMPTY)) {
        neg = crt16<ND + 1, 16>(y, y_plane, i * F.n + j, nmod, D);
    } else {
#pragma unroll
        for (int dd = 0; dd <= ND; ++dd) D[dd] = 0;
    }
    const uint32_t fa = (uint32_t)(F.alpha < 0 ? (uint64_t)0 - (uint64_t)F.alpha : (uint64_t)F.alpha);
    if (fa != 1) {
        uint32_t carry = 0;
#pragma unroll
        for (int dd = 0; dd <= ND; ++dd) {
            const uint32_t v = D[dd] * fa + carry;
            D[dd] = v & 0xffff;
            carry = v >> 16;
        }
    }
    if (F.alpha < 0) neg = !neg;
    store_bits<F64>(F.c, (int64_t)i * F.crs + (int64_t)j * F.ccs,
                    encode16<F64, ND + 1>(D, sa.lo + sb.lo, neg, F.mode));
}

// Every other CRT cell: each diagonal's sum into the digit register (signed
// digits, so differently signed diagonals cancel exactly; a sliced plan adds
// diagonal d W * d bits higher), then the epilogue shared with the direct
// route.
template <bool F64, int ND>
__device__ inline void crt_general_cell(const FArgs &F, const Reg &R, const LineStat &sa,
                                        const LineStat &sb, int flags, const CrtHdr &hd, int nm,
                                        const uint8_t *y, uint64_t y_plane, uint64_t i, uint64_t j) {
    using Fm = Fmt<F64>;
    constexpr int S = Fm::DIGITS;
    for (int q = 0; q < S; ++q) R[q] = 0;
    // The slots the diagonals touch, plus headroom for their carries, the
    // sign and an alpha of up to 64 bits.
    int wlo = S - 1, whi = 0;
    if (hd.nmod > 0 && !((sa.flags | sb.flags) & LS_EMPTY)) {
        const int ndiag = hd.sa + hd.sb - 1;
        const int E = sa.lo + sb.lo;
        for (int dg = 0; dg < ndiag; ++dg) {
            uint32_t X[ND];
            const bool neg = crt16<ND>(y + (uint64_t)dg * nm * y_plane, y_plane, i * F.n + j, hd.nmod, X);
            const int pos = E - Fm::RB + hd.w * dg;
            const int q0 = pos >> 5, r = pos & 31;
            wlo = min(wlo, q0);
            whi = max(whi, q0 + (ND + 1) / 2);
#pragma unroll
            for (int dd = 0; dd < ND; dd += 2) {
                const uint32_t pair = X[dd] | ((dd + 1 < ND ? X[dd + 1] : 0u) << 16);
                if (!pair) continue;
                const uint64_t wv = (uint64_t)pair << r;
                const int64_t lo = (int64_t)(wv & M32), hi = (int64_t)(wv >> 32);
                const int k0 = q0 + dd / 2;
                if (k0 < S) R[k0] += neg ? -lo : lo;
                if (k0 + 1 < S) R[k0 + 1] += neg ? -hi : hi;
            }
        }
    }
    if (wlo > whi) wlo = whi = 0;
    whi = min(S - 1, whi + 4);
    const bool neg = normalise<S>(R, wlo, whi);
    finish_cell<F64>(F, R, neg, flags, i, j, wlo, whi);
}

// ---------------------------------------------- the register-window finish --
//
// The CRT cells the register epilogue does not take, when beta = 0 and
// |alpha| < 2^32: the diagonals combine by Horner's rule from the top,
// T := T * 2^w + X_d, in a two's-complement window of NW 32-bit words held in
// VGPRs (the value is T * 2^E, E = the lines' lo exponents), then alpha and
// one rounding.  The window holds w * (diagonals - 1) + 16 * ND bits plus 32
// bits for alpha and two of sign and carry; the plan's w and diagonal count
// are uniform, so the shifts are the same for every lane.  Cells whose window
// would not fit, and every cell when beta != 0, take the LDS-register kernel.

constexpr int WIN_MAX_WORDS = 48;

// The window bits a plan needs at ND digits per diagonal.
__host__ __device__ inline int window_bits(const CrtHdr &hd, int nd) {
    const int ndiag = hd.sa + hd.sb - 1;
    return (ndiag > 1 ? hd.w * (ndiag - 1) : 0) + 16 * nd + 34;
}

__device__ inline int crt_nd_template(int nmod) {
    const int nd = crt_nd16[nmod];
    return nd <= 8 ? 8 : nd <= 12 ? 12 : nd <= 16 ? 16 : nd <= 20 ? 20 : CRT_ND16;
}

__device__ inline bool window_cell(const FArgs &F, const CrtHdr &hd, const LineStat &sa,
                                   const LineStat &sb) {
    const uint64_t fa = F.alpha < 0 ? (uint64_t)0 - (uint64_t)F.alpha : (uint64_t)F.alpha;
    return !hd.crt_off && !fast_cell(F, hd, sa, sb) && F.beta == 0 && (fa >> 32) == 0 &&
           window_bits(hd, crt_nd_template(hd.nmod)) <= 32 * WIN_MAX_WORDS;
}

// impl_encode_into_float (acc.rs:1734-1868) from a magnitude in NW 32-bit
// words T[] whose bit 0 has exponent E: encode16's rounding, read from words.
template <bool F64, int NW>
__device__ inline uint64_t encode32(const uint32_t (&T)[NW], int E, bool neg, int mode) {
    using Fm = Fmt<F64>;
    constexpr int MANT = Fm::MANT, EXPO = Fm::EXPO, P = MANT + 1;
    constexpr uint64_t EXPMASK = (1ull << EXPO) - 1;
    int top = -1;
#pragma unroll
    for (int t = 0; t < NW; ++t)
        if (T[t]) top = 32 * t + 31 - __builtin_clz(T[t]);
    if (top < 0) return 0;  // an exact zero is +0
    const int exp = E + top;
    int lsb_exp = exp - (P - 1) < Fm::SUB_LSB ? Fm::SUB_LSB : exp - (P - 1);
    const int lsb = lsb_exp - E;
    uint64_t sig;
    int round_bit = 0, sticky = 0;
    if (lsb <= 0) {
        // Every bit lies at or above the output's LSB: the value is below 2^P.
        sig = ((uint64_t)T[0] | (NW > 1 ? (uint64_t)T[1 < NW ? 1 : 0] << 32 : 0)) << (-lsb);
    } else {
        const int q = lsb >> 5, r = lsb & 31;
        const int rb = lsb - 1, qb = rb >> 5;
        const uint32_t below = (1u << (rb & 31)) - 1;
        uint64_t w0 = 0, w1 = 0, w2 = 0;
#pragma unroll
        for (int t = 0; t < NW; ++t) {
            const uint32_t v = T[t];
            w0 = t == q ? v : w0;
            w1 = t == q + 1 ? v : w1;
            w2 = t == q + 2 ? v : w2;
            if (t == qb) {
                round_bit = (int)((v >> (rb & 31)) & 1);
                if (v & below) sticky = 1;
            }
            if (t < qb && v) sticky = 1;
        }
        const uint64_t lo = w0 | (w1 << 32);
        sig = ((lo >> r) | (r ? (w2 << (64 - r)) : 0)) & ((1ull << P) - 1);
    }
    const int inc = (mode == UOR_ENCODE_NEAREST) ? (round_bit && (sticky || (sig & 1))) : 0;
    sig += (uint64_t)inc;
    if (sig >> P) {
        sig >>= 1;
        lsb_exp += 1;
    }
    const uint64_t sbit = (uint64_t)(neg ? 1 : 0) << (MANT + EXPO);
    if (sig == 0) return sbit;
    if ((sig >> (P - 1)) == 1) {
        const int biased = lsb_exp + (P - 1) + Fm::BIAS;
        if (biased >= (int)EXPMASK) {
            if (mode == UOR_ENCODE_NEAREST) return sbit | (EXPMASK << MANT);
            return sbit | ((EXPMASK - 1) << MANT) | ((1ull << MANT) - 1);
        }
        return sbit | ((uint64_t)biased << MANT) | (sig & ((1ull << MANT) - 1));
    }
    return sbit | sig;
}

// The special values encode_reg gives a cell with non-finite flags.
template <bool F64>
__device__ inline uint64_t encode_flags(int flags) {
    using Fm = Fmt<F64>;
    if ((flags & FL_NAN) || ((flags & FL_PINF) && (flags & FL_NINF))) return Fm::NAN_BITS;
    const uint64_t s = (flags & FL_NINF) ? 1 : 0;
    return (s << (Fm::MANT + Fm::EXPO)) | (((1ull << Fm::EXPO) - 1) << Fm::MANT);
}

template <bool F64, int ND, int NW>
__device__ inline void crt_window_cell(const FArgs &F, const LineStat &sa, const LineStat &sb,
                                       int flags, const CrtHdr &hd, int nm, const uint8_t *y,
                                       uint64_t y_plane, uint64_t i, uint64_t j) {
    const int64_t ci = (int64_t)i * F.crs + (int64_t)j * F.ccs;
    flags = scale_flags(flags, F.alpha);
    if (flags) {
        store_bits<F64>(F.c, ci, encode_flags<F64>(flags));
        return;
    }
    uint32_t T[NW];
#pragma unroll
    for (int t = 0; t < NW; ++t) T[t] = 0;
    if (hd.nmod > 0 && !((sa.flags | sb.flags) & LS_EMPTY) && F.alpha != 0) {
        const int ndiag = hd.sa + hd.sb - 1;
        const int qw = hd.w >> 5, r = hd.w & 31;
        int pre[8];  // the next diagonal's first plane bytes (crt16's chain)
        for (int dg = ndiag - 1; dg >= 0; --dg) {
            if (dg != ndiag - 1) {
                // T <<= w: whole words by stages of 4, 2 and 1, then r bits.
                if (qw & 4) {
#pragma unroll
                    for (int t = NW - 1; t >= 0; --t) T[t] = t >= 4 ? T[t - 4] : 0u;
                }
                if (qw & 2) {
#pragma unroll
                    for (int t = NW - 1; t >= 0; --t) T[t] = t >= 2 ? T[t - 2] : 0u;
                }
                if (qw & 1) {
#pragma unroll
                    for (int t = NW - 1; t >= 0; --t) T[t] = t >= 1 ? T[t - 1] : 0u;
                }
                if (r) {
#pragma unroll
                    for (int t = NW - 1; t >= 1; --t)
                        T[t] = __builtin_amdgcn_alignbit(T[t], T[t - 1], 32 - r);
                    T[0] <<= r;
                }
            }
            uint32_t D[ND];
            const bool negx = crt16<ND>(y + (uint64_t)dg * nm * y_plane, y_plane, i * F.n + j, hd.nmod, D,
                                        dg > 0 ? y + (uint64_t)(dg - 1) * nm * y_plane : nullptr, pre,
                                        dg != ndiag - 1);
            // T += (-1)^negx X, two's complement over the whole window.
            const uint32_t xm = negx ? 0xffffffffu : 0u;
            uint32_t c = negx ? 1u : 0u;
#pragma unroll
            for (int t = 0; t < NW; ++t) {
                uint32_t x = 0;
                if (2 * t < ND) x = D[2 * t] | (2 * t + 1 < ND ? D[2 * t + 1] << 16 : 0u);
                const uint64_t s = (uint64_t)T[t] + (x ^ xm) + c;
                T[t] = (uint32_t)s;
                c = (uint32_t)(s >> 32);
            }
        }
    }
    bool neg = (T[NW - 1] >> 31) != 0;
    if (neg) {
        uint32_t c = 1;
#pragma unroll
        for (int t = 0; t < NW; ++t) {
            const uint64_t s = (uint64_t)(~T[t]) + c;
            T[t] = (uint32_t)s;
            c = (uint32_t)(s >> 32);
        }
    }
    const uint32_t fa = (uint32_t)(F.alpha < 0 ? (uint64_t)0 - (uint64_t)F.alpha : (uint64_t)F.alpha);
    if (fa != 1) {
        uint32_t c = 0;
#pragma unroll
        for (int t = 0; t < NW; ++t) {
            const uint64_t v = (uint64_t)T[t] * fa + c;
            T[t] = (uint32_t)v;
            c = (uint32_t)(v >> 32);
        }
    }
    if (F.alpha < 0) neg = !neg;
    store_bits<F64>(F.c, ci, encode32<F64, NW>(T, sa.lo + sb.lo, neg, F.mode));
}

template <bool F64, int ND>
__device__ inline void crt_window_dispatch(const FArgs &F, const LineStat &sa, const LineStat &sb,
                                           int flags, const CrtHdr &hd, int nm, const uint8_t *y,
                                           uint64_t y_plane, uint64_t i, uint64_t j) {
    const int bits = window_bits(hd, ND);
    if (bits <= 32 * 16) crt_window_cell<F64, ND, 16>(F, sa, sb, flags, hd, nm, y, y_plane, i, j);
    else if (bits <= 32 * 32) crt_window_cell<F64, ND, 32>(F, sa, sb, flags, hd, nm, y, y_plane, i, j);
    else crt_window_cell<F64, ND, WIN_MAX_WORDS>(F, sa, sb, flags, hd, nm, y, y_plane, i, j);
}

template <bool F64, int TM, int TN>
__global__ void __launch_bounds__(TM * TN) crt_window_kernel(FArgs F, const LineStat *ra,
                                                             const LineStat *cb, const CrtHdr *h,
                                                             const uint8_t *y, uint64_t y_plane,
                                                             int nm, int gn) {
    const int t = threadIdx.x;
    const uint64_t i = (uint64_t)(blockIdx.x / gn) * TM + t / TN;
    const uint64_t j = (uint64_t)(blockIdx.x % gn) * TN + t % TN;
    if (i >= F.m || j >= F.n) return;
    const CrtHdr hd = *h;
    const LineStat sa = ra[i], sb = cb[j];
    if (!window_cell(F, hd, sa, sb)) return;
    const int flags = ((sa.flags | sb.flags) & LS_DIRTY) ? flags_cell<F64>(F, i, j) : 0;
    switch (crt_nd_template(hd.nmod)) {
    case 8: crt_window_dispatch<F64, 8>(F, sa, sb, flags, hd, nm, y, y_plane, i, j); break;
    case 12: crt_window_dispatch<F64, 12>(F, sa, sb, flags, hd, nm, y, y_plane, i, j); break;
    case 16: crt_window_dispatch<F64, 16>(F, sa, sb, flags, hd, nm, y, y_plane, i, j); break;
    case 20: crt_window_dispatch<F64, 20>(F, sa, sb, flags, hd, nm, y, y_plane, i, j); break;
    default: crt_window_dispatch<F64, CRT_ND16>(F, sa, sb, flags, hd, nm, y, y_plane, i, j); break;
    }
}

template <bool F64, int TM, int TN>
__global__ void __launch_bounds__(TM * TN) crt_fast_kernel(FArgs F, const LineStat *ra,
                                                           const LineStat *cb, const CrtHdr *h,
                                                           const uint8_t *y, uint64_t y_plane,
                                                           int gn) {
    const int t = threadIdx.x;
    const uint64_t i = (uint64_t)(blockIdx.x / gn) * TM + t / TN;
    const uint64_t j = (uint64_t)(blockIdx.x % gn) * TN + t % TN;
    if (i >= F.m || j >= F.n) return;
    const CrtHdr hd = *h;
    const LineStat sa = ra[i], sb = cb[j];
    if (!fast_cell(F, hd, sa, sb)) return;
    const int nd = crt_nd16[hd.nmod];
    if (nd <= 8) crt_fast_cell<F64, 8>(F, sa, sb, hd.nmod, y, y_plane, i, j);
    else if (nd <= 12) crt_fast_cell<F64, 12>(F, sa, sb, hd.nmod, y, y_plane, i, j);
    else if (nd <= 16) crt_fast_cell<F64, 16>(F, sa, sb, hd.nmod, y, y_plane, i, j);
    else crt_fast_cell<F64, CRT_ND16>(F, sa, sb, hd.nmod, y, y_plane, i, j);
}

template <bool F64, int TM, int TN>
__global__ void __launch_bounds__(TM * TN) crt_general_kernel(FArgs F, const LineStat *ra,
                                                              const LineStat *cb, const CrtHdr *h,
                                                              const uint8_t *y, uint64_t y_plane,
                                                              int nm, int gn) {
    using Fm = Fmt<F64>;
    constexpr int S = Fm::DIGITS, NT = TM * TN;
    __shared__ int64_t regs[S * NT];
    const int t = threadIdx.x;
    const uint64_t i = (uint64_t)(blockIdx.x / gn) * TM + t / TN;
    const uint64_t j = (uint64_t)(blockIdx.x % gn) * TN + t % TN;
    if (i >= F.m || j >= F.n) return;
    const CrtHdr hd = *h;
    const LineStat sa = ra[i], sb = cb[j];
    if (fast_cell(F, hd, sa, sb) || window_cell(F, hd, sa, sb)) return;
    const Reg R{regs + t, NT};
    if (hd.crt_off) {
        for (int q = 0; q < S; ++q) R[q] = 0;
        const int flags = direct_cell<F64>(F, R, i, j);
        const bool neg = normalise<S>(R);
        finish_cell<F64>(F, R, neg, flags, i, j);
        return;
    }
    const int flags = ((sa.flags | sb.flags) & LS_DIRTY) ? flags_cell<F64>(F, i, j) : 0;
    const int nd = crt_nd16[hd.nmod];
    if (nd <= 8) crt_general_cell<F64, 8>(F, R, sa, sb, flags, hd, nm, y, y_plane, i, j);
    else if (nd <= 12) crt_general_cell<F64, 12>(F, R, sa, sb, flags, hd, nm, y, y_plane, i, j);
    else if (nd <= 16) crt_general_cell<F64, 16>(F, R, sa, sb, flags, hd, nm, y, y_plane, i, j);
    else crt_general_cell<F64, CRT_ND16>(F, R, sa, sb, flags, hd, nm, y, y_plane, i, j);
}

// Scratch layout of the CRT route for nm moduli and up to sa_max / sb_max
// slices per line (every piece 256-aligned).
struct CrtLayout {
    uint64_t hdr, ra, cb, ap, bp, y, total;
    uint64_t kp, np, a_plane, b_plane, y_plane;
    int nm, sa_max, sb_max;
};

static inline uint64_t al256(uint64_t v) { return (v + 255) & ~255ull; }

static CrtLayout crt_layout(uint64_t m, uint64_t k, uint64_t n, int nm, int smax) {
    CrtLayout L;
    L.nm = nm;
    L.sa_max = L.sb_max = smax;
    L.kp = (k + DL_BK - 1) / DL_BK * DL_BK;
    L.np = (n + 15) / 16 * 16;
    L.a_plane = al256(m * (uint64_t)smax * L.kp);
    L.b_plane = al256((uint64_t)smax * L.kp * L.np);
    L.y_plane = al256(m * n);
    L.hdr = 0;
    L.ra = 256;
    L.cb = L.ra + al256(m * sizeof(LineStat));
    L.ap = L.cb + al256(n * sizeof(LineStat));
    L.bp = L.ap + (uint64_t)nm * L.a_plane;
    L.y = L.bp + (uint64_t)nm * L.b_plane;
    L.total = L.y + (uint64_t)(2 * smax - 1) * nm * L.y_plane;
    return L;
}

// The most slices a line of this format can need (its exponent range plus
// the significand, in WIDE_BITS slices), within the i32 bound on a
// diagonal's depth (slices * kp <= 2^17).
static int crt_slice_cap(bool f64, uint64_t k) {
    const int width = f64 ? (1024 + 1074) : (128 + 149);
    int s = (width + WIDE_BITS - 1) / WIDE_BITS;
    const uint64_t kp = (k + DL_BK - 1) / DL_BK * DL_BK;
    while (s > 1 && (uint64_t)s * kp > (uint64_t)CRT_BK_MAX) --s;
    return s;
}

// Line statistics with the lanes along a line when it is contiguous; a wave
// across 64, 16 or 4 neighbouring lines (the most that still makes 256
// workgroups), 16 waves on the lines' elements, when neighbouring lines are
// neighbouring elements (B's columns); else 16 lines by 16 lanes.
template <bool F64>
static void launch_line_stats(const char *base, int64_t s_line, int64_t s_elem, uint64_t lines,
                              uint64_t len, LineStat *out, hipStream_t s) {
    if (s_elem == 1)
        hipLaunchKernelGGL((line_stats_kernel<F64, 1>), dim3((unsigned)lines), dim3(256), 0, s, base, s_line,
                           s_elem, lines, len, out);
    else if (s_line == 1 && lines >= 64 * 256)  // neighbouring lines are neighbouring elements
        hipLaunchKernelGGL((line_stats_kernel<F64, 64, 1024>), dim3((unsigned)((lines + 63) / 64)), dim3(1024), 0, s,
                           base, s_line, s_elem, lines, len, out);
    else if (s_line == 1 && lines >= 16 * 256)  // (fewer lines per workgroup: 256 workgroups at least)
        hipLaunchKernelGGL((line_stats_kernel<F64, 16, 1024>), dim3((unsigned)((lines + 15) / 16)), dim3(1024), 0, s,
                           base, s_line, s_elem, lines, len, out);
    else if (s_line == 1)
        hipLaunchKernelGGL((line_stats_kernel<F64, 4, 1024>), dim3((unsigned)((lines + 3) / 4)), dim3(1024), 0, s,
                           base, s_line, s_elem, lines, len, out);
    else
        hipLaunchKernelGGL((line_stats_kernel<F64, 16>), dim3((unsigned)((lines + 15) / 16)), dim3(256), 0, s,
                           base, s_line, s_elem, lines, len, out);
}

template <bool F64>
static hipError_t launch_crt(const FArgs &F, char *scratch, const CrtLayout &L, hipStream_t s) {
    const uint64_t m = F.m, k = F.k, n = F.n;
    const int nm = L.nm;
    CrtHdr *h = (CrtHdr *)(scratch + L.hdr);
    LineStat *ra = (LineStat *)(scratch + L.ra), *cb = (LineStat *)(scratch + L.cb);
    int8_t *ap = (int8_t *)(scratch + L.ap), *bp = (int8_t *)(scratch + L.bp);
    uint8_t *y = (uint8_t *)(scratch + L.y);
    // 1. line statistics: rows of A (elements along acs), columns of B (along brs).
    launch_line_stats<F64>(F.a, F.ars, F.acs, m, k, ra, s);
    launch_line_stats<F64>(F.b, F.bcs, F.brs, n, k, cb, s);
    // 2. plan.
    hipLaunchKernelGGL(crt_plan_kernel, dim3(1), dim3(256), 0, s, ra, m, cb, n, k, nm, L.sa_max,
                       L.sb_max, h);
    // 3. residue planes.
    {
        const uint64_t ta = (uint64_t)L.sa_max * m * (L.kp / 4), tb = (uint64_t)L.sb_max * L.kp * (L.np / 4);
        const auto blocks = [](uint64_t t) { return (unsigned)std::min<uint64_t>((t + 255) / 256, 4096); };
        hipLaunchKernelGGL((residue_kernel<F64, true>), dim3(blocks(ta)), dim3(256), 0, s, F.a, F.ars,
                           F.acs, m, k, L.kp, L.np, L.sa_max, ra, h, ap, L.a_plane);
        hipLaunchKernelGGL((residue_kernel<F64, false>), dim3(blocks(tb)), dim3(256), 0, s, F.b, F.brs,
                           F.bcs, k, n, L.kp, L.np, L.sb_max, cb, h, bp, L.b_plane);
    }
    // 4. residue GEMMs: grid y = diagonal, z = modulus.
    {
        constexpr int BM = 256, BN = 256;
        ResOut R{y, L.y_plane, nm, ap, bp, L.a_plane, L.b_plane, L.kp, L.np, L.sa_max, L.sb_max, h};
        const int gm = (int)((m + BM - 1) / BM), gn = (int)((n + BN - 1) / BN);
        const dim3 grid((unsigned)(gm * gn), (unsigned)(L.sa_max + L.sb_max - 1), (unsigned)nm);
        switch (dl_variant()) {
        case DL_W4:
            hipLaunchKernelGGL((residue_gemm_kernel<BM, BN, 2, 2, false>), grid, dim3(256), 0, s, m, n, gm, gn, R);
            break;
        case DL_W8:
            hipLaunchKernelGGL((residue_gemm_kernel<BM, BN, 2, 4, false>), grid, dim3(512), 0, s, m, n, gm, gn, R);
            break;
        default:
            hipLaunchKernelGGL((residue_gemm_kernel<BM, BN, 2, 4, true>), grid, dim3(512), 0, s, m, n, gm, gn, R);
            break;
        }
    }
    // 5. reconstruction, epilogue, encode: the register epilogue's cells,
    // then every other cell.
    {
        constexpr int TM = 4, TN = 64;
        const uint64_t gm = (m + TM - 1) / TM, gn = (n + TN - 1) / TN;
        hipLaunchKernelGGL((crt_fast_kernel<F64, TM, TN>), dim3((unsigned)(gm * gn)), dim3(TM * TN), 0, s, F,
                           ra, cb, h, y, L.y_plane, (int)gn);
    }
    {
        constexpr int TM = 4, TN = 64;
        const uint64_t gm = (m + TM - 1) / TM, gn = (n + TN - 1) / TN;
        hipLaunchKernelGGL((crt_window_kernel<F64, TM, TN>), dim3((unsigned)(gm * gn)), dim3(TM * TN), 0, s,
                           F, ra, cb, h, y, L.y_plane, nm, (int)gn);
    }
    {
        constexpr int TM = F64 ? 1 : 4, TN = 64;
        const uint64_t gm = (m + TM - 1) / TM, gn = (n + TN - 1) / TN;
        hipLaunchKernelGGL((crt_general_kernel<F64, TM, TN>), dim3((unsigned)(gm * gn)), dim3(TM * TN), 0, s,
                           F, ra, cb, h, y, L.y_plane, nm, (int)gn);
    }
    return hipGetLastError();
}

// ------------------------------------------------ integer element route --
//
// The view API at E = i16, i32, i64: the reference's Kernelized families
// (crates/uor-matmul-gemm/src/kernel.rs:132-399; AccOf = i128 for i16 and
// i32, Limbs<3> for i64: alphabet.rs:559-616, acc.rs:215), on the residue
// pipeline above.  An element is its own integer (line lo = 0, width = the
// bit length of the line's largest magnitude, at most 64), so the plan is
// never sliced and |X_ij| < 2^B with B <= 128 + log2 k takes at most 28
// moduli.  Depth beyond 2^17 (the i32 reach of one residue GEMM) runs in
// chunks whose residues add mod p.  Cells the plan cannot cover, and every
// cell when the offer holds no planes, take the per-cell loop.

struct IArgs {
    const char *a;  // element (0,0)
    int64_t ars, acs;
    const char *b;
    int64_t brs, bcs;
    char *c;
    int64_t crs, ccs;
    uint64_t m, k, n;
    int64_t alpha, beta;
    int mode;
    int ob;     // output bytes
    int limbs;  // 1: i64 elements (the Limbs<3> accumulator and epilogue)
};

template <int EB>
__device__ inline int64_t load_ielem(const char *base, int64_t idx) {
    if constexpr (EB == 2) return ((const int16_t *)base)[idx];
    else if constexpr (EB == 4) return ((const int32_t *)base)[idx];
    else return ((const int64_t *)base)[idx];
}

__device__ inline uint64_t mag64(int64_t v) { return v < 0 ? (uint64_t)0 - (uint64_t)v : (uint64_t)v; }

// A 192-bit two's complement integer (Limbs<3>).
struct W192 {
    uint64_t w[3];
};

// Limbs::neg (acc.rs:345-357), Limbs::combine (:391-402) and ScaleExact for
// Limbs<L> (epilogue.rs:307-328): the register is 192 bits and does not grow,
// so scaling by an i64 factor is the product mod 2^192.
__device__ inline W192 w192_neg(const W192 &x) {
    W192 r;
    u128 t = (u128)(~x.w[0]) + 1;
    r.w[0] = (uint64_t)t;
    t = (u128)(~x.w[1]) + (uint64_t)(t >> 64);
    r.w[1] = (uint64_t)t;
    r.w[2] = ~x.w[2] + (uint64_t)(t >> 64);
    return r;
}

__device__ inline W192 w192_combine(const W192 &x, const W192 &y) {
    W192 r;
    u128 t = (u128)x.w[0] + y.w[0];
    r.w[0] = (uint64_t)t;
    t = (u128)x.w[1] + y.w[1] + (uint64_t)(t >> 64);
    r.w[1] = (uint64_t)t;
    r.w[2] = x.w[2] + y.w[2] + (uint64_t)(t >> 64);
    return r;
}

__device__ inline W192 w192_scale(const W192 &x, int64_t factor) {
    const uint64_t f = factor < 0 ? (uint64_t)0 - (uint64_t)factor : (uint64_t)factor;
    const u128 p0 = (u128)x.w[0] * f, p1 = (u128)x.w[1] * f;
    W192 r;
    r.w[0] = (uint64_t)p0;
    const u128 s1 = (u128)(uint64_t)p1 + (uint64_t)(p0 >> 64);
    r.w[1] = (uint64_t)s1;
    r.w[2] = x.w[2] * f + (uint64_t)(p1 >> 64) + (uint64_t)(s1 >> 64);
    return factor < 0 ? w192_neg(r) : r;
}

__device__ inline void w192_add(W192 &x, i128 v) {
    const u128 lo = (u128)x.w[0] + (uint64_t)(u128)v;
    x.w[0] = (uint64_t)lo;
    const u128 mid = (u128)x.w[1] + (uint64_t)((u128)v >> 64) + (uint64_t)(lo >> 64);
    x.w[1] = (uint64_t)mid;
    x.w[2] = x.w[2] + (v < 0 ? ~(uint64_t)0 : 0) + (uint64_t)(mid >> 64);
}

// Line statistics of integer lines: lo = 0, width = bit length of the
// largest magnitude, l1 an upper bound of log2 of the sum of magnitudes.
// Lines and threads as line_stats_kernel, and the same one pass: a running
// sum scaled by 2^-hi, rescaled by a power of two when hi rises.
template <int EB, int LPB, int NT = 256>
__global__ void __launch_bounds__(NT) int_line_stats_kernel(const char *base, int64_t s_line,
                                                            int64_t s_elem, uint64_t lines,
                                                            uint64_t len, LineStat *out) {
    constexpr int TPL = NT / LPB;  // threads per line
    __shared__ int s_hi[NT];
    __shared__ double s_sum[NT];
    const int t = threadIdx.x;
    const int tl = t % LPB, te = t / LPB;
    const uint64_t line = (uint64_t)blockIdx.x * LPB + tl;
    const bool live = line < lines;
    int hi = 0;
    double sum = 0;
    if (live)
        for (uint64_t e = te; e < len; e += TPL) {
            const uint64_t v = mag64(load_ielem<EB>(base, (int64_t)line * s_line + (int64_t)e * s_elem));
            if (!v) continue;
            const int top = bitlen64(v);
            if (top > hi) {
                sum = ldexp(sum, hi - top);
                hi = top;
            }
            sum += ldexp((double)v, -hi);
        }
    s_hi[t] = hi;
    s_sum[t] = sum;
    __syncthreads();
    for (int w = TPL / 2; w >= 1; w >>= 1) {
        if (te < w) {
            const int o = t + LPB * w;
            const int h0 = s_hi[t], h1 = s_hi[o], h = max(h0, h1);
            s_sum[t] = ldexp(s_sum[t], h0 - h) + ldexp(s_sum[o], h1 - h);
            s_hi[t] = h;
        }
        __syncthreads();
    }
    hi = s_hi[tl];
    if (te == 0 && live) {
        LineStat st;
        st.lo = 0;
        if (hi == 0) {
            st.width = 0;
            st.l1 = -1e30f;
            st.flags = LS_EMPTY;
        } else {
            st.width = hi;
            // Each term is rounded to 53 bits (relative 2^-53) and the sum
            // adds at most 2^-30 relative for any reachable length.
            const double sm = s_sum[tl] * (1.0 + 0x1p-28);
            st.l1 = (float)(log2(sm) + (double)hi + 1e-6);
            st.flags = 0;
        }
        out[line] = st;
    }
}

// The balanced int8 residue of an EB-byte element v modulo crt_mod[l]; xh
// and xl are +-(|v| >> 32) and +-(|v| mod 2^32) as doubles, signed as v
// (EB <= 4: xh = 0, xl = v).  As for the float residues, every modulus but
// 256 is odd, so for |x| < 2^32 (x * (1/p) errs by less than 2^-24, a
// quotient x / p is at least 1/(2p) >= 2^-9 from a half-integer) x - p
// rint(x / p) is the balanced residue, exact out of one fma; an i64 element
// combines its halves' residues as rh (2^32 mod p) + rl, below 2^15 in
// magnitude, and reduces that once more.
template <int EB>
__device__ inline int int_residue(int64_t v, double xh, double xl, int l) {
    if (l == 0) {
        int b = (int)(mag64(v) & 255);
        b = b >= 128 ? b - 256 : b;
        if (v < 0) b = -b;
        return b == 128 ? -128 : b;  // p = 256: 128 and -128 are one residue
    }
    const double p = (double)crt_mod[l], ip = crt_invp[l];
    double x = fma(-rint(xl * ip), p, xl);
    if constexpr (EB == 8) {
        const double rh = fma(-rint(xh * ip), p, xh);
        x = fma(rh, (double)crt_pow2[l][32], x);
        x = fma(-rint(x * ip), p, x);
    }
    return (int)x;
}

// Residue planes of an integer operand, laid out as residue_kernel's
// unsliced planes (A: plane l row i at i * kp; B: plane l row p at
// (s_max - 1) * kp + p, np bytes per row).  rows x cols of the source from
// src (already at the chunk's first k); padding is zero.
template <int EB, bool ROWS_A>
__global__ void __launch_bounds__(256) int_residue_kernel(const char *src, int64_t s_r, int64_t s_c,
                                                          uint64_t rows, uint64_t cols, uint64_t kp,
                                                          uint64_t np, int s_max, const CrtHdr *h,
                                                          int8_t *planes, uint64_t plane_bytes) {
    const int nmod = h->nmod;
    if (nmod == 0) return;
    const uint64_t R = ROWS_A ? rows : kp, C = ROWS_A ? kp : np;
    const uint64_t chunks = C / 4, total = R * chunks;
    for (uint64_t idx = (uint64_t)blockIdx.x * 256 + threadIdx.x; idx < total;
         idx += (uint64_t)gridDim.x * 256) {
        const uint64_t r = idx / chunks, c0 = (idx % chunks) * 4;
        int64_t v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint64_t sc = c0 + e;
            v[e] = (r < rows && sc < cols) ? load_ielem<EB>(src, (int64_t)r * s_r + (int64_t)sc * s_c) : 0;
        }
        double xh[4], xl[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if constexpr (EB == 8) {
                const uint64_t a = mag64(v[e]);
                const double sg = v[e] < 0 ? -1.0 : 1.0;
                xh[e] = sg * (double)(uint32_t)(a >> 32);
                xl[e] = sg * (double)(uint32_t)a;
            } else {
                xh[e] = 0;
                xl[e] = (double)v[e];
            }
        }
        int8_t *dst = ROWS_A ? planes + r * ((uint64_t)s_max * kp) + c0
                             : planes + ((uint64_t)(s_max - 1) * kp + r) * np + c0;
        for (int l = 0; l < nmod; ++l) {
            uint32_t wd = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                wd |= (uint32_t)(uint8_t)(int8_t)int_residue<EB>(v[e], xh[e], xl[e], l) << (8 * e);
            *(uint32_t *)(dst + (uint64_t)l * plane_bytes) = wd;
        }
    }
}

// The exact sum of one cell by the plain loop (driver::gemm,
// crates/uor-matmul-gemm/src/driver.rs:67-182).
template <int EB>
__device__ inline W192 int_direct_sum(const IArgs &F, uint64_t i, uint64_t j) {
    W192 x{{0, 0, 0}};
    const int64_t ab = (int64_t)i * F.ars, bb = (int64_t)j * F.bcs;
    for (uint64_t p = 0; p < F.k; ++p) {
        const int64_t a = load_ielem<EB>(F.a, ab + (int64_t)p * F.acs);
        const int64_t b = load_ielem<EB>(F.b, (int64_t)p * F.brs + bb);
        if constexpr (EB <= 4) w192_add(x, (i128)(a * b));  // |a * b| <= 2^62
        else w192_add(x, (i128)a * (i128)b);
    }
    return x;
}

// Linear::finish and the one encode (epilogue.rs:67-95; acc.rs:128-150 for
// i128, impl_encode_from_limbs acc.rs:405-442 for Limbs<3>).
template <int OB>
__device__ inline void int_finish(const IArgs &F, char *cp, const W192 &sum) {
    // i64 elements: Linear::finish in the Limbs<3> register, every step mod
    // 2^192 (scale_exact(alpha) + of_prior(C).scale_exact(beta)).
    W192 x = sum;
    if (F.limbs && (F.alpha != 1 || F.beta != 0)) {
        x = w192_scale(sum, F.alpha);
        if (F.beta != 0) {
            W192 prior{{0, 0, 0}};
            w192_add(prior, load_out<OB>(cp));
            x = w192_combine(x, w192_scale(prior, F.beta));
        }
    }
    i128 low = (i128)(((u128)x.w[1] << 64) | x.w[0]);
    // The public route's modular lane (kernel.rs:566-607, modular_spec and
    // modular_as_acc at :185-221, 250-279, 308-330): Wrapping into at most
    // 32 bits hands Linear::finish the sum in Z/2^32, sign-extended, so alpha
    // scales that lane and never saturates.  (i64 elements: Z/2^64 for
    // outputs of at most 64 bits, kernel.rs:371-398; every later step is mod
    // 2^192, so that lane wraps to the same bytes as the exact value.)
    if (!F.limbs && OB <= 4 && F.mode == UOR_ENCODE_WRAPPING) low = (i128)(int32_t)(uint32_t)x.w[0];
    if (!F.limbs) {
        // i16 / i32 elements: |X| < 2^126, the i128 accumulator.
        if (F.alpha == 1 && F.beta == 0) {
            store_out<OB>(cp, encode_int(low, OB, F.mode));
            return;
        }
        i128 t = sat_mul(low, F.alpha);
        if (F.beta != 0) t = (i128)((u128)t + (u128)sat_mul(load_out<OB>(cp), F.beta));
        store_out<OB>(cp, encode_int(t, OB, F.mode));
        return;
    }
    if (F.mode == UOR_ENCODE_WRAPPING) {
        store_out<OB>(cp, encode_int(low, OB, UOR_ENCODE_WRAPPING));
        return;
    }
    const bool neg = (int64_t)x.w[2] < 0;
    uint64_t m0 = x.w[0], m1 = x.w[1], m2 = x.w[2];
    if (neg) {
        m0 = ~m0;
        m1 = ~m1;
        m2 = ~m2;
        u128 t = (u128)m0 + 1;
        m0 = (uint64_t)t;
        t = (u128)m1 + (uint64_t)(t >> 64);
        m1 = (uint64_t)t;
        m2 += (uint64_t)(t >> 64);
    }
    i128 mn, mx;
    out_range(OB, &mn, &mx);
    const u128 mag = ((u128)m1 << 64) | m0;
    const u128 limit = neg ? (u128)0 - (u128)mn : (u128)mx;
    i128 v;
    if (m2 != 0 || mag > limit) v = neg ? mn : mx;
    else v = neg ? (i128)((u128)0 - mag) : (i128)mag;
    store_out<OB>(cp, v);
}

// (Always inlined: as a called function its arguments arrive in vector
// registers, and crt16 would then read the tables indexed by nmod with vector
// loads, each waited for, instead of on the scalar unit.)
template <int ND>
__device__ __attribute__((always_inline)) inline W192 crt_w192(const uint8_t *y, uint64_t y_plane, uint64_t cell,
                                                               int nmod) {
    uint32_t D[ND];
    const bool neg = crt16<ND>(y, y_plane, cell, nmod, D);
    // |X| < 2^192 (B <= 192), so the digits past the twelfth are zero.
    uint64_t w[3] = {0, 0, 0};
#pragma unroll
    for (int d = 0; d < ND && d < 12; ++d) w[d / 4] |= (uint64_t)D[d] << (16 * (d % 4));
    W192 x{{w[0], w[1], w[2]}};
    if (neg) {
        x.w[0] = ~x.w[0];
        x.w[1] = ~x.w[1];
        x.w[2] = ~x.w[2];
        u128 t = (u128)x.w[0] + 1;
        x.w[0] = (uint64_t)t;
        t = (u128)x.w[1] + (uint64_t)(t >> 64);
        x.w[1] = (uint64_t)t;
        x.w[2] += (uint64_t)(t >> 64);
    }
    return x;
}

// One thread per cell of a 4 x 64 tile: the CRT reconstruction (or, with no
// header, with crt_off, the per-cell loop), then the epilogue.
template <int EB>
__global__ void __launch_bounds__(256) int_finish_kernel(IArgs F, const LineStat *ra,
                                                         const LineStat *cb, const CrtHdr *h,
                                                         const uint8_t *y, uint64_t y_plane,
                                                         int gn) {
    const int t = threadIdx.x;
    const uint64_t i = (uint64_t)(blockIdx.x / gn) * 4 + t / 64;
    const uint64_t j = (uint64_t)(blockIdx.x % gn) * 64 + t % 64;
    if (i >= F.m || j >= F.n) return;
    W192 x{{0, 0, 0}};
    if (!h || h->crt_off) {
        x = int_direct_sum<EB>(F, i, j);
    } else {
        const int nmod = h->nmod;
        if (nmod > 0 && !((ra[i].flags | cb[j].flags) & LS_EMPTY)) {
            const uint64_t cell = i * F.n + j;
            const int nd = crt_nd16[nmod];
            if (nd <= 8) x = crt_w192<8>(y, y_plane, cell, nmod);
            else if (nd <= 12) x = crt_w192<12>(y, y_plane, cell, nmod);
            else x = crt_w192<16>(y, y_plane, cell, nmod);
        }
    }
    char *cp = F.c + ((int64_t)i * F.crs + (int64_t)j * F.ccs) * F.ob;
    switch (F.ob) {
    case 1: int_finish<1>(F, cp, x); break;
    case 2: int_finish<2>(F, cp, x); break;
    case 4: int_finish<4>(F, cp, x); break;
    case 8: int_finish<8>(F, cp, x); break;
    default: int_finish<16>(F, cp, x); break;
    }
}

// Moduli planes enough for any data of EB-byte elements at depth k: B <=
// 2 * 8 * EB + ceil(log2 k) bits, and each of the first 30 moduli adds at
// least 7 bits of capacity.
static int int_moduli_cap(int eb, uint64_t k) {
    int lk = 0;
    while (lk < 64 && (1ull << lk) < k) ++lk;
    const int need = 16 * eb + lk;
    return std::min(CRT_NMAX, (need + 6) / 7 + 1);
}

template <int EB>
static hipError_t launch_int_crt(const IArgs &F, char *scratch, const CrtLayout &L, uint64_t kc,
                                 hipStream_t s) {
    const uint64_t m = F.m, k = F.k, n = F.n;
    const int nm = L.nm;
    CrtHdr *h = (CrtHdr *)(scratch + L.hdr);
    LineStat *ra = (LineStat *)(scratch + L.ra), *cb = (LineStat *)(scratch + L.cb);
    int8_t *ap = (int8_t *)(scratch + L.ap), *bp = (int8_t *)(scratch + L.bp);
    uint8_t *y = (uint8_t *)(scratch + L.y);
    // 1. line statistics over the whole depth.
    const auto stats = [&](const char *base, int64_t s_line, int64_t s_elem, uint64_t lines, LineStat *out) {
        if (s_elem == 1)
            hipLaunchKernelGGL((int_line_stats_kernel<EB, 1>), dim3((unsigned)lines), dim3(256), 0, s, base,
                               s_line, s_elem, lines, k, out);
        else if (s_line == 1 && lines >= 64 * 256)  // B's columns: as launch_line_stats
            hipLaunchKernelGGL((int_line_stats_kernel<EB, 64, 1024>), dim3((unsigned)((lines + 63) / 64)),
                               dim3(1024), 0, s, base, s_line, s_elem, lines, k, out);
        else if (s_line == 1 && lines >= 16 * 256)
            hipLaunchKernelGGL((int_line_stats_kernel<EB, 16, 1024>), dim3((unsigned)((lines + 15) / 16)),
                               dim3(1024), 0, s, base, s_line, s_elem, lines, k, out);
        else if (s_line == 1)
            hipLaunchKernelGGL((int_line_stats_kernel<EB, 4, 1024>), dim3((unsigned)((lines + 3) / 4)),
                               dim3(1024), 0, s, base, s_line, s_elem, lines, k, out);
        else
            hipLaunchKernelGGL((int_line_stats_kernel<EB, 16>), dim3((unsigned)((lines + 15) / 16)), dim3(256),
                               0, s, base, s_line, s_elem, lines, k, out);
    };
    stats(F.a, F.ars, F.acs, m, ra);
    stats(F.b, F.bcs, F.brs, n, cb);
    // 2. plan (never sliced: every line is at most 64 bits wide).
    hipLaunchKernelGGL(crt_plan_kernel, dim3(1), dim3(256), 0, s, ra, m, cb, n, k, nm, 1, 1, h);
    // 3-4. per chunk of at most kc: residue planes, residue GEMMs.
    constexpr int BM = 256, BN = 256;
    const int gm = (int)((m + BM - 1) / BM), gn = (int)((n + BN - 1) / BN);
    const auto blocks = [](uint64_t t) { return (unsigned)std::min<uint64_t>((t + 255) / 256, 4096); };
    for (uint64_t k0 = 0; k0 < k; k0 += kc) {
        const uint64_t kl = std::min(kc, k - k0);
        const uint64_t ta = m * (L.kp / 4), tb = L.kp * (L.np / 4);
        hipLaunchKernelGGL((int_residue_kernel<EB, true>), dim3(blocks(ta)), dim3(256), 0, s,
                           F.a + (int64_t)k0 * F.acs * EB, F.ars, F.acs, m, kl, L.kp, L.np, 1, h, ap, L.a_plane);
        hipLaunchKernelGGL((int_residue_kernel<EB, false>), dim3(blocks(tb)), dim3(256), 0, s,
                           F.b + (int64_t)k0 * F.brs * EB, F.brs, F.bcs, kl, n, L.kp, L.np, 1, h, bp, L.b_plane);
        // (The GEMM runs over the layout's whole kp: a short last chunk's
        // padding residues are zero.)
        ResOut R{y, L.y_plane, nm, ap, bp, L.a_plane, L.b_plane, L.kp, L.np, 1, 1, h, k0 > 0 ? 1 : 0};
        const dim3 grid((unsigned)(gm * gn), 1, (unsigned)nm);
        hipLaunchKernelGGL((residue_gemm_kernel<BM, BN, 2, 4, true>), grid, dim3(512), 0, s, m, n, gm, gn, R);
    }
    // 5. reconstruction, epilogue, encode.
    const uint64_t fm = (m + 3) / 4, fn = (n + 63) / 64;
    hipLaunchKernelGGL((int_finish_kernel<EB>), dim3((unsigned)(fm * fn)), dim3(256), 0, s, F, ra, cb, h, y,
                       L.y_plane, (int)fn);
    return hipGetLastError();
}

template <int EB>
static hipError_t launch_int_direct(const IArgs &F, hipStream_t s) {
    const uint64_t fm = (F.m + 3) / 4, fn = (F.n + 63) / 64;
    hipLaunchKernelGGL((int_finish_kernel<EB>), dim3((unsigned)(fm * fn)), dim3(256), 0, s, F, nullptr, nullptr,
                       nullptr, nullptr, 0, (int)fn);
    return hipGetLastError();
}

}  // namespace uor

using namespace uor;

extern "C" uint64_t uor_gfx950_suggested_scratch_float(int is_f64, uint64_t m, uint64_t k,
                                                       uint64_t n) {
    // The CRT route's planes for every modulus and every slice a line of
    // this format can need, plus alignment slack; 0 where that route does
    // not apply (the direct route needs none).
    if (m == 0 || n == 0 || k == 0 || k > (uint64_t)CRT_BK_MAX) return 0;
    return crt_layout(m, k, n, CRT_NMAX, crt_slice_cap(is_f64 != 0, k)).total + 256;
}

extern "C" int uor_gfx950_gemm_float(int is_f64, const uor_view *a, const uor_view *b,
                                     const uor_view *c, int64_t alpha, int64_t beta, int encode,
                                     void *scratch, uint64_t scratch_bytes, void *stream,
                                     uor_route *route) {
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
    // The CRT route when the offer holds at least one modulus' planes: the
    // most slices the format can need if they fit with 40 or more moduli,
    // else fewer slices, else unsliced with what fits.
    int nm = 0;
    CrtLayout L{};
    char *sc = nullptr;
    if (scratch && F.k > 0 && F.k <= (uint64_t)CRT_BK_MAX) {
        const uintptr_t p0 = (uintptr_t)scratch, p1 = (p0 + 255) & ~(uintptr_t)255;
        const uint64_t have = scratch_bytes > (p1 - p0) ? scratch_bytes - (p1 - p0) : 0;
        sc = (char *)p1;
        for (int sm = crt_slice_cap(is_f64 != 0, F.k); sm >= 1 && nm == 0; --sm) {
            for (int q = CRT_NMAX; q >= (sm > 1 ? 40 : 1); --q) {
                const CrtLayout Lq = crt_layout(F.m, F.k, F.n, q, sm);
                if (Lq.total <= have) {
                    nm = q;
                    L = Lq;
                    break;
                }
            }
        }
        const uint64_t gm = (F.m + 255) / 256, gn = (F.n + 255) / 256;
        if (gm * gn > 0x7fffffffull || F.m > 0x7fffffffull || F.n > 0x7fffffffull) nm = 0;
    }
    if (nm > 0) {
        UOR_HIP(is_f64 ? launch_crt<true>(F, sc, L, s) : launch_crt<false>(F, sc, L, s));
        if (route) {
            route->kind = UOR_ROUTE_FLOAT_CRT;
            route->tile_m = route->tile_n = 256;
            route->tile_k = DL_BK;
            route->split_k = 1;
            route->launches = 9;
            route->moduli = nm;  // planes offered; the device uses the fewest that suffice
            route->scratch_used = L.total;
        }
        return UOR_OK;
    }
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

// slice.rs:405-421 gemm_float: gemm_float_ex at alpha 1, beta 0, lda = k,
// ldb = n, ldc = n.
extern "C" int uor_gfx950_slice_gemm_float(int is_f64, uint64_t m, uint64_t k, uint64_t n,
                                           const void *a, uint64_t a_len, const void *b,
                                           uint64_t b_len, void *c, uint64_t c_len, void *scratch,
                                           uint64_t scratch_bytes, void *stream) {
    return uor_gfx950_slice_gemm_float_ex(is_f64, m, k, n, 1, a, a_len, k, b, b_len, n, 0, c,
                                          c_len, n, scratch, scratch_bytes, stream);
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

// ------------------------------------------------------------ limb route --
//
// i16 / i32 elements as L = EB int8 limbs on the dense int8 route.  With
// l_t = ((a >> 8t) & 0xFF) - 128 for t < L - 1, l_{L-1} = a >> 8(L-1) and
// Ca = 128 (1 + 256 + ... + 256^{L-2}):  a = sum_t 256^t l_t + Ca, so
//   sum_p a b = sum_s 256^s G_s + Ca (RA_i + RB_j) - Ca^2 k,
// G_s = sum over t + u = s of the int8 products of limb planes t and u,
// RA_i = sum_p a[i,p], RB_j = sum_p b[p,j].  A's limbs sit side
// by side (m x Lk, plane t at column tk) and B's in reverse order (Lk x n,
// plane u at row (L-1-u)k), so each G_s is one GEMM over a contiguous window
// of both: depth (pairs of s) x k.  The planes hold G_s in i32: exact when
// Lk < 2^17 (|G_s| <= 2^14 L k), and for Wrapping into at most 32 bits --
// where only the sum mod 2^32 is used -- for any depth, with the shifts past
// 32 bits left out.
constexpr int LIMB_SPLIT_A = 16;   // A elements per thread
constexpr int LIMB_SPLIT_B = 64;   // B rows per thread

template <int EB>
__device__ inline int8_t limb_of(int64_t v, int t) {
    constexpr int L = EB;
    if (t == L - 1) return (int8_t)(v >> (8 * (L - 1)));
    return (int8_t)((int)((v >> (8 * t)) & 0xFF) - 128);
}

__global__ void __launch_bounds__(256) fill_i64_kernel(int64_t *p, uint64_t n) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = 0;
}

// Thread: LIMB_SPLIT_A consecutive p of row blockIdx.y; a block's partial
// row sum is added once.
template <int EB>
__global__ void __launch_bounds__(256) limb_split_a_kernel(IArgs F, int8_t *acat, int64_t *sa) {
    constexpr int L = EB;
    __shared__ int64_t part[4];
    const uint64_t i = blockIdx.y;
    const uint64_t p0 = ((uint64_t)blockIdx.x * 256 + threadIdx.x) * LIMB_SPLIT_A;
    int64_t sum = 0;
    if (p0 < F.k) {
        int8_t l[L][LIMB_SPLIT_A];
        int64_t v[LIMB_SPLIT_A];
        const char *src = F.a + ((int64_t)i * F.ars + (int64_t)p0 * F.acs) * EB;
        if (F.acs == 1 && p0 + LIMB_SPLIT_A <= F.k && ((uintptr_t)src & 15) == 0) {
            // EB 16-byte loads of the chunk's LIMB_SPLIT_A elements
#pragma unroll
            for (int q = 0; q < EB; ++q) {
                const uint4 x = ((const uint4 *)src)[q];
                const uint32_t d[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
                for (int h = 0; h < 16 / EB; ++h) {
                    const uint32_t dw = d[(h * EB) / 4];
                    if constexpr (EB == 2) v[q * 8 + h] = (int16_t)(dw >> (16 * (h & 1)));
                    else v[q * 4 + h] = (int32_t)dw;
                }
            }
        } else {
#pragma unroll
            for (int e = 0; e < LIMB_SPLIT_A; ++e)
                v[e] = p0 + e < F.k ? load_ielem<EB>(F.a, (int64_t)i * F.ars + (int64_t)(p0 + e) * F.acs) : 0;
        }
#pragma unroll
        for (int e = 0; e < LIMB_SPLIT_A; ++e) {
            sum += v[e];
#pragma unroll
            for (int t = 0; t < L; ++t) l[t][e] = limb_of<EB>(v[e], t);
        }
        int8_t *row = acat + i * (L * F.k);
        // 16-byte stores when the chunk is whole and k keeps planes aligned.
        const bool vec = p0 + LIMB_SPLIT_A <= F.k && (F.k % 16) == 0;
#pragma unroll
        for (int t = 0; t < L; ++t) {
            if (vec) {
                uint32_t w[4];
#pragma unroll
                for (int d = 0; d < 4; ++d)
                    w[d] = (uint32_t)(uint8_t)l[t][4 * d] | ((uint32_t)(uint8_t)l[t][4 * d + 1] << 8) |
                           ((uint32_t)(uint8_t)l[t][4 * d + 2] << 16) | ((uint32_t)(uint8_t)l[t][4 * d + 3] << 24);
                *(uint4 *)(row + (uint64_t)t * F.k + p0) = uint4{w[0], w[1], w[2], w[3]};
            } else {
#pragma unroll
                for (int e = 0; e < LIMB_SPLIT_A; ++e)
                    if (p0 + e < F.k) row[(uint64_t)t * F.k + p0 + e] = l[t][e];
            }
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) sum += __shfl_xor(sum, o, 64);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = sum;
    __syncthreads();
    if (threadIdx.x == 0) atomicAdd((unsigned long long *)&sa[i], (unsigned long long)(part[0] + part[1] + part[2] + part[3]));
}

// Thread: column j (VEC4: columns 4j .. 4j + 3, one 4-byte store per limb
// plane and row), LIMB_SPLIT_B consecutive rows of B.
template <int EB, bool VEC4>
__global__ void __launch_bounds__(256) limb_split_b_kernel(IArgs F, int8_t *brev, int64_t *sb) {
    constexpr int L = EB;
    constexpr int NJ = VEC4 ? 4 : 1;
    const uint64_t j = ((uint64_t)blockIdx.x * 256 + threadIdx.x) * NJ;
    const uint64_t p0 = (uint64_t)blockIdx.y * LIMB_SPLIT_B;
    if (j >= F.n) return;
    int64_t sum[NJ];
#pragma unroll
    for (int q = 0; q < NJ; ++q) sum[q] = 0;
    // U rows at a time, their loads issued together (rows past k read as
    // zero and are not stored).
    constexpr int U = 8;
    for (int e0 = 0; e0 < LIMB_SPLIT_B && p0 + e0 < F.k; e0 += U) {
        int64_t v[U][NJ];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint64_t p = p0 + e0 + u;
            const bool in = e0 + u < LIMB_SPLIT_B && p < F.k;
            if constexpr (VEC4) {
                const char *src = F.b + ((int64_t)p * F.brs + (int64_t)j) * EB;
                if constexpr (EB == 2) {
                    const uint2 x = in ? *(const uint2 *)src : uint2{0, 0};
                    v[u][0] = (int16_t)x.x, v[u][1] = (int16_t)(x.x >> 16), v[u][2] = (int16_t)x.y,
                    v[u][3] = (int16_t)(x.y >> 16);
                } else {
                    const uint4 x = in ? *(const uint4 *)src : uint4{0, 0, 0, 0};
                    v[u][0] = (int32_t)x.x, v[u][1] = (int32_t)x.y, v[u][2] = (int32_t)x.z, v[u][3] = (int32_t)x.w;
                }
            } else {
                v[u][0] = in ? load_ielem<EB>(F.b, (int64_t)p * F.brs + (int64_t)j * F.bcs) : 0;
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint64_t p = p0 + e0 + u;
            if (!(e0 + u < LIMB_SPLIT_B && p < F.k)) continue;
#pragma unroll
            for (int q = 0; q < NJ; ++q) sum[q] += v[u][q];
#pragma unroll
            for (int t = 0; t < L; ++t) {
                int8_t *dst = brev + ((uint64_t)(L - 1 - t) * F.k + p) * F.n + j;
                if constexpr (VEC4) {
                    uint32_t w = 0;
#pragma unroll
                    for (int q = 0; q < 4; ++q) w |= (uint32_t)(uint8_t)limb_of<EB>(v[u][q], t) << (8 * q);
                    *(uint32_t *)dst = w;
                } else {
                    *dst = limb_of<EB>(v[u][0], t);
                }
            }
        }
    }
#pragma unroll
    for (int q = 0; q < NJ; ++q) atomicAdd((unsigned long long *)&sb[j + q], (unsigned long long)sum[q]);
}

// One thread per cell: X from the NP planes and the line sums (two's-
// complement i128 arithmetic, exact when the planes are, right mod 2^32
// otherwise), then Linear::finish and the encode.  NP is a template
// argument so the plane loads are issued together (a loop over a run-time
// count waited for each in turn); cak = ca^2 k as an i128 (lo, hi).
template <int NP>
__global__ void __launch_bounds__(256) limb_combine_kernel(IArgs F, const int32_t *planes, const int64_t *sa,
                                                           const int64_t *sb, int64_t ca, uint64_t cak_lo,
                                                           uint64_t cak_hi) {
    const uint64_t j = (uint64_t)blockIdx.x * 256 + threadIdx.x, i = blockIdx.y;
    if (j >= F.n) return;
    const uint64_t cell = i * F.n + j, mn = F.m * F.n;
    int32_t pv[NP];
#pragma unroll
    for (int sft = 0; sft < NP; ++sft) pv[sft] = planes[(uint64_t)sft * mn + cell];
    u128 x = 0;
#pragma unroll
    for (int sft = NP - 1; sft >= 0; --sft) x = (x << 8) + (u128)(i128)pv[sft];
    x += (u128)((i128)ca * ((i128)sa[i] + (i128)sb[j]));
    x -= ((u128)cak_hi << 64) | (u128)cak_lo;
    const i128 v = (i128)x;
    W192 w{{(uint64_t)x, (uint64_t)(x >> 64), v < 0 ? ~(uint64_t)0 : 0}};
    char *cp = F.c + ((int64_t)i * F.crs + (int64_t)j * F.ccs) * F.ob;
    switch (F.ob) {
    case 1: int_finish<1>(F, cp, w); break;
    case 2: int_finish<2>(F, cp, w); break;
    case 4: int_finish<4>(F, cp, w); break;
    case 8: int_finish<8>(F, cp, w); break;
    default: int_finish<16>(F, cp, w); break;
    }
}

// The same for i16 elements (three planes): every term is far inside int64
// (|plane| < 2^31, so |sum of planes << 8s| < 2^48; |ca (sa + sb)| and
// ca^2 k below 2^34 at the limb route's depths, k < 2^16), so the
// combination runs in 64-bit words instead of 128-bit ones; modular lanes
// keep the low 32 bits either way.  cak = ca^2 k.
__global__ void __launch_bounds__(256) limb_combine16_kernel(IArgs F, const int32_t *planes, const int64_t *sa,
                                                             const int64_t *sb, int64_t ca, int64_t cak) {
    const uint64_t j = (uint64_t)blockIdx.x * 256 + threadIdx.x, i = blockIdx.y;
    if (j >= F.n) return;
    const uint64_t cell = i * F.n + j, mn = F.m * F.n;
    const uint64_t p0 = (uint64_t)(int64_t)planes[cell], p1 = (uint64_t)(int64_t)planes[mn + cell],
                   p2 = (uint64_t)(int64_t)planes[2 * mn + cell];
    const int64_t x = (int64_t)((p2 << 16) + (p1 << 8) + p0 + (uint64_t)(ca * (sa[i] + sb[j])) - (uint64_t)cak);
    W192 w{{(uint64_t)x, x < 0 ? ~(uint64_t)0 : 0, x < 0 ? ~(uint64_t)0 : 0}};
    char *cp = F.c + ((int64_t)i * F.crs + (int64_t)j * F.ccs) * F.ob;
    switch (F.ob) {
    case 1: int_finish<1>(F, cp, w); break;
    case 2: int_finish<2>(F, cp, w); break;
    case 4: int_finish<4>(F, cp, w); break;
    case 8: int_finish<8>(F, cp, w); break;
    default: int_finish<16>(F, cp, w); break;
    }
}

struct LimbLayout {
    uint64_t acat, brev, planes, sa, sb, rest;  // byte offsets
    int nplanes;
    bool modular;
};

static uint64_t up256(uint64_t x) { return (x + 255) & ~(uint64_t)255; }

// The limb route's plan, or nplanes = 0 when it does not apply.
static LimbLayout limb_layout(int eb, uint64_t m, uint64_t k, uint64_t n, int out_type, int encode) {
    LimbLayout Y{};
    if (!(eb == 2 || eb == 4) || m == 0 || n == 0 || k == 0) return Y;
    const uint64_t L = (uint64_t)eb;
    Y.modular = encode == UOR_ENCODE_WRAPPING && out_type <= 4;
    if (!Y.modular && L * k >= (1ull << 17)) return Y;
    if (m > 65535 || (n + 255) / 256 > 0x7fffffffull || (k + 255 * LIMB_SPLIT_A) / (256 * LIMB_SPLIT_A) > 0x7fffffffull ||
        (k + LIMB_SPLIT_B - 1) / LIMB_SPLIT_B > 65535)
        return Y;
    Y.nplanes = (int)(2 * L - 1);
    if (Y.modular && Y.nplanes > 4) Y.nplanes = 4;  // 256^s G_s vanishes mod 2^32 for s >= 4
    Y.acat = 0;
    Y.brev = up256(m * L * k);
    Y.planes = Y.brev + up256(L * k * n);
    Y.sa = Y.planes + up256((uint64_t)Y.nplanes * m * n * 4);
    Y.sb = Y.sa + up256(m * 8);
    Y.rest = Y.sb + up256(n * 8);
    return Y;
}

// The limb route's scratch: its buffers plus the dense route's own offer at
// the deepest plane GEMM.
static uint64_t limb_scratch(int eb, uint64_t m, uint64_t k, uint64_t n, int out_type, int encode) {
    const LimbLayout Y = limb_layout(eb, m, k, n, out_type, encode);
    if (!Y.nplanes) return 0;
    return Y.rest + uor_gfx950_suggested_scratch_i8(m, (uint64_t)eb * k, n) + 256;
}

template <int EB>
static int launch_int_limb(const IArgs &F, char *sc, uint64_t have, const LimbLayout &Y, hipStream_t s,
                           int *launches) {
    constexpr int L = EB;
    const uint64_t m = F.m, k = F.k, n = F.n;
    int8_t *acat = (int8_t *)(sc + Y.acat), *brev = (int8_t *)(sc + Y.brev);
    int32_t *planes = (int32_t *)(sc + Y.planes);
    int64_t *sa = (int64_t *)(sc + Y.sa), *sb = (int64_t *)(sc + Y.sb);
    hipLaunchKernelGGL(fill_i64_kernel, dim3((unsigned)((m + 255) / 256)), dim3(256), 0, s, sa, m);
    hipLaunchKernelGGL(fill_i64_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, sb, n);
    hipLaunchKernelGGL(limb_split_a_kernel<EB>,
                       dim3((unsigned)((k + 256 * LIMB_SPLIT_A - 1) / (256 * LIMB_SPLIT_A)), (unsigned)m), dim3(256),
                       0, s, F, acat, sa);
    // Four columns per thread when B's rows are contiguous, n is a multiple
    // of 4 and every row starts 4-element aligned.
    const bool vec4 = F.bcs == 1 && n % 4 == 0 && F.brs % 4 == 0 && ((uintptr_t)F.b % (4 * EB)) == 0;
    if (vec4)
        hipLaunchKernelGGL((limb_split_b_kernel<EB, true>),
                           dim3((unsigned)((n / 4 + 255) / 256), (unsigned)((k + LIMB_SPLIT_B - 1) / LIMB_SPLIT_B)),
                           dim3(256), 0, s, F, brev, sb);
    else
        hipLaunchKernelGGL((limb_split_b_kernel<EB, false>),
                           dim3((unsigned)((n + 255) / 256), (unsigned)((k + LIMB_SPLIT_B - 1) / LIMB_SPLIT_B)),
                           dim3(256), 0, s, F, brev, sb);
    UOR_HIP(hipGetLastError());
    *launches = 4;
    for (int sft = 0; sft < Y.nplanes; ++sft) {
        const int t0 = sft - (L - 1) > 0 ? sft - (L - 1) : 0, t1 = sft < L - 1 ? sft : L - 1;
        const uint64_t depth = (uint64_t)(t1 - t0 + 1) * k;
        const uint64_t v0 = (uint64_t)(L - 1 - sft + t0);
        const uor_view av{acat + (uint64_t)t0 * k, m * (uint64_t)L * k - (uint64_t)t0 * k, m, depth,
                          (int64_t)((uint64_t)L * k), 1};
        const uor_view bv{brev + v0 * k * n, (uint64_t)L * k * n - v0 * k * n, depth, n, (int64_t)n, 1};
        const uor_view cv{planes + (uint64_t)sft * m * n, m * n, m, n, (int64_t)n, 1};
        uor_route r{};
        const int st = uor_gfx950_gemm_i8(&av, &bv, &cv, UOR_OUT_I32, 1, 0,
                                          Y.modular ? UOR_ENCODE_WRAPPING : UOR_ENCODE_NEAREST, sc + Y.rest,
                                          have - Y.rest, (void *)s, &r);
        if (st) return st;
        *launches += r.launches;
    }
    const int64_t ca = L == 2 ? 128 : 128 * (1 + 256 + 65536);
    if (L == 2 && Y.nplanes == 3 && k < (1ull << 16))
        hipLaunchKernelGGL(limb_combine16_kernel, dim3((unsigned)((n + 255) / 256), (unsigned)m), dim3(256), 0, s,
                           F, planes, sa, sb, ca, ca * ca * (int64_t)k);
    else {
        const u128 cak = (u128)((i128)ca * (i128)ca * (i128)k);
        const dim3 grid((unsigned)((n + 255) / 256), (unsigned)m);
        if (Y.nplanes == 3)
            hipLaunchKernelGGL(limb_combine_kernel<3>, grid, dim3(256), 0, s, F, planes, sa, sb, ca, (uint64_t)cak,
                               (uint64_t)(cak >> 64));
        else if (Y.nplanes == 4)
            hipLaunchKernelGGL(limb_combine_kernel<4>, grid, dim3(256), 0, s, F, planes, sa, sb, ca, (uint64_t)cak,
                               (uint64_t)(cak >> 64));
        else  // 2 L - 1 planes, L = 4
            hipLaunchKernelGGL(limb_combine_kernel<7>, grid, dim3(256), 0, s, F, planes, sa, sb, ca, (uint64_t)cak,
                               (uint64_t)(cak >> 64));
    }
    UOR_HIP(hipGetLastError());
    *launches += 1;
    return UOR_OK;
}

extern "C" uint64_t uor_gfx950_suggested_scratch_int(int elem_bytes, uint64_t m, uint64_t k,
                                                     uint64_t n) {
    if (elem_bytes == 1) return uor_gfx950_suggested_scratch_i8(m, k, n);
    if (!(elem_bytes == 2 || elem_bytes == 4 || elem_bytes == 8)) return 0;
    if (m == 0 || n == 0 || k == 0) return 0;
    const uint64_t kc = std::min<uint64_t>(k, CRT_BK_MAX);
    const uint64_t crt = crt_layout(m, kc, n, int_moduli_cap(elem_bytes, k), 1).total + 256;
    // Enough for the limb route under any encode and output (exact planes).
    return std::max(crt, limb_scratch(elem_bytes, m, k, n, UOR_OUT_I64, UOR_ENCODE_NEAREST));
}

extern "C" int uor_gfx950_gemm_int(int elem_bytes, const uor_view *a, const uor_view *b,
                                   const uor_view *c, int out_type, int64_t alpha, int64_t beta,
                                   int encode, void *scratch, uint64_t scratch_bytes, void *stream,
                                   uor_route *route) {
    if (elem_bytes == 1)
        return uor_gfx950_gemm_i8(a, b, c, out_type, alpha, beta, encode, scratch, scratch_bytes, stream,
                                  route);
    route_set(route, UOR_ROUTE_NONE);
    if (!(elem_bytes == 2 || elem_bytes == 4 || elem_bytes == 8) || !valid_out_type(out_type) ||
        !valid_encode(encode))
        return UOR_INVALID_ARGUMENT;
    Placed A, B, C;
    int st = make_triple(a, elem_bytes, b, elem_bytes, c, out_type, &A, &B, &C);
    if (st) return st;
    if (C.rows == 0 || C.cols == 0) return UOR_OK;
    const uintptr_t oalign = (uintptr_t)(out_type < 8 ? out_type : 8) - 1;
    if ((((uintptr_t)A.base | (uintptr_t)B.base) & (uintptr_t)(elem_bytes - 1)) || ((uintptr_t)C.base & oalign))
        return UOR_INVALID_ARGUMENT;
    IArgs F{A.base, A.rs, A.cs, B.base, B.rs, B.cs, C.base, C.rs, C.cs, A.rows, A.cols, B.cols,
            alpha, beta, encode, out_type, elem_bytes == 8 ? 1 : 0};
    hipStream_t s = (hipStream_t)stream;
    // The residue route when the offer holds planes: as many moduli as the
    // element width can need at this depth, or as many as fit (the device
    // plan sends every cell to the per-cell loop if the data needs more).
    // The limb route first: i16 / i32 elements at depths whose limb planes
    // are exact in i32 (any depth for Wrapping into at most 32 bits).
    if (scratch && F.k > 0) {
        const LimbLayout Y = limb_layout(elem_bytes, F.m, F.k, F.n, out_type, encode);
        const uintptr_t p0 = (uintptr_t)scratch, p1 = (p0 + 255) & ~(uintptr_t)255;
        const uint64_t have = scratch_bytes > (p1 - p0) ? scratch_bytes - (p1 - p0) : 0;
        if (Y.nplanes && have >= Y.rest + uor_gfx950_suggested_scratch_i8(F.m, (uint64_t)elem_bytes * F.k, F.n)) {
            int launches = 0;
            const int st2 = elem_bytes == 2 ? launch_int_limb<2>(F, (char *)p1, have, Y, s, &launches)
                                            : launch_int_limb<4>(F, (char *)p1, have, Y, s, &launches);
            if (st2) return st2;
            if (route) {
                route->kind = UOR_ROUTE_INT_LIMB;
                route->tile_m = route->tile_n = 256;
                route->tile_k = DL_BK;
                route->split_k = Y.nplanes;  // plane GEMMs
                route->launches = launches;
                route->moduli = elem_bytes;  // limbs per element
                route->scratch_used = Y.rest;
            }
            return UOR_OK;
        }
    }
    int nm = 0;
    CrtLayout L{};
    char *sc = nullptr;
    const uint64_t kc = std::min<uint64_t>(F.k, CRT_BK_MAX);
    if (scratch && F.k > 0) {
        const uintptr_t p0 = (uintptr_t)scratch, p1 = (p0 + 255) & ~(uintptr_t)255;
        const uint64_t have = scratch_bytes > (p1 - p0) ? scratch_bytes - (p1 - p0) : 0;
        sc = (char *)p1;
        for (int q = int_moduli_cap(elem_bytes, F.k); q >= 1; --q) {
            const CrtLayout Lq = crt_layout(F.m, kc, F.n, q, 1);
            if (Lq.total <= have) {
                nm = q;
                L = Lq;
                break;
            }
        }
        const uint64_t gm = (F.m + 255) / 256, gn = (F.n + 255) / 256;
        if (gm * gn > 0x7fffffffull || F.m > 0x7fffffffull || F.n > 0x7fffffffull) nm = 0;
    }
    if (nm > 0) {
        UOR_HIP(elem_bytes == 2   ? launch_int_crt<2>(F, sc, L, kc, s)
                : elem_bytes == 4 ? launch_int_crt<4>(F, sc, L, kc, s)
                                  : launch_int_crt<8>(F, sc, L, kc, s));
        if (route) {
            route->kind = UOR_ROUTE_INT_CRT;
            route->tile_m = route->tile_n = 256;
            route->tile_k = DL_BK;
            route->split_k = (int)((F.k + kc - 1) / kc);  // depth chunks
            route->launches = 4 + 3 * route->split_k;
            route->moduli = nm;
            route->scratch_used = L.total;
        }
        return UOR_OK;
    }
    if ((F.m + 3) / 4 * ((F.n + 63) / 64) > 0x7fffffffull) return UOR_INVALID_ARGUMENT;
    UOR_HIP(elem_bytes == 2   ? launch_int_direct<2>(F, s)
            : elem_bytes == 4 ? launch_int_direct<4>(F, s)
                              : launch_int_direct<8>(F, s));
    if (route) {
        route->kind = F.k == 0 ? UOR_ROUTE_EPILOGUE_ONLY : UOR_ROUTE_INT_DIRECT;
        route->tile_m = 4;
        route->tile_n = 64;
        route->split_k = 1;
        route->launches = 1;
    }
    return UOR_OK;
}
