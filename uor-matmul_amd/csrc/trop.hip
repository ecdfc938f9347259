// (max, +) GEMM over Trop<i8> on gfx950 VALU.
//
// Replaces the reference's public tropical route, driver::gemm at
// E = Trop<i8> with the MaxPlus epilogue (crates/uor-matmul-gemm/src/
// driver.rs:67-182, epilogue.rs:137-192), whose fastest CPU sequence is the
// packed saturating-i16 TROP_I16 / AVX2_TROP_I16 (crates/uor-matmul-kernels/
// src/tropical.rs:91-166, isa/x86.rs:935-1055).  A max-plus product is not a
// contraction, so there is no MFMA form; it runs on packed 16-bit VALU.
//
// Exactness.  Each Trop<i8> operand becomes an i16: its value when finite,
// NEG (-16384) at the semiring zero.  A finite sum lies in [-256, 254]; a sum
// touching NEG lies in [-16512, -16257], and NEG + NEG = -32768 exactly, so
// plain 16-bit adds never wrap.  The max over k of the sums is therefore the
// exact TropAcc value when some pair is finite, and below -256 exactly when
// every pair touched -inf (tropical.rs:311-318: -inf absorbs).  No depth term
// enters: a max does not grow with k (trop_acc_bits, tropical.rs:289).
//
// Data path.  A 128 x 128 output tile per workgroup of 256 threads, 8 x 8
// cells per thread.  Each k-step of 32 stages A as [row][k] and B as
// [column][k] i16 in LDS; a thread reads eight consecutive k of its rows and
// columns with ds_read_b128 and runs v_pk_add_u16 + v_pk_max_i16 on (k, k+1)
// pairs, so one VALU instruction covers one term and the two halves of each
// cell's accumulator are maxed at the end.

#include "common.hpp"

namespace uor {

typedef short s2 __attribute__((ext_vector_type(2)));
typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int TB = 128;     // tile edge
constexpr int TK = 32;      // k per stage
constexpr int TSTR = TK + 8; // LDS row stride in i16 (80 bytes: conflict-free b128 reads)
constexpr short NEG = -16384;

struct TropArgs {
    const uint8_t *a;  // record (0,0) of A; records are 2 bytes
    int64_t ars, acs;
    const uint8_t *b;
    int64_t brs, bcs;
    uint64_t m, k, n;
    uint8_t *c;  // record (0,0) of C; records are 2*ob bytes
    int64_t crs, ccs;
    int ob;
    int64_t alpha;
    int alpha_finite;
    int64_t beta;
    int beta_finite;
    int mode;
};

__device__ inline short trop16(const uint8_t *rec) {
    const uint16_t r = *(const uint16_t *)rec;  // {value, finite}
    return (r >> 8) ? (short)(int8_t)(r & 0xFF) : NEG;
}

// encode_i128_into over [O::MIN + 1, O::MAX - 1] (tropical.rs:336-350).
__device__ inline i128 trop_encode(i128 v, int bytes, int mode) {
    i128 mn, mx;
    out_range(bytes, &mn, &mx);
    mn += 1;
    mx -= 1;
    if (v >= mn && v <= mx) return v;
    if (mode != UOR_ENCODE_WRAPPING) return v < mn ? mn : mx;
    const u128 span = (u128)mx - (u128)mn + 1;
    const u128 off = (u128)v - (u128)mn;
    return (i128)(off % span + (u128)mn);
}

template <int OB>
__device__ inline void trop_store(uint8_t *p, bool finite, i128 v) {
    store_out<OB>((char *)p, finite ? v : 0);
    p[OB] = finite ? 1 : 0;
}

template <int OB>
__device__ inline void trop_finish(const TropArgs &T, uint64_t i, uint64_t j, int acc) {
    // MaxPlus::finish (epilogue.rs:159-192): (alpha (x) P) (+) (beta (x) C).
    uint8_t *cp = T.c + ((int64_t)i * T.crs + (int64_t)j * T.ccs) * (2 * OB);
    bool fin = acc >= -256 && T.alpha_finite;
    i128 total = fin ? (i128)acc + T.alpha : 0;
    if (T.beta_finite) {
        const bool cf = cp[OB] != 0;
        if (cf) {
            const i128 prior = load_out<OB>((const char *)cp) + (i128)T.beta;
            if (!fin || prior > total) total = prior;
            fin = true;
        }
    }
    if (fin) trop_store<OB>(cp, true, trop_encode(total, OB, T.mode));
    else trop_store<OB>(cp, false, 0);
}

// The witness (gemm_selected, crates/uor-matmul-gemm/src/selection.rs:
// 212-320) wants, beside the maximum, the least p whose term attains it
// (Lex::combine, selection.rs:115-153).  SEL kernels carry (value, index)
// keys in the same packed i16 lanes:
//   A' = a << 6,  B' = (b << 6) + 63 - (p mod 64)       finite operands
//   A' = B' = -32768                                    -inf
// A saturating add (v_pk_add_i16 clamp) of a finite pair is the key
// ((a + b) << 6) | (63 - p mod 64), in [-16384, 16319], ordered by value and
// then by the least p; a pair touching -inf saturates into [-32768, -24577],
// below every finite key.  Every 64 terms each cell's best key is folded into
// a 32-bit key ((v + 257) << 21) + 2^21 - 1 - p, kept as a max: the greatest
// value, then the least p.  Its initial value 2^21 - 1 decodes as "every
// term -inf, witness 0" (selection.rs:179-182, 264-268).  Depth up to 2^21;
// deeper products take the per-cell loop.
constexpr int SEL_BITS = 21;
constexpr int SEL_IDX = (1 << SEL_BITS) - 1;

struct SelArgs {
    TropArgs T;
    uint64_t *w;  // witness (0,0); unused by the plain product
    int64_t wrs, wcs;
};

// Eight Trop<i8> records (16 bytes) -> eight i16 operands, two per dword:
// the value (SEL: value << 6) when the finite byte is nonzero, NEG (SEL:
// -32768) otherwise.
template <bool SEL>
__device__ inline v4i trop16x8(const v4i &r) {
    constexpr int MASKED = SEL ? -32768 : NEG;
    constexpr int SH = SEL ? 6 : 0;
    v4i o;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const uint32_t x = (uint32_t)r[d];
        const int lo = (x & 0x0000FF00u) ? ((int)(int8_t)(x & 0xFF) << SH) : MASKED;
        const int hi = (x & 0xFF000000u) ? ((int)(int8_t)((x >> 16) & 0xFF) << SH) : MASKED;
        o[d] = (int)(((uint32_t)lo & 0xFFFFu) | ((uint32_t)hi << 16));
    }
    return o;
}

// One record -> the A operand (SEL: the B operand adds its index field).
template <bool SEL>
__device__ inline short trop_op(const uint8_t *rec) {
    const short v = trop16(rec);
    if constexpr (!SEL) return v;
    else return v == NEG ? (short)-32768 : (short)(v << 6);
}

__device__ inline short sel_idx6(short op, uint64_t p) {
    return op == (short)-32768 ? op : (short)(op + 63 - (int)(p & 63));
}

// The inner product of one staged k-step: 8 x 8 cells per thread.
template <bool SEL>
__device__ inline void trop_step(const short *As, const short *Bs, int ty, int tx, s2 (&acc)[8][8]) {
#pragma unroll
    for (int p0 = 0; p0 < TK; p0 += 8) {
        v4i av[8], bv[8];
#pragma unroll
        for (int a = 0; a < 8; ++a) av[a] = *(const v4i *)(As + (ty + 16 * a) * TSTR + p0);
#pragma unroll
        for (int b = 0; b < 8; ++b) bv[b] = *(const v4i *)(Bs + (tx + 16 * b) * TSTR + p0);
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
            for (int a = 0; a < 8; ++a)
#pragma unroll
                for (int b = 0; b < 8; ++b) {
                    // Copy the lanes out before the cast: a bit_cast of a
                    // vector-subscript lvalue reads element 0 under this
                    // compiler, whatever the subscript.
                    const int xa = av[a][d], yb = bv[b][d];
                    const s2 x = __builtin_bit_cast(s2, xa);
                    const s2 y = __builtin_bit_cast(s2, yb);
                    if constexpr (SEL)
                        acc[a][b] = __builtin_elementwise_max(acc[a][b], __builtin_elementwise_add_sat(x, y));
                    else
                        acc[a][b] = __builtin_elementwise_max(acc[a][b], x + y);
                }
    }
}

// SEL: fold the i16 keys of the chunk of 64 terms starting at `base` into the
// 32-bit keys, and restart the i16 keys.
__device__ inline void sel_fold(s2 (&acc)[8][8], int (&key)[8][8], uint64_t base) {
    const int k0 = (257 << SEL_BITS) + SEL_IDX - 63 - (int)base;
#pragma unroll
    for (int a = 0; a < 8; ++a)
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const int lo = acc[a][b][0], hi = acc[a][b][1];
            const int s = lo > hi ? lo : hi;
            const int g = (int)((uint32_t)(s >> 6) << SEL_BITS) + (s & 63) + k0;
            key[a][b] = key[a][b] > g ? key[a][b] : g;
            acc[a][b] = s2{-32768, -32768};
        }
}

// One cell's epilogue from its 32-bit key.
__device__ inline void sel_finish(const SelArgs &S, uint64_t i, uint64_t j, int key) {
    const int vf = key >> SEL_BITS;  // key >= 2^21 - 1
    const uint64_t at = (uint64_t)(SEL_IDX - (key & SEL_IDX));
    const int v = vf ? vf - 257 : -32768;  // below -256: every term at -inf
    const TropArgs &T = S.T;
    switch (T.ob) {
    case 1: trop_finish<1>(T, i, j, v); break;
    case 2: trop_finish<2>(T, i, j, v); break;
    case 4: trop_finish<4>(T, i, j, v); break;
    default: trop_finish<8>(T, i, j, v); break;
    }
    S.w[(int64_t)i * S.wrs + (int64_t)j * S.wcs] = at;
}

// FAST: unit record strides along k (A) and n (B), 16-byte aligned rows, k
// and n multiples of 8 (the host checks).  Each k-step's records arrive as
// 16-byte loads of 8 records (two per operand per thread) instead of one
// 2-byte record per load.  (Loading the next step before this step's products,
// into double-buffered LDS, needs 16 more registers than the products leave:
// it spilled.)  SEL: the witness route (k <= 2^21, the host checks).
template <bool FAST, bool SEL>
__global__ void __launch_bounds__(256) trop_i8_kernel(SelArgs S, int gm, int gn) {
    __shared__ __attribute__((aligned(16))) short As[TB * TSTR];
    __shared__ __attribute__((aligned(16))) short Bs[TB * TSTR];
    const TropArgs &T = S.T;
    const int t = threadIdx.x;
    const int ty = t >> 4, tx = t & 15;
    const uint64_t tm = blockIdx.x / gn, tn = blockIdx.x % gn;
    const uint64_t m0 = tm * TB, n0 = tn * TB;

    s2 acc[8][8];
    int key[8][8];
#pragma unroll
    for (int a = 0; a < 8; ++a)
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            acc[a][b] = s2{-32768, -32768};
            if constexpr (SEL) key[a][b] = SEL_IDX;
        }
    // SEL: after the step at k0, fold when a chunk of 64 ends or k does.
    auto fold = [&](uint64_t k0) {
        if constexpr (SEL)
            if ((k0 & 32) || k0 + TK >= T.k) sel_fold(acc, key, k0 & ~(uint64_t)63);
    };

    if constexpr (FAST) {
        // A chunk q = t + 256h: row q/4, records k0 + 8(q%4) ..; B chunk:
        // k-row q/16, columns n0 + 8(q%16) ..  Missing records read as zero
        // bytes, i.e. not finite.
        v4i ra[2], rb[2];
        auto gload = [&](uint64_t k0) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int q = t + 256 * h;
                const uint64_t gi = m0 + (q >> 2), gk = k0 + 8 * (q & 3);
                ra[h] = (gi < T.m && gk < T.k) ? *(const v4i *)(T.a + ((int64_t)gi * T.ars + (int64_t)gk) * 2) : v4i{};
                const uint64_t gr = k0 + (q >> 4), gj = n0 + 8 * (q & 15);
                rb[h] = (gr < T.k && gj < T.n) ? *(const v4i *)(T.b + ((int64_t)gr * T.brs + (int64_t)gj) * 2) : v4i{};
            }
        };
        auto lstore = [&](uint64_t k0) {
            short *as = As, *bs = Bs;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int q = t + 256 * h;
                *(v4i *)(as + (q >> 2) * TSTR + 8 * (q & 3)) = trop16x8<SEL>(ra[h]);
                const v4i v = trop16x8<SEL>(rb[h]);
                const int kr = q >> 4, c8 = 8 * (q & 15);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const uint32_t w = (uint32_t)v[i >> 1];
                    const short e = (short)((i & 1) ? (w >> 16) : (w & 0xFFFF));
                    bs[(c8 + i) * TSTR + kr] = SEL ? sel_idx6(e, k0 + kr) : e;
                }
            }
        };
        for (uint64_t k0 = 0; k0 < T.k; k0 += TK) {
            gload(k0);
            lstore(k0);
            __syncthreads();
            trop_step<SEL>(As, Bs, ty, tx, acc);
            fold(k0);
            __syncthreads();
        }
    } else
    for (uint64_t k0 = 0; k0 < T.k; k0 += TK) {
        constexpr short MASKED = SEL ? (short)-32768 : NEG;
        // A tile: 128 rows x 32 k; consecutive threads walk k.
#pragma unroll 4
        for (int q = 0; q < 16; ++q) {
            const int p = t & 31, r = (t >> 5) + 8 * q;
            const uint64_t gi = m0 + r, gk = k0 + p;
            As[r * TSTR + p] = (gi < T.m && gk < T.k)
                                   ? trop_op<SEL>(T.a + ((int64_t)gi * T.ars + (int64_t)gk * T.acs) * 2)
                                   : MASKED;
        }
        // B tile: 32 k x 128 columns, stored [column][k]; consecutive threads
        // walk columns.
#pragma unroll 4
        for (int q = 0; q < 16; ++q) {
            const int col = t & 127, p = (t >> 7) + 2 * q;
            const uint64_t gj = n0 + col, gk = k0 + p;
            short e = MASKED;
            if (gj < T.n && gk < T.k) {
                e = trop_op<SEL>(T.b + ((int64_t)gk * T.brs + (int64_t)gj * T.bcs) * 2);
                if constexpr (SEL) e = sel_idx6(e, gk);
            }
            Bs[col * TSTR + p] = e;
        }
        __syncthreads();
        trop_step<SEL>(As, Bs, ty, tx, acc);
        fold(k0);
        __syncthreads();
    }

#pragma unroll
    for (int a = 0; a < 8; ++a) {
        const uint64_t i = m0 + ty + 16 * a;
        if (i >= T.m) continue;
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const uint64_t j = n0 + tx + 16 * b;
            if (j >= T.n) continue;
            if constexpr (SEL) {
                sel_finish(S, i, j, key[a][b]);
            } else {
                const int v = acc[a][b][0] > acc[a][b][1] ? acc[a][b][0] : acc[a][b][1];
                switch (T.ob) {
                case 1: trop_finish<1>(T, i, j, v); break;
                case 2: trop_finish<2>(T, i, j, v); break;
                case 4: trop_finish<4>(T, i, j, v); break;
                default: trop_finish<8>(T, i, j, v); break;
                }
            }
        }
    }
}

// The witness past 2^21 terms: the per-cell loop, one thread per cell.
__global__ void __launch_bounds__(256) trop_sel_direct_kernel(SelArgs S) {
    const TropArgs &T = S.T;
    const uint64_t cell = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (cell >= T.m * T.n) return;
    const uint64_t i = cell / T.n, j = cell % T.n;
    int best = -32768;
    uint64_t at = 0;
    for (uint64_t p = 0; p < T.k; ++p) {
        const short x = trop16(T.a + ((int64_t)i * T.ars + (int64_t)p * T.acs) * 2);
        const short y = trop16(T.b + ((int64_t)p * T.brs + (int64_t)j * T.bcs) * 2);
        if (x == NEG || y == NEG) continue;
        const int v = x + y;
        if (v > best) best = v, at = p;
    }
    switch (T.ob) {
    case 1: trop_finish<1>(T, i, j, best); break;
    case 2: trop_finish<2>(T, i, j, best); break;
    case 4: trop_finish<4>(T, i, j, best); break;
    default: trop_finish<8>(T, i, j, best); break;
    }
    S.w[(int64_t)i * S.wrs + (int64_t)j * S.wcs] = at;
}

}  // namespace uor

using namespace uor;

// 16-byte record loads: unit record strides, 16-byte aligned bases and rows,
// k and n multiples of 8 records.
static bool trop_fast(const TropArgs &T) {
    return T.acs == 1 && T.bcs == 1 && ((((uintptr_t)T.a) | ((uintptr_t)T.b)) & 15) == 0 && T.ars > 0 &&
           T.brs > 0 && (T.ars % 8) == 0 && (T.brs % 8) == 0 && T.k % 8 == 0 && T.n % 8 == 0;
}

extern "C" int uor_gfx950_gemm_trop_i8(const uor_view *a, const uor_view *b, const uor_view *c,
                                       int out_type, int64_t alpha, int alpha_finite, int64_t beta,
                                       int beta_finite, int encode, void *scratch,
                                       uint64_t scratch_bytes, void *stream, uor_route *route) {
    (void)scratch;
    (void)scratch_bytes;
    route_set(route, UOR_ROUTE_NONE);
    if (!(out_type == 1 || out_type == 2 || out_type == 4 || out_type == 8)) return UOR_INVALID_ARGUMENT;
    if (!valid_encode(encode)) return UOR_INVALID_ARGUMENT;
    Placed A, B, C;
    // Records: Trop<i8> is 2 bytes; Trop<O> is 2 * sizeof(O).
    int st = make_triple(a, 2, b, 2, c, 2 * out_type, &A, &B, &C);
    if (st) return st;
    if (C.rows == 0 || C.cols == 0) return UOR_OK;
    if (((uintptr_t)A.base | (uintptr_t)B.base) & 1) return UOR_INVALID_ARGUMENT;
    SelArgs S{{(const uint8_t *)A.base, A.rs, A.cs, (const uint8_t *)B.base, B.rs, B.cs, A.rows, A.cols,
               B.cols, (uint8_t *)C.base, C.rs, C.cs, out_type, alpha, alpha_finite != 0, beta,
               beta_finite != 0, encode},
              nullptr, 0, 0};
    const TropArgs &T = S.T;
    const uint64_t gm = (T.m + TB - 1) / TB, gn = (T.n + TB - 1) / TB;
    if (gm * gn > 0x7FFFFFFFull) return UOR_INVALID_ARGUMENT;
    if (route) {
        route->kind = UOR_ROUTE_TROP_VALU;
        route->tile_m = route->tile_n = TB;
        route->tile_k = TK;
        route->split_k = 1;
        route->launches = 1;
    }
    const bool fast = trop_fast(T);
    if (route) route->operand_modes = fast ? 1 : 0;
    if (fast)
        hipLaunchKernelGGL((trop_i8_kernel<true, false>), dim3((unsigned)(gm * gn)), dim3(256), 0,
                           (hipStream_t)stream, S, (int)gm, (int)gn);
    else
        hipLaunchKernelGGL((trop_i8_kernel<false, false>), dim3((unsigned)(gm * gn)), dim3(256), 0,
                           (hipStream_t)stream, S, (int)gm, (int)gn);
    UOR_HIP(hipGetLastError());
    return UOR_OK;
}

extern "C" int uor_gfx950_gemm_trop_i8_selected(const uor_view *a, const uor_view *b, const uor_view *c,
                                                const uor_view *w, int out_type, int64_t alpha,
                                                int alpha_finite, int64_t beta, int beta_finite,
                                                int encode, int mechanism, void *scratch,
                                                uint64_t scratch_bytes, void *stream, uor_route *route) {
    (void)scratch;
    (void)scratch_bytes;
    route_set(route, UOR_ROUTE_NONE);
    if (!(out_type == 1 || out_type == 2 || out_type == 4 || out_type == 8)) return UOR_INVALID_ARGUMENT;
    if (!valid_encode(encode)) return UOR_INVALID_ARGUMENT;
    if (mechanism != UOR_WITNESS_LEXICOGRAPHIC && mechanism != UOR_WITNESS_COMPARE_PASS)
        return UOR_INVALID_ARGUMENT;
    Placed A, B, C, W;
    int st = make_triple(a, 2, b, 2, c, 2 * out_type, &A, &B, &C);
    if (st) return st;
    // SelectedTriple::new (selection.rs:76-98): the witness is m x n and
    // maps no two cells onto one.
    if ((st = place(w, 8, &W))) return st;
    if (W.rows != A.rows || W.cols != B.cols) return UOR_NONCONFORMANT;
    if (self_aliases(W.rows, W.cols, W.rs, W.cs)) return UOR_OUTPUT_ALIASES_ITSELF;
    if (C.rows == 0 || C.cols == 0) return UOR_OK;
    if (((uintptr_t)A.base | (uintptr_t)B.base) & 1) return UOR_INVALID_ARGUMENT;
    if ((uintptr_t)W.base & 7) return UOR_INVALID_ARGUMENT;
    SelArgs S{{(const uint8_t *)A.base, A.rs, A.cs, (const uint8_t *)B.base, B.rs, B.cs, A.rows, A.cols,
               B.cols, (uint8_t *)C.base, C.rs, C.cs, out_type, alpha, alpha_finite != 0, beta,
               beta_finite != 0, encode},
              (uint64_t *)W.base, W.rs, W.cs};
    const TropArgs &T = S.T;
    const uint64_t gm = (T.m + TB - 1) / TB, gn = (T.n + TB - 1) / TB;
    if (gm * gn > 0x7FFFFFFFull) return UOR_INVALID_ARGUMENT;
    // Keys hold the index in 21 bits: deeper products take the per-cell loop.
    const bool tiled = T.k <= (uint64_t)SEL_IDX + 1;
    const bool fast = trop_fast(T);
    if (route) {
        route->kind = tiled ? UOR_ROUTE_TROP_SELECTED : UOR_ROUTE_TROP_SELECTED_DIRECT;
        route->tile_m = route->tile_n = tiled ? TB : 1;
        route->tile_k = tiled ? TK : 1;
        route->split_k = 1;
        route->launches = 1;
        route->operand_modes = tiled && fast ? 1 : 0;
    }
    if (tiled && fast) {
        hipLaunchKernelGGL((trop_i8_kernel<true, true>), dim3((unsigned)(gm * gn)), dim3(256), 0,
                           (hipStream_t)stream, S, (int)gm, (int)gn);
    } else if (tiled) {
        hipLaunchKernelGGL((trop_i8_kernel<false, true>), dim3((unsigned)(gm * gn)), dim3(256), 0,
                           (hipStream_t)stream, S, (int)gm, (int)gn);
    } else {
        const uint64_t cells = T.m * T.n, blocks = (cells + 255) / 256;
        if (blocks > 0x7FFFFFFFull) return UOR_INVALID_ARGUMENT;
        hipLaunchKernelGGL(trop_sel_direct_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, S);
    }
    UOR_HIP(hipGetLastError());
    return UOR_OK;
}
