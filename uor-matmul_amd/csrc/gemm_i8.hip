// Exact i8 x i8 GEMM on gfx950 int8 MFMA.
//
// Replaces the reference's packed auto route for i8 (gemm_auto ->
// gemm_packed_impl -> run, crates/uor-matmul-gemm/src/kernel.rs:523-1377, with
// the KernelSpec::mac_tile sequences of crates/uor-matmul-kernels/src/isa/
// x86.rs:80-96, 704-897) at the whole-product level.
//
// Exactness: each v_mfma_i32_32x32x32_i8 accumulates into i32.  A product of
// two i8 has magnitude <= 2^14, so an i32 lane holds any sum of at most
// KCHUNK = 65536 terms exactly (2^30 < 2^31) -- the reference's lane_depth
// argument (crates/uor-matmul-kernels/src/spec.rs:232-243).  Deeper sums are
// widened into i64 exactly: per-KCHUNK segments are added into i64 registers
// (WIDE) or into an i64 partial-sum workspace with integer atomics (SPLITK),
// which is order-independent, so the bytes never depend on the schedule
// (reference CD-02).  |sum| < 2^63 for every k a device can reach
// (k < 2^49), so i64 holds the exact value the reference keeps in i128.
//
// Data layout in LDS, per operand and pipeline stage: the tile's BK bytes of
// reduction are split in 16-byte chunks; chunk c of tile row r (an m row for
// A, an n column for B) sits at c*CSTRIDE + 16*r + 16*(r/16).  Each MFMA lane
// reads one 16-byte chunk with ds_read_b128; the 16-byte gap every 16 rows and
// the chunk-stride pad keep the 64 lanes on distinct banks for both the
// fragment reads and the transposing dword writes.

#include <stdlib.h>
#include <string.h>

#include <mutex>

#include "mfma_dl.hpp"

namespace uor {

constexpr int KCHUNK = 65536;
constexpr int NTHREADS = 256;

// How an operand tile reaches LDS.
enum : int {
    LOAD_K = 0,   // reduction axis contiguous (row-major A, column-major B): 16B loads
    LOAD_MN = 1,  // m/n axis contiguous (column-major A, row-major B): 16B loads + 4x4 byte transpose
    LOAD_GEN = 2  // any strides, including negative and zero: byte gathers
};

enum : int { EPI_FUSED = 0, EPI_PARTIAL = 1, EPI_WIDE = 2 };

struct OutArgs {
    char *base;  // element (0,0) of C
    int64_t rs, cs;  // in elements
    int ob;          // output bytes
    int64_t alpha, beta;
    int mode;
    long long *work;  // SPLITK: m x n exact partial sums, row-major
};

template <int BMN, int BK>
struct Layout {
    static constexpr int CHUNKS = BK / 16;
    static constexpr int CSTRIDE = BMN * 16 + (BMN / 16) * 16 + 64;
    static constexpr int BYTES = CHUNKS * CSTRIDE;
    __device__ static inline int off(int c, int r) { return c * CSTRIDE + r * 16 + (r >> 4) * 16; }
};

// ---------------------------------------------------------------- loaders --

// Sixteen bytes p[0], p[step], ..., p[15*step], each only if its index is
// below `valid`; missing bytes read as zero.  Fully unrolled so the result
// stays in registers.
__device__ inline v4i gather16(const int8_t *p, int64_t step, uint64_t valid) {
    uint32_t w0 = 0, w1 = 0, w2 = 0, w3 = 0;
#pragma unroll
    for (int b = 0; b < 16; ++b) {
        uint32_t x = (uint64_t)b < valid ? (uint32_t)(uint8_t)p[(int64_t)b * step] : 0u;
        x <<= 8 * (b & 3);
        if (b < 4) w0 |= x;
        else if (b < 8) w1 |= x;
        else if (b < 12) w2 |= x;
        else w3 |= x;
    }
    return v4i{(int)w0, (int)w1, (int)w2, (int)w3};
}

template <int MODE, int BMN, int BK>
struct Loader;

// Reduction axis contiguous: chunk q of the tile is row q/CHUNKS, chunk q%CHUNKS.
template <int BMN, int BK>
struct Loader<LOAD_K, BMN, BK> {
    static constexpr int CHUNKS = BK / 16;
    static constexpr int PER = (BMN * CHUNKS + NTHREADS - 1) / NTHREADS;
    v4i r[PER];

    __device__ inline void load(const Opnd &o, uint64_t mn0, uint64_t k0, uint64_t K) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            int q = threadIdx.x + NTHREADS * i;
            int row = q / CHUNKS, c = q % CHUNKS;
            uint64_t mn = mn0 + row, k = k0 + 16 * c;
            v4i v = {0, 0, 0, 0};
            if (q < BMN * CHUNKS && mn < o.mn && k < K) {
                const int8_t *p = o.base + (int64_t)mn * o.s_mn + (int64_t)k;
                if (k + 16 <= K) v = *(const v4i *)p;
                else v = gather16(p, 1, K - k);
            }
            r[i] = v;
        }
    }
    __device__ inline void store(char *lds) const {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            int q = threadIdx.x + NTHREADS * i;
            if (q < BMN * CHUNKS)
                *(v4i *)(lds + Layout<BMN, BK>::off(q % CHUNKS, q / CHUNKS)) = r[i];
        }
    }
};

// Any strides: the same chunk assignment as LOAD_K, gathered byte by byte.
template <int BMN, int BK>
struct Loader<LOAD_GEN, BMN, BK> {
    static constexpr int CHUNKS = BK / 16;
    static constexpr int PER = (BMN * CHUNKS + NTHREADS - 1) / NTHREADS;
    v4i r[PER];

    __device__ inline void load(const Opnd &o, uint64_t mn0, uint64_t k0, uint64_t K) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            int q = threadIdx.x + NTHREADS * i;
            int row = q / CHUNKS, c = q % CHUNKS;
            uint64_t mn = mn0 + row, k = k0 + 16 * c;
            v4i v = {0, 0, 0, 0};
            if (q < BMN * CHUNKS && mn < o.mn && k < K)
                v = gather16(o.base + (int64_t)mn * o.s_mn + (int64_t)k * o.s_k, o.s_k, K - k);
            r[i] = v;
        }
    }
    __device__ inline void store(char *lds) const {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            int q = threadIdx.x + NTHREADS * i;
            if (q < BMN * CHUNKS)
                *(v4i *)(lds + Layout<BMN, BK>::off(q % CHUNKS, q / CHUNKS)) = r[i];
        }
    }
};

// m/n axis contiguous: a thread loads a 4 (reduction) x 16 (m/n) byte block
// as four 16-byte rows and transposes it into sixteen dwords, each holding
// four consecutive reduction positions of one m/n index.
template <int BMN, int BK>
struct Loader<LOAD_MN, BMN, BK> {
    static constexpr int MB = BMN / 16;           // 16-wide m/n blocks
    static constexpr int BLOCKS = MB * (BK / 4);  // 4-deep reduction blocks
    static constexpr int PER = (BLOCKS + NTHREADS - 1) / NTHREADS;
    v4i r[PER][4];

    __device__ inline void load(const Opnd &o, uint64_t mn0, uint64_t k0, uint64_t K) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            int q = threadIdx.x + NTHREADS * i;
            int mb = q % MB, kb = q / MB;
            uint64_t mn = mn0 + 16 * mb;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                uint64_t k = k0 + 4 * kb + t;
                v4i v = {0, 0, 0, 0};
                if (q < BLOCKS && k < K && mn < o.mn) {
                    const int8_t *p = o.base + (int64_t)k * o.s_k + (int64_t)mn;
                    if (mn + 16 <= o.mn) v = *(const v4i *)p;
                    else v = gather16(p, 1, o.mn - mn);
                }
                r[i][t] = v;
            }
        }
    }
    __device__ inline void store(char *lds) const {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            int q = threadIdx.x + NTHREADS * i;
            if (q >= BLOCKS) continue;
            int mb = q % MB, kb = q / MB;
            int c = kb >> 2, sub = 4 * (kb & 3);
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                uint32_t r0 = r[i][0][d], r1 = r[i][1][d], r2 = r[i][2][d], r3 = r[i][3][d];
                uint32_t lo01 = __builtin_amdgcn_perm(r1, r0, 0x05010400u);
                uint32_t hi01 = __builtin_amdgcn_perm(r1, r0, 0x07030602u);
                uint32_t lo23 = __builtin_amdgcn_perm(r3, r2, 0x05010400u);
                uint32_t hi23 = __builtin_amdgcn_perm(r3, r2, 0x07030602u);
                uint32_t e0 = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u);
                uint32_t e1 = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u);
                uint32_t e2 = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u);
                uint32_t e3 = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u);
                int row = 16 * mb + 4 * d;
                *(uint32_t *)(lds + Layout<BMN, BK>::off(c, row + 0) + sub) = e0;
                *(uint32_t *)(lds + Layout<BMN, BK>::off(c, row + 1) + sub) = e1;
                *(uint32_t *)(lds + Layout<BMN, BK>::off(c, row + 2) + sub) = e2;
                *(uint32_t *)(lds + Layout<BMN, BK>::off(c, row + 3) + sub) = e3;
            }
        }
    }
};

// -------------------------------------------------------------- epilogue --

template <bool FAST>
__device__ inline void finish_any(const OutArgs &o, char *cp, int64_t sum) {
    switch (o.ob) {
    case 1: linear_finish<1, FAST>(cp, sum, o.alpha, o.beta, o.mode); break;
    case 2: linear_finish<2, FAST>(cp, sum, o.alpha, o.beta, o.mode); break;
    case 4: linear_finish<4, FAST>(cp, sum, o.alpha, o.beta, o.mode); break;
    case 8: linear_finish<8, FAST>(cp, sum, o.alpha, o.beta, o.mode); break;
    default: linear_finish<16, false>(cp, sum, o.alpha, o.beta, o.mode); break;
    }
}

// enc(alpha * sum + beta * prior) into i32 for alpha and beta that fit i32:
// two signed 32x32 -> 64 multiply-adds (v_mad_i64_i32, exact: each product is
// below 2^62 in magnitude), then Wrapping keeps the low word and every other
// mode clamps (encode_i128_into, acc.rs:128-150).  The general path's int64
// products cost four 32-bit multiplies and two 64-bit multiply-adds per cell.
// (v_mad_i64_i32 through inline assembly: the compiler spells a sign-extended
// 32x32 -> 64 product with a uniform factor as four 32-bit multiplies.)
__device__ __attribute__((always_inline)) inline int64_t mad_i64_i32(int32_t a, int32_t b, int64_t c) {
    int64_t r;
    uint64_t carry;
    asm("v_mad_i64_i32 %0, %1, %2, %3, %4" : "=v"(r), "=s"(carry) : "v"(a), "s"(b), "v"(c));
    return r;
}

template <bool RD>
__device__ __attribute__((always_inline)) inline int32_t enc32_small(int32_t sum, int32_t prior, int32_t a32,
                                                                     int32_t b32, bool wrap) {
    const int64_t ax = mad_i64_i32(sum, a32, 0);
    const int64_t x = RD ? mad_i64_i32(prior, b32, ax) : ax;
    const int32_t lo = (int32_t)x, hi = (int32_t)(x >> 32);
    const int32_t sat = (hi >> 31) ^ 0x7FFFFFFF;  // INT32_MIN below the range, INT32_MAX above
    return (wrap || hi == (lo >> 31)) ? lo : sat;
}

// Encode one 32x32 accumulator block parked row-major in LDS (row stride 33
// ints) into C.  Lanes 0-31 / 32-63 take columns l32 of rows 2t / 2t+1.
// The C values of a batch are all loaded before any is stored, so their
// loads are in flight together instead of one latency per cell.
template <int OB, bool FAST>
__device__ inline void encode_block(const OutArgs &o, const int *park, uint64_t rbase,
                                    uint64_t col, uint64_t M, uint64_t N) {
    const int lane = threadIdx.x & 63, half = lane >> 5, l32 = lane & 31;
    if (col >= N) return;
    char *const cbase = o.base + (int64_t)col * o.cs * OB;
    const int64_t rstride = o.rs * OB;
    if constexpr (FAST && OB == 4) {
        if (o.alpha == (int32_t)o.alpha && o.beta == (int32_t)o.beta) {
            const int32_t a32 = (int32_t)o.alpha, b32 = (int32_t)o.beta;
            const bool wrap = o.mode == UOR_ENCODE_WRAPPING;
            int32_t prior[16];
            if (b32 != 0) {
#pragma unroll
                for (int t = 0; t < 16; ++t) {
                    const uint64_t row = rbase + 2 * t + half;
                    prior[t] = row < M ? *(const int32_t *)(cbase + (int64_t)row * rstride) : 0;
                }
            }
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                const int lr = 2 * t + half;
                const uint64_t row = rbase + lr;
                if (row >= M) continue;
                const int32_t sum = park[lr * 33 + l32];
                *(int32_t *)(cbase + (int64_t)row * rstride) =
                    b32 != 0 ? enc32_small<true>(sum, prior[t], a32, b32, wrap)
                             : enc32_small<false>(sum, 0, a32, 0, wrap);
            }
            return;
        }
    }
    if constexpr (FAST && OB <= 8) {
        int64_t prior[16];
        if (o.beta != 0) {
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                const uint64_t row = rbase + 2 * t + half;
                prior[t] = row < M ? (int64_t)load_out<OB>(cbase + (int64_t)row * rstride) : 0;
            }
        }
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            const int lr = 2 * t + half;
            const uint64_t row = rbase + lr;
            if (row >= M) continue;
            int64_t x = (int64_t)park[lr * 33 + l32] * o.alpha;
            if (o.beta != 0) x += prior[t] * o.beta;
            store_out<OB>(cbase + (int64_t)row * rstride, encode_int((i128)x, OB, o.mode));
        }
    } else {
        // The full i128 evaluation (huge alpha/beta, or an i128 output): kept
        // rolled and unbatched, so it costs few registers in the kernel.
#pragma unroll 1
        for (int t = 0; t < 16; ++t) {
            const int lr = 2 * t + half;
            const uint64_t row = rbase + lr;
            if (row >= M) continue;
            char *cp = cbase + (int64_t)row * rstride;
            i128 x = sat_mul((i128)park[lr * 33 + l32], o.alpha);
            if (o.beta != 0) x = (i128)((u128)x + (u128)sat_mul(load_out<OB>(cp), o.beta));
            store_out<OB>(cp, encode_int(x, OB, o.mode));
        }
    }
}

// Add one parked 32x32 block into the exact partial-sum workspace.
__device__ inline void partial_block(const OutArgs &o, const int *park, uint64_t rbase,
                                     uint64_t col, uint64_t M, uint64_t N) {
    const int lane = threadIdx.x & 63, half = lane >> 5, l32 = lane & 31;
    if (col >= N) return;
#pragma unroll
    for (int t = 0; t < 16; ++t) {
        const int lr = 2 * t + half;
        const uint64_t row = rbase + lr;
        if (row < M)
            atomicAdd((unsigned long long *)(o.work + row * N + col),
                      (unsigned long long)(int64_t)park[lr * 33 + l32]);
    }
}

// ------------------------------------------------------------------ kernel --

template <int BM, int BN, int BK, int MA, int MB, int EPI, bool FAST>
__global__ void __launch_bounds__(NTHREADS, 1)
gemm_i8_kernel(Opnd A, Opnd B, OutArgs out, uint64_t K, uint64_t kslice, int gm, int gn) {
    static_assert(BM % 64 == 0 && BN % 64 == 0 && BK % 32 == 0, "tile shape");
    constexpr int FM = BM / 64, FN = BN / 64;  // 32x32 MFMA blocks per wave
    using LA = Layout<BM, BK>;
    using LB = Layout<BN, BK>;
    extern __shared__ __attribute__((aligned(16))) char smem[];
    char *const ldsA = smem;                  // two stages of LA::BYTES
    char *const ldsB = smem + 2 * LA::BYTES;  // two stages of LB::BYTES

    int tm, tn;
    tile_of(gm, gn, &tm, &tn);
    const uint64_t m0 = (uint64_t)tm * BM, n0 = (uint64_t)tn * BN;

    uint64_t kbeg = 0, kend = K;
    if constexpr (EPI == EPI_PARTIAL) {
        kbeg = (uint64_t)blockIdx.z * kslice;
        kend = kbeg + kslice < K ? kbeg + kslice : K;
    }

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int half = lane >> 5, l32 = lane & 31;

    v16i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = v16i{};
    [[maybe_unused]] long long wide[FM][FN][16];
    if constexpr (EPI == EPI_WIDE) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) wide[i][j][r] = 0;
    }

    Loader<MA, BM, BK> la;
    Loader<MB, BN, BK> lb;
    const uint64_t nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
    if (nk > 0) {
        la.load(A, m0, kbeg, kend);
        lb.load(B, n0, kbeg, kend);
        la.store(ldsA);
        lb.store(ldsB);
    }
    __syncthreads();

    for (uint64_t kt = 0; kt < nk; ++kt) {
        const int cur = (int)(kt & 1);
        const bool more = kt + 1 < nk;
        if (more) {
            la.load(A, m0, kbeg + (kt + 1) * BK, kend);
            lb.load(B, n0, kbeg + (kt + 1) * BK, kend);
        }
        const char *sa = ldsA + cur * LA::BYTES;
        const char *sb = ldsB + cur * LB::BYTES;
#pragma unroll
        for (int ks = 0; ks < BK / 32; ++ks) {
            v4i af[FM], bf[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i)
                af[i] = *(const v4i *)(sa + LA::off(2 * ks + half, wm * (BM / 2) + 32 * i + l32));
#pragma unroll
            for (int j = 0; j < FN; ++j)
                bf[j] = *(const v4i *)(sb + LB::off(2 * ks + half, wn * (BN / 2) + 32 * j + l32));
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if constexpr (EPI == EPI_WIDE) {
            // Fold the i32 lanes into i64 before they can hold KCHUNK terms.
            if ((((kt + 1) * BK) % KCHUNK) == 0) {
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j) {
#pragma unroll
                        for (int r = 0; r < 16; ++r) wide[i][j][r] += acc[i][j][r];
                        acc[i][j] = v16i{};
                    }
            }
        }
        if (more) {
            la.store(ldsA + (cur ^ 1) * LA::BYTES);
            lb.store(ldsB + (cur ^ 1) * LB::BYTES);
        }
        __syncthreads();
    }

    // Epilogue.  MFMA output register r of lane l in a 32x32 block holds
    // row 8*(r/4) + 4*(l/32) + r%4, column l%32.  Each wave parks one block
    // at a time in its own 4 KiB of LDS (free after the last barrier above)
    // and re-reads it row-major, so the encode runs in a short rolled loop
    // with lanes 0-31 / 32-63 on two consecutive rows.
    int *park = (int *)smem + wave * (32 * 32 + 32);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            if constexpr (EPI == EPI_WIDE) {
                // Two passes of 32-bit halves would lose the exact i64; the
                // wide variant encodes from registers (its tile is one block).
                const uint64_t col = n0 + wn * (BN / 2) + 32 * j + l32;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint64_t row = m0 + wm * (BM / 2) + 32 * i + 8 * (r >> 2) + 4 * half + (r & 3);
                    if (row >= A.mn || col >= B.mn) continue;
                    int64_t s = (int64_t)acc[i][j][r] + wide[i][j][r];
                    char *cp = out.base + ((int64_t)row * out.rs + (int64_t)col * out.cs) * out.ob;
                    finish_any<FAST>(out, cp, s);
                }
            } else {
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    park[(8 * (r >> 2) + 4 * half + (r & 3)) * 33 + l32] = acc[i][j][r];
                __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
                __builtin_amdgcn_wave_barrier();
                const uint64_t col = n0 + wn * (BN / 2) + 32 * j + l32;
                const uint64_t rbase = m0 + wm * (BM / 2) + 32 * i;
                if constexpr (EPI == EPI_PARTIAL) {
                    partial_block(out, park, rbase, col, A.mn, B.mn);
                } else if (col < B.mn) {
                    // Rolled, one cell at a time: the generic-layout kernels
                    // keep their registers for the gathering loaders.
                    for (int t = 0; t < 16; ++t) {
                        const int lr = 2 * t + half;
                        const uint64_t row = rbase + lr;
                        if (row >= A.mn) continue;
                        char *cp = out.base + ((int64_t)row * out.rs + (int64_t)col * out.cs) * out.ob;
                        finish_any<FAST>(out, cp, park[lr * 33 + l32]);
                    }
                }
                __builtin_amdgcn_wave_barrier();
            }
        }
    }
}

// WM x WN waves of 64 lanes (4 waves: one per SIMD, 128x128 each at BM=BN=256;
// 8 waves: two per SIMD, so one wave's LDS reads overlap the other's MFMAs).
// NS > 4: the k loop on a ring of NS stages (dl_mainloop_ring).
template <int BM, int BN, int WM, int WN, int EPI, bool FAST, int OB, bool PF, int NS = DL_NSTAGE>
__global__ void __launch_bounds__(64 * WM * WN, 1)
gemm_i8_dl_kernel(Opnd A, Opnd B, OutArgs out, uint64_t K, uint64_t kslice, int gm, int gn) {
    constexpr int FM = BM / WM / 32, FN = BN / WN / 32;
    using L = DlLayout<BM, BN, NS>;
    static_assert(WM * WN * (32 * 33) * 4 <= L::BYTES, "epilogue parking fits the stages");
    __shared__ __attribute__((aligned(16))) char lds[L::BYTES];
    char *st0 = lds, *st1 = lds + L::A_BYTES, *st2 = lds + 2 * L::A_BYTES, *st3 = lds + 3 * L::A_BYTES;

    int tm, tn;
    tile_of(gm, gn, &tm, &tn);
    const uint64_t m0 = (uint64_t)tm * BM, n0 = (uint64_t)tn * BN;
    // A reduction split takes every splits-th unit of DL_UNIT steps (256
    // bytes of each A row), starting at its own index: the resident splits
    // read neighbouring pieces of every A row at once, and each 128-byte line
    // of A is read whole by one split.  With kslice a multiple of 256, a
    // split sums at most kslice / 64 steps, so its i32 lanes stay exact.
    uint64_t kbeg = 0, kstep = DL_UNIT * DL_BK;
    int nk = (int)(K / DL_BK);
    if constexpr (EPI == EPI_PARTIAL) {
        const uint64_t steps = K / DL_BK, z = blockIdx.z, splits = gridDim.z;
        const uint64_t units = (steps + DL_UNIT - 1) / DL_UNIT;
        const uint64_t nu = z < units ? (units - z + splits - 1) / splits : 0;
        uint64_t n_ = nu * DL_UNIT;
        // The device's last unit may be short; it is this split's last.
        if (nu && (units - 1 - z) % splits == 0 && steps % DL_UNIT) n_ -= DL_UNIT - steps % DL_UNIT;
        kbeg = z * DL_UNIT * DL_BK;
        kstep = splits * DL_UNIT * DL_BK;
        nk = (int)n_;
    }

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int half = lane >> 5, l32 = lane & 31;

    v16i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = v16i{};

    if constexpr (NS != DL_NSTAGE) dl_mainloop_ring<BM, BN, WM, WN, NS>(A, B, m0, n0, kbeg, nk, lds, acc, kstep);
    else if constexpr (PF) dl_mainloop_pf<BM, BN, WM, WN>(A, B, m0, n0, kbeg, nk, st0, st1, st2, st3, acc, kstep);
    else dl_mainloop<BM, BN, WM, WN>(A, B, m0, n0, kbeg, nk, st0, st1, st2, st3, acc, kstep);
    __syncthreads();

    if constexpr (EPI == EPI_FUSED && FAST && OB <= 4 && WM * WN == 8 && FM * FN == 8) {
        // All four stages are free now: each wave parks four 32x32 blocks
        // (16 KiB, row stride 32 ints with the column XOR-swizzled by row bit
        // 2 against bank conflicts) and loads their 64 C values per lane in
        // one batch, so a tile costs two memory round trips per wave.
        static_assert(WM * WN * 16384 <= L::BYTES, "16 KiB of parking per wave");
        int *park4 = (int *)(lds + wave * 16384);
        // i32 output with unit column stride and 16-byte rows: each lane
        // takes four consecutive columns of a parked block, so C moves in
        // 16-byte loads and stores (8 lanes per 128-byte row segment).
        const bool vec = OB == 4 && out.cs == 1 && (out.rs & 3) == 0 && (((uintptr_t)out.base & 15) == 0);
        if constexpr (OB == 4) {
            // A full tile with beta != 0: stream C's 256 rows into the free
            // stages by LDS DMA (two halves of 128 rows, 1 KiB per row, one
            // wave instruction per row) so a CU keeps 128 KiB of C in
            // flight, then combine each accumulator with its prior in place.
            if (vec && out.beta != 0 && m0 + BM <= A.mn && n0 + BN <= B.mn) {
                static_assert(BN == 256 && BM == 256 && L::BYTES >= 128 * 1024, "one 1 KiB row per wave load");
                const int32_t *cbase = (const int32_t *)out.base + (int64_t)m0 * out.rs + (int64_t)n0;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    // Rows 128h + 16 * wave + u, u < 16: row r lands at lds + 1024 * (r - 128h).
#pragma unroll
                    for (int u = 0; u < 16; ++u) {
                        const int r = 16 * wave + u;
                        lds_dma16((const int8_t *)(cbase + (int64_t)(128 * h + r) * out.rs) + 16 * lane,
                                  lds + 1024 * r);
                    }
                    wait_vm<0>();
                    __syncthreads();
                    if (wm == h) {
#pragma unroll
                        for (int i = 0; i < FM; ++i) {
#pragma unroll
                            for (int j = 0; j < FN; ++j) {
                                const int cl = wn * (BN / WN) + 32 * j + l32;
#pragma unroll
                                for (int r = 0; r < 16; ++r) {
                                    const int rl = 32 * i + 8 * (r >> 2) + 4 * half + (r & 3);  // row within the half
                                    const int64_t prior = ((const int32_t *)lds)[rl * 256 + cl];
                                    const int64_t x = (int64_t)acc[i][j][r] * out.alpha + prior * out.beta;
                                    ((int32_t *)out.base)[(int64_t)(m0 + 128 * h + rl) * out.rs + (int64_t)(n0 + cl)] =
                                        (int32_t)encode_int((i128)x, 4, out.mode);
                                }
                            }
                        }
                    }
                    __syncthreads();
                }
                return;
            }
            if (vec) {
                const int rq = lane >> 3, c4 = 4 * (lane & 7);
#pragma unroll
                for (int g = 0; g < 2; ++g) {
                    v4i prior[4][4];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int i = 2 * g + q / 2, j = q % 2;
                        const uint64_t col = n0 + wn * (BN / WN) + 32 * j + c4;
                        const uint64_t rbase = m0 + wm * (BM / WM) + 32 * i;
#pragma unroll
                        for (int t = 0; t < 4; ++t) {
                            const uint64_t row = rbase + 8 * t + rq;
                            prior[q][t] = v4i{};
                            if (out.beta == 0 || row >= A.mn) continue;
                            const int32_t *cp = (const int32_t *)out.base + (int64_t)row * out.rs + (int64_t)col;
                            if (col + 3 < B.mn) {
                                prior[q][t] = *(const v4i *)cp;
                            } else {
#pragma unroll
                                for (int e = 0; e < 4; ++e)
                                    if (col + e < B.mn) prior[q][t][e] = cp[e];
                            }
                        }
                    }
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int i = 2 * g + q / 2, j = q % 2;
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const int row = 8 * (r >> 2) + 4 * half + (r & 3);
                            park4[q * 1024 + row * 32 + (l32 ^ (((row >> 2) & 1) << 4))] = acc[i][j][r];
                        }
                    }
                    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
                    __builtin_amdgcn_wave_barrier();
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int i = 2 * g + q / 2, j = q % 2;
                        const uint64_t col = n0 + wn * (BN / WN) + 32 * j + c4;
                        const uint64_t rbase = m0 + wm * (BM / WM) + 32 * i;
#pragma unroll
                        for (int t = 0; t < 4; ++t) {
                            const int lr = 8 * t + rq;
                            const uint64_t row = rbase + lr;
                            if (row >= A.mn || col >= B.mn) continue;
                            const v4i sum = *(const v4i *)&park4[q * 1024 + lr * 32 + (c4 ^ (((lr >> 2) & 1) << 4))];
                            v4i res;
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                int64_t x = (int64_t)sum[e] * out.alpha;
                                if (out.beta != 0) x += (int64_t)prior[q][t][e] * out.beta;
                                res[e] = (int32_t)encode_int((i128)x, 4, out.mode);
                            }
                            int32_t *cp = (int32_t *)out.base + (int64_t)row * out.rs + (int64_t)col;
                            if (col + 3 < B.mn) {
                                *(v4i *)cp = res;
                            } else {
#pragma unroll
                                for (int e = 0; e < 4; ++e)
                                    if (col + e < B.mn) cp[e] = res[e];
                            }
                        }
                    }
                    __builtin_amdgcn_wave_barrier();
                }
                return;
            }
        }
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            // Blocks q = 0..3 of this batch are (i, j) = (2g + q/2, q%2).
            int32_t prior[4][16];
            if (out.beta != 0) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int i = 2 * g + q / 2, j = q % 2;
                    const uint64_t col = n0 + wn * (BN / WN) + 32 * j + l32;
                    const uint64_t rbase = m0 + wm * (BM / WM) + 32 * i;
#pragma unroll
                    for (int t = 0; t < 16; ++t) {
                        const uint64_t row = rbase + 2 * t + half;
                        prior[q][t] = (row < A.mn && col < B.mn)
                                          ? (int32_t)load_out<OB>(out.base + ((int64_t)row * out.rs + (int64_t)col * out.cs) * OB)
                                          : 0;
                    }
                }
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int i = 2 * g + q / 2, j = q % 2;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = 8 * (r >> 2) + 4 * half + (r & 3);
                    park4[q * 1024 + row * 32 + (l32 ^ (((row >> 2) & 1) << 4))] = acc[i][j][r];
                }
            }
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int i = 2 * g + q / 2, j = q % 2;
                const uint64_t col = n0 + wn * (BN / WN) + 32 * j + l32;
                const uint64_t rbase = m0 + wm * (BM / WM) + 32 * i;
                if (col >= B.mn) continue;
#pragma unroll
                for (int t = 0; t < 16; ++t) {
                    const int lr = 2 * t + half;
                    const uint64_t row = rbase + lr;
                    if (row >= A.mn) continue;
                    int64_t x = (int64_t)park4[q * 1024 + lr * 32 + (l32 ^ (((lr >> 2) & 1) << 4))] * out.alpha;
                    if (out.beta != 0) x += (int64_t)prior[q][t] * out.beta;
                    store_out<OB>(out.base + ((int64_t)row * out.rs + (int64_t)col * out.cs) * OB,
                                  encode_int((i128)x, OB, out.mode));
                }
            }
            __builtin_amdgcn_wave_barrier();
        }
        return;
    }

    int *park = (int *)lds + wave * (32 * 33);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
#pragma unroll
            for (int r = 0; r < 16; ++r)
                park[(8 * (r >> 2) + 4 * half + (r & 3)) * 33 + l32] = acc[i][j][r];
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
            __builtin_amdgcn_wave_barrier();
            const uint64_t col = n0 + wn * (BN / WN) + 32 * j + l32;
            const uint64_t rbase = m0 + wm * (BM / WM) + 32 * i;
            if constexpr (EPI == EPI_PARTIAL) partial_block(out, park, rbase, col, A.mn, B.mn);
            else encode_block<OB, FAST>(out, park, rbase, col, A.mn, B.mn);
            __builtin_amdgcn_wave_barrier();
        }
    }
}

// The 256x256 tile on four scheduled waves (s4_loop), persistent: one
// workgroup per CU walks tiles blockIdx.x, blockIdx.x + gridDim.x, ...  Each
// wave's 128x128 block is 4x4 accumulators of 32x32.  The next tile's first
// three stages are requested before this tile's epilogue, so their loads
// overlap its C traffic.

// The epilogue straight from the accumulators: lane (l32, half) of block
// (i, j) holds column 32j + l32 of rows 8(r>>2) + 4half + (r&3), r < 16, so
// one instruction per r moves two rows of 32 consecutive columns.
//
// A wave whose 128x128 block lies inside C (with non-negative strides and
// offsets below 2^31 bytes) goes through a buffer resource based at the
// block's corner: each access is the lane's 32-bit offset plus a uniform
// scalar offset, so addresses cost no vector registers.  The priors of block
// row i+1 are requested before block row i is combined and stored (fenced, so
// at most two block rows of priors are live), and their waits are partial.
// Any other block takes the per-cell checked path.
// C is touched once per call, so its loads and stores carry the
// non-temporal hint (cache policy bit 1, "nt" on gfx950): measured 5% faster
// at 8192^3 than the default policy.
constexpr int C_NT = 2;
template <int OB>
__device__ inline int64_t buf_load(__amdgpu_buffer_rsrc_t r, int vo, int so) {
    if constexpr (OB == 1) return (int8_t)__builtin_amdgcn_raw_buffer_load_b8(r, vo, so, C_NT);
    else if constexpr (OB == 2) return (int16_t)__builtin_amdgcn_raw_buffer_load_b16(r, vo, so, C_NT);
    else if constexpr (OB == 4) return (int32_t)__builtin_amdgcn_raw_buffer_load_b32(r, vo, so, C_NT);
    else {
        const v2i v = (v2i)__builtin_amdgcn_raw_buffer_load_b64(r, vo, so, C_NT);
        return (int64_t)(((uint64_t)(uint32_t)v[1] << 32) | (uint32_t)v[0]);
    }
}
template <int OB>
__device__ inline void buf_store(__amdgpu_buffer_rsrc_t r, int vo, int so, int64_t x) {
    if constexpr (OB == 1) __builtin_amdgcn_raw_buffer_store_b8((uint8_t)x, r, vo, so, C_NT);
    else if constexpr (OB == 2) __builtin_amdgcn_raw_buffer_store_b16((uint16_t)x, r, vo, so, C_NT);
    else if constexpr (OB == 4) __builtin_amdgcn_raw_buffer_store_b32((uint32_t)x, r, vo, so, C_NT);
    else {
        typedef unsigned int v2u __attribute__((ext_vector_type(2)));
        __builtin_amdgcn_raw_buffer_store_b64(v2u{(unsigned)(uint64_t)x, (unsigned)((uint64_t)x >> 32)}, r, vo, so,
                                              C_NT);
    }
}

// (Always inlined: a call would pass the uniform strides in VGPRs, which the
// "s" constraint below cannot take.)  SMALL: i32 output, alpha and beta in
// i32 (enc32_small); 2: alpha = 1 and beta = 0, the exact sum itself.
template <int OB, bool RD, int SMALL = 0>
__device__ __attribute__((always_inline)) inline void s4_epilogue_full(const OutArgs &out, const v16i (&acc)[4][4], char *corner, int vo,
                                        int srs, int scs) {
    typedef typename std::conditional<OB == 8, int64_t, int32_t>::type P;
    constexpr int NB = OB == 8 ? 1 : 2;  // prior batches in flight
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(corner, 0, 0x7FFFFFFF, 0x00020000);
    // The row stride passes through an empty asm per use, so each offset is
    // formed next to its access instead of all 256 being held in SGPRs.
    auto offs = [&](int i, int j, int r) -> int {
        int rs_ = srs;
        asm volatile("" : "+s"(rs_));
        return (32 * i + 8 * (r >> 2) + (r & 3)) * rs_ + (32 * j) * scs;
    };
    P pr[NB][4][16];
    auto load = [&](int i, P (&p)[4][16]) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) p[j][r] = (P)buf_load<OB>(rs, vo, offs(i, j, r));
    };
    if constexpr (RD && NB == 2) load(0, pr[0]);
    S4_FENCE();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (RD) {
            if constexpr (NB == 2) {
                if (i + 1 < 4) load(i + 1, pr[(i + 1) & 1]);
            } else {
                load(i, pr[0]);
            }
        }
        S4_FENCE();
        const P (&p)[4][16] = pr[NB == 2 ? (i & 1) : 0];
        if constexpr (SMALL == 2) {
            static_assert(OB == 4 && !RD, "the i32 output, no prior");
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) buf_store<OB>(rs, vo, offs(i, j, r), acc[i][j][r]);
        } else if constexpr (SMALL) {
            static_assert(OB == 4, "the i32 output");
            const int32_t a32 = (int32_t)out.alpha, b32 = RD ? (int32_t)out.beta : 0;
            const bool wrap = out.mode == UOR_ENCODE_WRAPPING;
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    buf_store<OB>(rs, vo, offs(i, j, r),
                                  enc32_small<RD>(acc[i][j][r], RD ? (int32_t)p[j][r] : 0, a32, b32, wrap));
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    int64_t x = (int64_t)acc[i][j][r] * out.alpha;
                    if constexpr (RD) x += (int64_t)p[j][r] * out.beta;
                    buf_store<OB>(rs, vo, offs(i, j, r), (int64_t)encode_int((i128)x, OB, out.mode));
                }
        }
        S4_FENCE();
    }
}

template <int OB>
__device__ __attribute__((always_inline)) inline void s4_epilogue_fast(const OutArgs &out, const v16i (&acc)[4][4], uint64_t rw, uint64_t cw,
                                        uint64_t M, uint64_t N) {
    const int lane = threadIdx.x & 63, half = lane >> 5, l32 = lane & 31;
    const bool inside = rw + 128 <= M && cw + 128 <= N;
    const bool small = out.rs >= 0 && out.cs >= 0 && (127 * out.rs + 127 * out.cs + 1) * OB < ((int64_t)1 << 31);
    if (inside && small) {
        const int srs = (int)(out.rs * OB), scs = (int)(out.cs * OB);
        char *const corner = out.base + ((int64_t)rw * out.rs + (int64_t)cw * out.cs) * OB;
        const int vo = 4 * half * srs + l32 * scs;
        const bool small = OB == 4 && out.alpha == (int32_t)out.alpha && out.beta == (int32_t)out.beta;
        if constexpr (OB == 4) {
            if (small) {
                if (out.beta != 0) s4_epilogue_full<OB, true, 1>(out, acc, corner, vo, srs, scs);
                else if (out.alpha == 1) s4_epilogue_full<OB, false, 2>(out, acc, corner, vo, srs, scs);
                else s4_epilogue_full<OB, false, 1>(out, acc, corner, vo, srs, scs);
                return;
            }
        }
        if (out.beta != 0) s4_epilogue_full<OB, true>(out, acc, corner, vo, srs, scs);
        else s4_epilogue_full<OB, false>(out, acc, corner, vo, srs, scs);
        return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint64_t row = rw + 32 * i + 8 * (r >> 2) + 4 * half + (r & 3), col = cw + 32 * j + l32;
                if (row < M && col < N)
                    linear_finish<OB, true>(out.base + ((int64_t)row * out.rs + (int64_t)col * out.cs) * OB,
                                            acc[i][j][r], out.alpha, out.beta, out.mode);
            }
}

// BT: B k-contiguous (column-major), staged in A's layout.
template <bool FAST, int OB, bool BT = false>
__global__ void __launch_bounds__(256, 1)
gemm_i8_s4_kernel(Opnd A, Opnd B, OutArgs out, uint64_t K, int gm, int gn) {
    using L = S4::L;
    constexpr bool DIRECT = FAST && OB <= 8;
    __shared__ __attribute__((aligned(16))) char lds[L::BYTES];
    const int ntiles = gm * gn;
    int tile = blockIdx.x;
    if (tile >= ntiles) return;
    const int nk = (int)(K / DL_BK);
    // (The wave index through readfirstlane: the compiler then knows every
    // block corner, and so every buffer resource the epilogue builds, is
    // uniform, instead of looping over lanes for each access.)
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int half = lane >> 5, l32 = lane & 31;

    S4Lane ln;
    S4Scalars sc;
    s4_setup_lane<BT>(B, lds, ln, sc);
    int tm, tn;
    tile_coords(tile, gm, gn, &tm, &tn);
    s4_setup_tile<BT>(A, B, (uint64_t)tm * 256, (uint64_t)tn * 256, 0, ln, sc);
    s4_prologue(ln, sc, nk);
    for (;;) {
        v16i acc[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = v16i{};
        s4_loop<BT>(ln, sc, nk, acc);
        stage_barrier();  // every wave's stage reads retired: the slots are free
        const uint64_t rw = (uint64_t)tm * 256 + wm * 128, cw = (uint64_t)tn * 256 + wn * 128;
        const int next = tile + (int)gridDim.x;
        int nm = 0, nn = 0;
        if (next < ntiles) tile_coords(next, gm, gn, &nm, &nn);
        if constexpr (DIRECT) {
            if (next < ntiles) {
                s4_setup_tile<BT>(A, B, (uint64_t)nm * 256, (uint64_t)nn * 256, 0, ln, sc);
                s4_prologue(ln, sc, nk);
            }
            s4_epilogue_fast<OB>(out, acc, rw, cw, A.mn, B.mn);
        } else {
            // The full i128 evaluation: one 32x32 block at a time through a
            // padded park, then the next tile's stages.
            int *park = (int *)lds + wave * (32 * 33);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        park[(8 * (r >> 2) + 4 * half + (r & 3)) * 33 + l32] = acc[i][j][r];
                    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
                    __builtin_amdgcn_wave_barrier();
                    encode_block<OB, FAST>(out, park, rw + 32 * i, cw + 32 * j + l32, A.mn, B.mn);
                    __builtin_amdgcn_wave_barrier();
                }
            }
            __syncthreads();
            if (next < ntiles) {
                s4_setup_tile<BT>(A, B, (uint64_t)nm * 256, (uint64_t)nn * 256, 0, ln, sc);
                s4_prologue(ln, sc, nk);
            }
        }
        if (next >= ntiles) break;
        tile = next;
        tm = nm;
        tn = nn;
    }
}

// The encode step over an exact partial-sum workspace (or over a zero sum
// when k == 0: C := enc(beta * C)).
template <bool FAST, bool ZERO>
__global__ void __launch_bounds__(256) finish_kernel(OutArgs out, uint64_t m, uint64_t n) {
    uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= m * n) return;
    uint64_t row = idx / n, col = idx % n;
    int64_t s = ZERO ? 0 : (int64_t)out.work[idx];
    char *cp = out.base + ((int64_t)row * out.rs + (int64_t)col * out.cs) * out.ob;
    finish_any<FAST>(out, cp, s);
}

__global__ void __launch_bounds__(256) zero_i64_kernel(long long *p, uint64_t count) {
    uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx < count) p[idx] = 0;
}

// ------------------------------------------------- deep, narrow-tile split-K --
//
// For A rows far apart in memory (every row its own page, as in the deep
// shapes m = n = 128, k = 2^24), a 128-row tile touches 128 pages per step and
// the address translation, not HBM, sets the pace.  This tile is 32 rows x 128
// columns: a CU touches 32 row pages of A (plus B's one), and the four tiles
// that share B's k-range run on one XCD at the same time (ids 8 apart), so B
// comes from HBM once and from L2 for the others.  Per 256-deep stage: A is
// 32 rows x 256 bytes (8 KiB), B 256 k-rows x 128 bytes (32 KiB), both by
// global_load_lds_dwordx4; three stages in LDS (120 KiB), two in flight.
// Wave w owns columns [32w, 32w + 32): one 32x32 accumulator, eight
// v_mfma_i32_32x32x32_i8 per stage.  Split z sums the stages z, z + splits,
// ... (neighbouring splits read neighbouring 256-byte pieces of every row) and
// folds its i32 lanes into i64 every 256 stages (65 536 terms, |sum| < 2^30),
// then adds its i64 partial into the workspace.
//
// LDS: A row r (0..31), 16-byte chunk x (0..15) at r*256 + 16*(x ^ (r & 15));
// B as the 128-wide direct-to-LDS tile's B half (k*128 + 16*(x ^ swz(k))).
constexpr int DP_BM = 32, DP_BN = 128, DP_BK = 256;
constexpr int DP_A = DP_BM * DP_BK, DP_B = DP_BK * DP_BN, DP_STAGE = DP_A + DP_B;
constexpr int DP_LOADS = DP_STAGE / 1024 / 4;  // global_load_lds per wave per stage (10)
constexpr int DP_FOLD = 256;                   // stages per exact i32 segment

__device__ inline int dp_bswz(int k) { return (2 * (k & 7)) & (DP_BN / 16 - 1); }

__device__ inline void dp_issue(const Opnd &A, const Opnd &B, uint64_t m0, uint64_t n0, uint64_t k0,
                                char *stage) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // A: 512 chunks, slot s = row * 16 + physical chunk p; p holds chunk p ^ (row & 15).
#pragma unroll
    for (int i = 0; i < DP_A / 1024 / 4; ++i) {
        const int base = (wave * (DP_A / 1024 / 4) + i) * 64, slot = base + lane;
        const int row = slot >> 4, x = (slot & 15) ^ (row & 15);
        uint64_t gr = m0 + row;
        if (gr >= A.mn) gr = A.mn - 1;  // rows past m are computed and discarded
        lds_dma16(A.base + (int64_t)gr * A.s_mn + (int64_t)(k0 + 16 * x), stage + base * 16);
    }
    // B: 2048 chunks, slot s = k * 8 + physical chunk p; p holds chunk p ^ swz(k).
    char *bst = stage + DP_A;
#pragma unroll
    for (int i = 0; i < DP_B / 1024 / 4; ++i) {
        const int base = (wave * (DP_B / 1024 / 4) + i) * 64, slot = base + lane;
        const int k = slot >> 3, x = (slot & 7) ^ dp_bswz(k);
        uint64_t gn = n0 + 16 * x;
        if (gn >= B.mn) gn = 0;  // columns past n are computed and discarded
        lds_dma16(B.base + (int64_t)(k0 + k) * B.s_k + (int64_t)gn, bst + base * 16);
    }
}

__device__ inline void dp_compute(const char *st, v16i &acc) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int half = lane >> 5, l32 = lane & 31, grp = lane >> 4, t16 = lane & 15;
    const char *sb = st + DP_A;
    v4i af[DP_BK / 32], bf[DP_BK / 32];
#pragma unroll
    for (int ks = 0; ks < DP_BK / 32; ++ks) {
        const int x = 2 * ks + half;
        af[ks] = *(const v4i *)(st + l32 * DP_BK + 16 * (x ^ (l32 & 15)));
        const int nb = 32 * wave + 16 * (grp & 1) + 8 * (t16 & 1);
        const int k = 32 * ks + 16 * (grp >> 1) + (t16 >> 1);
        v2i lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
            (lds_v2i *)(sb + k * DP_BN + 16 * ((nb >> 4) ^ dp_bswz(k)) + (nb & 8)));
        v2i hi = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
            (lds_v2i *)(sb + (k + 8) * DP_BN + 16 * ((nb >> 4) ^ dp_bswz(k + 8)) + (nb & 8)));
        bf[ks] = v4i{lo[0], lo[1], hi[0], hi[1]};
    }
#pragma unroll
    for (int ks = 0; ks < DP_BK / 32; ++ks) acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[ks], bf[ks], acc, 0, 0, 0);
}

__global__ void __launch_bounds__(256, 1)
gemm_i8_deep_kernel(Opnd A, Opnd B, OutArgs out, uint64_t K, int gm, int gn, int splits) {
    __shared__ __attribute__((aligned(16))) char lds[3 * DP_STAGE];
    char *const s0 = lds, *const s1 = lds + DP_STAGE, *const s2 = lds + 2 * DP_STAGE;
    // id -> (tile, split): ids on one XCD (id % 8) take consecutive tiles of
    // one split, so the tiles sharing B's k-range meet in one L2.
    const int id = blockIdx.x, xcd = id % 8, slot = id / 8, tiles = gm * gn;
    const int tile = slot % tiles, z = (slot / tiles) * 8 + xcd;
    const uint64_t m0 = (uint64_t)(tile % gm) * DP_BM, n0 = (uint64_t)(tile / gm) * DP_BN;
    const uint64_t stages = K / DP_BK;
    const int nk = (uint64_t)z < stages ? (int)((stages - z + splits - 1) / splits) : 0;
    const uint64_t kbeg = (uint64_t)z * DP_BK, kstep = (uint64_t)splits * DP_BK;

    v16i acc = v16i{};
    long long wide[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) wide[r] = 0;
    if (0 < nk) dp_issue(A, B, m0, n0, kbeg, s0);
    if (1 < nk) dp_issue(A, B, m0, n0, kbeg + kstep, s1);
    // Stage t sits in buffer t % 3; step t refills buffer (t + 2) % 3, last
    // read at step t - 1, which every wave has finished once it passes the
    // barrier.
#define UOR_DP_STEP(CUR, NXT)                                                         \
    {                                                                                 \
        if (kt + 1 < nk) wait_vm<DP_LOADS>();                                         \
        else wait_vm<0>();                                                            \
        stage_barrier();                                                              \
        if (kt + 2 < nk) dp_issue(A, B, m0, n0, kbeg + (uint64_t)(kt + 2) * kstep, NXT); \
        dp_compute(CUR, acc);                                                         \
        if ((kt + 1) % DP_FOLD == 0) {                                                \
            _Pragma("unroll") for (int r = 0; r < 16; ++r) wide[r] += acc[r];         \
            acc = v16i{};                                                             \
        }                                                                             \
        if (++kt >= nk) break;                                                        \
    }
    for (int kt = 0; kt < nk;) {
        UOR_DP_STEP(s0, s2)
        UOR_DP_STEP(s1, s0)
        UOR_DP_STEP(s2, s1)
    }
#undef UOR_DP_STEP
    wait_vm<0>();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int half = lane >> 5, l32 = lane & 31;
    const uint64_t col = n0 + 32 * wave + l32;
    if (col >= B.mn) return;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const uint64_t row = m0 + 8 * (r >> 2) + 4 * half + (r & 3);
        const long long v = wide[r] + acc[r];
        if (row < A.mn && v != 0)
            atomicAdd((unsigned long long *)(out.work + row * B.mn + col), (unsigned long long)v);
    }
}

// ------------------------------------------------------------------- host --

template <int BM, int BN, int BK, int MA, int MB, int EPI, bool FAST>
static hipError_t launch_tile(const Opnd &A, const Opnd &B, const OutArgs &out, uint64_t K,
                              uint64_t kslice, int splits, hipStream_t s) {
    constexpr int LDS = 2 * Layout<BM, BK>::BYTES + 2 * Layout<BN, BK>::BYTES;
    auto kern = gemm_i8_kernel<BM, BN, BK, MA, MB, EPI, FAST>;
    static bool configured = false;
    if (!configured) {
        hipError_t e = hipFuncSetAttribute((const void *)kern,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, LDS);
        if (e != hipSuccess) return e;
        configured = true;
    }
    int gm = (int)((A.mn + BM - 1) / BM), gn = (int)((B.mn + BN - 1) / BN);
    dim3 grid((unsigned)(gm * gn), 1, (unsigned)splits);
    hipLaunchKernelGGL(kern, grid, dim3(NTHREADS), LDS, s, A, B, out, K, kslice, gm, gn);
    return hipGetLastError();
}


template <int BM, int BN, int WM, int WN, int EPI, bool FAST, bool PF = false, int NS = DL_NSTAGE>
static hipError_t launch_dl(const Opnd &A, const Opnd &B, const OutArgs &out, uint64_t K,
                            uint64_t kslice, int splits, hipStream_t s) {
    auto kern = gemm_i8_dl_kernel<BM, BN, WM, WN, EPI, FAST, 4, PF, NS>;
    if constexpr (EPI != EPI_PARTIAL) {
        switch (out.ob) {
        case 1: kern = gemm_i8_dl_kernel<BM, BN, WM, WN, EPI, FAST, 1, PF, NS>; break;
        case 2: kern = gemm_i8_dl_kernel<BM, BN, WM, WN, EPI, FAST, 2, PF, NS>; break;
        case 8: kern = gemm_i8_dl_kernel<BM, BN, WM, WN, EPI, FAST, 8, PF, NS>; break;
        case 16: kern = gemm_i8_dl_kernel<BM, BN, WM, WN, EPI, false, 16, PF, NS>; break;
        default: break;
        }
    }
    int gm = (int)((A.mn + BM - 1) / BM), gn = (int)((B.mn + BN - 1) / BN);
    dim3 grid((unsigned)(gm * gn), 1, (unsigned)splits);
    hipLaunchKernelGGL(kern, grid, dim3(64 * WM * WN), 0, s, A, B, out, K, kslice, gm, gn);
    return hipGetLastError();
}

static int device_cus();
// The most 64-wide tiles the ring kernel takes (UOR_GFX950_RING64 overrides,
// for measurement; 0 turns it off).
static int ring64_tiles() {
    static int t = [] {
        const char *e = getenv("UOR_GFX950_RING64");
        return e ? atoi(e) : device_cus();
    }();
    return t;
}

static int device_cus() {
    static int cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess) return 256;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 256;
        return n;
    }();
    return cus;
}

template <bool FAST, bool BT = false>
static hipError_t launch_s4(const Opnd &A, const Opnd &B, const OutArgs &out, uint64_t K, hipStream_t s) {
    auto kern = gemm_i8_s4_kernel<FAST, 4, BT>;
    switch (out.ob) {
    case 1: kern = gemm_i8_s4_kernel<FAST, 1, BT>; break;
    case 2: kern = gemm_i8_s4_kernel<FAST, 2, BT>; break;
    case 8: kern = gemm_i8_s4_kernel<FAST, 8, BT>; break;
    case 16: kern = gemm_i8_s4_kernel<false, 16, BT>; break;
    default: break;
    }
    const int gm = (int)((A.mn + 255) / 256), gn = (int)((B.mn + 255) / 256);
    const int tiles = gm * gn;
    const int grid = tiles < device_cus() ? tiles : device_cus();
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(256), 0, s, A, B, out, K, gm, gn);
    return hipGetLastError();
}

// The scheduled four-wave loop addresses its operands as a 64-bit scalar base
// plus 32-bit per-lane offsets: every row of A and 64 k-rows of B must lie
// within 4 GiB of the operand's base, with positive strides.
static bool s4_ok(const Opnd &A, const Opnd &B) {
    if (A.s_mn <= 0 || B.s_k <= 0) return false;
    const unsigned __int128 a_span = (unsigned __int128)A.mn * (uint64_t)A.s_mn + 64;
    const unsigned __int128 b_span = (unsigned __int128)64 * (uint64_t)B.s_k + B.mn + 16;
    return a_span < ((unsigned __int128)1 << 32) && b_span < ((unsigned __int128)1 << 32);
}

// The same for a k-contiguous B (column-major, the BT loop): every column of
// B within 4 GiB of its base.
static bool s4t_ok(const Opnd &A, const Opnd &B, uint64_t K) {
    if (A.s_mn <= 0 || B.s_mn <= 0 || B.s_k != 1 || K % DL_BK != 0) return false;
    const unsigned __int128 a_span = (unsigned __int128)A.mn * (uint64_t)A.s_mn + 64;
    const unsigned __int128 b_span = (unsigned __int128)B.mn * (uint64_t)B.s_mn + 64;
    return a_span < ((unsigned __int128)1 << 32) && b_span < ((unsigned __int128)1 << 32);
}

// The direct-to-LDS pipeline applies when both operands stream in 16-byte
// chunks along their contiguous axes and every chunk is whole: k a multiple
// of its 64-byte step (of the split slice too) and n of 16.
static bool dl_ok(int pair, uint64_t K, uint64_t N) {
    return pair == 0 && K % DL_BK == 0 && N % 16 == 0;
}

// Operand-mode pairs with a compiled kernel: (row-major A, row-major B),
// (row-major A, column-major B), (column-major A, row-major B),
// (column-major A, column-major B); anything else gathers.
static int mode_pair(int ma, int mb) {
    if (ma == LOAD_K && mb == LOAD_MN) return 0;
    if (ma == LOAD_K && mb == LOAD_K) return 1;
    if (ma == LOAD_MN && mb == LOAD_MN) return 2;
    if (ma == LOAD_MN && mb == LOAD_K) return 3;
    return 4;
}

template <int BM, int BN, int BK, int EPI, bool FAST>
static hipError_t launch_modes(int pair, const Opnd &A, const Opnd &B, const OutArgs &out,
                               uint64_t K, uint64_t kslice, int splits, hipStream_t s) {
    switch (pair) {
    case 0: return launch_tile<BM, BN, BK, LOAD_K, LOAD_MN, EPI, FAST>(A, B, out, K, kslice, splits, s);
    case 1: return launch_tile<BM, BN, BK, LOAD_K, LOAD_K, EPI, FAST>(A, B, out, K, kslice, splits, s);
    case 2: return launch_tile<BM, BN, BK, LOAD_MN, LOAD_MN, EPI, FAST>(A, B, out, K, kslice, splits, s);
    case 3: return launch_tile<BM, BN, BK, LOAD_MN, LOAD_K, EPI, FAST>(A, B, out, K, kslice, splits, s);
    default:
        // Byte gathers need more registers than the 256-wide tile leaves.
        if constexpr (BM <= 128)
            return launch_tile<BM, BN, BK, LOAD_GEN, LOAD_GEN, EPI, FAST>(A, B, out, K, kslice, splits, s);
        else
            return hipErrorInvalidValue;
    }
}

// The operand's load mode: vector loads need the contiguous axis to have unit
// stride and every 16-byte chunk to start 16-byte aligned.
static int load_mode(const Opnd &o) {
    bool aligned = ((uintptr_t)o.base & 15) == 0;
    if (o.s_k == 1 && aligned && (o.s_mn % 16) == 0) return LOAD_K;
    if (o.s_mn == 1 && aligned && (o.s_k % 16) == 0) return LOAD_MN;
    return LOAD_GEN;
}

// FAST: the int64 evaluation of alpha*sum + beta*C equals the i128 one for
// every input of this depth (|a*b| <= 2^14).
static bool fits_fast(int ob, uint64_t K, int64_t alpha, int64_t beta) {
    if (ob > 8) return false;
    long double maxsum = (long double)K * 16384.0L;
    long double bound = fabsl((long double)alpha) * maxsum +
                        fabsl((long double)beta) * ldexpl(1.0L, 8 * ob - 1);
    return bound < ldexpl(1.0L, 62);
}

static uint64_t splitk_bytes(uint64_t m, uint64_t n) { return m * n * 8; }

}  // namespace uor

using namespace uor;

extern "C" const char *uor_gfx950_status_string(int status) {
    switch (status) {
    case UOR_OK: return "ok";
    case UOR_NONCONFORMANT: return "nonconformant";
    case UOR_OUTPUT_ALIASES_ITSELF: return "output_aliases_itself";
    case UOR_SHORT_BUFFER: return "short_buffer";
    case UOR_INVALID_ARGUMENT: return "invalid_argument";
    case UOR_SCRATCH_LIMIT: return "scratch_limit";
    default: return status >= UOR_HIP_ERROR ? "hip_error" : "unknown";
    }
}

extern "C" uint64_t uor_gfx950_suggested_scratch_i8(uint64_t m, uint64_t k, uint64_t n) {
    (void)k;
    // The partial sums, plus the slack that aligns an offer at any address.
    const uint64_t b = splitk_bytes(m, n);
    return b ? b + 256 : 0;
}

template <bool FAST>
static int run_i8(const Placed &PA, const Placed &PB, const Placed &PC, int ob, int64_t alpha,
                  int64_t beta, int mode, void *scratch, uint64_t scratch_bytes, hipStream_t s,
                  uor_route *route) {
    const uint64_t M = PA.rows, K = PA.cols, N = PB.cols;
    Opnd A{(const int8_t *)PA.base, PA.rs, PA.cs, M};
    Opnd B{(const int8_t *)PB.base, PB.cs, PB.rs, N};
    OutArgs out{PC.base, PC.rs, PC.cs, ob, alpha, beta, mode, nullptr};
    const int ma = load_mode(A), mb = load_mode(B);
    const int pair = mode_pair(ma, mb);
    if (route) route->operand_modes = ma | (mb << 2);

    if (K == 0) {
        // alpha * 0 + beta * C: no product, one encode per cell.
        if (route) route->kind = UOR_ROUTE_EPILOGUE_ONLY, route->launches = 1;
        uint64_t cells = M * N;
        hipLaunchKernelGGL((finish_kernel<FAST, true>), dim3((unsigned)((cells + 255) / 256)), dim3(256), 0, s,
                           out, M, N);
        UOR_HIP(hipGetLastError());
        return UOR_OK;
    }

    const uint64_t t256 = ((M + 255) / 256) * ((N + 255) / 256);
    const uint64_t t128 = ((M + 127) / 128) * ((N + 127) / 128);
    const uint64_t t64 = ((M + 63) / 64) * ((N + 63) / 64);
    const bool have_work = scratch && scratch_bytes >= splitk_bytes(M, N);
    // Split the reduction when the output tiles alone cannot fill the 256
    // CUs and the offer holds the exact partial sums, or when the depth
    // exceeds one i32 lane.
    const bool want_split = (K > (uint64_t)KCHUNK) || (t64 < 256 && K >= 8192);
    if (want_split && have_work) {
        // The 128-wide direct-to-LDS tile whenever its layout applies (it
        // streams whole 128-byte B rows, which matters most for the deep,
        // HBM-bound shapes), else 128 or 64 by the tile count.
        const bool dl128 = dl_ok(pair, K, N);
        // A rows at least 1 MiB apart (each its own page) and few output
        // tiles: the 32x128 tile, one resident workgroup per CU, each split
        // folding its own i32 segments (no depth limit per split).
        if (pair == 0 && K % DP_BK == 0 && N % 16 == 0 && A.s_mn >= (1 << 20) && t128 <= 64) {
            const uint64_t gm = (M + DP_BM - 1) / DP_BM, gn = (N + DP_BN - 1) / DP_BN, tiles = gm * gn;
            const uint64_t cus = (uint64_t)device_cus();
            uint64_t splits = (cus + tiles - 1) / tiles;
            splits = (splits + 7) / 8 * 8;
            out.work = (long long *)scratch;
            const uint64_t cells = M * N;
            hipLaunchKernelGGL(zero_i64_kernel, dim3((unsigned)((cells + 255) / 256)), dim3(256), 0, s,
                               out.work, cells);
            UOR_HIP(hipGetLastError());
            hipLaunchKernelGGL(gemm_i8_deep_kernel, dim3((unsigned)(tiles * splits)), dim3(256), 0, s, A, B, out,
                               K, (int)gm, (int)gn, (int)splits);
            UOR_HIP(hipGetLastError());
            hipLaunchKernelGGL((finish_kernel<FAST, false>), dim3((unsigned)((cells + 255) / 256)), dim3(256), 0,
                               s, out, M, N);
            UOR_HIP(hipGetLastError());
            if (route) {
                route->kind = UOR_ROUTE_MFMA_SPLITK;
                route->tile_m = DP_BM;
                route->tile_n = DP_BN;
                route->tile_k = DP_BK;
                route->split_k = (int)splits;
                route->launches = 3;
                route->scratch_used = splitk_bytes(M, N);
            }
            return UOR_OK;
        }
        const int BMN = (t128 >= 64 || dl128) ? 128 : 64;
        const uint64_t tiles = BMN == 128 ? t128 : t64;
        // The 128-wide tile holds 64 KiB of LDS, two workgroups per CU: one
        // resident round of them; the other tiles, 1024 workgroups.
        const uint64_t target = dl128 ? 2 * (uint64_t)device_cus() : 1024;
        uint64_t splits = (target + tiles - 1) / tiles;
        uint64_t min_splits = (K + KCHUNK - 1) / KCHUNK;
        if (splits < min_splits) splits = min_splits;
        uint64_t kslice = (K + splits - 1) / splits;
        kslice = (kslice + 255) / 256 * 256;
        if (kslice > (uint64_t)KCHUNK) kslice = KCHUNK;
        splits = (K + kslice - 1) / kslice;
        // Grid z is 16 bits; a deeper split folds in registers instead.
        if (splits <= 65535) {
        out.work = (long long *)scratch;
        uint64_t cells = M * N;
        hipLaunchKernelGGL(zero_i64_kernel, dim3((unsigned)((cells + 255) / 256)), dim3(256), 0, s,
                           out.work, cells);
        UOR_HIP(hipGetLastError());
        if (BMN == 128 && dl128 && kslice % DL_BK == 0)
            UOR_HIP((launch_dl<128, 128, 2, 2, EPI_PARTIAL, FAST>(A, B, out, K, kslice, (int)splits, s)));
        else if (BMN == 128)
            UOR_HIP((launch_modes<128, 128, 128, EPI_PARTIAL, FAST>(pair, A, B, out, K, kslice, (int)splits, s)));
        else
            UOR_HIP((launch_modes<64, 64, 128, EPI_PARTIAL, FAST>(pair, A, B, out, K, kslice, (int)splits, s)));
        hipLaunchKernelGGL((finish_kernel<FAST, false>), dim3((unsigned)((cells + 255) / 256)), dim3(256), 0,
                           s, out, M, N);
        UOR_HIP(hipGetLastError());
        if (route) {
            route->kind = UOR_ROUTE_MFMA_SPLITK;
            route->tile_m = route->tile_n = BMN;
            route->tile_k = 128;
            route->split_k = (int)splits;
            route->launches = 3;
            route->scratch_used = splitk_bytes(M, N);
        }
        return UOR_OK;
        }
    }
    if (K > (uint64_t)KCHUNK) {
        UOR_HIP((launch_modes<64, 64, 64, EPI_WIDE, FAST>(pair, A, B, out, K, 0, 1, s)));
        if (route) {
            route->kind = UOR_ROUTE_MFMA_WIDE;
            route->tile_m = route->tile_n = 64;
            route->tile_k = 64;
            route->split_k = 1;
            route->launches = 1;
        }
        return UOR_OK;
    }
    // The 256-wide tile also below one tile per CU: at k = 8192 it ran
    // m = 512, n = 28672 (224 tiles) in 0.138 ms, m = 256 in 0.086 ms and
    // m = 128 in 0.080 ms, where the 128-wide tile took 0.337, 0.155 and
    // 0.136 ms (1024 x 4096 x 4096: 0.047 against 0.074 ms).  At 16 tiles the
    // two are even (512 x 2048 x 2048: 0.030 against 0.026 ms), hence 32.
    // From 16 rows up it still wins at depth (64 x 8192 x 28672: 0.091
    // against 0.137 ms; 16 rows 0.088 against 0.128 ms; 24 x 16384 x 16384
    // 0.129 against 0.200 ms) but not at k = 2048 (100 x 2048 x 16384: 0.039
    // against 0.032 ms).
    const bool use256 = t256 >= 256 || (N >= 128 && t256 >= 32 && (M >= 128 || (M >= 16 && K >= 4096)));
    int bm;
    const uint64_t r64 = (uint64_t)ring64_tiles();
    if (dl_ok(pair, K, N) && (t64 <= r64 || (t64 <= 2 * r64 && K <= 2048))) {
        // At most one round of 64-wide tiles (two at k <= 2048): the 64-wide
        // direct-to-LDS tile with sixteen stages of the reduction in flight
        // (128 KiB of LDS), so a short product is not a chain of memory round
        // trips, and a skinny one keeps every CU busy where the 256-wide tiles
        // would leave most idle (kernel times: 1024^3 16.3 -> 9.0 us;
        // 128 x 2048 x 8192 31.2 -> 13.8 us, 128 x 8192 x 8192 74.6 -> 42.5 us,
        // 16 x 8192 x 16384 69.3 -> 41.4 us, 1024 x 1024 x 2048 23.4 -> 14.6 us
        // against the 256-wide tile; 256 x 4096 x 4096 32.2 -> 23.4 us against
        // the 128-wide one).  Two rounds at k = 4096 measured even, at 8192
        // 10% slower (128 x 8192 x 16384: 82.8 against 75.0 us).
        bm = 64;
        UOR_HIP((launch_dl<64, 64, 2, 2, EPI_FUSED, FAST, false, 16>(A, B, out, K, 0, 1, s)));
        if (route) route->operand_modes |= 1 << 4;  // direct-to-LDS pipeline
    } else if (use256 && pair == 1 && dl_variant() == DL_S4 && s4t_ok(A, B, K)) {
        bm = 256;
        UOR_HIP((launch_s4<FAST, true>(A, B, out, K, s)));
        if (route) route->operand_modes |= 1 << 4;  // direct-to-LDS pipeline
    } else if (use256 && dl_ok(pair, K, N)) {
        bm = 256;
        const int v = dl_variant();
        if (v == DL_S4 && s4_ok(A, B)) {
            UOR_HIP((launch_s4<FAST>(A, B, out, K, s)));
        } else switch (v == DL_S4 ? (int)DL_W8PF : v) {
        case DL_W4: UOR_HIP((launch_dl<256, 256, 2, 2, EPI_FUSED, FAST, false>(A, B, out, K, 0, 1, s))); break;
        case DL_W8PF: UOR_HIP((launch_dl<256, 256, 2, 4, EPI_FUSED, FAST, true>(A, B, out, K, 0, 1, s))); break;
        default: UOR_HIP((launch_dl<256, 256, 2, 4, EPI_FUSED, FAST, false>(A, B, out, K, 0, 1, s))); break;
        }
        if (route) route->operand_modes |= 1 << 4;  // direct-to-LDS pipeline
    } else if (FAST && use256 && pair != 4) {
        // (The i128 epilogue does not fit beside a 256-wide generic tile's
        // registers; those requests take the 128-wide tile below.)
        bm = 256;
        if constexpr (FAST) UOR_HIP((launch_modes<256, 256, 64, EPI_FUSED, FAST>(pair, A, B, out, K, 0, 1, s)));
    } else if (dl_ok(pair, K, N) && M >= 128) {
        // Below one round of 256-wide tiles: the 128-wide direct-to-LDS tile
        // (measured 21.3 against 25.9 us at 512 x 2048 x 2048, 32.2 against
        // 46.0 us at 256 x 4096 x 4096 for the generic 64-wide tile; even at
        // 1024^3, 16.4 us, where every tile choice takes the same time).
        bm = 128;
        UOR_HIP((launch_dl<128, 128, 2, 2, EPI_FUSED, FAST>(A, B, out, K, 0, 1, s)));
        if (route) route->operand_modes |= 1 << 4;  // direct-to-LDS pipeline
    } else if (t128 >= 192) {
        bm = 128;
        UOR_HIP((launch_modes<128, 128, 64, EPI_FUSED, FAST>(pair, A, B, out, K, 0, 1, s)));
    } else {
        bm = 64;
        UOR_HIP((launch_modes<64, 64, 64, EPI_FUSED, FAST>(pair, A, B, out, K, 0, 1, s)));
    }
    if (route) {
        route->kind = UOR_ROUTE_MFMA_TILE;
        route->tile_m = route->tile_n = bm;
        route->tile_k = 64;
        route->split_k = 1;
        route->launches = 1;
    }
    return UOR_OK;
}

extern "C" int uor_gfx950_gemm_i8(const uor_view *a, const uor_view *b, const uor_view *c,
                                  int out_type, int64_t alpha, int64_t beta, int encode,
                                  void *scratch, uint64_t scratch_bytes, void *stream,
                                  uor_route *route) {
    route_set(route, UOR_ROUTE_NONE);
    if (!valid_out_type(out_type) || !valid_encode(encode)) return UOR_INVALID_ARGUMENT;
    Placed A, B, C;
    int st = make_triple(a, 1, b, 1, c, out_type, &A, &B, &C);
    if (st) return st;
    if (C.rows == 0 || C.cols == 0) return UOR_OK;
    hipStream_t s = (hipStream_t)stream;
    // The split-K partial sums take 8-byte atomics: the offer from its first
    // aligned byte.
    uint64_t have;
    char *work = offer_align(scratch, scratch_bytes, &have);
    if (fits_fast(out_type, A.cols, alpha, beta))
        return run_i8<true>(A, B, C, out_type, alpha, beta, encode, work, have, s, route);
    return run_i8<false>(A, B, C, out_type, alpha, beta, encode, work, have, s, route);
}

extern "C" int uor_gfx950_slice_gemm_ex_i8(uint64_t m, uint64_t k, uint64_t n, int64_t alpha,
                                           const int8_t *a, uint64_t a_len, uint64_t lda,
                                           const int8_t *b, uint64_t b_len, uint64_t ldb,
                                           int64_t beta, void *c, uint64_t c_len, uint64_t ldc,
                                           int out_type, void *scratch, uint64_t scratch_bytes,
                                           void *stream) {
    // slice.rs:87 ld(): row-major strides {rs: ld, cs: 1}.
    uor_view av{(void *)a, a_len, m, k, (int64_t)lda, 1};
    uor_view bv{(void *)b, b_len, k, n, (int64_t)ldb, 1};
    uor_view cv{c, c_len, m, n, (int64_t)ldc, 1};
    return uor_gfx950_gemm_i8(&av, &bv, &cv, out_type, alpha, beta, UOR_ENCODE_NEAREST, scratch,
                              scratch_bytes, stream, nullptr);
}

extern "C" int uor_gfx950_slice_gemm_i8(uint64_t m, uint64_t k, uint64_t n, const int8_t *a,
                                        uint64_t a_len, const int8_t *b, uint64_t b_len, void *c,
                                        uint64_t c_len, int out_type, void *scratch,
                                        uint64_t scratch_bytes, void *stream) {
    return uor_gfx950_slice_gemm_ex_i8(m, k, n, 1, a, a_len, k, b, b_len, n, 0, c, c_len, n,
                                       out_type, scratch, scratch_bytes, stream);
}

// ---------------------------------------------------- the no-alloc entry --
//
// For callers that cannot allocate device memory (code under graph capture,
// serving loops, harnesses that forbid it): gemm_i8 with its scratch taken
// from this file-scope array instead of an offer.  Each GPU holds its own
// copy until the process ends; host code reaches it only through the
// address hipGetSymbolAddress gives on that device (the array's name is a
// host-side stand-in).  Every call on a GPU shares that GPU's copy, so calls
// that overlap on one GPU race; what must start at zero (the split-K
// partial sums) is cleared by the route itself, in stream order.
static __device__ __align__(256) char scratch[UOR_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::once_flag g_scratch_once[kMaxDevices];
void *g_scratch_ptr[kMaxDevices];
hipError_t g_scratch_err[kMaxDevices];
}  // namespace

extern "C" int uor_gfx950_gemm_i8_noalloc(const uor_view *a, const uor_view *b, const uor_view *c, int out_type,
                                          int64_t alpha, int64_t beta, int encode, void *stream,
                                          uor_route *route) {
    route_set(route, UOR_ROUTE_NONE);
    if (!valid_out_type(out_type) || !valid_encode(encode)) return UOR_INVALID_ARGUMENT;
    Placed A, B, C;
    int st = make_triple(a, 1, b, 1, c, out_type, &A, &B, &C);
    if (st) return st;
    if (C.rows == 0 || C.cols == 0) return UOR_OK;
    // The scratch the fastest route takes (run_i8's split-K partial sums).
    const uint64_t M = A.rows, K = A.cols, N = B.cols;
    const uint64_t t64 = ((M + 63) / 64) * ((N + 63) / 64);
    const bool split = K > (uint64_t)KCHUNK || (t64 < 256 && K >= 8192);
    if (split && splitk_bytes(M, N) > (uint64_t)UOR_NOALLOC_SCRATCH_BYTES) return UOR_SCRATCH_LIMIT;
    int dev = 0;
    UOR_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return UOR_INVALID_ARGUMENT;
    std::call_once(g_scratch_once[dev], [dev] {
        g_scratch_err[dev] = hipGetSymbolAddress(&g_scratch_ptr[dev], HIP_SYMBOL(scratch));
    });
    UOR_HIP(g_scratch_err[dev]);
    void *const ptr = g_scratch_ptr[dev];
    hipStream_t s = (hipStream_t)stream;
    if (fits_fast(out_type, K, alpha, beta))
        return run_i8<true>(A, B, C, out_type, alpha, beta, encode, ptr, UOR_NOALLOC_SCRATCH_BYTES, s, route);
    return run_i8<false>(A, B, C, out_type, alpha, beta, encode, ptr, UOR_NOALLOC_SCRATCH_BYTES, s, route);
}
