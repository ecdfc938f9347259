// 4-bit table-lookup GEMM on gfx950: C = A * W^T with W coded as
// Packed<Grid<i8,16>,2> and one 16-entry i8 codebook per group of coded rows.
//
// Replaces the reference's gemm_tabulated over a TabulatedTriple
// (crates/uor-matmul-gemm/src/tabulated.rs:607-658, 2555-2745) for the i8
// element family and the packed 4-bit codec (crates/uor-matmul-codec/src/
// codecs.rs:80-259; low nibble = even k, CK-03).  The value is the reference's
// exactly: every product of an i8 activation and an i8 decoded weight is exact
// in the i32 lanes (|sum| <= k * 2^14 < 2^31 for k < 2^17; deeper rows fold
// into i64), then Linear{alpha, beta} and the one encode.
//
// Decode.  A code dword holds 8 nibbles: byte b's low nibble is weight 2b, its
// high nibble weight 2b+1.  With the column's codebook in four SGPRs
// (entries 0-3, 4-7, 8-11, 12-15), v_perm_b32 picks entries 0-7 and 8-15 for
// four nibbles at once (selector = nibble & 7), and a third v_perm_b32 picks
// between the two per byte (selector = byte index + 4 * bit 3).  The even
// weights [w0 w2 w4 w6] and odd weights [w1 w3 w5 w7] come out as two dwords;
// the activations they meet are permuted into the same order, once.
//
// Algorithmic bytes per call: n*k/2 (codes) + m*k (A) + m*n*out (C) + books;
// the codes dominate at decode shapes, so the kernels are built to stream
// them: every code byte is read from HBM exactly once.

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>

#include <type_traits>

#include "common.hpp"

namespace uor {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

struct LutArgs {
    const int8_t *a;  // element (0,0) of A
    int64_t ars, acs;
    const uint8_t *codes;  // coded row j at codes + j * half
    uint64_t half;         // k / 2
    const int8_t *books;
    uint64_t group;
    uint64_t m, k, n;
    char *c;  // element (0,0) of C
    int64_t crs, ccs;
    int ob;
    int64_t alpha, beta;
    int mode;
    uint32_t sel_mask, sel_base;  // 0x04040404, 0x03020100 (kernel arguments, so they live in SGPRs)
    // j / group for 32-bit j as ((hi(j * gm) + ((j - hi) >> gs1)) >> gs2)
    // (Granlund & Montgomery, division by invariant integers, fig. 4.1),
    // set by lut_group_magic; the tile kernels use it for their codebook rows.
    uint32_t gm, gs1, gs2;
};

// The magic numbers of LutArgs for a divisor d (1 <= d < 2^32): with
// l = ceil(log2 d), m = floor(2^32 (2^l - d) / d) + 1, s1 = min(l, 1),
// s2 = max(l - 1, 0), exact for every 32-bit dividend.
static void lut_group_magic(LutArgs &L, uint64_t d) {
    if (d > 0x80000000ull) d = 0x80000000ull;  // the tile kernels' columns are far below 2^31
    uint32_t l = 0;
    while ((1ull << l) < d) ++l;
    L.gm = (uint32_t)(((1ull << 32) * ((1ull << l) - d)) / d + 1);
    L.gs1 = l < 1 ? l : 1;
    L.gs2 = l > 0 ? l - 1 : 0;
}

// Column j's codebook row, j < 2^32.
__device__ inline uint32_t lut_group_of(uint32_t j, uint32_t gm, uint32_t gs1, uint32_t gs2) {
    const uint32_t t = __umulhi(j, gm);
    return (t + ((j - t) >> gs1)) >> gs2;
}

__device__ inline uint32_t perm(uint32_t s0, uint32_t s1, uint32_t sel) {
    return __builtin_amdgcn_perm(s0, s1, sel);
}

// 8 weights of one code dword through the codebook (q0..q3 = entries 0-3,
// 4-7, 8-11, 12-15): even = [w0 w2 w4 w6], odd = [w1 w3 w5 w7].
// v_and_or_b32 with the mask in an SGPR and the base in a VGPR (one SGPR per
// VALU op on gfx950): (x & m) | c in one instruction
// (gfx9 VOP3 takes no literal constants, so the compiler would otherwise
// spend an AND and an OR).
__device__ inline uint32_t and_or(uint32_t x, uint32_t m, uint32_t c) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "s"(m), "v"(c));
    return r;
}

__device__ inline void decode8(uint32_t w, uint32_t q0, uint32_t q1, uint32_t q2, uint32_t q3,
                               uint32_t m4, uint32_t id, uint32_t &even, uint32_t &odd) {
    // Final selector byte i = i + 4 * (nibble bit 3).
    uint32_t s = w & 0x07070707u;
    uint32_t lo = perm(q1, q0, s), hi = perm(q3, q2, s);
    even = perm(hi, lo, and_or(w >> 1, m4, id));
    s = (w >> 4) & 0x07070707u;
    lo = perm(q1, q0, s);
    hi = perm(q3, q2, s);
    odd = perm(hi, lo, and_or(w >> 5, m4, id));
}

// Eight activations A[row][k .. k+8) (zero past k_end or for a row past m)
// as (even, odd) dwords in the decode's order.
__device__ inline void act8(const LutArgs &L, uint64_t row, uint64_t k, bool fast, uint32_t &even,
                            uint32_t &odd) {
    uint32_t x0 = 0, x1 = 0;
    if (row < L.m && k < L.k) {
        const int8_t *p = L.a + (int64_t)row * L.ars + (int64_t)k * L.acs;
        if (fast && k + 8 <= L.k) {
            const uint2 v = *(const uint2 *)p;
            x0 = v.x;
            x1 = v.y;
        } else {
#pragma unroll
            for (int b = 0; b < 8; ++b) {
                const uint32_t byte =
                    k + b < L.k ? (uint32_t)(uint8_t)p[(int64_t)b * L.acs] : 0u;
                if (b < 4) x0 |= byte << (8 * b);
                else x1 |= byte << (8 * (b - 4));
            }
        }
    }
    even = perm(x1, x0, 0x06040200u);
    odd = perm(x1, x0, 0x07050301u);
}

// Sixteen code bytes of coded row j starting at byte `off` of the row (zero
// past the row's end or for a column past n).
__device__ inline uint4 codes16(const LutArgs &L, uint64_t j, uint64_t off, bool fast) {
    if (j >= L.n || off >= L.half) return make_uint4(0, 0, 0, 0);
    const uint8_t *p = L.codes + j * L.half + off;
    if (fast && off + 16 <= L.half) return *(const uint4 *)p;
    uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
    for (int b = 0; b < 16; ++b) {
        const uint32_t byte = off + b < L.half ? (uint32_t)p[b] : 0u;
        if (b < 4) w[0] |= byte << (8 * b);
        else if (b < 8) w[1] |= byte << (8 * (b - 4));
        else if (b < 12) w[2] |= byte << (8 * (b - 8));
        else w[3] |= byte << (8 * (b - 12));
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
}

// The four dwords of coded row j's codebook (entries 0-3, 4-7, 8-11, 12-15).
__device__ inline void load_book(const LutArgs &L, uint64_t j, bool aligned, uint32_t &q0,
                                 uint32_t &q1, uint32_t &q2, uint32_t &q3) {
    const int8_t *b = L.books + (j / L.group) * 16;
    if (aligned) {
        const uint32_t *w = (const uint32_t *)b;
        q0 = w[0]; q1 = w[1]; q2 = w[2]; q3 = w[3];
        return;
    }
    uint32_t q[4] = {0, 0, 0, 0};
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const uint32_t byte = (uint32_t)(uint8_t)b[e] << (8 * (e & 3));
        if (e < 4) q[0] |= byte;
        else if (e < 8) q[1] |= byte;
        else if (e < 12) q[2] |= byte;
        else q[3] |= byte;
    }
    q0 = q[0]; q1 = q[1]; q2 = q[2]; q3 = q[3];
}

template <int OB>
__device__ inline void lut_finish(const LutArgs &L, uint64_t row, uint64_t col, int64_t sum) {
    char *cp = L.c + ((int64_t)row * L.crs + (int64_t)col * L.ccs) * OB;
    linear_finish<OB, false>(cp, sum, L.alpha, L.beta, L.mode);
}

__device__ inline void lut_finish_any(const LutArgs &L, uint64_t row, uint64_t col, int64_t sum) {
    switch (L.ob) {
    case 1: lut_finish<1>(L, row, col, sum); break;
    case 2: lut_finish<2>(L, row, col, sum); break;
    case 4: lut_finish<4>(L, row, col, sum); break;
    case 8: lut_finish<8>(L, row, col, sum); break;
    default: lut_finish<16>(L, row, col, sum); break;
    }
}

__device__ inline int wave_sum(int v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// ------------------------------------------------ m <= 4: one wave per column
//
// A segment of 8192 weights is 64 lanes x 4 chunks x 32 weights; chunk c of
// lane l covers weights [(64c + l) * 32, +32) of the segment, i.e. code bytes
// [(64c + l) * 16, +16), so each code load instruction of the wave reads 1 KiB
// contiguously.  The lane's activations for the segment (MR rows x 128
// weights) sit in registers, permuted to the decode's order, and are reused
// for every column the wave visits.
constexpr int LUT_SEG = 8192;

template <bool FAST>
__device__ inline uint4 code_chunk(const LutArgs &L, uint64_t j, uint64_t off) {
    if constexpr (FAST) {
        // Rows are whole 16-byte chunks (k/2 % 16 == 0, 16-byte aligned).
        if (j < L.n && off < L.half) return *(const uint4 *)(L.codes + j * L.half + off);
        return make_uint4(0, 0, 0, 0);
    } else {
        return codes16(L, j, off, false);
    }
}

template <int MR, bool FAST>
__global__ void __launch_bounds__(256) lut4_dot4_kernel(LutArgs L, int book_aligned) {
    const int lane = threadIdx.x & 63;
    const uint64_t wave = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const uint64_t nwaves = ((uint64_t)gridDim.x * blockDim.x) >> 6;
    const bool segs1 = L.k <= (uint64_t)LUT_SEG;
    const uint32_t m4 = __builtin_amdgcn_readfirstlane(L.sel_mask), id = __builtin_amdgcn_readfirstlane(L.sel_base);

    uint32_t ae[MR][4][4], ao[MR][4][4];
    auto load_act = [&](uint64_t k0) {
#pragma unroll
        for (int r = 0; r < MR; ++r)
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int d = 0; d < 4; ++d)
                    act8(L, r, k0 + (uint64_t)(64 * c + lane) * 32 + 8 * d, FAST, ae[r][c][d], ao[r][c][d]);
    };
    if (segs1) load_act(0);

    // Two columns per pass, j and j + nwaves: their decodes and their wave
    // reductions are independent, so each hides the other's latency.
    for (uint64_t j = wave; j < L.n; j += 2 * nwaves) {
        const uint64_t jj[2] = {j, j + nwaves};
        uint32_t q[2][4];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const uint64_t ju = jj[u] < L.n ? jj[u] : j;
            load_book(L, ju, book_aligned, q[u][0], q[u][1], q[u][2], q[u][3]);
#pragma unroll
            for (int e = 0; e < 4; ++e) q[u][e] = __builtin_amdgcn_readfirstlane(q[u][e]);
        }
        int acc[2][MR];
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int r = 0; r < MR; ++r) acc[u][r] = 0;
        for (uint64_t k0 = 0; k0 < L.k; k0 += LUT_SEG) {
            if (!segs1) load_act(k0);
            uint4 cw[2][4];
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    cw[u][c] = code_chunk<FAST>(L, jj[u], k0 / 2 + (uint64_t)(64 * c + lane) * 16);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
#pragma unroll
                for (int d = 0; d < 4; ++d) {
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const uint32_t w = d == 0 ? cw[u][c].x : d == 1 ? cw[u][c].y : d == 2 ? cw[u][c].z : cw[u][c].w;
                        uint32_t e, o;
                        decode8(w, q[u][0], q[u][1], q[u][2], q[u][3], m4, id, e, o);
#pragma unroll
                        for (int r = 0; r < MR; ++r) {
                            acc[u][r] = __builtin_amdgcn_sdot4((int)e, (int)ae[r][c][d], acc[u][r], false);
                            acc[u][r] = __builtin_amdgcn_sdot4((int)o, (int)ao[r][c][d], acc[u][r], false);
                        }
                    }
                }
            }
        }
        // (k <= 65536 here: the host sends deeper rows to the MFMA kernel,
        // whose partial sums fold into i64.)
#pragma unroll
        for (int r = 0; r < MR; ++r) {
            int s0 = acc[0][r], s1 = acc[1][r];
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) {
                s0 += __shfl_xor(s0, o, 64);
                s1 += __shfl_xor(s1, o, 64);
            }
            if (lane == r && (uint64_t)r < L.m) lut_finish_any(L, r, jj[0], s0);
            if (lane == 32 + r && (uint64_t)r < L.m && jj[1] < L.n) lut_finish_any(L, r, jj[1], s1);
        }
    }
}

// The same decode, software-pipelined for k <= LUT_SEG: one column per step,
// with the code chunks and codebooks of the next two columns requested
// before the current one is decoded (a ring of three register buffers,
// unrolled by three so nothing is copied), so a wave keeps two columns (8 KiB)
// of codes in flight.  The activations, the same for every column, sit in
// LDS (MR x 8 KiB per workgroup, in the decode's order, lane-contiguous).
template <int MR, bool FAST>
__global__ void __launch_bounds__(256) lut4_dot4_pf_kernel(LutArgs L, int book_aligned) {
    __shared__ uint32_t act[MR][4][4][2][64];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const uint64_t wave = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const uint64_t nwaves = ((uint64_t)gridDim.x * blockDim.x) >> 6;
    const uint32_t m4 = __builtin_amdgcn_readfirstlane(L.sel_mask), id = __builtin_amdgcn_readfirstlane(L.sel_base);

    // The block's four waves fill the activation table together.
    for (int q = wv; q < MR * 16; q += 4) {
        const int r = q / 16, c = (q / 4) % 4, d = q % 4;
        uint32_t e, o;
        act8(L, r, (uint64_t)(64 * c + lane) * 32 + 8 * d, FAST, e, o);
        act[r][c][d][0][lane] = e;
        act[r][c][d][1][lane] = o;
    }
    __syncthreads();

    struct Col {
        uint4 cw[4];
        uint32_t q[4];
    };
    auto fetch = [&](uint64_t jf, Col &b) {
        load_book(L, jf, book_aligned, b.q[0], b.q[1], b.q[2], b.q[3]);
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) b.cw[cc] = code_chunk<FAST>(L, jf, (uint64_t)(64 * cc + lane) * 16);
    };
    typedef __attribute__((address_space(3))) const uint32_t lds_u32;
    int slot = 0, pend_sum = 0, pend_row = 0;  // slot: wave-uniform
    uint64_t pend_col = ~0ull;
    auto flush = [&]() {
        if (pend_col < L.n && (uint64_t)pend_row < L.m) lut_finish_any(L, pend_row, pend_col, pend_sum);
        pend_col = ~0ull;
        slot = 0;
    };
    auto compute = [&](uint64_t jc, const Col &b) {
        // The table's address passes through an empty asm each step, so the
        // compiler reads it from LDS per use instead of holding all of it in
        // registers across the loop.
        uint32_t abase = (uint32_t)(uintptr_t)(lds_u32 *)&act[0][0][0][0][lane];
        asm volatile("" : "+v"(abase));
        lds_u32 *ap = (lds_u32 *)(uintptr_t)abase;
        uint32_t qs[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) qs[e] = __builtin_amdgcn_readfirstlane(b.q[e]);
        int acc[MR];
#pragma unroll
        for (int r = 0; r < MR; ++r) acc[r] = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const uint32_t w = d == 0 ? b.cw[c].x : d == 1 ? b.cw[c].y : d == 2 ? b.cw[c].z : b.cw[c].w;
                uint32_t e, o;
                decode8(w, qs[0], qs[1], qs[2], qs[3], m4, id, e, o);
#pragma unroll
                for (int r = 0; r < MR; ++r) {
                    acc[r] = __builtin_amdgcn_sdot4((int)e, (int)ap[(((r * 4 + c) * 4 + d) * 2 + 0) * 64], acc[r], false);
                    acc[r] = __builtin_amdgcn_sdot4((int)o, (int)ap[(((r * 4 + c) * 4 + d) * 2 + 1) * 64], acc[r], false);
                }
            }
        }
        // Park each (row, column) sum on its own lane; the finish runs for
        // 64 of them at once (one pass of the output encode per 64 sums, not
        // one per sum with a single lane active).
#pragma unroll
        for (int r = 0; r < MR; ++r) {
            const int sum = wave_sum(acc[r]);
            if (lane == slot + r) pend_sum = sum, pend_row = r, pend_col = jc;
        }
        slot += MR;
        if (slot == 64) flush();
    };
    Col b0, b1, b2;
    uint64_t j = wave;
    if (j < L.n) fetch(j, b0);
    if (j + nwaves < L.n) fetch(j + nwaves, b1);
#define UOR_LUT_STEP(CUR, NN)                                    \
    {                                                            \
        if (j + 2 * nwaves < L.n) fetch(j + 2 * nwaves, NN);     \
        compute(j, CUR);                                         \
        j += nwaves;                                             \
        if (j >= L.n) break;                                     \
    }
    while (j < L.n) {
        UOR_LUT_STEP(b0, b2)
        UOR_LUT_STEP(b1, b0)
        UOR_LUT_STEP(b2, b1)
    }
#undef UOR_LUT_STEP
    flush();
}

// Resident blocks of a kernel on the whole device (one persistent round).
template <typename K>
static unsigned resident_blocks(K kern) {
    int dev = 0, cus = 0, per = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 1024;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 1024;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kern, 256, 0) != hipSuccess || per < 1) per = 1;
    return (unsigned)(per * cus);
}

static int device_cus_lut() {
    static int cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess) return 256;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 256;
        return n;
    }();
    return cus;
}

// The 16-column tile kernel for the decode shapes (UOR_GFX950_LUT_TILE=off
// turns it off, for measuring the kernels it replaced).
static bool lut_tile_on() {
    static bool on = [] {
        const char *e = getenv("UOR_GFX950_LUT_TILE");
        return !(e && !strcmp(e, "off"));
    }();
    return on;
}
// Waves per workgroup of the 16-column tile kernel (UOR_GFX950_LUT_TILE=8 or
// 16, for measurement; 16, the default, measured 23.3 against 24.7 us at
// m = 1 and the config weights).  Either value also turns the 8-column
// kernel off, so the 16-column one runs at every m it takes.
static int lut_tile_waves() {
    static int w = [] {
        const char *e = getenv("UOR_GFX950_LUT_TILE");
        return (e && !strcmp(e, "8")) ? 8 : 16;
    }();
    return w;
}
static bool lut_tile8_on() {
    static bool on = [] {
        const char *e = getenv("UOR_GFX950_LUT_TILE");
        return !(e && (!strcmp(e, "8") || !strcmp(e, "16")));
    }();
    return on;
}

static int lut_variant() {
    static int v = [] {
        const char *e = getenv("UOR_GFX950_LUT_VARIANT");
        return (e && e[0] == 'b') ? 0 : 1;  // "base": no pipelining
    }();
    return v;
}

// --------------------------------------- m > 4: decoded weights into MFMA
//
// A workgroup of 4 waves owns a 32-row x 32-column output tile; wave w sums
// the w-th quarter of k.  Lane l handles coded row (column) j0 + l%32 and
// half h = l/32 of each 128-weight step: its 32 code bytes cover weights
// [64h, 64h+64) of the step and decode into four MFMA B operands; the
// matching A operands are 16 activations each, permuted the same way.  The
// four quarters meet in LDS as exact i64 sums.
__global__ void __launch_bounds__(256) lut4_mfma_kernel(LutArgs L, int fast, int book_aligned, uint64_t kq) {
    __shared__ long long red[4][32 * 33];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int jl = lane & 31, h = lane >> 5;
    const uint64_t ntile = (L.n + 31) / 32;
    const uint64_t col_tile = blockIdx.x % ntile, row_tile = blockIdx.x / ntile;
    const uint64_t j0 = col_tile * 32, r0 = row_tile * 32;
    const uint64_t j = j0 + jl;
    const uint64_t kbeg = (uint64_t)wave * kq;
    const uint64_t kend = min(L.k, kbeg + kq);
    const uint32_t m4 = __builtin_amdgcn_readfirstlane(L.sel_mask), id = __builtin_amdgcn_readfirstlane(L.sel_base);

    uint32_t q0 = 0, q1 = 0, q2 = 0, q3 = 0;
    if (j < L.n) load_book(L, j, book_aligned, q0, q1, q2, q3);
    v16i acc = v16i{};
    long long wide[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) wide[r] = 0;
    uint64_t since_fold = 0;

    for (uint64_t k0 = kbeg; k0 < kend; k0 += 128) {
        const uint64_t kb = k0 + 64 * h;  // this lane's 64 weights
        const uint4 c0 = codes16(L, j, kb / 2, fast);
        const uint4 c1 = codes16(L, j, kb / 2 + 16, fast);
        const uint32_t cw[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            uint32_t e0, o0, e1, o1;
            decode8(cw[2 * t], q0, q1, q2, q3, m4, id, e0, o0);
            decode8(cw[2 * t + 1], q0, q1, q2, q3, m4, id, e1, o1);
            // Quarters are whole 128-weight steps, so only the last step of
            // the row can run past k: there the codes read as zero bytes
            // (book[0]) and act8 gives zero activations, so those products
            // vanish.
            const uint64_t ka = kb + 16 * t;
            uint32_t ae0, ao0, ae1, ao1;
            act8(L, r0 + jl, ka, fast, ae0, ao0);
            act8(L, r0 + jl, ka + 8, fast, ae1, ao1);
            const v4i bop = v4i{(int)e0, (int)o0, (int)e1, (int)o1};
            const v4i aop = v4i{(int)ae0, (int)ao0, (int)ae1, (int)ao1};
            acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop, bop, acc, 0, 0, 0);
        }
        since_fold += 128;
        if (since_fold >= 65536) {
#pragma unroll
            for (int r = 0; r < 16; ++r) wide[r] += acc[r];
            acc = v16i{};
            since_fold = 0;
        }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        wide[r] += acc[r];
        red[wave][(8 * (r >> 2) + 4 * h + (r & 3)) * 33 + jl] = wide[r];
    }
    __syncthreads();
    // 1024 cells, 256 threads: four each.
    for (int q = threadIdx.x; q < 1024; q += 256) {
        const int row = q >> 5, col = q & 31;
        const long long s = red[0][row * 33 + col] + red[1][row * 33 + col] +
                            red[2][row * 33 + col] + red[3][row * 33 + col];
        if (r0 + row < L.m && j0 + col < L.n) lut_finish_any(L, r0 + row, j0 + col, (int64_t)s);
    }
}

// ------------------------------- 4 < m <= 64: 16-column MFMA tiles, k/4
//
// A workgroup of four waves owns 16 coded rows (output columns) j0..j0+15;
// wave w sums the w-th quarter of the 128-weight steps.  Per step, lane
// (c = l%16, g = l/16) loads the 16 code bytes of column j0+c covering weights
// [32g, 32g+32) of the step (one 16-byte load; a column's 64 bytes per step
// are contiguous), decodes them and interleaves the even/odd halves back into
// natural k order, giving two v_mfma_i32_16x16x64_i8 A operands (weights
// 32g..+16 and 32g+16..+32).  The B operands are the activations of rows
// 16b + c at the same k, two 16-byte loads per row block, used as they lie in
// memory.  Lane l of a 16x16 result holds row 4(l/16)+i (an output column) and
// column l%16 (an activation row).  The four quarters meet in LDS as exact
// i64 sums (each quarter's i32 partial is below 2^30: at most 65536 weights).
template <int MB>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(7, 8)))
lut4_mfma16_kernel(LutArgs L, int book_aligned, uint64_t qsteps) {
    __shared__ v4i red[3][MB][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane & 15, g = lane >> 4;
    const uint64_t j0 = (uint64_t)blockIdx.x * 16;
    const uint64_t j = j0 + c;
    const uint64_t jl = j < L.n ? j : L.n - 1;  // columns past n load a valid row, discarded
    const uint64_t nsteps = L.k / 128;
    const uint64_t s0 = (uint64_t)wave * qsteps;
    const uint64_t s1 = min(nsteps, s0 + qsteps);
    const uint32_t m4 = __builtin_amdgcn_readfirstlane(L.sel_mask), id = __builtin_amdgcn_readfirstlane(L.sel_base);

    uint32_t q0, q1, q2, q3;
    load_book(L, jl, book_aligned, q0, q1, q2, q3);
    const uint8_t *cp = L.codes + jl * L.half + 16 * g;
    // Rows past m read row 0 (their products land in result columns that are
    // never stored), so every load is unconditional and the activation loads
    // of a step are all in flight before its decode.
    const int8_t *ap[MB];
#pragma unroll
    for (int b = 0; b < MB; ++b) {
        const uint64_t r = 16 * b + c;
        ap[b] = L.a + (int64_t)(r < L.m ? r : 0) * L.ars + 32 * g;
    }
    v4i acc[MB];
#pragma unroll
    for (int b = 0; b < MB; ++b) acc[b] = v4i{};

    auto step = [&](uint64_t st, const uint4 &cw) {
        v4i x0[MB], x1[MB];
#pragma unroll
        for (int b = 0; b < MB; ++b) {
            const int8_t *p = ap[b] + st * 128;
            x0[b] = *(const v4i *)p;
            x1[b] = *(const v4i *)(p + 16);
        }
        uint32_t e[4], o[4];
        decode8(cw.x, q0, q1, q2, q3, m4, id, e[0], o[0]);
        decode8(cw.y, q0, q1, q2, q3, m4, id, e[1], o[1]);
        decode8(cw.z, q0, q1, q2, q3, m4, id, e[2], o[2]);
        decode8(cw.w, q0, q1, q2, q3, m4, id, e[3], o[3]);
        // Natural order: [w0 w1 w2 w3] = e0 o0 e1 o1 bytes 0,0,1,1 ...
        const v4i w01 = v4i{(int)perm(o[0], e[0], 0x05010400u), (int)perm(o[0], e[0], 0x07030602u),
                            (int)perm(o[1], e[1], 0x05010400u), (int)perm(o[1], e[1], 0x07030602u)};
        const v4i w23 = v4i{(int)perm(o[2], e[2], 0x05010400u), (int)perm(o[2], e[2], 0x07030602u),
                            (int)perm(o[3], e[3], 0x05010400u), (int)perm(o[3], e[3], 0x07030602u)};
#pragma unroll
        for (int b = 0; b < MB; ++b) {
            acc[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(w01, x0[b], acc[b], 0, 0, 0);
            acc[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(w23, x1[b], acc[b], 0, 0, 0);
        }
    };
    // U steps of codes in flight per wave (fewer with more row blocks, so the
    // kernel stays within the 72 registers of seven waves per SIMD).
    constexpr int U = MB == 1 ? 4 : 2;
    uint64_t st = s0;
    for (; st + U <= s1; st += U) {
        uint4 cw[U];
#pragma unroll
        for (int u = 0; u < U; ++u) cw[u] = *(const uint4 *)(cp + (st + u) * 64);
#pragma unroll
        for (int u = 0; u < U; ++u) step(st + u, cw[u]);
    }
    for (; st < s1; ++st) step(st, *(const uint4 *)(cp + st * 64));

    if (wave > 0) {
#pragma unroll
        for (int b = 0; b < MB; ++b) red[wave - 1][b][lane] = acc[b];
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int b = 0; b < MB; ++b) {
        const uint64_t r = 16 * b + c;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint64_t col = j0 + 4 * g + i;
            const int64_t sum = (int64_t)acc[b][i] + red[0][b][lane][i] + red[1][b][lane][i] + red[2][b][lane][i];
            if (r < L.m && col < L.n) lut_finish_any(L, r, col, sum);
        }
    }
}

// ------------------------ 2 <= m <= 32, one workgroup per CU, activations in LDS
//
// The workgroup owns T consecutive 16-column tiles (T = tiles per CU), one
// wave per tile over the whole depth (more tiles than waves: rounds of W), so
// no partial sums cross waves.  Per 128-weight step, lane (c = l%16, g = l/16)
// loads the 16 code bytes of column j0+c covering weights [32g, 32g+32) of
// the step (a column's 64 bytes per step are contiguous) and decodes them, in
// natural weight order, into two v_mfma_i32_16x16x64_i8 A operands.  The
// activations are what the waves share: they pass through LDS in chunks of
// KC weights (16*MB rows x KC bytes, double-buffered), each 1 KiB piece (one
// row's 1024 consecutive weights) copied from global memory straight into LDS
// by global_load_lds_dwordx4, so each B operand is one ds_read_b128.  Chunk
// c+1's pieces are issued in the first steps of chunk c, one per wave per
// step; each wave waits for its own pieces before the barrier that closes
// the chunk, which otherwise leaves the code loads in flight.  Codes are
// loaded CR = 16 steps ahead through a buffer resource, so the loads past the
// last step read zeros instead of leaving the buffer.
//
// LDS layout of a chunk buffer: row r, 16-byte chunk x at r*KC + 16*(x ^ (r & 15)),
// so the 16 rows a B-operand read touches sit on distinct banks.  A piece
// lands contiguously (lane L at +16L), so lane L fetches the chunk whose
// place that is: x = 64p + (L ^ (r & 15)).

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// Lane L's 16 bytes at g land at LDS byte lds + 16*L.  M0 is reserved by the
// compiler, which warns on the clobber; the kernel that calls this makes no
// other use of M0.
__device__ inline void lut_dma16(const int8_t *g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                 :
                 : "s"(lds), "v"(g)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

// s_waitcnt vmcnt(min(n, 15)), expcnt and lgkmcnt unconstrained (n is
// wave-uniform; the immediate needs a branch per value).
__device__ inline void lut_wait_vm(int n) {
#define UOR_VM(N) case N: __builtin_amdgcn_s_waitcnt((N) | (0x7 << 4) | (0xF << 8)); break;
    switch (n < 15 ? (n < 0 ? 0 : n) : 15) {
        UOR_VM(0) UOR_VM(1) UOR_VM(2) UOR_VM(3) UOR_VM(4) UOR_VM(5) UOR_VM(6) UOR_VM(7)
        UOR_VM(8) UOR_VM(9) UOR_VM(10) UOR_VM(11) UOR_VM(12) UOR_VM(13) UOR_VM(14)
        default: __builtin_amdgcn_s_waitcnt(15 | (0x7 << 4) | (0xF << 8)); break;
    }
#undef UOR_VM
}

// decode8 in natural order: lo = [w0 w1 w2 w3], hi = [w4 w5 w6 w7].
__device__ inline void decode8n(uint32_t w, uint32_t q0, uint32_t q1, uint32_t q2, uint32_t q3,
                                uint32_t m4, uint32_t id, uint32_t &lo, uint32_t &hi) {
    uint32_t e, o;
    decode8(w, q0, q1, q2, q3, m4, id, e, o);
    lo = perm(o, e, 0x05010400u);
    hi = perm(o, e, 0x07030602u);
}

template <int MB>
__global__ void __launch_bounds__(512) lut4_lds_kernel(LutArgs L, int book_aligned, uint32_t tpw) {
    constexpr int CR = 16;         // code ring (steps ahead)
    constexpr int ROWS = 16 * MB;
    constexpr int KC = 4096 / MB;  // weights per chunk
    constexpr int S = KC / 128;    // steps per chunk
    constexpr int PPR = KC / 1024; // pieces per row per chunk
    constexpr int CB = ROWS * KC;  // bytes per chunk buffer (64 KiB)
    static_assert(S % CR == 0 && PPR >= 1, "chunk shape");
    __shared__ __attribute__((aligned(16))) int8_t abuf[2 * CB];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int W = blockDim.x >> 6;
    const int c = lane & 15, g = lane >> 4;
    const uint64_t nsteps = L.k / 128, nchunks = (L.k + KC - 1) / KC;
    const uint64_t ntiles = (L.n + 15) / 16;
    const uint64_t t0 = (uint64_t)blockIdx.x * tpw, t1 = min(t0 + tpw, ntiles);
    const int P = (int)L.m * PPR;  // pieces per chunk
    const uint32_t m4 = __builtin_amdgcn_readfirstlane(L.sel_mask), id = __builtin_amdgcn_readfirstlane(L.sel_base);
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) int8_t *)abuf;
    typedef __attribute__((address_space(3))) const v4i lds_v4i_c;

    // Piece q of chunk ch into chunk buffer buf (all wave-uniform but the
    // lane's source): row q / PPR, weights ch*KC + (q % PPR)*1024 ...; false
    // (and nothing issued) past the chunk's last piece or past k.
    auto piece_dma = [&](uint64_t ch, int q, int buf) -> bool {
        const int row = q / PPR, part = q % PPR;
        const uint64_t kb = ch * KC + (uint64_t)part * 1024;
        if (q >= P || kb >= L.k) return false;
        const int8_t *src = L.a + (int64_t)row * L.ars + (int64_t)kb + 16 * (lane ^ (row & 15));
        lut_dma16(src, lds0 + (uint32_t)(buf * CB + row * KC + part * 1024));
        return true;
    };
    // B-operand read offsets: weights 128*sl + 32g + [0,16) are chunk
    // x = 8sl + 2g, at 256*(sl >> 1) + 16*((8*(sl & 1) + 2g) ^ c) in the row
    // (c = row & 15); the next 16 weights are chunk x + 1.
    uint32_t boff[2][2];
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int h = 0; h < 2; ++h) boff[p][h] = lds0 + (uint32_t)(c * KC) + 16u * (uint32_t)((8 * p + 2 * g + h) ^ c);
    // Codes through a buffer resource (the host checks that they lie below 2^31 bytes).
    const __amdgpu_buffer_rsrc_t crs =
        __builtin_amdgcn_make_buffer_rsrc((void *)L.codes, 0, (int)min(L.n * L.half, (uint64_t)0x7FFFFFFF), 0x00020000);

    const int rounds = (int)((tpw + W - 1) / W);
    for (int rd = 0; rd < rounds; ++rd) {
        const uint64_t tile = t0 + (uint64_t)rd * W + wave;
        const bool active = tile < t1;
        const uint64_t j0 = (active ? tile : t0) * 16;
        const uint64_t j = j0 + c;
        const uint64_t jl = j < L.n ? j : L.n - 1;
        uint32_t q0, q1, q2, q3;
        load_book(L, jl, book_aligned, q0, q1, q2, q3);
        const uint32_t cvo = (uint32_t)(jl * L.half) + 16u * g;  // this lane's code offset at step 0

        // Chunk 0's pieces, then the first CR steps of codes; waiting until
        // at most CR loads are left retires every piece (loads retire in
        // order).
        for (int q = wave; q < P; q += W) piece_dma(0, q, 0);
        v4i ring[CR];
#pragma unroll
        for (int u = 0; u < CR; ++u) ring[u] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(crs, cvo, u * 64, 0));
        lut_wait_vm(CR);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");

        v4i acc[MB];
#pragma unroll
        for (int b = 0; b < MB; ++b) acc[b] = v4i{};
        for (uint64_t ch = 0; ch < nchunks; ++ch) {
            const int cur = (int)(ch & 1), nxt = cur ^ 1;
            const bool more = ch + 1 < nchunks;
            const uint64_t sbeg = ch * S, send = min(nsteps, sbeg + S);
            int last = -1;  // the step of this wave's last piece copy in the chunk
            for (uint64_t s8 = sbeg; s8 < send; s8 += CR) {
                const uint32_t cb_off = (uint32_t)(cur * CB) + 128u * (uint32_t)(s8 - sbeg);
#pragma unroll
                for (int u = 0; u < CR; ++u) {
                    const uint64_t st = s8 + u;
                    const int sl = (int)(s8 - sbeg) + u;
                    // One of the next chunk's pieces (wave-uniform branch).
                    if (more && sl * W + wave < P && piece_dma(ch + 1, sl * W + wave, nxt)) last = sl;
                    // Codes of step st.
                    const v4i cw = ring[u];
                    // B operands from LDS.
                    v4i x0[MB], x1[MB];
#pragma unroll
                    for (int b = 0; b < MB; ++b) {
                        const uint32_t ro = cb_off + 256u * (uint32_t)(u >> 1) + (uint32_t)(16 * b * KC);
                        x0[b] = *(lds_v4i_c *)(uintptr_t)(boff[u & 1][0] + ro);
                        x1[b] = *(lds_v4i_c *)(uintptr_t)(boff[u & 1][1] + ro);
                    }
                    uint32_t lo[4], hi[4];
#pragma unroll
                    for (int d = 0; d < 4; ++d) decode8n((uint32_t)cw[d], q0, q1, q2, q3, m4, id, lo[d], hi[d]);
                    const v4i w01 = v4i{(int)lo[0], (int)hi[0], (int)lo[1], (int)hi[1]};
                    const v4i w23 = v4i{(int)lo[2], (int)hi[2], (int)lo[3], (int)hi[3]};
                    // The load of step st + CR goes into the ring slot just
                    // read, after the decode: issued earlier, it would need a
                    // second register set and copies (each waiting for its
                    // load) on the loop's back edge.
                    __builtin_amdgcn_sched_barrier(0);
                    ring[u] = __builtin_bit_cast(
                        v4i, __builtin_amdgcn_raw_buffer_load_b128(crs, cvo, (int)((st + CR) * 64), 0));
#pragma unroll
                    for (int b = 0; b < MB; ++b) {
                        acc[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(w01, x0[b], acc[b], 0, 0, 0);
                        acc[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(w23, x1[b], acc[b], 0, 0, 0);
                    }
                }
            }
            // Close the chunk: this wave's piece copies have landed once at
            // most the code loads issued after the last of them are left
            // (one per step from that step on); then the barrier (every
            // wave's reads of this chunk done, the next one written).
            if (last >= 0) lut_wait_vm((int)(send - sbeg) - last);
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
        }
        if (active) {
            // Lane (c, g) holds row 16b + c, columns j0 + 4g .. + 3.  i32 output
            // with a unit column stride and 16-byte aligned rows leaves in one
            // 16-byte store per lane (and, with beta != 0, one 16-byte load).
            const bool vec = L.ob == 4 && L.ccs == 1 && ((uintptr_t)L.c & 15) == 0 && (L.crs & 3) == 0;
#pragma unroll
            for (int b = 0; b < MB; ++b) {
                const uint64_t r = 16 * b + c, col0 = j0 + 4 * g;
                if (r >= L.m) continue;
                if (vec && col0 + 4 <= L.n) {
                    int32_t *cp = (int32_t *)L.c + (int64_t)r * L.crs + (int64_t)col0;
                    v4i out = acc[b];
                    if (L.alpha != 1 || L.beta != 0) {
                        const v4i prior = L.beta != 0 ? *(const v4i *)cp : v4i{};
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            i128 t = sat_mul((i128)acc[b][i], L.alpha);
                            if (L.beta != 0) t = (i128)((u128)t + (u128)sat_mul((i128)prior[i], L.beta));
                            out[i] = (int)encode_int(t, 4, L.mode);
                        }
                    }
                    *(v4i *)cp = out;
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (col0 + i < L.n) lut_finish_any(L, r, col0 + i, (int64_t)acc[b][i]);
                }
            }
        }
    }
}

// ------------------------- 1 <= m <= 32: 16-column tiles through LDS, MFMA
//
// The decode shapes read every code byte once and little else, so this
// kernel is built around the code stream.  HBM served it best (measured over
// load patterns, in-flight depths and wave counts on MI355X) when each CU
// reads one contiguous 16-column tile (64 KiB at k = 8192) at a time with
// nothing else in flight: one workgroup of 16 waves per CU owns the tiles
// t = b, b + G, b + 2G, ... (G workgroups: the chip reads a window of G
// consecutive tiles); wave w loads column w of the next tile -- k/2
// consecutive bytes, 1 KiB per load (16 bytes per lane, non-temporal: the
// codes are read once) -- after computing the current one, and stores it
// into the other of two LDS tile buffers; one barrier per tile.
//
// Compute: wave w takes weights [w*k/16, (w+1)*k/16) of every column of the
// tile.  Lane (c = l%16, g = l/16) reads column c's 16 code bytes for
// weights [32*(4*KQ*w + 4p + g), +32) per pair p (ds_read_b128), giving two
// v_mfma_i32_16x16x64_i8 A operands (weights +0..16 and +16..32).  The wave's
// activations for its weight range sit in registers for the whole kernel,
// already in the decode's order ([a0 a2 a4 a6 | a1 a3 a5 a7 | a8 .. a14 |
// a9 .. a15] per 16-byte operand), so a code dword costs the 13 VALU ops of
// decode8 and nothing else; rows past m are zero B operands.  The waves' i32
// partials of a tile meet in LDS through ds_add (exact: |sum| <= k * 2^14 <
// 2^31), and the workgroup finishes its (at most NTB) tiles at the end.
//
// LDS: column c's 16-byte chunk x lands at slot x ^ c, so the 16 lanes of a
// ds_read_b128 phase (one chunk index, 16 columns) hit 16 distinct slots.
constexpr int LT_NTB = 12;  // tiles per workgroup at most (their sums stay in LDS)

typedef __attribute__((address_space(1))) const v4i global_v4i_c;
typedef __attribute__((address_space(3))) const v4i lds_v4i_c;
typedef __attribute__((address_space(3))) v4i lds_v4i;

// A 16-byte non-temporal global load (global_load_dwordx4 ... nt: the
// address space is explicit so the compiler never falls back to a flat load,
// whose lgkmcnt share would make every LDS wait also wait for it).
__device__ inline v4i ld_nt16(const void *p) { return __builtin_nontemporal_load((global_v4i_c *)p); }
__device__ inline v4i lds_rd16(uint32_t a) { return *(lds_v4i_c *)(uintptr_t)a; }
// ds_read_b128 the compiler neither moves nor waits for (the caller waits with
// s_waitcnt lgkmcnt and then takes the registers over).
__device__ inline v4i lds_rd16_asm(uint32_t a) {
    v4i r;
    asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(a));
    return r;
}
__device__ inline void lds_wr16(uint32_t a, v4i v) { *(lds_v4i *)(uintptr_t)a = v; }
// LDS writes done, then the workgroup barrier (no wait on the loads in
// flight, which a memory fence would add).
__device__ inline void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Finish the batch of tiles [t0, t0 + cnt) of workgroup b (tiles b + G*i,
// TW columns each) from the tile sums in LDS: 4 consecutive columns per item.
template <int ROWS, int TSW, int TW = 16>
__device__ __attribute__((noinline)) void lut_tile_finish(char *cbase, int64_t crs, int64_t ccs, int ob, int64_t alpha,
                                                          int64_t beta, int mode, uint64_t m, uint64_t n,
                                                          const int *tsum, uint32_t b, uint32_t G, uint32_t t0,
                                                          uint32_t cnt) {
    LutArgs L{};
    L.c = cbase;
    L.crs = crs;
    L.ccs = ccs;
    L.ob = ob;
    L.alpha = alpha;
    L.beta = beta;
    L.mode = mode;
    const bool vec = ob == 4 && ccs == 1 && ((uintptr_t)cbase & 15) == 0 && (crs & 3) == 0 && alpha == 1 && beta == 0;
    constexpr uint32_t Q = TW / 4;
    for (uint32_t e = threadIdx.x; e < cnt * ROWS * Q; e += blockDim.x) {
        const uint32_t sl = e / (ROWS * Q), row = (e / Q) % ROWS, c4 = e % Q;
        if (row >= m) continue;
        const uint64_t col0 = (uint64_t)(b + G * (t0 + sl)) * TW + 4 * c4;
        const int *ts = &tsum[(sl * ROWS + row) * TSW + 4 * c4];
        if (vec && col0 + 4 <= n) {
            *(v4i *)((int32_t *)cbase + (int64_t)row * crs + (int64_t)col0) = v4i{ts[0], ts[1], ts[2], ts[3]};
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (col0 + i < n) lut_finish_any(L, row, col0 + i, (int64_t)ts[i]);
        }
    }
}

template <int MB, int KQ, int W>
__global__ void __launch_bounds__(64 * W) lut4_tile_kernel(LutArgs L, uint32_t ntiles) {
    constexpr int ROWS = 16 * MB;
    constexpr int TSW = 17;              // words per tile-sum row (16 columns + pad)
    constexpr int CB = KQ * 1024;        // code bytes per column (k / 2)
    constexpr int TB = 16 * CB;          // code bytes per tile
    constexpr int NT = W * 64;           // threads
    constexpr int CPW = 16 / W;          // columns each wave loads per tile
    constexpr int PW = CPW * KQ;         // 1 KiB pieces each wave loads per tile
    constexpr int NP = 16 * KQ / W;      // 128-weight pairs each wave computes per column
    __shared__ __attribute__((aligned(16))) uint8_t tbuf[2 * TB];
    __shared__ int tsum[LT_NTB * ROWS * TSW];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = lane & 15, g = lane >> 4;
    const uint32_t G = gridDim.x, b = blockIdx.x;
    const uint32_t ntl = b < ntiles ? (ntiles - 1 - b) / G + 1 : 0;  // this workgroup's tiles
    if (ntl == 0) return;
    const uint32_t m4 = __builtin_amdgcn_readfirstlane(L.sel_mask), id = __builtin_amdgcn_readfirstlane(L.sel_base);
    const uint64_t n = L.n, m = L.m, half = L.half;
    const uint32_t n32 = (uint32_t)n, gm = __builtin_amdgcn_readfirstlane(L.gm),
                   gs1 = __builtin_amdgcn_readfirstlane(L.gs1), gs2 = __builtin_amdgcn_readfirstlane(L.gs2);
    const uint8_t *const codes = L.codes;
    const int8_t *const books = L.books;
    const uint32_t tb0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)tbuf;

    // Column c's codebook of tile i (16 bytes; a ragged tile's missing
    // columns read the last column's).
#define UOR_LT_BOOK(I)                                                                         \
    ([&]() -> v4i {                                                                            \
        const uint32_t j_ = min((b + G * (I)) * 16u + (uint32_t)c, n32 - 1);                   \
        return *(global_v4i_c *)(books + (uint64_t)lut_group_of(j_, gm, gs1, gs2) * 16);        \
    }())
    // This wave's piece e of tile i: column CPW*w + e / KQ, bytes
    // [1024 * (e % KQ), +1024), lane l's 16 bytes at +16l (the wave's pieces
    // are consecutive bytes).  A ragged last tile re-reads a valid row
    // (never stored).
#define UOR_LT_PIECE(I, E)                                                                     \
    ([&]() -> const uint8_t * {                                                               \
        uint64_t j_ = (uint64_t)(b + G * (I)) * 16 + CPW * wave + (E) / KQ;                    \
        if (j_ >= n) j_ = n - 1;                                                               \
        return codes + j_ * half + 1024 * ((E) % KQ) + 16 * lane;                              \
    }())
    // Lane l stores chunk 64q + l of column cc at slot (64q + l) ^ cc.
#define UOR_LT_STORE(BUF, E, V)                                                                \
    {                                                                                          \
        const uint32_t cc_ = (uint32_t)(CPW * wave + (E) / KQ);                                \
        lds_wr16((BUF) + cc_ * CB + 16u * ((64u * ((E) % KQ) + lane) ^ cc_), (V));             \
    }

    // Activations in the decode's order: act[p][h][b] covers row 16b + c,
    // weights w*k/W + 128p + 32g + 16h + [0, 16).  Rows past m read row m-1
    // and are zeroed.
    v4i act[NP][2][MB];
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int bb = 0; bb < MB; ++bb) {
                const uint64_t r = 16 * bb + c < m ? 16 * bb + c : m - 1;
                const uint64_t kk = (uint64_t)(128 * NP) * wave + 128 * p + 32 * g + 16 * h;
                act[p][h][bb] = *(global_v4i_c *)(L.a + (int64_t)r * L.ars + (int64_t)kk);
            }
    v4i bk = UOR_LT_BOOK(0u);
    // Tiles 0 and 1 are requested together, after the activations and the
    // first codebook (the loads complete in order, so whatever waits for
    // those does not wait for the codes): tile 1 is in flight while tile 0
    // is stored.  A workgroup with one tile reads tile 0 twice, the second
    // time from the cache.
    v4i ring[PW], ring1[PW];
#pragma unroll
    for (int e = 0; e < PW; ++e) ring[e] = ld_nt16(UOR_LT_PIECE(0u, e));
#pragma unroll
    for (int e = 0; e < PW; ++e) ring1[e] = ld_nt16(UOR_LT_PIECE(ntl > 1 ? 1u : 0u, e));
    for (int e = threadIdx.x; e < LT_NTB * ROWS * TSW; e += NT) tsum[e] = 0;
    // Activations into the decode's order (rows past m zero).
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int bb = 0; bb < MB; ++bb) {
                v4i x = act[p][h][bb];
                if ((uint64_t)(16 * bb + c) >= m) x = v4i{0, 0, 0, 0};
                act[p][h][bb] = v4i{(int)perm(x[1], x[0], 0x06040200u), (int)perm(x[1], x[0], 0x07050301u),
                                    (int)perm(x[3], x[2], 0x06040200u), (int)perm(x[3], x[2], 0x07050301u)};
            }
    // Tile 0 into its buffer; tile 1 stays in flight.
#pragma unroll
    for (int e = 0; e < PW; ++e) {
        UOR_LT_STORE(tb0, e, ring[e])
        ring[e] = ring1[e];
    }
    lds_barrier();

    // Iteration i computes tile i, then stores tile i+1 (its pieces arrived
    // in `ring` meanwhile) into the other buffer and requests tile i+2.
    // NEXT: tile i+1 exists; AFTER: tile i+2 does (the loads per iteration
    // are then the same everywhere, and the compiler's waits stay exact).
#define UOR_LT_ITER(I, NEXT, AFTER)                                                            \
    {                                                                                          \
        const uint32_t i_ = (I);                                                               \
        const uint32_t cur = tb0 + (i_ & 1) * TB, nxt = tb0 + ((i_ + 1) & 1) * TB;             \
        const uint32_t q0 = (uint32_t)bk[0], q1 = (uint32_t)bk[1], q2 = (uint32_t)bk[2],       \
                       q3 = (uint32_t)bk[3];                                                   \
        if (NEXT) bk = UOR_LT_BOOK(i_ + 1);                                                    \
        /* All of the wave's code chunks first (their LDS latencies overlap), */             \
        /* then decode and MFMA into two accumulator chains per row block. */                   \
        /* (as asm: the scheduler would otherwise sink each read next to its */               \
        /* use and wait for it there) */                                                       \
        /* (with two row blocks the registers are short: there the compiler */                \
        /* places the reads) */                                                                \
        v4i cw[NP];                                                                            \
        _Pragma("unroll") for (int p = 0; p < NP; ++p) {                                       \
            const uint32_t x = (uint32_t)(4 * NP * wave + 4 * p + g);                          \
            const uint32_t a_ = cur + (uint32_t)c * CB + 16u * (x ^ (uint32_t)c);               \
            cw[p] = MB == 1 ? lds_rd16_asm(a_) : lds_rd16(a_);                                 \
        }                                                                                      \
        if (MB == 1) {                                                                         \
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");                                \
            _Pragma("unroll") for (int p = 0; p < NP; ++p) asm volatile("" : "+v"(cw[p]));      \
        }                                                                                      \
        constexpr int CH = MB == 1 ? 2 : 1; /* independent MFMA chains per row block */      \
        v4i acc[CH][MB];                                                                       \
        _Pragma("unroll") for (int ch = 0; ch < CH; ++ch)                                      \
            _Pragma("unroll") for (int bb = 0; bb < MB; ++bb) acc[ch][bb] = v4i{0, 0, 0, 0};   \
        _Pragma("unroll") for (int p = 0; p < NP; ++p) {                                       \
            _Pragma("unroll") for (int h = 0; h < 2; ++h) {                                    \
                uint32_t e0, o0, e1, o1;                                                       \
                decode8((uint32_t)cw[p][2 * h], q0, q1, q2, q3, m4, id, e0, o0);               \
                decode8((uint32_t)cw[p][2 * h + 1], q0, q1, q2, q3, m4, id, e1, o1);           \
                const v4i wop = v4i{(int)e0, (int)o0, (int)e1, (int)o1};                       \
                _Pragma("unroll") for (int bb = 0; bb < MB; ++bb) acc[h % CH][bb] =            \
                    __builtin_amdgcn_mfma_i32_16x16x64_i8(wop, act[p][h][bb], acc[h % CH][bb], 0, 0, 0); \
            }                                                                                  \
        }                                                                                      \
        _Pragma("unroll") for (int bb = 0; bb < MB; ++bb)                                      \
            _Pragma("unroll") for (int v = 0; v < 4; ++v)                                      \
                atomicAdd(&tsum[(i_ * ROWS + 16 * bb + c) * TSW + 4 * g + v],                  \
                          acc[0][bb][v] + (CH > 1 ? acc[CH - 1][bb][v] : 0));                  \
        if (NEXT) {                                                                            \
            _Pragma("unroll") for (int e = 0; e < PW; ++e) {                                   \
                UOR_LT_STORE(nxt, e, ring[e])                                                  \
                if (AFTER) ring[e] = ld_nt16(UOR_LT_PIECE(i_ + 2, e));                         \
            }                                                                                  \
        }                                                                                      \
        lds_barrier();                                                                         \
    }
    uint32_t i = 0;
    for (; i + 2 < ntl; ++i) UOR_LT_ITER(i, true, true)
    if (i + 1 < ntl) {
        UOR_LT_ITER(i, true, false)
        ++i;
    }
    UOR_LT_ITER(i, false, false)
    lut_tile_finish<ROWS, TSW>(L.c, L.crs, L.ccs, L.ob, L.alpha, L.beta, L.mode, m, n, tsum, b, G, 0, ntl);
#undef UOR_LT_ITER
#undef UOR_LT_STORE
#undef UOR_LT_PIECE
#undef UOR_LT_BOOK
}

// ------------------------------ m = 1 (up to 8): 8-column tiles, two per CU
//
// The same code stream at half the tile: one workgroup of 8 waves owns the
// 8-column tiles t = b, b + G, ... (32 KiB at k = 8192; G = two workgroups
// per CU), wave w loads column w of the next tile, one tile in flight, one
// barrier per tile.  Two workgroups per CU, each on its own barrier, kept
// the code stream at 6.4 TB/s where one 16-column workgroup per CU ran at
// 6.0 (the same loads with no compute, MI355X), and a workgroup's last tile
// is half the decode.
//
// The MFMA still takes 16 rows: with at most 8 activation rows, rows 0-7 of
// the A operand carry the tile's 8 columns over the first half of a wave's
// weights and rows 8-15 the same columns over the second half; the B
// operand's columns 0-7 and 8-15 carry the activation rows over the same two
// halves.  The two diagonal 8x8 blocks of the result are then the two
// halves' sums (the off-diagonal blocks pair different weights and are
// dropped), and both are added into the tile sums.
//
// Lane (c = l%16, g = l/16) works on virtual column c: tile column c%8, half
// r = c/8.  Wave w' takes weights [w'*k/8, (w'+1)*k/8) of every column, half
// r the r-th half of that; per pair p of its half it reads 16 code bytes
// (weights 32g..+32 of the pair) and makes two A operands, as the 16-column
// kernel does.  LDS: virtual column c holds its CB/2 bytes in chunk order,
// chunk x of it at slot x ^ c, so a read phase (16 lanes, one chunk index)
// hits 16 distinct slots; a wave's 1 KiB piece scatters over the two halves
// it spans.
template <int KQ>
__global__ void __launch_bounds__(512) lut4_tile8_kernel(LutArgs L, uint32_t ntiles) {
    constexpr int TSW = 9;           // words per tile-sum row (8 columns + pad)
    constexpr int CB = KQ * 1024;    // code bytes per column (k / 2)
    constexpr int VB = CB / 2;       // bytes per virtual column
    constexpr int TB = 8 * CB;       // code bytes per tile
    constexpr int HC = 4 * KQ;       // chunks per half of a wave's range
    constexpr int NP = KQ;           // pairs per half
    __shared__ __attribute__((aligned(16))) uint8_t tbuf[2 * TB];
    __shared__ int tsum[LT_NTB * 8 * TSW];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = lane & 15, g = lane >> 4;
    const int cc = c & 7, r = c >> 3;
    const uint32_t G = gridDim.x, b = blockIdx.x;
    const uint32_t ntl = b < ntiles ? (ntiles - 1 - b) / G + 1 : 0;
    if (ntl == 0) return;
    const uint32_t m4 = __builtin_amdgcn_readfirstlane(L.sel_mask), id = __builtin_amdgcn_readfirstlane(L.sel_base);
    const uint64_t n = L.n, m = L.m, half = L.half;
    const uint32_t n32 = (uint32_t)n, gm = __builtin_amdgcn_readfirstlane(L.gm),
                   gs1 = __builtin_amdgcn_readfirstlane(L.gs1), gs2 = __builtin_amdgcn_readfirstlane(L.gs2);
    const uint8_t *const codes = L.codes;
    const int8_t *const books = L.books;
    const uint32_t tb0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)tbuf;

    // Activations: act[p][h] covers row cc, weights
    // 128 * (2KQ*w + KQ*r + p) + 32g + 16h + [0, 16).  Rows past m read row
    // m-1 and are zeroed.
    v4i act[NP][2];
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint64_t row = (uint64_t)cc < m ? (uint64_t)cc : m - 1;
            const uint64_t kk = (uint64_t)128 * (2 * KQ * wave + KQ * r + p) + 32 * g + 16 * h;
            act[p][h] = *(global_v4i_c *)(L.a + (int64_t)row * L.ars + (int64_t)kk);
        }
#define UOR_LT8_BOOK(I)                                                                        \
    ([&]() -> v4i {                                                                            \
        const uint32_t j_ = min((b + G * (I)) * 8u + (uint32_t)cc, n32 - 1);                   \
        return *(global_v4i_c *)(books + (uint64_t)lut_group_of(j_, gm, gs1, gs2) * 16);        \
    }())
    // Wave w's piece e of tile i: column w, bytes [1024e, +1024), lane l's
    // 16 bytes at +16l.  A ragged last tile re-reads a valid row (never stored).
#define UOR_LT8_PIECE(I, E)                                                                    \
    ([&]() -> const uint8_t * {                                                               \
        uint64_t j_ = (uint64_t)(b + G * (I)) * 8 + wave;                                      \
        if (j_ >= n) j_ = n - 1;                                                               \
        return codes + j_ * half + 1024 * (E) + 16 * lane;                                     \
    }())
    // Chunk x = 64e + l of column w: wave range x / (2HC), half (x / HC) & 1,
    // place x % HC within it; virtual column w + 8 * half, chunk
    // HC * range + place, at slot chunk ^ virtual column.
#define UOR_LT8_STORE(BUF, E, V)                                                               \
    {                                                                                          \
        const uint32_t x_ = 64u * (E) + (uint32_t)lane;                                        \
        const uint32_t vc_ = (uint32_t)wave + 8u * ((x_ / HC) & 1u);                           \
        const uint32_t vx_ = HC * (x_ / (2 * HC)) + x_ % HC;                                   \
        lds_wr16((BUF) + vc_ * VB + 16u * (vx_ ^ vc_), (V));                                   \
    }

    v4i bk = UOR_LT8_BOOK(0u);
    v4i ring[KQ], ring1[KQ];
#pragma unroll
    for (int e = 0; e < KQ; ++e) ring[e] = ld_nt16(UOR_LT8_PIECE(0u, e));
#pragma unroll
    for (int e = 0; e < KQ; ++e) ring1[e] = ld_nt16(UOR_LT8_PIECE(ntl > 1 ? 1u : 0u, e));
    for (int e = threadIdx.x; e < LT_NTB * 8 * TSW; e += 512) tsum[e] = 0;
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            v4i x = act[p][h];
            if ((uint64_t)cc >= m) x = v4i{0, 0, 0, 0};
            act[p][h] = v4i{(int)perm(x[1], x[0], 0x06040200u), (int)perm(x[1], x[0], 0x07050301u),
                            (int)perm(x[3], x[2], 0x06040200u), (int)perm(x[3], x[2], 0x07050301u)};
        }
#pragma unroll
    for (int e = 0; e < KQ; ++e) {
        UOR_LT8_STORE(tb0, e, ring[e])
        ring[e] = ring1[e];
    }
    lds_barrier();

    // Lane l's share of a result: column 4(q&1) + i of the tile and activation
    // row l%8 for q = l/16, valid on the diagonal blocks (q/2 == (l%16)/8).
    const bool diag = (g >> 1) == r;
#define UOR_LT8_ITER(I, NEXT, AFTER)                                                           \
    {                                                                                          \
        const uint32_t i_ = (I);                                                               \
        const uint32_t cur = tb0 + (i_ & 1) * TB, nxt = tb0 + ((i_ + 1) & 1) * TB;             \
        const uint32_t q0 = (uint32_t)bk[0], q1 = (uint32_t)bk[1], q2 = (uint32_t)bk[2],       \
                       q3 = (uint32_t)bk[3];                                                   \
        if (NEXT) bk = UOR_LT8_BOOK(i_ + 1);                                                   \
        v4i cw[NP];                                                                            \
        _Pragma("unroll") for (int p = 0; p < NP; ++p) {                                       \
            const uint32_t x = (uint32_t)(HC * wave + 4 * p + g);                              \
            cw[p] = lds_rd16_asm(cur + (uint32_t)c * VB + 16u * (x ^ (uint32_t)c));             \
        }                                                                                      \
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");                                    \
        _Pragma("unroll") for (int p = 0; p < NP; ++p) asm volatile("" : "+v"(cw[p]));          \
        v4i acc[2] = {v4i{0, 0, 0, 0}, v4i{0, 0, 0, 0}};                                       \
        _Pragma("unroll") for (int p = 0; p < NP; ++p) {                                       \
            _Pragma("unroll") for (int h = 0; h < 2; ++h) {                                    \
                uint32_t e0, o0, e1, o1;                                                       \
                decode8((uint32_t)cw[p][2 * h], q0, q1, q2, q3, m4, id, e0, o0);               \
                decode8((uint32_t)cw[p][2 * h + 1], q0, q1, q2, q3, m4, id, e1, o1);           \
                const v4i wop = v4i{(int)e0, (int)o0, (int)e1, (int)o1};                       \
                acc[h] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wop, act[p][h], acc[h], 0, 0, 0); \
            }                                                                                  \
        }                                                                                      \
        if (diag && (uint64_t)cc < m) {                                                        \
            _Pragma("unroll") for (int v = 0; v < 4; ++v)                                      \
                atomicAdd(&tsum[(i_ * 8 + cc) * TSW + 4 * (g & 1) + v], acc[0][v] + acc[1][v]); \
        }                                                                                      \
        if (NEXT) {                                                                            \
            _Pragma("unroll") for (int e = 0; e < KQ; ++e) {                                   \
                UOR_LT8_STORE(nxt, e, ring[e])                                                 \
                if (AFTER) ring[e] = ld_nt16(UOR_LT8_PIECE(i_ + 2, e));                        \
            }                                                                                  \
        }                                                                                      \
        lds_barrier();                                                                         \
    }
    uint32_t i = 0;
    for (; i + 2 < ntl; ++i) UOR_LT8_ITER(i, true, true)
    if (i + 1 < ntl) {
        UOR_LT8_ITER(i, true, false)
        ++i;
    }
    UOR_LT8_ITER(i, false, false)
    lut_tile_finish<8, TSW, 8>(L.c, L.crs, L.ccs, L.ob, L.alpha, L.beta, L.mode, m, n, tsum, b, G, 0, ntl);
#undef UOR_LT8_ITER
#undef UOR_LT8_STORE
#undef UOR_LT8_PIECE
#undef UOR_LT8_BOOK
}

// ------------------------------------------- many rows: decode, then dense
//
// For m >= LUT_PREFILL_M (or m >= 80 at k >= 4096, where the dense route
// takes its 256-wide tile: m = 80..112 at the config weights 0.18 ms against
// 0.20-0.26 ms for the table-lookup kernel) the weights are decoded once into
// W^T (k x n int8,
// row-major, leading dimension ldw, a multiple of 16) and the product runs on
// the dense int8 MFMA route: the reference's decode-then-multiply spelling of
// the same value (coded_gemm, crates/uor-matmul-gemm/src/coded.rs:98-140;
// `decline`, tabulated.rs:2555-2745; CD-13).  A workgroup decodes a tile of
// 128 columns x 128 weights into LDS ([k][column]: thread t owns column t %
// 128 and 64 of the weights), then writes the tile's 128 rows of W^T as
// 128-byte row segments (8 lanes x 16 bytes per row).
constexpr uint64_t LUT_PREFILL_M = 128;

static bool lut_prefill(uint64_t m, uint64_t k) { return m >= LUT_PREFILL_M || (m >= 80 && k >= 4096); }

__global__ void __launch_bounds__(256) lut4_decode_t_kernel(LutArgs L, int book_aligned, int code_fast,
                                                            int8_t *wt, uint64_t ldw) {
    __shared__ __attribute__((aligned(16))) int8_t tile[128][128];
    const int t = threadIdx.x;
    const uint64_t j0 = (uint64_t)blockIdx.x * 128, k0 = (uint64_t)blockIdx.y * 128;
    {
        const int cl = t & 127, kh = t >> 7;  // column in the tile, half of the tile's depth
        const uint64_t j = j0 + cl;
        if (j < L.n) {
            uint32_t q0, q1, q2, q3;
            load_book(L, j, book_aligned, q0, q1, q2, q3);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int kt = 64 * kh + 32 * h;  // first weight of this chunk in the tile
                const uint4 cw = codes16(L, j, (k0 + kt) / 2, code_fast != 0);
                const uint32_t w[4] = {cw.x, cw.y, cw.z, cw.w};
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    uint32_t e, o;
                    decode8(w[d], q0, q1, q2, q3, L.sel_mask, L.sel_base, e, o);
#pragma unroll
                    for (int b = 0; b < 4; ++b) {
                        tile[kt + 8 * d + 2 * b][cl] = (int8_t)(e >> (8 * b));
                        tile[kt + 8 * d + 2 * b + 1][cl] = (int8_t)(o >> (8 * b));
                    }
                }
            }
        }
    }
    __syncthreads();
    const int ch = t & 7;  // 16-byte chunk of a 128-byte row segment
#pragma unroll
    for (int pass = 0; pass < 4; ++pass) {
        const int r = pass * 32 + (t >> 3);
        const uint64_t kk = k0 + r, jc = j0 + 16 * ch;
        if (kk < L.k && jc < ldw) *(uint4 *)(wt + kk * ldw + jc) = *(const uint4 *)&tile[r][16 * ch];
    }
}

}  // namespace uor

using namespace uor;

extern "C" int uor_gfx950_gemm_lut4(const uor_view *a, const uint8_t *codes, uint64_t codes_len,
                                    uint64_t n, const int8_t *books, uint64_t books_len,
                                    uint64_t group, const uor_view *c, int out_type, int64_t alpha,
                                    int64_t beta, int encode, void *scratch, uint64_t scratch_bytes,
                                    void *stream, uor_route *route) {
    route_set(route, UOR_ROUTE_NONE);
    if (!valid_out_type(out_type) || !valid_encode(encode)) return UOR_INVALID_ARGUMENT;
    if (!a || !c) return UOR_INVALID_ARGUMENT;
    Placed A, C;
    int st;
    if ((st = place(a, 1, &A))) return st;
    const uint64_t m = A.rows, k = A.cols;
    // CodedMatrix::new (matrix.rs:36-75): a fixed-width tier of MAX_BLOCK 2
    // needs an even row width and exactly n * k/2 codes.
    if (k % 2 != 0) return UOR_SHORT_BUFFER;
    uint64_t need;
    if (__builtin_mul_overflow(n, k / 2, &need) || need != codes_len) return UOR_SHORT_BUFFER;
    if (group == 0) return UOR_INVALID_ARGUMENT;
    const uint64_t ngroups = n == 0 ? 0 : (n + group - 1) / group;
    if (books_len < ngroups * 16) return UOR_SHORT_BUFFER;
    if (n > 0 && need > 0 && !codes) return UOR_SHORT_BUFFER;
    if (ngroups > 0 && !books) return UOR_SHORT_BUFFER;
    if ((st = place(c, out_type, &C))) return st;
    // TabulatedTriple::new (tabulated.rs:628-658).
    if (C.rows != m || C.cols != n) return UOR_NONCONFORMANT;
    if (self_aliases(C.rows, C.cols, C.rs, C.cs)) return UOR_OUTPUT_ALIASES_ITSELF;
    if (m == 0 || n == 0) return UOR_OK;

    LutArgs L{(const int8_t *)A.base, A.rs, A.cs, codes, k / 2, books, group, m, k, n,
              C.base, C.rs, C.cs, out_type, alpha, beta, encode, 0x04040404u, 0x03020100u, 0, 0, 0};
    lut_group_magic(L, group);
    hipStream_t s = (hipStream_t)stream;
    // 16-byte code loads need 16-byte aligned rows; 8-byte activation loads
    // need a unit column stride and 8-byte aligned rows.
    const bool code_fast = ((uintptr_t)codes % 16 == 0) && ((k / 2) % 16 == 0);
    const bool act_fast = A.cs == 1 && ((uintptr_t)A.base % 8 == 0) && (A.rs % 8 == 0 || m == 1);
    const int fast = code_fast && act_fast;
    const int book_aligned = (uintptr_t)books % 4 == 0;
    if (route) {
        route->kind = UOR_ROUTE_LUT4_DOT4;
        route->launches = 1;
        route->operand_modes = fast;
    }
    const bool a16 = A.cs == 1 && ((uintptr_t)A.base % 16 == 0) && (A.rs % 16 == 0 || m == 1);
    // lut_prefill(m, k) with an offer that holds W^T: decode, then the dense
    // int8 route (whatever is left of the offer goes to it).
    const uint64_t ldw = (n + 15) / 16 * 16;
    if (lut_prefill(m, k) && scratch && k > 0 && k <= (1ull << 40) / ldw) {
        const uintptr_t p0 = (uintptr_t)scratch, p1 = (p0 + 255) & ~(uintptr_t)255;
        const uint64_t have = scratch_bytes > (p1 - p0) ? scratch_bytes - (p1 - p0) : 0;
        const uint64_t wbytes = (k * ldw + 255) & ~255ull;
        if (wbytes <= have && (n + 127) / 128 <= 0x7fffffffull && (k + 127) / 128 <= 65535) {
            int8_t *wt = (int8_t *)p1;
            const dim3 grid((unsigned)((n + 127) / 128), (unsigned)((k + 127) / 128));
            hipLaunchKernelGGL(lut4_decode_t_kernel, grid, dim3(256), 0, s, L, book_aligned, (int)code_fast, wt,
                               ldw);
            UOR_HIP(hipGetLastError());
            const uor_view bv{wt, k * ldw, k, n, (int64_t)ldw, 1};
            const int st2 = uor_gfx950_gemm_i8(a, &bv, c, out_type, alpha, beta, encode, wt + wbytes,
                                               have - wbytes, stream, route);
            if (route && st2 == UOR_OK) {
                route->kind = UOR_ROUTE_LUT4_PREFILL;
                route->launches += 1;
                route->scratch_used += wbytes;
            }
            return st2;
        }
    }
    // 1 <= m <= 32, k a multiple of 2048 up to 8192 (a wave's activations
    // fit its registers), at most LT_NTB tiles per CU (their sums fit LDS),
    // 16-byte aligned code and activation rows and codebooks: the 16-column
    // tiles through LDS, one workgroup per CU.
    if (m <= 32 && k % 2048 == 0 && k >= 2048 && k <= 8192 && code_fast && a16 &&
        ((uintptr_t)books & 15) == 0 && lut_tile_on()) {
        const uint64_t ntiles = (n + 15) / 16;
        const uint64_t cus = (uint64_t)device_cus_lut();
        // m = 1: the 8-column tiles, two workgroups per CU (measured at the
        // config weights: m = 1 22.0-22.4 against 22.3-22.8 us for the
        // 16-column tiles; from m = 2 on even, and 0.5-1.7 us slower at m = 8).
        const uint64_t nt8 = (n + 7) / 8;
        if (m == 1 && lut_tile8_on() && (nt8 + 2 * cus - 1) / (2 * cus) <= (uint64_t)LT_NTB) {
            const unsigned G = (unsigned)std::min<uint64_t>(2 * cus, nt8);
            if (route) route->tile_m = 8, route->tile_n = 8, route->tile_k = (int)(k / 16), route->split_k = 16,
                       route->kind = UOR_ROUTE_LUT4_MFMA;
#define UOR_LT8(KQ) hipLaunchKernelGGL((lut4_tile8_kernel<KQ>), dim3(G), dim3(512), 0, s, L, (uint32_t)nt8);
            switch (k / 2048) {
            case 1: UOR_LT8(1); break;
            case 2: UOR_LT8(2); break;
            case 3: UOR_LT8(3); break;
            default: UOR_LT8(4); break;
            }
#undef UOR_LT8
            UOR_HIP(hipGetLastError());
            return UOR_OK;
        }
        if ((ntiles + cus - 1) / cus <= (uint64_t)LT_NTB) {
            const unsigned G = (unsigned)std::min<uint64_t>(cus, ntiles);
            const int w = lut_tile_waves();
            if (route) route->tile_m = m <= 16 ? 16 : 32, route->tile_n = 16, route->tile_k = (int)(k / w),
                       route->split_k = w, route->kind = UOR_ROUTE_LUT4_MFMA;
#define UOR_LT(MB, KQ)                                                                                       \
    if (w == 16) hipLaunchKernelGGL((lut4_tile_kernel<MB, KQ, 16>), dim3(G), dim3(1024), 0, s, L, (uint32_t)ntiles); \
    else hipLaunchKernelGGL((lut4_tile_kernel<MB, KQ, 8>), dim3(G), dim3(512), 0, s, L, (uint32_t)ntiles);
            const int kq = (int)(k / 2048);
            if (m <= 16) {
                switch (kq) {
                case 1: UOR_LT(1, 1); break;
                case 2: UOR_LT(1, 2); break;
                case 3: UOR_LT(1, 3); break;
                default: UOR_LT(1, 4); break;
                }
            } else {
                switch (kq) {
                case 1: UOR_LT(2, 1); break;
                case 2: UOR_LT(2, 2); break;
                case 3: UOR_LT(2, 3); break;
                default: UOR_LT(2, 4); break;
                }
            }
#undef UOR_LT
            UOR_HIP(hipGetLastError());
            return UOR_OK;
        }
    }
    // 2 <= m <= 32, whole 2048-weight blocks, k <= 65536 (each wave's i32 sum
    // over the whole depth is exact), 16-byte aligned code rows (all below
    // 2^31 bytes) and activation rows: one workgroup per CU with the
    // activations in LDS.  Its waves must cover a chunk's m*KC/1024 pieces at
    // one per wave per step: W >= m/8.  (At k = 8192, n = 28672 it takes
    // 29.8 us for every m from 1 to 8; the dot4 kernel below takes 25.4 us at
    // m = 1 and 30.2, 37.7, 39.1 us at m = 2, 3, 4.)
    if (m >= 2 && m <= 32 && k % 2048 == 0 && k <= 65536 && code_fast && a16 && n * (k / 2) < (1ull << 31) &&
        lut_variant() == 1) {
        const uint64_t ntiles = (n + 15) / 16;
        const uint64_t cus = (uint64_t)device_cus_lut();
        const uint64_t tpw = (ntiles + cus - 1) / cus;
        uint64_t w = tpw < 8 ? tpw : 8;
        const uint64_t wmin = (m + 7) / 8;
        if (w < wmin) w = wmin;
        const uint64_t blocks = (ntiles + tpw - 1) / tpw;
        if (blocks <= 0x7FFFFFFFull && tpw <= 0xFFFFFFFFull) {
            const int mb = (int)((m + 15) / 16);
            if (route) route->tile_m = 16 * mb, route->tile_n = 16, route->split_k = 1, route->kind = UOR_ROUTE_LUT4_MFMA;
            const dim3 grid((unsigned)blocks), block((unsigned)(64 * w));
            if (mb == 1) hipLaunchKernelGGL((lut4_lds_kernel<1>), grid, block, 0, s, L, book_aligned, (uint32_t)tpw);
            else hipLaunchKernelGGL((lut4_lds_kernel<2>), grid, block, 0, s, L, book_aligned, (uint32_t)tpw);
            UOR_HIP(hipGetLastError());
            return UOR_OK;
        }
    }
    if (m <= 4 && k <= 65536) {
        // 4096 persistent waves (four per SIMD), each walking columns j,
        // j + W, ...: a sweep of 2048..14336 on MI355X put the optimum here.
        const uint64_t waves = n < 4096 ? n : 4096;
        const unsigned blocks = (unsigned)((waves + 3) / 4);
        if (route) route->tile_m = m <= 1 ? 1 : m <= 2 ? 2 : 4, route->tile_n = 1;
        const bool pf = lut_variant() == 1 && k <= (uint64_t)LUT_SEG;
        if (pf) {
            // One resident round of the pipelined kernel (its register use
            // sets how many blocks a CU holds), capped by the columns.
            auto kern = fast ? (m <= 1 ? lut4_dot4_pf_kernel<1, true> : m <= 2 ? lut4_dot4_pf_kernel<2, true>
                                                                                  : lut4_dot4_pf_kernel<4, true>)
                             : (m <= 1 ? lut4_dot4_pf_kernel<1, false> : m <= 2 ? lut4_dot4_pf_kernel<2, false>
                                                                                   : lut4_dot4_pf_kernel<4, false>);
            static unsigned cap[2][3] = {{0, 0, 0}, {0, 0, 0}};
            unsigned &cp = cap[fast ? 1 : 0][m <= 1 ? 0 : m <= 2 ? 1 : 2];
            if (!cp) cp = resident_blocks(kern);
            const unsigned pblocks = (unsigned)std::min<uint64_t>(cp, (n + 3) / 4);
            hipLaunchKernelGGL(kern, dim3(pblocks), dim3(256), 0, s, L, book_aligned);
        } else if (fast) {
            if (m <= 1) hipLaunchKernelGGL((lut4_dot4_kernel<1, true>), dim3(blocks), dim3(256), 0, s, L, book_aligned);
            else if (m <= 2) hipLaunchKernelGGL((lut4_dot4_kernel<2, true>), dim3(blocks), dim3(256), 0, s, L, book_aligned);
            else hipLaunchKernelGGL((lut4_dot4_kernel<4, true>), dim3(blocks), dim3(256), 0, s, L, book_aligned);
        } else {
            if (m <= 1) hipLaunchKernelGGL((lut4_dot4_kernel<1, false>), dim3(blocks), dim3(256), 0, s, L, book_aligned);
            else if (m <= 2) hipLaunchKernelGGL((lut4_dot4_kernel<2, false>), dim3(blocks), dim3(256), 0, s, L, book_aligned);
            else hipLaunchKernelGGL((lut4_dot4_kernel<4, false>), dim3(blocks), dim3(256), 0, s, L, book_aligned);
        }
        UOR_HIP(hipGetLastError());
        return UOR_OK;
    }
    // 4 < m <= 64 with whole 128-weight steps, 16-byte aligned code rows and
    // 16-byte activation rows: the 16-column tiles.  A quarter holds at most
    // 512 steps (65536 weights), so its i32 partial is exact.
    if (m <= 64 && k % 128 == 0 && k <= 4 * 65536 && code_fast && a16) {
        const uint64_t nsteps = k / 128, qsteps = (nsteps + 3) / 4;
        const uint64_t tiles = (n + 15) / 16;
        if (tiles > 0x7FFFFFFFull) return UOR_INVALID_ARGUMENT;
        const int mb = (int)((m + 15) / 16);
        if (route) route->tile_m = 16 * mb, route->tile_n = 16, route->split_k = 4, route->kind = UOR_ROUTE_LUT4_MFMA;
        switch (mb) {
        case 1: hipLaunchKernelGGL((lut4_mfma16_kernel<1>), dim3((unsigned)tiles), dim3(256), 0, s, L, book_aligned, qsteps); break;
        case 2: hipLaunchKernelGGL((lut4_mfma16_kernel<2>), dim3((unsigned)tiles), dim3(256), 0, s, L, book_aligned, qsteps); break;
        case 3: hipLaunchKernelGGL((lut4_mfma16_kernel<3>), dim3((unsigned)tiles), dim3(256), 0, s, L, book_aligned, qsteps); break;
        default: hipLaunchKernelGGL((lut4_mfma16_kernel<4>), dim3((unsigned)tiles), dim3(256), 0, s, L, book_aligned, qsteps); break;
        }
        UOR_HIP(hipGetLastError());
        return UOR_OK;
    }
    // Quarter of k per wave, in whole 128-weight steps.
    uint64_t kq = (k + 3) / 4;
    kq = (kq + 127) / 128 * 128;
    if (kq == 0) kq = 128;
    const uint64_t tiles = ((n + 31) / 32) * ((m + 31) / 32);
    if (route) route->tile_m = 32, route->tile_n = 32, route->split_k = 4, route->kind = UOR_ROUTE_LUT4_MFMA;
    if (tiles > 0x7FFFFFFFull) return UOR_INVALID_ARGUMENT;
    hipLaunchKernelGGL(lut4_mfma_kernel, dim3((unsigned)tiles), dim3(256), 0, s, L, fast, book_aligned, kq);
    UOR_HIP(hipGetLastError());
    return UOR_OK;
}

extern "C" uint64_t uor_gfx950_suggested_scratch_lut4(uint64_t m, uint64_t k, uint64_t n) {
    // W^T for the decode-then-dense route (lut_prefill(m, k)), plus the
    // dense route's own offer; none below (the LUT kernels use no scratch).
    if (!lut_prefill(m, k) || k == 0 || n == 0) return 0;
    const uint64_t ldw = (n + 15) / 16 * 16;
    return 256 + ((k * ldw + 255) & ~255ull) + uor_gfx950_suggested_scratch_i8(m, k, n);
}
