// The direct-to-LDS int8 MFMA pipeline shared by the integer GEMM and the
// residue GEMMs of the exact float route: operand descriptors, the XCD-aware
// tile order, the LDS stage layout, and the four-stage k loop.
#pragma once

#include <stdlib.h>
#include <string.h>

#include "common.hpp"

namespace uor {

// Which 256x256 pipeline runs (UOR_GFX950_DL_VARIANT at load time): 4 waves
// (one per SIMD) with the explicitly interleaved schedule (s4, the default),
// 8 waves (two per SIMD) with the first half of each step's fragments
// prefetched one step ahead (w8pf), the same without the prefetch (w8), or 4
// waves in compiler order (w4).  All give the same bytes.
enum : int { DL_W8 = 0, DL_W4 = 1, DL_W8PF = 2, DL_S4 = 3 };
static inline int dl_variant() {
    static int v = [] {
        const char *e = getenv("UOR_GFX950_DL_VARIANT");
        if (e && !strcmp(e, "w8")) return (int)DL_W8;
        if (e && !strcmp(e, "w4")) return (int)DL_W4;
        if (e && !strcmp(e, "w8pf")) return (int)DL_W8PF;
        return (int)DL_S4;
    }();
    return v;
}

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// A placed operand seen from the reduction: element (mn, p) is at
// base + mn*s_mn + p*s_k.
struct Opnd {
    const int8_t *base;
    int64_t s_mn, s_k;
    uint64_t mn;  // extent along m (A) or n (B)
};

// Tile index -> (tile row, tile column).  Workgroups are dealt round-robin to
// the 8 XCDs, so consecutive ids are remapped onto one XCD first, then walked
// in groups of 8 tile rows so that the tiles one XCD holds at a time share
// A rows and B columns in its L2.  (A persistent grid whose size is a
// multiple of 8 keeps tile id b on XCD b % 8 as well.)
__device__ inline void tile_coords(int id, int gm, int gn, int *tm, int *tn) {
    int nb = gm * gn;
    int b = id;
    if ((nb & 7) == 0) b = (b & 7) * (nb >> 3) + (b >> 3);
    const int G = 8;
    int per = G * gn;
    int g = b / per;
    int first = g * G;
    int gs = min(gm - first, G);
    int w = b - g * per;
    *tm = first + w % gs;
    *tn = w / gs;
}
__device__ inline void tile_of(int gm, int gn, int *tm, int *tn) { tile_coords(blockIdx.x, gm, gn, tm, tn); }

// ------------------------------------------------- direct-to-LDS pipeline --
//
// The row-major x row-major case (A's reduction axis contiguous, B's n axis
// contiguous) with k a multiple of 64 and n of 16 streams both operands
// straight from global memory into LDS (global_load_lds_dwordx4: lane L of an
// instruction lands at base + 16*L), NSTAGE stages deep, so each wave keeps
// three k-steps of loads in flight while its MFMAs run.  B stays row-major
// ([k][n]) in LDS and reaches the MFMA through ds_read_b64_tr_b8, which
// transposes 8x8 bytes across each 16-lane group: output lane t, byte b is
// byte t%8 of the row addressed by lane 2b + t/8.
//
// LDS swizzles (16-byte granularity) keep every read pass on distinct banks:
//   A stage: row r, k-chunk c at r*64 + 16*(c ^ ((r >> 2) & 3))
//   B stage: k-row k, n-chunk x at k*BN + 16*(x ^ (2*(k & 7) & (BN/16 - 1)))

typedef int v2i __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) v2i lds_v2i;
typedef __attribute__((address_space(3))) void lds_void;

#ifndef UOR_DL_ASM
#define UOR_DL_ASM 1
#endif

constexpr int DL_BK = 64;
constexpr int DL_NSTAGE = 4;

// Steps come in units of DL_UNIT consecutive 64-deep steps (256 bytes of each
// A row); unit u of a k walk starts kstep bytes after unit u - 1, so kstep =
// DL_UNIT * DL_BK is the plain contiguous walk.
constexpr int DL_UNIT = 4;
__device__ inline uint64_t dl_koff(int t, uint64_t kstep) {
    return (uint64_t)(t / DL_UNIT) * kstep + (uint64_t)(t % DL_UNIT) * DL_BK;
}

// One LDS array per workgroup: the A halves of all stages first, then the B
// halves, so that a stage handle (its A half) reaches its B half at a fixed
// offset and every fragment read is a lane base plus an immediate offset
// (DS offsets are 16 bits: the four 16 KiB A halves fit below 64 KiB).
template <int BM, int BN, int NS = DL_NSTAGE>
struct DlLayout {
    static_assert(BM == BN, "the B halves sit one A region above their A halves");
    static constexpr int A_BYTES = BM * DL_BK;
    static constexpr int B_BYTES = BN * DL_BK;
    static constexpr int STAGE = A_BYTES + B_BYTES;
    static constexpr int BYTES = NS * STAGE;
    static constexpr int B_OFF = NS * A_BYTES;  // stage handle -> its B half
    __device__ static inline int a_off(int r, int c) { return r * 64 + 16 * (c ^ ((r >> 2) & 3)); }
    __device__ static inline int b_swz(int k) { return (2 * (k & 7)) & (BN / 16 - 1); }
    __device__ static inline int b_off(int k, int x) { return k * BN + 16 * (x ^ b_swz(k)); }
};

template <int N>
__device__ inline void wait_vm() {
    // s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt split in [3:0] and [15:14]),
    // leaving expcnt and lgkmcnt unconstrained.
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// A workgroup barrier without the release fence __syncthreads() carries: the
// fence would wait for every LDS-DMA load in flight (all stages), while each
// thread has already waited (vmcnt) for the one stage the next step reads.
// The empty asm statements keep the compiler from moving LDS accesses across.
__device__ inline void stage_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// One 16-byte-per-lane global -> LDS load: lane L's 16 bytes land at
// lds + 16*L.  Issued through inline assembly so the compiler's wait
// insertion, which cannot tell the four stages apart across the loop's back
// edge, does not drain every stage before a read; the explicit vmcnt waits in
// the k loop order each stage instead.
// M0 is reserved by the compiler, which warns on the clobber; the kernels that
// call this make no other use of M0 (checked in their ISA).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ inline void lds_dma16(const int8_t *g, char *lds) {
#if UOR_DL_ASM
    const uint32_t l = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char *)lds;
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                 :
                 : "s"(__builtin_amdgcn_readfirstlane(l)), "v"(g)
                 : "memory", "m0");
#else
    __builtin_amdgcn_global_load_lds((const void *)g, (lds_void *)lds, 16, 0, 0);
#endif
}
#pragma clang diagnostic pop

template <int BM, int BN, int NT, int NS = DL_NSTAGE>
__device__ inline void dl_issue(const Opnd &A, const Opnd &B, uint64_t m0, uint64_t n0, uint64_t k0,
                                char *stage) {
    using L = DlLayout<BM, BN, NS>;
    constexpr int PA = BM * 4 / NT, PB = BN * 4 / NT;  // 16-byte chunks per thread
    static_assert(PA >= 1 && PB >= 1, "tile too small for the workgroup");
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // A: BM*4 chunks, slot s = row*4 + physical chunk.
#pragma unroll
    for (int i = 0; i < PA; ++i) {
        const int base = (wave * PA + i) * 64;
        const int slot = base + lane;
        const int row = slot >> 2, pc = slot & 3;
        const int c = pc ^ ((row >> 2) & 3);
        uint64_t gr = m0 + row;
        if (gr >= A.mn) gr = A.mn - 1;  // rows past m are computed and discarded
        lds_dma16(A.base + (int64_t)gr * A.s_mn + (int64_t)(k0 + 16 * c), stage + base * 16);
    }
    // B: BN/16 chunks per k-row, slot s = k*(BN/16) + physical chunk.
    char *bst = stage + L::B_OFF;
#pragma unroll
    for (int i = 0; i < PB; ++i) {
        const int base = (wave * PB + i) * 64;
        const int slot = base + lane;
        const int k = slot / (BN / 16), px = slot % (BN / 16);
        const int x = px ^ L::b_swz(k);
        uint64_t gn = n0 + 16 * x;
        if (gn >= B.mn) gn = 0;  // columns past n are computed and discarded
        lds_dma16(B.base + (int64_t)(k0 + k) * B.s_k + (int64_t)gn, bst + base * 16);
    }
}

// One k-step's fragments of a wave: FM A and FN B operands per 32-deep half.
template <int BM, int BN, int WM, int WN>
struct DlFrag {
    v4i af[2][BM / WM / 32];
    v4i bf[2][BN / WN / 32];
};

// The fragment reads of one k-step of 64 from LDS stage `sa` (A) / `sb` (B).
template <int BM, int BN, int WM, int WN>
__device__ inline void dl_frag_read(const char *sa, const char *sb, DlFrag<BM, BN, WM, WN> &f) {
    constexpr int FM = BM / WM / 32, FN = BN / WN / 32;
    using L = DlLayout<BM, BN>;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int half = lane >> 5, l32 = lane & 31;
    const int grp = lane >> 4, t16 = lane & 15;
#pragma unroll
    for (int ks = 0; ks < DL_BK / 32; ++ks) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
            f.af[ks][i] = *(const v4i *)(sa + L::a_off(wm * (BM / WM) + 32 * i + l32, 2 * ks + half));
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int nb = wn * (BN / WN) + 32 * j + 16 * (grp & 1) + 8 * (t16 & 1);
            const int k = 32 * ks + 16 * (grp >> 1) + (t16 >> 1);
            v2i lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                (lds_v2i *)(sb + L::b_off(k, nb >> 4) + (nb & 8)));
            v2i hi = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                (lds_v2i *)(sb + L::b_off(k + 8, nb >> 4) + (nb & 8)));
            f.bf[ks][j] = v4i{lo[0], lo[1], hi[0], hi[1]};
        }
    }
}

// The MFMAs of one k-step: each of the wave's FM x FN 32x32 blocks, two
// 32-deep MFMAs each.
template <int BM, int BN, int WM, int WN>
__device__ inline void dl_frag_mma(const DlFrag<BM, BN, WM, WN> &f, v16i (&acc)[BM / WM / 32][BN / WN / 32]) {
    constexpr int FM = BM / WM / 32, FN = BN / WN / 32;
#pragma unroll
    for (int ks = 0; ks < DL_BK / 32; ++ks)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.af[ks][i], f.bf[ks][j], acc[i][j], 0, 0, 0);
}

// One k-step of 64 from LDS stage `sa` (A) / `sb` (B): each wave's FM x FN
// 32x32 blocks, two 32-deep MFMAs each.
template <int BM, int BN, int WM, int WN>
__device__ inline void dl_compute(const char *sa, const char *sb,
                                  v16i (&acc)[BM / WM / 32][BN / WN / 32]) {
    DlFrag<BM, BN, WM, WN> f;
    dl_frag_read<BM, BN, WM, WN>(sa, sb, f);
    dl_frag_mma<BM, BN, WM, WN>(f, acc);
}

// The k loop over nk steps of DL_BK, step t at kbeg + dl_koff(t, kstep): each
// wave's FM x FN 32x32 accumulators, stage handles st0..st3 (A halves; B halves
// at B_OFF above).  Ends with every load retired; the caller's barrier then
// frees the stages.
template <int BM, int BN, int WM, int WN>
__device__ inline void dl_mainloop(const Opnd &A, const Opnd &B, uint64_t m0, uint64_t n0,
                                   uint64_t kbeg, int nk, char *st0, char *st1, char *st2,
                                   char *st3, v16i (&acc)[BM / WM / 32][BN / WN / 32],
                                   uint64_t kstep = DL_UNIT * DL_BK) {
    constexpr int NT = 64 * WM * WN;
    using L = DlLayout<BM, BN>;
    constexpr int LOADS = (BM + BN) * 4 / NT;  // global_load_lds per thread per stage
    static_assert(DL_NSTAGE == 4, "the k loop below is unrolled by four stages");
    if (0 < nk) dl_issue<BM, BN, NT>(A, B, m0, n0, kbeg, st0);
    if (1 < nk) dl_issue<BM, BN, NT>(A, B, m0, n0, kbeg + dl_koff(1, kstep), st1);
    if (2 < nk) dl_issue<BM, BN, NT>(A, B, m0, n0, kbeg + dl_koff(2, kstep), st2);

    // Step kt reads stage kt % 4 and refills stage (kt + 3) % 4, last read at
    // step kt - 1, which every wave has finished once it passes the barrier.
#define UOR_DL_STEP(CUR, NXT)                                                                  \
    {                                                                                          \
        const int ahead = min(DL_NSTAGE - 2, nk - 1 - kt);                                     \
        if (ahead >= 2) wait_vm<2 * LOADS>();                                                  \
        else if (ahead == 1) wait_vm<LOADS>();                                                 \
        else wait_vm<0>();                                                                     \
        stage_barrier();                                                                       \
        if (kt + DL_NSTAGE - 1 < nk)                                                           \
            dl_issue<BM, BN, NT>(A, B, m0, n0, kbeg + dl_koff(kt + DL_NSTAGE - 1, kstep), NXT); \
        dl_compute<BM, BN, WM, WN>(CUR, CUR + L::B_OFF, acc);                                \
        if (++kt >= nk) break;                                                                 \
    }
    for (int kt = 0; kt < nk;) {
        UOR_DL_STEP(st0, st3)
        UOR_DL_STEP(st1, st0)
        UOR_DL_STEP(st2, st1)
        UOR_DL_STEP(st3, st2)
    }
#undef UOR_DL_STEP
    wait_vm<0>();
}

// s_waitcnt vmcnt(n) for a wave-uniform n < 64 known only at run time.
__device__ inline void wait_vm_rt(int n) {
#define UOR_VMR(N) case N: wait_vm<N>(); break;
    switch (n) {
        UOR_VMR(0) UOR_VMR(1) UOR_VMR(2) UOR_VMR(3) UOR_VMR(4) UOR_VMR(5) UOR_VMR(6) UOR_VMR(7)
        UOR_VMR(8) UOR_VMR(9) UOR_VMR(10) UOR_VMR(11) UOR_VMR(12) UOR_VMR(13) UOR_VMR(14) UOR_VMR(15)
        UOR_VMR(16) UOR_VMR(17) UOR_VMR(18) UOR_VMR(19) UOR_VMR(20) UOR_VMR(21) UOR_VMR(22) UOR_VMR(23)
        UOR_VMR(24) UOR_VMR(25) UOR_VMR(26) UOR_VMR(27) UOR_VMR(28) UOR_VMR(29) UOR_VMR(30) UOR_VMR(31)
        default: wait_vm<0>(); break;
    }
#undef UOR_VMR
}

// The same k loop on a ring of NS stages: for a tile whose product is too
// small to hide a memory round trip behind three steps of MFMAs, every stage
// a short reduction needs is in flight at once, and a longer one keeps
// NS - 1 stages in flight.
template <int BM, int BN, int WM, int WN, int NS>
__device__ inline void dl_mainloop_ring(const Opnd &A, const Opnd &B, uint64_t m0, uint64_t n0, uint64_t kbeg,
                                        int nk, char *lds, v16i (&acc)[BM / WM / 32][BN / WN / 32],
                                        uint64_t kstep = DL_UNIT * DL_BK) {
    constexpr int NT = 64 * WM * WN;
    using L = DlLayout<BM, BN, NS>;
    constexpr int LOADS = (BM + BN) * 4 / NT;  // global_load_lds per thread per stage
    static_assert((NS - 2) * LOADS < 32, "the run-time wait covers vmcnt below 32");
    if (nk <= NS) {
        // The whole reduction fits the ring: every stage requested at once,
        // one wait and one barrier, then the steps back to back (no barrier
        // between them, so each step's fragment reads overlap the MFMAs
        // before them).
        for (int t = 0; t < nk; ++t)
            dl_issue<BM, BN, NT, NS>(A, B, m0, n0, kbeg + dl_koff(t, kstep), lds + t * L::A_BYTES);
        wait_vm<0>();
        stage_barrier();
        // Step kt + 1's fragments are read before step kt's MFMAs.
        DlFrag<BM, BN, WM, WN> f0, f1;
        dl_frag_read<BM, BN, WM, WN>(lds, lds + L::B_OFF, f0);
        for (int kt = 0; kt < nk; kt += 2) {
            if (kt + 1 < nk) dl_frag_read<BM, BN, WM, WN>(lds + (kt + 1) * L::A_BYTES,
                                                          lds + (kt + 1) * L::A_BYTES + L::B_OFF, f1);
            dl_frag_mma<BM, BN, WM, WN>(f0, acc);
            if (kt + 1 >= nk) break;
            if (kt + 2 < nk) dl_frag_read<BM, BN, WM, WN>(lds + (kt + 2) * L::A_BYTES,
                                                          lds + (kt + 2) * L::A_BYTES + L::B_OFF, f0);
            dl_frag_mma<BM, BN, WM, WN>(f1, acc);
        }
        return;
    }
    // Longer reductions: NS - 1 stages requested; step kt waits for stage kt
    // (the stages after it may stay in flight), passes the barrier, refills
    // slot (kt - 1) % NS, which every wave finished reading before it, with
    // stage kt + NS - 1, and computes.  (Reading step kt + 1's fragments
    // before step kt's MFMAs, which needs stage kt + 1 one step earlier,
    // measured 6-8% slower here.)
    for (int t = 0; t < NS - 1; ++t)
        dl_issue<BM, BN, NT, NS>(A, B, m0, n0, kbeg + dl_koff(t, kstep), lds + t * L::A_BYTES);
    for (int kt = 0; kt < nk; ++kt) {
        wait_vm_rt(min(NS - 2, nk - 1 - kt) * LOADS);
        stage_barrier();
        if (kt + NS - 1 < nk)
            dl_issue<BM, BN, NT, NS>(A, B, m0, n0, kbeg + dl_koff(kt + NS - 1, kstep),
                                     lds + ((kt + NS - 1) % NS) * L::A_BYTES);
        char *cur = lds + (kt % NS) * L::A_BYTES;
        dl_compute<BM, BN, WM, WN>(cur, cur + L::B_OFF, acc);
    }
    wait_vm<0>();
}

// ---------------------------------------------- half-prefetch variant --
//
// The same stages and loads.  Each 64-deep step is two 32-deep halves: the
// first half's fragments (f0) are read during the previous step, so the
// step's MFMAs start as soon as its barrier passes; the second half's (f1)
// are read right after the barrier and arrive while the first half's MFMAs
// run; then the next step's first half is read into f0.  Register use is the
// same as reading both halves in-step.  A stage's last reads happen in its
// own step, so step t's barrier frees stage t-1, which takes step t+3.

template <int BM, int BN, int WM, int WN>
struct DlHalf {
    static constexpr int FM = BM / WM / 32, FN = BN / WN / 32;
    v4i a[FM];
    v4i b[FN];
};

template <int BM, int BN, int WM, int WN>
__device__ inline void dl_read_half(const char *sa, const char *sb, int ks,
                                    DlHalf<BM, BN, WM, WN> &f) {
    constexpr int FM = BM / WM / 32, FN = BN / WN / 32;
    using L = DlLayout<BM, BN>;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int half = lane >> 5, l32 = lane & 31;
    const int grp = lane >> 4, t16 = lane & 15;
#pragma unroll
    for (int i = 0; i < FM; ++i)
        f.a[i] = *(const v4i *)(sa + L::a_off(wm * (BM / WM) + 32 * i + l32, 2 * ks + half));
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const int nb = wn * (BN / WN) + 32 * j + 16 * (grp & 1) + 8 * (t16 & 1);
        const int k = 32 * ks + 16 * (grp >> 1) + (t16 >> 1);
        v2i lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i *)(sb + L::b_off(k, nb >> 4) + (nb & 8)));
        v2i hi = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i *)(sb + L::b_off(k + 8, nb >> 4) + (nb & 8)));
        f.b[j] = v4i{lo[0], lo[1], hi[0], hi[1]};
    }
}

// MFMAs q0 <= q < q1 of one half, q = i * FN + j.
template <int BM, int BN, int WM, int WN, int Q0, int Q1>
__device__ inline void dl_mfma_half(const DlHalf<BM, BN, WM, WN> &f,
                                    v16i (&acc)[BM / WM / 32][BN / WN / 32]) {
    constexpr int FN = BN / WN / 32;
#pragma unroll
    for (int q = Q0; q < Q1; ++q)
        acc[q / FN][q % FN] =
            __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a[q / FN], f.b[q % FN], acc[q / FN][q % FN], 0, 0, 0);
}

template <int BM, int BN, int WM, int WN>
__device__ inline void dl_mainloop_pf(const Opnd &A, const Opnd &B, uint64_t m0, uint64_t n0,
                                      uint64_t kbeg, int nk, char *st0, char *st1, char *st2,
                                      char *st3, v16i (&acc)[BM / WM / 32][BN / WN / 32],
                                      uint64_t kstep = DL_UNIT * DL_BK) {
    constexpr int NT = 64 * WM * WN;
    using L = DlLayout<BM, BN>;
    constexpr int LOADS = (BM + BN) * 4 / NT;  // global_load_lds per thread per stage
    static_assert(DL_NSTAGE == 4, "the k loop below is unrolled by four stages");
    static_assert(DL_BK == 64, "two 32-deep halves per step");
    if (nk <= 0) return;
    DlHalf<BM, BN, WM, WN> f0, f1;
    dl_issue<BM, BN, NT>(A, B, m0, n0, kbeg, st0);
    if (1 < nk) dl_issue<BM, BN, NT>(A, B, m0, n0, kbeg + dl_koff(1, kstep), st1);
    if (2 < nk) dl_issue<BM, BN, NT>(A, B, m0, n0, kbeg + dl_koff(2, kstep), st2);
    {
        const int later = min(2, nk - 1);
        if (later >= 2) wait_vm<2 * LOADS>();
        else if (later == 1) wait_vm<LOADS>();
        else wait_vm<0>();
    }
    stage_barrier();
    dl_read_half<BM, BN, WM, WN>(st0, st0 + L::B_OFF, 0, f0);

    // Step t: CUR = stage t, NXT = stage t+1, FREE = stage t-1 (= t+3).
    // The empty asm statement (a compiler memory barrier) keeps the next f0
    // reads behind the first-half MFMAs.
    constexpr int NQ = DlHalf<BM, BN, WM, WN>::FM * DlHalf<BM, BN, WM, WN>::FN;
#define UOR_DL_PF_STEP(CUR, NXT, FREE)                                                        \
    {                                                                                          \
        if (kt + 1 < nk) {                                                                     \
            if (kt + 2 < nk) wait_vm<LOADS>();                                                 \
            else wait_vm<0>();                                                                 \
        }                                                                                      \
        stage_barrier();                                                                       \
        dl_read_half<BM, BN, WM, WN>(CUR, CUR + L::B_OFF, 1, f1);                               \
        dl_mfma_half<BM, BN, WM, WN, 0, NQ / 2>(f0, acc);                                      \
        if (kt + 3 < nk) dl_issue<BM, BN, NT>(A, B, m0, n0, kbeg + dl_koff(kt + 3, kstep), FREE); \
        dl_mfma_half<BM, BN, WM, WN, NQ / 2, NQ>(f0, acc);                                     \
        asm volatile("" ::: "memory");                                                         \
        if (kt + 1 < nk) dl_read_half<BM, BN, WM, WN>(NXT, NXT + L::B_OFF, 0, f0);              \
        dl_mfma_half<BM, BN, WM, WN, 0, NQ>(f1, acc);                                          \
        if (++kt >= nk) break;                                                                 \
    }
    for (int kt = 0; kt < nk;) {
        UOR_DL_PF_STEP(st0, st1, st3)
        UOR_DL_PF_STEP(st1, st2, st0)
        UOR_DL_PF_STEP(st2, st3, st1)
        UOR_DL_PF_STEP(st3, st0, st2)
    }
#undef UOR_DL_PF_STEP
    wait_vm<0>();
}

// ------------------------------------------ four-wave scheduled pipeline --
//
// The 256x256 tile with four waves (2x2, one per SIMD), each owning a 128x128
// block of the tile (4x4 accumulators of 32x32): per 64-deep step a wave issues
// 32 MFMAs against 8 ds_read_b128 (A) and 16 ds_read_b64_tr_b8 (B), a third
// less LDS traffic per MFMA than the eight-wave 128x64 split.  With one wave
// per SIMD nothing overlaps unless the wave itself interleaves, so every step
// is written out in issue order and fenced (sched_barrier) against the
// scheduler, one memory instruction after each MFMA:
//
//   P1  the 16 MFMAs of k-half 0 (fragments f0, read during the previous
//       step); after MFMA q < 12 the q-th read of k-half 1 (f1), after MFMAs
//       12..15 the four A loads of stage t+3 (into stage t-1's slot).
//   P2  wait until this wave's loads of stage t+1 have landed and its f1 reads
//       have returned, then the workgroup barrier.  After it stage t+1 is
//       complete for every wave, and every read of slot t has retired, so the
//       next step may refill that slot (with stage t+4).
//   P3  the 16 MFMAs of k-half 1, each of the first 12 followed by one read of
//       step t+1's f0, the last four by the four B loads of stage t+3.
//
// A stage's loads are issued about three steps before its first read.  The
// loads use the scalar-base form (global_load_lds_dwordx4 voffset, sbase):
// per-lane 32-bit offsets fixed for the whole k loop and one 64-bit scalar
// base per operand advanced per step, so the host routes here only views
// whose offsets fit in 32 bits.

struct S4 {
    static constexpr int BM = 256, BN = 256, NT = 256;
    using L = DlLayout<256, 256>;
    static constexpr int LOADS = 8;  // LDS-DMA loads per thread per stage (4 A, 4 B)
};

// Per-lane constants of the scheduled loop.
struct S4Lane {
    uint32_t voa[4], vob[4];  // global offsets of this lane's A / B chunks (per tile)
    uint32_t ra[2];           // LDS byte address of A fragment 0, k-halves 0 / 1 (stage 0)
    uint32_t rb[4];           // LDS byte address of B fragment j, k-half 0 (stage 0)
    uint32_t rbt[2];          // BT: LDS byte address of B fragment 0, k-halves 0 / 1
};

// Scalar state: operand bases at the next stage to load and the LDS targets.
struct S4Scalars {
    const int8_t *a;   // A.base + (next k0)
    const int8_t *b;   // B.base + (next k0) * s_k
    int64_t bstep;     // 64 * s_k
    uint32_t mla, mlb; // LDS byte address of this wave's first A / B chunk in stage 0
};

// BT: B arrives k-contiguous (column-major, B.s_k == 1): its stage half takes
// A's layout (row = output column, 64 k-bytes) and its fragments are plain
// 16-byte reads like A's, 8 reads per k-half instead of 12.

// The tile-independent part: fragment read addresses and LDS targets.
template <bool BT = false>
__device__ inline void s4_setup_lane(const Opnd &B, const char *lds, S4Lane &ln, S4Scalars &sc) {
    using L = S4::L;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int half = lane >> 5, l32 = lane & 31, grp = lane >> 4, t16 = lane & 15;
    const uint32_t base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const char *)lds;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        ln.ra[ks] = base + L::a_off(wm * 128 + l32, 2 * ks + half);
        ln.rbt[ks] = base + L::B_OFF + L::a_off(wn * 128 + l32, 2 * ks + half);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int nb = wn * 128 + 32 * j + 16 * (grp & 1) + 8 * (t16 & 1);
        const int k = 16 * (grp >> 1) + (t16 >> 1);
        ln.rb[j] = base + L::B_OFF + L::b_off(k, nb >> 4) + (nb & 8);
    }
    sc.bstep = (int64_t)DL_BK * B.s_k;
    sc.mla = base + wave * 4 * 1024;
    sc.mlb = base + L::B_OFF + wave * 4 * 1024;
}

// The per-tile part: this lane's chunk offsets and the bases at k = kbeg.
template <bool BT = false>
__device__ inline void s4_setup_tile(const Opnd &A, const Opnd &B, uint64_t m0, uint64_t n0, uint64_t kbeg,
                                     S4Lane &ln, S4Scalars &sc) {
    using L = S4::L;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // A chunk: slot (wave*4 + i)*64 + lane = row*4 + physical chunk.
        const int slot = (wave * 4 + i) * 64 + lane;
        const int row = slot >> 2, pc = slot & 3;
        const int c = pc ^ ((row >> 2) & 3);
        uint64_t gr = m0 + row;
        if (gr >= A.mn) gr = A.mn - 1;  // rows past m are computed and discarded
        ln.voa[i] = (uint32_t)(gr * (uint64_t)A.s_mn + 16 * c);
        if constexpr (BT) {
            // B chunk, A's layout: slot = output column*4 + physical chunk.
            uint64_t gc = n0 + row;
            if (gc >= B.mn) gc = B.mn - 1;  // columns past n are computed and discarded
            ln.vob[i] = (uint32_t)(gc * (uint64_t)B.s_mn + 16 * c);
        } else {
            // B chunk: slot = k*16 + physical chunk.
            const int k = slot >> 4, px = slot & 15;
            const int x = px ^ L::b_swz(k);
            uint64_t gn = n0 + 16 * x;
            if (gn >= B.mn) gn = 0;  // columns past n are computed and discarded
            ln.vob[i] = (uint32_t)((uint64_t)k * (uint64_t)B.s_k + gn);
        }
    }
    sc.a = A.base + kbeg;
    sc.b = B.base + (int64_t)kbeg * B.s_k;
}

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// One 16-byte LDS-DMA load: lane L's bytes at sbase + voff land at m0 + 16*L.
__device__ inline void s4_dma(uint32_t m0v, uint32_t voff, const int8_t *sbase) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                 :
                 : "s"(m0v), "v"(voff), "s"(sbase)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

// Load number q (0..7: A chunks 0..3, then B chunks 0..3) of the stage in slot SLOT.
template <int SLOT>
__device__ inline void s4_load(const S4Lane &ln, const S4Scalars &sc, int q) {
    using L = S4::L;
    if (q < 4) s4_dma(sc.mla + SLOT * L::A_BYTES + q * 1024, ln.voa[q], sc.a);
    else s4_dma(sc.mlb + SLOT * L::B_BYTES + (q - 4) * 1024, ln.vob[q - 4], sc.b);
}

// Fragment read number q (0..11) of k-half KS from slot SLOT, in the order
// A0, B0 lo, B0 hi, A1, B1 lo, B1 hi, ...; with BT, q in 0..7: A0, B0, A1, ...
template <int SLOT, int KS, bool BT = false>
__device__ inline void s4_read(const S4Lane &ln, int q, v4i (&fa)[4], v4i (&fb)[4]) {
    using L = S4::L;
    typedef __attribute__((address_space(3))) const v4i lds_v4i_c;
    if constexpr (BT) {
        const int f = q >> 1;
        if ((q & 1) == 0) fa[f] = *(lds_v4i_c *)(uintptr_t)(ln.ra[KS] + SLOT * L::A_BYTES + f * 32 * 64);
        else fb[f] = *(lds_v4i_c *)(uintptr_t)(ln.rbt[KS] + SLOT * L::B_BYTES + f * 32 * 64);
        return;
    }
    const int f = q / 3, part = q % 3;
    if (part == 0) {
        fa[f] = *(lds_v4i_c *)(uintptr_t)(ln.ra[KS] + SLOT * L::A_BYTES + f * 32 * 64);
    } else {
        const v2i h = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
            (lds_v2i *)(uintptr_t)(ln.rb[f] + SLOT * L::B_BYTES + KS * 32 * 256 + (part - 1) * 8 * 256));
        if (part == 1) { fb[f][0] = h[0]; fb[f][1] = h[1]; }
        else { fb[f][2] = h[0]; fb[f][3] = h[1]; }
    }
}

// The MFMA order within a half: fragment pairs in the order their reads
// arrive (A0 B0, A1, B1, A2, B2, A3, B3).
__device__ constexpr int s4_qi(int q) {
    constexpr int I[16] = {0, 1, 0, 1, 2, 2, 0, 1, 2, 3, 3, 3, 0, 1, 2, 3};
    return I[q];
}
__device__ constexpr int s4_qj(int q) {
    constexpr int J[16] = {0, 0, 1, 1, 0, 1, 2, 2, 2, 0, 1, 2, 3, 3, 3, 3};
    return J[q];
}

#define S4_FENCE() __builtin_amdgcn_sched_barrier(0)

// One 64-deep step on slot CUR: the loads of stage t+3 go into slot
// (CUR+3)%4, and P3 reads step t+1's f0 from slot (CUR+1)%4.  Every step has
// the same shape: past the last stage the loads repeat the last stage's k
// (their slot is never read again) and the last step's f0 reads are
// discarded, so the vmcnt and lgkmcnt accounting is the same in every step.
template <int CUR, bool BT = false>
__device__ inline void s4_step(const S4Lane &ln, S4Scalars &sc, bool advance, v4i (&fa0)[4], v4i (&fb0)[4],
                               v4i (&fa1)[4], v4i (&fb1)[4], v16i (&acc)[4][4]) {
    constexpr int NXT = (CUR + 1) & 3, FREE = (CUR + 3) & 3;
    constexpr int NR = BT ? 8 : 12;  // fragment reads per k-half
    // P1
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        acc[s4_qi(q)][s4_qj(q)] =
            __builtin_amdgcn_mfma_i32_32x32x32_i8(fa0[s4_qi(q)], fb0[s4_qj(q)], acc[s4_qi(q)][s4_qj(q)], 0, 0, 0);
        if (q < NR) s4_read<CUR, 1, BT>(ln, q, fa1, fb1);
        else if (q >= 12) s4_load<FREE>(ln, sc, q - 12);
        S4_FENCE();
    }
    // P2: stage t+1 landed (allowed in flight: stage t+2's eight loads and
    // the four A loads of stage t+3 just issued), f1 returned and slot CUR's
    // reads retired; then the barrier.
    wait_vm<S4::LOADS + 4>();
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    stage_barrier();
    S4_FENCE();
    // P3
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        acc[s4_qi(q)][s4_qj(q)] =
            __builtin_amdgcn_mfma_i32_32x32x32_i8(fa1[s4_qi(q)], fb1[s4_qj(q)], acc[s4_qi(q)][s4_qj(q)], 0, 0, 0);
        if (q < NR) s4_read<NXT, 0, BT>(ln, q, fa0, fb0);
        else if (q >= 12) s4_load<FREE>(ln, sc, q - 8);
        S4_FENCE();
    }
    if (advance) {
        sc.a += DL_BK;
        sc.b += sc.bstep;
    }
}

// Stages 0..2 of a tile into slots 0..2 (a stage past the last repeats it).
// The slots must be free: every earlier read retired and a barrier passed.
__device__ inline void s4_prologue(const S4Lane &ln, S4Scalars &sc, int nk) {
#pragma unroll
    for (int q = 0; q < 8; ++q) s4_load<0>(ln, sc, q);
    if (1 < nk) sc.a += DL_BK, sc.b += sc.bstep;
#pragma unroll
    for (int q = 0; q < 8; ++q) s4_load<1>(ln, sc, q);
    if (2 < nk) sc.a += DL_BK, sc.b += sc.bstep;
#pragma unroll
    for (int q = 0; q < 8; ++q) s4_load<2>(ln, sc, q);
    if (3 < nk) sc.a += DL_BK, sc.b += sc.bstep;
}

// The k loop over nk >= 1 steps whose stages 0..2 the prologue issued (any
// vector memory instructions issued after the prologue must have retired, as
// must the prologue's stage 0 by the wait below).  Adds into acc, this
// wave's 128x128 block.  Ends with every load landed and every LDS read of
// this wave retired, but without a barrier.
template <bool BT = false>
__device__ inline void s4_loop(const S4Lane &ln, S4Scalars &sc, int nk, v16i (&acc)[4][4]) {
    v4i fa0[4], fb0[4], fa1[4], fb1[4];
    wait_vm<2 * S4::LOADS>();
    stage_barrier();
    S4_FENCE();
#pragma unroll
    for (int q = 0; q < (BT ? 8 : 12); ++q) s4_read<0, 0, BT>(ln, q, fa0, fb0);
    S4_FENCE();
    // Step t issues stage t+3 and advances the bases while stage t+4 exists.
    int t = 0;
    for (; t + 4 <= nk; t += 4) {
        s4_step<0, BT>(ln, sc, t + 4 < nk, fa0, fb0, fa1, fb1, acc);
        s4_step<1, BT>(ln, sc, t + 5 < nk, fa0, fb0, fa1, fb1, acc);
        s4_step<2, BT>(ln, sc, t + 6 < nk, fa0, fb0, fa1, fb1, acc);
        s4_step<3, BT>(ln, sc, t + 7 < nk, fa0, fb0, fa1, fb1, acc);
    }
    if (t < nk) s4_step<0, BT>(ln, sc, t + 4 < nk, fa0, fb0, fa1, fb1, acc);
    if (t + 1 < nk) s4_step<1, BT>(ln, sc, t + 5 < nk, fa0, fb0, fa1, fb1, acc);
    if (t + 2 < nk) s4_step<2, BT>(ln, sc, t + 6 < nk, fa0, fb0, fa1, fb1, acc);
    wait_vm<0>();
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the discarded f0 reads
}

}  // namespace uor
