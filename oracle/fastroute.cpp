// fastroute.cpp -- TEST/BENCH INFRASTRUCTURE ONLY: the CPU baseline.
//
// A C++ restatement of the reference's fastest CPU route for each hot-path
// configuration, timed beside the GPU by bench.py (cpu_baseline, kind
// "port").  The reference binary is Rust and cannot be built here; this
// follows its files:
//   i8 GEMM  -- the blocked full-depth traversal kernel.rs::run
//               (crates/uor-matmul-gemm/src/kernel.rs:1016-1377) with
//               blocking MC=128, NC=1024 (generated.rs:181-205), B packed in
//               16-column panels grouped by k-quads, A in 8-row panels, and the
//               AVX-512 VNNI dpbusd 8x16 tile with the offset identity
//               sum (a+128)*b - 128*sum b (crates/uor-matmul-kernels/src/isa/
//               x86.rs:704-715, 843-897); the AVX2 6x16 madd tile when VNNI is
//               absent (x86.rs:80-96).  Exact i32 lanes fold to i128, then the
//               Linear epilogue and the saturating i32 encode.
//   LUT      -- tabulation (crates/uor-matmul-gemm/src/tabulated.rs:3867-4555,
//               crates/uor-matmul-kernels/src/table.rs:2050-3227): per row of A
//               and k-pair, a 256-entry table of partial sums indexed by the
//               packed byte, then one gather-add per byte per column.
//   Trop     -- driver::gemm's (max,+) loop (driver.rs:147-181) in the packed
//               saturating-i16 form of TROP_I16 / AVX2_TROP_I16
//               (isa/portable.rs:312-359, isa/x86.rs:935-1055).
// Parallelism is the reference's caller-driven Partition
// (crates/uor-matmul-gemm/src/partition.rs): disjoint output blocks, one
// worker thread each; the library itself spawns nothing.
#include <immintrin.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <thread>
#include <vector>

typedef __int128 i128;

namespace {

constexpr int MC = 128, NC = 1024;
constexpr int VMR = 8, VNR = 16;  // dpbusd tile

inline int32_t enc_i32(i128 v) {
    if (v > INT32_MAX) return INT32_MAX;
    if (v < INT32_MIN) return INT32_MIN;
    return (int32_t)v;
}

inline i128 sat_mul(i128 x, int64_t f) {
    i128 r;
    if (__builtin_mul_overflow(x, (i128)f, &r)) {
        const i128 MX = (i128)(((unsigned __int128)1 << 127) - 1);
        return ((x < 0) != (f < 0)) ? -MX - 1 : MX;
    }
    return r;
}

inline void finish(int32_t *cp, int64_t s, int64_t alpha, int64_t beta) {
    i128 t = sat_mul((i128)s, alpha);
    if (beta != 0) t = (i128)((unsigned __int128)t + (unsigned __int128)sat_mul((i128)*cp, beta));
    *cp = enc_i32(t);
}

// Pack B[k][j0 .. j0+16) into quads: for quad q, 16 columns x 4 k bytes.
void pack_b_panel(const int8_t *b, int64_t ldb, int k, int j0, int n, int8_t *out) {
    int kq = (k + 3) / 4;
    for (int q = 0; q < kq; ++q)
        for (int j = 0; j < VNR; ++j)
            for (int t = 0; t < 4; ++t) {
                int p = 4 * q + t, col = j0 + j;
                out[(q * VNR + j) * 4 + t] = (p < k && col < n) ? b[(int64_t)p * ldb + col] : 0;
            }
}

// Pack A rows [i0, i0+8) into quads: for quad q, 8 rows x 4 k bytes.
void pack_a_panel(const int8_t *a, int64_t lda, int k, int i0, int m, int8_t *out) {
    int kq = (k + 3) / 4;
    for (int q = 0; q < kq; ++q)
        for (int i = 0; i < VMR; ++i)
            for (int t = 0; t < 4; ++t) {
                int p = 4 * q + t, row = i0 + i;
                out[(q * VMR + i) * 4 + t] = (p < k && row < m) ? a[(int64_t)row * lda + p] : 0;
            }
}

__attribute__((target("avx512f,avx512bw,avx512vnni")))
void tile_vnni(int kq, const int8_t *pa, const int8_t *pb, int32_t *acc) {
    __m512i t[VMR];
    for (int i = 0; i < VMR; ++i) t[i] = _mm512_setzero_si512();
    __m512i colsum = _mm512_setzero_si512();
    const __m512i ones = _mm512_set1_epi32(0x01010101);
    for (int q = 0; q < kq; ++q) {
        __m512i bv = _mm512_loadu_si512((const void *)(pb + q * VNR * 4));
        colsum = _mm512_dpbusd_epi32(colsum, ones, bv);
        for (int i = 0; i < VMR; ++i) {
            uint32_t quad;
            memcpy(&quad, pa + (q * VMR + i) * 4, 4);
            __m512i av = _mm512_set1_epi32((int)(quad ^ 0x80808080u));
            t[i] = _mm512_dpbusd_epi32(t[i], av, bv);
        }
    }
    __m512i scaled = _mm512_mullo_epi32(colsum, _mm512_set1_epi32(128));
    for (int i = 0; i < VMR; ++i)
        _mm512_storeu_si512((void *)(acc + i * VNR), _mm512_sub_epi32(t[i], scaled));
}

__attribute__((target("avx2")))
void tile_avx2(int kq, const int8_t *pa, const int8_t *pb, int32_t *acc) {
    // Each quad of 4 columns is sign-extended to i16 [k0 k1 k2 k3] per
    // column; vpmaddwd against the row's broadcast [a0 a1 a2 a3] leaves two
    // exact pair sums per column, added at the end.
    __m256i t[VMR][4];
    for (int i = 0; i < VMR; ++i)
        for (int h = 0; h < 4; ++h) t[i][h] = _mm256_setzero_si256();
    for (int q = 0; q < kq; ++q) {
        __m256i bw[4];
        for (int h = 0; h < 4; ++h)
            bw[h] = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(pb + q * VNR * 4 + 16 * h)));
        for (int i = 0; i < VMR; ++i) {
            const int8_t *aq = pa + (q * VMR + i) * 4;
            uint64_t pat = (uint64_t)(uint16_t)aq[0] | ((uint64_t)(uint16_t)aq[1] << 16) |
                           ((uint64_t)(uint16_t)aq[2] << 32) | ((uint64_t)(uint16_t)aq[3] << 48);
            __m256i av = _mm256_set1_epi64x((long long)pat);
            for (int h = 0; h < 4; ++h) t[i][h] = _mm256_add_epi32(t[i][h], _mm256_madd_epi16(av, bw[h]));
        }
    }
    for (int i = 0; i < VMR; ++i)
        for (int h = 0; h < 4; ++h) {
            alignas(32) int32_t d[8];
            _mm256_store_si256((__m256i *)d, t[i][h]);
            for (int e = 0; e < 4; ++e) acc[i * VNR + 4 * h + e] = d[2 * e] + d[2 * e + 1];
        }
}

bool have_vnni() {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("avx512bw");
}

}  // namespace

extern "C" {

int fr_has_vnni(void) { return have_vnni() ? 1 : 0; }

int fr_hw_threads(void) { return (int)std::max(1u, std::thread::hardware_concurrency()); }

// slice::gemm_ex::<i8, i32> on the reference's packed route, rows
// [row0, row0+rows) only (a deterministic slab; rows are independent).
// k must be <= the dpbusd lane depth (65793 at |a|,|b| <= 128) so the i32
// lanes are exact at full depth, as the reference's suggested offer runs.
int fr_gemm_i8_i32(int m, int k, int n, int64_t alpha, const int8_t *a, int64_t lda,
                   const int8_t *b, int64_t ldb, int64_t beta, int32_t *c, int64_t ldc,
                   int row0, int rows, int threads, int force_avx2) {
    if (k > 65793 || threads < 1) return 4;
    const bool vnni = have_vnni() && !force_avx2;
    const int kq = (k + 3) / 4;
    const int r_end = std::min(m, row0 + rows);
    const int nblocks_n = (n + NC - 1) / NC;
    const int nblocks_m = (r_end - row0 + MC - 1) / MC;
    const int items = nblocks_n * nblocks_m;
    std::atomic<int> next{0};
    auto worker = [&]() {
        std::vector<int8_t> pb((size_t)kq * 4 * NC), pa((size_t)kq * 4 * MC);
        int32_t acc[VMR * VNR];
        int last_nb = -1;
        for (;;) {
            int it = next.fetch_add(1);
            if (it >= items) break;
            int nb = it / nblocks_m, mb = it % nblocks_m;
            int j0 = nb * NC, jn = std::min(n, j0 + NC);
            int i0 = row0 + mb * MC, in = std::min(r_end, i0 + MC);
            if (nb != last_nb) {
                for (int jp = j0; jp < jn; jp += VNR)
                    pack_b_panel(b, ldb, k, jp, n, pb.data() + (size_t)(jp - j0) * kq * 4);
                last_nb = nb;
            }
            for (int ip = i0; ip < in; ip += VMR)
                pack_a_panel(a, lda, k, ip, m, pa.data() + (size_t)(ip - i0) * kq * 4);
            for (int ip = i0; ip < in; ip += VMR)
                for (int jp = j0; jp < jn; jp += VNR) {
                    const int8_t *A = pa.data() + (size_t)(ip - i0) * kq * 4;
                    const int8_t *B = pb.data() + (size_t)(jp - j0) * kq * 4;
                    if (vnni) tile_vnni(kq, A, B, acc);
                    else tile_avx2(kq, A, B, acc);
                    for (int i = 0; i < VMR && ip + i < in; ++i)
                        for (int j = 0; j < VNR && jp + j < jn; ++j)
                            finish(c + (int64_t)(ip + i) * ldc + (jp + j), acc[i * VNR + j], alpha, beta);
                }
        }
    };
    std::vector<std::thread> pool;
    for (int t = 1; t < threads; ++t) pool.emplace_back(worker);
    worker();
    for (auto &t : pool) t.join();
    return 0;
}

}  // extern "C"
