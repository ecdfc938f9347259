// fastroute.cpp -- TEST/BENCH INFRASTRUCTURE ONLY: the CPU baseline.
//
// C++ restatements of the reference's CPU routes for the hot-path
// configurations, timed beside the GPU by bench.py (cpu_baseline, kind
// "port").  The reference binary is Rust and cannot be built here; these
// follow its files:
//   fr_gemm_i8_i32 -- the blocked full-depth traversal kernel.rs::run
//               (crates/uor-matmul-gemm/src/kernel.rs:1016-1377) with
//               blocking MC=128, NC=1024 (generated.rs:181-205), B packed in
//               16-column panels grouped by k-quads, A in 8-row panels, and the
//               AVX-512 VNNI dpbusd 8x16 tile with the offset identity
//               sum (a+128)*b - 128*sum b (crates/uor-matmul-kernels/src/isa/
//               x86.rs:704-715, 843-897); the AVX2 madd tile when VNNI is
//               absent (x86.rs:80-96).  Exact i32 lanes fold to i128, then the
//               Linear epilogue and the saturating i32 encode.
//   fr_gemm_i8_i64_chunked -- the same tiles past one i32 lane: k streamed in
//               65536-deep chunks folded into i64 (kernel.rs:1310-1376).
//   fr_lut4        -- the table-lookup product over Packed<Grid<16>,2> codes,
//               one call per codebook group as the decode-shape case makes
//               them.  mode 0, tabulation (tabulated.rs:3867-4555 row_tile):
//               per tile of rows and k-pair, a 256-entry table of exact pair
//               sums indexed by the packed byte, then one table read-add per
//               code byte per column.  mode 1, the decline to decode-then-dense
//               (tabulated.rs:2555-2745, coded.rs:98-140): the group's codes
//               decoded to i8 and multiplied by the dpbusd/madd tile above.
//   fr_trop_i8     -- driver::gemm's (max,+) at Trop<i8> (driver.rs:147-181)
//               on the AVX2_TROP_I16 tile (isa/x86.rs:935-1055): packed i16
//               with -inf as i16::MIN, max(acc, adds(a, b)) on a 4 x 16 tile,
//               unpacked by the TROP_I16 separation (tropical.rs:91-125).
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

// Items 0..items-1 claimed by `threads` workers (the caller is one of them).
template <class Make>
void parallel_items(int items, int threads, Make make_worker) {
    std::atomic<int> next{0};
    auto run = [&]() {
        auto work = make_worker();
        for (;;) {
            int it = next.fetch_add(1);
            if (it >= items) break;
            work(it);
        }
    };
    std::vector<std::thread> pool;
    for (int t = 1; t < threads; ++t) pool.emplace_back(run);
    run();
    for (auto &t : pool) t.join();
}

// ------------------------------------------------------------ LUT decode --

inline int nib(const uint8_t *row, int p) { return (row[p >> 1] >> ((p & 1) * 4)) & 15; }

// Tabulation, one row of A: per block of PB k-pairs, T[pp][hi*16 + lo] =
// book[lo]*a[2p] + book[hi]*a[2p+1], then acc[j] += T[pp][code byte].
__attribute__((target("avx2")))
void lut_tab_row(int k, const int8_t *a, const uint8_t *codes, int cols, const int8_t *book,
                 int32_t *acc, int32_t *T) {
    constexpr int PB = 32;
    const int kp = k / 2;
    const __m256i b0 = _mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i *)book));
    const __m256i b1 = _mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i *)(book + 8)));
    for (int j = 0; j < cols; ++j) acc[j] = 0;
    for (int p0 = 0; p0 < kp; p0 += PB) {
        const int pn = std::min(PB, kp - p0);
        for (int pp = 0; pp < pn; ++pp) {
            const int p = p0 + pp;
            const __m256i ae = _mm256_set1_epi32(a[2 * p]);
            const __m256i lo0 = _mm256_mullo_epi32(b0, ae), lo1 = _mm256_mullo_epi32(b1, ae);
            int32_t *t = T + pp * 256;
            for (int h = 0; h < 16; ++h) {
                const __m256i bh = _mm256_set1_epi32((int)book[h] * a[2 * p + 1]);
                _mm256_storeu_si256((__m256i *)(t + 16 * h), _mm256_add_epi32(lo0, bh));
                _mm256_storeu_si256((__m256i *)(t + 16 * h + 8), _mm256_add_epi32(lo1, bh));
            }
        }
        for (int j = 0; j < cols; ++j) {
            const uint8_t *cj = codes + (int64_t)j * kp + p0;
            int32_t sum = acc[j];
            for (int pp = 0; pp < pn; ++pp) sum += T[pp * 256 + cj[pp]];
            acc[j] = sum;
        }
    }
}

// Tabulation, a tile of 8 rows of A: the table's entries are 8-lane vectors
// (one lane per row), so each code byte costs one vector read-add.
__attribute__((target("avx2")))
void lut_tab_rows8(int k, const int8_t *a, int64_t lda, int rows, const uint8_t *codes,
                   int cols, const int8_t *book, int32_t *acc_out, int32_t *T_mem) {
    constexpr int PB = 4;
    const int kp = k / 2;
    // acc_out: cols x 8 lanes; T_mem: PB x 256 x 8 lanes (unaligned is fine).
    __m256i *acc = (__m256i *)acc_out, *T = (__m256i *)T_mem;
    for (int j = 0; j < cols; ++j) _mm256_storeu_si256(acc + j, _mm256_setzero_si256());
    for (int p0 = 0; p0 < kp; p0 += PB) {
        const int pn = std::min(PB, kp - p0);
        for (int pp = 0; pp < pn; ++pp) {
            const int p = p0 + pp;
            alignas(32) int32_t ev[8] = {0}, od[8] = {0};
            for (int r = 0; r < rows; ++r) {
                ev[r] = a[r * lda + 2 * p];
                od[r] = a[r * lda + 2 * p + 1];
            }
            const __m256i e = _mm256_load_si256((const __m256i *)ev);
            const __m256i o = _mm256_load_si256((const __m256i *)od);
            __m256i lo[16];
            for (int l = 0; l < 16; ++l) lo[l] = _mm256_mullo_epi32(e, _mm256_set1_epi32(book[l]));
            __m256i *t = T + pp * 256;
            for (int h = 0; h < 16; ++h) {
                const __m256i hv = _mm256_mullo_epi32(o, _mm256_set1_epi32(book[h]));
                for (int l = 0; l < 16; ++l)
                    _mm256_storeu_si256(t + 16 * h + l, _mm256_add_epi32(lo[l], hv));
            }
        }
        for (int j = 0; j < cols; ++j) {
            const uint8_t *cj = codes + (int64_t)j * kp + p0;
            __m256i sum = _mm256_loadu_si256(acc + j);
            for (int pp = 0; pp < pn; ++pp)
                sum = _mm256_add_epi32(sum, _mm256_loadu_si256(T + pp * 256 + cj[pp]));
            _mm256_storeu_si256(acc + j, sum);
        }
    }
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

// The chunked full-depth route (kernel.rs:1310-1376) for depths past one i32
// lane: C (m x n, i64, alpha 1, beta 0) += the exact sums over k, each 8 x 16
// output tile streaming k in chunks of 65536 (|a|, |b| <= 128 keeps a chunk's
// i32 lanes exact) folded into i64.  Output tiles are the work items (the
// caller-driven partition).  Rows of A and B are k bytes apart (lda, ldb).
int fr_gemm_i8_i64_chunked(int m, int64_t k, int n, const int8_t *a, int64_t lda, const int8_t *b,
                           int64_t ldb, int64_t *c, int64_t ldc, int threads) {
    constexpr int64_t KC = 65536;
    if (threads < 1 || k % 4 != 0) return 4;
    const bool vnni = have_vnni();
    const int tm = (m + VMR - 1) / VMR, tn = (n + VNR - 1) / VNR;
    parallel_items(tm * tn, threads, [&]() {
        return [&, pa = std::vector<int8_t>((size_t)KC * VMR), pb = std::vector<int8_t>((size_t)KC * VNR)](
                   int it) mutable {
            const int i0 = it / tn * VMR, j0 = it % tn * VNR;
            int64_t sum[VMR * VNR] = {0};
            int32_t acc[VMR * VNR];
            for (int64_t k0 = 0; k0 < k; k0 += KC) {
                const int kc = (int)std::min<int64_t>(KC, k - k0);
                pack_a_panel(a + k0, lda, kc, i0, m, pa.data());
                pack_b_panel(b + k0 * ldb, ldb, kc, j0, n, pb.data());
                if (vnni) tile_vnni(kc / 4, pa.data(), pb.data(), acc);
                else tile_avx2(kc / 4, pa.data(), pb.data(), acc);
                for (int e = 0; e < VMR * VNR; ++e) sum[e] += acc[e];
            }
            for (int i = 0; i < VMR && i0 + i < m; ++i)
                for (int j = 0; j < VNR && j0 + j < n; ++j) c[(int64_t)(i0 + i) * ldc + j0 + j] = sum[i * VNR + j];
        };
    });
    return 0;
}

// The table-lookup product C (m x n, i32, Nearest, alpha 1, beta 0) of A (m x
// k, row-major lda) and W (n x k as Packed<Grid<16>,2> codes, k/2 bytes per
// row, low nibble first) with one 16-entry codebook per `group` rows of W: one
// call per group, groups split over threads.  mode 0 tabulation, mode 1
// decode-then-dense.  Returns 4 on arguments it does not handle.
int fr_lut4(int m, int k, int n, const int8_t *a, int64_t lda, const uint8_t *codes,
            const int8_t *books, int group, int32_t *c, int64_t ldc, int groups_run, int threads,
            int mode) {
    if (k % 4 != 0 || group % VNR != 0 || n % group != 0 || threads < 1 || k > 65793) return 4;
    const int ngroups = std::min(n / group, groups_run);
    const int kp = k / 2, kq = k / 4;
    const bool vnni = have_vnni();
    if (mode == 0) {
        parallel_items(ngroups, threads, [&]() {
            return [&, acc = std::vector<int32_t>(8 * group), T = std::vector<int32_t>(8 * 4 * 256),
                    acc1 = std::vector<int32_t>(group),
                    T1 = std::vector<int32_t>(32 * 256)](int g) mutable {
                const uint8_t *cg = codes + (int64_t)g * group * kp;
                const int8_t *book = books + 16 * g;
                if (m < 8) {
                    for (int i = 0; i < m; ++i) {
                        lut_tab_row(k, a + i * lda, cg, group, book, acc1.data(), T1.data());
                        for (int j = 0; j < group; ++j) c[i * ldc + g * group + j] = acc1[j];
                    }
                    return;
                }
                for (int i0 = 0; i0 < m; i0 += 8) {
                    const int rows = std::min(8, m - i0);
                    lut_tab_rows8(k, a + i0 * lda, lda, rows, cg, group, book, acc.data(),
                                  T.data());
                    for (int j = 0; j < group; ++j)
                        for (int r = 0; r < rows; ++r)
                            c[(i0 + r) * ldc + g * group + j] = acc[8 * j + r];
                }
            };
        });
        return 0;
    }
    // Decode-then-dense: A packed once per worker, each group's codes decoded
    // straight into the dense tile's B panel layout.
    const int mp = (m + VMR - 1) / VMR;
    parallel_items(ngroups, threads, [&]() {
        std::vector<int8_t> pa((size_t)mp * kq * 4 * VMR);
        for (int ip = 0; ip < mp; ++ip)
            pack_a_panel(a, lda, k, ip * VMR, m, pa.data() + (size_t)ip * kq * 4 * VMR);
        return [&, pa = std::move(pa), pb = std::vector<int8_t>((size_t)kq * 4 * group)](
                   int g) mutable {
            const uint8_t *cg = codes + (int64_t)g * group * kp;
            const int8_t *book = books + 16 * g;
            for (int jp = 0; jp < group; jp += VNR) {
                int8_t *out = pb.data() + (size_t)jp * kq * 4;
                for (int q = 0; q < kq; ++q)
                    for (int j = 0; j < VNR; ++j) {
                        const uint8_t *row = cg + (int64_t)(jp + j) * kp;
                        for (int t = 0; t < 4; ++t)
                            out[(q * VNR + j) * 4 + t] = book[nib(row, 4 * q + t)];
                    }
            }
            int32_t acc[VMR * VNR];
            for (int ip = 0; ip < mp; ++ip)
                for (int jp = 0; jp < group; jp += VNR) {
                    const int8_t *A = pa.data() + (size_t)ip * kq * 4 * VMR;
                    const int8_t *B = pb.data() + (size_t)jp * kq * 4;
                    if (vnni) tile_vnni(kq, A, B, acc);
                    else tile_avx2(kq, A, B, acc);
                    for (int i = 0; i < VMR && ip * VMR + i < m; ++i)
                        for (int j = 0; j < VNR; ++j)
                            c[(ip * VMR + i) * ldc + g * group + jp + j] = acc[i * VNR + j];
                }
        };
    });
    return 0;
}

// Max-plus at Trop<i8> -> Trop<i32> under the default MaxPlus (alpha = 0
// finite, beta = -inf), rows [row0, row0+rows): A and B are 2-byte {value,
// finite} records (m x k, k x n, row-major), C 8-byte {i32 value, u8 finite}
// records (value 0 when not finite).
int fr_trop_i8(int m, int k, int n, const uint8_t *a, const uint8_t *b, uint8_t *c, int row0,
               int rows, int threads);

}  // extern "C"

namespace {

constexpr int TMR = 4, TNR = 16;      // the AVX2_TROP_I16 tile
constexpr int16_t TROP_ZERO = INT16_MIN;

__attribute__((target("avx2")))
void trop_tile(int kc, const int16_t *pa, const int16_t *pb, int16_t *acc) {
    __m256i t[TMR];
    for (int i = 0; i < TMR; ++i) t[i] = _mm256_set1_epi16(TROP_ZERO);
    for (int p = 0; p < kc; ++p) {
        const __m256i bv = _mm256_loadu_si256((const __m256i *)(pb + p * TNR));
        for (int i = 0; i < TMR; ++i)
            t[i] = _mm256_max_epi16(t[i], _mm256_adds_epi16(_mm256_set1_epi16(pa[p * TMR + i]), bv));
    }
    for (int i = 0; i < TMR; ++i) _mm256_storeu_si256((__m256i *)(acc + i * TNR), t[i]);
}

inline int16_t trop_lane(const uint8_t *rec) {
    return rec[1] ? (int16_t)(int8_t)rec[0] : TROP_ZERO;
}

}  // namespace

extern "C" int fr_trop_i8(int m, int k, int n, const uint8_t *a, const uint8_t *b, uint8_t *c,
                          int row0, int rows, int threads) {
    if (n % TNR != 0 || threads < 1) return 4;
    const int r_end = std::min(m, row0 + rows);
    const int panels = n / TNR;
    // B packed once: panel q is k-major, 16 columns per k-step.
    std::vector<int16_t> pb((size_t)panels * k * TNR);
    parallel_items(panels, threads, [&]() {
        return [&](int q) {
            int16_t *out = pb.data() + (size_t)q * k * TNR;
            for (int p = 0; p < k; ++p)
                for (int j = 0; j < TNR; ++j)
                    out[p * TNR + j] = trop_lane(b + 2 * ((int64_t)p * n + q * TNR + j));
        };
    });
    // Work items: 32 rows x 16 panels (256 columns); B's panel stays in L2
    // across the block's eight 4-row tiles.
    constexpr int RB = 32, PBK = 16;
    const int rblocks = (r_end - row0 + RB - 1) / RB, cblocks = (panels + PBK - 1) / PBK;
    // Finite sums lie in [-256, 254]; an absorbed lane is at most
    // i16::MIN + 127, far below (tropical.rs:109-125).
    parallel_items(rblocks * cblocks, threads, [&]() {
        return [&, pa = std::vector<int16_t>((size_t)RB * k)](int it) mutable {
            const int rb = it / cblocks, cb = it % cblocks;
            const int i0 = row0 + rb * RB, in = std::min(r_end, i0 + RB);
            for (int ip = i0; ip < in; ip += TMR)
                for (int p = 0; p < k; ++p)
                    for (int i = 0; i < TMR; ++i) {
                        const int row = ip + i;
                        pa[(size_t)(ip - i0) * k + p * TMR + i] =
                            row < in ? trop_lane(a + 2 * ((int64_t)row * k + p)) : TROP_ZERO;
                    }
            int16_t acc[TMR * TNR];
            for (int q = cb * PBK; q < std::min(panels, (cb + 1) * PBK); ++q)
                for (int ip = i0; ip < in; ip += TMR) {
                    trop_tile(k, pa.data() + (size_t)(ip - i0) * k, pb.data() + (size_t)q * k * TNR,
                              acc);
                    for (int i = 0; i < TMR && ip + i < in; ++i)
                        for (int j = 0; j < TNR; ++j) {
                            const int16_t v = acc[i * TNR + j];
                            uint8_t *rec = c + 8 * ((int64_t)(ip + i) * n + q * TNR + j);
                            const int fin = v >= -256;
                            const int32_t val = fin ? v : 0;
                            memcpy(rec, &val, 4);
                            rec[4] = (uint8_t)fin;
                        }
                }
        };
    });
    return 0;
}
