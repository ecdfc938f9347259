// Products with one coded operand, any fixed-width codec tier over the i8
// alphabet, on gfx950.
//
// Replaces gemm_tabulated (crates/uor-matmul-gemm/src/tabulated.rs:2555, W
// n x k, transposed by declaration) and coded_gemm (crates/uor-matmul-gemm/
// src/coded.rs:98-140, B k x n) for the tiers of crates/uor-matmul-codec/src/
// codecs.rs: Identity, Grid<N>, Book<N,BLK,K>, Sign<BLK,K>, Ternary<BLK,K>,
// each optionally inside Packed<_, P> and Offset<_, zero>.  The codec is not an
// argument of the arithmetic (CK-05, CD-13): every element decodes to one i8
// value and the product is the exact i8 product of the decoded operand.
//
// Routes.  With a scratch offer of k * round_up(n, 16) bytes (plus the dense
// route's own), `coded_decode_kernel` writes the decoded operand once as a
// k x n int8 matrix -- 128 x 128 tiles through LDS, 16-byte row stores -- and
// the dense int8 MFMA route multiplies it.  Without an offer, one thread per
// output cell decodes its column as it sums.  Both give the same bytes.

#include "common.hpp"
#include "collapse.hpp"

extern "C" int uor_gfx950_gemm_i8(const uor_view *a, const uor_view *b, const uor_view *c, int out_type,
                                  int64_t alpha, int64_t beta, int encode, void *scratch,
                                  uint64_t scratch_bytes, void *stream, uor_route *route);
extern "C" uint64_t uor_gfx950_suggested_scratch_i8(uint64_t m, uint64_t k, uint64_t n);

namespace uor {

// A codec as the decode reads it (see uor_codec).
struct CodecDev {
    int tier, code_bits, packed, has_zero;
    int zero;                // Offset's zero point (i8)
    uint32_t sub_bits, sub_mask;
    uint64_t entries, block;
    uint64_t ib, mb;         // the base tier's MAX_BLOCK, and the codec's
    const int8_t *table;
};

// A coded operand: rows x cols over `cd`, codes row-major, `cb` bytes each.
struct CodedArgs {
    CodecDev cd;
    const uint8_t *codes;
    int cb;
    uint64_t rows, cols, per_row;
};

// Codec<i8, Bd>::decode_element of the base tier (codecs.rs:49-51 Identity,
// :102-104 Grid, :306-308 Book, :387-400 Sign, :492-516 Ternary).
__device__ inline int dec_base(const CodecDev &c, uint32_t code, uint64_t i) {
    switch (c.tier) {
    case UOR_TIER_IDENTITY: return (int)(int8_t)(uint8_t)code;
    case UOR_TIER_GRID: return c.table[code % c.entries];
    case UOR_TIER_BOOK: return c.table[(code % c.entries) * c.block + i % c.block];
    case UOR_TIER_SIGN: {
        const uint64_t bit = i % c.block;
        return (bit < (uint64_t)c.code_bits && ((code >> bit) & 1u)) ? 1 : -1;
    }
    default: {
        const uint64_t shift = 2 * (i % c.block);
        const uint32_t d = shift < (uint64_t)c.code_bits ? (code >> shift) & 3u : 0u;
        return d == 0 ? -1 : (d == 2 ? 1 : 0);
    }
    }
}

// Packed (codecs.rs:181-199: the low sub-code first) and Offset
// (codecs.rs:608-616: i8 wrapping_sub) around the base tier.
__device__ inline int8_t dec(const CodecDev &c, uint32_t code, uint64_t i) {
    int v;
    if (c.packed) {
        const uint64_t p = i / c.ib;
        v = dec_base(c, (code >> (c.sub_bits * (uint32_t)p)) & c.sub_mask, i % c.ib);
    } else {
        v = dec_base(c, code, i);
    }
    if (c.has_zero) v -= c.zero;
    return (int8_t)v;
}

// CodedMatrix::at for a fixed-width tier (matrix.rs:202-207).
__device__ inline int8_t coded_at(const CodedArgs &W, uint64_t r, uint64_t q) {
    const uint64_t at = r * W.per_row + q / W.cd.mb;
    const uint32_t code = W.cb == 1 ? (uint32_t)W.codes[at] : (uint32_t)((const uint16_t *)W.codes)[at];
    return dec(W.cd, code, q % W.cd.mb);
}

// A cursor along one row of a coded operand: the stored code, the sub-code
// of a packed byte it is at, and the position inside the base tier's block,
// advanced one element at a time without divisions.
struct Walk {
    uint64_t at;      // index of the stored code
    uint32_t code;    // the stored code
    uint32_t sub;     // the base tier's code (sub-code of a packed byte), % N for Grid/Book
    uint32_t sp, ii;  // sub-code index in the byte, position in the base block
};

__device__ inline uint32_t load_code(const CodedArgs &W, uint64_t at) {
    return W.cb == 1 ? (uint32_t)W.codes[at] : (uint32_t)((const uint16_t *)W.codes)[at];
}

__device__ inline void walk_sub(const CodedArgs &W, Walk &w) {
    const CodecDev &c = W.cd;
    uint32_t s = c.packed ? (w.code >> (c.sub_bits * w.sp)) & c.sub_mask : w.code;
    if ((c.tier == UOR_TIER_GRID || c.tier == UOR_TIER_BOOK) && c.entries <= 0xFFFFu) s %= (uint32_t)c.entries;
    w.sub = s;
}

// The cursor at element (r, q) of the operand.
__device__ inline void walk_start(const CodedArgs &W, Walk &w, uint64_t r, uint64_t q) {
    const uint32_t pos = (uint32_t)(q % W.cd.mb);
    w.at = r * W.per_row + q / W.cd.mb;
    w.sp = pos / (uint32_t)W.cd.ib;
    w.ii = pos % (uint32_t)W.cd.ib;
    w.code = load_code(W, w.at);
    walk_sub(W, w);
}

// The element under the cursor (dec, with the cursor's state).
__device__ inline int8_t walk_value(const CodedArgs &W, const Walk &w) {
    const CodecDev &c = W.cd;
    int v;
    switch (c.tier) {
    case UOR_TIER_IDENTITY: v = (int)(int8_t)(uint8_t)w.sub; break;
    case UOR_TIER_GRID: v = c.table[w.sub]; break;
    case UOR_TIER_BOOK: v = c.table[(uint64_t)w.sub * c.block + w.ii]; break;
    case UOR_TIER_SIGN: v = (w.ii < (uint32_t)c.code_bits && ((w.sub >> w.ii) & 1u)) ? 1 : -1; break;
    default: {
        const uint32_t sh = 2 * w.ii;
        const uint32_t d = sh < (uint32_t)c.code_bits ? (w.sub >> sh) & 3u : 0u;
        v = d == 0 ? -1 : (d == 2 ? 1 : 0);
    }
    }
    if (c.has_zero) v -= c.zero;
    return (int8_t)v;
}

// Advance by one element; `more` says whether another element follows in
// this row (so no code past the row's last is read).
__device__ inline void walk_next(const CodedArgs &W, Walk &w, bool more) {
    if (++w.ii < (uint32_t)W.cd.ib) return;
    w.ii = 0;
    if (W.cd.packed && ++w.sp < (uint32_t)W.cd.packed) {
        walk_sub(W, w);
        return;
    }
    w.sp = 0;
    ++w.at;
    if (more) {
        w.code = load_code(W, w.at);
        walk_sub(W, w);
    }
}

// The decoded operand as a k x n int8 matrix (row stride ldw, a multiple of
// 16).  W n x k (tabulated): one 128 x 128 tile per workgroup; each thread
// walks 64 consecutive elements of one row of W (one column of the tile) into
// LDS, then the tile leaves as 16-byte row chunks.
__global__ void __launch_bounds__(256) coded_decode_t_kernel(CodedArgs W, uint64_t k, uint64_t n, int8_t *out,
                                                             uint64_t ldw) {
    __shared__ __attribute__((aligned(16))) int8_t tile[128][128];
    const int t = threadIdx.x;
    const uint64_t j0 = (uint64_t)blockIdx.x * 128, k0 = (uint64_t)blockIdx.y * 128;
    const int cl = t & 127, kh = t >> 7;
    const uint64_t j = j0 + cl, p0 = k0 + 64 * kh;
    if (j < n && p0 < k) {
        const int cnt = (int)(k - p0 < 64 ? k - p0 : 64);
        Walk w;
        walk_start(W, w, j, p0);
        for (int q = 0; q < cnt; ++q) {
            tile[64 * kh + q][cl] = walk_value(W, w);
            walk_next(W, w, q + 1 < cnt);
        }
    }
    __syncthreads();
    const int ch = t & 7;
#pragma unroll
    for (int pass = 0; pass < 4; ++pass) {
        const int r = pass * 32 + (t >> 3);
        const uint64_t kk = k0 + r, jc = j0 + 16 * ch;
        if (kk < k && jc < ldw) *(uint4 *)(out + kk * ldw + jc) = *(const uint4 *)&tile[r][16 * ch];
    }
}

// The same tile for one-byte codes of 4 or 8 elements whose rows are whole
// 16-byte runs: the workgroup first decodes all 256 codes into an LDS table
// of D = MAX_BLOCK / 4 packed dwords, then each thread loads its 64 elements'
// codes with one 16-byte (D = 1) or 8-byte (D = 2) load and expands them
// through the table.
template <int D>
__global__ void __launch_bounds__(256) coded_decode_t_lut_kernel(CodedArgs W, uint64_t k, uint64_t n, int8_t *out,
                                                                 uint64_t ldw) {
    __shared__ __attribute__((aligned(16))) int8_t tile[128][128];
    __shared__ uint32_t lut[256 * D];
    const int t = threadIdx.x;
    for (int idx = t; idx < 256 * D; idx += 256) {
        const uint32_t code = (uint32_t)idx / D, part = (uint32_t)idx % D;
        uint32_t v = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) v |= (uint32_t)(uint8_t)dec(W.cd, code, 4 * part + e) << (8 * e);
        lut[idx] = v;
    }
    __syncthreads();
    const uint64_t j0 = (uint64_t)blockIdx.x * 128, k0 = (uint64_t)blockIdx.y * 128;
    const int cl = t & 127, kh = t >> 7;
    const uint64_t j = j0 + cl, p0 = k0 + 64 * kh;
    constexpr int NC = 16 / D;  // codes of this thread's 64 elements
    if (j < n && p0 < k) {
        const uint8_t *src = W.codes + j * W.per_row + p0 / (4 * D);
        uint32_t cw[4];
        if constexpr (D == 1) {
            const uint4 x = *(const uint4 *)src;
            cw[0] = x.x, cw[1] = x.y, cw[2] = x.z, cw[3] = x.w;
        } else {
            const uint2 x = *(const uint2 *)src;
            cw[0] = x.x, cw[1] = x.y, cw[2] = 0, cw[3] = 0;
        }
#pragma unroll
        for (int q = 0; q < NC; ++q) {
            const uint32_t code = (cw[q >> 2] >> (8 * (q & 3))) & 0xFFu;
#pragma unroll
            for (int part = 0; part < D; ++part) {
                const uint32_t v = lut[code * D + part];
#pragma unroll
                for (int e = 0; e < 4; ++e) tile[64 * kh + q * 4 * D + 4 * part + e][cl] = (int8_t)(v >> (8 * e));
            }
        }
    }
    __syncthreads();
    const int ch = t & 7;
#pragma unroll
    for (int pass = 0; pass < 4; ++pass) {
        const int r = pass * 32 + (t >> 3);
        const uint64_t kk = k0 + r, jc = j0 + 16 * ch;
        if (kk < k && jc < ldw) *(uint4 *)(out + kk * ldw + jc) = *(const uint4 *)&tile[r][16 * ch];
    }
}

// W k x n (coded_gemm): the rows are already the output's; each thread walks
// 16 consecutive elements of one row and stores them as one 16-byte chunk
// (zeros past column n, inside the row stride).
__global__ void __launch_bounds__(256) coded_decode_kernel(CodedArgs W, uint64_t k, uint64_t n, int8_t *out,
                                                           uint64_t ldw) {
    const uint64_t chunks = ldw / 16;
    const uint64_t id = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (id >= k * chunks) return;
    const uint64_t p = id / chunks, j0 = 16 * (id % chunks);
    union {
        uint4 v;
        int8_t b[16];
    } u;
    u.v = uint4{0, 0, 0, 0};
    if (j0 < n) {
        const int cnt = (int)(n - j0 < 16 ? n - j0 : 16);
        Walk w;
        walk_start(W, w, p, j0);
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            if (q < cnt) {
                u.b[q] = walk_value(W, w);
                walk_next(W, w, q + 1 < cnt);
            }
        }
    }
    *(uint4 *)(out + p * ldw + j0) = u.v;
}

// ------------------------------------------------------------ few rows --
//
// m <= 8 and W n x k (the table-lookup orientation): no decoded copy.  One
// wave per output column j; lane l walks its 16-aligned slice of row j of W
// (contiguous codes, so a wave reads one run of the row), decodes each
// element in registers and multiplies it into up to MR rows of A (int32 per
// lane: a slice is at most 2^16 elements), then the wave adds its lanes in
// int64 and lane r finishes row r.  The tier is a template parameter, so the
// per-element decode is a handful of VALU instructions.
constexpr uint64_t GEMV_MAX_K = 1ull << 22;

struct GemvArgs {
    const int8_t *a;
    int64_t ars, acs;
    int a_vec;  // unit column stride, 16-byte aligned rows: 16-byte loads
    char *c;
    int64_t crs, ccs;
    uint64_t m, k, n;
    int64_t alpha, beta;
    int mode, ob;
};

template <int TIER>
__device__ inline int8_t walk_value_t(const CodedArgs &W, const Walk &w) {
    const CodecDev &c = W.cd;
    int v;
    if constexpr (TIER == UOR_TIER_IDENTITY) v = (int)(int8_t)(uint8_t)w.sub;
    else if constexpr (TIER == UOR_TIER_GRID) v = c.table[w.sub];
    else if constexpr (TIER == UOR_TIER_BOOK) v = c.table[(uint64_t)w.sub * c.block + w.ii];
    else if constexpr (TIER == UOR_TIER_SIGN) v = (w.ii < (uint32_t)c.code_bits && ((w.sub >> w.ii) & 1u)) ? 1 : -1;
    else {
        const uint32_t sh = 2 * w.ii;
        const uint32_t d = sh < (uint32_t)c.code_bits ? (w.sub >> sh) & 3u : 0u;
        v = d == 0 ? -1 : (d == 2 ? 1 : 0);
    }
    if (c.has_zero) v -= c.zero;
    return (int8_t)v;
}

__device__ inline void finish_any(char *cp, int64_t sum, const GemvArgs &G) {
    switch (G.ob) {
    case 1: linear_finish<1, false>(cp, sum, G.alpha, G.beta, G.mode); break;
    case 2: linear_finish<2, false>(cp, sum, G.alpha, G.beta, G.mode); break;
    case 4: linear_finish<4, false>(cp, sum, G.alpha, G.beta, G.mode); break;
    case 8: linear_finish<8, false>(cp, sum, G.alpha, G.beta, G.mode); break;
    default: linear_finish<16, false>(cp, sum, G.alpha, G.beta, G.mode); break;
    }
}

template <int TIER, int MR>
__global__ void __launch_bounds__(256) coded_gemv_kernel(CodedArgs W, GemvArgs G) {
    const int lane = threadIdx.x & 63;
    const uint64_t j = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (j >= G.n) return;  // whole waves
    const uint64_t slice = ((G.k + 63) / 64 + 15) / 16 * 16;
    const uint64_t p0 = (uint64_t)lane * slice;
    const uint64_t p1 = p0 + slice < G.k ? p0 + slice : G.k;
    int acc[MR];
#pragma unroll
    for (int r = 0; r < MR; ++r) acc[r] = 0;
    if (p0 < p1) {
        Walk w;
        walk_start(W, w, j, p0);
        for (uint64_t p = p0; p < p1; p += 16) {
            const int cnt = (int)(p1 - p < 16 ? p1 - p : 16);
            int8_t av[MR][16];
#pragma unroll
            for (int r = 0; r < MR; ++r) {
                if ((uint64_t)r < G.m) {
                    if (G.a_vec && cnt == 16) {
                        *(uint4 *)av[r] = *(const uint4 *)(G.a + (int64_t)r * G.ars + (int64_t)p);
                    } else {
#pragma unroll
                        for (int e = 0; e < 16; ++e)
                            av[r][e] = e < cnt ? G.a[(int64_t)r * G.ars + (int64_t)(p + e) * G.acs] : 0;
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < 16; ++e) av[r][e] = 0;
                }
            }
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                if (e < cnt) {
                    const int wv = walk_value_t<TIER>(W, w);
                    walk_next(W, w, p + e + 1 < p1);
#pragma unroll
                    for (int r = 0; r < MR; ++r) acc[r] += (int)av[r][e] * wv;
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < MR; ++r) {
        int64_t v = acc[r];
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
        if (lane == r && (uint64_t)r < G.m)
            finish_any(G.c + ((int64_t)r * G.crs + (int64_t)j * G.ccs) * G.ob, v, G);
    }
}

// The same product when each row of W is a whole number of 16-byte code
// windows and A's rows are 16-byte aligned (the common case): lane l of the
// wave takes windows l, l + 64, ... of row j, so a wave step reads 1 KiB of
// the row with one 16-byte load per lane, and the next step's window is
// loaded before this one is decoded.  A window holds 16 / cb codes, i.e.
// E = (16 / cb) * MAX_BLOCK elements, a multiple of 16 (the host checks).
template <int TIER, int MR>
__global__ void __launch_bounds__(256) coded_gemv_win_kernel(CodedArgs W, GemvArgs G) {
    const int lane = threadIdx.x & 63;
    const uint64_t j = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (j >= G.n) return;  // whole waves
    const CodecDev &c = W.cd;
    const uint64_t row_bytes = W.per_row * (uint64_t)W.cb;
    const uint64_t nwin = row_bytes / 16;
    const uint8_t *row = W.codes + j * row_bytes;
    const uint32_t cpw = 16u / (uint32_t)W.cb;             // codes per window
    const uint64_t E = (uint64_t)cpw * c.mb;                // elements per window
    const uint32_t P = c.packed ? (uint32_t)c.packed : 1u;
    const uint32_t ib = (uint32_t)c.ib;
    int acc[MR];
#pragma unroll
    for (int r = 0; r < MR; ++r) acc[r] = 0;
    uint64_t wi = (uint64_t)lane;
    uint4 nxt = wi < nwin ? *(const uint4 *)(row + 16 * wi) : uint4{0, 0, 0, 0};
    for (; wi < nwin; wi += 64) {
        const uint4 cur = nxt;
        if (wi + 64 < nwin) nxt = *(const uint4 *)(row + 16 * (wi + 64));
        const uint32_t d[4] = {cur.x, cur.y, cur.z, cur.w};
        // The cursor inside this window: code q, sub-code sp, position ii.
        uint32_t q = 0, sp = 0, ii = 0;
        auto code_at = [&](uint32_t qq) -> uint32_t {
            const uint32_t b = qq * (uint32_t)W.cb;
            const uint32_t dw = b >> 2;
            const uint32_t x = dw == 0 ? d[0] : dw == 1 ? d[1] : dw == 2 ? d[2] : d[3];
            return W.cb == 1 ? (x >> (8 * (b & 3))) & 0xFFu : (x >> (8 * (b & 3))) & 0xFFFFu;
        };
        Walk w;
        w.code = code_at(0);
        w.sp = 0;
        w.ii = 0;
        walk_sub(W, w);
        const uint64_t e0 = wi * E;
        for (uint64_t g = 0; g < E; g += 16) {
            int8_t av[MR][16];
#pragma unroll
            for (int r = 0; r < MR; ++r) {
                if ((uint64_t)r < G.m) *(uint4 *)av[r] = *(const uint4 *)(G.a + (int64_t)r * G.ars + (int64_t)(e0 + g));
                else *(uint4 *)av[r] = uint4{0, 0, 0, 0};
            }
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int wv = walk_value_t<TIER>(W, w);
#pragma unroll
                for (int r = 0; r < MR; ++r) acc[r] += (int)av[r][e] * wv;
                // advance inside the window
                if (++ii == ib) {
                    ii = 0;
                    if (++sp == P) {
                        sp = 0;
                        if (++q < cpw) w.code = code_at(q);
                    }
                    w.sp = sp;
                    walk_sub(W, w);
                }
                w.ii = ii;
            }
        }
    }
#pragma unroll
    for (int r = 0; r < MR; ++r) {
        int64_t v = acc[r];
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
        if (lane == r && (uint64_t)r < G.m)
            finish_any(G.c + ((int64_t)r * G.crs + (int64_t)j * G.ccs) * G.ob, v, G);
    }
}

// One-byte codes of 4 or 8 elements (Ternary<4,u8>, Sign<8,u8>,
// Packed<Grid<4>,4>, Book<_, 4|8, u8>, ...), m <= 4: the table variant.  Each
// workgroup first decodes all 256 codes into an LDS table of D = MAX_BLOCK / 4
// packed dwords per code (four i8 values each, through the same decode), so a
// code costs one byte extract, D LDS reads and D x MR v_dot4_i32_i8.  A wave
// takes 4 columns: the A bytes of a window are loaded once for all four, and
// each column's next code window is loaded before this one is used.
template <int MR, int D, int NCOL = 4>
__global__ void __launch_bounds__(256) coded_gemv_lut_kernel(CodedArgs W, GemvArgs G) {
    // CP copies of the table, entry x of copy c at word x * CP + c, lane l
    // reading copy l % CP: the lanes of one read meet in at most 64 / CP ways
    // on a bank, where random codes into one copy meet in 4-5.
    constexpr int CP = 16;
    __shared__ uint32_t lut[256 * D * CP];
    const int lane = threadIdx.x & 63;
    const uint64_t jb = ((uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * NCOL;
    const uint64_t nwin = W.per_row / 16;  // one-byte codes: a row is per_row bytes
    constexpr int E = 64 * D;              // elements per 16-byte window
    // Each column's first code window is requested before the table is
    // built, so the loads are in flight meanwhile.
    uint4 nxt[NCOL];
#pragma unroll
    for (int c = 0; c < NCOL; ++c)
        nxt[c] = ((uint64_t)lane < nwin && jb + c < G.n)
                     ? *(const uint4 *)(W.codes + (jb + c) * W.per_row + 16 * (uint64_t)lane)
                     : uint4{0, 0, 0, 0};
    for (int idx = threadIdx.x; idx < 256 * D; idx += 256) {
        const uint32_t code = (uint32_t)idx / D, part = (uint32_t)idx % D;
        uint32_t v = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) v |= (uint32_t)(uint8_t)dec(W.cd, code, 4 * part + e) << (8 * e);
#pragma unroll
        for (int c = 0; c < CP; ++c) lut[idx * CP + c] = v;
    }
    __syncthreads();
    if (jb >= G.n) return;  // whole waves, after the barrier
    int acc[NCOL][MR];
#pragma unroll
    for (int c = 0; c < NCOL; ++c)
#pragma unroll
        for (int r = 0; r < MR; ++r) acc[c][r] = 0;
    for (uint64_t wi = (uint64_t)lane; wi < nwin; wi += 64) {
        uint4 cur[NCOL];
#pragma unroll
        for (int c = 0; c < NCOL; ++c) {
            cur[c] = nxt[c];
            if (wi + 64 < nwin && jb + c < G.n)
                nxt[c] = *(const uint4 *)(W.codes + (jb + c) * W.per_row + 16 * (wi + 64));
        }
        uint32_t a[MR][E / 4];
#pragma unroll
        for (int r = 0; r < MR; ++r)
#pragma unroll
            for (int h = 0; h < E / 16; ++h) {
                uint4 v = uint4{0, 0, 0, 0};
                if ((uint64_t)r < G.m) v = *(const uint4 *)(G.a + (int64_t)r * G.ars + (int64_t)(wi * E + 16 * h));
                a[r][4 * h] = v.x;
                a[r][4 * h + 1] = v.y;
                a[r][4 * h + 2] = v.z;
                a[r][4 * h + 3] = v.w;
            }
#pragma unroll
        for (int c = 0; c < NCOL; ++c) {
            const uint32_t d[4] = {cur[c].x, cur[c].y, cur[c].z, cur[c].w};
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const uint32_t code = (d[q >> 2] >> (8 * (q & 3))) & 0xFFu;
#pragma unroll
                for (int part = 0; part < D; ++part) {
                    const int wv = (int)lut[(code * D + part) * CP + (lane % CP)];
#pragma unroll
                    for (int r = 0; r < MR; ++r)
                        acc[c][r] = __builtin_amdgcn_sdot4((int)a[r][q * D + part], wv, acc[c][r], false);
                }
            }
        }
    }
#pragma unroll
    for (int c = 0; c < NCOL; ++c)
#pragma unroll
        for (int r = 0; r < MR; ++r) {
            int64_t v = acc[c][r];
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
            if (lane == c * MR + r && (uint64_t)r < G.m && jb + c < G.n)
                finish_any(G.c + ((int64_t)r * G.crs + (int64_t)(jb + c) * G.ccs) * G.ob, v, G);
        }
}

template <int MR>
static void launch_gemv_lut(const CodedArgs &W, const GemvArgs &G, hipStream_t s) {
    if constexpr (MR == 8) {
        // Eight rows: two columns per wave, four-element codes only (the
        // eight-element codes' A window would not fit beside them).
        const dim3 grid((unsigned)((G.n + 7) / 8));
        hipLaunchKernelGGL((coded_gemv_lut_kernel<8, 1, 2>), grid, dim3(256), 0, s, W, G);
    } else {
        const dim3 grid((unsigned)((G.n + 15) / 16));
        if (W.cd.mb == 4) hipLaunchKernelGGL((coded_gemv_lut_kernel<MR, 1>), grid, dim3(256), 0, s, W, G);
        else hipLaunchKernelGGL((coded_gemv_lut_kernel<MR, 2>), grid, dim3(256), 0, s, W, G);
    }
}

template <int TIER, int MR>
static void launch_gemv_mr(const CodedArgs &W, const GemvArgs &G, bool win, dim3 grid, hipStream_t s) {
    if (win) hipLaunchKernelGGL((coded_gemv_win_kernel<TIER, MR>), grid, dim3(256), 0, s, W, G);
    else hipLaunchKernelGGL((coded_gemv_kernel<TIER, MR>), grid, dim3(256), 0, s, W, G);
}

template <int TIER>
static void launch_gemv_t(const CodedArgs &W, const GemvArgs &G, bool win, dim3 grid, hipStream_t s) {
    if (G.m <= 1) launch_gemv_mr<TIER, 1>(W, G, win, grid, s);
    else if (G.m <= 2) launch_gemv_mr<TIER, 2>(W, G, win, grid, s);
    else if (G.m <= 4) launch_gemv_mr<TIER, 4>(W, G, win, grid, s);
    else launch_gemv_mr<TIER, 8>(W, G, win, grid, s);
}

static void launch_gemv(const CodedArgs &W, const GemvArgs &G, bool win, hipStream_t s) {
    const dim3 grid((unsigned)((G.n + 3) / 4));
    switch (W.cd.tier) {
    case UOR_TIER_IDENTITY: launch_gemv_t<UOR_TIER_IDENTITY>(W, G, win, grid, s); break;
    case UOR_TIER_GRID: launch_gemv_t<UOR_TIER_GRID>(W, G, win, grid, s); break;
    case UOR_TIER_BOOK: launch_gemv_t<UOR_TIER_BOOK>(W, G, win, grid, s); break;
    case UOR_TIER_SIGN: launch_gemv_t<UOR_TIER_SIGN>(W, G, win, grid, s); break;
    default: launch_gemv_t<UOR_TIER_TERNARY>(W, G, win, grid, s); break;
    }
}

struct DirectArgs {
    const int8_t *a;
    int64_t ars, acs;
    char *c;
    int64_t crs, ccs;
    uint64_t m, k, n;
    int64_t alpha, beta;
    int mode;
};

// No offer: one thread per cell, its column of W decoded as it is summed
// (coded.rs:120-131's walk), then Linear::finish.
template <bool TRANS, int OB>
__global__ void __launch_bounds__(256) coded_direct_kernel(CodedArgs W, DirectArgs D) {
    const uint64_t cell = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (cell >= D.m * D.n) return;
    const uint64_t i = cell / D.n, j = cell % D.n;
    int64_t sum = 0;
    for (uint64_t p = 0; p < D.k; ++p) {
        const int8_t w = TRANS ? coded_at(W, j, p) : coded_at(W, p, j);
        sum += (int64_t)D.a[(int64_t)i * D.ars + (int64_t)p * D.acs] * w;
    }
    linear_finish<OB, false>(D.c + ((int64_t)i * D.crs + (int64_t)j * D.ccs) * OB, sum, D.alpha, D.beta,
                             D.mode);
}

template <bool TRANS>
static void launch_direct(const CodedArgs &W, const DirectArgs &D, int ob, dim3 grid, hipStream_t s) {
    switch (ob) {
    case 1: hipLaunchKernelGGL((coded_direct_kernel<TRANS, 1>), grid, dim3(256), 0, s, W, D); break;
    case 2: hipLaunchKernelGGL((coded_direct_kernel<TRANS, 2>), grid, dim3(256), 0, s, W, D); break;
    case 4: hipLaunchKernelGGL((coded_direct_kernel<TRANS, 4>), grid, dim3(256), 0, s, W, D); break;
    case 8: hipLaunchKernelGGL((coded_direct_kernel<TRANS, 8>), grid, dim3(256), 0, s, W, D); break;
    default: hipLaunchKernelGGL((coded_direct_kernel<TRANS, 16>), grid, dim3(256), 0, s, W, D); break;
    }
}

static uint64_t round_up(uint64_t x, uint64_t a) { return (x + a - 1) / a * a; }

// The decoded operand's bytes in the scratch (k x round_up(n, 16), 256-byte
// aligned end).
static uint64_t decoded_bytes(uint64_t k, uint64_t n) { return round_up(k * round_up(n, 16), 256); }

// What the decode needs of a codec (the constructors' own bound checks are
// the caller's): a known tier, P dividing 8, the tier's code widths, a table
// of N (x BLK) entries.
static int codec_dev(const uor_codec *c, CodecDev *d) {
    if (!c) return UOR_INVALID_ARGUMENT;
    if (c->tier < UOR_TIER_IDENTITY || c->tier > UOR_TIER_TERNARY) return UOR_INVALID_ARGUMENT;
    if (!(c->packed == 0 || c->packed == 1 || c->packed == 2 || c->packed == 4 || c->packed == 8))
        return UOR_INVALID_ARGUMENT;
    if (c->tier == UOR_TIER_IDENTITY && (c->packed || c->code_bits != 8)) return UOR_INVALID_ARGUMENT;
    if (c->tier == UOR_TIER_GRID && c->code_bits != 16) return UOR_INVALID_ARGUMENT;
    if (c->code_bits != 8 && c->code_bits != 16) return UOR_INVALID_ARGUMENT;
    if (c->has_zero && (c->zero < -128 || c->zero > 127)) return UOR_INVALID_ARGUMENT;
    if (c->tier == UOR_TIER_GRID || c->tier == UOR_TIER_BOOK) {
        if (c->entries == 0) return UOR_INVALID_ARGUMENT;
        uint64_t need = c->entries;
        if (c->tier == UOR_TIER_BOOK && __builtin_mul_overflow(c->entries, c->block, &need))
            return UOR_INVALID_ARGUMENT;
        if (!c->table || c->table_len < need) return UOR_SHORT_BUFFER;
    }
    // The cursor keeps positions inside a block in 32 bits.
    if (c->tier >= UOR_TIER_BOOK && c->block >= (1ull << 31)) return UOR_INVALID_ARGUMENT;
    d->tier = c->tier;
    d->code_bits = c->code_bits;
    d->packed = c->packed;
    d->has_zero = c->has_zero != 0;
    d->zero = (int)c->zero;
    d->sub_bits = c->packed ? 8u / (uint32_t)c->packed : 8u;
    d->sub_mask = d->sub_bits >= 8 ? 0xFFu : ((1u << d->sub_bits) - 1u);
    d->entries = c->entries;
    d->block = c->block;
    d->ib = (c->tier == UOR_TIER_IDENTITY || c->tier == UOR_TIER_GRID) ? 1 : c->block;
    if (__builtin_mul_overflow(d->ib, (uint64_t)(c->packed ? c->packed : 1), &d->mb)) return UOR_SHORT_BUFFER;
    d->table = c->table;
    return UOR_OK;
}

}  // namespace uor

using namespace uor;

extern "C" uint64_t uor_gfx950_suggested_scratch_coded(uint64_t m, uint64_t k, uint64_t n) {
    if (m == 0 || n == 0 || k == 0) return 0;
    return 256 + decoded_bytes(k, n) + uor_gfx950_suggested_scratch_i8(m, k, n);
}

static int gemm_coded_impl(const uor_view *a, const uor_codec *codec, const void *codes, uint64_t codes_len,
                           uint64_t w_rows, uint64_t w_cols, int transposed, const uor_view *c, int out_type,
                           int64_t alpha, int64_t beta, int encode, void *scratch, uint64_t scratch_bytes,
                           void *stream, uor_route *route, bool collapse);

extern "C" int uor_gfx950_gemm_coded(const uor_view *a, const uor_codec *codec, const void *codes,
                                     uint64_t codes_len, uint64_t w_rows, uint64_t w_cols, int transposed,
                                     const uor_view *c, int out_type, int64_t alpha, int64_t beta, int encode,
                                     void *scratch, uint64_t scratch_bytes, void *stream, uor_route *route) {
    return gemm_coded_impl(a, codec, codes, codes_len, w_rows, w_cols, transposed, c, out_type, alpha, beta, encode,
                           scratch, scratch_bytes, stream, route, false);
}

extern "C" int uor_gfx950_gemm_coded_collapsed(const uor_view *a, const uor_codec *codec, const void *codes,
                                               uint64_t codes_len, uint64_t w_rows, uint64_t w_cols, int transposed,
                                               const uor_view *c, int out_type, int64_t alpha, int64_t beta,
                                               int encode, void *scratch, uint64_t scratch_bytes, void *stream,
                                               uor_route *route) {
    return gemm_coded_impl(a, codec, codes, codes_len, w_rows, w_cols, transposed, c, out_type, alpha, beta, encode,
                           scratch, scratch_bytes, stream, route, true);
}

extern "C" uint64_t uor_gfx950_suggested_scratch_coded_collapse(uint64_t m, uint64_t k, uint64_t n) {
    if (m == 0 || n == 0 || k == 0 || m > 0xFFFFFFFEull) return 0;
    return collapse_layout(m, k, n, 16).rest + uor_gfx950_suggested_scratch_coded(m, k, n) + 256;
}

static int gemm_coded_impl(const uor_view *a, const uor_codec *codec, const void *codes, uint64_t codes_len,
                           uint64_t w_rows, uint64_t w_cols, int transposed, const uor_view *c, int out_type,
                           int64_t alpha, int64_t beta, int encode, void *scratch, uint64_t scratch_bytes,
                           void *stream, uor_route *route, bool collapse) {
    route_set(route, UOR_ROUTE_NONE);
    if (!valid_out_type(out_type) || !valid_encode(encode)) return UOR_INVALID_ARGUMENT;
    CodedArgs W{};
    int st = codec_dev(codec, &W.cd);
    if (st) return st;
    // CodedMatrix::new for a fixed-width tier (matrix.rs:36-55).
    if (W.cd.mb == 0 || w_cols % W.cd.mb != 0) return UOR_SHORT_BUFFER;
    W.per_row = w_cols / W.cd.mb;
    uint64_t ncodes;
    if (__builtin_mul_overflow(w_rows, W.per_row, &ncodes) || ncodes != codes_len) return UOR_SHORT_BUFFER;
    if (ncodes != 0 && codes == nullptr) return UOR_SHORT_BUFFER;
    W.codes = (const uint8_t *)codes;
    W.cb = codec->packed ? 1 : codec->code_bits / 8;
    W.rows = w_rows;
    W.cols = w_cols;
    // MatView::new for A and C, then TabulatedTriple::new (tabulated.rs:
    // 624-650) or CodedTriple::new (coded.rs:50-78).
    Placed A, C;
    if ((st = place(a, 1, &A))) return st;
    if ((st = place(c, out_type, &C))) return st;
    const uint64_t k = transposed ? w_cols : w_rows, n = transposed ? w_rows : w_cols;
    if (A.cols != k || C.rows != A.rows || C.cols != n) return UOR_NONCONFORMANT;
    if (self_aliases(C.rows, C.cols, C.rs, C.cs)) return UOR_OUTPUT_ALIASES_ITSELF;
    if (C.rows == 0 || C.cols == 0) return UOR_OK;
    if (W.cb == 2 && ((uintptr_t)codes & 1)) return UOR_INVALID_ARGUMENT;
    if ((uintptr_t)C.base % (uint64_t)(out_type > 8 ? 8 : out_type)) return UOR_INVALID_ARGUMENT;
    const uint64_t m = A.rows;
    hipStream_t s = (hipStream_t)stream;

    // The row collapse (tabulated.rs:2627-2660, collapse.rs): with beta = 0
    // and room for the pass, equal rows of A share one product row.
    if (collapse && beta == 0 && k > 0 && m > 1 && m <= 0xFFFFFFFEull && (m + 3) / 4 <= 0x7FFFFFFFull &&
        ((uintptr_t)C.base % (uintptr_t)(out_type < 8 ? out_type : 8)) == 0) {
        const CollapseLayout CL = collapse_layout(m, k, n, out_type);
        const uintptr_t p0 = (uintptr_t)scratch, p1 = (p0 + 255) & ~(uintptr_t)255;
        const uint64_t have = scratch && scratch_bytes > (p1 - p0) ? scratch_bytes - (p1 - p0) : 0;
        if (have >= CL.rest) {
            char *sc = (char *)p1;
            const RowsArgs R{(const int8_t *)A.base, A.rs, A.cs, m, k};
            uint32_t d = 0;
            if ((st = collapse_pass(R, sc, CL, s, &d))) return st;
            if (d < m) {
                const uor_view cav{sc + CL.compact, (uint64_t)d * CL.ldc, d, k, (int64_t)CL.ldc, 1};
                const uor_view pv{sc + CL.prod, (uint64_t)d * n, d, n, (int64_t)n, 1};
                uor_route r{};
                st = gemm_coded_impl(&cav, codec, codes, codes_len, w_rows, w_cols, transposed, &pv, out_type, alpha,
                                     0, encode, sc + CL.rest, have - CL.rest, stream, &r, false);
                if (st) return st;
                if ((st = collapse_expand(sc + CL.prod, (const uint32_t *)(sc + CL.index), m, n, C.base, C.rs, C.cs,
                                          out_type, s)))
                    return st;
                if (route) {
                    *route = r;
                    route->kind = UOR_ROUTE_COLLAPSED;
                    route->moduli = (int)d;  // distinct rows
                    route->launches = r.launches + 6;
                    route->scratch_used = CL.rest + r.scratch_used;
                }
                return UOR_OK;
            }
            // Pairwise distinct rows: the routes below, having paid the pass.
        }
    }

    const uint64_t wbytes = k ? decoded_bytes(k, n) : 0;
    // The decoded operand takes 16-byte stores: the offer from its first
    // aligned byte.
    uint64_t have_dense;
    char *const dscr = offer_align(scratch, scratch_bytes, &have_dense);
    const bool dense = k > 0 && dscr && have_dense >= wbytes + uor_gfx950_suggested_scratch_i8(m, k, n) &&
                       (n + 127) / 128 <= 0x7FFFFFFFull && (k + 127) / 128 <= 65535ull &&
                       (k * (round_up(n, 16) / 16) + 255) / 256 <= 0x7FFFFFFFull;
    if (transposed && k > 0 && m <= 8 && k <= GEMV_MAX_K && (n + 3) / 4 <= 0x7FFFFFFFull) {
        const bool a_vec = A.cs == 1 && A.rs > 0 && (A.rs % 16) == 0 && ((uintptr_t)A.base & 15) == 0;
        GemvArgs G{(const int8_t *)A.base, A.rs, A.cs, a_vec ? 1 : 0, C.base, C.rs, C.cs, m, k, n,
                   alpha, beta, encode, out_type};
        // Whole 16-byte code windows per row, a window a multiple of 16
        // elements, 16-byte aligned codes and A rows.
        const uint64_t row_bytes = W.per_row * (uint64_t)W.cb;
        const bool win = a_vec && row_bytes % 16 == 0 && ((uintptr_t)codes & 15) == 0 &&
                         ((16 / (uint64_t)W.cb) * W.cd.mb) % 16 == 0;
        // The table variant: one-byte codes of 4 or 8 elements, m <= 4; of 4
        // elements, m <= 8.
        const bool lut = win && W.cb == 1 &&
                         (((W.cd.mb == 4 || W.cd.mb == 8) && m <= 4) || (W.cd.mb == 4 && m <= 8)) &&
                         (n + 15) / 16 <= 0x7FFFFFFFull;
        // Past four rows the per-element decode costs more than decoding
        // into the scratch (Ternary<4,u8> at the config weights, m = 5: 244
        // against about 180 us): with the offer, the dense route below.
        const bool gemv = m <= 4 || lut || !dense;
        if (gemv) {
        if (route) {
            route->kind = UOR_ROUTE_CODED_GEMV;
            route->tile_m = (int)m;
            route->tile_n = lut ? 4 : 1;
            route->tile_k = win ? (int)((16 / W.cb) * W.cd.mb) : (int)(((k + 63) / 64 + 15) / 16 * 16);
            route->split_k = 64;
            route->launches = 1;
            route->operand_modes = lut ? 3 : win ? 2 : (a_vec ? 1 : 0);
        }
        if (lut) {
            if (m <= 1) launch_gemv_lut<1>(W, G, s);
            else if (m <= 2) launch_gemv_lut<2>(W, G, s);
            else if (m <= 4) launch_gemv_lut<4>(W, G, s);
            else launch_gemv_lut<8>(W, G, s);
        } else {
            launch_gemv(W, G, win, s);
        }
        UOR_HIP(hipGetLastError());
        return UOR_OK;
        }
    }
    if (dense) {
        const uint64_t ldw = round_up(n, 16);
        int8_t *wt = (int8_t *)dscr;
        if (transposed) {
            const dim3 grid((unsigned)((n + 127) / 128), (unsigned)((k + 127) / 128));
            // One-byte codes of 4 or 8 elements in whole 16-byte row runs,
            // 16-byte aligned: the table variant.
            const bool lut = W.cb == 1 && (W.cd.mb == 4 || W.cd.mb == 8) && W.per_row % 16 == 0 &&
                             ((uintptr_t)codes & 15) == 0;
            if (lut && W.cd.mb == 4)
                hipLaunchKernelGGL(coded_decode_t_lut_kernel<1>, grid, dim3(256), 0, s, W, k, n, wt, ldw);
            else if (lut)
                hipLaunchKernelGGL(coded_decode_t_lut_kernel<2>, grid, dim3(256), 0, s, W, k, n, wt, ldw);
            else
                hipLaunchKernelGGL(coded_decode_t_kernel, grid, dim3(256), 0, s, W, k, n, wt, ldw);
        } else {
            const uint64_t blocks = (k * (ldw / 16) + 255) / 256;
            hipLaunchKernelGGL(coded_decode_kernel, dim3((unsigned)blocks), dim3(256), 0, s, W, k, n, wt, ldw);
        }
        UOR_HIP(hipGetLastError());
        const uor_view bv{wt, k * ldw, k, n, (int64_t)ldw, 1};
        const int st2 = uor_gfx950_gemm_i8(a, &bv, c, out_type, alpha, beta, encode, dscr + wbytes,
                                           have_dense - wbytes, stream, route);
        if (route && st2 == UOR_OK) {
            route->kind = UOR_ROUTE_CODED_DENSE;
            route->launches += 1;
            route->scratch_used += wbytes;
        }
        return st2;
    }
    {
        const uint64_t cells = m * n, blocks = (cells + 255) / 256;
        if (cells / n != m || blocks > 0x7FFFFFFFull) return UOR_INVALID_ARGUMENT;
        DirectArgs D{(const int8_t *)A.base, A.rs, A.cs, C.base, C.rs, C.cs, m, k, n, alpha, beta, encode};
        if (route) {
            route->kind = k ? UOR_ROUTE_CODED_DIRECT : UOR_ROUTE_EPILOGUE_ONLY;
            route->tile_m = route->tile_n = route->tile_k = 1;
            route->split_k = 1;
            route->launches = 1;
        }
        if (transposed) launch_direct<true>(W, D, out_type, dim3((unsigned)blocks), s);
        else launch_direct<false>(W, D, out_type, dim3((unsigned)blocks), s);
        UOR_HIP(hipGetLastError());
    }
    return UOR_OK;
}

// ------------------------------------------------------------ Arena tier --
//
// Arena<E, N, K> over f32 / f64 (codecs.rs:894-960): a one-element block
// whose decode is table[code % N], the table an artifact's distinct bit
// patterns.  The coded operand is decoded once into the scratch as a k x n
// matrix of E, then the exact float route multiplies it (the decode carries
// bit patterns, so the product is the float product of the dense spelling).

template <typename T>
__global__ void __launch_bounds__(256) arena_decode_kernel(const T *table, uint64_t entries, const uint8_t *codes,
                                                           int cb, uint64_t w_cols, int trans, uint64_t k,
                                                           uint64_t n, T *out) {
    const uint64_t j = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (j >= n) return;
    for (uint64_t p = blockIdx.y; p < k; p += gridDim.y) {
        const uint64_t at = trans ? j * w_cols + p : p * w_cols + j;
        const uint32_t code = cb == 1 ? (uint32_t)codes[at] : (uint32_t)((const uint16_t *)codes)[at];
        out[p * n + j] = table[code % entries];
    }
}

extern "C" int uor_gfx950_gemm_float(int is_f64, const uor_view *a, const uor_view *b, const uor_view *c,
                                     int64_t alpha, int64_t beta, int encode, void *scratch, uint64_t scratch_bytes,
                                     void *stream, uor_route *route);
extern "C" uint64_t uor_gfx950_suggested_scratch_float(int is_f64, uint64_t m, uint64_t k, uint64_t n);

extern "C" uint64_t uor_gfx950_suggested_scratch_coded_float(int is_f64, uint64_t m, uint64_t k, uint64_t n) {
    if (m == 0 || n == 0 || k == 0) return 0;
    return round_up(k * n * (is_f64 ? 8 : 4), 256) + uor_gfx950_suggested_scratch_float(is_f64, m, k, n);
}

extern "C" int uor_gfx950_gemm_coded_float(int is_f64, const uor_view *a, const void *table, uint64_t entries,
                                           int code_bits, const void *codes, uint64_t codes_len, uint64_t w_rows,
                                           uint64_t w_cols, int transposed, const uor_view *c, int64_t alpha,
                                           int64_t beta, int encode, void *scratch, uint64_t scratch_bytes,
                                           void *stream, uor_route *route) {
    route_set(route, UOR_ROUTE_NONE);
    if (!(is_f64 == 0 || is_f64 == 1) || !(code_bits == 8 || code_bits == 16) || !valid_encode(encode))
        return UOR_INVALID_ARGUMENT;
    if (entries == 0 || !table) return UOR_INVALID_ARGUMENT;
    const int eb = is_f64 ? 8 : 4;
    // CodedMatrix::new at MAX_BLOCK 1 (matrix.rs:36-55).
    uint64_t ncodes;
    if (__builtin_mul_overflow(w_rows, w_cols, &ncodes) || ncodes != codes_len) return UOR_SHORT_BUFFER;
    if (ncodes != 0 && codes == nullptr) return UOR_SHORT_BUFFER;
    Placed A, C;
    int st;
    if ((st = place(a, eb, &A))) return st;
    if ((st = place(c, eb, &C))) return st;
    const uint64_t k = transposed ? w_cols : w_rows, n = transposed ? w_rows : w_cols;
    if (A.cols != k || C.rows != A.rows || C.cols != n) return UOR_NONCONFORMANT;
    if (self_aliases(C.rows, C.cols, C.rs, C.cs)) return UOR_OUTPUT_ALIASES_ITSELF;
    if (C.rows == 0 || C.cols == 0) return UOR_OK;
    if ((((uintptr_t)table) & (uintptr_t)(eb - 1)) || (code_bits == 16 && ((uintptr_t)codes & 1)))
        return UOR_INVALID_ARGUMENT;
    // The decoded operand lives in the offer: there is no decode-free float
    // route, so an offer below its size is refused before any launch.
    const uint64_t wbytes = k ? round_up(k * n * (uint64_t)eb, 256) : 0;
    const uintptr_t p0 = (uintptr_t)scratch, p1 = (p0 + 255) & ~(uintptr_t)255;
    const uint64_t have = scratch && scratch_bytes > (p1 - p0) ? scratch_bytes - (p1 - p0) : 0;
    if (k > 0 && have < wbytes) return UOR_INVALID_ARGUMENT;
    hipStream_t s = (hipStream_t)stream;
    char *sc = (char *)p1;
    if (k > 0) {
        const dim3 grid((unsigned)((n + 255) / 256), (unsigned)(k < 65535 ? k : 65535));
        if ((n + 255) / 256 > 0x7FFFFFFFull) return UOR_INVALID_ARGUMENT;
        if (is_f64)
            hipLaunchKernelGGL(arena_decode_kernel<double>, grid, dim3(256), 0, s, (const double *)table, entries,
                               (const uint8_t *)codes, code_bits / 8, w_cols, transposed, k, n, (double *)sc);
        else
            hipLaunchKernelGGL(arena_decode_kernel<float>, grid, dim3(256), 0, s, (const float *)table, entries,
                               (const uint8_t *)codes, code_bits / 8, w_cols, transposed, k, n, (float *)sc);
        UOR_HIP(hipGetLastError());
    }
    const uor_view bv{k ? (void *)sc : (void *)sc, k * n, k, n, (int64_t)n, 1};
    st = uor_gfx950_gemm_float(is_f64, a, &bv, c, alpha, beta, encode, sc + wbytes, have - wbytes, stream, route);
    if (route && st == UOR_OK) route->launches += k > 0 ? 1 : 0;
    return st;
}
