// The collapse traversal on gfx950: one product row per distinct row of A.
//
// Replaces gemm_collapsed (crates/uor-matmul-gemm/src/collapse.rs:169-220)
// at E = i8: an epilogue that reads C (beta != 0), an empty product, k = 0, an
// A whose rows are pairwise distinct, or an offer too small for the buffers
// below runs the plain route; otherwise each distinct row is multiplied once
// and its output row copied to every row that equals it.  An exact sum is a
// function of the row's values, so the bytes are the plain route's (CD-12).
// Columns collapse through the transposed triple, (A B)^T = B^T A^T, with
// the same passes (collapse.rs module note "Columns").
//
// The distinct rows are found on the device:
//   row_hash_kernel    one wave per row: a position-keyed 64-bit hash
//   table_insert       an open-addressed table of 2^ceil(log2 2m) slots (at
//                      most half full, so every probe ends), the least row
//                      index per hash by atomicMin
//   class_kernel       one wave per row: its table entry, checked byte for
//                      byte (a hash collision leaves the row its own class);
//                      a class's first row takes the next compacted number
//                      and copies itself into the compacted A
//   index_kernel       every row's compacted number
// then the host reads back the count d (one 4-byte copy), runs the dense
// route on the d x k compacted A into a d x n buffer, and expand_kernel
// copies row index[i] of that buffer to row i of C.

#include "common.hpp"
#include "collapse.hpp"

extern "C" int uor_gfx950_gemm_i8(const uor_view *a, const uor_view *b, const uor_view *c, int out_type,
                                  int64_t alpha, int64_t beta, int encode, void *scratch,
                                  uint64_t scratch_bytes, void *stream, uor_route *route);
extern "C" uint64_t uor_gfx950_suggested_scratch_i8(uint64_t m, uint64_t k, uint64_t n);

namespace uor {



__device__ inline uint64_t mix64(uint64_t z) {
    // splitmix64's finaliser (Steele, Lea, Flood 2014).
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Eight bytes of row i from column q (zeros past k).
__device__ inline uint64_t row_word(const RowsArgs &R, uint64_t i, uint64_t q) {
    const int8_t *p = R.a + (int64_t)i * R.rs;
    uint64_t w = 0;
    if (R.cs == 1 && q + 8 <= R.k) {
#pragma unroll
        for (int b = 0; b < 8; ++b) w |= (uint64_t)(uint8_t)p[q + b] << (8 * b);
        return w;
    }
    for (int b = 0; b < 8 && q + b < R.k; ++b) w |= (uint64_t)(uint8_t)p[(int64_t)(q + b) * R.cs] << (8 * b);
    return w;
}

// Lines of contiguous, 16-byte aligned bytes (every line start a multiple of
// 16): read 16 bytes per lane and step.
__device__ inline bool rows16(const RowsArgs &R) {
    return R.cs == 1 && ((uintptr_t)R.a & 15) == 0 && (R.rs & 15) == 0;
}

// Chunk t (16 bytes) of a whole-chunk run of row i (16t + 16 <= k).
__device__ inline uint4 row_chunk(const RowsArgs &R, uint64_t i, uint64_t t) {
    return *(const uint4 *)(R.a + (int64_t)i * R.rs + (int64_t)(16 * t));
}

// Words 2t and 2t + 1 of the last, partial chunk t of row i (16t < k <
// 16t + 16; the second zero when 16t + 8 >= k, where it is not a word of the
// row).
__device__ inline void row_tail16(const RowsArgs &R, uint64_t i, uint64_t t, uint64_t &w0, uint64_t &w1) {
    w0 = row_word(R, i, 16 * t);
    w1 = 16 * t + 8 < R.k ? row_word(R, i, 16 * t + 8) : 0;
}

__device__ inline uint64_t word_key(uint64_t w) { return w * 0x9E3779B97F4A7C15ull; }

// A sum of keyed word mixes: independent of how the words are split among
// lanes.  Zero is the table's empty key, so a zero hash becomes one.
__global__ void __launch_bounds__(256) row_hash_kernel(RowsArgs R, uint64_t *hash) {
    const uint64_t i = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (i >= R.m) return;
    uint64_t h = 0;
    if (rows16(R)) {
        // The whole chunks, U per lane and step with their loads issued
        // together; then the partial chunk, if any, by one lane.
        constexpr int U = 4;
        const uint64_t nfull = R.k / 16;
        for (uint64_t t0 = lane; t0 < nfull; t0 += 64 * U) {
            uint4 x[U];
#pragma unroll
            for (int u = 0; u < U; ++u) x[u] = row_chunk(R, i, min(t0 + 64 * u, nfull - 1));  // (clamped: no branch)
#pragma unroll
            for (int u = 0; u < U; ++u) {
                // (a mask, not a branch: the compiler would sink the loads
                // into one and wait for each)
                const uint64_t t = t0 + 64 * u, keep = (uint64_t)0 - (uint64_t)(t < nfull);
                h += (mix64(((uint64_t)x[u].x | (uint64_t)x[u].y << 32) ^ word_key(2 * t)) +
                      mix64(((uint64_t)x[u].z | (uint64_t)x[u].w << 32) ^ word_key(2 * t + 1))) &
                     keep;
            }
        }
        if (R.k % 16 && (uint64_t)lane == nfull % 64) {
            uint64_t w0, w1;
            row_tail16(R, i, nfull, w0, w1);
            h += mix64(w0 ^ word_key(2 * nfull));
            if (16 * nfull + 8 < R.k) h += mix64(w1 ^ word_key(2 * nfull + 1));
        }
    } else {
        for (uint64_t w = lane; 8 * w < R.k; w += 64) h += mix64(row_word(R, i, 8 * w) ^ (w * 0x9E3779B97F4A7C15ull));
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) h += __shfl_xor(h, o, 64);
    if (lane == 0) hash[i] = h ? h : 1;
}

__global__ void __launch_bounds__(256) table_clear_kernel(unsigned long long *key, uint32_t *row, uint64_t slots,
                                                          uint32_t *counter) {
    const uint64_t s = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (s < slots) {
        key[s] = 0;
        row[s] = 0xFFFFFFFFu;
    }
    if (s == 0) *counter = 0;
}

// One thread per row: claim or find the slot of its hash, keep the least row.
__global__ void __launch_bounds__(256) table_insert_kernel(const uint64_t *hash, uint64_t m, unsigned long long *key,
                                                           uint32_t *row, uint64_t mask) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= m) return;
    const unsigned long long h = hash[i];
    uint64_t s = h & mask;
    for (uint64_t probes = 0; probes <= mask; ++probes) {
        const unsigned long long old = atomicCAS(&key[s], 0ull, h);
        if (old == 0ull || old == h) {
            atomicMin(&row[s], (uint32_t)i);
            return;
        }
        s = (s + 1) & mask;
    }
}

// One wave per row: its class representative (the least row with its hash,
// if equal byte for byte; else itself); a representative takes a number.
__global__ void __launch_bounds__(256) class_kernel(RowsArgs R, const uint64_t *hash,
                                                    const unsigned long long *key, const uint32_t *row,
                                                    uint64_t mask, uint32_t *rep, uint32_t *id,
                                                    uint32_t *counter, int8_t *compact, uint64_t ldc) {
    const uint64_t i = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (i >= R.m) return;
    const unsigned long long h = hash[i];
    uint64_t s = h & mask;
    for (uint64_t probes = 0; probes <= mask && key[s] != h; ++probes) s = (s + 1) & mask;
    uint64_t r = key[s] == h ? row[s] : i;
    const bool v16 = rows16(R);
    if (r != i) {
        bool same = true;
        if (v16) {
            constexpr int U = 4;  // as row_hash_kernel
            const uint64_t nfull = R.k / 16;
            for (uint64_t t0 = lane; t0 < nfull; t0 += 64 * U) {
                uint4 x[U], y[U];
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const uint64_t t = min(t0 + 64 * u, nfull - 1);  // (clamped: no branch)
                    x[u] = row_chunk(R, i, t);
                    y[u] = row_chunk(R, r, t);
                }
#pragma unroll
                for (int u = 0; u < U; ++u)
                    same &= x[u].x == y[u].x && x[u].y == y[u].y && x[u].z == y[u].z && x[u].w == y[u].w;
            }
            if (R.k % 16 && (uint64_t)lane == nfull % 64) {
                uint64_t a0, a1, b0, b1;
                row_tail16(R, i, nfull, a0, a1);
                row_tail16(R, r, nfull, b0, b1);
                same &= a0 == b0 && a1 == b1;
            }
        } else {
            for (uint64_t w = lane; 8 * w < R.k; w += 64) same &= row_word(R, i, 8 * w) == row_word(R, r, 8 * w);
        }
        if (__any(!same)) r = i;  // a collision: its own class
    }
    uint32_t num = 0;
    if (r == i) {
        if (lane == 0) num = atomicAdd(counter, 1u);
        num = __shfl(num, 0, 64);
        int8_t *dst = compact + num * ldc;
        if (v16 && ((uintptr_t)compact & 15) == 0 && (ldc & 15) == 0) {
            // 16 bytes per lane; the tail past the last whole chunk byte by byte
            const uint64_t whole = R.k / 16;
            const int8_t *src = R.a + (int64_t)i * R.rs;
            for (uint64_t t = lane; t < whole; t += 64) ((uint4 *)dst)[t] = ((const uint4 *)src)[t];
            for (uint64_t q = 16 * whole + lane; q < R.k; q += 64) dst[q] = src[q];
        } else {
            for (uint64_t q = lane; q < R.k; q += 64) dst[q] = R.a[(int64_t)i * R.rs + (int64_t)q * R.cs];
        }
    }
    if (lane == 0) {
        rep[i] = (uint32_t)r;
        if (r == i) id[i] = num;
    }
}

__global__ void __launch_bounds__(256) index_kernel(uint64_t m, const uint32_t *rep, const uint32_t *id,
                                                    uint32_t *index) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < m) index[i] = id[rep[i]];
}

// C[i, j] := P[index[i], j], element by element (ob bytes); rows i step by
// gridDim.y.
__global__ void __launch_bounds__(256) expand_kernel(const char *P, uint64_t n, const uint32_t *index, uint64_t m,
                                                     char *c, int64_t crs, int64_t ccs, int ob) {
    const uint64_t j = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (j >= n) return;
    for (uint64_t i = blockIdx.y; i < m; i += gridDim.y) {
        const char *src = P + ((uint64_t)index[i] * n + j) * ob;
        char *dst = c + ((int64_t)i * crs + (int64_t)j * ccs) * ob;
        switch (ob) {
        case 1: *(int8_t *)dst = *(const int8_t *)src; break;
        case 2: *(int16_t *)dst = *(const int16_t *)src; break;
        case 4: *(int32_t *)dst = *(const int32_t *)src; break;
        case 8: *(int64_t *)dst = *(const int64_t *)src; break;
        default:
            ((int64_t *)dst)[0] = ((const int64_t *)src)[0];
            ((int64_t *)dst)[1] = ((const int64_t *)src)[1];
        }
    }
}

// The same copy for row-contiguous C with 16-byte aligned rows: one 16-byte
// chunk per thread.
__global__ void __launch_bounds__(256) expand16_kernel(const char *P, uint64_t row_bytes, const uint32_t *index,
                                                       uint64_t m, char *c, int64_t crs_bytes) {
    const uint64_t q = ((uint64_t)blockIdx.x * 256 + threadIdx.x) * 16;
    if (q >= row_bytes) return;
    for (uint64_t i = blockIdx.y; i < m; i += gridDim.y)
        *(uint4 *)(c + (int64_t)i * crs_bytes + (int64_t)q) = *(const uint4 *)(P + (uint64_t)index[i] * row_bytes + q);
}



static uint64_t up256(uint64_t x) { return (x + 255) & ~(uint64_t)255; }

static uint64_t next_pow2(uint64_t x) {
    uint64_t p = 1;
    while (p < x) p <<= 1;
    return p;
}

CollapseLayout collapse_layout(uint64_t m, uint64_t k, uint64_t n, int ob) {
    CollapseLayout L{};
    L.slots = next_pow2(2 * m);
    L.ldc = (k + 15) / 16 * 16;
    L.hash = 0;
    L.key = L.hash + up256(m * 8);
    L.row = L.key + up256(L.slots * 8);
    L.rep = L.row + up256(L.slots * 4);
    L.id = L.rep + up256(m * 4);
    L.index = L.id + up256(m * 4);
    L.counter = L.index + up256(m * 4);
    L.compact = L.counter + 256;
    L.prod = L.compact + up256(m * L.ldc);
    L.rest = L.prod + up256(m * n * (uint64_t)ob);
    return L;
}

// The pass over the m lines of R: their classes, the compacted distinct
// lines (d x ldc at `compact`) and every line's class number (`index`),
// then the count d read back to the host.  Buffers in `sc` by `L`.
int collapse_pass(const RowsArgs &R, char *sc, const CollapseLayout &L, hipStream_t s, uint32_t *d_out) {
    const uint64_t m = R.m;
    uint64_t *hash = (uint64_t *)(sc + L.hash);
    unsigned long long *key = (unsigned long long *)(sc + L.key);
    uint32_t *row = (uint32_t *)(sc + L.row), *rep = (uint32_t *)(sc + L.rep), *id = (uint32_t *)(sc + L.id);
    uint32_t *index = (uint32_t *)(sc + L.index), *counter = (uint32_t *)(sc + L.counter);
    int8_t *compact = (int8_t *)(sc + L.compact);
    const unsigned wgrid = (unsigned)((m + 3) / 4);
    hipLaunchKernelGGL(row_hash_kernel, dim3(wgrid), dim3(256), 0, s, R, hash);
    hipLaunchKernelGGL(table_clear_kernel, dim3((unsigned)((L.slots + 255) / 256)), dim3(256), 0, s, key, row,
                       L.slots, counter);
    hipLaunchKernelGGL(table_insert_kernel, dim3((unsigned)((m + 255) / 256)), dim3(256), 0, s, hash, m, key, row,
                       L.slots - 1);
    hipLaunchKernelGGL(class_kernel, dim3(wgrid), dim3(256), 0, s, R, hash, key, row, L.slots - 1, rep, id, counter,
                       compact, L.ldc);
    hipLaunchKernelGGL(index_kernel, dim3((unsigned)((m + 255) / 256)), dim3(256), 0, s, m, rep, id, index);
    UOR_HIP(hipGetLastError());
    uint32_t d = 0;
    UOR_HIP(hipMemcpyAsync(&d, counter, 4, hipMemcpyDeviceToHost, s));
    UOR_HIP(hipStreamSynchronize(s));
    if (d == 0 || d > m) return UOR_HIP_ERROR;
    *d_out = d;
    return UOR_OK;
}

// C[i, j] := P[index[i], j] for the m x n output (ob-byte elements).
int collapse_expand(const char *P, const uint32_t *index, uint64_t m, uint64_t n, char *c, int64_t crs, int64_t ccs,
                    int ob, hipStream_t s) {
    const unsigned gy = (unsigned)(m < 65535 ? m : 65535);
    const uint64_t row_bytes = n * (uint64_t)ob;
    if (ccs == 1 && row_bytes % 16 == 0 && ((uintptr_t)c & 15) == 0 && ((crs * ob) % 16) == 0)
        hipLaunchKernelGGL(expand16_kernel, dim3((unsigned)((row_bytes / 16 + 255) / 256), gy), dim3(256), 0, s, P,
                           row_bytes, index, m, c, crs * (int64_t)ob);
    else
        hipLaunchKernelGGL(expand_kernel, dim3((unsigned)((n + 255) / 256), gy), dim3(256), 0, s, P, n, index, m, c,
                           crs, ccs, ob);
    UOR_HIP(hipGetLastError());
    return UOR_OK;
}

}  // namespace uor

using namespace uor;

extern "C" uint64_t uor_gfx950_suggested_scratch_collapse(uint64_t m, uint64_t k, uint64_t n) {
    if (m == 0 || n == 0 || k == 0 || m > 0xFFFFFFFEull) return 0;
    const CollapseLayout L = collapse_layout(m, k, n, 16);
    return L.rest + uor_gfx950_suggested_scratch_i8(m, k, n) + 256;
}

extern "C" int uor_gfx950_gemm_collapsed_i8(const uor_view *a, const uor_view *b, const uor_view *c, int out_type,
                                            int64_t alpha, int64_t beta, int encode, int columns, void *scratch,
                                            uint64_t scratch_bytes, void *stream, uor_route *route) {
    route_set(route, UOR_ROUTE_NONE);
    if (!(columns == 0 || columns == 1)) return UOR_INVALID_ARGUMENT;
    if (!valid_out_type(out_type) || !valid_encode(encode)) return UOR_INVALID_ARGUMENT;
    Placed A, B, C;
    int st = make_triple(a, 1, b, 1, c, out_type, &A, &B, &C);
    if (st) return st;
    const int ob = out_type;
    // The plain route: an epilogue that reads C, an empty product, k = 0, or
    // an offer without room for the pass.
    auto plain = [&]() {
        return uor_gfx950_gemm_i8(a, b, c, out_type, alpha, beta, encode, scratch, scratch_bytes, stream, route);
    };
    if (beta != 0 || C.rows == 0 || C.cols == 0 || A.cols == 0) return plain();
    if ((uintptr_t)C.base % (uintptr_t)(ob < 8 ? ob : 8)) return plain();
    // Columns: the transposed triple, B^T A^T = (A B)^T.
    RowsArgs R;
    uint64_t m, k = A.cols, n;
    uor_view bv;  // the right operand of the product over the collapsed side
    int64_t crs, ccs;
    if (!columns) {
        R = RowsArgs{(const int8_t *)A.base, A.rs, A.cs, A.rows, k};
        m = A.rows;
        n = B.cols;
        bv = *b;
        crs = C.rs;
        ccs = C.cs;
    } else {
        R = RowsArgs{(const int8_t *)B.base, B.cs, B.rs, B.cols, k};
        m = B.cols;
        n = A.rows;
        // A^T as the right operand: the caller's A view transposed (the same
        // buffer and reach, so it is placed at the same origin).
        bv = uor_view{a->data, a->len, a->cols, a->rows, a->cs, a->rs};
        crs = C.cs;
        ccs = C.rs;
    }
    if (m > 0xFFFFFFFEull || (m + 3) / 4 > 0x7FFFFFFFull || n > 0xFFFFFFFFull) return plain();
    const CollapseLayout L = collapse_layout(m, k, n, ob);
    const uintptr_t p0 = (uintptr_t)scratch, p1 = (p0 + 255) & ~(uintptr_t)255;
    const uint64_t have = scratch && scratch_bytes > (p1 - p0) ? scratch_bytes - (p1 - p0) : 0;
    if (have < L.rest) return plain();
    char *sc = (char *)p1;
    hipStream_t s = (hipStream_t)stream;
    uint32_t *index = (uint32_t *)(sc + L.index);
    int8_t *compact = (int8_t *)(sc + L.compact);
    char *prod = sc + L.prod;
    // The count of distinct rows decides the product's size.
    uint32_t d = 0;
    if ((st = collapse_pass(R, sc, L, s, &d))) return st;
    // Pairwise distinct lines: the plain route, having paid the pass.
    if (d == m) return plain();
    // The distinct lines' product, with the caller's scalars and encode, into
    // a d x n buffer, then copied out.
    const uor_view cav{compact, (uint64_t)d * L.ldc, d, k, (int64_t)L.ldc, 1};
    const uor_view pv{prod, (uint64_t)d * n, d, n, (int64_t)n, 1};
    uor_route r{};
    st = uor_gfx950_gemm_i8(&cav, &bv, &pv, out_type, alpha, 0, encode, sc + L.rest, have - L.rest, stream, &r);
    if (st) return st;
    if ((st = collapse_expand(prod, index, m, n, C.base, crs, ccs, ob, s))) return st;
    if (route) {
        *route = r;
        route->kind = UOR_ROUTE_COLLAPSED;
        route->moduli = (int)d;  // distinct lines
        route->launches = r.launches + 6;
        route->scratch_used = L.rest + r.scratch_used;
    }
    return UOR_OK;
}
