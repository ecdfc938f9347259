// The collapse pass, shared by the dense and the coded products.
#pragma once

#include "common.hpp"

namespace uor {

// m lines of k int8 elements: element q of line i at a + i * rs + q * cs.
struct RowsArgs {
    const int8_t *a;  // element (0,0)
    int64_t rs, cs;
    uint64_t m, k;
};

// Byte offsets of the pass's buffers in the scratch, and the compacted
// lines' row stride.
struct CollapseLayout {
    uint64_t hash, key, row, rep, id, index, counter, compact, prod, rest;
    uint64_t slots, ldc;
};

// The layout for m lines of k elements and an m x n product of ob-byte
// elements beside them.
CollapseLayout collapse_layout(uint64_t m, uint64_t k, uint64_t n, int ob);

// The pass: classes, compacted lines, every line's class number; the count
// of classes read back to the host (a stream synchronisation).
int collapse_pass(const RowsArgs &R, char *sc, const CollapseLayout &L, hipStream_t s, uint32_t *d_out);

// C[i, j] := P[index[i], j], P row-major d x n.
int collapse_expand(const char *P, const uint32_t *index, uint64_t m, uint64_t n, char *c, int64_t crs, int64_t ccs,
                    int ob, hipStream_t s);

}  // namespace uor
