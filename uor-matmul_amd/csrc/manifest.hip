// The canonical weight-artifact manifest (host code): Manifest::
// write_canonical_json (crates/uor-matmul-codec/src/kappa.rs:321-360), the
// JSON whose kappa label is a coded artifact's identity.  Keys in
// lexicographic order, no whitespace, integers in decimal, digests checked as
// `sha256:` plus 64 lowercase hex digits (is_sha256, kappa.rs:392-400).  The
// label itself (address_into) needs the uor-addr-1 crate and is not built.

#include "common.hpp"

#include <cstring>

namespace {

// TierId::as_str (crates/uor-matmul-codec/src/tier.rs:265-278).
const char *tier_name(int tier) {
    switch (tier) {
    case UOR_TIER_IDENTITY: return "Identity";
    case UOR_TIER_GRID: return "Grid";
    case UOR_TIER_BOOK: return "Book";
    case UOR_TIER_SIGN: return "Sign";
    case UOR_TIER_TERNARY: return "Ternary";
    case UOR_TIER_PACKED: return "Packed";
    case UOR_TIER_OFFSET: return "Offset";
    case UOR_TIER_RUNS: return "Runs";
    case UOR_TIER_TRANSCODE: return "Transcode";
    case UOR_TIER_ARENA: return "Arena";
    default: return nullptr;
    }
}

bool is_sha256(const char *s) {
    if (!s || std::strncmp(s, "sha256:", 7) != 0) return false;
    const char *h = s + 7;
    for (int i = 0; i < 64; ++i) {
        const char c = h[i];
        if (!((c >= '0' && c <= '9') || (c >= 'a' && c <= 'f'))) return false;
    }
    return h[64] == '\0';
}

// Appends, counting what would be written even past the buffer.
struct Out {
    char *buf;
    uint64_t len, at;
    void push(const char *s) {
        for (; *s; ++s, ++at)
            if (at < len) buf[at] = *s;
    }
    void push_u128(unsigned __int128 v) {
        char d[40];
        int n = 0;
        do {
            d[n++] = (char)('0' + (int)(v % 10));
            v /= 10;
        } while (v);
        char s[41];
        for (int i = 0; i < n; ++i) s[i] = d[n - 1 - i];
        s[n] = '\0';
        push(s);
    }
};

}  // namespace

extern "C" int uor_gfx950_manifest_json(int tier, uint64_t bound_lo, uint64_t bound_hi, uint64_t rows, uint64_t cols,
                                        uint64_t block, const char *codebook_sha256, const char *codes_sha256,
                                        const char *spec, char *out, uint64_t out_len, uint64_t *written) {
    if (written) *written = 0;
    const char *name = tier_name(tier);
    if (!name || !spec) return UOR_INVALID_ARGUMENT;
    if (!is_sha256(codebook_sha256) || !is_sha256(codes_sha256)) return UOR_INVALID_ARGUMENT;
    Out w{out, out ? out_len : 0, 0};
    w.push("{\"block\":");
    w.push_u128(block);
    w.push(",\"bound\":");
    w.push_u128(((unsigned __int128)bound_hi << 64) | bound_lo);
    w.push(",\"codebook_sha256\":\"");
    w.push(codebook_sha256);
    w.push("\",\"codes_sha256\":\"");
    w.push(codes_sha256);
    w.push("\",\"cols\":");
    w.push_u128(cols);
    w.push(",\"rows\":");
    w.push_u128(rows);
    w.push(",\"spec\":\"");
    w.push(spec);
    w.push("\",\"tier\":\"");
    w.push(name);
    w.push("\"}");
    if (written) *written = w.at;
    return w.at > w.len ? UOR_SHORT_BUFFER : UOR_OK;
}
