"""Manifest::write_canonical_json through the C ABI (host code, no GPU),
against the reference's own known answers (kappa.rs CK-08 tests): the Book
and Arena spellings byte for byte, the short-buffer report, and malformed
digests."""
import uor_gfx950 as u

D0 = "sha256:" + "0" * 64
D1 = "sha256:" + "1" * 64


def test_book_spelling_is_byte_stable():
    st, text = u.manifest_json("book", 127, 4096, 4096, 8, D0, D1)
    assert st == 0
    assert text == ('{"block":8,"bound":127,'
                    '"codebook_sha256":"sha256:' + "0" * 64 + '",'
                    '"codes_sha256":"sha256:' + "1" * 64 + '",'
                    '"cols":4096,"rows":4096,"spec":"uor-matmul/1","tier":"Book"}')


def test_arena_spelling_with_the_largest_bound():
    st, text = u.manifest_json("arena", (1 << 128) - 1, 4096, 4096, 1, D0, D1)
    assert st == 0
    assert text == ('{"block":1,"bound":340282366920938463463374607431768211455,'
                    '"codebook_sha256":"sha256:' + "0" * 64 + '",'
                    '"codes_sha256":"sha256:' + "1" * 64 + '",'
                    '"cols":4096,"rows":4096,"spec":"uor-matmul/1","tier":"Arena"}')


def test_short_buffer_reports_the_need():
    st, needed = u.manifest_json("identity", 1, 1, 1, 1, D0, D1, out_len=8)
    assert u.STATUS[st] == "short_buffer" and needed > 8
    st, text = u.manifest_json("identity", 1, 1, 1, 1, D0, D1, out_len=needed)
    assert st == 0 and len(text) == needed


def test_malformed_digests_and_tiers():
    for bad in ("not-a-digest", "sha256:" + "A" * 64, "sha256:" + "0" * 63,
                "sha256:" + "0" * 65, "sha512:" + "0" * 64):
        assert u.STATUS[u.manifest_json("identity", 1, 1, 1, 1, bad, D1)[0]] == "invalid_argument"
        assert u.STATUS[u.manifest_json("identity", 1, 1, 1, 1, D0, bad)[0]] == "invalid_argument"
    assert u.STATUS[u.manifest_json(42, 1, 1, 1, 1, D0, D1)[0]] == "invalid_argument"
    st, text = u.manifest_json("packed", 8, 2, 16, 2, D0, D1)
    assert st == 0 and text.endswith('"tier":"Packed"}')
