"""The Arena float symbol tier (Arena<f32, 256, u8>, codecs.rs:894-960)
pinned by the reference's CK-14 artifact (oracles/symbols, committed under
tests/golden/symbols_ck14 as data): the codebook is in canonical order
(unsigned bit-pattern order, distinct, CK-10), and table[code % N] over the
committed codes gives the committed dense weights -- byte for byte for
13 x 257, by digest for 1024 x 1024."""
import hashlib
import json

import numpy as np

from conftest import GOLDEN

D = GOLDEN / "symbols_ck14"


def sha(raw):
    return "sha256:" + hashlib.sha256(raw).hexdigest()


def test_fixture_digests_and_canonical_codebook():
    man = json.loads((D / "manifest.json").read_text())
    book = (D / "codebook.f32.bin").read_bytes()
    assert sha(book) == man["codebook_sha256"]
    bits = np.frombuffer(book, "<u4")
    assert len(bits) == man["codebook_symbols"]
    assert np.all(bits[1:] > bits[:-1]), "distinct, in unsigned bit-pattern order"
    for case in man["cases"]:
        raw = (D / f"{case['stem']}.codes.bin").read_bytes()
        assert sha(raw) == case["codes_sha256"]


def test_decode_is_the_dense_spelling():
    man = json.loads((D / "manifest.json").read_text())
    book = np.frombuffer((D / "codebook.f32.bin").read_bytes(), "<f4")
    for case in man["cases"]:
        codes = np.frombuffer((D / f"{case['stem']}.codes.bin").read_bytes(), np.uint8)
        dense = book[codes.astype(np.int64) % len(book)]
        assert sha(dense.tobytes()) == case["weights_sha256"], case["stem"]
        if case["stem"] == "13x257":
            raw = (D / "13x257.weights.f32.bin").read_bytes()
            assert dense.tobytes() == raw
