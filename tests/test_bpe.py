"""The build's BPE tokenizer (skv_bpe_train / skv_bpe_encode, BPETokenizer)
against the reference's own program (simple-llm/src/common/bpe_tokenizer.c):
golden merges and encodings it produced (tests/golden/bpe_golden.json), and,
where oracle/_ref/bpe_tokenizer is built, a live comparison on more corpora.
CPU only. Merges, their order and token ids must match exactly.
"""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

from oracle import bpe_ref
from simple_llm_amd.bpe_tokenizer import BPETokenizer, encode_bytes, train_merges

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "bpe_golden.json")
REF_DATA = "/root/reference/simple-llm/data"


def golden_cases():
    with open(GOLDEN) as f:
        return json.load(f)["cases"]


@pytest.mark.parametrize("case", range(len(golden_cases())))
def test_matches_reference_golden(case):
    c = golden_cases()[case]
    data, vs = bytes.fromhex(c["corpus_hex"]), c["vocab_size"]
    got = train_merges(data, vs)
    assert [[a, b, i] for (a, b), i in got.items()] == c["merges"]
    merges = {(a, b): i for a, b, i in c["merges"]}
    assert encode_bytes(bytes.fromhex(c["probe_hex"]), merges) == c["probe_ids"]


@pytest.mark.skipif(not bpe_ref.available(), reason="oracle/_ref/bpe_tokenizer not built")
def test_matches_reference_program_live(tmp_path):
    r = np.random.default_rng(3)
    corpora = [(bytes(r.integers(97, 97 + int(r.integers(2, 7)), int(r.integers(2, 600)))
                      .astype(np.uint8)), int(r.integers(257, 360))) for _ in range(40)]
    for name in ("sherlock_red_2.txt", "sherlock_red.txt"):
        path = os.path.join(REF_DATA, name)
        if os.path.exists(path):
            corpora.append((open(path, "rb").read(), 600))
    for data, vs in corpora:
        want = bpe_ref.train(data, vs)
        got = {f"{a},{b}": i for (a, b), i in train_merges(data, vs).items()}
        assert list(got.items()) == list(want.items())
        mf = tmp_path / "m.json"
        mf.write_text(json.dumps(want))
        probe = data[:3000] + bytes(r.integers(97, 100, 100).astype(np.uint8))
        assert encode_bytes(probe, {tuple(map(int, k.split(","))): v for k, v in want.items()}) \
            == bpe_ref.encode(probe, str(mf))


def test_edges():
    assert train_merges(b"", 300) == {}
    assert train_merges(b"q", 300) == {}
    assert train_merges(b"abab", 256) == {}  # vocab_size <= 256: no merges
    # merges stop when no pair is left
    m = train_merges(b"aaaa", 300)
    assert m == {(97, 97): 256, (256, 256): 257}
    # overlapping occurrences count: "aaa" has two (a, a) pairs, merged left to right
    assert encode_bytes(b"aaa", {(97, 97): 256}) == [256, 97]
    # only raw-byte pairs apply when encoding, and the first merge of a pair wins
    assert encode_bytes(b"abab", {(256, 256): 300, (97, 98): 256, (97, 98): 256}) == [256, 256]
    assert encode_bytes(b"", {}) == []


def test_tokenizer_api_round_trip(tmp_path):
    text = "It was the best of times, it was the worst of times — naïve café ✓\n" * 30
    tok = BPETokenizer()
    path = str(tmp_path / "tokenizer.json")
    tok.train(text, 320, path)
    # the repeated line can collapse into one token before 64 merges: the
    # reference stops when no pair is left, and so does this
    n = len(tok.merges)
    assert 0 < n <= 64 and tok.vocab_size == 256 + n
    saved = json.loads(open(path).read())
    assert list(saved.values()) == list(range(256, 256 + n))  # "p1,p2": id in merge order
    ids = tok.encode(text, path)
    assert tok.decode(ids) == text  # byte-level: lossless
    assert len(ids) < len(text.encode("utf-8"))
    again = BPETokenizer.load(path)
    assert again.merges == tok.merges and again.vocab == tok.vocab
    assert again.decode([999999]) == "?"  # unknown id, as the reference
