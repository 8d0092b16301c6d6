"""Writes tests/golden/bpe_golden.json: merges and encodings produced by the
reference's own BPE program (oracle/_ref/bpe_tokenizer, compiled by
`make -C oracle ref` from simple-llm/src/common/bpe_tokenizer.c) on seeded
synthetic corpora. Run in the build container, where the reference exists:

    python tests/golden/make_bpe_golden.py
"""
from __future__ import annotations

import json
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import bpe_ref  # noqa: E402


def corpora():
    r = np.random.default_rng(2024)
    out = []
    for k in range(12):  # small alphabets: many equal pair counts (tie order)
        alpha = 2 + k % 4
        n = 50 + 40 * k
        out.append((bytes(r.integers(97, 97 + alpha, n).astype(np.uint8)), 256 + 5 + 7 * k))
    words = ["the", "cat", "sat", "on", "a", "mat", "über", "naïve", "✓", "—"]
    text = " ".join(words[i] for i in r.integers(0, len(words), 400))
    out.append((text.encode("utf-8"), 330))
    out.append((bytes(range(256)) * 2, 300))
    out.append((b"", 300))
    out.append((b"x", 300))
    out.append((b"aaaa", 200))  # vocab_size < 256: no merges
    return out


def main():
    if not bpe_ref.available() and not bpe_ref.build():
        raise SystemExit("reference tokenizer source not found")
    r = np.random.default_rng(7)
    cases = []
    for data, vs in corpora():
        merges = bpe_ref.train(data, vs)
        probe = bytes(r.integers(97, 102, 120).astype(np.uint8)) + data[:200]
        with tempfile.NamedTemporaryFile("w", suffix=".json", delete=False) as f:
            json.dump(merges, f)
            path = f.name
        ids = bpe_ref.encode(probe, path)
        os.unlink(path)
        cases.append({"corpus_hex": data.hex(), "vocab_size": vs,
                      "merges": [[*map(int, k.split(",")), v] for k, v in merges.items()],
                      "probe_hex": probe.hex(), "probe_ids": ids})
    with open(os.path.join(HERE, "bpe_golden.json"), "w") as f:
        json.dump({"generator": "oracle/_ref/bpe_tokenizer (the reference's bpe_tokenizer.c)",
                   "cases": cases}, f, separators=(",", ":"))
    print(f"{len(cases)} cases")


if __name__ == "__main__":
    main()
