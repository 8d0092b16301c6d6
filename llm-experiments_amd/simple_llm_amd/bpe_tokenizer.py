"""Byte-level BPE tokenizer over the native library (skv_bpe_train,
skv_bpe_encode in libskv.so).

Drop-in for the reference's BPETokenizer (simple-llm/src/common/
bpe_tokenizer.py:10-95): the same methods, arguments and merges file
({"p1,p2": new_id, ...} JSON). The reference runs its C program as a
subprocess; here the same algorithm is a call into the library.
"""
from __future__ import annotations

import ctypes
import json
import os
from typing import Dict, List, Tuple

import numpy as np

from . import _lib


def _merges_array(merges: Dict[Tuple[int, int], int]) -> np.ndarray:
    arr = np.array([(p[0], p[1], idx) for p, idx in merges.items()], dtype=np.int32)
    return np.ascontiguousarray(arr.reshape(-1, 3))


def train_merges(data: bytes, vocab_size: int) -> Dict[Tuple[int, int], int]:
    """Merge rules learned from the corpus bytes, in order."""
    L = _lib.lib()
    rounds = max(0, min(int(vocab_size), 50000) - 256)
    out = np.zeros((max(rounds, 1), 3), np.int32)
    buf = np.frombuffer(data, dtype=np.uint8) if data else np.zeros(1, np.uint8)
    n = ctypes.c_int(0)
    _lib.check(L.skv_bpe_train(buf.ctypes.data, len(data), int(vocab_size), out.ctypes.data,
                               max(rounds, 1), ctypes.byref(n)), "skv_bpe_train")
    return {(int(a), int(b)): int(c) for a, b, c in out[:n.value]}


def encode_bytes(data: bytes, merges: Dict[Tuple[int, int], int]) -> List[int]:
    L = _lib.lib()
    arr = _merges_array(merges) if merges else np.zeros((1, 3), np.int32)
    buf = np.frombuffer(data, dtype=np.uint8) if data else np.zeros(1, np.uint8)
    ids = np.zeros(max(len(data), 1), np.int32)
    n = ctypes.c_size_t(0)
    _lib.check(L.skv_bpe_encode(buf.ctypes.data, len(data), arr.ctypes.data, len(merges),
                                ids.ctypes.data, ctypes.byref(n)), "skv_bpe_encode")
    return ids[:n.value].tolist()


class BPETokenizer:
    """Byte-level BPE: 256 byte tokens plus learned merges."""

    def __init__(self):
        self.merges: Dict[Tuple[int, int], int] = {}
        self.vocab: Dict[int, bytes] = {i: bytes([i]) for i in range(256)}

    @property
    def vocab_size(self):
        return len(self.vocab)

    def train(self, text: str, vocab_size: int, token_file: str, verbose: bool = False):
        """Learn vocab_size - 256 merges from text (its UTF-8 bytes) and save
        them to token_file (bpe_tokenizer.py:20-42)."""
        self.merges = train_merges(text.encode("utf-8"), vocab_size)
        self._reconstruct_vocab()
        if verbose:
            print(f"BPE training complete. Learned {len(self.merges)} merges.")
        self._save_merges_to_file(token_file)

    def encode(self, text: str, token_file: str) -> List[int]:
        """Token ids of text with the merges in token_file, read in file order
        as the reference's encoder does (bpe_tokenizer.py:44-57)."""
        with open(token_file, "r", encoding="utf-8") as f:
            merges = {tuple(map(int, k.split(","))): v for k, v in json.load(f).items()}
        return encode_bytes(text.encode("utf-8"), merges)

    def decode(self, ids: List[int]) -> str:
        """bpe_tokenizer.py:59-65: concatenated token bytes, UTF-8 with
        replacement; unknown ids become b"?"."""
        return b"".join(self.vocab.get(idx, b"?") for idx in ids).decode("utf-8",
                                                                          errors="replace")

    def _reconstruct_vocab(self):
        for (p0, p1), idx in self.merges.items():
            self.vocab[idx] = self.vocab[p0] + self.vocab[p1]

    def _save_merges_to_file(self, filepath: str):
        serializable = {f"{p[0]},{p[1]}": idx for p, idx in self.merges.items()}
        with open(filepath, "w", encoding="utf-8") as f:
            json.dump(serializable, f)
        print(f"INFO: Custom BPE tokenizer saved to '{filepath}'")

    def save(self, filepath: str):
        """The reference's save is a no-op (training already wrote the file)."""

    @classmethod
    def load(cls, filepath: str):
        tok = cls()
        with open(filepath, "r", encoding="utf-8") as f:
            tok.merges = {tuple(map(int, k.split(","))): v for k, v in json.load(f).items()}
        tok._reconstruct_vocab()
        print(f"INFO: Custom BPE tokenizer loaded from '{filepath}'")
        return tok
