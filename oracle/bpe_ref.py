"""Runs the reference's own BPE tokenizer program (oracle/_ref/bpe_tokenizer,
compiled by oracle/Makefile from simple-llm/src/common/bpe_tokenizer.c).

TEST INFRASTRUCTURE ONLY: the checker of the build's tokenizer and the CPU
baseline of its measurement. It drives the program the way the reference's
wrapper does (common/bpe_tokenizer.py:21-57): the corpus or text on stdin,
the merges JSON or the ids on stdout.
"""
from __future__ import annotations

import json
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "_ref", "bpe_tokenizer")


def available() -> bool:
    return os.path.exists(BIN)


def build() -> bool:
    """Compile the reference program where its source exists."""
    subprocess.run(["make", "-C", HERE, "ref"], check=True, capture_output=True, text=True)
    return available()


def train(data: bytes, vocab_size: int) -> dict:
    """{"p1,p2": new_id} in merge order, as the program prints it."""
    out = subprocess.run([BIN, "train", str(vocab_size)], input=data, stdout=subprocess.PIPE,
                         stderr=subprocess.DEVNULL, check=True).stdout
    return json.loads(out)


def encode(data: bytes, merges_path: str) -> list:
    out = subprocess.run([BIN, "encode", merges_path], input=data, stdout=subprocess.PIPE,
                         stderr=subprocess.DEVNULL, check=True).stdout
    return [int(t) for t in out.split()]
