"""CPU oracle of next-token sampling (the reference's sample_token).

TEST INFRASTRUCTURE ONLY. A float64 numpy restatement used by tests/ as the
checker of skv_sample; the product (llm-experiments_amd/) never imports it.

Reference: sample_token, s-i-e-v-e/llm-experiments simple-llm/src/
jax_backend.py:413-515, called from generate_text (generate.py:49-64) with the
last repetition_window tokens (the prompt included) and a fresh subkey per
token:
  :463-467  repetition penalty: for each token in set(recent), logit / penalty
  :470-472  temperature == 0: argmax (first index on ties)
  :474-477  probs = softmax(logits / temperature)
  :480-486  min_p: probs < min_p * max(probs) -> 0, renormalise
  :489-495  top_k: keep argsort(probs)[-top_k:] (numpy's stable argsort; of
            equal probabilities the later index sorts higher), renormalise
  :498-511  top_p: order = argsort(probs)[::-1]; keep where the cumulative sum
            in that order is <= top_p, and always the first; renormalise
  :514      jax.random.choice(key, arange(V), p=probs)

The draw is the build's own rule (sample_draw): the first index whose running
sum, in index order, exceeds u * sum(p). The reference's jax.random stream is
not reproduced (jax is absent), so which token a given key draws is "parity
unpinned"; the filtered distribution it draws from is pinned.
"""
from __future__ import annotations

import numpy as np


def sample_filter(logits, temperature=1.0, top_k=0, top_p=1.0, min_p=0.0,
                  repetition_penalty=1.0, recent_tokens=()):
    """The distribution sample_token draws from (jax_backend.py:413-511), in
    float64; a one-hot vector for greedy (temperature == 0)."""
    x = np.array(logits, dtype=np.float64).copy()
    if repetition_penalty != 1.0 and len(recent_tokens) > 0:
        for tok in set(int(t) for t in recent_tokens):
            x[tok] = x[tok] / repetition_penalty
    if temperature == 0.0:
        out = np.zeros_like(x)
        out[int(np.argmax(x))] = 1.0
        return out
    x = x / temperature
    e = np.exp(x - x.max())
    probs = e / e.sum()
    if min_p > 0.0:
        probs = np.where(probs >= min_p * probs.max(), probs, 0.0)
        probs = probs / probs.sum()
    if top_k > 0:
        keep = np.argsort(probs, kind="stable")[-top_k:]
        mask = np.zeros(probs.shape, bool)
        mask[keep] = True
        probs = np.where(mask, probs, 0.0)
        probs = probs / probs.sum()
    if top_p < 1.0:
        order = np.argsort(probs, kind="stable")[::-1]
        csum = np.cumsum(probs[order])
        keep = csum <= top_p
        keep[0] = True
        filtered = np.zeros_like(probs)
        filtered[order] = np.where(keep, probs[order], 0.0)
        probs = filtered / filtered.sum()
    return probs


def sample_draw(probs, u: float) -> int:
    """First index whose running sum (index order) exceeds u * sum(probs)."""
    c = np.cumsum(np.asarray(probs, np.float64))
    i = int(np.searchsorted(c, u * c[-1], side="right"))
    if i >= len(c):  # u * total rounded onto the end: last nonzero entry
        i = int(np.nonzero(np.asarray(probs) > 0)[0][-1])
    return i


def splitmix_uniform(seed: int, row: int, pos: int) -> float:
    """The build's uniform for (seed, row, position): splitmix64 (S. Vigna's
    public-domain finaliser) of seed ^ (row << 32 | pos), top 24 bits."""
    mask = (1 << 64) - 1
    z = (seed ^ (((row & 0xFFFFFFFF) << 32) | (pos & 0xFFFFFFFF))) & mask
    z = (z + 0x9E3779B97F4A7C15) & mask
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & mask
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & mask
    z ^= z >> 31
    return (z >> 40) / 16777216.0
