"""Pins the sampling oracle (oracle/sample_oracle.py) before it checks the GPU
sampler. CPU only.

Each filter is checked against something it was not written from: torch's
softmax / topk / sort, brute-force loops over the descending order, closed
forms (one-hot cases) and the tie rule of a stable ascending argsort
(jax_backend.py:490 and :500 sort with jnp.argsort).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import sample_oracle as so

rng = np.random.default_rng(11)


def test_plain_softmax_with_temperature():
    x = rng.standard_normal(500) * 3
    for T in (0.3, 1.0, 1.7):
        want = torch.softmax(torch.from_numpy(x) / T, 0).numpy()
        np.testing.assert_allclose(so.sample_filter(x, T), want, rtol=1e-12, atol=1e-15)


def test_greedy_is_first_argmax_one_hot():
    x = rng.standard_normal(64)
    x[[7, 40]] = x.max() + 1.0  # a tie: the first index wins (jnp.argmax)
    p = so.sample_filter(x, 0.0)
    assert p[7] == 1.0 and p.sum() == 1.0


def test_repetition_penalty_is_a_set_division():
    x = rng.standard_normal(32)
    got = so.sample_filter(x, 0.0, repetition_penalty=2.0, recent_tokens=[5, 5, 5, 9])
    y = x.copy()
    y[5] /= 2.0  # once, although 5 appears three times
    y[9] /= 2.0
    assert got.argmax() == y.argmax()
    # at T = 1 the whole distribution follows the penalised logits
    p = so.sample_filter(x, 1.0, repetition_penalty=2.0, recent_tokens=[5, 5, 5, 9])
    np.testing.assert_allclose(p, torch.softmax(torch.from_numpy(y), 0).numpy(), rtol=1e-12)
    # negative logits are divided too (moving them up), as the reference does
    x2 = -np.abs(x)
    p2 = so.sample_filter(x2, 1.0, repetition_penalty=4.0, recent_tokens=[3])
    assert p2[3] > so.sample_filter(x2, 1.0)[3]


def test_top_k_matches_torch_topk():
    x = rng.standard_normal(1000)  # distinct values
    for k in (1, 7, 50, 999):
        p = so.sample_filter(x, 0.9, top_k=k)
        full = torch.softmax(torch.from_numpy(x) / 0.9, 0)
        v, idx = torch.topk(full, k)
        want = np.zeros(1000)
        want[idx.numpy()] = (v / v.sum()).numpy()
        np.testing.assert_allclose(p, want, rtol=1e-12, atol=1e-15)
    # k = 1 is greedy's one-hot
    p1 = so.sample_filter(x, 1.3, top_k=1)
    assert p1[np.argmax(x)] == 1.0


def test_top_k_ties_keep_larger_indices():
    x = np.zeros(10)
    x[[2, 5, 8]] = 1.0  # three equal maxima, k = 2
    p = so.sample_filter(x, 1.0, top_k=2)
    assert p[8] > 0 and p[5] > 0 and p[2] == 0


def _top_p_brute(p, top_p):
    order = sorted(range(len(p)), key=lambda i: (-p[i], -i))  # descending, later index first
    out, run = np.zeros_like(p), 0.0
    for r, i in enumerate(order):
        run += p[i]
        if run <= top_p or r == 0:
            out[i] = p[i]
    return out / out.sum()


@pytest.mark.parametrize("top_p", [0.0, 0.05, 0.5, 0.9, 0.999])
def test_top_p_matches_brute_force(top_p):
    x = rng.standard_normal(300) * 2
    p = so.sample_filter(x, 1.0)
    np.testing.assert_allclose(so.sample_filter(x, 1.0, top_p=top_p), _top_p_brute(p, top_p),
                               rtol=1e-12, atol=1e-15)


def test_top_p_ties_and_first_entry():
    x = np.zeros(6)
    x[[1, 4]] = 3.0  # two equal tops; a tiny top_p keeps only the later index
    p = so.sample_filter(x, 1.0, top_p=1e-6)
    assert p[4] == 1.0


def test_min_p_threshold():
    x = rng.standard_normal(200)
    base = so.sample_filter(x, 1.0)
    p = so.sample_filter(x, 1.0, min_p=0.3)
    keep = base >= 0.3 * base.max()
    assert ((p > 0) == keep).all()
    np.testing.assert_allclose(p[keep], base[keep] / base[keep].sum(), rtol=1e-12)
    assert so.sample_filter(x, 1.0, min_p=1.0)[np.argmax(x)] == 1.0


def test_filters_compose_in_reference_order():
    """min_p, then top_k on the renormalised result, then top_p on that."""
    x = rng.standard_normal(400) * 1.5
    p = so.sample_filter(x, 0.8)
    p = np.where(p >= 0.02 * p.max(), p, 0.0)
    p /= p.sum()
    idx = np.argsort(-p, kind="stable")[:30]
    q = np.zeros_like(p)
    q[idx] = p[idx]
    q /= q.sum()
    want = _top_p_brute(q, 0.7)
    got = so.sample_filter(x, 0.8, top_k=30, top_p=0.7, min_p=0.02)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-15)


def test_draw_is_inverse_cdf_in_index_order():
    p = np.array([0.0, 0.2, 0.0, 0.5, 0.3])
    assert so.sample_draw(p, 0.0) == 1
    assert so.sample_draw(p, 0.199) == 1
    assert so.sample_draw(p, 0.2) == 3
    assert so.sample_draw(p, 0.7) == 4
    assert so.sample_draw(p, 0.99999) == 4
    # brute force over many u
    q = rng.random(50)
    q[rng.random(50) < 0.4] = 0.0
    for u in rng.random(200):
        i = next(j for j in range(50) if q[: j + 1].sum() > u * q.sum())
        assert so.sample_draw(q, u) == i


def test_splitmix_uniform_range_and_spread():
    u = np.array([so.splitmix_uniform(42, r, p) for r in range(20) for p in range(500)])
    assert (u >= 0).all() and (u < 1).all()
    assert len(np.unique(u)) > 0.99 * len(u)
    hist = np.histogram(u, bins=10, range=(0, 1))[0]
    assert hist.min() > 0.85 * len(u) / 10  # close to uniform
