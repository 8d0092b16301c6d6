"""The flash-attention backward oracle (oracle/kv_oracle.flash_attention_backward)
against what pins it, on the CPU:
  * the seed-42 golden fixture of the reference's test_flash_attention_backward
    (gpu_test.py:871-1060), whose expected gradients come from torch float64
    autograd of the test's causal attention (tests/golden/make_golden.py);
  * central finite differences of sum(O * dO), independent of any library
    gradient;
  * the reference's two-stage form (gpu_kernels.py:2038-2455): per-Q-block
    partial dK/dV summed by the reduce pass, restated with loops;
  * a planted mistake in the oracle (mask off by one) fails the fixture.
"""
from __future__ import annotations

import os

import numpy as np

import make_golden as mg
from conftest import GOLDEN
from oracle import kv_oracle as ko


def _rel(a, b):
    return float(np.linalg.norm(np.asarray(a) - np.asarray(b)) / max(np.linalg.norm(b), 1e-300))


def _forward(Q, K, V, b, t, h, d):
    return ko.flash_attention(Q.reshape(b * t, -1), K.reshape(b * t, -1), V.reshape(b * t, -1),
                              b, t, h, d)


def test_backward_golden_kat():
    z = np.load(os.path.join(GOLDEN, "flash_bwd_kat_seed42.npz"))
    for i, (b, t, h, d) in enumerate(z["configs"]):
        Q, K, V, dO = mg.flash_bwd_inputs(b, t, h, d)
        O, L, M = _forward(Q, K, V, b, t, h, d)
        assert _rel(O, z[f"o_{i}"]) < 1e-12 and _rel(L, z[f"l_{i}"]) < 1e-12
        assert np.array_equal(M, z[f"m_{i}"]) or _rel(M, z[f"m_{i}"]) < 1e-12
        dq, dk, dv = ko.flash_attention_backward(Q, K, V, O, L, M, dO.reshape(b * t, -1),
                                                 b, t, h, d)
        for name, got in (("dq", dq), ("dk", dk), ("dv", dv)):
            assert _rel(got, z[f"{name}_{i}"]) < 1e-10, (i, name)


def test_backward_matches_finite_differences():
    rng = np.random.default_rng(5)
    b, t, h, d = 1, 5, 2, 4
    Q, K, V, dO = (rng.standard_normal((b * t, h * d)) for _ in range(4))

    def loss(q, k, v):
        return float((_forward(q, k, v, b, t, h, d)[0] * dO).sum())

    O, L, M = _forward(Q, K, V, b, t, h, d)
    grads = ko.flash_attention_backward(Q, K, V, O, L, M, dO, b, t, h, d)
    eps = 1e-6
    for which, g in enumerate(grads):
        num = np.zeros_like(g)
        for idx in np.ndindex(*g.shape):
            args = [Q.copy(), K.copy(), V.copy()]
            args[which][idx] += eps
            up = loss(*args)
            args[which][idx] -= 2 * eps
            num[idx] = (up - loss(*args)) / (2 * eps)
        assert _rel(g, num) < 1e-7, which


def _two_stage_loops(Q, K, V, O, L, M, dO, b, t, h, d, Br=4):
    """Stage 1 per Q block into per-block partials, then stage 2 sums them."""
    scale = 1.0 / np.sqrt(d)
    E = h * d
    nqb = (t + Br - 1) // Br
    dq = np.zeros((b * t, E))
    wk = np.zeros((nqb, b * t, E))
    wv = np.zeros((nqb, b * t, E))
    for bb in range(b):
        for hh in range(h):
            cols = slice(hh * d, (hh + 1) * d)
            for blk in range(nqb):
                for i in range(blk * Br, min(blk * Br + Br, t)):
                    r = bb * t + i
                    st = (bb * t + i) * h + hh
                    Di = float(np.dot(dO[r, cols], O[r, cols]))
                    for j in range(i + 1):
                        c = bb * t + j
                        s = float(np.dot(Q[r, cols], K[c, cols])) * scale
                        p = np.exp(s - M[st]) / L[st]
                        dp = float(np.dot(dO[r, cols], V[c, cols]))
                        ds = p * (dp - Di)
                        dq[r, cols] += ds * K[c, cols] * scale
                        wk[blk, c, cols] += ds * Q[r, cols] * scale
                        wv[blk, c, cols] += p * dO[r, cols]
    return dq, wk.sum(0), wv.sum(0)


def test_backward_equals_reference_two_stage_form():
    rng = np.random.default_rng(9)
    b, t, h, d = 2, 7, 2, 8
    Q, K, V, dO = (rng.standard_normal((b * t, h * d)) for _ in range(4))
    O, L, M = _forward(Q, K, V, b, t, h, d)
    want = _two_stage_loops(Q, K, V, O, L, M, dO, b, t, h, d)
    got = ko.flash_attention_backward(Q, K, V, O, L, M, dO, b, t, h, d)
    for g, w in zip(got, want):
        assert _rel(g, w) < 1e-12


def test_planted_mask_mistake_fails_fixture(monkeypatch):
    z = np.load(os.path.join(GOLDEN, "flash_bwd_kat_seed42.npz"))
    b, t, h, d = z["configs"][0]
    Q, K, V, dO = mg.flash_bwd_inputs(b, t, h, d)
    O, L, M = _forward(Q, K, V, b, t, h, d)
    real_tril = np.tril
    monkeypatch.setattr(ko.np, "tril", lambda m, k=0: real_tril(m, k - 1))  # key < query
    dq, dk, dv = ko.flash_attention_backward(Q, K, V, O, L, M, dO.reshape(b * t, -1), b, t, h, d)
    monkeypatch.undo()
    assert _rel(dq, z["dq_0"]) > 1e-2 and _rel(dv, z["dv_0"]) > 1e-2
