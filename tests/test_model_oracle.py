"""Pins the model oracle (oracle/model_oracle.py) before it is used as the
checker of the GPU decode step. CPU only.

Each piece is checked against something it was not written from: closed-form
values, torch's float64 library routines, and the equivalence of two
different algorithms (full causal forward vs per-token cached recurrence).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import model_oracle as mo

rng = np.random.default_rng(7)


def test_positional_encoding_closed_form():
    d = 16
    pe = mo.positional_encoding(40, d)
    assert pe.shape == (40, d)
    # position 0: sin(0) = 0 in the first half, cos(0) = 1 in the second
    np.testing.assert_array_equal(pe[0, : d // 2], 0.0)
    np.testing.assert_array_equal(pe[0, d // 2:], 1.0)
    # concatenated halves: column j is sin(p w_j), column d/2 + j is cos(p w_j),
    # w_j = 10000^(-2j/d) (jax_backend.py:25-33 takes even angles for sin and
    # odd angles, whose rate equals the preceding even one, for cos)
    for p, j in [(5, 3), (39, 0), (17, 7), (1, 1)]:
        w = 10000.0 ** (-2 * j / d)
        assert pe[p, j] == pytest.approx(math.sin(p * w), abs=1e-15)
        assert pe[p, d // 2 + j] == pytest.approx(math.cos(p * w), abs=1e-15)
    # not interleaved: column 1 is a sine, not a cosine
    assert pe[3, 1] == pytest.approx(math.sin(3 * 10000.0 ** (-2 / d)), abs=1e-15)


def test_layer_norm_matches_torch():
    x = rng.standard_normal((5, 7, 96)) * 3 + 1
    g = rng.standard_normal(96)
    b = rng.standard_normal(96)
    want = F.layer_norm(torch.from_numpy(x), (96,), torch.from_numpy(g), torch.from_numpy(b),
                        eps=1e-5).numpy()
    np.testing.assert_allclose(mo.layer_norm(x, g, b), want, rtol=1e-12, atol=1e-12)


def test_gelu_matches_torch_tanh_form():
    x = np.linspace(-8, 8, 2001)
    want = F.gelu(torch.from_numpy(x), approximate="tanh").numpy()
    np.testing.assert_allclose(mo.gelu_tanh(x), want, rtol=1e-12, atol=1e-14)
    # and differs from the exact erf GELU (so the wrong variant would fail)
    exact = F.gelu(torch.from_numpy(x)).numpy()
    assert np.abs(mo.gelu_tanh(x) - exact).max() > 1e-4


def torch_forward(params, tokens, n_heads):
    """Independent float64 model from torch library routines."""
    E = torch.from_numpy(np.asarray(params["embedding"], np.float64))
    PE = torch.from_numpy(np.asarray(params["pos_encoding"], np.float64))
    ids = torch.from_numpy(np.asarray(tokens))
    B, T = ids.shape
    d = E.shape[1]
    x = E[ids] + PE[:T]
    for lp in params["layers"]:
        t = {k: torch.from_numpy(np.asarray(v, np.float64)) for k, v in lp.items()}
        h = F.layer_norm(x, (d,), t["ln_gamma1"], t["ln_beta1"], eps=1e-5)

        def heads(y):
            return y.reshape(B, T, n_heads, d // n_heads).transpose(1, 2)

        a = F.scaled_dot_product_attention(heads(h @ t["attn_wq"]), heads(h @ t["attn_wk"]),
                                           heads(h @ t["attn_wv"]), is_causal=True)
        x = x + a.transpose(1, 2).reshape(B, T, d) @ t["attn_wo"]
        h = F.layer_norm(x, (d,), t["ln_gamma2"], t["ln_beta2"], eps=1e-5)
        x = x + F.gelu(h @ t["ff_w1"] + t["ff_b1"], approximate="tanh") @ t["ff_w2"] + t["ff_b2"]
    return (x @ E.T).numpy()


def small_params(seed=0, vocab=37, dim=32, layers=2, ctx=24, std=0.3):
    p = mo.init_params(vocab, dim, layers, ctx, seed=seed, std=std)
    r = np.random.default_rng(seed + 1)
    for lp in p["layers"]:  # non-trivial LayerNorm affine and biases
        for k in ("ff_b1", "ff_b2", "ln_beta1", "ln_beta2"):
            lp[k] = (r.standard_normal(lp[k].shape) * 0.1).astype(np.float32)
        for k in ("ln_gamma1", "ln_gamma2"):
            lp[k] = (1 + r.standard_normal(lp[k].shape) * 0.1).astype(np.float32)
    return p


def test_forward_matches_torch_model():
    p = small_params()
    toks = rng.integers(0, 37, (3, 24))
    np.testing.assert_allclose(mo.forward(p, toks, 4), torch_forward(p, toks, 4),
                               rtol=1e-10, atol=1e-12)


def test_forward_is_causal():
    p = small_params(seed=3)
    a = rng.integers(0, 37, (1, 20))
    b = a.copy()
    b[0, 12] = (b[0, 12] + 5) % 37
    la, lb = mo.forward(p, a, 4), mo.forward(p, b, 4)
    np.testing.assert_array_equal(la[0, :12], lb[0, :12])
    assert np.abs(la[0, 12:] - lb[0, 12:]).max() > 1e-6


def test_decode_step_equals_forward_rows():
    p = small_params(seed=5)
    toks = rng.integers(0, 37, (2, 18))
    full = mo.forward(p, toks, 4)
    st = mo.DecodeState(2, 2)
    for t in range(18):
        lg = mo.decode_step(p, st, toks[:, t], [t, t], 4)
        np.testing.assert_allclose(lg, full[:, t], rtol=1e-10, atol=1e-12)


def test_decode_step_ragged_positions():
    """Sequences at different positions (the ragged-batch case)."""
    p = small_params(seed=6)
    toks = rng.integers(0, 37, (2, 16))
    full = mo.forward(p, toks, 4)
    st = mo.DecodeState(2, 2)
    # sequence 1 starts 5 steps later
    for t in range(16):
        act = [True, t >= 5]
        lg = mo.decode_step(p, st, [toks[0, t], toks[1, max(t - 5, 0)]], [t, max(t - 5, 0)], 4,
                            active=act)
        np.testing.assert_allclose(lg[0], full[0, t], rtol=1e-10, atol=1e-12)
        if act[1]:
            np.testing.assert_allclose(lg[1], full[1, t - 5], rtol=1e-10, atol=1e-12)


def test_greedy_generate_is_teacher_forced_forward():
    p = small_params(seed=8)
    toks, logits = mo.greedy_generate(p, [1, 2, 3, 4], 12, 4)
    assert len(toks) == 16
    full = mo.forward(p, np.array([toks]), 4)[0]
    np.testing.assert_allclose(logits, full[3:15], rtol=1e-10, atol=1e-12)
    assert toks[4:] == [int(np.argmax(r)) for r in full[3:15]]


def test_reference_generate_left_pads_window():
    """generate.py:31-36: the window is the last context_size tokens, left-
    padded with token 0; the next token is the argmax of the last row."""
    p = small_params(seed=9)
    seen = []

    def spy(params, ids):
        seen.append(ids[0].tolist())
        return mo.forward(params, ids, 4)

    out = mo.reference_generate(p, [5, 6, 7], 3, 4, context_size=8, forward_fn=spy)
    assert seen[0] == [0, 0, 0, 0, 0, 5, 6, 7]
    assert seen[1][:4] == [0, 0, 0, 0] and seen[1][5:7] == [6, 7]
    assert len(out) == 6
    # once the sequence exceeds the window, only the last 8 tokens are fed
    out2 = mo.reference_generate(p, list(range(1, 11)), 2, 4, context_size=8, forward_fn=spy)
    assert seen[-2] == list(range(3, 11))
    assert out2[:10] == list(range(1, 11))


def test_torch_fp32_forward_matches_oracle():
    """The CPU-baseline forward (float32 torch) agrees with the float64
    oracle to float32 accuracy."""
    p = small_params(seed=11, std=0.1)
    toks = rng.integers(0, 37, (2, 24))
    got = mo.torch_forward_fp32(p, toks, 4).numpy()
    want = mo.forward(p, toks, 4)
    err = np.linalg.norm(got - want, axis=-1) / np.linalg.norm(want, axis=-1)
    assert err.max() < 1e-4


def test_torch_cached_decoder_matches_decode_step():
    """The float32 batched cache decoder (bench.py's same-algorithm CPU
    baseline) equals the float64 cached recurrence step by step."""
    params = mo.init_params(61, 32, 2, 40, seed=3, std=0.1)
    rng = np.random.default_rng(8)
    B, steps = 3, 12
    toks = rng.integers(0, 61, (B, steps))
    dec = mo.TorchCachedDecoder(params, 4, B, 40)
    state = mo.DecodeState(2, B)
    for t in range(steps):
        got = dec.step(toks[:, t])
        want = mo.decode_step(params, state, toks[:, t], [t] * B, 4)
        err = np.linalg.norm(got - want, axis=1) / np.linalg.norm(want, axis=1)
        assert err.max() < 1e-5, (t, err.max())
    assert dec.len.tolist() == [steps] * B
