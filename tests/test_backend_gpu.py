"""Parity of the module-level drop-ins for the reference backend's free
functions (simple_llm_amd/backend.py): forward(params, inputs, n_layers,
n_heads, head_dim) (jax_backend.py:143-148) against the float64 model
oracle, and sample_token(key, logits, ...) (jax_backend.py:413-515) against
the sampling oracle; then the reference's own generate loop
(generate.py:29-64) run on the two. Needs the MI355X.

Tolerance: logits within the north star's 1e-4 relative error (norm-wise per
row); greedy picks exact; a draw equals the oracle's inverse-CDF draw with the
same uniform except where u * total lies within 1e-5 of a running-sum step.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import banner
from oracle import model_oracle as mo
from oracle import sample_oracle as so

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-4


def rel_rows(got, want):
    got = np.asarray(got, np.float64).reshape(-1, np.shape(got)[-1])
    want = np.asarray(want, np.float64).reshape(-1, np.shape(want)[-1])
    return float((np.linalg.norm(got - want, axis=1) /
                  np.maximum(np.linalg.norm(want, axis=1), 1e-30)).max())


def c1_params():
    """BASELINE configs[0]'s model: 4 layers, d 256, 4 heads x 64, MLP 1024,
    vocab 256, context 256, N(0, 0.02) from seed 0."""
    return mo.init_params(256, 256, 4, 256, seed=0, std=0.02)


def as_objects(params):
    from simple_llm_amd.backend import LayerParams, ModelParams
    return ModelParams(embedding=params["embedding"], pos_encoding=params["pos_encoding"],
                       layers=[LayerParams(**lp) for lp in params["layers"]])


@pytest.mark.parametrize("B,T", [(2, 256), (3, 77), (1, 1)])
def test_forward_matches_oracle(gpu_ctx, B, T):
    """forward() of the C1 model at the reference's T = context_size and at
    shorter T, with params as a dict and as ModelParams / LayerParams."""
    banner(f"backend.forward C1 B={B} T={T}")
    from simple_llm_amd import backend
    params = c1_params()
    toks = np.random.default_rng(B * 1000 + T).integers(0, 256, (B, T))
    got = backend.forward(params, toks, n_layers=4, n_heads=4, head_dim=64)
    assert isinstance(got, torch.Tensor) and got.is_cuda
    assert tuple(got.shape) == (B, T, 256) and got.dtype == torch.float32
    got = got.cpu().numpy()
    want = mo.forward(params, toks, 4)
    err = rel_rows(got, want)
    print(f"rel_err={err:.3e}")
    assert err < FP32_TOL
    # the same weights as LayerParams objects and token ids as a tensor: the
    # same kernels on the same values, so the same bits
    obj = backend.forward(as_objects(params), torch.from_numpy(toks), 4, 4, 64).cpu().numpy()
    np.testing.assert_array_equal(obj, got)


def test_forward_fewer_layers_and_weight_cache(gpu_ctx):
    """n_layers below the params' layer count uses the first layers; device
    weights are made once per params object and remade when an array is
    replaced."""
    banner("backend.forward n_layers and weight cache")
    from simple_llm_amd import backend
    params = mo.init_params(97, 128, 3, 48, seed=3, std=0.1)
    toks = np.random.default_rng(5).integers(0, 97, (2, 48))
    got = backend.forward(params, toks, 2, 2, 64).cpu().numpy()
    two = {"embedding": params["embedding"], "pos_encoding": params["pos_encoding"],
           "layers": params["layers"][:2]}
    assert rel_rows(got, mo.forward(two, toks, 2)) < FP32_TOL
    m1 = backend.device_model(params, 2, 2, 64)
    assert backend.device_model(params, 2, 2, 64) is m1
    # a replaced array: new weights, new device model, new logits
    params["layers"][0] = dict(params["layers"][0])
    params["layers"][0]["attn_wq"] = params["layers"][0]["attn_wq"] * 2.0
    assert backend.device_model(params, 2, 2, 64) is not m1
    got2 = backend.forward(params, toks, 2, 2, 64).cpu().numpy()
    two["layers"] = params["layers"][:2]
    assert rel_rows(got2, mo.forward(two, toks, 2)) < FP32_TOL
    assert not np.array_equal(got, got2)
    backend.forward_cache_clear()
    with pytest.raises(ValueError):
        backend.forward(params, toks[:, :1].repeat(49, 1), 2, 2, 64)  # T > pos rows
    with pytest.raises(ValueError):
        backend.forward(params, toks.astype(np.float32), 2, 2, 64)


@pytest.mark.parametrize("V", [256, 5000, 50304])
def test_sample_token_greedy_is_the_first_maximum(gpu_ctx, V):
    """temperature 0: the first index of the largest (penalised) logit, for
    logits on the device or the host."""
    banner(f"sample_token greedy V={V}")
    from simple_llm_amd import backend
    r = np.random.default_rng(V)
    for trial in range(6):
        lg = r.standard_normal(V).astype(np.float32)
        if trial % 2:
            top = int(r.integers(0, V - 1))
            lg[top] = lg[top + 1] = lg.max() + 1.0  # a tie: the first wins
        recent = r.integers(0, V, 40)
        pen = (1.0, 1.3, 0.7)[trial % 3]
        want = int(np.argmax(so.sample_filter(lg, 0.0, 0, 1.0, 0.0, pen, recent)))
        src = torch.from_numpy(lg).cuda() if trial < 3 else lg
        got = backend.sample_token(trial, src, 0.0, 0, 1.0, 0.0, pen, recent)
        assert got == want, (trial, got, want)


CASES = [dict(temperature=1.0), dict(temperature=0.7, top_k=40),
         dict(temperature=1.2, top_p=0.9), dict(temperature=1.0, min_p=0.05),
         dict(temperature=0.9, top_k=200, top_p=0.8, min_p=0.01, repetition_penalty=1.3)]


@pytest.mark.parametrize("V", [300, 50304])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_sample_token_draws_match_oracle(gpu_ctx, V, case):
    """Each draw is the oracle's draw from sample_token's filtered
    distribution with the uniform of (seed, 0, len(recent_tokens)); the same
    key gives the same token; a key may be an array of words."""
    banner(f"sample_token draws V={V} case={case}")
    from simple_llm_amd import backend
    p = dict(temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, repetition_penalty=1.0)
    p.update(CASES[case])
    r = np.random.default_rng(V + case)
    lg = (r.standard_normal(V) * 2.0).astype(np.float32)
    lgd = torch.from_numpy(lg).cuda()
    exact = 0
    for seed in range(24):
        recent = r.integers(0, V, int(r.integers(0, 65)))
        got = backend.sample_token(seed, lgd, p["temperature"], p["top_k"], p["top_p"],
                                   p["min_p"], p["repetition_penalty"], recent)
        probs = so.sample_filter(lg, p["temperature"], p["top_k"], p["top_p"], p["min_p"],
                                 p["repetition_penalty"], recent)
        u = so.splitmix_uniform(seed, 0, len(recent))
        want = so.sample_draw(probs, u)
        assert probs[got] > 0, (seed, got)
        if got == want:
            exact += 1
        else:
            # only the neighbour across a step of the running sum within fp32
            # rounding of u * total (with V = 50304 the steps are ~1e-5 apart)
            c = np.cumsum(probs)
            lo, hi = min(got, want), max(got, want)
            assert not probs[lo + 1:hi].any(), (seed, got, want)  # adjacent in the support
            assert abs(c[lo] - u * c[-1]) < 1e-5 * c[-1], (seed, got, want)
        again = backend.sample_token(seed, lg, p["temperature"], p["top_k"], p["top_p"],
                                     p["min_p"], p["repetition_penalty"], list(recent))
        assert again == got
    assert exact >= 18, exact
    key = np.array([0, 42], np.uint32)
    a = backend.sample_token(key, lgd, 1.0, 0, 1.0, 0.0, 1.0, [])
    assert a == backend.sample_token(key.copy(), lgd, 1.0, 0, 1.0, 0.0, 1.0, [])


def test_reference_generate_loop_on_the_drop_ins(gpu_ctx):
    """The reference's generate_text loop (generate.py:29-64: left-padded
    context_size window, logits[0, -1], recent tokens, sample_token at
    temperature 0) written against forward and sample_token gives the
    float64 oracle's tokens, up to a near-tie of the oracle's top two."""
    banner("reference generate loop on backend.forward + sample_token")
    from simple_llm_amd import backend
    params = c1_params()
    ctx_len, n_heads, head_dim = 256, 4, 64
    prompt = np.random.default_rng(1).integers(0, 256, 20).tolist()
    tokens = list(prompt)
    margins = []
    for step in range(6):
        ctx = tokens[max(0, len(tokens) - ctx_len):]
        if len(ctx) < ctx_len:
            ctx = [0] * (ctx_len - len(ctx)) + ctx
        logits = backend.forward(params, np.array([ctx], np.int32), n_layers=4,
                                 n_heads=n_heads, head_dim=head_dim)
        nxt = backend.sample_token(step, logits[0, -1, :], temperature=0.0, top_k=0, top_p=1.0,
                                   min_p=0.0, repetition_penalty=1.0,
                                   recent_tokens=np.array(tokens[-64:], np.int32))
        want_row = mo.forward(params, np.array([ctx]), n_heads, last=1)[0, -1]
        top2 = np.sort(want_row)[-2:]
        margins.append(top2[1] - top2[0])
        if nxt != int(np.argmax(want_row)):
            assert top2[1] - top2[0] < 1e-4 * max(1.0, abs(top2[1])), (step, nxt)
            break
        tokens.append(int(nxt))
    print("top-2 margins:", ["%.2e" % m for m in margins])
