"""Parity of the device sampler (skv_sample) with the sampling oracle
(sample_token, jax_backend.py:413-515, restated in oracle/sample_oracle.py).
Needs the MI355X.

The filtered distribution (probs_out) must match the float64 oracle: the same
kept entries and values within 1e-4 relative. The GPU computes in fp32, so an
entry whose keep/drop decision lies within float rounding of a cut (a top-p
running sum within 1e-5 of top_p) may differ. The drawn token must equal the
oracle's inverse-CDF draw with the same u, except when u * total lies within
1e-5 of a cumulative-sum step. Greedy picks and ties are exact.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import banner
from oracle import sample_oracle as so

pytestmark = pytest.mark.gpu


def lib():
    from simple_llm_amd import _lib
    return _lib


def run_sample(logits, seq, lens, T=1.0, top_k=0, top_p=1.0, min_p=0.0, pen=1.0, window=64,
               seed=42, probs=True, ws=False):
    """ws: pass skv_sample_workspace_bytes(M, V) bytes of workspace (the split
    path of unfiltered draws from rows of >= 8192 entries, when probs is off)."""
    _lib = lib()
    L = _lib.lib()
    M, V = logits.shape
    lg = torch.from_numpy(np.ascontiguousarray(logits, np.float32)).cuda()
    sq = torch.from_numpy(np.ascontiguousarray(seq, np.int32)).cuda()
    ln = torch.from_numpy(np.ascontiguousarray(lens, np.int32)).cuda()
    out = torch.full((M,), -7, dtype=torch.int32, device="cuda")
    pr = torch.full((M, V), float("nan"), device="cuda") if probs else None
    wsb = L.skv_sample_workspace_bytes(M, V) if ws else 0
    wst = torch.full((max(wsb, 8),), 0xFF, dtype=torch.uint8, device="cuda")  # stale bytes
    rc = L.skv_sample(out.data_ptr(), pr.data_ptr() if probs else None, lg.data_ptr(),
                      sq.data_ptr(), seq.shape[1], ln.data_ptr(), M, V, T, top_k, top_p, min_p,
                      pen, window, seed, wst.data_ptr() if ws else None, wsb,
                      _lib.stream_handle())
    _lib.check(rc, "skv_sample")
    return out.cpu().numpy(), (pr.cpu().numpy() if probs else None)


def oracle_row(logits_row, seq_row, L, T, top_k, top_p, min_p, pen, window):
    recent = seq_row[max(0, L - window):L] if pen != 1.0 else []
    return so.sample_filter(logits_row.astype(np.float64), T, top_k, top_p, min_p, pen, recent)


def top_p_ambiguous(logits_row, seq_row, L, T, top_k, top_p, min_p, pen, window):
    """Entries whose top-p decision is within float rounding of the cut."""
    if top_p >= 1.0:
        return set()
    pre = oracle_row(logits_row, seq_row, L, T, top_k, 1.0, min_p, pen, window)
    order = np.argsort(pre, kind="stable")[::-1]
    c = np.cumsum(pre[order])
    return {int(order[i]) for i in np.nonzero(np.abs(c - top_p) < 1e-5)[0]}


CASES = [
    dict(T=1.0),
    dict(T=0.7, top_k=40),
    dict(T=1.2, top_p=0.9),
    dict(T=1.0, min_p=0.05),
    dict(T=0.9, top_k=200, top_p=0.8, min_p=0.01, pen=1.3, window=64),
    dict(T=0.5, top_p=0.3, pen=0.8, window=16),
]


@pytest.mark.parametrize("V", [100, 256, 5000, 20000, 50304, 60000])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_sample_matches_oracle(gpu_ctx, V, case):
    p = dict(top_k=0, top_p=1.0, min_p=0.0, pen=1.0, window=64)
    p.update(CASES[case])
    banner(f"sample V={V} {p}")
    r = np.random.default_rng(V * 10 + case)
    M, ctx = 3, 300
    logits = (r.standard_normal((M, V)) * 2.5).astype(np.float32)
    seq = r.integers(0, V, (M, ctx)).astype(np.int32)
    lens = np.array([1, 150, ctx])
    seed = 1234 + case
    tok, probs = run_sample(logits, seq, lens, seed=seed, **p)
    tok2, probs2 = run_sample(logits, seq, lens, seed=seed, **p)
    np.testing.assert_array_equal(tok, tok2)  # bitwise reproducible
    np.testing.assert_array_equal(probs, probs2)
    for m in range(M):
        want = oracle_row(logits[m], seq[m], int(lens[m]), **p)
        amb = top_p_ambiguous(logits[m], seq[m], int(lens[m]), **p)
        diff = set(np.nonzero((probs[m] > 0) != (want > 0))[0].tolist())
        assert diff <= amb, f"row {m}: kept sets differ at {sorted(diff)[:10]}"
        if not diff:
            keep = want > 0
            np.testing.assert_allclose(probs[m][keep], want[keep], rtol=1e-4, atol=1e-9)
            assert np.abs(probs[m].sum() - 1.0) < 1e-5
            u = so.splitmix_uniform(seed, m, int(lens[m]))
            c = np.cumsum(want)
            near = np.abs(c - u * c[-1]).min() < 1e-5
            if not near:
                assert tok[m] == so.sample_draw(want, u), f"row {m}"
        assert probs[m][tok[m]] > 0


@pytest.mark.parametrize("V", [256, 50304])
def test_greedy_with_penalty_is_exact(gpu_ctx, V):
    banner(f"sample greedy V={V}")
    r = np.random.default_rng(V)
    M, ctx = 4, 64
    logits = r.standard_normal((M, V)).astype(np.float32)
    logits[:, 10] = logits[:, 20] = logits.max() + 1  # a tie: index 10 wins
    seq = r.integers(0, V, (M, ctx)).astype(np.int32)
    seq[1, -5:] = 10  # row 1 penalises token 10 (positive logit -> smaller)
    lens = np.full(M, ctx)
    tok, probs = run_sample(logits, seq, lens, T=0.0, pen=4.0, window=8)
    for m in range(M):
        want = oracle_row(logits[m], seq[m], ctx, 0.0, 0, 1.0, 0.0, 4.0, 8)
        assert tok[m] == int(np.argmax(want))
        assert probs[m][tok[m]] == 1.0 and probs[m].sum() == 1.0
    assert tok[0] == 10 and tok[1] == 20


def test_ties_follow_the_stable_argsort(gpu_ctx):
    banner("sample ties")
    V = 3000
    logits = np.zeros((2, V), np.float32)
    logits[:, [100, 900, 2500]] = 5.0  # three equal tops
    seq = np.zeros((2, 4), np.int32)
    lens = np.full(2, 4)
    _, pk = run_sample(logits, seq, lens, T=1.0, top_k=2)
    want = so.sample_filter(logits[0].astype(np.float64), 1.0, top_k=2)
    np.testing.assert_array_equal(pk[0] > 0, want > 0)  # 900 and 2500 kept
    assert pk[0][2500] > 0 and pk[0][900] > 0 and pk[0][100] == 0
    tok, pp = run_sample(logits, seq, lens, T=1.0, top_p=1e-6)
    assert (tok == 2500).all() and pp[0][2500] == 1.0


def test_draws_follow_the_distribution(gpu_ctx):
    """Many rows with the same logits and different positions: the draw
    frequencies follow the filtered distribution."""
    banner("sample frequencies")
    V, M = 50, 4000
    r = np.random.default_rng(5)
    row = r.standard_normal(V).astype(np.float32)
    logits = np.tile(row, (M, 1))
    seq = np.zeros((M, 1), np.int32)
    lens = np.ones(M, np.int32)
    tok, _ = run_sample(logits, seq, lens, T=1.0, top_k=10, probs=False, seed=7)
    want = so.sample_filter(row.astype(np.float64), 1.0, top_k=10)
    freq = np.bincount(tok, minlength=V) / M
    assert (freq[want == 0] == 0).all()
    assert np.abs(freq - want).max() < 0.03


SPLIT_CASES = [dict(T=1.0), dict(T=0.9, pen=1.3, window=64), dict(T=0.6, pen=0.7, window=200)]


@pytest.mark.parametrize("V", [8192, 20000, 50304, 65536])
@pytest.mark.parametrize("case", range(len(SPLIT_CASES)))
def test_split_sample_matches_oracle(gpu_ctx, V, case):
    """Unfiltered draws from wide rows on the split path (slice statistics,
    then one workgroup per row): u * total lies within the drawn token's step
    of the oracle's running sum (to 1e-5), and the token is the oracle's
    inverse-CDF draw with the same u, and k_sample's, where u * total is not
    within 1e-5 of a step; two calls give the same tokens."""
    p = dict(pen=1.0, window=64)
    p.update(SPLIT_CASES[case])
    banner(f"split sample V={V} {p}")
    L = lib().lib()
    assert L.skv_sample_workspace_bytes(16, V) == 16 * ((V + 2047) // 2048) * 8
    r = np.random.default_rng(V * 7 + case)
    M, ctx = 16, 300
    logits = (r.standard_normal((M, V)) * 2.5).astype(np.float32)
    seq = r.integers(0, V, (M, ctx)).astype(np.int32)
    lens = r.integers(1, ctx + 1, M)
    seed = 99 + case
    tok, _ = run_sample(logits, seq, lens, seed=seed, probs=False, ws=True, **p)
    tok2, _ = run_sample(logits, seq, lens, seed=seed, probs=False, ws=True, **p)
    one, _ = run_sample(logits, seq, lens, seed=seed, probs=False, ws=False, **p)
    np.testing.assert_array_equal(tok, tok2)
    for m in range(M):
        want = oracle_row(logits[m], seq[m], int(lens[m]), p["T"], 0, 1.0, 0.0, p["pen"],
                          p["window"])
        u = so.splitmix_uniform(seed, m, int(lens[m]))
        c = np.cumsum(want)
        target = u * c[-1]
        assert want[tok[m]] > 0
        below = c[tok[m] - 1] if tok[m] > 0 else 0.0
        assert below - 1e-5 <= target < c[tok[m]] + 1e-5, f"row {m}"
        if np.abs(c - target).min() >= 1e-5:
            assert tok[m] == so.sample_draw(want, u) == one[m], f"row {m}"


def test_split_sample_edge_rows(gpu_ctx):
    """Rows the split path must answer as k_sample does: no finite logit
    (token 0), a NaN logit (token 0), a whole slice at -inf (never drawn),
    the mass in the last entry of the last, ragged slice, and in entry 0."""
    banner("split sample edge rows")
    V, M = 20000, 6
    r = np.random.default_rng(3)
    logits = r.standard_normal((M, V)).astype(np.float32)
    logits[0, :] = -np.inf
    logits[1, 5] = np.nan
    logits[2, 2048:4096] = -np.inf
    logits[3, V - 1] = 200.0
    logits[4, 0] = 200.0
    seq = np.zeros((M, 4), np.int32)
    lens = np.arange(1, M + 1)
    for seed in (1, 2, 3):
        tok, _ = run_sample(logits, seq, lens, seed=seed, probs=False, ws=True)
        one, _ = run_sample(logits, seq, lens, seed=seed, probs=False, ws=False)
        assert tok[0] == 0 and tok[1] == 0 and tok[3] == V - 1 and tok[4] == 0
        assert not 2048 <= tok[2] < 4096
        np.testing.assert_array_equal(tok[[0, 1, 3, 4]], one[[0, 1, 3, 4]])
        want = so.sample_filter(logits[2].astype(np.float64), 1.0)
        u = so.splitmix_uniform(seed, 2, 3)
        if np.abs(np.cumsum(want) - u).min() >= 1e-5:
            assert tok[2] == so.sample_draw(want, u) == one[2]


def test_split_draws_follow_the_distribution(gpu_ctx):
    """Many rows with the same logits and different positions, the mass
    spread over entries of different slices: the split path's draw
    frequencies follow the softmax (the slices are weighted correctly)."""
    banner("split sample frequencies")
    V, M = 8192, 3000
    r = np.random.default_rng(11)
    row = np.full(V, -30.0, np.float32)
    hot = np.array([3, 2047, 2048, 4000, 4095, 6000, 8191])
    row[hot] = r.standard_normal(len(hot)).astype(np.float32)
    logits = np.tile(row, (M, 1))
    seq = np.zeros((M, 1), np.int32)
    lens = np.ones(M, np.int32)
    tok, _ = run_sample(logits, seq, lens, T=1.0, probs=False, ws=True, seed=13)
    want = so.sample_filter(row.astype(np.float64), 1.0)
    freq = np.bincount(tok, minlength=V) / M
    assert np.isin(tok, hot).all()
    assert np.abs(freq - want).max() < 0.03
