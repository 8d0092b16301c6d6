"""Pins the CPU oracle (oracle/) before it is trusted as the checker.

Each oracle function is checked against something it was not derived from:
the seed-42 golden fixtures (expected values from torch's float64
scaled_dot_product_attention), torch's bf16 conversion, closed forms and
invariants that a dropped term, a wrong index or a transposed operand would
break. CPU only.
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import GOLDEN
from oracle import c_oracle
from oracle import kv_oracle as ko

rng = np.random.default_rng(1234)


# ---------------------------------------------------------------------------
# bf16 storage
# ---------------------------------------------------------------------------


def _torch_bf16_bits(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def test_bf16_round_matches_torch_random():
    x = (rng.standard_normal(200_000) * np.exp(rng.uniform(-30, 30, 200_000))).astype(np.float32)
    np.testing.assert_array_equal(ko.bf16_bits(x), _torch_bf16_bits(x))


def test_bf16_round_special_values():
    bits = np.array([
        0x00000000, 0x80000000,  # +-0
        0x7F800000, 0xFF800000,  # +-inf
        0x3F808000,  # 1 + 2^-8: tie, rounds down to even 0x3F80
        0x3F818000,  # tie, rounds up to even 0x3F82
        0x3F808001,  # just above the tie: up
        0x00000001, 0x807FFFFF,  # denormals
        0x7F7FFFFF,  # max finite: rounds to inf
    ], dtype=np.uint32)
    x = bits.view(np.float32)
    np.testing.assert_array_equal(ko.bf16_bits(x), _torch_bf16_bits(x))
    assert ko.bf16_bits(np.array([0x3F808000], np.uint32).view(np.float32))[0] == 0x3F80
    assert ko.bf16_bits(np.array([0x3F818000], np.uint32).view(np.float32))[0] == 0x3F82
    nan = np.array([np.nan], dtype=np.float32)
    assert np.isnan(ko.bf16_round(nan)[0])


# ---------------------------------------------------------------------------
# cache layout and append
# ---------------------------------------------------------------------------


def test_cache_offset_is_row_major_b_t_h_d():
    B, T, H, D = 3, 5, 4, 8
    idx = np.indices((B, T, H, D)).reshape(4, -1).T
    offs = np.array([ko.cache_offset(b, t, h, d, T, H, D) for b, t, h, d in idx])
    np.testing.assert_array_equal(offs, np.arange(B * T * H * D))
    # the reference's formula: batch*max_seq*E + pos*E + dim (gpu_kernels.py:2791-2793)
    E = H * D
    assert ko.cache_offset(2, 3, 1, 5, T, H, D) == 2 * T * E + 3 * E + 1 * D + 5


def test_append_positions_and_lengths():
    """The reference test's invariants (gpu_test.py:2241-2306) plus full-cache skip."""
    B, T, H, D = 2, 4, 2, 8
    kc = np.zeros((B, T, H, D), np.float32)
    vc = np.zeros_like(kc)
    lens = np.zeros(B, np.int64)
    steps = []
    for step in range(1, T + 2):
        k = rng.standard_normal((B, H, D)).astype(np.float32)
        v = rng.standard_normal((B, H, D)).astype(np.float32)
        lens = ko.append(kc, vc, k, v, lens)
        steps.append((k, v))
        assert list(lens) == [min(step, T)] * B
    flat = kc.reshape(-1)
    for t in range(T):
        k, _ = steps[t]
        for b in range(B):
            for h in range(H):
                off = ko.cache_offset(b, t, h, 0, T, H, D)
                np.testing.assert_array_equal(flat[off:off + D], k[b, h])
    # the (T+1)-th append hit a full cache: nothing overwritten
    np.testing.assert_array_equal(kc[:, T - 1], steps[T - 1][0])


def test_append_ragged_and_bf16():
    B, T, H, D = 3, 6, 1, 8
    kc = np.zeros((B, T, H, D), np.float32)
    vc = np.zeros_like(kc)
    lens = np.array([0, 5, 6])
    k = rng.standard_normal((B, H, D)).astype(np.float32)
    new = ko.append(kc, vc, k, -k, lens, dtype="bf16")
    assert list(new) == [1, 6, 6]
    np.testing.assert_array_equal(kc[0, 0], ko.bf16_round(k[0]))
    np.testing.assert_array_equal(kc[1, 5], ko.bf16_round(k[1]))
    assert not kc[2].any()


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
def test_append_chunk_offsets_clamp_and_no_wrap(dtype):
    """append_chunk against two independent statements of the chunk rule:
    (1) the reference's flat offsets (cache_offset) over a [B*T_cap, E] buffer
    pre-filled with a sentinel: row i < n_new[b] lands at position lens[b]+i
    while that is < T_cap, and every other element keeps the sentinel (so no
    row spills into the next sequence's positions); (2) the same rows fed one
    token at a time through append() with the sequences that have no row
    left masked out. Ragged n_new (0, partial, full C, beyond T_cap)."""
    B, T, H, D, C = 4, 10, 2, 4, 6
    lens = np.array([0, 7, 3, 10])
    n_new = np.array([6, 6, 0, 2])  # 7+6 runs past T_cap: rows 7..9 only
    k = rng.standard_normal((B, C, H, D)).astype(np.float32)
    v = rng.standard_normal((B, C, H, D)).astype(np.float32)
    sentinel = np.float32(-777.0)
    kc = np.full((B, T, H, D), sentinel, np.float32)
    vc = np.full_like(kc, sentinel)
    ko.append_chunk(kc, vc, k, v, lens, n_new, dtype=dtype)
    want_k = np.full(B * T * H * D, sentinel, np.float32)
    want_v = np.full_like(want_k, sentinel)
    kr, vr = ko.storage_round(k, dtype), ko.storage_round(v, dtype)
    for b in range(B):
        for i in range(n_new[b]):
            t = lens[b] + i
            if t >= T:
                continue
            for h in range(H):
                for d in range(D):
                    off = ko.cache_offset(b, t, h, d, T, H, D)
                    want_k[off], want_v[off] = kr[b, i, h, d], vr[b, i, h, d]
    np.testing.assert_array_equal(kc.reshape(-1), want_k)
    np.testing.assert_array_equal(vc.reshape(-1), want_v)
    # (2) token by token through append()
    k1 = np.full((B, T, H, D), sentinel, np.float32)
    v1 = np.full_like(k1, sentinel)
    cur = lens.copy()
    for i in range(C):
        live = i < n_new
        step_lens = np.where(live, cur, T)  # a sequence without a row i: "full", skipped
        out = ko.append(k1, v1, k[:, i], v[:, i], step_lens, dtype=dtype)
        cur = np.where(live, out, cur)
    np.testing.assert_array_equal(k1, kc)
    np.testing.assert_array_equal(v1, vc)
    # a planted off-by-one (rows written one position late) is caught
    bad = np.full((B, T, H, D), sentinel, np.float32)
    ko.append_chunk(bad, bad.copy(), k, v, lens + 1, n_new, dtype=dtype)
    assert not np.array_equal(bad, kc)


def test_paged_gather_matches_direct_scatter():
    B, H, D, bs, max_blocks = 3, 2, 8, 4, 5
    n_blocks = B * max_blocks
    table = rng.permutation(n_blocks).reshape(B, max_blocks)
    lens = np.array([17, 3, 20])
    contiguous = rng.standard_normal((B, max_blocks * bs, H, D)).astype(np.float32)
    pool = np.zeros((n_blocks * bs, H, D), np.float32)
    for b in range(B):
        for t in range(lens[b]):
            pool[table[b, t // bs] * bs + t % bs] = contiguous[b, t]
    got = ko.paged_gather(pool, table, lens, bs, max_blocks * bs)
    for b in range(B):
        np.testing.assert_array_equal(got[b, :lens[b]], contiguous[b, :lens[b]])
        assert not got[b, lens[b]:].any()


# ---------------------------------------------------------------------------
# decode attention
# ---------------------------------------------------------------------------


def _sdpa_decode(q, kc, vc, lens):
    """Library float64 attention per sequence (GQA by repeating kv heads)."""
    B, Hq, D = q.shape
    G = Hq // kc.shape[2]
    out = np.zeros((B, Hq, D))
    for b in range(B):
        L = int(lens[b])
        if L == 0:
            continue
        k = torch.from_numpy(kc[b, :L].astype(np.float64)).permute(1, 0, 2)
        v = torch.from_numpy(vc[b, :L].astype(np.float64)).permute(1, 0, 2)
        k = k.repeat_interleave(G, 0)
        v = v.repeat_interleave(G, 0)
        qq = torch.from_numpy(q[b].astype(np.float64))[:, None, :]
        out[b] = F.scaled_dot_product_attention(qq, k, v)[:, 0].numpy()
    return out


@pytest.mark.parametrize("B,T,Hq,Hkv,D", [(2, 40, 4, 4, 64), (3, 33, 8, 2, 128), (1, 7, 4, 1, 64)])
def test_decode_attention_matches_sdpa(B, T, Hq, Hkv, D):
    q = rng.standard_normal((B, Hq, D)).astype(np.float32)
    kc = rng.standard_normal((B, T, Hkv, D)).astype(np.float32)
    vc = rng.standard_normal((B, T, Hkv, D)).astype(np.float32)
    lens = rng.integers(0, T + 1, B)
    lens[0] = T
    got = ko.decode_attention(q, kc, vc, lens)
    np.testing.assert_allclose(got, _sdpa_decode(q, kc, vc, lens), rtol=1e-12, atol=1e-13)


def test_decode_attention_golden_kat():
    """Seed-42 protocol of test_kv_cache_operations (gpu_test.py:2207-2384)."""
    z = np.load(os.path.join(GOLDEN, "kv_kat_seed42.npz"))
    k_steps, v_steps, q = z["k_steps"], z["v_steps"], z["q"]
    B, T_cap, _, H, D = z["config"]
    kc = np.zeros((B, T_cap, H, D), np.float32)
    vc = np.zeros_like(kc)
    lens = np.zeros(B, np.int64)
    for s in range(k_steps.shape[0]):
        lens = ko.append(kc, vc, k_steps[s], v_steps[s], lens)
    assert list(lens) == [5, 5]
    got = ko.decode_attention(q, kc, vc, lens)
    np.testing.assert_allclose(got, z["expected_o"], rtol=1e-12, atol=1e-14)


def test_decode_attention_special_cases():
    B, T, H, D = 2, 16, 2, 64
    q = rng.standard_normal((B, H, D)).astype(np.float32)
    kc = rng.standard_normal((B, T, H, D)).astype(np.float32)
    vc = rng.standard_normal((B, T, H, D)).astype(np.float32)
    # one token: the output is that token's value row
    out = ko.decode_attention(q, kc, vc, np.array([1, 1]))
    np.testing.assert_allclose(out, vc[:, 0], rtol=0, atol=1e-15)
    # equal keys: uniform weights, the output is the mean of V
    ke = np.repeat(kc[:, :1], T, axis=1)
    out = ko.decode_attention(q, ke, vc, np.array([T, 9]))
    np.testing.assert_allclose(out[0], vc[0].astype(np.float64).mean(0), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(out[1], vc[1, :9].astype(np.float64).mean(0), rtol=1e-12,
                               atol=1e-12)
    # one dominant key: the output is (almost) its value row
    kd = kc.copy()
    kd[:, 5] = q * 50.0
    out = ko.decode_attention(q, kd, vc, np.array([T, T]))
    np.testing.assert_allclose(out, vc[:, 5], atol=1e-6)
    # permuting the (k, v) pairs leaves the output unchanged
    perm = rng.permutation(T)
    out1 = ko.decode_attention(q, kc, vc, np.array([T, T]))
    out2 = ko.decode_attention(q, kc[:, perm], vc[:, perm], np.array([T, T]))
    np.testing.assert_allclose(out1, out2, rtol=1e-12, atol=1e-13)
    # adding the same vector c to every key shifts all scores of a head by q.c
    c = rng.standard_normal((1, 1, H, D)).astype(np.float32)
    out3 = ko.decode_attention(q, (kc.astype(np.float64) + c), vc, np.array([T, T]))
    np.testing.assert_allclose(out1, out3, rtol=1e-9, atol=1e-11)
    # an empty sequence gives a zero row
    assert not ko.decode_attention(q, kc, vc, np.array([0, 3]))[0].any()


def test_c_oracle_matches_numpy_oracle():
    B, T, Hq, Hkv, D = 3, 300, 8, 2, 128
    q = rng.standard_normal((B, Hq, D)).astype(np.float32)
    kc = rng.standard_normal((B, T, Hkv, D)).astype(np.float32)
    vc = rng.standard_normal((B, T, Hkv, D)).astype(np.float32)
    lens = np.array([300, 1, 123])
    want = ko.decode_attention(q, kc, vc, lens)
    got = c_oracle.decode_attn(q, kc, vc, lens, cache_bf16=False)
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5)
    # bf16 storage: both read the same rounded values
    kb, vb = ko.bf16_bits(kc), ko.bf16_bits(vc)
    want = ko.decode_attention(q, ko.bf16_to_f32(kb), ko.bf16_to_f32(vb), lens)
    got = c_oracle.decode_attn(q, kb, vb, lens, cache_bf16=True)
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5)


# ---------------------------------------------------------------------------
# prefill and flash attention
# ---------------------------------------------------------------------------


def test_prefill_attention_matches_masked_sdpa():
    B, C, Hq, Hkv, D, T = 2, 7, 4, 2, 32, 30
    start = np.array([0, 11])
    q = rng.standard_normal((B, C, Hq, D)).astype(np.float32)
    kc = rng.standard_normal((B, T, Hkv, D)).astype(np.float32)
    vc = rng.standard_normal((B, T, Hkv, D)).astype(np.float32)
    got = ko.prefill_attention(q, kc, vc, start)
    G = Hq // Hkv
    for b in range(B):
        L = start[b] + C
        k = torch.from_numpy(kc[b, :L].astype(np.float64)).permute(1, 0, 2).repeat_interleave(G, 0)
        v = torch.from_numpy(vc[b, :L].astype(np.float64)).permute(1, 0, 2).repeat_interleave(G, 0)
        qq = torch.from_numpy(q[b].astype(np.float64)).permute(1, 0, 2)
        # query i at position start+i sees keys [0, start+i]
        mask = torch.arange(L)[None, :] <= (start[b] + torch.arange(C))[:, None]
        want = F.scaled_dot_product_attention(qq, k, v, attn_mask=mask).permute(1, 0, 2)
        np.testing.assert_allclose(got[b], want.numpy(), rtol=1e-12, atol=1e-13)


def test_prefill_attention_ragged_rows_and_stats():
    B, C, H, D, T = 2, 5, 2, 16, 12
    q = rng.standard_normal((B, C, H, D)).astype(np.float32)
    kc = rng.standard_normal((B, T, H, D)).astype(np.float32)
    vc = rng.standard_normal((B, T, H, D)).astype(np.float32)
    start = np.array([3, 0])
    qlens = np.array([5, 2])
    o, M, L = ko.prefill_attention(q, kc, vc, start, qlens, with_stats=True)
    assert not o[1, 2:].any()
    # stats by brute force for one row: position start+i = 3+2 = 5
    s = kc[0, :6, 1].astype(np.float64) @ q[0, 2, 1].astype(np.float64) / np.sqrt(D)
    assert M[0, 2, 1] == pytest.approx(s.max(), rel=1e-12)
    assert L[0, 2, 1] == pytest.approx(np.exp(s - s.max()).sum(), rel=1e-12)
    # a row's output equals decode attention at that length
    dec = ko.decode_attention(q[:, 2], kc, vc, start + 3)
    np.testing.assert_allclose(o[0, 2], dec[0], rtol=1e-12, atol=1e-14)


def test_flash_attention_golden_kat():
    """Seed-42 protocol of test_flash_attention (gpu_test.py:747-810)."""
    import make_golden as mg

    z = np.load(os.path.join(GOLDEN, "flash_kat_seed42.npz"))
    for i in z["stored"]:
        b, t, h, d = z["configs"][i]
        Q, K, V = mg.flash_inputs(b, t, h, d)
        O, L, M = ko.flash_attention(Q.reshape(b * t, -1), K.reshape(b * t, -1),
                                     V.reshape(b * t, -1), b, t, h, d)
        np.testing.assert_allclose(O, z[f"o_{i}"], rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(L, z[f"l_{i}"], rtol=1e-10)
        np.testing.assert_allclose(M, z[f"m_{i}"], rtol=1e-10, atol=1e-12)
