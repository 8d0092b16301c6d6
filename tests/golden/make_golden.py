"""Regenerate the golden fixtures of the KV-cache hot path.

The reference stores no golden files; its tests draw inputs from numpy's
legacy seed-42 stream and compute the expected output on the fly. This
script replays those input protocols exactly and computes the expected
outputs with torch.nn.functional.scaled_dot_product_attention in float64,
a library routine independent of oracle/.

  kv_kat_seed42.npz     simple-llm/src/gpu_test.py:2207-2317
                        (test_kv_cache_operations: B=2, T_cap=128, 2 layers,
                        H=4, D=64; five appended (k, v) steps, then Q)
  flash_kat_seed42.npz  simple-llm/src/gpu_test.py:747-810
                        (test_flash_attention: causal, seed 42 per config).
                        The "Medium" config (8, 32, 8, 64) is left out to keep
                        the file small; tests regenerate it from the seed.
  flash_bwd_kat_seed42.npz
                        simple-llm/src/gpu_test.py:871-1060
                        (test_flash_attention_backward: Q, K, V, grad_out
                        drawn in that order after seed 42; expected
                        gradients by torch float64 autograd of the test's
                        causal attention with its -1e10 mask, in place of
                        jax.vjp; O, L, M of the forward stored alongside)

Usage: python tests/golden/make_golden.py
"""
from __future__ import annotations

import os

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))

# (batch, seq_len, n_heads, head_dim, description), gpu_test.py:747-756
FLASH_CONFIGS = [
    (2, 8, 2, 16, "Tiny: 8d"),
    (2, 4, 2, 16, "Tiny (debug)"),
    (2, 16, 2, 16, "Small: 16d"),
    (4, 16, 4, 64, "Small"),
    (8, 32, 8, 64, "Medium"),
    (4, 32, 4, 32, "Medium: 32d"),
    (2, 64, 2, 32, "Large: 64seq x 32d"),
]
FLASH_STORED = [0, 1, 2, 3, 5, 6]
# (batch, seq_len, n_heads, head_dim, description), gpu_test.py:874-877
FLASH_BWD_CONFIGS = [(2, 8, 2, 16, "Small"), (4, 16, 4, 32, "Medium")]


def kv_kat_inputs():
    """Inputs of test_kv_cache_operations in the reference's draw order."""
    batch_size, n_heads, head_dim = 2, 4, 64
    np.random.seed(42)
    ks, vs = [], []
    for _ in range(5):
        ks.append(np.random.randn(batch_size, 1, n_heads, head_dim).astype(np.float32))
        vs.append(np.random.randn(batch_size, 1, n_heads, head_dim).astype(np.float32))
    q = np.random.randn(batch_size, 1, n_heads, head_dim).astype(np.float32)
    # [steps, B, H, D] and [B, H, D]
    return np.stack([k[:, 0] for k in ks]), np.stack([v[:, 0] for v in vs]), q[:, 0]


def flash_inputs(batch, seq_len, n_heads, head_dim):
    """Q, K, V of test_flash_attention for one config ([B, T, H*D] fp32)."""
    np.random.seed(42)
    Q = np.random.randn(batch, seq_len, n_heads * head_dim).astype(np.float32)
    K = np.random.randn(batch, seq_len, n_heads * head_dim).astype(np.float32)
    V = np.random.randn(batch, seq_len, n_heads * head_dim).astype(np.float32)
    return Q, K, V


def sdpa64(q, k, v, causal):
    """[B, H, Tq, D] float64 attention via torch's library routine."""
    return F.scaled_dot_product_attention(torch.from_numpy(q), torch.from_numpy(k),
                                          torch.from_numpy(v), is_causal=causal).numpy()


def flash_expected(Q, K, V, batch, seq_len, n_heads, head_dim):
    def heads(x):
        return x.astype(np.float64).reshape(batch, seq_len, n_heads, head_dim).transpose(0, 2, 1, 3)
    q, k, v = heads(Q), heads(K), heads(V)
    o = sdpa64(q, k, v, causal=True).transpose(0, 2, 1, 3).reshape(batch * seq_len, -1)
    # row statistics of the scaled, causally masked scores
    s = np.einsum("bhqd,bhkd->bhqk", q, k) / np.sqrt(head_dim)
    mask = np.tril(np.ones((seq_len, seq_len), dtype=bool))
    s = np.where(mask, s, -np.inf)
    m = s.max(-1)
    l = np.exp(s - m[..., None]).sum(-1)
    # stats index b*T*H + t*H + h (gpu_kernels.py:762-768)
    return o, l.transpose(0, 2, 1).reshape(-1), m.transpose(0, 2, 1).reshape(-1)


def flash_bwd_inputs(batch, seq_len, n_heads, head_dim):
    """Q, K, V, grad_out of test_flash_attention_backward ([B, T, H*D] fp32)."""
    np.random.seed(42)
    return tuple(np.random.randn(batch, seq_len, n_heads * head_dim).astype(np.float32)
                 for _ in range(4))


def flash_bwd_expected(Q, K, V, dO, batch, seq_len, n_heads, head_dim):
    """dQ, dK, dV [B*T, H*D] float64: torch autograd of gpu_test.py:899-915."""
    def heads(x):
        return torch.tensor(x, dtype=torch.float64).reshape(
            batch, seq_len, n_heads, head_dim).transpose(1, 2).requires_grad_(True)
    q, k, v = heads(Q), heads(K), heads(V)
    s = (q @ k.transpose(-1, -2)) / np.sqrt(float(head_dim))
    mask = torch.tril(torch.ones(seq_len, seq_len, dtype=torch.bool))
    s = torch.where(mask, s, torch.tensor(-1e10, dtype=torch.float64))
    o = torch.softmax(s, -1) @ v
    g = torch.tensor(dO, dtype=torch.float64).reshape(batch, seq_len, n_heads,
                                                      head_dim).transpose(1, 2)
    dq, dk, dv = torch.autograd.grad(o, (q, k, v), g)
    return tuple(x.transpose(1, 2).reshape(batch * seq_len, -1).numpy() for x in (dq, dk, dv))


def write_flash_bwd():
    out = {}
    for i, (b, t, h, d, _) in enumerate(FLASH_BWD_CONFIGS):
        Q, K, V, dO = flash_bwd_inputs(b, t, h, d)
        o, l, m = flash_expected(Q, K, V, b, t, h, d)
        dq, dk, dv = flash_bwd_expected(Q, K, V, dO, b, t, h, d)
        out.update({f"o_{i}": o, f"l_{i}": l, f"m_{i}": m, f"dq_{i}": dq, f"dk_{i}": dk,
                    f"dv_{i}": dv})
    out["configs"] = np.array([c[:4] for c in FLASH_BWD_CONFIGS])
    np.savez_compressed(os.path.join(HERE, "flash_bwd_kat_seed42.npz"), **out)


def main():
    k_steps, v_steps, q = kv_kat_inputs()
    # cache holds the 5 steps in order; attention over all of them
    K = k_steps.transpose(1, 2, 0, 3).astype(np.float64)  # [B, H, 5, D]
    V = v_steps.transpose(1, 2, 0, 3).astype(np.float64)
    o = sdpa64(q.astype(np.float64)[:, :, None, :], K, V, causal=False)[:, :, 0, :]
    np.savez_compressed(os.path.join(HERE, "kv_kat_seed42.npz"), k_steps=k_steps,
                        v_steps=v_steps, q=q, expected_o=o,
                        config=np.array([2, 128, 2, 4, 64]))  # B, T_cap, layers, H, D

    out = {}
    for i in FLASH_STORED:
        b, t, h, d, _ = FLASH_CONFIGS[i]
        Q, Kf, Vf = flash_inputs(b, t, h, d)
        o, l, m = flash_expected(Q, Kf, Vf, b, t, h, d)
        out[f"o_{i}"], out[f"l_{i}"], out[f"m_{i}"] = o, l, m
    out["configs"] = np.array([c[:4] for c in FLASH_CONFIGS])
    out["stored"] = np.array(FLASH_STORED)
    np.savez_compressed(os.path.join(HERE, "flash_kat_seed42.npz"), **out)
    write_flash_bwd()
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
