"""CPU oracle for the KV-cache hot path.

TEST INFRASTRUCTURE ONLY. This module restates the reference's algorithm in
float64 numpy so that the HIP kernels can be checked against it. Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import it, and
only as the checker or the timed CPU baseline. The product path never calls it.

Reference (s-i-e-v-e/llm-experiments, paths relative to simple-llm/src/):
  * cache layout and append:  gpu/gpu_kernels.py:2784-2796 (update kernel),
    gpu/gpu_kv_cache.py:113-186 (kv_cache_update: checks, position rule)
  * decode attention:         gpu/gpu_kernels.py:2846-2936 (scores * 1/sqrt(D),
    max from -1e10, exp(s - max), divide by the sum, weighted sum of V), and
    the test's closed form gpu_test.py:2329-2364
  * causal flash attention:   gpu/gpu_kernels.py:631-768 (mask kv_pos <= q_pos,
    online softmax, O / max(l, 1e-8), L = l, M = m) and the test's closed form
    gpu_test.py:776-810
  * flash attention backward: gpu/gpu_kernels.py:2038-2455 (P from the saved
    L and M, D = rowsum(dO * O), dS = P * (dP - D), dQ = scale dS K,
    dK = scale dS^T Q, dV = P^T dO; partials per Q block, then summed)

How each function is pinned (tests/test_oracle.py):
  cache_offset / append      closed-form offsets over every element of small
                             caches; the reference test's length invariants
  bf16_round                 torch.Tensor.to(torch.bfloat16) on random data
                             and on the special values (ties, inf, nan, denormals)
  decode_attention           torch.nn.functional.scaled_dot_product_attention
                             (float64), the seed-42 golden fixture, closed-form
                             special cases (one token, equal keys, dominant key,
                             permutation and shift invariance)
  prefill_attention          scaled_dot_product_attention with an explicit
                             prefix-offset causal mask; brute-force loops
  flash_attention            the seed-42 golden fixture (7 reference configs);
                             its L and M statistics by direct sums
  paged_gather               contiguous equality against direct scatter
  flash_attention_backward   the seed-42 golden fixture of the reference's
                             backward test (torch float64 autograd); central
                             finite differences of sum(O * dO); the
                             reference's stage-1/stage-2 split (per-Q-block
                             partials summed) restated by loops
"""
from __future__ import annotations

import numpy as np

# ---------------------------------------------------------------------------
# bf16 storage
# ---------------------------------------------------------------------------


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns (uint16), round to nearest even; NaN -> quiet NaN."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    quiet = (u >> 16) | 0x0040
    return np.where(nan, quiet, rounded).astype(np.uint16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Value of x after a store to bf16 and a load back (as float32)."""
    return bf16_to_f32(bf16_bits(x))


def storage_round(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype in ("bf16", "bfloat16"):
        return bf16_round(x)
    if dtype in ("fp32", "float32"):
        return np.asarray(x, dtype=np.float32)
    raise ValueError(f"unknown storage dtype {dtype}")


# ---------------------------------------------------------------------------
# Cache layout and append
# ---------------------------------------------------------------------------


def cache_offset(b: int, t: int, h: int, d: int, T_cap: int, H: int, D: int) -> int:
    """Flat element offset of (b, t, h, d) in a [B*T_cap, H*D] cache buffer.

    Follows gpu/gpu_kernels.py:2791-2793: batch*max_seq_len*E + pos*E + dim,
    with dim = h*D + d (E = H*D).
    """
    E = H * D
    return b * T_cap * E + t * E + h * D + d


def append(k_cache: np.ndarray, v_cache: np.ndarray, k_new: np.ndarray, v_new: np.ndarray,
           lens: np.ndarray, dtype: str = "fp32") -> np.ndarray:
    """One-token append into 4-D caches [B, T_cap, H, D] (modified in place).

    k_new, v_new: [B, H, D]. Sequence b is written at position lens[b] unless
    lens[b] >= T_cap (full: skipped). Returns the new lens (lens + 1 where
    written). Mirrors gpu/gpu_kernels.py:2784-2796 with a per-sequence position.
    """
    B, T_cap = k_cache.shape[:2]
    lens = np.asarray(lens, dtype=np.int64).copy()
    kr = storage_round(k_new, dtype)
    vr = storage_round(v_new, dtype)
    for b in range(B):
        p = int(lens[b])
        if p < 0 or p >= T_cap:
            continue
        k_cache[b, p] = kr[b]
        v_cache[b, p] = vr[b]
        lens[b] = p + 1
    return lens


def append_chunk(k_cache, v_cache, k_new, v_new, lens, n_new=None, dtype="fp32"):
    """Chunk append: row i < n_new[b] of k_new[b] ([B, C, H, D]) goes to lens[b] + i."""
    B, T_cap = k_cache.shape[:2]
    C = k_new.shape[1]
    kr = storage_round(k_new, dtype)
    vr = storage_round(v_new, dtype)
    for b in range(B):
        n = C if n_new is None else min(int(n_new[b]), C)
        for i in range(n):
            p = int(lens[b]) + i
            if p < 0 or p >= T_cap:
                break
            k_cache[b, p] = kr[b, i]
            v_cache[b, p] = vr[b, i]


def paged_gather(pool: np.ndarray, block_table: np.ndarray, lens: np.ndarray,
                 block_size: int, T_out: int) -> np.ndarray:
    """Gather a paged pool [n_blocks*block_size, H, D] into [B, T_out, H, D].

    Token t of sequence b lives in block block_table[b, t // block_size],
    row t % block_size. Positions >= lens[b] are zero.
    """
    B = block_table.shape[0]
    out = np.zeros((B, T_out) + pool.shape[1:], dtype=pool.dtype)
    for b in range(B):
        for t in range(int(lens[b])):
            blk = int(block_table[b, t // block_size])
            out[b, t] = pool[blk * block_size + t % block_size]
    return out


# ---------------------------------------------------------------------------
# Attention
# ---------------------------------------------------------------------------


def _softmax_rows(s: np.ndarray) -> np.ndarray:
    m = np.max(s, axis=-1, keepdims=True)
    e = np.exp(s - m)
    return e / np.sum(e, axis=-1, keepdims=True)


def decode_attention(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                     lens: np.ndarray, scale: float | None = None) -> np.ndarray:
    """Single-query attention over the filled prefix, float64.

    q: [B, Hq, D]; caches [B, T_cap, Hkv, D]; query head h reads kv head
    h // (Hq // Hkv). Sequence b attends positions [0, lens[b]). lens[b] == 0
    gives a zero row. Follows gpu/gpu_kernels.py:2846-2936: s = scale * q.k,
    p = exp(s - max) / sum, o = sum p V.
    """
    B, Hq, D = q.shape
    Hkv = k_cache.shape[2]
    G = Hq // Hkv
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    out = np.zeros((B, Hq, D), dtype=np.float64)
    for b in range(B):
        L = int(lens[b])
        if L <= 0:
            continue
        K = np.asarray(k_cache[b, :L], dtype=np.float64)  # [L, Hkv, D]
        V = np.asarray(v_cache[b, :L], dtype=np.float64)
        for h in range(Hq):
            hk = h // G
            s = (K[:, hk, :] @ np.asarray(q[b, h], dtype=np.float64)) * scale
            p = _softmax_rows(s[None, :])[0]
            out[b, h] = p @ V[:, hk, :]
    return out


def prefill_attention(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                      start: np.ndarray, q_lens: np.ndarray | None = None,
                      scale: float | None = None, with_stats: bool = False):
    """Causal attention of a chunk of queries over the cache, float64.

    q: [B, C, Hq, D]. Query row i of sequence b sits at position start[b] + i
    and attends cache positions [0, start[b] + i] (the chunk's own K/V must
    already be in the cache). Rows i >= q_lens[b] are left zero. With prefix
    start = 0 this is the reference's causal flash attention
    (gpu/gpu_kernels.py:695-701 mask kv_pos <= q_pos).

    with_stats: also return M (row max of the scaled scores) and L (sum of
    exp(s - M)), the statistics the reference kernel writes (:762-768).
    """
    B, C, Hq, D = q.shape
    Hkv = k_cache.shape[2]
    G = Hq // Hkv
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    out = np.zeros((B, C, Hq, D), dtype=np.float64)
    M = np.zeros((B, C, Hq), dtype=np.float64)
    Ls = np.zeros((B, C, Hq), dtype=np.float64)
    for b in range(B):
        n = C if q_lens is None else int(q_lens[b])
        for i in range(n):
            L = int(start[b]) + i + 1
            K = np.asarray(k_cache[b, :L], dtype=np.float64)
            V = np.asarray(v_cache[b, :L], dtype=np.float64)
            for h in range(Hq):
                hk = h // G
                s = (K[:, hk, :] @ np.asarray(q[b, i, h], dtype=np.float64)) * scale
                m = s.max()
                e = np.exp(s - m)
                out[b, i, h] = (e @ V[:, hk, :]) / e.sum()
                M[b, i, h] = m
                Ls[b, i, h] = e.sum()
    if with_stats:
        return out, M, Ls
    return out


def flash_attention(Q: np.ndarray, K: np.ndarray, V: np.ndarray, batch_size: int, seq_len: int,
                    n_heads: int, head_dim: int):
    """Reference flash_attention contract on [B*T, H*D] buffers (float64).

    Returns O [B*T, H*D], L [B*T*H] (softmax denominators) and M [B*T*H] (row
    max of the scaled scores), indexed as the reference kernel writes them
    (gpu/gpu_kernels.py:747-768: stats offset = b*T*H + t*H + h).
    """
    B, T, H, D = batch_size, seq_len, n_heads, head_dim
    q = np.asarray(Q, dtype=np.float64).reshape(B, T, H, D)
    k = np.asarray(K, dtype=np.float64).reshape(B, T, H, D)
    v = np.asarray(V, dtype=np.float64).reshape(B, T, H, D)
    o, m, l = prefill_attention(q, k, v, np.zeros(B, dtype=np.int64), None, None, True)
    return o.reshape(B * T, H * D), l.reshape(-1), m.reshape(-1)


def flash_attention_backward(Q, K, V, O, L, M, dO, batch_size: int, seq_len: int, n_heads: int,
                             head_dim: int):
    """Reference flash_attention_backward contract on [B*T, H*D] buffers (float64).

    Follows the stage-1 kernel (gpu/gpu_kernels.py:2161-2340): P is rebuilt
    from the forward's statistics, P = exp(scale * q.k - M) / L for
    key <= query and 0 otherwise; D = rowsum(dO * O) uses the given O;
    dP = dO V^T; dS = P * (dP - D); dQ = scale * dS K; the partial
    dK = scale * dS^T Q and dV = P^T dO of each Q block are summed by stage 2
    (:2378-2455), which is the plain sum over all queries.
    Returns dQ, dK, dV as [B*T, H*D] float64.
    """
    B, T, H, D = batch_size, seq_len, n_heads, head_dim
    scale = 1.0 / np.sqrt(D)

    def heads(x):
        return np.asarray(x, dtype=np.float64).reshape(B, T, H, D).transpose(0, 2, 1, 3)

    q, k, v, o, do = heads(Q), heads(K), heads(V), heads(O), heads(dO)
    m = np.asarray(M, dtype=np.float64).reshape(B, T, H).transpose(0, 2, 1)[..., None]
    l = np.asarray(L, dtype=np.float64).reshape(B, T, H).transpose(0, 2, 1)[..., None]
    mask = np.tril(np.ones((T, T), dtype=bool))
    s = np.einsum("bhqd,bhkd->bhqk", q, k) * scale
    p = np.where(mask, np.exp(np.where(mask, s, 0.0) - m) / l, 0.0)
    dlt = (do * o).sum(-1, keepdims=True)
    dp = np.einsum("bhqd,bhkd->bhqk", do, v)
    ds = p * (dp - dlt)
    dq = np.einsum("bhqk,bhkd->bhqd", ds, k) * scale
    dk = np.einsum("bhqk,bhqd->bhkd", ds, q) * scale
    dv = np.einsum("bhqk,bhqd->bhkd", p, do)

    def flat(x):
        return x.transpose(0, 2, 1, 3).reshape(B * T, H * D)

    return flat(dq), flat(dk), flat(dv)
