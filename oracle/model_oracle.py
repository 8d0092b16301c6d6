"""CPU oracle of the reference model around the KV-cache path.

TEST INFRASTRUCTURE ONLY. A float64 numpy restatement of the JAX model that
the reference's CPU path runs, used by tests/ as the checker and by
bench.py's cpu_baseline leg (as the reference's generate loop). The product
(llm-experiments_amd/) never imports it.

Reference (s-i-e-v-e/llm-experiments, paths relative to simple-llm/src/):
  positional_encoding   jax_backend.py:25-33  (sin of the even-index angles,
                        then cos of the odd-index angles, concatenated)
  layer_norm            jax_backend.py:78-82  (eps 1e-5, population variance)
  attention             jax_backend.py:97-122 (x.W projections without bias,
                        scores / sqrt(D), additive -1e9 causal mask, softmax)
  feed_forward          jax_backend.py:125-129 (jax.nn.gelu default = tanh form)
  transformer_block     jax_backend.py:132-140 (pre-LN, two residuals)
  forward               jax_backend.py:143-148 (embedding + PE, tied logits
                        x . embedding^T, no final LayerNorm)
  greedy sampling       jax_backend.py:466-469 (argmax, first index on ties)
  generate_text         generate.py:8-71 (left-padded window of context_size,
                        full forward per token, last row's logits)

How each function is pinned (tests/test_model_oracle.py):
  positional_encoding   closed-form values (position 0, a hand-computed row)
                        and the concatenated (not interleaved) layout
  layer_norm            torch.nn.functional.layer_norm in float64
  gelu_tanh             torch.nn.functional.gelu(approximate="tanh")
  forward               a float64 torch model built from library routines
                        (F.layer_norm, F.gelu, F.scaled_dot_product_attention
                        with is_causal) on the same weights; causality
  decode_step           equals forward's rows (a different algorithm: the
                        per-token cached recurrence the GPU path uses)
  reference_generate    the left-padding rule of generate.py:31-36 observed
                        through a spy forward, while the window is not full
                        and once the sequence is longer than the window
  torch_forward_fp32    equals forward to float32 accuracy
  TorchCachedDecoder    its step logits equal decode_step's (the float64
                        cached recurrence) to float32 accuracy
"""
from __future__ import annotations

import numpy as np

LAYER_FIELDS = ("attn_wq", "attn_wk", "attn_wv", "attn_wo", "ff_w1", "ff_b1", "ff_w2",
                "ff_b2", "ln_gamma1", "ln_beta1", "ln_gamma2", "ln_beta2")


def positional_encoding(seq_len: int, dim: int) -> np.ndarray:
    """[seq_len, dim] float64; jax_backend.py:25-33."""
    pos = np.arange(seq_len, dtype=np.float64)[:, None]
    i = np.arange(dim)[None, :]
    angle_rates = 1.0 / (10000.0 ** (2 * (i // 2) / dim))
    ang = pos * angle_rates
    return np.concatenate([np.sin(ang[:, 0::2]), np.cos(ang[:, 1::2])], axis=-1)


def layer_norm(x, gamma, beta, eps=1e-5):
    x = np.asarray(x, np.float64)
    mean = x.mean(-1, keepdims=True)
    var = ((x - mean) ** 2).mean(-1, keepdims=True)
    return (x - mean) / np.sqrt(var + eps) * gamma + beta


def gelu_tanh(x):
    x = np.asarray(x, np.float64)
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


def _f64(params):
    layers = [{k: np.asarray(lp[k], np.float64) for k in LAYER_FIELDS}
              for lp in params["layers"]]
    return (np.asarray(params["embedding"], np.float64),
            np.asarray(params["pos_encoding"], np.float64), layers)


def forward(params: dict, tokens: np.ndarray, n_heads: int, last: int | None = None) -> np.ndarray:
    """Full causal forward of [B, T] token ids -> logits [B, T, V] (float64).

    params: {"embedding": [V, d], "pos_encoding": [ctx, d], "layers": [dict of
    LAYER_FIELDS]} with the reference's shapes (W as [in, out]). last: only
    the logits of the last `last` positions, [B, last, V] (the same rows).
    """
    E, PE, layers = _f64(params)
    tokens = np.asarray(tokens)
    B, T = tokens.shape
    d = E.shape[1]
    D = d // n_heads
    x = E[tokens] + PE[None, :T]
    mask = np.triu(np.ones((T, T)), k=1) * -1e9
    for lp in layers:
        h = layer_norm(x, lp["ln_gamma1"], lp["ln_beta1"])
        q = (h @ lp["attn_wq"]).reshape(B, T, n_heads, D).transpose(0, 2, 1, 3)
        k = (h @ lp["attn_wk"]).reshape(B, T, n_heads, D).transpose(0, 2, 1, 3)
        v = (h @ lp["attn_wv"]).reshape(B, T, n_heads, D).transpose(0, 2, 1, 3)
        s = q @ k.transpose(0, 1, 3, 2) / np.sqrt(D) + mask
        s = s - s.max(-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(-1, keepdims=True)
        a = (p @ v).transpose(0, 2, 1, 3).reshape(B, T, d)
        x = x + a @ lp["attn_wo"]
        h = layer_norm(x, lp["ln_gamma2"], lp["ln_beta2"])
        f = gelu_tanh(h @ lp["ff_w1"] + lp["ff_b1"])
        x = x + f @ lp["ff_w2"] + lp["ff_b2"]
    if last is not None:
        x = x[:, T - last:]
    return x @ E.T


class DecodeState:
    """Per-sequence K/V of every layer for decode_step (float64)."""

    def __init__(self, n_layers: int, batch: int):
        self.k = [[[] for _ in range(batch)] for _ in range(n_layers)]
        self.v = [[[] for _ in range(batch)] for _ in range(n_layers)]


def decode_step(params: dict, state: DecodeState, tokens, positions, n_heads: int,
                active=None) -> np.ndarray:
    """One token per sequence through every layer with cached K/V: the
    recurrence the GPU path runs. tokens, positions: [B]. Returns logits
    [B, V]. Sequences with active[b] False are skipped (zero logits)."""
    E, PE, layers = _f64(params)
    B = len(tokens)
    d = E.shape[1]
    D = d // n_heads
    out = np.zeros((B, E.shape[0]))
    for b in range(B):
        if active is not None and not active[b]:
            continue
        x = E[int(tokens[b])] + PE[int(positions[b])]
        for li, lp in enumerate(layers):
            h = layer_norm(x, lp["ln_gamma1"], lp["ln_beta1"])
            q = (h @ lp["attn_wq"]).reshape(n_heads, D)
            state.k[li][b].append((h @ lp["attn_wk"]).reshape(n_heads, D))
            state.v[li][b].append((h @ lp["attn_wv"]).reshape(n_heads, D))
            K = np.stack(state.k[li][b], 1)  # [H, L, D]
            V = np.stack(state.v[li][b], 1)
            s = np.einsum("hd,hld->hl", q, K) / np.sqrt(D)
            p = np.exp(s - s.max(-1, keepdims=True))
            p /= p.sum(-1, keepdims=True)
            a = np.einsum("hl,hld->hd", p, V).reshape(d)
            x = x + a @ lp["attn_wo"]
            h = layer_norm(x, lp["ln_gamma2"], lp["ln_beta2"])
            x = x + gelu_tanh(h @ lp["ff_w1"] + lp["ff_b1"]) @ lp["ff_w2"] + lp["ff_b2"]
        out[b] = x @ E.T
    return out


def greedy_generate(params: dict, prompt, max_tokens: int, n_heads: int):
    """Greedy decode with a KV cache (no window): returns (tokens, step logits)."""
    state = DecodeState(len(params["layers"]), 1)
    toks = list(int(t) for t in prompt)
    logits = []
    for t, tok in enumerate(toks):
        lg = decode_step(params, state, [tok], [t], n_heads)[0]
    for _ in range(max_tokens):
        logits.append(lg)
        nxt = int(np.argmax(lg))
        toks.append(nxt)
        lg = decode_step(params, state, [nxt], [len(toks) - 1], n_heads)[0]
    return toks, np.array(logits)


def reference_generate(params: dict, prompt, max_tokens: int, n_heads: int,
                       context_size: int, forward_fn=None):
    """generate.py:29-69 with temperature 0: every token re-runs the full
    forward over the last context_size tokens, left-padded with token 0,
    and appends the argmax of the last row. forward_fn(params, ids[1, T])
    -> logits [1, T, V] defaults to this module's float64 forward."""
    fwd = forward_fn or (lambda p, ids: forward(p, ids, n_heads))
    tokens = list(int(t) for t in prompt)
    for _ in range(max_tokens):
        ctx = tokens[max(0, len(tokens) - context_size):]
        if len(ctx) < context_size:
            ctx = [0] * (context_size - len(ctx)) + ctx
        lg = fwd(params, np.array([ctx]))[0, -1]
        tokens.append(int(np.argmax(lg)))
    return tokens


def init_params(vocab: int, dim: int, n_layers: int, context: int, mlp: int | None = None,
                seed: int = 0, std: float = 0.02) -> dict:
    """Seeded N(0, std) weights in the reference's layout (float32), biases
    0, LayerNorm gamma 1 / beta 0, and the reference's positional table.
    Drawn in the field order of jax_backend.py:327-359 from
    numpy.random.default_rng(seed); the same generator feeds the GPU model."""
    rng = np.random.default_rng(seed)
    mlp = mlp or 4 * dim

    def w(*shape):
        return (rng.standard_normal(shape) * std).astype(np.float32)

    layers = []
    for _ in range(n_layers):
        layers.append({
            "attn_wq": w(dim, dim), "attn_wk": w(dim, dim), "attn_wv": w(dim, dim),
            "attn_wo": w(dim, dim), "ff_w1": w(dim, mlp), "ff_b1": np.zeros(mlp, np.float32),
            "ff_w2": w(mlp, dim), "ff_b2": np.zeros(dim, np.float32),
            "ln_gamma1": np.ones(dim, np.float32), "ln_beta1": np.zeros(dim, np.float32),
            "ln_gamma2": np.ones(dim, np.float32), "ln_beta2": np.zeros(dim, np.float32),
        })
    return {"embedding": w(vocab, dim),
            "pos_encoding": positional_encoding(context, dim).astype(np.float32),
            "layers": layers}


def torch_forward_fp32(params: dict, tokens, n_heads: int):
    """The same forward in float32 torch on the CPU (jax_backend.py:143-148
    with its float32 dtypes): the timed CPU restatement of the reference's
    JAX CPU path in bench.py's cpu_baseline legs. Returns a float32 tensor
    [B, T, V]. Weights are converted on each call's first use and cached."""
    import torch

    cache = params.setdefault("_torch_fp32", {})
    if not cache:
        cache["E"] = torch.from_numpy(np.asarray(params["embedding"], np.float32))
        cache["PE"] = torch.from_numpy(np.asarray(params["pos_encoding"], np.float32))
        cache["L"] = [{k: torch.from_numpy(np.asarray(lp[k], np.float32)) for k in LAYER_FIELDS}
                      for lp in params["layers"]]
    E, PE = cache["E"], cache["PE"]
    ids = torch.as_tensor(np.asarray(tokens), dtype=torch.long)
    B, T = ids.shape
    d = E.shape[1]
    D = d // n_heads
    x = E[ids] + PE[:T]
    mask = torch.triu(torch.ones(T, T), diagonal=1) * -1e9

    def ln(y, g, b):
        mu = y.mean(-1, keepdim=True)
        var = ((y - mu) ** 2).mean(-1, keepdim=True)
        return (y - mu) / torch.sqrt(var + 1e-5) * g + b

    for lp in cache["L"]:
        h = ln(x, lp["ln_gamma1"], lp["ln_beta1"])
        q = (h @ lp["attn_wq"]).reshape(B, T, n_heads, D).transpose(1, 2)
        k = (h @ lp["attn_wk"]).reshape(B, T, n_heads, D).transpose(1, 2)
        v = (h @ lp["attn_wv"]).reshape(B, T, n_heads, D).transpose(1, 2)
        s = q @ k.transpose(-1, -2) / (D ** 0.5) + mask
        a = torch.softmax(s, -1) @ v
        x = x + a.transpose(1, 2).reshape(B, T, d) @ lp["attn_wo"]
        h = ln(x, lp["ln_gamma2"], lp["ln_beta2"])
        f = h @ lp["ff_w1"] + lp["ff_b1"]
        f = 0.5 * f * (1 + torch.tanh(0.7978845608028654 * (f + 0.044715 * f ** 3)))
        x = x + f @ lp["ff_w2"] + lp["ff_b2"]
    return x @ E.T


class TorchCachedDecoder:
    """The cached recurrence of decode_step in float32 torch on the CPU,
    batched: bench.py's second CPU baseline for C1/C3 (the same algorithm as
    the GPU path, so it separates the algorithmic gain of the cache from the
    hardware gain). K/V live in [B, H, T_cap, D] tensors per layer; one call
    advances every sequence by one token."""

    def __init__(self, params: dict, n_heads: int, batch: int, t_cap: int):
        import torch

        self.torch = torch
        f = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32))  # noqa: E731
        self.E, self.PE = f(params["embedding"]), f(params["pos_encoding"])
        self.L = [{k: f(lp[k]) for k in LAYER_FIELDS} for lp in params["layers"]]
        self.H, self.B, self.T = n_heads, batch, t_cap
        d = self.E.shape[1]
        self.D = d // n_heads
        shape = (batch, n_heads, t_cap, self.D)
        self.k = [torch.zeros(shape) for _ in self.L]
        self.v = [torch.zeros(shape) for _ in self.L]
        self.len = torch.zeros(batch, dtype=torch.long)

    def step(self, tokens) -> "np.ndarray":
        """Feeds tokens[b] at position len[b] of each sequence; returns the
        float32 logits [B, V] and advances every length by one."""
        torch = self.torch
        B, H, D = self.B, self.H, self.D
        ids = torch.as_tensor(np.asarray(tokens), dtype=torch.long)
        pos = self.len.clone()
        x = self.E[ids] + self.PE[pos]
        rows = torch.arange(B)
        mask = torch.arange(self.T)[None, :] > pos[:, None]  # [B, T]: beyond the new token

        def ln(y, g, b):
            mu = y.mean(-1, keepdim=True)
            var = ((y - mu) ** 2).mean(-1, keepdim=True)
            return (y - mu) / torch.sqrt(var + 1e-5) * g + b

        for li, lp in enumerate(self.L):
            h = ln(x, lp["ln_gamma1"], lp["ln_beta1"])
            q = (h @ lp["attn_wq"]).reshape(B, H, 1, D)
            self.k[li][rows, :, pos] = (h @ lp["attn_wk"]).reshape(B, H, D)
            self.v[li][rows, :, pos] = (h @ lp["attn_wv"]).reshape(B, H, D)
            s = (q @ self.k[li].transpose(-1, -2))[:, :, 0] / (D ** 0.5)  # [B, H, T]
            s = s.masked_fill(mask[:, None, :], float("-inf"))
            a = (torch.softmax(s, -1)[:, :, None] @ self.v[li])[:, :, 0]  # [B, H, D]
            x = x + a.reshape(B, H * D) @ lp["attn_wo"]
            h = ln(x, lp["ln_gamma2"], lp["ln_beta2"])
            f = h @ lp["ff_w1"] + lp["ff_b1"]
            f = 0.5 * f * (1 + torch.tanh(0.7978845608028654 * (f + 0.044715 * f ** 3)))
            x = x + f @ lp["ff_w2"] + lp["ff_b2"]
        self.len += 1
        return (x @ self.E.T).numpy()
