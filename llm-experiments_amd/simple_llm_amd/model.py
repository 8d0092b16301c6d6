"""The reference model's generate path on the KV cache, on gfx950.

Drop-in for the caller side of the hot path:
  TransformerModelParams   simple-llm/src/common_backend.py:4-11
  LayerParams field names  simple-llm/src/jax_backend.py:36-55
  forward                  simple-llm/src/jax_backend.py:143-148 (logits of every
                           position: one multi-token prefill over the cache)
  generate_text            simple-llm/src/generate.py:8-71 (same signature)

The model is the reference's JAX model (pre-LN blocks, bias-free attention
projections, tanh GELU MLP, tied logits, positional table of
jax_backend.py:25-33). Generation runs in two phases, all HIP kernels of
libskv.so:
  * prefill: every prompt (a ragged batch) goes through all layers at once:
    embedding + position of every prompt row, the fused q/k/v projection as
    a tiled MFMA GEMM (LayerNorm applied as the rows are staged), the chunk
    append into the cache, causal attention over it and the fill advance in
    one call (skv_append_prefill_attn: the fp32 MFMA kernel for an fp32
    cache, the bf16 one for a bf16 cache), output projection and MLP as
    GEMMs; then the logits of
    each sequence's last prompt row only;
  * decode: one token per sequence and step: embedding + position, fused
    q/k/v projection (LayerNorm folded into its reads), the cache append and
    decode attention in one call (skv_append_decode_attn), output projection
    with residual, MLP (LayerNorm folded in, GELU, residual), tied logits and
    the next token, replayed as one HIP graph.
The next token is skv_argmax when greedy (temperature 0, the reference's
jnp.argmax branch, jax_backend.py:466-469), otherwise skv_sample (repetition
penalty, temperature, min-p, top-k, top-p, then a draw). PyTorch only owns
the memory.

Differences from the reference's generate_text, both documented choices:
  * while the sequence is shorter than context_size, tokens attend their
    cached prefix at their absolute positions; the reference re-runs a
    left-padded window of context_size per token, which shifts positions
    while the window is not full (its tokens are therefore not a parity
    target; parity is checked on the logits of the final sequence, teacher
    forced). From context_size tokens on, generate_text does what the
    reference does: one full-window forward of the last context_size tokens
    per token (a prefill at positions 0..context_size-1);
  * the draw's uniform comes from splitmix64 of (seed, row, position), so a
    captured step replays deterministically; the reference's jax.random
    stream is not reproduced, only its filtered distribution.
"""
from __future__ import annotations

import ctypes
import dataclasses
from typing import List, Optional, Sequence

import numpy as np
import torch

from . import _lib
from .gpu import gpu
from .gpu.gpu_kv_cache import _prefill_workspace
from .gpu.gpu_types import GPUContext, KVCache

LAYER_FIELDS = ("attn_wq", "attn_wk", "attn_wv", "attn_wo", "ff_w1", "ff_b1", "ff_w2",
                "ff_b2", "ln_gamma1", "ln_beta1", "ln_gamma2", "ln_beta2")


@dataclasses.dataclass
class TransformerModelParams:
    """Model shape record (reference: common_backend.py:4-11)."""

    vocab_size: int
    embedding_dim: int
    context_size: int
    n_heads: int
    n_layers: int
    epochs: list = dataclasses.field(default_factory=list)


def positional_encoding(seq_len: int, dim: int) -> np.ndarray:
    """The reference's positional table (jax_backend.py:25-33), float32:
    sin of the even-index angles, then cos of the odd-index angles."""
    pos = np.arange(seq_len, dtype=np.float64)[:, None]
    i = np.arange(dim)[None, :]
    ang = pos / (10000.0 ** (2 * (i // 2) / dim))
    return np.concatenate([np.sin(ang[:, 0::2]), np.cos(ang[:, 1::2])], -1).astype(np.float32)


def initialize_params(tm: TransformerModelParams, seed: int = 0, std: float = 0.02,
                      mlp_dim: Optional[int] = None) -> dict:
    """Seeded N(0, std) weights in the reference's layout ([in, out] float32
    matrices, zero biases, LayerNorm gamma 1 / beta 0), drawn in the field
    order of jax_backend.py:327-359 from numpy.random.default_rng(seed)."""
    rng = np.random.default_rng(seed)
    d, mlp = tm.embedding_dim, mlp_dim or 4 * tm.embedding_dim

    def w(*shape):
        return (rng.standard_normal(shape) * std).astype(np.float32)

    layers = []
    for _ in range(tm.n_layers):
        layers.append({
            "attn_wq": w(d, d), "attn_wk": w(d, d), "attn_wv": w(d, d), "attn_wo": w(d, d),
            "ff_w1": w(d, mlp), "ff_b1": np.zeros(mlp, np.float32), "ff_w2": w(mlp, d),
            "ff_b2": np.zeros(d, np.float32), "ln_gamma1": np.ones(d, np.float32),
            "ln_beta1": np.zeros(d, np.float32), "ln_gamma2": np.ones(d, np.float32),
            "ln_beta2": np.zeros(d, np.float32),
        })
    return {"embedding": w(tm.vocab_size, d),
            "pos_encoding": positional_encoding(tm.context_size, d), "layers": layers}


class _Buffers:
    """Per-batch-size activations of one decode step (all device, fp32)."""

    def __init__(self, dev, B, d, mlp, vocab):
        self.B = B
        self.ids = torch.zeros(B, dtype=torch.int32, device=dev)
        self.x = torch.zeros((B, d), device=dev)
        self.h = torch.zeros((B, d), device=dev)
        self.qkv = torch.zeros((3, B, d), device=dev)
        self.attn = torch.zeros((B, d), device=dev)
        self.ff = torch.zeros((B, mlp), device=dev)
        self.logits = torch.zeros((B, vocab), device=dev)
        self.argmax = torch.zeros(B, dtype=torch.int32, device=dev)
        # argmax workspace: the per-slice candidates of rows wider than one
        # slice (stream ordered, like the step's other buffers)
        L = _lib.lib()
        arg = L.skv_argmax_workspace_bytes(B, vocab)
        self.arg_ws = torch.zeros(max(arg, 4), dtype=torch.uint8, device=dev)
        # split-K partials of the narrow projections, shared by the step's
        # linears (stream ordered)
        lin = max(L.skv_linear_workspace_bytes(B, n, k)
                  for n, k in ((3 * d, d), (d, d), (mlp, d), (d, mlp), (vocab, d)))
        self.lin_ws = torch.zeros(max(lin, 4), dtype=torch.uint8, device=dev)
        # per-row argmax candidates of the logits projection (the step's
        # argmax, finished by skv_next_embed): skv_linear_packed's or
        # skv_linear_cand's, whichever the model's sizes take
        cb = max(L.skv_linear_packed_cand_bytes(B), L.skv_linear_cand_bytes(B, vocab, d))
        self.cand = torch.zeros(max(cb // 4, 1), device=dev)
        # slice statistics of skv_sample's split path (stream ordered)
        self.samp_ws = torch.zeros(max(L.skv_sample_workspace_bytes(B, vocab), 8),
                                   dtype=torch.uint8, device=dev)


class _PrefillBuffers:
    """Activations of a prefill of B sequences x C prompt rows (device, fp32).

    Rows are laid out [B, C]: row b*C + i is position start[b] + i of
    sequence b, valid for i < n_new[b] (the padding rows of shorter prompts
    run through the projections too, and their attention output is zero)."""

    def __init__(self, dev, B, C, d, mlp):
        M = B * C
        self.B, self.C = B, C
        self.ids = torch.zeros(M, dtype=torch.int32, device=dev)
        self.pos = torch.zeros(M, dtype=torch.int32, device=dev)
        self.n_new = torch.zeros(B, dtype=torch.int32, device=dev)
        self.last = torch.zeros(B, dtype=torch.int32, device=dev)  # each sequence's last row
        self.x = torch.zeros((M, d), device=dev)
        self.qkv = torch.zeros((3, M, d), device=dev)
        self.attn = torch.zeros((M, d), device=dev)
        self.ff = torch.zeros((M, mlp), device=dev)
        self.x_last = torch.zeros((B, d), device=dev)
        # row maps of a packed (ragged) prefill: packed q, k, v -> [B, C] rows
        # (three planes), and the attention output's valid rows -> packed
        self.gather_pad = torch.zeros(3 * M, dtype=torch.int32, device=dev)
        self.gather_pk = torch.zeros(M, dtype=torch.int32, device=dev)
        L = _lib.lib()
        lin = max(L.skv_linear_workspace_bytes(M, n, k)
                  for n, k in ((3 * d, d), (d, d), (mlp, d), (d, mlp)))
        self.lin_ws = torch.zeros(max(lin, 4), dtype=torch.uint8, device=dev)


class TransformerModel:
    """The reference model's weights on the device, laid out for the decode
    kernels: every matrix transposed to [out, in] (rows read contiguously by
    skv_linear) and the q/k/v projections fused into one [3d, d] matrix."""

    def __init__(self, ctx: GPUContext, tm_params: TransformerModelParams,
                 params: Optional[dict] = None, kv_dtype: torch.dtype = torch.float32):
        self.ctx = ctx
        self.tm_params = tm_params
        self.kv_dtype = kv_dtype
        d = tm_params.embedding_dim
        if d % tm_params.n_heads:
            raise ValueError("embedding_dim must be a multiple of n_heads")
        self.head_dim = d // tm_params.n_heads
        params = params if params is not None else initialize_params(tm_params)
        self.params = params
        dev = ctx.device

        def t(a, transpose=False):
            a = np.asarray(a, np.float32)
            return torch.from_numpy(np.ascontiguousarray(a.T if transpose else a)).to(dev)

        self.emb = t(params["embedding"])
        if tuple(self.emb.shape) != (tm_params.vocab_size, d):
            raise ValueError(f"embedding must be [{tm_params.vocab_size}, {d}]")
        self.pe = t(params["pos_encoding"])
        if self.pe.shape[0] < tm_params.context_size:
            raise ValueError("pos_encoding has fewer rows than context_size")
        self.layers = []
        for lp in params["layers"][:tm_params.n_layers]:
            wqkv = np.concatenate([np.asarray(lp[k], np.float32).T
                                   for k in ("attn_wq", "attn_wk", "attn_wv")], 0)
            self.layers.append({
                "wqkv_t": t(wqkv), "wo_t": t(lp["attn_wo"], True),
                "w1_t": t(lp["ff_w1"], True), "b1": t(lp["ff_b1"]),
                "w2_t": t(lp["ff_w2"], True), "b2": t(lp["ff_b2"]),
                "g1": t(lp["ln_gamma1"]), "be1": t(lp["ln_beta1"]),
                "g2": t(lp["ln_gamma2"]), "be2": t(lp["ln_beta2"]),
            })
        if len(self.layers) != tm_params.n_layers:
            raise ValueError("params hold fewer layers than n_layers")
        self.mlp_dim = self.layers[0]["w1_t"].shape[0]
        self._bufs = {}
        self.direct_splits = 0  # 0: direct_split() picks per batch size

    # -- cache and buffers ---------------------------------------------------

    def new_cache(self, batch_size: int) -> KVCache:
        tm = self.tm_params
        return gpu.kv_cache_create(self.ctx, gpu.KVCacheConfig(
            batch_size=batch_size, max_seq_len=tm.context_size, n_layers=tm.n_layers,
            n_heads=tm.n_heads, head_dim=self.head_dim, dtype=self.kv_dtype))

    def buffers(self, B: int) -> _Buffers:
        if B not in self._bufs:
            tm = self.tm_params
            bf = _Buffers(self.ctx.device, B, tm.embedding_dim, self.mlp_dim, tm.vocab_size)
            # the direct attention's split partials and arrival counters (zero
            # between calls; stream ordered), sized for its largest split
            nb = _lib.lib().skv_decode_direct_workspace_bytes(B, tm.n_heads, self.head_dim, 4)
            bf.dir_ws = torch.zeros(max(nb, 4), dtype=torch.uint8, device=self.ctx.device)
            self._bufs[B] = bf
        return self._bufs[B]

    def direct_split(self, B: int, dtype: torch.dtype) -> int:
        """Workgroups per (sequence, head) of the direct attention (1, 2 or
        4; direct_splits overrides it): 4 where a batch has fewer (sequence,
        head) pairs than CUs, else 1. Measured on MI355X, whole generate
        runs: C1 (4 pairs) 11,330 tokens/s at 4 against 11,040 at 1; C3 (192
        pairs) fp32 22,556 at 4 against 21,744 at 1 and 21,569 at 2, bf16
        24,493-24,503 at 4 against 24,135-24,165 at 1 and 23,865-23,888 at 2.
        dtype is kept for callers; both cache dtypes take the same rule."""
        if self.direct_splits:
            return int(self.direct_splits)
        pairs = B * self.tm_params.n_heads
        return 4 if pairs < 256 else 1

    def prefill_buffers(self, B: int, C: int) -> _PrefillBuffers:
        key = ("prefill", B, C)
        if key not in self._bufs:
            self._bufs[key] = _PrefillBuffers(self.ctx.device, B, C, self.tm_params.embedding_dim,
                                              self.mlp_dim)
        return self._bufs[key]

    # -- one decode step -----------------------------------------------------

    def forward_step(self, cache: KVCache, ids: torch.Tensor, direct: bool = False) -> torch.Tensor:
        """Run token ids[b] of every sequence at its current fill through all
        layers, appending its K/V to the cache; returns logits [B, V] (a
        buffer reused by the next call). ids: int32 device tensor [B].
        Sequences whose cache is full are not appended to (their logits are
        not meaningful). direct: the attention of Generator's greedy steps
        (skv_append_decode_attn_direct, which leaves the fills in place),
        followed here by the fill advance of every layer that Generator's
        next-token kernel does at the start of the following step."""
        B = cache.batch_size
        if cache.n_kv_heads != cache.n_heads or cache.paged:
            raise ValueError("the model path uses a contiguous multi-head cache")
        if direct and not self._direct_ok():
            raise ValueError("the direct attention takes head_dim 64 or 128 and contexts up "
                             "to 1024 tokens")
        bf = self.buffers(B)
        if ids.data_ptr() != bf.ids.data_ptr():
            bf.ids.copy_(ids)
        self._launch_step(cache, bf, direct=direct)
        if direct:
            L = _lib.lib()
            s = _lib.stream_handle(self.ctx.device)
            for layer in cache.layers:
                _lib.check(L.skv_advance(layer.lens.data_ptr(), None, 1, B, cache.max_seq_len,
                                         s), "skv_advance")
        # host mirror: every layer appended where the sequence had room
        for layer in cache.layers:
            layer.host_lens = np.minimum(layer.host_lens + 1, cache.max_seq_len)
        return bf.logits

    def _decode_plan(self, cache: KVCache):
        key = ("plan", cache.batch_size)
        if key not in self._bufs:
            T = cache.max_seq_len
            chunk, n = gpu.decode_plan(self.ctx, cache.batch_size, cache.n_heads,
                                       cache.n_kv_heads, T, cache.batch_size * T,
                                       head_dim=cache.head_dim, dtype=cache.dtype)
            L = _lib.lib()
            need = L.skv_decode_workspace_bytes(cache.batch_size, cache.n_heads, cache.head_dim, n)
            ws = torch.empty(max(need, 1), dtype=torch.uint8, device=self.ctx.device)
            self._bufs[key] = (chunk, n, ws)
        return self._bufs[key]

    def _folded(self):
        """Per layer, the LayerNorm-folded q/k/v and MLP-up weights of
        skv_linear_folded (made once, on the current stream), or None when
        the decode kernels do not take d (K = 16 * s * w, s in {3, 4, 6, 8,
        12}, 4 <= w <= 16)."""
        key = "folded"
        if key not in self._bufs:
            d = self.tm_params.embedding_dim
            if not any(d % (16 * st) == 0 and 4 <= d // (16 * st) <= 16
                       for st in (3, 4, 6, 8, 12)):
                self._bufs[key] = None
                return None
            L = _lib.lib()
            s = _lib.stream_handle(self.ctx.device)
            out = []
            for lw in self.layers:
                f = {}
                for name, w, g, be, b in (("qkv", lw["wqkv_t"], lw["g1"], lw["be1"], None),
                                          ("w1", lw["w1_t"], lw["g2"], lw["be2"], lw["b1"])):
                    n, k = w.shape
                    wf = torch.empty_like(w)
                    c1 = torch.empty(n, device=w.device)
                    c2 = torch.empty(n, device=w.device)
                    _lib.check(L.skv_linear_fold_ln(wf.data_ptr(), c1.data_ptr(), c2.data_ptr(),
                                                    w.data_ptr(), g.data_ptr(), be.data_ptr(),
                                                    b.data_ptr() if b is not None else None, n,
                                                    k, s), "skv_linear_fold_ln")
                    f[name] = (wf, c1, c2)
                out.append(f)
            self._bufs[key] = out
        return self._bufs[key]

    def _packed_logits(self):
        """The tied output projection in skv_linear_pack's lane order (made
        once), or None when skv_linear_packed does not take the sizes
        (K in {512, 768, 1024}, 16384 <= vocab <= 65536)."""
        key = "packed_logits"
        if key not in self._bufs:
            V, d = self.emb.shape
            ok = d in (512, 768, 1024) and 16384 <= V <= 65536
            wp = None
            if ok:
                L = _lib.lib()
                wp = torch.empty(L.skv_linear_packed_bytes(V, d) // 4, device=self.emb.device)
                _lib.check(L.skv_linear_pack(wp.data_ptr(), self.emb.data_ptr(), V, d,
                                             _lib.stream_handle(self.ctx.device)),
                           "skv_linear_pack")
            self._bufs[key] = wp
        return self._bufs[key]

    def _n_cand(self, B: int) -> int:
        """Argmax candidates per row the logits projection of a B-row step
        can write (0: none): one per workgroup of skv_linear_packed, else one
        per 16-column tile of skv_linear_cand."""
        if B > 16:
            return 0
        L = _lib.lib()
        if self._packed_logits() is not None:
            return L.skv_linear_packed_cand_bytes(B) // (8 * B)
        V, d = self.emb.shape
        return L.skv_linear_cand_bytes(B, V, d) // (8 * B)

    def _direct_ok(self) -> bool:
        """Whether the decode step can take skv_append_decode_attn_direct:
        head_dim 64 or 128 and contexts up to 1024 tokens (past them the
        split attention spreads a long row over more CUs and is faster)."""
        return self.head_dim in (64, 128) and self.tm_params.context_size <= 1024

    def _launch_step(self, cache: KVCache, bf: _Buffers, embedded: bool = False,
                     cand: bool = False, direct: bool = False) -> None:
        """One decode step's launches. embedded: x already holds the step's
        input rows (skv_next_embed ran). cand: the logits projection also
        writes the argmax candidates into bf.cand (skv_next_embed finishes
        them at the next step); needs _n_cand(B) > 0. direct: the attention
        appends without advancing the fills (skv_append_decode_attn_direct;
        the next step's next-token kernel advances them)."""
        L = _lib.lib()
        tm = self.tm_params
        B, d, H, D, T = cache.batch_size, tm.embedding_dim, tm.n_heads, self.head_dim, \
            cache.max_seq_len
        s = _lib.stream_handle(self.ctx.device)
        chk = _lib.check
        cdt = _lib.dtype_code(cache.dtype)
        chunk, n_chunks, ws = self._decode_plan(cache)
        scale = 1.0 / float(np.sqrt(D))
        x, h, qkv, attn, ff = bf.x.data_ptr(), bf.h.data_ptr(), bf.qkv.data_ptr(), \
            bf.attn.data_ptr(), bf.ff.data_ptr()
        q_ptr, k_ptr, v_ptr = qkv, qkv + B * d * 4, qkv + 2 * B * d * 4
        lw_ws, lw_n = bf.lin_ws.data_ptr(), bf.lin_ws.numel()
        lens0 = cache.layers[0].lens.data_ptr()
        nsplit = self.direct_split(B, cache.dtype) if direct else 1
        # up to 16 rows: LayerNorm folded into the weights (skv_linear_folded)
        folded = self._folded() if B <= 16 else None
        if not embedded:
            chk(L.skv_embed(x, bf.ids.data_ptr(), lens0, self.emb.data_ptr(), self.pe.data_ptr(),
                            B, d, tm.vocab_size, self.pe.shape[0], s), "skv_embed")
        for li, (lw, layer) in enumerate(zip(self.layers, cache.layers)):
            kc, vc = layer.k_cache.buffer.data_ptr(), layer.v_cache.buffer.data_ptr()
            # q, k, v = LN1(x) . [Wq Wk Wv] (LayerNorm folded into the projection)
            if folded is not None:
                wf, c1, c2 = folded[li]["qkv"]
                chk(L.skv_linear_folded(qkv, x, wf.data_ptr(), c1.data_ptr(), c2.data_ptr(), None,
                                        1e-5, B, 3 * d, d, 0, d, s), "skv_linear_folded")
            else:
                chk(L.skv_linear(qkv, x, lw["wqkv_t"].data_ptr(), None, None,
                                 lw["g1"].data_ptr(), lw["be1"].data_ptr(), 1e-5, B, 3 * d, d,
                                 0, d, lw_ws, lw_n, s), "skv_linear")
            # append k, v at each sequence's fill and attend [0, fill] (one call)
            if direct:
                chk(L.skv_append_decode_attn_direct(attn, q_ptr, kc, vc, k_ptr, v_ptr,
                                                    layer.lens.data_ptr(), B, H, D, T, scale,
                                                    cdt, _lib.F32, _lib.F32, _lib.F32, nsplit,
                                                    bf.dir_ws.data_ptr(), bf.dir_ws.numel(), s),
                    "skv_append_decode_attn_direct")
            else:
                chk(L.skv_append_decode_attn(attn, q_ptr, kc, vc, k_ptr, v_ptr,
                                             layer.lens.data_ptr(), B, H, H, D, T, scale, chunk,
                                             n_chunks, ws.data_ptr(), ws.numel(), cdt, _lib.F32,
                                             _lib.F32, _lib.F32, s), "skv_append_decode_attn")
            # x += attn . Wo
            chk(L.skv_linear(x, attn, lw["wo_t"].data_ptr(), None, x, None, None, 0.0, B, d, d, 0,
                             0, lw_ws, lw_n, s), "skv_linear")
            # ff = gelu(LN2(x) . W1 + b1); x += ff . W2 + b2
            if folded is not None:
                wf, c1, c2 = folded[li]["w1"]
                chk(L.skv_linear_folded(ff, x, wf.data_ptr(), c1.data_ptr(), c2.data_ptr(), None,
                                        1e-5, B, self.mlp_dim, d, 1, 0, s), "skv_linear_folded")
            else:
                chk(L.skv_linear(ff, x, lw["w1_t"].data_ptr(), lw["b1"].data_ptr(), None,
                                 lw["g2"].data_ptr(), lw["be2"].data_ptr(), 1e-5, B,
                                 self.mlp_dim, d, 1, 0, lw_ws, lw_n, s), "skv_linear")
            chk(L.skv_linear(x, ff, lw["w2_t"].data_ptr(), lw["b2"].data_ptr(), x, None, None, 0.0,
                             B, d, self.mlp_dim, 0, 0, lw_ws, lw_n, s), "skv_linear")
        packed = self._packed_logits() if B <= 16 else None
        if cand and self._n_cand(B) == 0:
            raise ValueError("argmax candidates need B <= 16 and a logits projection that "
                             "writes them (skv_linear_packed or skv_linear_cand sizes)")
        if packed is not None:
            chk(L.skv_linear_packed(bf.logits.data_ptr(), x, packed.data_ptr(), None, None, B,
                                    tm.vocab_size, d, 0, bf.cand.data_ptr() if cand else None,
                                    s), "skv_linear_packed")
        elif cand:
            chk(L.skv_linear_cand(bf.logits.data_ptr(), x, self.emb.data_ptr(), None, B,
                                  tm.vocab_size, d, bf.cand.data_ptr(), lw_ws, lw_n, s),
                "skv_linear_cand")
        else:
            chk(L.skv_linear(bf.logits.data_ptr(), x, self.emb.data_ptr(), None, None, None,
                             None, 0.0, B, tm.vocab_size, d, 0, 0, lw_ws, lw_n, s), "skv_linear")

    # -- many steps ----------------------------------------------------------

    # -- prefill ---------------------------------------------------------------

    def prefill(self, cache: KVCache, tokens: np.ndarray, n_new: Optional[np.ndarray] = None,
                all_logits: bool = False) -> torch.Tensor:
        """Run C prompt tokens of every sequence through all layers at once,
        appending their K/V to the cache after each sequence's current fill.

        tokens: host int array [B, C]; n_new: valid tokens per sequence (<= C,
        default C), the rest of a row is padding. Returns the logits of each
        sequence's last new token, [B, V] (the decode buffer, reused by the
        next call), or with all_logits those of every row, [B, C, V] (a new
        tensor). The fills advance by n_new."""
        tm = self.tm_params
        B = cache.batch_size
        if cache.n_kv_heads != cache.n_heads or cache.paged:
            raise ValueError("the model path uses a contiguous multi-head cache")
        tokens = np.asarray(tokens, np.int64)
        if tokens.ndim != 2 or tokens.shape[0] != B or tokens.shape[1] <= 0:
            raise ValueError(f"tokens must be [batch_size={B}, C] with C >= 1")
        C = int(tokens.shape[1])
        n_host = (np.full(B, C, np.int64) if n_new is None
                  else np.asarray(n_new, np.int64).reshape(B))
        if (n_host < 0).any() or (n_host > C).any():
            raise ValueError(f"n_new entries must lie in [0, {C}]")
        if tokens.size and (tokens.min() < 0 or tokens.max() >= tm.vocab_size):
            raise ValueError("token out of the vocabulary")
        start = cache.layers[0].host_lens.copy()
        if int((start + n_host).max()) > cache.max_seq_len:
            raise ValueError(f"Cache is full: a prefill of {int(n_host.max())} tokens after "
                             f"{int(start.max())}, max_seq_len={cache.max_seq_len}")
        pb = self.prefill_buffers(B, C)
        d, H, D, T = tm.embedding_dim, tm.n_heads, self.head_dim, cache.max_seq_len
        M = B * C
        pos = start[:, None] + np.arange(C)[None, :]
        pb.n_new.copy_(torch.from_numpy(n_host.astype(np.int32)))
        # Ragged prompts: the projections run over the valid rows only, packed
        # (row off_b + i is token i of sequence b); q, k, v are gathered into
        # the [B, C] layout of the chunk append and the attention, and the
        # attention output back. The projections then run over Mp rows instead
        # of B * C, which can select another skv_linear kernel (it picks one by
        # row count), so the valid rows agree with the padded layout's within
        # fp32 rounding, not necessarily bit for bit.
        Mp = int(n_host.sum())
        # (packed q, k, v are staged in ff's space: 3 Mp d <= M mlp)
        packed = (not all_logits and 0 < Mp <= (3 * M) // 4
                  and 3 * Mp * d <= M * self.mlp_dim)
        if packed:
            off = np.concatenate([[0], np.cumsum(n_host)[:-1]]).astype(np.int64)
            bi = np.repeat(np.arange(B), n_host)
            ii = np.arange(Mp) - np.repeat(off, n_host)
            pb.ids[:Mp].copy_(torch.from_numpy(tokens[bi, ii].astype(np.int32)))
            pb.pos[:Mp].copy_(torch.from_numpy(np.minimum(start[bi] + ii, T - 1).astype(np.int32)))
            # padded row b*C + i <- packed row off_b + min(i, n_b - 1) (rows past
            # n_b are padding the attention masks), for the q, k and v planes
            pad = off[:, None] + np.minimum(np.arange(C)[None, :],
                                            np.maximum(n_host - 1, 0)[:, None])
            to_pad = (np.arange(3)[:, None] * Mp + pad.reshape(1, -1)).reshape(-1)
            pb.gather_pad[:3 * M].copy_(torch.from_numpy(to_pad.astype(np.int32)))
            pb.gather_pk[:Mp].copy_(torch.from_numpy((bi * C + ii).astype(np.int32)))
            pb.last.copy_(torch.from_numpy(
                (off + np.maximum(n_host - 1, 0)).astype(np.int32)))
        else:
            pb.ids.copy_(torch.from_numpy(tokens.reshape(-1).astype(np.int32)))
            pb.pos.copy_(torch.from_numpy(np.minimum(pos, T - 1).reshape(-1).astype(np.int32)))
            pb.last.copy_(torch.from_numpy(
                (np.arange(B) * C + np.maximum(n_host - 1, 0)).astype(np.int32)))
        Mr = Mp if packed else M  # rows of the projections
        L = _lib.lib()
        s = _lib.stream_handle(self.ctx.device)
        chk = _lib.check
        cdt = _lib.dtype_code(cache.dtype)
        scale = 1.0 / float(np.sqrt(D))
        x, qkv, attn, ff = pb.x.data_ptr(), pb.qkv.data_ptr(), pb.attn.data_ptr(), pb.ff.data_ptr()
        q_ptr, k_ptr, v_ptr = qkv, qkv + M * d * 4, qkv + 2 * M * d * 4
        ws, wn = pb.lin_ws.data_ptr(), pb.lin_ws.numel()
        n_ptr = pb.n_new.data_ptr()
        ns = ctypes.c_int()
        chk(L.skv_prefill_plan(B, C, H, H, max(int((start + n_host).max()), 1), ctypes.byref(ns)),
            "skv_prefill_plan")
        need = L.skv_prefill_workspace_bytes(B, C, H, D, ns.value)
        pws = _prefill_workspace(self.ctx, need)
        pws_ptr = pws.data_ptr() if pws is not None else None
        pws_n = pws.numel() if pws is not None else 0
        chk(L.skv_embed(x, pb.ids.data_ptr(), pb.pos.data_ptr(), self.emb.data_ptr(),
                        self.pe.data_ptr(), Mr, d, tm.vocab_size, self.pe.shape[0], s),
            "skv_embed")
        for lw, layer in zip(self.layers, cache.layers):
            kc, vc = layer.k_cache.buffer.data_ptr(), layer.v_cache.buffer.data_ptr()
            lens = layer.lens.data_ptr()
            # q, k, v = LN1(x) . [Wq Wk Wv] over every prompt row: [3][B, C, H, D]
            # (packed: [3][Mp, d] into ff's space, then gathered into the layout)
            chk(L.skv_linear(ff if packed else qkv, x, lw["wqkv_t"].data_ptr(), None, None,
                             lw["g1"].data_ptr(), lw["be1"].data_ptr(), 1e-5, Mr, 3 * d, d, 0, d,
                             ws, wn, s), "skv_linear")
            if packed:
                chk(L.skv_gather_rows(qkv, ff, pb.gather_pad.data_ptr(), 3 * M, d, 3 * Mp, s),
                    "skv_gather_rows")
            # the chunk's k, v at each sequence's fill, then causal attention of
            # its queries over prefix + chunk; then the fill moves past the chunk
            # (one call)
            chk(L.skv_append_prefill_attn(attn, q_ptr, kc, vc, k_ptr, v_ptr, lens, n_ptr, B, C,
                                          H, H, D, T, scale, ns.value, pws_ptr, pws_n, cdt,
                                          _lib.F32, _lib.F32, _lib.F32, s),
                "skv_append_prefill_attn")
            a_rows = attn
            if packed:  # the valid rows of the attention output, packed, into qkv's space
                chk(L.skv_gather_rows(qkv, attn, pb.gather_pk.data_ptr(), Mp, d, M, s),
                    "skv_gather_rows")
                a_rows = qkv
            # x += attn . Wo; ff = gelu(LN2(x) . W1 + b1); x += ff . W2 + b2
            chk(L.skv_linear(x, a_rows, lw["wo_t"].data_ptr(), None, x, None, None, 0.0, Mr, d, d,
                             0, 0, ws, wn, s), "skv_linear")
            chk(L.skv_linear(ff, x, lw["w1_t"].data_ptr(), lw["b1"].data_ptr(), None,
                             lw["g2"].data_ptr(), lw["be2"].data_ptr(), 1e-5, Mr, self.mlp_dim, d,
                             1, 0, ws, wn, s), "skv_linear")
            chk(L.skv_linear(x, ff, lw["w2_t"].data_ptr(), lw["b2"].data_ptr(), x, None, None, 0.0,
                             Mr, d, self.mlp_dim, 0, 0, ws, wn, s), "skv_linear")
        for layer in cache.layers:
            layer.host_lens = np.minimum(start + n_host, T)
        if all_logits:
            out = torch.empty((B, C, tm.vocab_size), device=self.ctx.device)
            lws = torch.zeros(max(L.skv_linear_workspace_bytes(M, tm.vocab_size, d), 4),
                              dtype=torch.uint8, device=self.ctx.device)
            chk(L.skv_linear(out.data_ptr(), x, self.emb.data_ptr(), None, None, None, None, 0.0,
                             M, tm.vocab_size, d, 0, 0, lws.data_ptr(), lws.numel(), s),
                "skv_linear")
            return out
        # the logits of each sequence's last new row (generate.py:52 takes logits[0, -1])
        bf = self.buffers(B)
        chk(L.skv_gather_rows(pb.x_last.data_ptr(), x, pb.last.data_ptr(), B, d, Mr, s),
            "skv_gather_rows")
        chk(L.skv_linear(bf.logits.data_ptr(), pb.x_last.data_ptr(), self.emb.data_ptr(), None,
                         None, None, None, 0.0, B, tm.vocab_size, d, 0, 0, bf.lin_ws.data_ptr(),
                         bf.lin_ws.numel(), s), "skv_linear")
        return bf.logits

    # -- logits of whole sequences ------------------------------------------

    def forward(self, tokens: np.ndarray) -> np.ndarray:
        """Logits of every position of [B, T] token ids (T <= context_size),
        as the reference's forward (jax_backend.py:143-148): one prefill of
        all T tokens on a fresh cache. Returns float32 host array [B, T, V]."""
        tokens = np.asarray(tokens, np.int32)
        B, T = tokens.shape
        if T > self.tm_params.context_size:
            raise ValueError("sequence longer than context_size")
        cache = self.new_cache(B)
        return self.prefill(cache, tokens, all_logits=True).cpu().numpy()

    def forward_decode(self, tokens: np.ndarray, n_prefill: int = 0) -> np.ndarray:
        """forward() computed through the decode step instead: the first
        n_prefill tokens as one prefill (logits of every row), then one cached
        decode step per token. Returns float32 host array [B, T, V]."""
        tokens = np.asarray(tokens, np.int32)
        B, T = tokens.shape
        if T > self.tm_params.context_size:
            raise ValueError("sequence longer than context_size")
        cache = self.new_cache(B)
        out = np.zeros((B, T, self.tm_params.vocab_size), np.float32)
        if n_prefill > 0:
            out[:, :n_prefill] = self.prefill(cache, tokens[:, :n_prefill],
                                              all_logits=True).cpu().numpy()
        ids = torch.from_numpy(tokens).to(self.ctx.device)
        for t in range(n_prefill, T):
            out[:, t] = self.forward_step(cache, ids[:, t].contiguous()).cpu().numpy()
        return out


class Generator:
    """Generation of a batch of (possibly ragged) prompts on the device.

    run() prefills every prompt at once (TransformerModel.prefill: the
    logits of each prompt's last token give its first new token), then
    decodes one token per sequence and step, feeding each sequence its
    previous token (skv_next_tokens), so the loop never waits for the host.
    With use_graph the decode step is captured once into a HIP graph
    (torch.cuda.CUDAGraph over the library's launches) and replayed.
    With retire_rows (the default) a sequence is retired once its last token
    is recorded: every layer's fill of its row becomes -1, so the remaining
    steps read none of its cache. When run() returns, every row's fill is
    back at the positions its cache holds, so forward_step or prefill can
    continue on self.cache; run() starts from reset() each time.
    """

    def __init__(self, model: TransformerModel, prompts: Sequence[Sequence[int]],
                 total_len: Sequence[int] | int, use_graph: bool = False,
                 temperature: float = 0.0, top_k: int = 0, top_p: float = 1.0,
                 min_p: float = 0.0, repetition_penalty: float = 1.0,
                 repetition_window: int = 64, seed: int = 42, fused_tail: bool = True,
                 retire_rows: bool = True, direct_attention: bool = True):
        tm = model.tm_params
        self.model = model
        B = len(prompts)
        if B == 0:
            raise ValueError("no prompts")
        plen = np.array([len(p) for p in prompts], np.int32)
        if (plen <= 0).any():
            raise ValueError("every prompt needs at least one token")
        tot = np.broadcast_to(np.asarray(total_len, np.int64), (B,)).astype(np.int64)
        if (tot < plen).any():
            raise ValueError("total_len shorter than a prompt")
        if int(tot.max()) > tm.context_size:
            raise ValueError(f"total length {int(tot.max())} exceeds context_size "
                             f"{tm.context_size} (the cache does not slide; generate_text "
                             f"continues past it with full-window forwards)")
        for p in prompts:
            if min(p) < 0 or max(p) >= tm.vocab_size:
                raise ValueError("prompt token out of the vocabulary")
        if temperature < 0 or top_k < 0 or min_p < 0 or repetition_penalty <= 0 \
                or repetition_window < 0:
            raise ValueError("bad sampling parameters")
        if tm.vocab_size > 65536 and (temperature != 0.0 or repetition_penalty != 1.0):
            raise ValueError("device sampling supports vocab_size <= 65536")
        dev = model.ctx.device
        self.B, self.plen, self.tot = B, plen, tot
        Pm = int(plen.max())
        pr = np.zeros((B, Pm), np.int32)
        for b, p in enumerate(prompts):
            pr[b, :len(p)] = p
        self.prompt_host = pr
        self.prompt = torch.from_numpy(pr).to(dev)
        self.prompt_len = torch.from_numpy(plen).to(dev)
        self.seq = torch.zeros((B, tm.context_size), dtype=torch.int32, device=dev)
        self.cache = model.new_cache(B)
        # Every layer's fills in one [n_layers, B] array, so that the step's
        # next-token kernel can retire a row once its last token is recorded
        # (all its fills to -1: the decode kernels then skip it); the rows of
        # a ragged batch that are done stop costing attention reads.
        self.retire = bool(retire_rows)
        self.lens_all = torch.zeros((tm.n_layers, B), dtype=torch.int32, device=dev)
        for li, layer in enumerate(self.cache.layers):
            layer.lens = self.lens_all[li]
        self.stop = torch.from_numpy(tot.astype(np.int32)).to(dev)
        # per-row flags of the deferred fill advance (direct attention)
        self.adv = torch.zeros(B, dtype=torch.int32, device=dev)
        self.bufs = model.buffers(B)
        # decode steps after the prefill: the step at position p produces token p + 1
        self.steps = max(int((tot - 1 - plen).max()), 0)
        self.use_graph = use_graph
        self.graph = None
        self.sampling = (float(temperature), int(top_k), float(top_p), float(min_p),
                         float(repetition_penalty), int(repetition_window))
        self.seed = int(seed) & ((1 << 64) - 1)
        # greedy without a penalty takes the multi-workgroup argmax
        self.greedy = temperature == 0.0 and repetition_penalty == 1.0
        # Every step starts with skv_next_embed (skv_next_tokens and
        # skv_embed in one launch), reading the previous token from argmax.
        # Greedy up to 16 rows also folds the argmax in where the logits
        # projection can leave per-workgroup candidates (skv_linear_packed,
        # skv_linear_cand): skv_next_embed finishes them (no skv_argmax
        # launches).
        self.fused = bool(fused_tail)
        self.n_cand = model._n_cand(B) if self.fused and self.greedy else 0
        self.cand_mode = self.n_cand > 0
        # Greedy steps of contexts up to 1024 take the direct attention (one
        # workgroup per sequence and head, no merge pass): the step's append
        # leaves the fill where it was and the next step's next-token kernel
        # advances it. Sampling keeps the split attention, whose advance gives
        # skv_sample the fill that includes the step's token.
        self.direct = bool(direct_attention) and self.greedy and model._direct_ok()
        self.reset()

    def reset(self) -> None:
        """Rewind to before the prefill (empty cache, only the prompts in the
        token buffer), keeping the captured graph, so run() can be repeated."""
        self.cache.current_len = 0
        self.seq.zero_()
        self.seq[:, :self.prompt.shape[1]].copy_(self.prompt)
        self.bufs.argmax.zero_()
        self.adv.zero_()
        # with candidates, skv_next_embed reads the previous step's, or the
        # prefill's argmax before the first step
        self._cand_ready = False
        self._fresh = True

    def _next_embed(self, embed: bool) -> None:
        """skv_next_embed: the previous token from the candidates (after a
        fused step) or from argmax (after the prefill), recorded in seq,
        embedded into x when embed."""
        L = _lib.lib()
        m, c, bf = self.model, self.cache, self.bufs
        s = _lib.stream_handle(m.ctx.device)
        tm = m.tm_params
        _lib.check(L.skv_next_embed(bf.x.data_ptr() if embed else None, bf.ids.data_ptr(),
                                    self.seq.data_ptr(), bf.argmax.data_ptr(),
                                    bf.cand.data_ptr(),
                                    self.n_cand if self._cand_ready else 0,
                                    self.prompt.data_ptr(), self.prompt_len.data_ptr(),
                                    c.layers[0].lens.data_ptr(), self.B, self.prompt.shape[1],
                                    self.seq.shape[1], m.emb.data_ptr() if embed else None,
                                    m.pe.data_ptr() if embed else None, tm.embedding_dim,
                                    tm.vocab_size, m.pe.shape[0], *self._retire_args(), s),
                   "skv_next_embed")

    def _retire_args(self):
        """(stop, lens_all, n_layers, adv) of the next-token calls: retire
        finished rows, and advance the fills deferred by the direct attention."""
        stop = self.stop.data_ptr() if self.retire else None
        adv = self.adv.data_ptr() if self.direct else None
        if stop is None and adv is None:
            return None, None, 0, None
        return stop, self.lens_all.data_ptr(), self.lens_all.shape[0], adv

    def _pick(self) -> None:
        """Next token of every sequence from the logits buffer into argmax."""
        L = _lib.lib()
        m, c, bf = self.model, self.cache, self.bufs
        s = _lib.stream_handle(m.ctx.device)
        if self.greedy:
            _lib.check(L.skv_argmax(bf.argmax.data_ptr(), bf.logits.data_ptr(), self.B,
                                    m.tm_params.vocab_size, bf.arg_ws.data_ptr(),
                                    bf.arg_ws.numel(), s), "skv_argmax")
        else:
            # sample_token (jax_backend.py:413-515) over the sequence's tokens so
            # far (seq[b, :lens[b]], the prompt included); the draw is keyed by
            # (seed, sequence, position)
            T, k, p, mp, pen, win = self.sampling
            _lib.check(L.skv_sample(bf.argmax.data_ptr(), None, bf.logits.data_ptr(),
                                    self.seq.data_ptr(), self.seq.shape[1],
                                    c.layers[0].lens.data_ptr(), self.B,
                                    m.tm_params.vocab_size, T, k, p, mp, pen, win, self.seed,
                                    bf.samp_ws.data_ptr(), bf.samp_ws.numel(), s), "skv_sample")

    def _one_step(self):
        L = _lib.lib()
        m, c, bf = self.model, self.cache, self.bufs
        s = _lib.stream_handle(m.ctx.device)
        if self.fused:
            self._next_embed(embed=True)
            m._launch_step(c, bf, embedded=True, cand=self.cand_mode, direct=self.direct)
            if self.cand_mode:
                self._cand_ready = True
            else:
                self._pick()
            return
        _lib.check(L.skv_next_tokens(bf.ids.data_ptr(), self.seq.data_ptr(), bf.argmax.data_ptr(),
                                     self.prompt.data_ptr(), self.prompt_len.data_ptr(),
                                     c.layers[0].lens.data_ptr(), self.B, self.prompt.shape[1],
                                     self.seq.shape[1], *self._retire_args(), s),
                   "skv_next_tokens")
        m._launch_step(c, bf, direct=self.direct)
        self._pick()

    def prefill(self) -> None:
        """Every prompt through the model at once; the first new token of
        each sequence goes to the argmax buffer."""
        self._fresh = False
        self.model.prefill(self.cache, self.prompt_host, self.plen)
        self._pick()

    def run(self, on_step=None) -> List[List[int]]:
        """From the start (reset(): an empty cache, the prompts only), the
        prefill, then all decode steps; returns every sequence's tokens
        (prompt + output). Repeated calls reuse the captured graph.
        on_step(j, logits) (optional) is called after decode step j with the
        step's logits buffer [B, V] (stream ordered: copy it on the device,
        it is overwritten by the next step); row b's step j ran the token at
        position prompt_len[b] + j."""
        if not self._fresh:  # an explicit reset() since the last run or prefill is enough
            self.reset()
        self.prefill()
        steps = self.steps
        if steps > 0:
            if self.use_graph:
                self._one_step()  # eager first step: workspaces exist before capture
                if on_step is not None:
                    on_step(0, self.bufs.logits)
                torch.cuda.synchronize()
                if self.graph is None and steps > 1:
                    # stream capture records the launches without running them
                    g = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(g):
                        self._one_step()
                    self.graph = g
                for j in range(1, steps):
                    self.graph.replay()
                    if on_step is not None:
                        on_step(j, self.bufs.logits)
            else:
                for j in range(steps):
                    self._one_step()
                    if on_step is not None:
                        on_step(j, self.bufs.logits)
        # record the last new token at its position
        L = _lib.lib()
        s = _lib.stream_handle(self.model.ctx.device)
        if self.fused:
            self._next_embed(embed=False)
        else:
            _lib.check(L.skv_next_tokens(self.bufs.ids.data_ptr(), self.seq.data_ptr(),
                                         self.bufs.argmax.data_ptr(), self.prompt.data_ptr(),
                                         self.prompt_len.data_ptr(),
                                         self.cache.layers[0].lens.data_ptr(), self.B,
                                         self.prompt.shape[1], self.seq.shape[1],
                                         *self._retire_args(), s), "skv_next_tokens")
        # The fills left behind are the cache's real contents: retired rows
        # (-1 on the device) get back the positions they hold, every token but
        # the last one recorded (the prompt's when nothing was generated), and
        # no deferred advance stays pending, so forward_step or prefill on
        # self.cache continue from there.
        if self.retire:
            held = np.minimum(np.maximum(self.tot - 1, self.plen), self.cache.max_seq_len)
            self.lens_all.copy_(torch.from_numpy(
                np.broadcast_to(held.astype(np.int32), self.lens_all.shape).copy()))
        self.adv.zero_()
        for layer in self.cache.layers:
            layer.host_lens = layer.lens.cpu().numpy().astype(np.int64)
        seq = self.seq.cpu().numpy()
        return [seq[b, :int(self.tot[b])].tolist() for b in range(self.B)]


class _WindowDecoder:
    """Next tokens past context_size, as the reference's generate_text makes
    them (generate.py:29-69): each from a full forward of the last
    context_size tokens at positions 0..context_size-1 (one prefill on a
    one-sequence cache, logits of its last row), then greedy or sample_token
    over the tokens so far."""

    def __init__(self, model: TransformerModel, max_len: int, sampling, seed: int):
        tm = model.tm_params
        self.model = model
        self.ctx_len = tm.context_size
        self.cache = model.new_cache(1)
        self.bufs = model.buffers(1)
        self.seq = torch.zeros((1, max(max_len, 1)), dtype=torch.int32, device=model.ctx.device)
        self.lens = torch.zeros(1, dtype=torch.int32, device=model.ctx.device)
        self.sampling = sampling
        self.seed = seed
        self.greedy = sampling[0] == 0.0 and sampling[4] == 1.0

    def next_token(self, tokens: List[int]) -> int:
        m, bf = self.model, self.bufs
        L = _lib.lib()
        s = _lib.stream_handle(m.ctx.device)
        self.cache.current_len = 0
        m.prefill(self.cache, np.asarray([tokens[-self.ctx_len:]], np.int64))
        if self.greedy:
            _lib.check(L.skv_argmax(bf.argmax.data_ptr(), bf.logits.data_ptr(), 1,
                                    m.tm_params.vocab_size, bf.arg_ws.data_ptr(),
                                    bf.arg_ws.numel(), s), "skv_argmax")
        else:
            n = len(tokens)
            self.seq[0, :n].copy_(torch.tensor(tokens, dtype=torch.int32))
            self.lens.fill_(n)
            T, k, p, mp, pen, win = self.sampling
            _lib.check(L.skv_sample(bf.argmax.data_ptr(), None, bf.logits.data_ptr(),
                                    self.seq.data_ptr(), self.seq.shape[1], self.lens.data_ptr(),
                                    1, m.tm_params.vocab_size, T, k, p, mp, pen, win, self.seed,
                                    bf.samp_ws.data_ptr(), bf.samp_ws.numel(), s), "skv_sample")
        return int(bf.argmax[0].item())


def generate_text(model: TransformerModel, prompt_tokens, max_tokens=100, temperature=1.0,
                  top_k=0, top_p=1.0, min_p=0.0, repetition_penalty=1.0, repetition_window=64,
                  use_graph: bool = True, seed: int = 42):
    """Generate max_tokens tokens after prompt_tokens (generate.py:8-71's
    signature and defaults); returns prompt + generated tokens as a list of
    ints. temperature = 0 is greedy; otherwise each token is drawn on the
    device from sample_token's filtered distribution (jax_backend.py:413-515)
    with a uniform keyed by (seed, position) -- the reference's jax.random
    stream itself is not reproduced. Up to context_size tokens the prompt is
    prefilled and the rest decoded on the cache; past it, every token comes
    from a full forward of the last context_size tokens, the reference's
    sliding window (generate.py:30-33)."""
    prompt = [int(t) for t in prompt_tokens]
    if max_tokens <= 0:
        return prompt
    tm = model.tm_params
    if not prompt:
        raise ValueError("every prompt needs at least one token")
    if min(prompt) < 0 or max(prompt) >= tm.vocab_size:
        raise ValueError("prompt token out of the vocabulary")
    total = len(prompt) + int(max_tokens)
    sampling = dict(temperature=temperature, top_k=top_k, top_p=top_p, min_p=min_p,
                    repetition_penalty=repetition_penalty, repetition_window=repetition_window,
                    seed=seed)
    if len(prompt) < tm.context_size:
        g = Generator(model, [prompt], min(total, tm.context_size), use_graph=use_graph,
                      **sampling)
        tokens = g.run()[0]
        if len(tokens) == total:
            return tokens
        win = _WindowDecoder(model, total, g.sampling, g.seed)
    else:
        Generator(model, [prompt[:1]], 1, **sampling)  # the same argument checks
        tokens = list(prompt)
        win = _WindowDecoder(model, total, (float(temperature), int(top_k), float(top_p),
                                            float(min_p), float(repetition_penalty),
                                            int(repetition_window)),
                             int(seed) & ((1 << 64) - 1))
    while len(tokens) < total:
        tokens.append(win.next_token(tokens))
    return tokens


def generate_batch(model: TransformerModel, prompts: Sequence[Sequence[int]], total_len,
                   use_graph: bool = True, **sampling) -> List[List[int]]:
    """Generation of a ragged batch until each sequence holds total_len
    tokens (an int or one per sequence, at most context_size); greedy unless
    sampling parameters (temperature, top_k, top_p, min_p, repetition_penalty,
    repetition_window, seed) are given."""
    return Generator(model, prompts, total_len, use_graph=use_graph, **sampling).run()
