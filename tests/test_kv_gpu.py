"""Parity of the HIP KV-cache path (append + split-K decode attention) with the
CPU oracle, through the drop-in API and the C ABI. Needs the MI355X.

Tolerances (the north star's): outputs within 1e-4 relative error for fp32
storage and 2e-2 for bf16 storage with fp32 accumulation, relative error
taken norm-wise per (sequence, head) against the float64 oracle fed the same
(bf16-rounded) K/V. Positions, lengths and appended cache bytes: bit-exact.
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN, banner
from oracle import kv_oracle as ko

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-4
BF16_TOL = 2e-2


def _gpu():
    from simple_llm_amd.gpu import gpu
    return gpu


def rel_err(got: np.ndarray, want: np.ndarray) -> float:
    """max over (b, h) of ||got - want|| / ||want|| (last axis = head_dim)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    num = np.linalg.norm(got - want, axis=-1)
    den = np.maximum(np.linalg.norm(want, axis=-1), 1e-30)
    return float((num / den).max())


def to_dev(x: np.ndarray, dtype=torch.float32, dev="cuda"):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev).to(dtype)


def cache_host(layer, cache, dtype=np.float32):
    """Device cache of one layer as a host array [B, T_cap, Hkv, D] (or pool)."""
    k = layer.k_cache.buffer.detach().float().cpu().numpy()
    v = layer.v_cache.buffer.detach().float().cpu().numpy()
    shp = (-1, cache.n_kv_heads, cache.head_dim)
    if not cache.paged:
        shp = (cache.batch_size, cache.max_seq_len) + shp[1:]
    return k.reshape(shp), v.reshape(shp)


# ---------------------------------------------------------------------------
# The reference's own KV test, replayed through the drop-in API
# ---------------------------------------------------------------------------


def test_reference_kv_cache_operations(gpu_ctx):
    """test_kv_cache_operations (simple-llm/src/gpu_test.py:2200-2406)."""
    banner("reference kv_cache_operations KAT")
    gpu = _gpu()
    ctx = gpu_ctx
    z = np.load(os.path.join(GOLDEN, "kv_kat_seed42.npz"))
    B, T_cap, n_layers, H, D = (int(x) for x in z["config"])
    E = H * D
    cache = gpu.kv_cache_create(ctx, gpu.KVCacheConfig(batch_size=B, max_seq_len=T_cap,
                                                       n_layers=n_layers, n_heads=H, head_dim=D))
    assert len(cache.layers) == n_layers
    assert cache.current_len == 0
    cache.current_len = 50
    gpu.kv_cache_reset(cache)
    assert cache.current_len == 0
    for step in range(1, 6):
        k = gpu.gpu_buffer_2d_create(ctx, B, E, z["k_steps"][step - 1].reshape(B, E))
        v = gpu.gpu_buffer_2d_create(ctx, B, E, z["v_steps"][step - 1].reshape(B, E))
        gpu.batch_begin(ctx)
        gpu.kv_cache_update(ctx, cache, 0, k, v)
        gpu.batch_commit(ctx)
        assert cache.current_len == step
    q = gpu.gpu_buffer_2d_create(ctx, B, E, z["q"].reshape(B, E))
    o = gpu.gpu_buffer_2d_create(ctx, B, E)
    gpu.batch_begin(ctx)
    gpu.attention_with_kv_cache(ctx, cache, 0, q, o)
    gpu.batch_commit(ctx)
    out = np.zeros((B, E), np.float32)
    gpu.gpu_buffer_2d_read(ctx, o, out)
    want = z["expected_o"].reshape(B, E)
    # the reference's own comparison (gpu_test.py:83-85, :2431) and the north star's
    assert np.allclose(out, want, rtol=1e-4, atol=1e-3)
    assert rel_err(out.reshape(B, H, D), want.reshape(B, H, D)) < FP32_TOL
    # device lengths and cache bytes: bit-exact against the oracle's scatter
    assert cache.layers[0].lens.cpu().tolist() == [5, 5]
    assert cache.layers[1].lens.cpu().tolist() == [0, 0]
    kc, vc = cache_host(cache.layers[0], cache)
    kw = np.zeros_like(kc)
    vw = np.zeros_like(vc)
    lens = np.zeros(B, np.int64)
    for s in range(5):
        lens = ko.append(kw, vw, z["k_steps"][s], z["v_steps"][s], lens)
    np.testing.assert_array_equal(kc, kw)
    np.testing.assert_array_equal(vc, vw)


def test_update_errors_match_reference(gpu_ctx):
    gpu = _gpu()
    ctx = gpu_ctx
    cache = gpu.kv_cache_create(ctx, gpu.KVCacheConfig(2, 3, 1, 2, 64))
    E = 128
    k = gpu.gpu_buffer_2d_create(ctx, 2, E)
    with pytest.raises(ValueError, match="out of range"):
        gpu.kv_cache_update(ctx, cache, 1, k, k)
    with pytest.raises(ValueError, match="Cache is empty"):
        gpu.attention_with_kv_cache(ctx, cache, 0, k, k)
    with pytest.raises(ValueError, match="new_k shape mismatch"):
        gpu.kv_cache_update(ctx, cache, 0, gpu.gpu_buffer_2d_create(ctx, 1, E), k)
    for _ in range(3):
        gpu.kv_cache_update(ctx, cache, 0, k, k)
    with pytest.raises(ValueError, match="Cache is full"):
        gpu.kv_cache_update(ctx, cache, 0, k, k)
    gpu.batch_begin(ctx)
    gpu.batch_commit(ctx)
    with pytest.raises(RuntimeError, match="Batch already submitted"):
        gpu.batch_commit(ctx)


# ---------------------------------------------------------------------------
# Append: bit-exact
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("cache_dt,in_dt", [(torch.float32, torch.float32),
                                            (torch.bfloat16, torch.float32),
                                            (torch.bfloat16, torch.bfloat16),
                                            (torch.float32, torch.bfloat16)])
@pytest.mark.parametrize("paged", [False, True])
def test_append_bit_exact(gpu_ctx, cache_dt, in_dt, paged):
    banner(f"append cache={cache_dt} in={in_dt} paged={paged}")
    gpu = _gpu()
    ctx = gpu_ctx
    rng = np.random.default_rng(7)
    B, T, Hkv, D = 5, 48, 2, 128
    cfg = gpu.KVCacheConfig(B, T, 1, 2 * Hkv, D, n_kv_heads=Hkv, dtype=cache_dt,
                            block_size=16 if paged else 0)
    cache = gpu.kv_cache_create(ctx, cfg)
    if paged:
        table = rng.permutation(cache.n_blocks).reshape(B, -1).astype(np.int32)
        gpu.kv_cache_set_block_table(cache, torch.from_numpy(table))
    start = np.array([0, 7, 47, 48, 20])
    cache.layers[0].lens.copy_(torch.from_numpy(start.astype(np.int32)))
    cache.layers[0].host_lens[:] = start
    kw = np.zeros((B, T, Hkv, D), np.float32)
    vw = np.zeros_like(kw)
    lens = start.copy()
    sdt = "bf16" if cache_dt == torch.bfloat16 else "fp32"
    for _ in range(3):
        k = rng.standard_normal((B, Hkv, D)).astype(np.float32) * 3
        v = rng.standard_normal((B, Hkv, D)).astype(np.float32)
        if in_dt == torch.bfloat16:  # the input itself is bf16
            k, v = ko.bf16_round(k), ko.bf16_round(v)
        host = gpu.kv_cache_append(ctx, cache, 0, to_dev(k, in_dt), to_dev(v, in_dt))
        lens = ko.append(kw, vw, k, v, lens, dtype=sdt)
        np.testing.assert_array_equal(host, lens)
    np.testing.assert_array_equal(cache.layers[0].lens.cpu().numpy(), lens)
    kc, vc = cache_host(cache.layers[0], cache)
    if paged:
        kc = ko.paged_gather(kc, table, lens, 16, T)
        vc = ko.paged_gather(vc, table, lens, 16, T)
        for b in range(B):
            kw[b, lens[b]:] = 0
            vw[b, lens[b]:] = 0
    np.testing.assert_array_equal(kc, kw)
    np.testing.assert_array_equal(vc, vw)


def test_append_chunk_and_advance(gpu_ctx):
    from simple_llm_amd import _lib
    banner("append_chunk + advance")
    rng = np.random.default_rng(3)
    B, T, H, D, C = 3, 40, 2, 64, 9
    kc = torch.zeros((B, T, H, D), device="cuda")
    vc = torch.zeros_like(kc)
    lens = torch.tensor([0, 30, 35], dtype=torch.int32, device="cuda")
    n_new = torch.tensor([9, 4, 9], dtype=torch.int32, device="cuda")
    k = rng.standard_normal((B, C, H, D)).astype(np.float32)
    v = rng.standard_normal((B, C, H, D)).astype(np.float32)
    L = _lib.lib()
    s = _lib.stream_handle()
    kd, vd = to_dev(k), to_dev(v)  # keep both alive until the launch is enqueued
    rc = L.skv_append_chunk(kc.data_ptr(), vc.data_ptr(), kd.data_ptr(), vd.data_ptr(),
                            lens.data_ptr(), n_new.data_ptr(), B, C, H, D, T, 0, 0, s)
    _lib.check(rc, "append_chunk")
    _lib.check(L.skv_advance(lens.data_ptr(), n_new.data_ptr(), 0, B, T, s), "advance")
    kw = np.zeros((B, T, H, D), np.float32)
    vw = np.zeros_like(kw)
    ko.append_chunk(kw, vw, k, v, np.array([0, 30, 35]), np.array([9, 4, 9]))
    np.testing.assert_array_equal(kc.cpu().numpy(), kw)
    np.testing.assert_array_equal(vc.cpu().numpy(), vw)
    assert lens.cpu().tolist() == [9, 34, 40]  # the third one is clamped at T


# ---------------------------------------------------------------------------
# Decode attention
# ---------------------------------------------------------------------------


def _filled_cache(gpu, ctx, rng, B, T, Hq, Hkv, D, dtype, lens, paged=False, scale_kv=1.0):
    cfg = gpu.KVCacheConfig(B, T, 1, Hq, D, n_kv_heads=Hkv, dtype=dtype,
                            block_size=16 if paged else 0)
    cache = gpu.kv_cache_create(ctx, cfg)
    k = (rng.standard_normal((B, T, Hkv, D)) * scale_kv).astype(np.float32)
    v = rng.standard_normal((B, T, Hkv, D)).astype(np.float32)
    if dtype == torch.bfloat16:
        k, v = ko.bf16_round(k), ko.bf16_round(v)
    table = None
    layer = cache.layers[0]
    if paged:
        table = rng.permutation(cache.n_blocks).reshape(B, -1).astype(np.int32)
        gpu.kv_cache_set_block_table(cache, torch.from_numpy(table))
        pool_k = np.zeros((cache.n_blocks * 16, Hkv, D), np.float32)
        pool_v = np.zeros_like(pool_k)
        for b in range(B):
            for t in range(T):
                r = table[b, t // 16] * 16 + t % 16
                pool_k[r], pool_v[r] = k[b, t], v[b, t]
        layer.k_cache.buffer.copy_(to_dev(pool_k.reshape(-1, Hkv * D), dtype))
        layer.v_cache.buffer.copy_(to_dev(pool_v.reshape(-1, Hkv * D), dtype))
    else:
        layer.k_cache.buffer.copy_(to_dev(k.reshape(-1, Hkv * D), dtype))
        layer.v_cache.buffer.copy_(to_dev(v.reshape(-1, Hkv * D), dtype))
    layer.lens.copy_(torch.from_numpy(np.asarray(lens, np.int32)))
    layer.host_lens[:] = lens
    return cache, k, v, table


def _decode(gpu, ctx, cache, q_np, q_dtype=torch.float32, out_dtype=torch.float32, **kw):
    q = to_dev(q_np, q_dtype)
    out = torch.empty(q.shape, dtype=out_dtype, device="cuda")
    gpu.decode_attention(ctx, cache, 0, q, out, **kw)
    return out.float().cpu().numpy()


CASES = [
    # B, T, Hq, Hkv, D, dtype, paged
    (8, 2048, 8, 8, 64, torch.float32, False),   # C2 shape
    (4, 4096, 16, 16, 128, torch.bfloat16, False),  # C4 head shape, shorter
    (6, 1500, 32, 8, 128, torch.bfloat16, True),  # C5 GQA paged
    (3, 700, 8, 4, 64, torch.float32, False),
    (3, 700, 16, 2, 128, torch.float32, True),
    (2, 900, 16, 2, 64, torch.bfloat16, False),  # G = 8
    (16, 1024, 12, 12, 64, torch.float32, False),  # C3 head shape
]


@pytest.mark.parametrize("B,T,Hq,Hkv,D,dtype,paged", CASES)
def test_decode_matches_oracle(gpu_ctx, B, T, Hq, Hkv, D, dtype, paged):
    banner(f"decode B={B} T={T} Hq={Hq} Hkv={Hkv} D={D} {dtype} paged={paged}")
    gpu = _gpu()
    rng = np.random.default_rng(B * 1000 + T)
    lens = rng.integers(1, T + 1, B)
    lens[0] = T
    cache, k, v, _ = _filled_cache(gpu, gpu_ctx, rng, B, T, Hq, Hkv, D, dtype, lens, paged)
    q = (rng.standard_normal((B, Hq, D))).astype(np.float32)
    got = _decode(gpu, gpu_ctx, cache, q)
    want = ko.decode_attention(q, k, v, lens)
    err = rel_err(got, want)
    print(f"rel_err={err:.3e}")
    assert err < (BF16_TOL if dtype == torch.bfloat16 else FP32_TOL)
    # the bf16 path accumulates in fp32 over the same rounded inputs
    assert err < 1e-4


def test_paged_equals_contiguous_bitwise(gpu_ctx):
    """C5's check: the paged cache gives the result of the same data gathered
    into a contiguous cache (same kernel arithmetic, so bit-identical)."""
    banner("paged vs contiguous")
    gpu = _gpu()
    rng = np.random.default_rng(11)
    B, T, Hq, Hkv, D = 8, 640, 32, 8, 128
    lens = np.clip(np.exp(rng.normal(np.log(300), 0.8, B)), 16, T).astype(np.int64)
    cp, k, v, _ = _filled_cache(gpu, gpu_ctx, np.random.default_rng(5), B, T, Hq, Hkv, D,
                                torch.bfloat16, lens, paged=True)
    cc, k2, v2, _ = _filled_cache(gpu, gpu_ctx, np.random.default_rng(5), B, T, Hq, Hkv, D,
                                  torch.bfloat16, lens, paged=False)
    np.testing.assert_array_equal(k, k2)
    q = rng.standard_normal((B, Hq, D)).astype(np.float32)
    a = _decode(gpu, gpu_ctx, cp, q, max_len=T)
    b = _decode(gpu, gpu_ctx, cc, q, max_len=T)
    np.testing.assert_array_equal(a, b)


# fp32 at 256-token chunks; bf16 (4 tokens in flight per lane) at the
# 512-token chunks the plan gives long MHA streams
@pytest.mark.parametrize("dtype,chunk", [(torch.float32, 256), (torch.bfloat16, 512)])
@pytest.mark.parametrize("L", [1, 2, 15, 16, 17, 255, 256, 257, 511, 513, 1023, 1024, 1025, 2047,
                               2048])
def test_decode_chunk_boundaries(gpu_ctx, L, dtype, chunk):
    banner(f"decode boundary L={L} {dtype} chunk={chunk}")
    gpu = _gpu()
    gpu_ctx.config.decode_chunk_tokens = chunk
    try:
        rng = np.random.default_rng(L)
        B, T, H, D = 2, 2048, 4, 128
        lens = np.array([L, max(1, L // 2)])
        cache, k, v, _ = _filled_cache(gpu, gpu_ctx, rng, B, T, H, H, D, dtype, lens)
        q = rng.standard_normal((B, H, D)).astype(np.float32)
        got = _decode(gpu, gpu_ctx, cache, q)
        want = ko.decode_attention(q, k, v, lens)
        assert rel_err(got, want) < FP32_TOL
        if L == 1:  # one token: exactly its value row
            np.testing.assert_array_equal(got[0], v[0, 0])
    finally:
        gpu_ctx.config.decode_chunk_tokens = 0


def test_decode_empty_sequence_and_plan_overflow(gpu_ctx):
    banner("decode len=0 and under-sized plan")
    gpu = _gpu()
    rng = np.random.default_rng(2)
    B, T, H, D = 3, 1024, 2, 64
    lens = np.array([0, 300, 1024])
    cache, k, v, _ = _filled_cache(gpu, gpu_ctx, rng, B, T, H, H, D, torch.float32, lens)
    q = rng.standard_normal((B, H, D)).astype(np.float32)
    got = _decode(gpu, gpu_ctx, cache, q)
    assert not got[0].any()
    want = ko.decode_attention(q, k, v, lens)
    assert rel_err(got[1:], want[1:]) < FP32_TOL
    # the Python API rejects a max_len below the fills before any GPU work
    with pytest.raises(ValueError, match="max_len=256 is below the longest fill 1024"):
        _decode(gpu, gpu_ctx, cache, q, max_len=256)
    # the C ABI with a plan sized for max_len=256: its workgroups cover
    # B * 256 = 768 tokens of the flat token stream [0 | 300 | 1024].
    # Sequence 1 (tokens 0-299) fits and is exact although longer than
    # max_len; sequence 2 runs past the planned grid and is flagged with NaN,
    # never read out of bounds.
    import ctypes
    from simple_llm_amd import _lib
    L = _lib.lib()
    chunk, nch = ctypes.c_int(), ctypes.c_int()
    _lib.check(L.skv_decode_plan(B, H, H, D, _lib.F32, 256, 0, 256, ctypes.byref(chunk),
                                 ctypes.byref(nch)), "plan")
    need = L.skv_decode_workspace_bytes(B, H, D, nch.value)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    qd = to_dev(q)
    out = torch.empty_like(qd)
    layer = cache.layers[0]
    _lib.check(L.skv_decode_attn(out.data_ptr(), qd.data_ptr(), layer.k_cache.buffer.data_ptr(),
                                 layer.v_cache.buffer.data_ptr(), layer.lens.data_ptr(), B, H, H,
                                 D, T, float(D ** -0.5), chunk.value, nch.value, ws.data_ptr(),
                                 need, 0, 0, 0, _lib.stream_handle()), "decode")
    got = out.cpu().numpy()
    assert not got[0].any()
    assert rel_err(got[1:2], want[1:2]) < FP32_TOL
    assert np.isnan(got[2]).all()


@pytest.mark.parametrize("kind", ["shift+50", "peaky*100", "zeros"])
def test_decode_softmax_stability(gpu_ctx, kind):
    """The reference's softmax stability cases (gpu_test.py:1647-1657) applied
    to the attention scores."""
    banner(f"decode stability {kind}")
    gpu = _gpu()
    rng = np.random.default_rng(4)
    B, T, H, D = 2, 3000, 4, 128
    lens = np.array([3000, 1777])
    cache, k, v, _ = _filled_cache(gpu, gpu_ctx, rng, B, T, H, H, D, torch.float32, lens)
    q = rng.standard_normal((B, H, D)).astype(np.float32)
    if kind == "peaky*100":
        q *= 100.0 / np.sqrt(D)
    elif kind == "zeros":
        q[:] = 0
    elif kind == "shift+50":  # add 50 to every score: keys += 50*sqrt(D) q/|q|^2
        c = 50.0 * np.sqrt(D) * q / (q * q).sum(-1, keepdims=True)
        k = (k + c[:, None]).astype(np.float32)
        cache.layers[0].k_cache.buffer.copy_(to_dev(k.reshape(-1, H * D)))
    got = _decode(gpu, gpu_ctx, cache, q)
    want = ko.decode_attention(q, k, v, lens)
    assert np.isfinite(got).all()
    tol = 2e-4 if kind == "peaky*100" else FP32_TOL  # |s| ~ 1e3: fp32 rounding of s
    assert rel_err(got, want) < tol
    if kind == "zeros":  # uniform weights: mean of V
        np.testing.assert_allclose(got[1], v[1, :1777].astype(np.float64).mean(0), atol=1e-5)


@pytest.mark.parametrize("q_dt,o_dt", [(torch.bfloat16, torch.float32),
                                       (torch.float32, torch.bfloat16),
                                       (torch.bfloat16, torch.bfloat16)])
def test_decode_io_dtypes(gpu_ctx, q_dt, o_dt):
    banner(f"decode q={q_dt} out={o_dt}")
    gpu = _gpu()
    rng = np.random.default_rng(9)
    B, T, H, D = 2, 1000, 8, 128
    lens = np.array([1000, 640])
    cache, k, v, _ = _filled_cache(gpu, gpu_ctx, rng, B, T, H, H, D, torch.bfloat16, lens)
    q = rng.standard_normal((B, H, D)).astype(np.float32)
    qr = ko.bf16_round(q) if q_dt == torch.bfloat16 else q
    got = _decode(gpu, gpu_ctx, cache, qr, q_dtype=q_dt, out_dtype=o_dt)
    want = ko.decode_attention(qr, k, v, lens)
    assert rel_err(got, want) < (BF16_TOL if o_dt == torch.bfloat16 else 1e-4)


def test_decode_deterministic(gpu_ctx):
    banner("decode determinism")
    gpu = _gpu()
    rng = np.random.default_rng(12)
    B, T, H, D = 4, 5000, 16, 128
    lens = rng.integers(1000, T + 1, B)
    cache, k, v, _ = _filled_cache(gpu, gpu_ctx, rng, B, T, H, H, D, torch.bfloat16, lens)
    q = rng.standard_normal((B, H, D)).astype(np.float32)
    a = _decode(gpu, gpu_ctx, cache, q)
    b = _decode(gpu, gpu_ctx, cache, q)
    np.testing.assert_array_equal(a, b)


def test_decode_full_size_c4_sampled(gpu_ctx):
    """C4 at full size (B=4, H=16, D=128, T_cap=32768, bf16, filled to 32000),
    one append + decode step; the oracle checks sampled (b, h) pairs."""
    banner("decode C4 full size, sampled oracle")
    gpu = _gpu()
    B, T, H, D, fill = 4, 32768, 16, 128, 32000
    cache = gpu.kv_cache_create(gpu_ctx, gpu.KVCacheConfig(B, T, 1, H, D,
                                                           dtype=torch.bfloat16))
    g = torch.Generator(device="cuda").manual_seed(0)
    layer = cache.layers[0]
    kv = layer.k_cache.buffer.view(B, T, H, D)
    vv = layer.v_cache.buffer.view(B, T, H, D)
    kv[:, :fill].copy_(torch.randn((B, fill, H, D), generator=g, device="cuda"))
    vv[:, :fill].copy_(torch.randn((B, fill, H, D), generator=g, device="cuda"))
    cache.current_len = fill
    rng = np.random.default_rng(0)
    kn = rng.standard_normal((B, H, D)).astype(np.float32)
    vn = rng.standard_normal((B, H, D)).astype(np.float32)
    q = rng.standard_normal((B, H, D)).astype(np.float32)
    gpu.kv_cache_append(gpu_ctx, cache, 0, to_dev(kn), to_dev(vn))
    got = _decode(gpu, gpu_ctx, cache, q)
    assert cache.layers[0].lens.cpu().tolist() == [fill + 1] * B
    for b, h in [(0, 0), (1, 7), (2, 15), (3, 3)]:
        kh = kv[b, :fill + 1, h].float().cpu().numpy()[:, None, :]
        vh = vv[b, :fill + 1, h].float().cpu().numpy()[:, None, :]
        np.testing.assert_array_equal(kh[fill, 0], ko.bf16_round(kn[b, h]))
        want = ko.decode_attention(q[b:b + 1, h:h + 1], kh[None], vh[None], [fill + 1])
        assert rel_err(got[b:b + 1, h:h + 1], want) < 1e-4


def test_decode_full_size_c5(gpu_ctx):
    """C5 at full size, built as bench.py builds it: 64 sequences, 32 query
    heads over 8 kv heads, D=128, bf16 16-token pages under a seeded random
    page table, lognormal lengths (median 1500, sigma 0.8, clipped to
    [16, 8192]). The paged decode equals the same data gathered into a
    contiguous cache bit for bit (C5's own check), and the C restatement of
    the oracle on the same bf16 values within 1e-4."""
    banner("decode C5 full size")
    from oracle import c_oracle
    gpu = _gpu()
    B, Hq, Hkv, D, bs = 64, 32, 8, 128, 16
    r = np.random.default_rng(0)
    lens = np.clip(np.exp(r.normal(np.log(1500), 0.8, B)), 16, 8192).astype(np.int64)
    max_seq = 8192
    need = -(-lens // bs)
    n_blocks = int(need.sum())
    cache = gpu.kv_cache_create(gpu_ctx, gpu.KVCacheConfig(B, max_seq, 1, Hq, D, n_kv_heads=Hkv,
                                                           dtype=torch.bfloat16, block_size=bs,
                                                           n_blocks=n_blocks))
    perm = r.permutation(n_blocks).astype(np.int32)
    table = np.zeros((B, -(-max_seq // bs)), np.int32)
    o = 0
    for b in range(B):
        table[b, :need[b]] = perm[o:o + need[b]]
        o += need[b]
    gpu.kv_cache_set_block_table(cache, torch.from_numpy(table))
    layer = cache.layers[0]
    g = torch.Generator(device="cuda").manual_seed(0)
    for buf in (layer.k_cache.buffer, layer.v_cache.buffer):
        buf.copy_(torch.randn(buf.shape, generator=g, device="cuda"))
    layer.lens.copy_(torch.from_numpy(lens.astype(np.int32)))
    layer.host_lens[:] = lens
    q = r.standard_normal((B, Hq, D)).astype(np.float32)
    got = _decode(gpu, gpu_ctx, cache, q, max_len=int(lens.max()))
    # the pool gathered into a contiguous [B, T, H_kv, D] cache
    nb = int(need.max())
    tab = torch.from_numpy(table[:, :nb].astype(np.int64)).cuda()
    kc = layer.k_cache.buffer.view(n_blocks, bs, Hkv, D)[tab].reshape(B, nb * bs, Hkv, D)
    vc = layer.v_cache.buffer.view(n_blocks, bs, Hkv, D)[tab].reshape(B, nb * bs, Hkv, D)
    cc = gpu.kv_cache_create(gpu_ctx, gpu.KVCacheConfig(B, nb * bs, 1, Hq, D, n_kv_heads=Hkv,
                                                        dtype=torch.bfloat16))
    cc.layers[0].k_cache.buffer.copy_(kc.reshape(-1, Hkv * D))
    cc.layers[0].v_cache.buffer.copy_(vc.reshape(-1, Hkv * D))
    cc.layers[0].lens.copy_(torch.from_numpy(lens.astype(np.int32)))
    cc.layers[0].host_lens[:] = lens
    np.testing.assert_array_equal(got, _decode(gpu, gpu_ctx, cc, q, max_len=int(lens.max())))
    bits = lambda x: x.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    want = c_oracle.decode_attn(q, bits(kc), bits(vc), lens, cache_bf16=True)
    err = rel_err(got, want)
    print(f"rel_err={err:.3e}")
    assert err < 1e-4  # the same bf16 values, fp32 accumulation on both sides


# ---------------------------------------------------------------------------
# Fused append + decode attention (skv_append_decode_attn)
# ---------------------------------------------------------------------------

def test_launches_follow_torch_current_stream(gpu_ctx):
    """The ops enqueue on torch's current stream: the raw stream query the
    launches use equals torch's Stream handle, also inside a stream context."""
    from simple_llm_amd import _lib
    dev = gpu_ctx.device
    idx = dev.index or 0
    assert _lib.stream_handle(dev) == torch.cuda.current_stream(dev).cuda_stream
    assert _lib.stream_handle(idx) == torch.cuda.current_stream(dev).cuda_stream
    side = torch.cuda.Stream(device=dev)  # default priority
    with torch.cuda.stream(side):
        assert _lib.stream_handle(dev) == side.cuda_stream
        assert side.cuda_stream != torch.cuda.default_stream(dev).cuda_stream
    assert _lib.stream_handle(dev) == torch.cuda.current_stream(dev).cuda_stream


FUSED_CASES = [
    # B, T, Hq, Hkv, D, cache dtype, input dtype, paged
    (8, 300, 8, 8, 64, torch.float32, torch.float32, False),      # C2 head shape
    (4, 600, 16, 16, 128, torch.bfloat16, torch.float32, False),  # C4 head shape, fp32 input
    (6, 400, 32, 8, 128, torch.bfloat16, torch.bfloat16, True),   # C5 GQA paged
    (3, 200, 16, 2, 64, torch.bfloat16, torch.float32, False),    # G = 8
    (16, 128, 12, 12, 64, torch.float32, torch.float32, False),   # C3 head shape
]


@pytest.mark.parametrize("B,T,Hq,Hkv,D,cdt,idt,paged", FUSED_CASES)
def test_append_attend_equals_append_then_attend(gpu_ctx, B, T, Hq, Hkv, D, cdt, idt, paged):
    """Three steps of the fused call against skv_append + skv_decode_attn on a
    copy of the same cache: bit-identical caches and fills, outputs equal to
    fp32 rounding (the new token enters the online softmax in its own step),
    and against the oracle. One sequence starts empty and one full (skipped)."""
    banner(f"fused append+attend B={B} T={T} Hq={Hq} Hkv={Hkv} D={D} {cdt} in={idt} "
           f"paged={paged}")
    gpu = _gpu()
    rng = np.random.default_rng(B * 31 + T)
    lens = rng.integers(1, T - 4, B)
    lens[0], lens[-1] = 0, T  # an empty sequence and a full one
    ca, k, v, _ = _filled_cache(gpu, gpu_ctx, np.random.default_rng(7), B, T, Hq, Hkv, D, cdt,
                                lens, paged)
    cb, _, _, _ = _filled_cache(gpu, gpu_ctx, np.random.default_rng(7), B, T, Hq, Hkv, D, cdt,
                                lens, paged)
    kw, vw = k.copy(), v.copy()
    fills = lens.copy()
    for step in range(3):
        kn = rng.standard_normal((B, Hkv, D)).astype(np.float32)
        vn = rng.standard_normal((B, Hkv, D)).astype(np.float32)
        q = rng.standard_normal((B, Hq, D)).astype(np.float32)
        out_a = torch.empty((B, Hq, D), device="cuda")
        out_b = torch.empty_like(out_a)
        gpu.kv_cache_append(gpu_ctx, ca, 0, to_dev(kn, idt), to_dev(vn, idt))
        gpu.decode_attention(gpu_ctx, ca, 0, to_dev(q), out_a)
        got_fills = gpu.kv_cache_append_attend(gpu_ctx, cb, 0, to_dev(kn, idt), to_dev(vn, idt),
                                               to_dev(q), out_b)
        # the oracle's view: the same append rule and rounding
        knr = ko.bf16_round(kn) if (cdt == torch.bfloat16 or idt == torch.bfloat16) else kn
        vnr = ko.bf16_round(vn) if (cdt == torch.bfloat16 or idt == torch.bfloat16) else vn
        for b in range(B):
            if fills[b] < T:
                kw[b, fills[b]], vw[b, fills[b]] = knr[b], vnr[b]
                fills[b] += 1
        np.testing.assert_array_equal(got_fills, fills)
        np.testing.assert_array_equal(cb.layers[0].lens.cpu().numpy(), fills)
        np.testing.assert_array_equal(ca.layers[0].lens.cpu().numpy(), fills)
        ka, va = cache_host(ca.layers[0], ca)
        kb_, vb_ = cache_host(cb.layers[0], cb)
        np.testing.assert_array_equal(ka, kb_)
        np.testing.assert_array_equal(va, vb_)
        a_, b_ = out_a.cpu().numpy(), out_b.cpu().numpy()
        assert rel_err(b_, a_) < 1e-6, step
        want = ko.decode_attention(q, kw, vw, fills)
        assert rel_err(b_, want) < 1e-4, step


@pytest.mark.parametrize("variant", ["bench", "retiring"])
def test_c2_full_run_every_step_matches_c_oracle(gpu_ctx, variant):
    """C2 as the bench runs it (fp32 cache [8, 8, 2048, 64], start lengths
    U[1, 2047] from seed 0, 256 steps of append + attention through
    kv_cache_append_attend). Every step's output is checked against
    oracle/c/kv_attn_ref.c over a host mirror of the cache updated by the
    append rule, and the fills against that rule exactly. With seed 0 no
    sequence reaches 2048 within 256 steps (the longest starts at 1742), so
    the "retiring" variant starts four of the sequences at 2047, 1998, 1900
    and 1793: they reach 2048 at steps 1, 50, 148 and 255 and then retire (no
    append; their output stays attention over the full cache)."""
    banner(f"C2 full run ({variant}): 256 steps vs C oracle")
    from oracle import c_oracle
    gpu = _gpu()
    B, H, T, Dh, steps = 8, 8, 2048, 64, 256
    lens0 = np.random.default_rng(0).integers(1, 2048, B).astype(np.int64)
    if variant == "retiring":
        lens0[::2] = [2047, 1998, 1900, 1793]
    cache = gpu.kv_cache_create(gpu_ctx, gpu.KVCacheConfig(B, T, 1, H, Dh))
    layer = cache.layers[0]
    g = torch.Generator(device="cuda").manual_seed(0)
    layer.k_cache.buffer.copy_(torch.randn(layer.k_cache.buffer.shape, generator=g,
                                           device="cuda"))
    layer.v_cache.buffer.copy_(torch.randn(layer.v_cache.buffer.shape, generator=g,
                                           device="cuda"))
    layer.lens.copy_(torch.from_numpy(lens0.astype(np.int32)))
    layer.host_lens = lens0.copy()
    kc = layer.k_cache.buffer.cpu().numpy().reshape(B, T, H, Dh).copy()
    vc = layer.v_cache.buffer.cpu().numpy().reshape(B, T, H, Dh).copy()
    q_all = torch.randn((steps, B, H, Dh), generator=g, device="cuda")
    k_all = torch.randn((steps, B, H, Dh), generator=g, device="cuda")
    v_all = torch.randn((steps, B, H, Dh), generator=g, device="cuda")
    qs, ks, vs = q_all.cpu().numpy(), k_all.cpu().numpy(), v_all.cpu().numpy()
    out = torch.empty((B, H, Dh), device="cuda")
    lens = lens0.astype(np.int32).copy()
    worst = 0.0
    for n in range(steps):
        fills = gpu.kv_cache_append_attend(gpu_ctx, cache, 0, k_all[n], v_all[n], q_all[n], out,
                                           max_len=min(int(lens0.max()) + steps, T))
        for b in range(B):
            if lens[b] < T:
                kc[b, lens[b]], vc[b, lens[b]] = ks[n, b], vs[n, b]
                lens[b] += 1
        np.testing.assert_array_equal(fills, lens)
        want = c_oracle.decode_attn(qs[n], kc, vc, lens, cache_bf16=False)
        err = rel_err(out.cpu().numpy(), want)
        worst = max(worst, err)
        assert err < FP32_TOL, (n, err)
    np.testing.assert_array_equal(layer.lens.cpu().numpy(), lens)
    retired = int((lens == T).sum())
    print(f"worst rel_err over {steps} steps = {worst:.3e}; sequences retired: {retired}")
    assert retired == (0 if variant == "bench" else 4)


# ---------------------------------------------------------------------------
# The exact calls the benchmarks time, at their full sizes
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("n_split", [1, 2, 4])
@pytest.mark.parametrize("B,H,D,T,dt", [(1, 4, 64, 256, "f32"), (1, 4, 64, 256, "bf16"),
                                         (16, 12, 64, 1024, "f32"), (16, 12, 64, 1024, "bf16"),
                                         (3, 5, 128, 700, "bf16"), (5, 7, 64, 300, "f32"),
                                         (5, 7, 128, 300, "f32")])
def test_direct_attention_matches_oracle(gpu_ctx, B, H, D, T, dt, n_split):
    """skv_append_decode_attn_direct, the attention of the C1 (B=1, 4 x 64,
    context 256) and C3 (B=16, 12 x 64, context 1024) greedy steps, against
    the float64 oracle over a host mirror of the cache: empty, ragged, last
    free position, full (no append) and retired (negative fill: zero output)
    rows; the appended rows bit-exact and the fills left in place. With the
    row split over 2 or 4 workgroups (the last to finish merges), every call
    leaves the arrival counters at zero, so calls in a row stay right."""
    banner(f"direct attention vs oracle B={B} H={H} D={D} T={T} {dt} n_split={n_split}")
    from simple_llm_amd import _lib
    L = _lib.lib()
    s = _lib.stream_handle()
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    cdt = _lib.BF16 if dt == "bf16" else _lib.F32
    r = np.random.default_rng(B * 7 + T)
    kc = torch.from_numpy(r.standard_normal((B, T, H, D)).astype(np.float32)).cuda().to(tdt)
    vc = torch.from_numpy(r.standard_normal((B, T, H, D)).astype(np.float32)).cuda().to(tdt)
    kw = kc.float().cpu().numpy()
    vw = vc.float().cpu().numpy()
    # B = 1: one call per kind of row; B >= 5: every kind in one call, twice
    special = [0, int(r.integers(1, T - 1)), T - 1, T, -1]
    if B == 1:
        calls = [np.array([f]) for f in special]
    elif B < len(special):
        calls = [np.array(special[:B]), np.array(special[-B:])]
    else:
        calls = [np.concatenate([special, r.integers(0, T, B - len(special))])] * 2
    wsb = L.skv_decode_direct_workspace_bytes(B, H, D, n_split)
    ws = torch.zeros(max(wsb, 4), dtype=torch.uint8, device="cuda")
    for fills in calls:
        q, kn, vn = (r.standard_normal((B, H, D)).astype(np.float32) for _ in range(3))
        lens = to_dev(fills.astype(np.int32), torch.int32)
        out = torch.full((B, H, D), float("nan"), device="cuda")
        qd, knd, vnd = to_dev(q), to_dev(kn), to_dev(vn)  # held: the call reads them later
        _lib.check(L.skv_append_decode_attn_direct(
            out.data_ptr(), qd.data_ptr(), kc.data_ptr(), vc.data_ptr(), knd.data_ptr(),
            vnd.data_ptr(), lens.data_ptr(), B, H, D, T, D ** -0.5, cdt, _lib.F32, _lib.F32,
            _lib.F32, n_split, ws.data_ptr(), wsb, s), "skv_append_decode_attn_direct")
        torch.cuda.synchronize()
        att = np.zeros(B, np.int64)
        for b, f in enumerate(fills):
            if 0 <= f < T:
                kw[b, f] = ko.storage_round(kn[b], "bf16" if dt == "bf16" else "fp32")
                vw[b, f] = ko.storage_round(vn[b], "bf16" if dt == "bf16" else "fp32")
                att[b] = f + 1
            elif f >= T:
                att[b] = T
        np.testing.assert_array_equal(lens.cpu().numpy(), fills)  # no advance
        np.testing.assert_array_equal(kc.float().cpu().numpy(), kw)
        np.testing.assert_array_equal(vc.float().cpu().numpy(), vw)
        got = out.cpu().numpy()
        want = ko.decode_attention(q, kw, vw, att)
        live = att > 0
        err = rel_err(got[live], want[live]) if live.any() else 0.0
        print(f"fills={fills.tolist()[:6]} rel_err={err:.3e}")
        assert err < FP32_TOL  # the same (rounded) cache values on both sides
        assert not got[~live].any()  # retired rows give 0
        if n_split > 1:  # every arrival counter (the fixed 256 KiB block) is back at zero
            assert not ws[:65536 * 4].any()


def test_direct_attention_split_shapes_share_a_workspace(gpu_ctx):
    """Split calls of different shapes (B x H, head dim, dtype) through one
    zero-filled workspace, interleaved: the arrival counters sit in a fixed
    block before every shape's partials, so no call's partials land on
    another's counters; each output matches the float64 oracle and the
    counters read zero after every call."""
    banner("direct attention: shapes sharing one workspace")
    from simple_llm_amd import _lib
    L = _lib.lib()
    s = _lib.stream_handle()
    shapes = [(16, 12, 64, 300, torch.float32), (2, 3, 128, 200, torch.bfloat16),
              (40, 8, 64, 100, torch.float32)]
    need = max(L.skv_decode_direct_workspace_bytes(B, H, D, 4) for B, H, D, _, _ in shapes)
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    r = np.random.default_rng(5)
    for rnd in range(2):
        for B, H, D, T, tdt in shapes:
            kc = torch.from_numpy(r.standard_normal((B, T, H, D)).astype(np.float32)).cuda().to(tdt)
            vc = torch.from_numpy(r.standard_normal((B, T, H, D)).astype(np.float32)).cuda().to(tdt)
            fills = r.integers(0, T, B).astype(np.int32)
            q, kn, vn = (r.standard_normal((B, H, D)).astype(np.float32) for _ in range(3))
            qd, knd, vnd = to_dev(q), to_dev(kn), to_dev(vn)
            lens = to_dev(fills, torch.int32)
            out = torch.full((B, H, D), float("nan"), device="cuda")
            cdt = _lib.BF16 if tdt == torch.bfloat16 else _lib.F32
            _lib.check(L.skv_append_decode_attn_direct(
                out.data_ptr(), qd.data_ptr(), kc.data_ptr(), vc.data_ptr(), knd.data_ptr(),
                vnd.data_ptr(), lens.data_ptr(), B, H, D, T, D ** -0.5, cdt, _lib.F32, _lib.F32,
                _lib.F32, 4, ws.data_ptr(), need, s), "skv_append_decode_attn_direct")
            torch.cuda.synchronize()
            kw, vw = kc.float().cpu().numpy(), vc.float().cpu().numpy()  # the appended rows in place
            want = ko.decode_attention(q, kw, vw, fills.astype(np.int64) + 1)
            err = rel_err(out.cpu().numpy(), want)
            print(f"round {rnd} B={B} H={H} D={D} {tdt}: rel_err={err:.3e}")
            assert err < FP32_TOL
            assert not ws[:65536 * 4].any()


def _c4_bench_cache(gpu, ctx):
    """The C4 cache as bench.py builds it: [4, 32768, 16, 128] bf16, each
    sequence filled to 32000 with N(0, 1) from torch generator seed 0."""
    B, T, H, D, fill = 4, 32768, 16, 128, 32000
    cache = gpu.kv_cache_create(ctx, gpu.KVCacheConfig(B, T, 1, H, D, dtype=torch.bfloat16))
    layer = cache.layers[0]
    g = torch.Generator(device="cuda").manual_seed(0)
    kv = layer.k_cache.buffer.view(B, T, H, D)
    vv = layer.v_cache.buffer.view(B, T, H, D)
    for b in range(B):
        kv[b, :fill].copy_(torch.randn((fill, H, D), generator=g, device="cuda"))
        vv[b, :fill].copy_(torch.randn((fill, H, D), generator=g, device="cuda"))
    cache.current_len = fill
    return cache, kv, vv


def test_append_attend_full_size_c4_bench_plan(gpu_ctx):
    """Three steps of kv_cache_append_attend at C4's full size with the plan
    of bench.py's C4 line (max_len = 32000 + 256 steps), the call the
    headline number times: the fills, the appended rows (bit-exact) and the
    output of sampled (sequence, head) pairs against the float64 oracle over
    the device cache's own bf16 values."""
    banner("append+attend C4 full size, bench plan")
    gpu = _gpu()
    B, T, H, D, fill = 4, 32768, 16, 128, 32000
    cache, kv, vv = _c4_bench_cache(gpu, gpu_ctx)
    chunk, n_chunks = gpu.decode_plan(gpu_ctx, B, H, H, fill + 256, head_dim=D,
                                      dtype=torch.bfloat16)
    print(f"plan: chunk_tokens={chunk} n_chunks={n_chunks}")
    g = torch.Generator(device="cuda").manual_seed(2)
    out = torch.empty((B, H, D), device="cuda")
    pairs = [(0, 0), (0, 15), (1, 7), (2, 3), (2, 12), (3, 9)]
    worst = 0.0
    for step in range(3):
        q, kn, vn = (torch.randn((B, H, D), generator=g, device="cuda") for _ in range(3))
        fills = gpu.kv_cache_append_attend(gpu_ctx, cache, 0, kn, vn, q, out, max_len=fill + 256)
        n = fill + step + 1
        np.testing.assert_array_equal(fills, [n] * B)
        assert cache.layers[0].lens.cpu().tolist() == [n] * B
        np.testing.assert_array_equal(kv[:, n - 1].float().cpu().numpy(),
                                      ko.bf16_round(kn.cpu().numpy()))
        np.testing.assert_array_equal(vv[:, n - 1].float().cpu().numpy(),
                                      ko.bf16_round(vn.cpu().numpy()))
        got, qh = out.cpu().numpy(), q.cpu().numpy()
        for b, h in pairs:
            kh = kv[b, :n, h].float().cpu().numpy()[None, :, None, :]
            vh = vv[b, :n, h].float().cpu().numpy()[None, :, None, :]
            want = ko.decode_attention(qh[b:b + 1, h:h + 1], kh, vh, [n])
            worst = max(worst, rel_err(got[b:b + 1, h:h + 1], want))
    print(f"worst rel_err over 3 steps x {len(pairs)} heads = {worst:.3e}")
    assert worst < FP32_TOL  # the same bf16 values, fp32 accumulation


def test_append_attend_full_size_c5_bench_plan(gpu_ctx):
    """Three steps of the paged kv_cache_append_attend at C5's full size, built
    as bench.py's C5 line builds it (64 sequences, 32 query heads over 8 kv
    heads, D=128, bf16 16-token pages under the seeded page table, lognormal
    lengths, max_len = longest + 128 steps: the matrix-core plan): every
    output against the C restatement of the oracle over a host copy of the
    pool gathered into a contiguous cache and updated by the append rule, and
    the appended rows bit-exact."""
    banner("append+attend C5 full size, bench plan")
    from oracle import c_oracle
    gpu = _gpu()
    B, Hq, Hkv, D, bs, steps = 64, 32, 8, 128, 16, 128
    r = np.random.default_rng(0)
    lens0 = np.clip(np.exp(r.normal(np.log(1500), 0.8, B)), 16, 8192).astype(np.int64)
    max_seq = 8192 + steps
    max_blocks = -(-max_seq // bs)
    need = -(-(lens0 + steps) // bs)
    n_blocks = int(need.sum())
    cache = gpu.kv_cache_create(gpu_ctx, gpu.KVCacheConfig(B, max_seq, 1, Hq, D, n_kv_heads=Hkv,
                                                           dtype=torch.bfloat16, block_size=bs,
                                                           n_blocks=n_blocks))
    perm = r.permutation(n_blocks).astype(np.int32)
    table = np.zeros((B, max_blocks), np.int32)
    o = 0
    for b in range(B):
        table[b, :need[b]] = perm[o:o + need[b]]
        o += need[b]
    gpu.kv_cache_set_block_table(cache, torch.from_numpy(table))
    layer = cache.layers[0]
    g = torch.Generator(device="cuda").manual_seed(0)
    for buf in (layer.k_cache.buffer, layer.v_cache.buffer):
        for i in range(0, buf.shape[0], 1 << 16):
            part = buf[i:i + (1 << 16)]
            part.copy_(torch.randn(part.shape, generator=g, device="cuda"))
    layer.lens.copy_(torch.from_numpy(lens0.astype(np.int32)))
    layer.host_lens = lens0.copy()
    max_len = int(min(lens0.max() + steps, max_blocks * bs))
    chunk, n_chunks = gpu.decode_plan(gpu_ctx, B, Hq, Hkv, max_len, int(lens0.sum()),
                                      head_dim=D, dtype=torch.bfloat16)
    print(f"plan: chunk_tokens={chunk} n_chunks={n_chunks}")
    nb = int(need.max())
    tab = torch.from_numpy(table[:, :nb].astype(np.int64)).cuda()

    def gather(buf):
        x = buf.view(n_blocks, bs, Hkv, D)[tab].reshape(B, nb * bs, Hkv, D)
        return x.view(torch.int16).cpu().numpy().view(np.uint16).copy()

    kc, vc = gather(layer.k_cache.buffer), gather(layer.v_cache.buffer)
    g2 = torch.Generator(device="cuda").manual_seed(2)
    out = torch.empty((B, Hq, D), device="cuda")
    lens = lens0.copy()
    bits = lambda x: x.to(torch.bfloat16).view(torch.int16).cpu().numpy().view(np.uint16)
    for step in range(3):
        q = torch.randn((B, Hq, D), generator=g2, device="cuda")
        kn = torch.randn((B, Hkv, D), generator=g2, device="cuda")
        vn = torch.randn((B, Hkv, D), generator=g2, device="cuda")
        fills = gpu.kv_cache_append_attend(gpu_ctx, cache, 0, kn, vn, q, out, max_len=max_len)
        kb, vb = bits(kn), bits(vn)
        for b in range(B):
            kc[b, lens[b]], vc[b, lens[b]] = kb[b], vb[b]
        lens += 1
        np.testing.assert_array_equal(fills, lens)
        # the appended rows in the pool (row lens-1 of each sequence's pages)
        t = lens - 1
        rows = torch.from_numpy((table[np.arange(B), t // bs].astype(np.int64) * bs + t % bs)).cuda()
        pk = layer.k_cache.buffer.view(-1, Hkv, D)[rows]
        pv = layer.v_cache.buffer.view(-1, Hkv, D)[rows]
        np.testing.assert_array_equal(pk.view(torch.int16).cpu().numpy().view(np.uint16), kb)
        np.testing.assert_array_equal(pv.view(torch.int16).cpu().numpy().view(np.uint16), vb)
        want = c_oracle.decode_attn(q.cpu().numpy(), kc, vc, lens, cache_bf16=True)
        err = rel_err(out.cpu().numpy(), want)
        print(f"step {step}: rel_err={err:.3e}")
        assert err < FP32_TOL  # the same bf16 values, fp32 accumulation on both sides
