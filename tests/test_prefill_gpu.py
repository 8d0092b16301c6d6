"""Parity of the MFMA chunked prefill (skv_append_prefill_attn: skv_append_chunk
+ skv_prefill_attn + the fill advance, driven through kv_cache_prefill) with
the CPU oracle. Needs the MI355X.

On bf16 caches the prefill feeds Q, K, V and the softmax probabilities to
v_mfma_f32_32x32x16_bf16 in bf16, with fp32 accumulation and softmax (fp32
caches take the fp32 kernel, tested in test_flash_fwd_gpu.py). Tolerance: the north star's 2e-2 relative error for bf16
storage with fp32 accumulation, norm-wise per (sequence, query, head),
against the float64 oracle fed the same bf16-rounded q, K and V. Cache bytes
and fills after the chunk append: bit-exact.
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN, banner
from oracle import kv_oracle as ko

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2


def _gpu():
    from simple_llm_amd.gpu import gpu
    return gpu


def rel_err(got, want, valid=None):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    num = np.linalg.norm(got - want, axis=-1)
    den = np.maximum(np.linalg.norm(want, axis=-1), 1e-30)
    r = num / den
    return float(r[valid].max() if valid is not None else r.max())


def to_dev(x, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda").to(dtype)


def run_prefill(ctx, B, T, Hq, Hkv, D, prefix, C, n_new=None, seed=0, n_splits=0,
                q_dtype=torch.float32, out_dtype=torch.float32):
    """Fill a bf16 cache to `prefix`, prefill a chunk of C tokens through the
    drop-in API, and return (gpu out, oracle out, valid-row mask, cache, k, v)."""
    gpu = _gpu()
    rng = np.random.default_rng(seed)
    cache = gpu.kv_cache_create(ctx, gpu.KVCacheConfig(B, T, 1, Hq, D, n_kv_heads=Hkv,
                                                       dtype=torch.bfloat16))
    layer = cache.layers[0]
    k = ko.bf16_round(rng.standard_normal((B, T, Hkv, D)).astype(np.float32))
    v = ko.bf16_round(rng.standard_normal((B, T, Hkv, D)).astype(np.float32))
    prefix = np.asarray(prefix, np.int64)
    # the prefix comes from earlier steps: write it straight into the cache
    kp, vp = np.zeros_like(k), np.zeros_like(v)
    for b in range(B):
        kp[b, :prefix[b]] = k[b, :prefix[b]]
        vp[b, :prefix[b]] = v[b, :prefix[b]]
    layer.k_cache.buffer.copy_(to_dev(kp.reshape(-1, Hkv * D), torch.bfloat16))
    layer.v_cache.buffer.copy_(to_dev(vp.reshape(-1, Hkv * D), torch.bfloat16))
    layer.lens.copy_(torch.from_numpy(prefix.astype(np.int32)))
    layer.host_lens[:] = prefix
    # the chunk's own k/v: rows prefix[b] .. prefix[b]+C-1 of k, v
    kn = np.stack([k[b, prefix[b]:prefix[b] + C] for b in range(B)])
    vn = np.stack([v[b, prefix[b]:prefix[b] + C] for b in range(B)])
    q = rng.standard_normal((B, C, Hq, D)).astype(np.float32)
    if q_dtype == torch.bfloat16:
        q = ko.bf16_round(q)
    # NaN-filled: every element, the zeros of rows past n_new included, must be written
    out = torch.full((B, C, Hq, D), float("nan"), dtype=out_dtype, device="cuda")
    fills = gpu.kv_cache_prefill(ctx, cache, 0, to_dev(kn), to_dev(vn), to_dev(q, q_dtype), out,
                                 n_new=n_new, n_splits=n_splits)
    nn = np.full(B, C) if n_new is None else np.asarray(n_new)
    np.testing.assert_array_equal(fills, prefix + nn)
    np.testing.assert_array_equal(layer.lens.cpu().numpy(), prefix + nn)
    # oracle over the bf16-rounded q (the kernel rounds q to bf16 for the MFMA)
    want = ko.prefill_attention(ko.bf16_round(q), k, v, prefix, q_lens=nn)
    valid = np.zeros((B, C, Hq), bool)
    for b in range(B):
        valid[b, :nn[b]] = True
    return out.float().cpu().numpy(), want, valid, cache, k, v, nn


@pytest.mark.parametrize("B,T,Hq,Hkv,D,prefix,C", [
    (2, 1024, 16, 16, 128, [0, 700], 300),        # C4 head shape, one prefix empty
    (3, 2400, 32, 8, 128, [100, 0, 2000], 200),   # GQA G=4
    (2, 1200, 12, 12, 64, [1000, 33], 129),       # C3 head shape, C not a tile multiple
    (1, 700, 8, 4, 64, [37], 600),                # G=2, chunk spans 3 query tiles
    (2, 600, 16, 2, 128, [64, 300], 96),          # G=8
])
def test_prefill_matches_oracle(gpu_ctx, B, T, Hq, Hkv, D, prefix, C):
    banner(f"prefill B={B} T={T} Hq={Hq} Hkv={Hkv} D={D} prefix={prefix} C={C}")
    got, want, valid, *_ = run_prefill(gpu_ctx, B, T, Hq, Hkv, D, prefix, C, seed=B * 7 + C)
    err = rel_err(got, want, valid)
    print(f"rel_err={err:.3e}")
    assert err < BF16_TOL


@pytest.mark.parametrize("n_splits", [1, 2, 3, 4, 5, 7])
def test_prefill_split_counts_agree(gpu_ctx, n_splits):
    """Forced split counts (no merge pass, and merges of 2 to 7 partials)."""
    banner(f"prefill n_splits={n_splits}")
    got, want, valid, *_ = run_prefill(gpu_ctx, 2, 4096, 8, 8, 128, [2900, 1500], 256,
                                       seed=5, n_splits=n_splits)
    assert rel_err(got, want, valid) < BF16_TOL


def test_prefill_split_merge_repeats_bit_exact(gpu_ctx):
    """Calls of other shapes and split counts between two runs of the same call
    share its workspace and leave nothing behind: the repeat gives the same bits."""
    banner("prefill split merge: repeat after other shapes")
    first = {}
    for rnd in range(2):
        for ns in (2, 4, 3):
            got, want, valid, *_ = run_prefill(gpu_ctx, 2, 3000, 8, 4, 128, [2500, 900], 200,
                                               n_new=[200, 131], seed=11, n_splits=ns)
            assert rel_err(got, want, valid) < BF16_TOL
            if rnd == 0:
                first[ns] = got
            else:
                np.testing.assert_array_equal(got, first[ns])
            # another shape between the repeats, through the same workspace
            run_prefill(gpu_ctx, 3, 1500, 16, 16, 64, [700, 0, 1200], 96, seed=ns, n_splits=ns)


def test_prefill_ragged_chunk_zero_rows(gpu_ctx):
    banner("prefill ragged n_new")
    for ns in (1, 3):
        got, want, valid, cache, k, v, nn = run_prefill(
            gpu_ctx, 3, 1500, 16, 4, 128, [10, 500, 0], 300, n_new=[300, 17, 0], seed=9,
            n_splits=ns)
        assert rel_err(got, want, valid) < BF16_TOL
        assert not got[~valid].any()  # rows past n_new[b] are zeros
        # the chunk append wrote exactly the n_new rows (bit-exact), nothing past them
        kc = cache.layers[0].k_cache.buffer.float().cpu().numpy().reshape(k.shape)
        for b, (p, n) in enumerate(zip([10, 500, 0], nn)):
            np.testing.assert_array_equal(kc[b, p:p + n], k[b, p:p + n])
            assert not kc[b, p + n:].any()


@pytest.mark.parametrize("q_dt,o_dt", [(torch.bfloat16, torch.bfloat16),
                                       (torch.float32, torch.bfloat16)])
def test_prefill_io_dtypes(gpu_ctx, q_dt, o_dt):
    banner(f"prefill q={q_dt} out={o_dt}")
    got, want, valid, *_ = run_prefill(gpu_ctx, 2, 900, 8, 8, 64, [400, 100], 128, seed=3,
                                       q_dtype=q_dt, out_dtype=o_dt)
    assert rel_err(got, want, valid) < BF16_TOL


def test_prefill_reference_flash_kat(gpu_ctx):
    """test_flash_attention's seed-42 "Small" config (B=4, T=16, H=4, D=64;
    simple-llm/src/gpu_test.py:747-810) as a prefill with an empty prefix:
    the reference's causal flash attention is the prefix-0 case."""
    banner("prefill reference flash KAT (4, 16, 4, 64)")
    import make_golden as mg

    gpu = _gpu()
    z = np.load(os.path.join(GOLDEN, "flash_kat_seed42.npz"))
    b, t, h, d = (int(x) for x in z["configs"][3])
    Q, K, V = mg.flash_inputs(b, t, h, d)
    cache = gpu.kv_cache_create(gpu_ctx, gpu.KVCacheConfig(b, 64, 1, h, d, dtype=torch.bfloat16))
    out = torch.empty((b, t, h, d), device="cuda")
    gpu.kv_cache_prefill(gpu_ctx, cache, 0, to_dev(K.reshape(b, t, h, d)),
                         to_dev(V.reshape(b, t, h, d)), to_dev(Q.reshape(b, t, h, d)), out)
    got = out.cpu().numpy().reshape(b * t, h, d)
    want = z["o_3"].reshape(b * t, h, d)  # float64 SDPA on the fp32 inputs
    # against the fp32-input expected value, bf16 rounding of q, k, v included
    assert rel_err(got, want) < BF16_TOL
    # against the same bf16-rounded inputs the error is the kernel's alone
    o_r, _, _ = ko.flash_attention(ko.bf16_round(Q).reshape(b * t, -1),
                                   ko.bf16_round(K).reshape(b * t, -1),
                                   ko.bf16_round(V).reshape(b * t, -1), b, t, h, d)
    assert rel_err(got, o_r.reshape(b * t, h, d)) < 1e-2


def test_decode_after_prefill(gpu_ctx):
    """A decode step right after a prefill reads the chunk the prefill appended
    and the fills it advanced (fp32-exact decode over the bf16 cache)."""
    banner("decode after prefill")
    gpu = _gpu()
    _, _, _, cache, k, v, nn = run_prefill(gpu_ctx, 2, 1000, 8, 8, 128, [300, 50], 64, seed=21)
    qn = np.random.default_rng(99).standard_normal((2, 8, 128)).astype(np.float32)
    q = to_dev(qn)
    out = torch.empty_like(q)
    gpu.decode_attention(gpu_ctx, cache, 0, q, out)
    want = ko.decode_attention(qn, k, v, np.array([300, 50]) + nn)
    assert rel_err(out.cpu().numpy(), want) < 1e-4


def test_prefill_rejects_bad_calls(gpu_ctx):
    banner("prefill argument checks")
    gpu = _gpu()
    cache = gpu.kv_cache_create(gpu_ctx, gpu.KVCacheConfig(2, 100, 1, 4, 64,
                                                           dtype=torch.bfloat16))
    kn = torch.zeros((2, 60, 4, 64), device="cuda")
    gpu.kv_cache_prefill(gpu_ctx, cache, 0, kn, kn)  # append only: fills 60
    with pytest.raises(ValueError, match="Cache is full"):
        gpu.kv_cache_prefill(gpu_ctx, cache, 0, kn, kn)
    with pytest.raises(ValueError, match="n_kv_heads"):
        gpu.kv_cache_prefill(gpu_ctx, cache, 0, torch.zeros((2, 4, 3, 64), device="cuda"),
                             torch.zeros((2, 4, 3, 64), device="cuda"))
    f32 = gpu.kv_cache_create(gpu_ctx, gpu.KVCacheConfig(2, 100, 1, 4, 64))
    q = torch.zeros((2, 4, 4, 64), device="cuda")
    with pytest.raises(ValueError, match="float32 cache takes float32"):
        gpu.kv_cache_prefill(gpu_ctx, f32, 0, q, q, q.bfloat16(), torch.empty_like(q))
    np.testing.assert_array_equal(f32.seq_lens(), [0, 0])  # nothing ran


def test_prefill_c4_full_size_sampled(gpu_ctx):
    """C4's prefill at full size: B=4, H=16, D=128, bf16 cache of 32768 filled
    to 32256, one 512-token chunk (exactly fills it). Sampled rows are checked
    against the oracle."""
    banner("prefill C4 full size, sampled oracle")
    gpu = _gpu()
    B, T, H, D, P, C = 4, 32768, 16, 128, 32256, 512
    cache = gpu.kv_cache_create(gpu_ctx, gpu.KVCacheConfig(B, T, 1, H, D, dtype=torch.bfloat16))
    layer = cache.layers[0]
    g = torch.Generator(device="cuda").manual_seed(1)
    kv = layer.k_cache.buffer.view(B, T, H, D)
    vv = layer.v_cache.buffer.view(B, T, H, D)
    for b in range(B):
        kv[b, :P].copy_(torch.randn((P, H, D), generator=g, device="cuda"))
        vv[b, :P].copy_(torch.randn((P, H, D), generator=g, device="cuda"))
    cache.current_len = P
    kn = torch.randn((B, C, H, D), generator=g, device="cuda")
    vn = torch.randn((B, C, H, D), generator=g, device="cuda")
    q = torch.randn((B, C, H, D), generator=g, device="cuda")
    out = torch.empty_like(q)
    fills = gpu.kv_cache_prefill(gpu_ctx, cache, 0, kn, vn, q, out)
    assert fills.tolist() == [T] * B
    got = out.cpu().numpy()
    qh = ko.bf16_round(q.cpu().numpy())
    for b, i, h in [(0, 0, 0), (1, 511, 5), (2, 256, 15), (3, 77, 9)]:
        kh = kv[b, :P + i + 1, h].float().cpu().numpy()[None, :, None, :]
        vh = vv[b, :P + i + 1, h].float().cpu().numpy()[None, :, None, :]
        want = ko.decode_attention(qh[b:b + 1, i, h:h + 1], kh, vh, [P + i + 1])
        assert rel_err(got[b:b + 1, i, h:h + 1], want) < BF16_TOL


@pytest.mark.parametrize("cache_dt,n_splits,ragged", [("bf16", 1, False), ("bf16", 2, True),
                                                      ("bf16", 3, False), ("f32", 1, True)])
def test_fused_prefill_call_equals_the_three_calls(gpu_ctx, cache_dt, n_splits, ragged):
    """skv_append_prefill_attn against skv_append_chunk + skv_prefill_attn +
    skv_advance on the same inputs: the same output bits, cache bytes and
    fills (on the split bf16 path the merge pass advances the fills from the
    snapshot in the workspace's tail)."""
    banner(f"fused prefill call vs three calls: {cache_dt} n_splits={n_splits} ragged={ragged}")
    from simple_llm_amd import _lib
    L = _lib.lib()
    s = _lib.stream_handle()
    B, T, Hq, Hkv, D, C = 3, 1500, 8, 4, 128, 160
    tdt = torch.bfloat16 if cache_dt == "bf16" else torch.float32
    cdt = _lib.BF16 if cache_dt == "bf16" else _lib.F32
    rng = np.random.default_rng(n_splits * 10 + ragged)
    prefix = np.array([1200, 0, 777], np.int32)
    n_new = np.array([160, 1, 93], np.int32) if ragged else None
    base_k = torch.from_numpy(rng.standard_normal((B * T, Hkv * D)).astype(np.float32)).cuda().to(tdt)
    base_v = torch.from_numpy(rng.standard_normal((B * T, Hkv * D)).astype(np.float32)).cuda().to(tdt)
    kn = to_dev(rng.standard_normal((B, C, Hkv, D)).astype(np.float32))
    vn = to_dev(rng.standard_normal((B, C, Hkv, D)).astype(np.float32))
    q = to_dev(rng.standard_normal((B, C, Hq, D)).astype(np.float32))
    nd = to_dev(n_new, torch.int32) if ragged else None
    n_ptr = nd.data_ptr() if nd is not None else None
    need = L.skv_prefill_workspace_bytes(B, C, Hq, D, n_splits)
    results = []
    for fused in (False, True):
        kc, vc = base_k.clone(), base_v.clone()
        lens = to_dev(prefix, torch.int32)
        out = torch.full((B, C, Hq, D), float("nan"), device="cuda")
        ws = torch.full((max(need, 16),), 0xAB, dtype=torch.uint8, device="cuda")
        args = (B, C, Hq, Hkv, D, T, D ** -0.5, n_splits, ws.data_ptr(), ws.numel())
        if fused:
            _lib.check(L.skv_append_prefill_attn(out.data_ptr(), q.data_ptr(), kc.data_ptr(),
                                                 vc.data_ptr(), kn.data_ptr(), vn.data_ptr(),
                                                 lens.data_ptr(), n_ptr, *args, cdt, _lib.F32,
                                                 _lib.F32, _lib.F32, s), "skv_append_prefill_attn")
        else:
            _lib.check(L.skv_append_chunk(kc.data_ptr(), vc.data_ptr(), kn.data_ptr(),
                                          vn.data_ptr(), lens.data_ptr(), n_ptr, B, C, Hkv, D, T,
                                          cdt, _lib.F32, s), "skv_append_chunk")
            _lib.check(L.skv_prefill_attn(out.data_ptr(), q.data_ptr(), kc.data_ptr(),
                                          vc.data_ptr(), lens.data_ptr(), n_ptr, *args, cdt,
                                          _lib.F32, _lib.F32, s), "skv_prefill_attn")
            _lib.check(L.skv_advance(lens.data_ptr(), n_ptr, C, B, T, s), "skv_advance")
        torch.cuda.synchronize()
        results.append((out.cpu(), kc.cpu(), vc.cpu(), lens.cpu()))
    (o0, k0, v0, l0), (o1, k1, v1, l1) = results
    nn = n_new if ragged else np.full(B, C)
    np.testing.assert_array_equal(l1.numpy(), np.minimum(prefix + nn, T))
    np.testing.assert_array_equal(l1.numpy(), l0.numpy())
    assert torch.equal(k1, k0) and torch.equal(v1, v0)
    assert torch.equal(o1, o0)  # NaN-filled before: every element written, the same bits
