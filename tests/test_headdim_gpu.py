"""Head dims other than 64 and 128 on the MI355X.

The reference's decode kernel loops over any head_dim
(simple-llm/src/gpu/gpu_kernels.py:2846, 2856-2866, 2916-2921; its cache
checks only head_dim > 0, gpu/gpu_kv_cache.py:55-64), its flash kernels take
any head_dim up to flash_attn_max_head_dim (gpu/gpu_pass_forward.py:531-536),
and the models its auto-configuration trains have head dims of 24 to 80
(src/hyper.py:63-79). These tests run every entry point of the path at such
head dims -- odd ones, ones that are not a multiple of 4 or 8 (element loads),
and the padded-size edges -- against the CPU oracle:

  * append (single token, paged, chunk): bit-exact cache bytes and fills;
  * decode attention (contiguous, paged, GQA) and the fused append + decode:
    1e-4 relative (fp32 and bf16 storage alike: the oracle sees the same
    rounded K/V, accumulation is fp32 on both sides);
  * the bf16 MFMA prefill: 2e-2 (q and P enter the MFMA as bf16);
  * the fp32 prefill and flash forward/backward: 1e-4.

Past the reference's typical sizes: decode takes head dims up to 2048 (G <=
2), 1024 (G = 4) and 512 (G = 8), the prefills and the flash forward up to
256 (the reference's largest flash_attn_max_head_dim, gpu/gpu_device.py:
468-471), the flash backward too (past 128 at a far lower rate).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import banner
from oracle import kv_oracle as ko
from test_kv_gpu import _decode, _filled_cache, cache_host, rel_err, to_dev
from test_prefill_gpu import rel_err as rel_err_rows
from test_prefill_gpu import run_prefill

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-4
BF16_TOL = 2e-2

# 64 and 128 take the tuned kernels; everything else the padded (masked) ones
HEAD_DIMS = [1, 8, 20, 24, 28, 30, 32, 36, 40, 48, 56, 72, 80, 96, 100, 160, 200, 256]


def _gpu():
    from simple_llm_amd.gpu import gpu
    return gpu


# ---------------------------------------------------------------------------
# decode attention
# ---------------------------------------------------------------------------

_DECODE_LAYOUTS = [
    (6, 6, torch.float32, False),
    (8, 2, torch.bfloat16, True),    # G = 4 over a paged cache
    (8, 1, torch.bfloat16, False),   # G = 8 (past 128: wavefront rows)
    (3, 3, torch.float32, True),
]
# head dims past 256: rows of 64 lanes (a wavefront) instead of 16
WIDE_DIMS = [264, 320, 384, 512]


@pytest.mark.parametrize("D,Hq,Hkv,dtype,paged", [
    (D, *lay) for lay in _DECODE_LAYOUTS for D in HEAD_DIMS + WIDE_DIMS] + [
    (1024, 8, 2, torch.bfloat16, False), (1000, 4, 1, torch.float32, True),
    (2048, 2, 1, torch.float32, False), (2040, 4, 4, torch.bfloat16, True)])
def test_decode_any_head_dim(gpu_ctx, D, Hq, Hkv, dtype, paged):
    banner(f"decode D={D} Hq={Hq} Hkv={Hkv} {dtype} paged={paged}")
    gpu = _gpu()
    rng = np.random.default_rng(D * 10 + Hq)
    B, T = 3, 320
    lens = np.array([T, 1, 177])
    cache, k, v, _ = _filled_cache(gpu, gpu_ctx, rng, B, T, Hq, Hkv, D, dtype, lens, paged)
    q = rng.standard_normal((B, Hq, D)).astype(np.float32)
    got = _decode(gpu, gpu_ctx, cache, q)
    want = ko.decode_attention(q, k, v, lens)
    err = rel_err(got, want)
    print(f"rel_err={err:.3e}")
    assert err < FP32_TOL
    np.testing.assert_array_equal(got[1], np.broadcast_to(
        np.repeat(v[1, 0], Hq // Hkv, axis=0), got[1].shape))  # one token: its value row


@pytest.mark.parametrize("D,G", [(520, 8), (1032, 4), (2056, 1), (2056, 2)])
def test_decode_head_dims_past_the_kernels_are_rejected(gpu_ctx, D, G):
    """Past G * head_dim = 4096 (head_dim 2048 at G <= 2) there is no kernel:
    ValueError (SKV_E_UNSUPPORTED) before any launch."""
    gpu = _gpu()
    cache = gpu.kv_cache_create(gpu_ctx, gpu.KVCacheConfig(1, 8, 1, G, D, n_kv_heads=1))
    cache.current_len = 1
    q = torch.zeros((1, G, D), device="cuda")
    with pytest.raises(ValueError, match=f"head_dim {D} with {G} query heads"):
        gpu.decode_attention(gpu_ctx, cache, 0, q, torch.empty_like(q))


@pytest.mark.parametrize("D,Hq,Hkv,cdt,idt,paged", [
    (24, 4, 4, torch.float32, torch.float32, False),
    (36, 8, 2, torch.bfloat16, torch.float32, True),
    (48, 8, 8, torch.bfloat16, torch.bfloat16, False),
    (80, 16, 16, torch.float32, torch.float32, True),
    (30, 2, 2, torch.bfloat16, torch.bfloat16, False),  # element loads
    (200, 4, 2, torch.bfloat16, torch.float32, False),
    (192, 8, 1, torch.bfloat16, torch.float32, True),   # G = 8 past 128
    (320, 4, 2, torch.float32, torch.float32, False),   # wavefront rows
    (512, 8, 8, torch.bfloat16, torch.bfloat16, True),
    (1024, 4, 1, torch.bfloat16, torch.float32, False),
])
def test_fused_append_attend_any_head_dim(gpu_ctx, D, Hq, Hkv, cdt, idt, paged):
    """Three fused append + decode steps against skv_append then skv_decode_attn
    on a copy of the cache (bit-identical caches and fills) and the oracle."""
    banner(f"fused append+attend D={D} Hq={Hq} Hkv={Hkv} {cdt} in={idt} paged={paged}")
    gpu = _gpu()
    rng = np.random.default_rng(D)
    B, T = 4, 96
    lens = np.array([0, 17, 95, 96])  # empty, middle, one slot left, full (skipped)
    ca, k, v, _ = _filled_cache(gpu, gpu_ctx, np.random.default_rng(3), B, T, Hq, Hkv, D, cdt,
                                lens, paged)
    cb, _, _, _ = _filled_cache(gpu, gpu_ctx, np.random.default_rng(3), B, T, Hq, Hkv, D, cdt,
                                lens, paged)
    kw, vw, fills = k.copy(), v.copy(), lens.copy()
    rounds = cdt == torch.bfloat16 or idt == torch.bfloat16
    for step in range(3):
        kn = rng.standard_normal((B, Hkv, D)).astype(np.float32)
        vn = rng.standard_normal((B, Hkv, D)).astype(np.float32)
        q = rng.standard_normal((B, Hq, D)).astype(np.float32)
        out_a = torch.empty((B, Hq, D), device="cuda")
        out_b = torch.empty_like(out_a)
        gpu.kv_cache_append(gpu_ctx, ca, 0, to_dev(kn, idt), to_dev(vn, idt))
        gpu.decode_attention(gpu_ctx, ca, 0, to_dev(q), out_a)
        got = gpu.kv_cache_append_attend(gpu_ctx, cb, 0, to_dev(kn, idt), to_dev(vn, idt),
                                         to_dev(q), out_b)
        knr, vnr = (ko.bf16_round(kn), ko.bf16_round(vn)) if rounds else (kn, vn)
        for b in range(B):
            if fills[b] < T:
                kw[b, fills[b]], vw[b, fills[b]] = knr[b], vnr[b]
                fills[b] += 1
        np.testing.assert_array_equal(got, fills)
        np.testing.assert_array_equal(cb.layers[0].lens.cpu().numpy(), fills)
        ka, va = cache_host(ca.layers[0], ca)
        kb_, vb_ = cache_host(cb.layers[0], cb)
        np.testing.assert_array_equal(ka, kb_)
        np.testing.assert_array_equal(va, vb_)
        assert rel_err(out_b.cpu().numpy(), out_a.cpu().numpy()) < 1e-6, step
        assert rel_err(out_b.cpu().numpy(), ko.decode_attention(q, kw, vw, fills)) < FP32_TOL


# ---------------------------------------------------------------------------
# append: bit-exact
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("D,Hkv", [(20, 2), (30, 1), (30, 3), (36, 2), (48, 4), (80, 1), (7, 5)])
@pytest.mark.parametrize("cache_dt,in_dt", [(torch.float32, torch.float32),
                                            (torch.bfloat16, torch.float32),
                                            (torch.bfloat16, torch.bfloat16),
                                            (torch.float32, torch.bfloat16)])
@pytest.mark.parametrize("paged", [False, True])
def test_append_any_head_dim_bit_exact(gpu_ctx, D, Hkv, cache_dt, in_dt, paged):
    """E = H_kv * D not a multiple of 8 (30, 90, 35: element path) and
    multiples of 8 (vector path)."""
    banner(f"append D={D} Hkv={Hkv} cache={cache_dt} in={in_dt} paged={paged}")
    gpu = _gpu()
    rng = np.random.default_rng(D * 7 + Hkv)
    B, T = 4, 40
    cfg = gpu.KVCacheConfig(B, T, 1, Hkv, D, dtype=cache_dt, block_size=8 if paged else 0)
    cache = gpu.kv_cache_create(gpu_ctx, cfg)
    if paged:
        table = rng.permutation(cache.n_blocks).reshape(B, -1).astype(np.int32)
        gpu.kv_cache_set_block_table(cache, torch.from_numpy(table))
    start = np.array([0, 11, 39, 40])
    cache.layers[0].lens.copy_(torch.from_numpy(start.astype(np.int32)))
    cache.layers[0].host_lens[:] = start
    kw = np.zeros((B, T, Hkv, D), np.float32)
    vw = np.zeros_like(kw)
    lens = start.copy()
    sdt = "bf16" if cache_dt == torch.bfloat16 else "fp32"
    for _ in range(2):
        k = rng.standard_normal((B, Hkv, D)).astype(np.float32) * 3
        v = rng.standard_normal((B, Hkv, D)).astype(np.float32)
        if in_dt == torch.bfloat16:
            k, v = ko.bf16_round(k), ko.bf16_round(v)
        host = gpu.kv_cache_append(gpu_ctx, cache, 0, to_dev(k, in_dt), to_dev(v, in_dt))
        lens = ko.append(kw, vw, k, v, lens, dtype=sdt)
        np.testing.assert_array_equal(host, lens)
    np.testing.assert_array_equal(cache.layers[0].lens.cpu().numpy(), lens)
    kc, vc = cache_host(cache.layers[0], cache)
    if paged:
        kc = ko.paged_gather(kc, table, lens, 8, T)
        vc = ko.paged_gather(vc, table, lens, 8, T)
        for b in range(B):
            kw[b, lens[b]:] = 0
            vw[b, lens[b]:] = 0
    np.testing.assert_array_equal(kc, kw)
    np.testing.assert_array_equal(vc, vw)


@pytest.mark.parametrize("D,H", [(30, 1), (36, 2), (80, 3), (5, 3)])
@pytest.mark.parametrize("cache_dt,in_dt", [(torch.float32, torch.float32),
                                            (torch.bfloat16, torch.float32)])
def test_append_chunk_any_head_dim(gpu_ctx, D, H, cache_dt, in_dt):
    from simple_llm_amd import _lib
    banner(f"append_chunk D={D} H={H} {cache_dt} in={in_dt}")
    rng = np.random.default_rng(D + H)
    B, T, C = 3, 40, 9
    kc = torch.zeros((B, T, H, D), dtype=cache_dt, device="cuda")
    vc = torch.zeros_like(kc)
    lens = torch.tensor([0, 30, 35], dtype=torch.int32, device="cuda")
    n_new = torch.tensor([9, 4, 9], dtype=torch.int32, device="cuda")
    k = rng.standard_normal((B, C, H, D)).astype(np.float32)
    v = rng.standard_normal((B, C, H, D)).astype(np.float32)
    L = _lib.lib()
    s = _lib.stream_handle()
    kd, vd = to_dev(k, in_dt), to_dev(v, in_dt)
    rc = L.skv_append_chunk(kc.data_ptr(), vc.data_ptr(), kd.data_ptr(), vd.data_ptr(),
                            lens.data_ptr(), n_new.data_ptr(), B, C, H, D, T,
                            _lib.dtype_code(cache_dt), _lib.dtype_code(in_dt), s)
    _lib.check(rc, "append_chunk")
    kw = np.zeros((B, T, H, D), np.float32)
    vw = np.zeros_like(kw)
    sdt = "bf16" if cache_dt == torch.bfloat16 else "fp32"
    ko.append_chunk(kw, vw, k, v, np.array([0, 30, 35]), np.array([9, 4, 9]), dtype=sdt)
    np.testing.assert_array_equal(kc.float().cpu().numpy(), kw)
    np.testing.assert_array_equal(vc.float().cpu().numpy(), vw)


# ---------------------------------------------------------------------------
# prefill (bf16 MFMA kernel; fp32 caches take the fp32 kernel)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("D,G", [(D, 2) for D in (1, 8, 20, 24, 28, 36, 40, 48, 56, 80, 96,
                                                  100, 120, 136, 160, 192, 200, 256)]
                         + [(160, 1), (256, 1), (192, 8), (256, 4)])
@pytest.mark.parametrize("n_splits", [1, 3])
def test_prefill_bf16_any_head_dim(gpu_ctx, D, G, n_splits):
    """Past 128 the kernel runs at 256 (4 wavefronts of 32 query rows a
    workgroup): exact 256 by LDS DMA, others through registers."""
    banner(f"prefill bf16 D={D} G={G} n_splits={n_splits}")
    got, want, valid, *_ = run_prefill(gpu_ctx, 2, 900, 4 * G, 4, D, [300, 0], 200,
                                       n_new=[200, 77], seed=D, n_splits=n_splits)
    # norm-wise per query row over all heads (the reference's [B*T, E] output
    # row): at D = 1 a single head's output is one scalar, often near zero
    B_, C_, Hq_, D_ = got.shape
    err = rel_err_rows(got.reshape(B_, C_, Hq_ * D_), want.reshape(B_, C_, Hq_ * D_), valid[..., 0])
    print(f"rel_err={err:.3e}")
    assert err < BF16_TOL
    assert not got[~valid].any()


@pytest.mark.parametrize("D", [4, 20, 24, 30, 36, 48, 80, 100, 127, 130, 160, 192, 200, 255, 256])
def test_prefill_fp32_any_head_dim(gpu_ctx, D):
    banner(f"prefill fp32 D={D}")
    gpu = _gpu()
    rng = np.random.default_rng(D)
    B, T, Hq, Hkv, C = 2, 400, 6, 3, 70
    prefix = np.array([130, 0])
    cache = gpu.kv_cache_create(gpu_ctx, gpu.KVCacheConfig(B, T, 1, Hq, D, n_kv_heads=Hkv))
    layer = cache.layers[0]
    k = rng.standard_normal((B, T, Hkv, D)).astype(np.float32)
    v = rng.standard_normal((B, T, Hkv, D)).astype(np.float32)
    kp, vp = np.zeros_like(k), np.zeros_like(v)
    for b in range(B):
        kp[b, :prefix[b]], vp[b, :prefix[b]] = k[b, :prefix[b]], v[b, :prefix[b]]
    layer.k_cache.buffer.copy_(to_dev(kp.reshape(-1, Hkv * D)))
    layer.v_cache.buffer.copy_(to_dev(vp.reshape(-1, Hkv * D)))
    layer.lens.copy_(torch.from_numpy(prefix.astype(np.int32)))
    layer.host_lens[:] = prefix
    kn = np.stack([k[b, prefix[b]:prefix[b] + C] for b in range(B)])
    vn = np.stack([v[b, prefix[b]:prefix[b] + C] for b in range(B)])
    q = rng.standard_normal((B, C, Hq, D)).astype(np.float32)
    out = torch.empty((B, C, Hq, D), device="cuda")
    gpu.kv_cache_prefill(gpu_ctx, cache, 0, to_dev(kn), to_dev(vn), to_dev(q), out)
    want = ko.prefill_attention(q, k, v, prefix)
    err = rel_err(out.cpu().numpy(), want)
    print(f"rel_err={err:.3e}")
    assert err < FP32_TOL
    kc, vc = cache_host(layer, cache)
    for b in range(B):  # the chunk append is bit-exact
        np.testing.assert_array_equal(kc[b, :prefix[b] + C], k[b, :prefix[b] + C])
        np.testing.assert_array_equal(vc[b, :prefix[b] + C], v[b, :prefix[b] + C])


# ---------------------------------------------------------------------------
# flash forward and backward (fp32)
# ---------------------------------------------------------------------------

FLASH_DIMS = [1, 3, 8, 20, 24, 28, 36, 40, 48, 56, 72, 80, 96, 100, 112, 127]


@pytest.mark.parametrize("D", FLASH_DIMS)
def test_flash_fwd_bwd_any_head_dim(gpu_ctx, D):
    from test_flash_bwd_gpu import _rel, flash_bwd
    from test_flash_fwd_gpu import _rel_rows, flash_fwd
    banner(f"flash fwd+bwd D={D}")
    B, N, H = 2, 150, 3
    rng = np.random.default_rng(D)
    Q, K, V, dO = (rng.standard_normal((B * N, H * D)).astype(np.float32) for _ in range(4))
    O_w, L_w, M_w = ko.flash_attention(Q, K, V, B, N, H, D)
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()
    o, Ls, Ms = flash_fwd(dev(Q), dev(K), dev(V), B, N, H, D)
    assert _rel_rows(o.cpu().numpy().reshape(-1, H, D), O_w.reshape(-1, H, D)) < FP32_TOL
    assert _rel(Ls.cpu().numpy(), L_w) < FP32_TOL
    assert _rel(Ms.cpu().numpy(), M_w) < FP32_TOL
    O32, L32, M32 = (x.astype(np.float32) for x in (O_w, L_w, M_w))
    want = ko.flash_attention_backward(Q, K, V, O32, L32, M32, dO, B, N, H, D)
    got = flash_bwd(dev(Q), dev(K), dev(V), dev(O32), dev(L32), dev(M32), dev(dO), B, N, H, D)
    for name, g, w in zip(("dq", "dk", "dv"), got, want):
        err = _rel(g.cpu().numpy(), w)
        print(f"{name} rel_err={err:.2e}")
        assert err < FP32_TOL, (name, err)


@pytest.mark.parametrize("D", [130, 160, 192, 200, 255, 256])
def test_flash_fwd_head_dims_to_256(gpu_ctx, D):
    """The flash forward (and with it the fp32 prefill) past 128: padded to
    192 or 256, O, L and M against the oracle."""
    from test_flash_bwd_gpu import _rel
    from test_flash_fwd_gpu import _rel_rows, flash_fwd
    banner(f"flash fwd D={D}")
    B, N, H = 2, 150, 3
    rng = np.random.default_rng(D)
    Q, K, V = (rng.standard_normal((B * N, H * D)).astype(np.float32) for _ in range(3))
    O_w, L_w, M_w = ko.flash_attention(Q, K, V, B, N, H, D)
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()
    o, Ls, Ms = flash_fwd(dev(Q), dev(K), dev(V), B, N, H, D)
    err = _rel_rows(o.cpu().numpy().reshape(-1, H, D), O_w.reshape(-1, H, D))
    print(f"rel_err={err:.3e}")
    assert err < FP32_TOL
    assert _rel(Ls.cpu().numpy(), L_w) < FP32_TOL
    assert _rel(Ms.cpu().numpy(), M_w) < FP32_TOL


def test_flash_head_dim_above_256_is_rejected(gpu_ctx):
    from test_flash_fwd_gpu import flash_fwd
    q = torch.zeros((1 * 4, 2 * 264), device="cuda")
    with pytest.raises(ValueError, match="supported: 1 to 256"):
        flash_fwd(q, q, q, 1, 4, 2, 264)


@pytest.mark.parametrize("D", [136, 160, 192, 200, 255, 256])
def test_flash_bwd_head_dims_to_256(gpu_ctx, D):
    """The flash backward past 128 (padded to 192 or 256; the kernels of the
    wide translation unit): dq, dk, dv against the float64 oracle."""
    from test_flash_bwd_gpu import _rel, flash_bwd
    banner(f"flash bwd D={D}")
    B, N, H = 2, 150, 2
    rng = np.random.default_rng(D + 1)
    Q, K, V, dO = (rng.standard_normal((B * N, H * D)).astype(np.float32) for _ in range(4))
    O_w, L_w, M_w = ko.flash_attention(Q, K, V, B, N, H, D)
    O32, L32, M32 = (x.astype(np.float32) for x in (O_w, L_w, M_w))
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()
    want = ko.flash_attention_backward(Q, K, V, O32, L32, M32, dO, B, N, H, D)
    got = flash_bwd(dev(Q), dev(K), dev(V), dev(O32), dev(L32), dev(M32), dev(dO), B, N, H, D)
    for name, g, w in zip(("dq", "dk", "dv"), got, want):
        err = _rel(g.cpu().numpy(), w)
        print(f"{name} rel_err={err:.2e}")
        assert err < FP32_TOL, (name, err)


def test_flash_bwd_head_dim_above_256_is_rejected(gpu_ctx):
    from test_flash_bwd_gpu import flash_bwd
    x = torch.zeros((1 * 4, 2 * 264), device="cuda")
    s = torch.zeros(1 * 4 * 2, device="cuda")
    with pytest.raises(ValueError, match="supported: 1 to 256"):
        flash_bwd(x, x, x, x, s, s, x, 1, 4, 2, 264)
