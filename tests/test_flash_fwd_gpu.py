"""Parity of the fp32 flash-attention forward (skv_flash_fwd) and of the
fp32-cache prefill that shares its kernel, on the MI355X.

  * the reference's own test (test_flash_attention, gpu_test.py:743-870)
    through the drop-in gpu.flash_attention: its seven seed-42 configs, O, L
    and M against tests/golden/flash_kat_seed42.npz (float64 SDPA and direct
    sums), the "Medium" config regenerated from the seed;
  * ragged shapes (N off the 64/128-row tiles, every head_dim) against the
    float64 oracle kv_oracle.flash_attention;
  * the bench shape against torch fp32, and the forward's O, L, M fed to
    skv_flash_bwd against torch fp32 autograd (the training pair);
  * kv_cache_prefill on float32 caches (prefix offsets, GQA, ragged n_new)
    against kv_oracle.prefill_attention.
Tolerance: 1e-4 relative, the fp32 bar (norm-wise per row for O, per tensor
for L and M).
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import make_golden as mg
from conftest import GOLDEN, banner
from oracle import kv_oracle as ko

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def _rel_rows(a, b):
    a = np.asarray(a, np.float64).reshape(-1, np.shape(a)[-1])
    b = np.asarray(b, np.float64).reshape(-1, np.shape(b)[-1])
    return float((np.linalg.norm(a - b, axis=1) / np.maximum(np.linalg.norm(b, axis=1), 1e-30)).max())


def flash_fwd(q, k, v, B, N, H, D):
    from simple_llm_amd import _lib
    L_ = _lib.lib()
    o = torch.empty_like(q)
    Ls = torch.empty(B * N * H, device=q.device)
    Ms = torch.empty(B * N * H, device=q.device)
    rc = L_.skv_flash_fwd(o.data_ptr(), Ls.data_ptr(), Ms.data_ptr(), q.data_ptr(), k.data_ptr(),
                          v.data_ptr(), B, N, H, D, float(1 / np.sqrt(D)),
                          _lib.stream_handle(q.device))
    _lib.check(rc, "skv_flash_fwd")
    return o, Ls, Ms


def test_reference_flash_kat_through_dropin(gpu_ctx):
    from simple_llm_amd.gpu import gpu
    z = np.load(os.path.join(GOLDEN, "flash_kat_seed42.npz"))
    for i, (b, t, h, d, desc) in enumerate(mg.FLASH_CONFIGS):
        banner(f"flash fwd reference KAT {desc} B={b} N={t} H={h} D={d}")
        Q, K, V = (x.reshape(b * t, h * d) for x in mg.flash_inputs(b, t, h, d))
        if i in mg.FLASH_STORED:
            o_w, l_w, m_w = z[f"o_{i}"], z[f"l_{i}"], z[f"m_{i}"]
        else:
            o_w, l_w, m_w = mg.flash_expected(Q, K, V, b, t, h, d)
        T, E = b * t, h * d
        Qg, Kg, Vg = (gpu.gpu_buffer_2d_create(gpu_ctx, T, E, x) for x in (Q, K, V))
        Og = gpu.gpu_buffer_2d_create(gpu_ctx, T, E)
        Lg = gpu.gpu_buffer_1d_create(gpu_ctx, T * h)
        Mg = gpu.gpu_buffer_1d_create(gpu_ctx, T * h)
        gpu.batch_begin(gpu_ctx)
        gpu.flash_attention(gpu_ctx, Qg, Kg, Vg, Og, Lg, Mg, b, t, h, d)
        gpu.batch_commit(gpu_ctx)
        o = np.zeros((T, E), np.float32)
        gpu.gpu_buffer_2d_read(gpu_ctx, Og, o)
        l_ = Lg.buffer.cpu().numpy()
        m_ = Mg.buffer.cpu().numpy()
        eo = _rel_rows(o.reshape(T, h, d), o_w.reshape(T, h, d))
        el, em = _rel(l_, l_w), _rel(m_, m_w)
        print(f"O {eo:.2e} L {el:.2e} M {em:.2e}")
        assert eo < TOL and el < TOL and em < TOL, (desc, eo, el, em)


def test_dropin_rejects_like_the_reference(gpu_ctx):
    from simple_llm_amd.gpu import gpu
    b, t, h, d = 1, 8, 2, 16
    T, E = b * t, h * d
    Q, K, V, O = (gpu.gpu_buffer_2d_create(gpu_ctx, T, E) for _ in range(4))
    Lg, Mg = (gpu.gpu_buffer_1d_create(gpu_ctx, T * h) for _ in range(2))
    with pytest.raises(ValueError, match="exceeds maximum"):
        gpu.flash_attention(gpu_ctx, Q, K, V, O, Lg, Mg, b, t, h, 256)
    with pytest.raises(ValueError, match="Invalid dimensions"):
        gpu.flash_attention(gpu_ctx, Q, K, V, O, Lg, Mg, 0, t, h, d)
    with pytest.raises(ValueError, match="L shape mismatch"):
        gpu.flash_attention(gpu_ctx, Q, K, V, O, gpu.gpu_buffer_1d_create(gpu_ctx, T), Mg,
                            b, t, h, d)


SHAPES = [(1, 1, 1, 16), (2, 5, 3, 16), (1, 63, 2, 32), (2, 64, 1, 32), (1, 65, 2, 64),
          (1, 129, 3, 64), (2, 200, 2, 128), (1, 300, 1, 64), (1, 513, 2, 128), (3, 40, 2, 64)]


@pytest.mark.parametrize("B,N,H,D", SHAPES)
def test_ragged_shapes_match_oracle(gpu_ctx, B, N, H, D):
    banner(f"flash fwd vs oracle B={B} N={N} H={H} D={D}")
    rng = np.random.default_rng(B * 100 + N + D)
    Q, K, V = (rng.standard_normal((B * N, H * D)).astype(np.float32) for _ in range(3))
    o_w, l_w, m_w = ko.flash_attention(Q, K, V, B, N, H, D)
    dev = lambda x: torch.from_numpy(x).cuda()
    o, L, M = flash_fwd(dev(Q), dev(K), dev(V), B, N, H, D)
    eo = _rel_rows(o.cpu().numpy().reshape(-1, D), o_w.reshape(-1, D))
    el, em = _rel(L.cpu().numpy(), l_w), _rel(M.cpu().numpy(), m_w)
    print(f"O {eo:.2e} L {el:.2e} M {em:.2e}")
    assert eo < TOL and el < TOL and em < TOL


def _torch_attention(q, k, v, do, B, N, H, D):
    torch.backends.cuda.matmul.allow_tf32 = False
    heads = lambda x: x.view(B, N, H, D).transpose(1, 2).contiguous().requires_grad_(True)
    q4, k4, v4 = heads(q), heads(k), heads(v)
    s = (q4 @ k4.transpose(-1, -2).contiguous()) * (1.0 / np.sqrt(D))
    mask = torch.ones(N, N, dtype=torch.bool, device=q.device).tril()
    s = s.masked_fill(~mask, float("-inf"))
    m = s.amax(-1, keepdim=True)
    e = torch.exp(s - m)
    l = e.sum(-1, keepdim=True)
    o4 = (e / l) @ v4
    g = do.view(B, N, H, D).transpose(1, 2).contiguous()
    grads = torch.autograd.grad(o4, (q4, k4, v4), g)
    flat = lambda x: x.transpose(1, 2).reshape(B * N, H * D).contiguous().detach()
    stats = lambda x: x.squeeze(-1).transpose(1, 2).reshape(-1).contiguous().detach()
    return flat(o4), stats(l), stats(m), [flat(x) for x in grads]


@pytest.mark.parametrize("B,N,H,D", [(8, 2048, 16, 64), (2, 2048, 8, 128)])
def test_forward_backward_pair_against_torch_fp32(gpu_ctx, B, N, H, D):
    banner(f"flash fwd+bwd B={B} N={N} H={H} D={D}")
    from simple_llm_amd import _lib
    g = torch.Generator(device="cuda").manual_seed(17)
    q, k, v, do = (torch.randn(B * N, H * D, device="cuda", generator=g) for _ in range(4))
    o_r, l_r, m_r, grads_r = _torch_attention(q, k, v, do, B, N, H, D)
    o, L, M = flash_fwd(q, k, v, B, N, H, D)
    for name, x, r in (("O", o, o_r), ("L", L, l_r), ("M", M, m_r)):
        err = float((x - r).double().norm() / r.double().norm())
        print(f"{name} rel_err vs torch fp32 = {err:.2e}")
        assert err < TOL, (name, err)
    L_ = _lib.lib()
    dq, dk, dv = (torch.empty_like(q) for _ in range(3))
    ws = torch.empty(L_.skv_flash_bwd_workspace_bytes(B, N, H), dtype=torch.uint8, device="cuda")
    rc = L_.skv_flash_bwd(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), q.data_ptr(), k.data_ptr(),
                          v.data_ptr(), o.data_ptr(), L.data_ptr(), M.data_ptr(), do.data_ptr(),
                          B, N, H, D, float(1 / np.sqrt(D)), ws.data_ptr(), ws.numel(),
                          _lib.stream_handle(q.device))
    _lib.check(rc, "skv_flash_bwd")
    for name, x, r in zip(("dq", "dk", "dv"), (dq, dk, dv), grads_r):
        err = float((x - r).double().norm() / r.double().norm())
        print(f"{name} rel_err vs torch fp32 autograd = {err:.2e}")
        assert err < TOL, (name, err)


@pytest.mark.parametrize("B,T,Hq,Hkv,D,prefix,C,n_new", [
    (2, 1024, 16, 16, 128, [0, 700], 300, None),
    (3, 2400, 32, 8, 128, [100, 0, 2000], 200, [200, 5, 0]),  # GQA G=4, ragged chunk
    (2, 1200, 12, 12, 64, [1000, 33], 129, None),             # C3 head shape
    (1, 700, 6, 2, 32, [37], 600, None),                       # G=3, head_dim 32
])
def test_fp32_cache_prefill_matches_oracle(gpu_ctx, B, T, Hq, Hkv, D, prefix, C, n_new):
    banner(f"fp32 prefill B={B} T={T} Hq={Hq} Hkv={Hkv} D={D} prefix={prefix} C={C}")
    from simple_llm_amd.gpu import gpu
    rng = np.random.default_rng(B * 11 + C)
    cache = gpu.kv_cache_create(gpu_ctx, gpu.KVCacheConfig(B, T, 1, Hq, D, n_kv_heads=Hkv))
    layer = cache.layers[0]
    k = rng.standard_normal((B, T, Hkv, D)).astype(np.float32)
    v = rng.standard_normal((B, T, Hkv, D)).astype(np.float32)
    prefix = np.asarray(prefix, np.int64)
    kp, vp = np.zeros_like(k), np.zeros_like(v)
    for b in range(B):
        kp[b, :prefix[b]], vp[b, :prefix[b]] = k[b, :prefix[b]], v[b, :prefix[b]]
    layer.k_cache.buffer.copy_(torch.from_numpy(kp.reshape(-1, Hkv * D)))
    layer.v_cache.buffer.copy_(torch.from_numpy(vp.reshape(-1, Hkv * D)))
    layer.lens.copy_(torch.from_numpy(prefix.astype(np.int32)))
    layer.host_lens[:] = prefix
    kn = np.stack([k[b, prefix[b]:prefix[b] + C] for b in range(B)])
    vn = np.stack([v[b, prefix[b]:prefix[b] + C] for b in range(B)])
    q = rng.standard_normal((B, C, Hq, D)).astype(np.float32)
    out = torch.full((B, C, Hq, D), float("nan"), device="cuda")
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()
    gpu.kv_cache_prefill(gpu_ctx, cache, 0, dev(kn), dev(vn), dev(q), out, n_new=n_new)
    nn = np.full(B, C) if n_new is None else np.asarray(n_new)
    want = ko.prefill_attention(q, k, v, prefix, q_lens=nn)
    got = out.cpu().numpy()
    valid = np.zeros((B, C, Hq), bool)
    for b in range(B):
        valid[b, :nn[b]] = True
    err = _rel_rows(got[valid], want[valid])
    print(f"rel_err={err:.2e}")
    assert err < TOL
    assert not got[~valid].any()  # rows past n_new are zeros (and were written)
