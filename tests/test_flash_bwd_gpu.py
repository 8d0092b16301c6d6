"""Parity of skv_flash_bwd (causal FlashAttention backward, fp32) on the MI355X.

  * the reference's own test (gpu_test.py:871-1060) through the drop-in
    gpu.flash_attention_backward: its seed-42 inputs, the forward's O, L, M and
    the expected gradients from tests/golden/flash_bwd_kat_seed42.npz;
  * ragged shapes (N not a multiple of the 64/128-row tiles, every head_dim)
    against oracle/kv_oracle.flash_attention_backward on the same fp32 inputs;
  * the bench shape (B=8, N=2048, H=16, D=64) against a torch fp32 autograd
    reference, and through two identities that hold at any size when O, L, M
    come from the forward: the key-sum of dV equals the query-sum of dO, and
    the key-sum of dK vanishes (softmax is shift invariant);
  * bitwise-identical results on repeated calls (no atomics).
Tolerance: 1e-4 relative (Frobenius norm per tensor), the fp32 bar.
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
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def _lib():
    from simple_llm_amd import _lib
    return _lib


def flash_bwd(q, k, v, o, L, M, do, B, N, H, D, fast=False):
    """dq, dk, dv of device fp32 tensors through the C ABI; fast: with the
    workspace of the five-product form (dS stored, where it applies)."""
    lib = _lib()
    L_ = lib.lib()
    dq, dk, dv = (torch.empty_like(q) for _ in range(3))
    nb = (L_.skv_flash_bwd_fast_workspace_bytes(B, N, H, D) if fast
          else L_.skv_flash_bwd_workspace_bytes(B, N, H))
    ws = torch.empty(max(nb, 16), dtype=torch.uint8, device=q.device)
    rc = L_.skv_flash_bwd(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), q.data_ptr(), k.data_ptr(),
                          v.data_ptr(), o.data_ptr(), L.data_ptr(), M.data_ptr(), do.data_ptr(),
                          B, N, H, D, float(1 / np.sqrt(D)), ws.data_ptr(), ws.numel(),
                          lib.stream_handle(q.device))
    lib.check(rc, "skv_flash_bwd")
    return dq, dk, dv


def test_reference_backward_kat_through_dropin(gpu_ctx):
    from simple_llm_amd.gpu import gpu
    z = np.load(os.path.join(GOLDEN, "flash_bwd_kat_seed42.npz"))
    for i, (b, t, h, d) in enumerate(z["configs"]):
        b, t, h, d = int(b), int(t), int(h), int(d)
        banner(f"flash bwd reference KAT B={b} N={t} H={h} D={d}")
        Q, K, V, dO = (x.reshape(b * t, h * d) for x in mg.flash_bwd_inputs(b, t, h, d))
        E, T = h * d, b * t
        mk = lambda x: gpu.gpu_buffer_2d_create(gpu_ctx, T, E, np.asarray(x, np.float32))
        Qg, Kg, Vg, Og, dOg = mk(Q), mk(K), mk(V), mk(z[f"o_{i}"]), mk(dO)
        Lg = gpu.gpu_buffer_1d_create(gpu_ctx, T * h, z[f"l_{i}"].astype(np.float32))
        Mg = gpu.gpu_buffer_1d_create(gpu_ctx, T * h, z[f"m_{i}"].astype(np.float32))
        gQ, gK, gV = (gpu.gpu_buffer_2d_create(gpu_ctx, T, E) for _ in range(3))
        nqb = (t + gpu_ctx.config.flash_attn_br - 1) // gpu_ctx.config.flash_attn_br
        wK = gpu.gpu_buffer_2d_create(gpu_ctx, nqb * T, E)
        wV = gpu.gpu_buffer_2d_create(gpu_ctx, nqb * T, E)
        gpu.batch_begin(gpu_ctx)
        gpu.flash_attention_backward(gpu_ctx, Qg, Kg, Vg, Og, Lg, Mg, dOg, gQ, wK, wV, gK, gV,
                                     b, t, h, d)
        gpu.batch_commit(gpu_ctx)
        for name, buf in (("dq", gQ), ("dk", gK), ("dv", gV)):
            got = np.zeros((T, E), np.float32)
            gpu.gpu_buffer_2d_read(gpu_ctx, buf, got)
            err = _rel(got, z[f"{name}_{i}"])
            print(f"{name} rel_err={err:.2e}")
            assert err < TOL, (i, name, err)


def test_dropin_rejects_like_the_reference(gpu_ctx):
    from simple_llm_amd.gpu import gpu
    b, t, h, d = 1, 8, 2, 16
    T, E = b * t, h * d
    bufs = [gpu.gpu_buffer_2d_create(gpu_ctx, T, E) for _ in range(5)]
    Lg, Mg = (gpu.gpu_buffer_1d_create(gpu_ctx, T * h) for _ in range(2))
    outs = [gpu.gpu_buffer_2d_create(gpu_ctx, T, E) for _ in range(3)]
    wK = gpu.gpu_buffer_2d_create(gpu_ctx, T, E)
    wV = gpu.gpu_buffer_2d_create(gpu_ctx, T, E)
    args = [gpu_ctx, *bufs[:4], Lg, Mg, bufs[4], outs[0], wK, wV, outs[1], outs[2]]
    with pytest.raises(ValueError, match="exceeds maximum"):
        gpu.flash_attention_backward(*args, b, t, h, 256)
    with pytest.raises(ValueError, match="Invalid dimensions"):
        gpu.flash_attention_backward(*args, b, 0, h, d)
    bad = gpu.gpu_buffer_2d_create(gpu_ctx, T, E + 1)
    with pytest.raises(ValueError, match="grad_O shape mismatch"):
        gpu.flash_attention_backward(*args[:7], bad, *args[8:], b, t, h, d)


SHAPES = [(1, 1, 1, 16), (2, 5, 3, 16), (1, 63, 2, 32), (2, 64, 1, 32), (1, 65, 2, 64),
          (1, 129, 3, 64), (2, 200, 2, 128), (1, 300, 1, 64), (1, 513, 2, 128), (3, 40, 2, 64)]


@pytest.mark.parametrize("fast", [False, True])
@pytest.mark.parametrize("B,N,H,D", SHAPES)
def test_ragged_shapes_match_oracle(gpu_ctx, B, N, H, D, fast):
    banner(f"flash bwd vs oracle B={B} N={N} H={H} D={D} fast={fast}")
    rng = np.random.default_rng(B * 1000 + N * 10 + D)
    Q, K, V, dO = (rng.standard_normal((B * N, H * D)).astype(np.float32) for _ in range(4))
    O, L, M = ko.flash_attention(Q, K, V, B, N, H, D)
    O, L, M = O.astype(np.float32), L.astype(np.float32), M.astype(np.float32)
    want = ko.flash_attention_backward(Q, K, V, O, L, M, dO, B, N, H, D)
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()
    got = flash_bwd(dev(Q), dev(K), dev(V), dev(O), dev(L), dev(M), dev(dO), B, N, H, D,
                    fast=fast)
    for name, g, w in zip(("dq", "dk", "dv"), got, want):
        g = g.cpu().numpy()
        if N == 1 and name != "dv":
            # one key: dS = dP - Dl = dO.V - dO.O = 0, so dq = dk = 0; fp32 leaves rounding
            assert np.abs(g).max() < 1e-5
            continue
        err = _rel(g, w)
        print(f"{name} rel_err={err:.2e}")
        assert err < TOL, (name, err)


@pytest.mark.parametrize("B,N,H,D", [(2, 300, 3, 64), (1, 517, 2, 48), (3, 128, 2, 40),
                                     (2, 261, 2, 20), (1, 64, 4, 16), (2, 1024, 4, 32),
                                     (1, 1, 2, 64), (2, 33, 3, 36)])
def test_five_product_form_gives_the_same_bits(gpu_ctx, B, N, H, D):
    """With the larger workspace (D <= 64) the dK/dV kernel writes
    dS and dQ is formed from it instead of from S and dP recomputed: the same
    products in the same order, so dq, dk and dv are bit-identical to the
    seven-product form's (head dims with every load mode)."""
    banner(f"flash bwd five-product form B={B} N={N} H={H} D={D}")
    L_ = _lib().lib()
    assert L_.skv_flash_bwd_fast_workspace_bytes(B, N, H, D) > L_.skv_flash_bwd_workspace_bytes(
        B, N, H)
    rng = np.random.default_rng(N + D)
    Q, K, V, dO = (rng.standard_normal((B * N, H * D)).astype(np.float32) for _ in range(4))
    O, L, M = ko.flash_attention(Q, K, V, B, N, H, D)
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()
    args = (dev(Q), dev(K), dev(V), dev(O), dev(L), dev(M), dev(dO), B, N, H, D)
    slow = flash_bwd(*args)
    fast = flash_bwd(*args, fast=True)
    for name, a, b in zip(("dq", "dk", "dv"), slow, fast):
        assert torch.equal(a, b), name


def _torch_reference(q, k, v, do, B, N, H, D):
    """fp32 O, L, M and autograd gradients of causal attention, [B*N, H*D] layout."""
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
    dq, dk, dv = torch.autograd.grad(o4, (q4, k4, v4), g)
    flat = lambda x: x.transpose(1, 2).reshape(B * N, H * D).contiguous().detach()
    stats = lambda x: x.squeeze(-1).transpose(1, 2).reshape(-1).contiguous().detach()
    return flat(o4), stats(l), stats(m), flat(dq), flat(dk), flat(dv)


@pytest.mark.parametrize("B,N,H,D", [(8, 2048, 16, 64), (2, 2048, 8, 128)])
def test_bench_shape_against_torch_fp32_and_identities(gpu_ctx, B, N, H, D):
    banner(f"flash bwd bench shape B={B} N={N} H={H} D={D}")
    g = torch.Generator(device="cuda").manual_seed(11)
    q, k, v, do = (torch.randn(B * N, H * D, device="cuda", generator=g) for _ in range(4))
    o, L, M, rq, rk, rv = _torch_reference(q, k, v, do, B, N, H, D)
    # the form the bench times: five products where D <= 64 (the workspace holds dS)
    dq, dk, dv = flash_bwd(q, k, v, o, L, M, do, B, N, H, D, fast=True)
    for name, x, r in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        err = float((x - r).double().norm() / r.double().norm())
        print(f"{name} rel_err vs torch fp32 = {err:.2e}")
        assert err < TOL, (name, err)
    # key-sum of dV = query-sum of dO; key-sum of dK = 0, per (b, h, d)
    sdv = dv.double().view(B, N, H, D).sum(1)
    sdo = do.double().view(B, N, H, D).sum(1)
    assert float((sdv - sdo).norm() / sdo.norm()) < TOL
    sdk = dk.double().view(B, N, H, D).sum(1)
    assert float(sdk.abs().max() / dk.double().view(B, N, H, D).abs().sum(1).max()) < TOL
    again = flash_bwd(q, k, v, o, L, M, do, B, N, H, D, fast=True)
    for x, y in zip((dq, dk, dv), again):
        assert torch.equal(x, y)  # bitwise reproducible
    seven = flash_bwd(q, k, v, o, L, M, do, B, N, H, D)
    for x, y in zip((dq, dk, dv), seven):
        assert torch.equal(x, y)  # the seven-product form gives the same bits
