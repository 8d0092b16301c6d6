"""skv_decode_attn_noalloc, the allocation-free decode entry point, against
skv_decode_attn (the same kernels with a caller workspace) through the C ABI.

The entry point keeps its split-K partials in a file-scope device array of
SKV_DECODE_NOALLOC_MAX_BYTES per GPU. Two calls in a row, the second with a
smaller batch and shorter fills, must each equal skv_decode_attn bit for bit
(same plan, same kernels) and the float64 oracle within 1e-4; the array
keeps the first call's contents, so the second also checks that nothing
stale is read. A plan above the maximum is rejected before any GPU work.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from conftest import banner
from oracle import kv_oracle as ko

pytestmark = pytest.mark.gpu

MAX_BYTES = 64 << 20


def _case(rng, B, T, Hq, Hkv, D, dtype):
    k = rng.standard_normal((B, T, Hkv, D)).astype(np.float32)
    v = rng.standard_normal((B, T, Hkv, D)).astype(np.float32)
    if dtype == torch.bfloat16:
        k, v = ko.bf16_round(k), ko.bf16_round(v)
    q = rng.standard_normal((B, Hq, D)).astype(np.float32)
    return k, v, q


def _both(L, _lib, k, v, q, lens, Hq, Hkv, D, dtype):
    """(noalloc output, workspace output) of one decode call."""
    B, T = k.shape[:2]
    dev = lambda x, dt=torch.float32: torch.from_numpy(np.ascontiguousarray(x)).cuda().to(dt)
    kd, vd, qd = dev(k, dtype), dev(v, dtype), dev(q)
    ld = torch.from_numpy(np.asarray(lens, np.int32)).cuda()
    chunk, nch = ctypes.c_int(), ctypes.c_int()
    _lib.check(L.skv_decode_plan(B, Hq, Hkv, D, _lib.dtype_code(dtype), int(max(lens)),
                                 int(np.sum(lens)), 0, ctypes.byref(chunk), ctypes.byref(nch)),
               "plan")
    cdt = _lib.dtype_code(dtype)
    s = _lib.stream_handle(qd.device)
    out_n = torch.full_like(qd, float("nan"))
    rc = L.skv_decode_attn_noalloc(out_n.data_ptr(), qd.data_ptr(), kd.data_ptr(), vd.data_ptr(),
                                   ld.data_ptr(), B, Hq, Hkv, D, T, float(D ** -0.5), chunk.value,
                                   nch.value, cdt, _lib.F32, _lib.F32, s)
    _lib.check(rc, "skv_decode_attn_noalloc")
    need = L.skv_decode_workspace_bytes(B, Hq, D, nch.value)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    out_w = torch.full_like(qd, float("nan"))
    rc = L.skv_decode_attn(out_w.data_ptr(), qd.data_ptr(), kd.data_ptr(), vd.data_ptr(),
                           ld.data_ptr(), B, Hq, Hkv, D, T, float(D ** -0.5), chunk.value,
                           nch.value, ws.data_ptr(), need, cdt, _lib.F32, _lib.F32, s)
    _lib.check(rc, "skv_decode_attn")
    return out_n.cpu().numpy(), out_w.cpu().numpy()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_equals_workspace_entry_point(gpu_ctx, dtype):
    from simple_llm_amd import _lib
    L = _lib.lib()
    rng = np.random.default_rng(17)
    # first call: 6 sequences, GQA, long fills; second: 2 sequences, short fills
    for B, T, Hq, Hkv, D, lens in [(6, 3000, 16, 4, 128, [3000, 2999, 17, 1500, 1, 2048]),
                                   (2, 200, 16, 4, 128, [200, 33])]:
        banner(f"noalloc decode B={B} T={T} Hq={Hq} Hkv={Hkv} D={D} {dtype}")
        k, v, q = _case(rng, B, T, Hq, Hkv, D, dtype)
        got_n, got_w = _both(L, _lib, k, v, q, lens, Hq, Hkv, D, dtype)
        np.testing.assert_array_equal(got_n, got_w)
        want = ko.decode_attention(q, k, v, np.asarray(lens))
        err = float((np.linalg.norm(got_n - want, axis=-1) /
                     np.linalg.norm(want, axis=-1)).max())
        print(f"rel_err={err:.3e}")
        assert err < 1e-4


def test_noalloc_rejects_plans_above_the_maximum(gpu_ctx):
    from simple_llm_amd import _lib
    L = _lib.lib()
    # a plan of 64 sequences x 64 heads x 2049 slots needs ~2.2 GB: rejected
    # by the size check, before any pointer is used (the pointers are NULL, so
    # the null-pointer check would stop the call before any launch even if the
    # size check did not)
    B, Hq, D, n = 64, 64, 128, 2049
    assert L.skv_decode_workspace_bytes(B, Hq, D, n) > MAX_BYTES
    rc = L.skv_decode_attn_noalloc(None, None, None, None, None, B, Hq, Hq, D, 1 << 20, 0.1, 512,
                                   n, 1, 0, 0, None)
    assert rc == _lib.SKV_E_WORKSPACE
    assert b"maximum" in L.skv_last_error()
