"""The C ABI library loads, exports what include/skv.h declares and rejects
bad arguments before any device work. CPU only: no call here reaches a
kernel launch."""
from __future__ import annotations

import ctypes

import pytest

from simple_llm_amd import _lib


def test_library_exports_every_header_function():
    names = _lib.header_functions()
    assert len(names) >= 10
    L = _lib.lib()
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, f"libskv.so lacks {missing}"
    # the ctypes signature table covers the header exactly
    assert sorted(names) == sorted(_lib._SIGNATURES)


def test_version():
    assert _lib.lib().skv_version() == 100


def _plan(B, Hkv, max_len, hint=0, total=0, Hq=None, D=64, dt=_lib.F32):
    c, n = ctypes.c_int(), ctypes.c_int()
    rc = _lib.lib().skv_decode_plan(B, Hkv if Hq is None else Hq, Hkv, D, dt, max_len, total, hint,
                                    ctypes.byref(c), ctypes.byref(n))
    return rc, c.value, n.value


@pytest.mark.parametrize("B,Hkv,L", [(4, 16, 32256), (8, 8, 2048), (64, 8, 8192), (1, 1, 1),
                                     (16, 12, 1024), (1, 4, 256), (2, 24, 100000)])
def test_decode_plan_covers_every_length(B, Hkv, L):
    rc, chunk, n = _plan(B, Hkv, L)
    assert rc == 0
    assert chunk % 32 == 0 and 32 <= chunk <= 8192
    # one workgroup range per chunk of every sequence, plus one spare slot
    # per sequence for the piece that starts inside a workgroup's range
    assert (n - 1) * chunk >= L > (n - 2) * chunk


def test_decode_plan_c4_and_ragged_total():
    # C4 (MHA): 4 sequences x 16 kv heads (one head group) at 32256 -> one
    # workgroup per CU: 512-token chunks, 4 * 63 = 252 workgroups, 64 slots
    # per sequence
    assert _plan(4, 16, 32256) == (0, 512, 64)
    # the same stream with 4 query heads per kv head keeps two per CU:
    # 256-token chunks, 4 * 126 = 504 workgroups, 127 slots
    assert _plan(4, 16, 32256, Hq=64) == (0, 256, 127)
    # a ragged batch plans from its total fill, not from B * max_len (C5:
    # 64 sequences, 32 query / 8 kv heads)
    rc, chunk, n = _plan(64, 8, 8192, total=64 * 2000, Hq=32)
    assert rc == 0 and chunk == 256 and n == 33
    assert _plan(64, 8, 8192, Hq=32)[1] > chunk
    # short MHA streams (C2: 8 x 2048, 8 heads; C3: 16 x 1024, 12 heads)
    # stay at two workgroups per CU, with the 32-token minimum chunk
    assert _plan(8, 8, 2048)[:2] == (0, 32)
    assert _plan(16, 12, 1024)[:2] == (0, 32)


@pytest.mark.parametrize("B,Hkv,Hq,L,total", [(64, 8, 32, 8192, 0), (64, 8, 32, 8192, 132154),
                                                (4, 8, 32, 32768, 128000), (1, 2, 8, 300, 0),
                                                (16, 16, 32, 1024, 0), (8, 4, 32, 100000, 0)])
def test_decode_plan_gqa_matrix_core_kernel(B, Hkv, Hq, L, total):
    """Grouped queries over a bf16 cache with head_dim 64/128 run the MFMA
    kernel: one busy workgroup per CU for 224 of the 256 CUs, chunks a
    multiple of 16, every length covered."""
    rc, chunk, n = _plan(B, Hkv, L, total=total, Hq=Hq, D=128, dt=_lib.BF16)
    assert rc == 0
    assert chunk % 16 == 0 and 32 <= chunk <= 8192
    assert (n - 1) * chunk >= L > (n - 2) * chunk
    groups = Hkv // min(8, Hkv & -Hkv)
    tot = total if total > 0 else B * L
    if 32 < chunk < 8192:
        assert -(-tot * groups // chunk) <= 224 < -(-tot * groups // (chunk - 16))


def test_decode_plan_c5_kernel_choice():
    # C5 (64 sequences, 32 query / 8 kv heads, lengths summing to 132154):
    # the bf16 D=128 cache gets 592-token chunks (224 workgroups), the same
    # shapes over an fp32 cache (VALU kernel) 288-token ones (459)
    assert _plan(64, 8, 8192, total=132154, Hq=32, D=128, dt=_lib.BF16) == (0, 592, 15)
    assert _plan(64, 8, 8192, total=132154, Hq=32, D=128, dt=_lib.F32) == (0, 288, 30)
    # head dims other than 64 and 128 and MHA keep the VALU plans
    assert _plan(64, 8, 8192, total=132154, Hq=32, D=96, dt=_lib.BF16)[1] == 288
    assert _plan(4, 16, 32256, D=128, dt=_lib.BF16) == (0, 512, 64)


def test_decode_plan_hint_and_errors():
    rc, chunk, n = _plan(4, 16, 32768, hint=1000)
    assert rc == 0 and chunk == 1008 and n == 34
    assert _plan(0, 16, 100)[0] == _lib.SKV_E_INVALID
    assert _plan(4, 16, 0)[0] == _lib.SKV_E_INVALID
    assert b"dims must be > 0" in _lib.lib().skv_last_error()
    assert _plan(4, 16, 100, Hq=0)[0] == _lib.SKV_E_INVALID
    assert _plan(4, 16, 100, Hq=24)[0] == _lib.SKV_E_INVALID
    assert b"not a multiple" in _lib.lib().skv_last_error()


def test_workspace_bytes():
    L = _lib.lib()
    # partials (o, m, l) per (query head, slot), then B + 1 int64 prefix sums
    assert L.skv_decode_workspace_bytes(4, 16, 128, 32) == 4 * 16 * 32 * (128 + 2) * 4 + 5 * 8
    assert L.skv_decode_workspace_bytes(0, 16, 128, 32) == 0


def test_entry_points_reject_bad_arguments():
    L = _lib.lib()
    fake = 4096  # never dereferenced: each call below fails validation first
    rc = L.skv_append(None, None, None, None, None, 2, 4, 64, 128, 0, 0, None)
    assert rc == _lib.SKV_E_INVALID
    rc = L.skv_append(fake, fake, fake, fake, fake, 2, 4, 64, 128, 7, 0, None)
    assert rc == _lib.SKV_E_INVALID and b"dtype" in L.skv_last_error()
    rc = L.skv_append_paged(fake, fake, fake, fake, fake, fake, 4, 12, 2, 4, 64, 0, 0, None)
    assert rc == _lib.SKV_E_INVALID and b"power of two" in L.skv_last_error()
    ws = L.skv_decode_workspace_bytes(2, 4, 64, 2)
    args = dict(B=2, Hq=4, Hkv=4, D=64, T=128, scale=0.125, chunk=256, n=2)

    def dec(**kw):
        a = {**args, **kw}
        return L.skv_decode_attn(fake, fake, fake, fake, fake, a["B"], a["Hq"], a["Hkv"], a["D"],
                                 a["T"], a["scale"], a["chunk"], a["n"], fake,
                                 kw.get("ws", ws), 0, 0, 0, None)

    assert dec(D=2056) == _lib.SKV_E_UNSUPPORTED  # head dims 1 to 2048 at G <= 2
    ws8 = L.skv_decode_workspace_bytes(2, 8, 520, 2)
    assert dec(Hq=8, Hkv=1, D=520, ws=ws8) == _lib.SKV_E_UNSUPPORTED  # G = 8: up to 512
    assert b"head_dim 520 with 8 query heads" in L.skv_last_error()
    assert dec(D=0) == _lib.SKV_E_INVALID
    assert dec(Hq=6, Hkv=4) == _lib.SKV_E_INVALID
    assert dec(chunk=100) == _lib.SKV_E_INVALID  # not a multiple of 16
    assert dec(ws=ws - 1) == _lib.SKV_E_WORKSPACE
    assert dec(n=1) == _lib.SKV_E_INVALID  # no spare slot per sequence
    ws48 = L.skv_decode_workspace_bytes(2, 48, 64, 2)
    assert dec(Hq=48, Hkv=3, ws=ws48) == _lib.SKV_E_UNSUPPORTED  # G = 16 has no kernel
    rc = L.skv_append_chunk(fake, fake, fake, fake, fake, None, 2, 0, 4, 64, 128, 0, 0, None)
    assert rc == _lib.SKV_E_INVALID
    assert L.skv_advance(None, None, 1, 2, 128, None) == _lib.SKV_E_INVALID


def test_sample_rejects_bad_arguments():
    L = _lib.lib()
    fake = 4096  # never dereferenced: each call below fails validation first
    args = [fake, None, fake, fake, 8, fake, 2, 100, 1.0, 0, 1.0, 0.0, 1.0, 64, 42, None, 0, None]

    def call(**kw):
        a = list(args)
        for k, v in kw.items():
            a[{"V": 7, "T": 8, "top_k": 9, "pen": 12, "M": 6}[k]] = v
        return L.skv_sample(*a)

    assert call(V=70000) == _lib.SKV_E_UNSUPPORTED
    assert call(T=-1.0) == _lib.SKV_E_INVALID
    assert call(top_k=-3) == _lib.SKV_E_INVALID
    assert call(pen=0.0) == _lib.SKV_E_INVALID
    assert call(M=0) == _lib.SKV_E_INVALID
    # the split path's workspace: rows of 8192..65536 entries, ceil(V / 2048) slices a row
    assert L.skv_sample_workspace_bytes(16, 50304) == 16 * 25 * 8
    assert L.skv_sample_workspace_bytes(3, 8192) == 3 * 4 * 8
    assert L.skv_sample_workspace_bytes(3, 8191) == 0
    assert L.skv_sample_workspace_bytes(3, 65537) == 0


def test_flash_bwd_rejects_bad_arguments():
    L = _lib.lib()
    fake = 4096  # never dereferenced: each call below fails validation first
    B, N, H = 2, 100, 3
    need = L.skv_flash_bwd_workspace_bytes(B, N, H)
    assert need == B * N * H * 4 and L.skv_flash_bwd_workspace_bytes(0, N, H) == 0
    # the five-product form: the row deltas (256-byte aligned block), then dS [B*H][N][N]
    # in 32 x 32 tiles (N = 100 -> 4 x 4 tiles)
    assert L.skv_flash_bwd_fast_workspace_bytes(B, N, H, 64) == 2560 + B * H * 128 * 128 * 4
    assert L.skv_flash_bwd_fast_workspace_bytes(B, N, H, 65) == need  # D > 64: seven products

    def call(D=64, ws_bytes=None, ptr=fake, scale=0.125, n=N):
        return L.skv_flash_bwd(ptr, fake, fake, fake, fake, fake, fake, fake, fake, fake, B, n,
                               H, D, scale, fake, need - 4 if ws_bytes is None else ws_bytes,
                               None)

    assert call() == _lib.SKV_E_WORKSPACE
    assert call(D=257, ws_bytes=need) == _lib.SKV_E_UNSUPPORTED  # head dims 1 to 256
    assert b"supported: 1 to 256" in L.skv_last_error()
    assert call(ptr=None, ws_bytes=need) == _lib.SKV_E_INVALID
    assert call(ptr=fake + 4, ws_bytes=need) == _lib.SKV_E_INVALID  # not 16-byte aligned
    assert call(scale=0.0, ws_bytes=need) == _lib.SKV_E_INVALID
    assert call(n=0, ws_bytes=need) == _lib.SKV_E_INVALID
    assert "workspace" in (call() and _lib.lib().skv_last_error().decode())


def test_flash_fwd_rejects_bad_arguments():
    L = _lib.lib()
    fake = 4096  # never dereferenced: each call below fails validation first

    def call(D=64, ptr=fake, scale=0.125, n=100):
        return L.skv_flash_fwd(ptr, None, None, fake, fake, fake, 2, n, 3, D, scale, None)

    assert call(D=257) == _lib.SKV_E_UNSUPPORTED  # head dims 1 to 256
    assert b"supported: 1 to 256" in L.skv_last_error()
    assert call(ptr=None) == _lib.SKV_E_INVALID
    assert call(ptr=fake + 4) == _lib.SKV_E_INVALID  # not 16-byte aligned
    assert call(scale=-1.0) == _lib.SKV_E_INVALID
    assert call(n=0) == _lib.SKV_E_INVALID


def test_prefill_rejects_bad_arguments():
    L = _lib.lib()
    fake = 4096  # never dereferenced: each call below fails validation first

    def call(out=fake, D=128, Hq=4, ns=1, ws=None, ws_bytes=0):
        return L.skv_prefill_attn(out, fake, fake, fake, fake, None, 2, 16, Hq, 4, D, 1024, 0.125,
                                  ns, ws, ws_bytes, 1, 1, 1, None)

    assert call(D=264) == _lib.SKV_E_UNSUPPORTED  # head dims 1 to 256
    assert call(out=fake + 8) == _lib.SKV_E_INVALID  # bf16 path: 16-byte alignment
    assert b"16-byte aligned" in L.skv_last_error()
    assert call(ns=2, ws=fake + 4, ws_bytes=1 << 30) == _lib.SKV_E_INVALID
    assert call(Hq=12) == _lib.SKV_E_UNSUPPORTED  # G = 3
    assert call(ns=33) == _lib.SKV_E_INVALID
    need = L.skv_prefill_workspace_bytes(2, 16, 4, 128, 2)
    assert need == 2 * 2 * 16 * 4 * (128 + 2) * 4 + 16  # partials, then the fills' snapshot
    assert call(ns=2, ws=fake, ws_bytes=need - 1) == _lib.SKV_E_WORKSPACE
    # 65536 kv heads of 256: a 64-row K/V tile spans more than 2 GB of cache rows
    assert L.skv_prefill_attn(fake, fake, fake, fake, fake, None, 2, 16, 65536, 65536, 256, 1024,
                              0.125, 1, None, 0, 1, 1, 1, None) == _lib.SKV_E_UNSUPPORTED
    assert b"too wide" in L.skv_last_error()


def test_argmax_workspace_and_rejects():
    L = _lib.lib()
    # one 2048-column slice per workgroup; candidates (value, index) per slice
    # when a row needs more than one
    assert L.skv_argmax_workspace_bytes(16, 50304) == 16 * 2 * 25 * 4
    assert L.skv_argmax_workspace_bytes(4, 2048) == 0
    assert L.skv_argmax_workspace_bytes(0, 10) == 0
    fake = 4096  # never dereferenced: each call below fails validation first
    assert L.skv_argmax(fake, fake, 16, 50304, None, 0, None) == _lib.SKV_E_WORKSPACE
    assert L.skv_argmax(fake, fake, 16, 50304, fake, 16 * 2 * 25 * 4 - 1, None) == \
        _lib.SKV_E_WORKSPACE
    assert L.skv_argmax(None, fake, 1, 10, None, 0, None) == _lib.SKV_E_INVALID


def test_check_maps_status_to_exceptions():
    L = _lib.lib()
    L.skv_append(None, None, None, None, None, 1, 1, 64, 1, 0, 0, None)
    with pytest.raises(ValueError, match="null pointer"):
        _lib.check(_lib.SKV_E_INVALID, "x")
    with pytest.raises(_lib.SkvError):
        _lib.check(_lib.SKV_E_HIP, "x")


@pytest.mark.parametrize("B,Hq,Hkv,D,dt,L,hint", [
    (8, 8, 8, 64, _lib.F32, 2048, 0),        # C2
    (16, 12, 12, 64, _lib.F32, 1024, 0),     # C3
    (4, 16, 16, 128, _lib.BF16, 32768, 0),   # C4
    (64, 32, 8, 128, _lib.BF16, 8320, 0),    # C5 (matrix-core GQA plan)
    (3, 6, 2, 48, _lib.F32, 5000, 0),
    (8, 8, 8, 64, _lib.F32, 2048, 100),      # a caller's chunk hint
])
def test_decode_plan_is_monotone_in_total(B, Hq, Hkv, D, dt, L, hint):
    """The host's plan memo relies on it: the chunk never decreases as the
    batch's total fill grows, and the slot count follows the chunk. (A total
    of 0 stands for B * max_len.)"""
    assert _plan(B, Hkv, L, hint=hint, total=0, Hq=Hq, D=D, dt=dt) == \
        _plan(B, Hkv, L, hint=hint, total=B * L, Hq=Hq, D=D, dt=dt)
    prev = None
    for total in sorted(set(list(range(1, B * L + 1, max(1, B * L // 4000))) + [B * L])):
        rc, chunk, n = _plan(B, Hkv, L, hint=hint, total=total, Hq=Hq, D=D, dt=dt)
        assert rc == 0
        if prev is not None:
            assert chunk >= prev[0], (total, prev, chunk)
            if chunk == prev[0]:
                assert n == prev[1]
        prev = (chunk, n)


def test_memoised_plan_matches_the_query():
    import random

    import numpy as np
    import torch

    from simple_llm_amd.gpu import gpu_kv_cache as kvc
    from simple_llm_amd.gpu.gpu_types import GPUConfig, GPUContext, PipelineCache

    ctx = GPUContext(device=torch.device("cpu"), config=GPUConfig(), batch_state=None,
                     pipeline_cache=PipelineCache())
    rng = random.Random(0)
    for B, Hq, Hkv, D, dtype, L in [(8, 8, 8, 64, torch.float32, 2048),
                                    (64, 32, 8, 128, torch.bfloat16, 8320),
                                    (4, 16, 16, 128, torch.bfloat16, 32768)]:
        kvc._PLAN_SPANS.clear()
        # a decode loop (totals grow by B), then resets and random totals
        totals = [B + i * B for i in range(300)] + [rng.randrange(0, B * L + 1) for _ in range(300)]
        totals += list(np.linspace(0, B * L, 200).astype(int))
        for t in totals:
            want = kvc.decode_plan(ctx, B, Hq, Hkv, L, int(t), head_dim=D, dtype=dtype)
            got = kvc._decode_plan_span(ctx, B, Hq, Hkv, L, int(t), D, dtype)
            assert got == want, (B, Hq, Hkv, D, L, t, got, want)


def test_step_entry_points_reject_bad_arguments():
    """The decode step's fused entry points (LayerNorm-folded and packed
    projections, the skinny logits with candidates, argmax candidates + next
    token + embedding) fail validation before any device work."""
    L = _lib.lib()
    fake = 4096  # never dereferenced
    # packed logits: M <= 16, K in {512, 768, 1024}, 16384 <= N <= 65536
    for M, N, K in [(17, 50304, 768), (16, 1000, 768), (16, 50304, 640), (16, 70000, 768)]:
        assert L.skv_linear_packed(fake, fake, fake, None, None, M, N, K, 0, None, None) == \
            _lib.SKV_E_UNSUPPORTED, (M, N, K)
    assert L.skv_linear_packed(fake, fake, fake, None, None, 16, 50304, 768, 2, None, None) == \
        _lib.SKV_E_INVALID  # activation
    assert L.skv_linear_packed(None, fake, fake, None, None, 16, 50304, 768, 0, None, None) == \
        _lib.SKV_E_INVALID
    assert L.skv_linear_packed_cand_bytes(16) == 16 * 256 * 8
    # skinny logits with candidates: M <= 16, K a shape of the one-tile kernel
    for M, K in [(17, 256), (16, 100), (1, 4096)]:
        assert L.skv_linear_cand(fake, fake, fake, None, M, 256, K, fake, None, 0, None) == \
            _lib.SKV_E_UNSUPPORTED, (M, K)
        assert L.skv_linear_cand_bytes(M, 256, K) == 0
    assert L.skv_linear_cand(fake, fake, fake, None, 1, 256, 256, None, None, 0, None) == \
        _lib.SKV_E_INVALID  # candidates missing
    assert L.skv_linear_cand(fake, fake, fake, None, 1, 0, 256, fake, None, 0, None) == \
        _lib.SKV_E_INVALID
    assert L.skv_linear_cand_bytes(1, 256, 256) == 16 * 8
    assert L.skv_linear_cand_bytes(16, 300, 768) == 16 * 19 * 8
    # folded projections: up to 16 rows, K a shape of the one-tile kernel
    assert L.skv_linear_folded(fake, fake, fake, fake, fake, None, 1e-5, 17, 768, 768, 0, 0,
                               None) == _lib.SKV_E_UNSUPPORTED
    assert L.skv_linear_folded(fake, fake, fake, fake, fake, None, 1e-5, 16, 768, 100, 0, 0,
                               None) == _lib.SKV_E_UNSUPPORTED
    assert L.skv_linear_folded(fake, fake, fake, None, fake, None, 1e-5, 16, 768, 768, 0, 0,
                               None) == _lib.SKV_E_INVALID  # c1 missing
    assert L.skv_linear_folded(fake, fake, fake, fake, fake, None, 1e-5, 16, 768, 768, 0, 5,
                               None) == _lib.SKV_E_INVALID  # split_cols
    # next token + embedding

    def ne(**kw):
        a = dict(x=fake, argmax_prev=fake, cand=None, n_cand=0, B=4, emb=fake, d=64, vocab=100,
                 ctx=32, stop=None, lens_all=None, n_layers=0)
        a.update(kw)
        return L.skv_next_embed(a["x"], fake, fake, a["argmax_prev"], a["cand"], a["n_cand"],
                                fake, fake, fake, a["B"], 8, 64, a["emb"], fake, a["d"],
                                a["vocab"], a["ctx"], a["stop"], a["lens_all"], a["n_layers"],
                                a.get("adv"), None)

    assert ne(B=0) == _lib.SKV_E_INVALID
    assert ne(n_cand=-1) == _lib.SKV_E_INVALID
    assert ne(n_cand=256) == _lib.SKV_E_INVALID  # candidates missing
    assert b"candidates or the previous argmax" in L.skv_last_error()
    assert ne(argmax_prev=None) == _lib.SKV_E_INVALID
    assert ne(x=None) == _lib.SKV_E_INVALID  # an embedding needs x
    assert ne(d=0) == _lib.SKV_E_INVALID
    # retiring rows needs every layer's fills
    assert ne(stop=fake) == _lib.SKV_E_INVALID
    assert ne(stop=fake, lens_all=fake, n_layers=0) == _lib.SKV_E_INVALID
    assert b"retiring rows" in L.skv_last_error()
    assert L.skv_next_tokens(fake, fake, fake, fake, fake, fake, 4, 8, 64, fake, None, 2,
                             None, None) == _lib.SKV_E_INVALID
    assert ne(adv=fake) == _lib.SKV_E_INVALID  # a deferred advance needs every layer's fills
    # the direct decode attention: MHA, head_dim 64 or 128
    assert L.skv_append_decode_attn_direct(fake, fake, fake, fake, fake, fake, fake, 2, 4, 48,
                                           64, 0.1, 0, 0, 0, 0, 1, None, 0,
                                           None) == _lib.SKV_E_UNSUPPORTED
    assert L.skv_append_decode_attn_direct(fake, fake, fake, fake, None, fake, fake, 2, 4, 64,
                                           64, 0.1, 0, 0, 0, 0, 1, None, 0,
                                           None) == _lib.SKV_E_INVALID
    # split over the row: 1, 2 or 4 parts, the partials in a workspace
    need = L.skv_decode_direct_workspace_bytes(2, 4, 64, 2)
    assert need == 65536 * 4 + 2 * 4 * 2 * 66 * 4  # the fixed counter block, then partials
    assert L.skv_decode_direct_workspace_bytes(2, 4, 64, 1) == 0
    for ns, ws, wsb, rc_want in ((3, fake, need, _lib.SKV_E_INVALID),
                                 (2, None, need, _lib.SKV_E_WORKSPACE),
                                 (2, fake, need - 4, _lib.SKV_E_WORKSPACE)):
        rc = L.skv_append_decode_attn_direct(fake, fake, fake, fake, fake, fake, fake, 2, 4, 64,
                                             64, 0.1, 0, 0, 0, 0, ns, ws, wsb, None)
        assert rc == rc_want, ns
    # the cache rows are read as vectors: 16-byte (fp32) or 8-byte (bf16)
    # aligned caches only (rejected before any launch)
    for cdt, off in ((0, 8), (0, 4), (1, 4), (1, 2)):
        rc = L.skv_append_decode_attn_direct(fake, fake, fake + off, fake, fake, fake, fake, 2, 4,
                                             64, 64, 0.1, cdt, 0, 0, 0, 1, None, 0, None)
        assert rc == _lib.SKV_E_UNSUPPORTED, (cdt, off)
        assert b"aligned" in L.skv_last_error()
        rc = L.skv_append_decode_attn_direct(fake, fake, fake, fake + off, fake, fake, fake, 2, 4,
                                             128, 64, 0.1, cdt, 0, 0, 0, 1, None, 0, None)
        assert rc == _lib.SKV_E_UNSUPPORTED, (cdt, off)
