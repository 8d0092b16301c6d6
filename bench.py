"""Benchmark of the KV-cache decode hot path on one MI355X.

Workload ("C4"): long-context decode, batch 4,
16 heads x head_dim 128, cache capacity 32768 with bf16 storage and fp32
accumulation, filled to 32000 with N(0,1) K/V. One step = the append of one
new k/v row per sequence into the cache, then single-query attention of
every sequence over its filled prefix (QK^T, softmax, PV): the reference's
kv_cache_update + attention_with_kv_cache
(simple-llm/src/gpu/gpu_kv_cache.py:113-186, 194-289), run through this
build's kv_cache_append_attend, which computes exactly that pair in one call
(the new token is written and attended inside the attention's first pass). The timed steps go 32000 -> 32000+K filled positions
(the cache is rewound to 32000 after warm-up), exactly as the config states
for K = 256.

Output: one JSON line (rank 0) with
  value      decode tokens/s = B * K / wall time of the K timed steps
  roofline   the step's fused append + decode attention (split-K pass 1 +
             merge pass 2, bracketed by HIP events on the launch stream)
             against 8 TB/s HBM:
             achieved = algorithmic bytes per call / mean call time, where
             bytes = sum_b 2*H_kv*L_b*D*2 (K and V rows read) + H_q*D*(4+4)
             (q read, out written); traffic = HBM bytes per call measured by
             rocprofv3 FETCH_SIZE + WRITE_SIZE (profiles/), or null
  prefill    C4's one 512-token chunked prefill into the cache (MFMA path),
             timed separately with HIP events: TFLOP/s of its QK^T + PV flops
             against the 2.5 PFLOP/s dense bf16 peak
  cpu_baseline  the C restatement of the reference's decode attention
             (oracle/c/kv_attn_ref.c, OpenMP over (sequence, head)) plus the
             host append, timed on this box's cores over the first steps of
             the same workload (~10 s of CPU work)

Inputs (q, k, v of every step) are generated on the device before timing.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "llm-experiments_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0  # MI355X published HBM3E bandwidth
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 matrix peak
PREFILL_C = 512  # C4's chunked prefill: 512 tokens from fill 32256 to 32768
# Before the warm-up steps, the attention workloads run their own step,
# untimed, for this long (rewinding the cache between bursts): from idle, an
# MI355X's clock ramps over the first few milliseconds of load, and with
# --warmup 5 the first ~20 timed C4 calls ran at 170-176 us against ~152 us
# after the ramp (profiles/decode_attn_c4_per_step.md).
SETTLE_S = 0.25

# C4 workload
B, H, D, T_CAP, FILL = 4, 16, 128, 32768, 32000


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--workload", choices=["c4", "c1", "c2", "c3", "c5", "fb", "sample"],
                   default="c4",
                   help="BASELINE config: c4 (default, the headline line), c1 tiny LM "
                        "generate, c2 fp32 KV microbench, c3 GPT-2-small ragged batch, "
                        "c5 GQA paged ragged decode; fb: flash-attention backward (fp32); "
                        "sample: next-token sampling at the C3 shape")
    p.add_argument("--steps", type=int, default=256)
    p.add_argument("--warmup", type=int, default=16)
    p.add_argument("--cpu-seconds", type=float, default=10.0,
                   help="CPU time budget of the cpu_baseline sample")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-prefill", action="store_true",
                   help="skip the separate timing of C4's 512-token MFMA chunked prefill")
    p.add_argument("--chunk-tokens", type=int, default=0,
                   help="split-K chunk size of decode attention (0: the library's plan)")
    p.add_argument("--copy-calibration", action="store_true",
                   help="instead of the benchmark, time a plain 1 GiB device copy (the "
                        "reference kernel for the HBM counters and the measured copy GB/s)")
    return p.parse_args()


def copy_calibration():
    """A plain device-to-device copy of 1 GiB, 10 times: its FETCH_SIZE and
    WRITE_SIZE per dispatch calibrate the counters (1 GiB each way), and its
    rate is the measured copy bandwidth (bytes read + bytes written)."""
    import torch

    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(10):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    s = e0.elapsed_time(e1) * 1e-3 / 10
    print(json.dumps({"copy_bytes_each_way": n, "mean_copy_us": s * 1e6,
                      "copy_GBps_read_plus_write": 2 * n / s / 1e9}), flush=True)


def algorithmic_bytes(lens, h_q=H, h_kv=H, d=D, s_kv=2, s_q=4, s_o=4) -> int:
    """Bytes one decode-attention call must move at minimum."""
    return int(sum(2 * h_kv * int(L) * d * s_kv + h_q * d * (s_q + s_o) for L in lens))


def rel_err_rows(got, want) -> float:
    """max over rows (all axes but the last) of ||got - want|| / ||want||."""
    import numpy as np

    got = np.asarray(got, np.float64).reshape(-1, np.shape(got)[-1])
    want = np.asarray(want, np.float64).reshape(-1, np.shape(want)[-1])
    num = np.linalg.norm(got - want, axis=1)
    den = np.maximum(np.linalg.norm(want, axis=1), 1e-30)
    live = np.linalg.norm(want, axis=1) > 0
    if not live.any():
        return 0.0
    return float((num / den)[live].max())


def replay_outputs(step, n, reset, out):
    """The outputs of steps 0..n-1 of an attention workload, run again from
    its start fills (reset()) after the timed region: the kernels are
    deterministic and the plan is the timed run's, so these are the timed
    steps' outputs bit for bit (the appends rewrite the same rows)."""
    import torch

    reset()
    outs = []
    for i in range(n):
        step(i)
        outs.append(out.detach().clone())
    torch.cuda.synchronize()
    return [o.cpu().numpy() for o in outs]


def accuracy_record(gpu_outs, oracle_outs, tol, against):
    errs = [rel_err_rows(g, w) for g, w in zip(gpu_outs, oracle_outs)]
    worst = max(errs) if errs else None
    return {"max_rel_err": worst, "tolerance": tol, "steps_checked": len(errs),
            "pass": worst is not None and worst <= tol, "against": against,
            "norm": "per (sequence, head) row: ||gpu - oracle||_2 / ||oracle||_2, max over rows "
                    "and steps"}


def sclk_sampler():
    """A thread that samples the GPU's current shader clock (the level marked
    '*' in sysfs pp_dpm_sclk of the card torch runs on) every 2 ms until
    stopped; returns (start, stop) where stop() gives the MHz samples. Empty
    when the file is not readable."""
    import glob
    import threading

    paths = sorted(glob.glob("/sys/class/drm/card*/device/pp_dpm_sclk"))
    samples, done = [], threading.Event()
    path = None
    for pth in paths:  # the first card whose file is readable (one GPU per box)
        try:
            with open(pth) as f:
                f.read()
            path = pth
            break
        except OSError:
            continue

    def read():
        try:
            with open(path) as f:
                for line in f:
                    if "*" in line:
                        m = re.search(r"(\d+)\s*[Mm]hz", line)
                        if m:
                            return int(m.group(1))
        except OSError:
            return None
        return None

    def loop():
        while not done.is_set():
            v = read()
            if v is not None:
                samples.append(v)
            time.sleep(0.002)

    th = threading.Thread(target=loop, daemon=True)

    def start():
        if path is not None:
            th.start()

    def stop():
        done.set()
        if path is not None:
            th.join()
        return samples

    return start, stop, path


def measured_traffic(workload: str = "c4"):
    """HBM bytes per decode-attention call from the committed rocprofv3 PMC
    summary of the workload (profiles/decode_attn_<workload>_pmc.md), or None
    if absent."""
    path = os.path.join(ROOT, "profiles", f"decode_attn_{workload}_pmc.md")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        m = re.search(r"^traffic_bytes_per_call:\s*([0-9.eE+]+)", f.read(), flags=re.M)
    return float(m.group(1)) if m else None


def prefill_flops(start, c=PREFILL_C, h_q=H, d=D, batch=B) -> float:
    """QK^T and PV flops of a causal chunk after a prefix of `start` tokens."""
    attended = c * start + c * (c + 1) // 2  # sum over the chunk's queries of their spans
    return 4.0 * d * h_q * batch * attended


def time_prefill(ctx, cache, reps: int):
    """C4's 512-token chunked prefill (chunk append + MFMA causal attention over
    prefix + chunk + fill advance), rewound to fill 32256 before each rep.
    The same call runs back to back for SETTLE_S first: the matrix-core load
    moves the shader clock (power management) for a few milliseconds after
    the decode steps, and the timed reps then see the clock the call runs at
    in steady state."""
    import numpy as np
    import torch

    from simple_llm_amd.gpu import gpu

    dev = ctx.device
    start = T_CAP - PREFILL_C
    g = torch.Generator(device=dev).manual_seed(1)
    kn = torch.randn((B, PREFILL_C, H, D), generator=g, device=dev)
    vn = torch.randn((B, PREFILL_C, H, D), generator=g, device=dev)
    q = torch.randn((B, PREFILL_C, H, D), generator=g, device=dev)
    out = torch.empty_like(q)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(reps)]

    def rewind():
        cache.current_len = start

    settle_s = settle(lambda: [(rewind(), gpu.kv_cache_prefill(ctx, cache, 0, kn, vn, q, out))
                               for _ in range(4)], rewind)
    for i in range(reps + 2):
        cache.current_len = start
        if i >= 2:
            evs[i - 2][0].record()
        gpu.kv_cache_prefill(ctx, cache, 0, kn, vn, q, out)
        if i >= 2:
            evs[i - 2][1].record()
    torch.cuda.synchronize()
    ms = np.array([a.elapsed_time(b) for a, b in evs])
    fl = prefill_flops(start)
    mean_s = float(ms.mean()) * 1e-3
    # the shader clock while the same call runs back to back for ~0.3 s (sysfs
    # pp_dpm_sclk, sampled by a host thread): the box's clock under this load
    start_clk, stop_clk, clk_path = sclk_sampler()
    n_clk = max(int(0.3 / max(mean_s, 1e-5)), 1)
    start_clk()
    t0 = time.perf_counter()
    for _ in range(n_clk):
        cache.current_len = start
        gpu.kv_cache_prefill(ctx, cache, 0, kn, vn, q, out)
    torch.cuda.synchronize()
    burst_us = (time.perf_counter() - t0) / n_clk * 1e6
    mhz = stop_clk()
    # accuracy of the last call: sampled query rows against the float64
    # oracle over the device cache's own bf16 values (prefix + chunk)
    from oracle import kv_oracle as ko

    got = out.cpu().numpy()
    qh = q.cpu().numpy()
    kvw = cache.layers[0].k_cache.buffer.view(B, T_CAP, H, D)
    vvw = cache.layers[0].v_cache.buffer.view(B, T_CAP, H, D)
    errs = []
    for b, i, h in ((0, 0, 0), (1, 255, 7), (2, 511, 15), (3, 100, 3)):
        n = start + i + 1
        kh = kvw[b, :n, h].float().cpu().numpy()[None, :, None, :]
        vh = vvw[b, :n, h].float().cpu().numpy()[None, :, None, :]
        want = ko.decode_attention(qh[b:b + 1, i, h:h + 1], kh, vh, [n])
        errs.append(rel_err_rows(got[b, i, h][None], want[0]))
    return {
        "chunk_tokens": PREFILL_C, "start_fill": start, "reps": reps,
        "mean_us": mean_s * 1e6, "tflops": fl / mean_s / 1e12,
        "peak_tflops": MFMA_BF16_PEAK_TFLOPS,
        "frac": fl / mean_s / 1e12 / MFMA_BF16_PEAK_TFLOPS,
        "flops": fl,
        "per_rep_us": [round(float(x) * 1e3, 1) for x in ms],
        "median_us": float(np.median(ms)) * 1e3, "min_us": float(ms.min()) * 1e3,
        "settle_s": round(settle_s, 3),
        "clock": {"source": clk_path, "back_to_back_calls": n_clk,
                  "wall_us_per_call": burst_us, "samples": len(mhz),
                  "sclk_mhz_median": float(np.median(mhz)) if mhz else None,
                  "sclk_mhz_min": min(mhz) if mhz else None,
                  "sclk_mhz_max": max(mhz) if mhz else None},
        "accuracy": {"max_rel_err": max(errs), "tolerance": 2e-2, "rows_checked": len(errs),
                     "pass": max(errs) <= 2e-2,
                     "against": "float64 oracle (kv_oracle) over the cache's bf16 values, "
                                "sampled (sequence, query row, head) of the last call"},
        "includes": "chunk append + MFMA attention + split merge + fill advance",
    }


def cpu_baseline(args, k_dev, v_dev, q_all, k_all, v_all, outs=None):
    """Time the CPU restatement on the first steps of the same workload;
    the oracle's output of each step goes to outs (a list) when given."""
    import numpy as np
    import torch

    from oracle import c_oracle

    # the same cache contents, as bf16 bit patterns on the host
    kc = k_dev.view(torch.int16).cpu().numpy().view(np.uint16).reshape(B, T_CAP, H, D).copy()
    vc = v_dev.view(torch.int16).cpu().numpy().view(np.uint16).reshape(B, T_CAP, H, D).copy()
    qs = q_all.cpu().numpy()
    ks = k_all.to(torch.bfloat16).view(torch.int16).cpu().numpy().view(np.uint16)
    vs = v_all.to(torch.bfloat16).view(torch.int16).cpu().numpy().view(np.uint16)
    lens = np.full(B, FILL, np.int32)
    c_oracle.decode_attn(qs[0], kc, vc, lens + 1, cache_bf16=True)  # warm-up (pages, threads)
    steps = 0
    t0 = time.perf_counter()
    while steps < args.steps and (time.perf_counter() - t0) < args.cpu_seconds:
        for b in range(B):  # host append at lens[b]
            kc[b, lens[b]] = ks[steps, b]
            vc[b, lens[b]] = vs[steps, b]
        lens += 1
        o = c_oracle.decode_attn(qs[steps], kc, vc, lens, cache_bf16=True)
        if outs is not None:
            outs.append(o)
        steps += 1
    dt = time.perf_counter() - t0
    return {
        "value": B * steps / dt,
        "unit": "tokens/s",
        "cores": c_oracle.threads(),
        "kind": "port",
        "sample": f"first {steps} of the {args.steps} C4 decode steps (append + decode attention "
                  f"over 32001.. positions, B={B} H={H} D={D} bf16 KV, fp32 math); "
                  f"oracle/c/kv_attn_ref.c with OpenMP, {dt:.1f} s",
    }


def cpu_model() -> str:
    """The host CPU's model name (lscpu's "Model name", from /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.lower().startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _with_cpu_model(cpu):
    if cpu is not None:
        cpu = dict(cpu)
        cpu.setdefault("cpu_model", cpu_model())
    return cpu


def settle(run_burst, reset) -> float:
    """Run run_burst() (a few of the workload's own steps) untimed, calling
    reset() before each burst and once after, for SETTLE_S seconds; returns the
    seconds spent."""
    import torch

    t0 = time.perf_counter()
    while time.perf_counter() - t0 < SETTLE_S:
        reset()
        run_burst()
        torch.cuda.synchronize()
    reset()
    torch.cuda.synchronize()
    return time.perf_counter() - t0


def _record(metric, value, unit, steps, warmup, ms_per_step, dtype, config, roofline, cpu,
            **extra):
    cpu = _with_cpu_model(cpu)
    for k in list(extra):
        if k.startswith("cpu") and isinstance(extra[k], dict):
            extra[k] = _with_cpu_model(extra[k])
    rec = {"metric": metric, "value": value, "unit": unit, "n_gpus": 1, "steps": steps,
           "warmup": warmup, "ms_per_step": ms_per_step, "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": dtype, "data": "synthetic",
           "config": config, "roofline": roofline, "cpu_baseline": cpu}
    rec.update(extra)
    return rec


def _time_cached_cpu(params, n_heads, batch, t_cap, budget_s):
    """The same cached algorithm as the GPU path on the CPU (torch fp32,
    oracle/model_oracle.TorchCachedDecoder): steps of `batch` sequences from
    an empty cache until the budget is spent (at most t_cap steps)."""
    import numpy as np
    import torch

    from oracle import model_oracle as mo

    with torch.no_grad():
        dec = mo.TorchCachedDecoder(params, n_heads, batch, t_cap)
        vocab = int(np.asarray(params["embedding"]).shape[0])
        toks = np.random.default_rng(0).integers(0, vocab, (t_cap, batch))
        dec.step(toks[0])  # warm-up
        n, t0 = 0, time.perf_counter()
        while n + 1 < t_cap and time.perf_counter() - t0 < budget_s:
            dec.step(toks[n + 1])
            n += 1
        dt = time.perf_counter() - t0
    return n, dt


def _time_reference_generate(params, prompt, n_heads, context, budget_s, max_tokens):
    """The reference's generate loop (generate.py:29-69, greedy): a full
    float32 torch CPU forward over the left-padded window per token."""
    import torch

    from oracle import model_oracle as mo

    fwd = lambda p, ids: mo.torch_forward_fp32(p, ids, n_heads).numpy()  # noqa: E731
    with torch.no_grad():
        mo.reference_generate(params, prompt, 1, n_heads, context, forward_fn=fwd)  # warm-up
        n, t0 = 0, time.perf_counter()
        while n < max_tokens and time.perf_counter() - t0 < budget_s:
            mo.reference_generate(params, prompt + [0] * n, 1, n_heads, context, forward_fn=fwd)
            n += 1
        dt = time.perf_counter() - t0
    return n, dt


def _model_workload(args, ctx, tm, prompts, total_len, label, kv_dtypes, acc_rows, acc_last):
    """Greedy generation of `prompts` to `total_len` tokens: one prefill of
    every prompt, then the decode steps with HIP-graph replay; per KV dtype,
    the mean of 3 timed runs after a warm-up run, and the prefill alone over
    3 more runs; then the logits of the last acc_last decode steps of rows
    acc_rows against the float64 oracle."""
    import numpy as np
    import torch

    from simple_llm_amd import model as M

    params = M.initialize_params(tm, seed=0, std=0.02)
    model = M.TransformerModel(ctx, tm, params)
    runs = {}
    for kvd in kv_dtypes:
        model.kv_dtype = kvd
        g = M.Generator(model, prompts, total_len, use_graph=True)
        out = g.run()  # warm-up: eager first step, graph capture, replays
        times = []
        for _ in range(3):
            g.reset()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            out2 = g.run()
            torch.cuda.synchronize()
            times.append(time.perf_counter() - t0)
        assert out2 == out, "graph replays must reproduce the first run"
        pre = []
        for _ in range(3):
            g.reset()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            g.prefill()
            torch.cuda.synchronize()
            pre.append(time.perf_counter() - t0)
        gen = sum(total_len - len(p) for p in prompts)
        run_s, pre_s = float(np.mean(times)), float(np.mean(pre))
        acc, again = _model_accuracy(g, params, tm.n_heads, acc_rows, acc_last,
                                     1e-4 if kvd == torch.float32 else 2e-2)
        assert again == out  # the accuracy run made the timed run's tokens
        runs[str(kvd).replace("torch.", "")] = {
            "run_s": run_s, "prefill_s": pre_s, "prompt_tokens": int(sum(len(p) for p in prompts)),
            "steps": g.steps, "generated_tokens": gen, "tokens_per_s": gen / run_s,
            "step_us": (run_s - pre_s) / max(g.steps, 1) * 1e6,
            "direct_attention": bool(g.direct), "accuracy": acc}
    d, L, V = tm.embedding_dim, tm.n_layers, tm.vocab_size
    weight_bytes = 4 * (V * d + L * (4 * d * d + 2 * d * model.mlp_dim + model.mlp_dim + 7 * d))
    return params, model, runs, weight_bytes


def _model_accuracy(g, params, n_heads, rows, last_k, tol):
    """Same-run accuracy of a greedy generate workload: the logits of the last
    last_k decode steps of each row in `rows`, from one more run of the timed
    Generator (deterministic kernels: the timed run's values), against the
    float64 forward of oracle/model_oracle.py over the tokens that run made
    (teacher forced)."""
    import numpy as np

    from oracle import model_oracle as mo

    plen, tot = g.plen.astype(np.int64), g.tot.astype(np.int64)
    want = {}  # decode step -> rows whose logits that step are checked
    for b in rows:
        last = int(tot[b]) - 2  # position of the row's last decode step
        for p in range(max(last - last_k + 1, int(plen[b])), last + 1):
            want.setdefault(p - int(plen[b]), []).append(b)
    got = {}

    def on_step(j, logits):
        for b in want.get(j, ()):
            got[(b, j)] = logits[b].detach().clone()

    g.reset()
    seqs = g.run(on_step=on_step)
    errs = []
    for b in rows:
        last = int(tot[b]) - 2
        first = max(last - last_k + 1, int(plen[b]))
        ref = mo.forward(params, np.array([seqs[b][:last + 1]]), n_heads,
                         last=last - first + 1)[0]
        gl = np.stack([got[(b, p - int(plen[b]))].cpu().numpy() for p in range(first, last + 1)])
        num = np.linalg.norm(gl - ref, axis=1)
        errs.append(float((num / np.linalg.norm(ref, axis=1)).max()))
    worst = max(errs)
    return {"max_rel_err": worst, "tolerance": tol, "pass": worst <= tol,
            "rows_checked": [int(b) for b in rows], "positions_per_row": last_k,
            "against": "float64 forward (oracle/model_oracle.py) over the tokens the timed "
                       "run generated (teacher forced), the logits of each checked row's last "
                       "decode steps",
            "norm": "per logits row: ||gpu - oracle||_2 / ||oracle||_2, max over rows"}, seqs


def run_c1(args, ctx):
    """tiny LM (4 layers, d 256, 4 x 64, MLP 1024, vocab
    256, context 256, fp32, N(0, 0.02) weights from seed 0), 64-token prompt
    drawn from seed 1, greedy decode of 192 tokens, batch 1."""
    import numpy as np
    import torch

    from simple_llm_amd import model as M

    tm = M.TransformerModelParams(256, 256, 256, 4, 4)
    prompt = np.random.default_rng(1).integers(0, 256, 64).tolist()
    params, model, runs, wbytes = _model_workload(args, ctx, tm, [prompt], 256, "c1",
                                                  [torch.float32], [0], 191)
    r = runs["float32"]
    cpu = cpu_cached = None
    if not args.no_cpu_baseline:
        n, dt = _time_reference_generate(params, prompt, 4, 256, args.cpu_seconds, 192)
        cpu = {"value": n / dt, "unit": "tokens/s", "cores": torch.get_num_threads(),
               "kind": "port",
               "sample": f"{n} greedy tokens of the reference's generate loop (full float32 "
                         f"forward over the 256-token left-padded window per token, torch CPU), "
                         f"{dt:.1f} s"}
        n2, dt2 = _time_cached_cpu(params, 4, 1, 256, args.cpu_seconds)
        cpu_cached = {"value": n2 / dt2, "unit": "tokens/s", "cores": torch.get_num_threads(),
                      "kind": "port",
                      "sample": f"{n2} steps of the cached recurrence (torch CPU fp32, batch 1, "
                                f"positions 1..{n2}), {dt2:.1f} s"}
    return _record(
        "decode tokens/sec", r["tokens_per_s"], "tokens/s", r["steps"], 1, r["step_us"] / 1e3,
        "fp32",
        {"workload": "C1 tiny LM: 4 layers, d 256, 4 heads x 64, MLP 1024, vocab 256, context "
                     "256, fp32 weights and KV, 64-token prompt + 192 greedy tokens, batch 1; "
                     "the prompt prefilled in one multi-token pass (its logits give the first "
                     "token), then 191 cached decode steps replayed from one HIP graph; value "
                     "= generated tokens / whole run (prefill included)",
         "batch": 1, "prompt": 64, "generated": 192},
        {"bound": "launch latency", "note": "12.8 MB of weights per token; 22 kernels per "
                                            "step replayed from one HIP graph",
         "achieved": wbytes / (r["step_us"] * 1e-6) / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s",
         "frac": wbytes / (r["step_us"] * 1e-6) / 1e9 / HBM_PEAK_GBS, "traffic": None},
        cpu, max_rel_err=r["accuracy"]["max_rel_err"], accuracy=r["accuracy"], runs=runs,
        cpu_cached_baseline=cpu_cached)


def run_c3(args, ctx):
    """GPT-2-small shape (12 layers, d 768, 12 x 64,
    vocab 50304, context 1024), batch 16, prompt lengths U[32, 512] (ragged),
    greedy decode to 1024 tokens each; KV in fp32 and in bf16."""
    import numpy as np
    import torch

    from simple_llm_amd import model as M

    tm = M.TransformerModelParams(50304, 768, 1024, 12, 12)
    r = np.random.default_rng(1)
    plen = r.integers(32, 513, 16)
    prompts = [r.integers(0, 50304, int(n)).tolist() for n in plen]
    params, model, runs, wbytes = _model_workload(args, ctx, tm, prompts, 1024, "c3",
                                                  [torch.float32, torch.bfloat16], [0, 9], 16)
    # per step: all weights + the K and V prefixes the step reads, averaged over the run's
    # steps. Decode step s reads sequence b's fill plen_b + s plus its new token while
    # plen_b + s < 1023; from the step that records its last token (position 1023) on, the
    # sequence is retired and reads nothing.
    fill = plen[None, :] + np.arange(runs["float32"]["steps"])[:, None]
    mean_tokens = float(np.where(fill < 1023, fill + 1, 0).sum(axis=1).mean())
    kv = {"float32": 4, "bfloat16": 2}
    roof = {}
    for k, run in runs.items():
        by = wbytes + 12 * 2 * mean_tokens * 768 * kv[k]
        roof[k] = by / (run["step_us"] * 1e-6) / 1e9
    cpu = cpu_cached = None
    if not args.no_cpu_baseline:
        n, dt = _time_reference_generate(params, prompts[0], 12, 1024, args.cpu_seconds, 4)
        cpu = {"value": n / dt, "unit": "tokens/s", "cores": torch.get_num_threads(),
               "kind": "port",
               "sample": f"{n} greedy tokens of one sequence through the reference's generate "
                         f"loop (full float32 forward over the 1024-token window per token, "
                         f"~292 GFLOP each, torch CPU), {dt:.1f} s; the reference runs batch 1"}
        n2, dt2 = _time_cached_cpu(params, 12, 16, 1024, args.cpu_seconds)
        cpu_cached = {"value": 16 * n2 / dt2, "unit": "tokens/s",
                      "cores": torch.get_num_threads(), "kind": "port",
                      "sample": f"{n2} steps of the cached recurrence for 16 sequences (torch "
                                f"CPU fp32, fp32 KV, positions 1..{n2}), {dt2:.1f} s"}
    r32 = runs["float32"]
    return _record(
        "decode tokens/sec", r32["tokens_per_s"], "tokens/s", r32["steps"], 1,
        r32["step_us"] / 1e3, "fp32",
        {"workload": "C3 GPT-2-small shape: 12 layers, d 768, 12 heads x 64, vocab 50304, "
                     "context 1024, batch 16, prompts U[32,512], greedy to 1024 tokens, fp32 "
                     "weights; the prompts prefilled in one ragged multi-token pass, then the "
                     "cached decode steps (HIP graph); value = generated tokens / whole run "
                     "(prefill included) with the fp32 KV cache (bf16 KV in runs)",
         "batch": 16, "prompt_lens": plen.tolist()},
        {"bound": "hbm", "achieved": roof["float32"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
         "frac": roof["float32"] / HBM_PEAK_GBS, "traffic": None,
         "note": "per step: all weights + the K/V prefixes of the sequences not yet "
                 "finished (mean over the run's steps), over step time",
         "mean_kv_tokens_per_step": mean_tokens,
         "achieved_bf16_kv": roof["bfloat16"]},
        cpu, max_rel_err=r32["accuracy"]["max_rel_err"], accuracy=r32["accuracy"], runs=runs,
        cpu_cached_baseline=cpu_cached)


def _attention_workload(args, ctx, cache, lens0, steps, Hq, Hkv, Dh, s_kv, q_dt, label):
    """Timed loop of append + decode attention on one prepared cache layer."""
    import numpy as np
    import torch

    from simple_llm_amd.gpu import gpu

    dev = ctx.device
    B = cache.batch_size
    g = torch.Generator(device=dev).manual_seed(2)
    n_in = args.warmup + steps
    q_all = torch.randn((n_in, B, Hq, Dh), generator=g, device=dev)
    k_all = torch.randn((n_in, B, Hkv, Dh), generator=g, device=dev)
    v_all = torch.randn((n_in, B, Hkv, Dh), generator=g, device=dev)
    out = torch.empty((B, Hq, Dh), device=dev)
    cap = (cache.block_table.shape[1] * cache.block_size) if cache.paged else cache.max_seq_len
    max_len = int(min(lens0.max() + steps, cap))
    layer = cache.layers[0]

    def set_lens(v):
        layer.lens.copy_(torch.from_numpy(v.astype(np.int32)))
        layer.host_lens = v.astype(np.int64).copy()

    # per-step views made once, outside the timed loop (indexing a tensor costs ~1 us of
    # host time, and each call is ~13 us of it)
    qs, ks, vs = q_all.unbind(0), k_all.unbind(0), v_all.unbind(0)

    def step(i):
        gpu.kv_cache_append_attend(ctx, cache, 0, ks[i], vs[i], qs[i], out, max_len=max_len)

    roofline_settle = settle(lambda: [step(i) for i in range(min(steps, 32))],
                             lambda: set_lens(lens0))
    for i in range(args.warmup):
        step(steps + i)
    torch.cuda.synchronize()
    set_lens(lens0)
    # one HIP event pair around the timed region, on the launch stream
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record()
    for i in range(steps):
        step(i)
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # fills at each call: lens after the append (full sequences stay put)
    fills, active = [], 0
    cur = lens0.astype(np.int64).copy()
    for _ in range(steps):
        act = cur < cap
        active += int(act.sum())
        cur = np.where(act, cur + 1, cur)
        fills.append(cur.copy())
    byts = float(np.mean([algorithmic_bytes(f, h_q=Hq, h_kv=Hkv, d=Dh, s_kv=s_kv, s_q=4, s_o=4)
                          for f in fills]))
    mean_s = ev0.elapsed_time(ev1) * 1e-3 / steps
    chunk, n_chunks = gpu.decode_plan(ctx, B, Hq, Hkv, max_len, int(lens0.sum()),
                                      head_dim=cache.head_dim, dtype=cache.dtype)
    # grouped queries over a bf16 cache with head_dim 64/128 run the matrix-core pass 1
    pass1 = ("k_decode_gqa" if Hq > Hkv and Hq // Hkv in (2, 4, 8) and s_kv == 2
             and Dh in (64, 128) else "k_decode_partial")
    roof = {"kernel": f"append + decode attention ({pass1} + k_decode_merge)", "bound": "hbm",
            "achieved": byts / mean_s / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": byts / mean_s / 1e9 / HBM_PEAK_GBS, "traffic": measured_traffic(label),
            "mean_call_us": mean_s * 1e6, "algorithmic_bytes_per_call": byts,
            "split_k": {"chunk_tokens": chunk, "n_chunks": n_chunks},
            "warmup_settle_s": round(roofline_settle, 3)}

    def replay(n):
        return replay_outputs(step, n, lambda: set_lens(lens0), out)

    return wall, active, roof, (q_all, k_all, v_all), replay


def run_c5(args, ctx):
    """64 sequences, 32 query heads over 8 kv heads,
    head_dim 128, bf16, lognormal lengths (median 1500, sigma 0.8, clipped to
    [16, 8192]), 16-token pages with a seeded random page table, 128 steps of
    append + decode attention."""
    import numpy as np
    import torch

    from simple_llm_amd.gpu import gpu

    B, Hq, Hkv, Dh, bs, steps = 64, 32, 8, 128, 16, 128
    r = np.random.default_rng(0)
    lens0 = np.clip(np.exp(r.normal(np.log(1500), 0.8, B)), 16, 8192).astype(np.int64)
    max_seq = 8192 + steps
    max_blocks = -(-max_seq // bs)
    need = -(-(lens0 + steps) // bs)
    n_blocks = int(need.sum())
    cache = gpu.kv_cache_create(ctx, gpu.KVCacheConfig(B, max_seq, 1, Hq, Dh, n_kv_heads=Hkv,
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
    g = torch.Generator(device=ctx.device).manual_seed(0)
    for buf in (layer.k_cache.buffer, layer.v_cache.buffer):
        for i in range(0, buf.shape[0], 1 << 16):
            chunk = buf[i:i + (1 << 16)]
            chunk.copy_(torch.randn(chunk.shape, generator=g, device=ctx.device))
    wall, active, roof, (q_all, k_all, v_all), replay = _attention_workload(
        args, ctx, cache, lens0, steps, Hq, Hkv, Dh, 2, 0, "c5")
    cpu = None
    oracle_outs = []
    if True:  # the CPU leg: timed unless --no-cpu-baseline; its outputs check the GPU's
        from oracle import c_oracle

        # the pool gathered into a contiguous [B, T, H_kv, D] cache on the host (the
        # reference's layout; pages are this build's extension), as bf16 bit patterns
        nb = int(need.max())
        tab = torch.from_numpy(table[:, :nb].astype(np.int64)).to(ctx.device)

        def gather(buf):
            g_ = buf.view(n_blocks, bs, Hkv, Dh)[tab].reshape(B, nb * bs, Hkv, Dh)
            return g_.view(torch.int16).cpu().numpy().view(np.uint16).copy()

        kc, vc = gather(layer.k_cache.buffer), gather(layer.v_cache.buffer)
        qs = q_all.cpu().numpy()
        ks = k_all.to(torch.bfloat16).view(torch.int16).cpu().numpy().view(np.uint16)
        vs = v_all.to(torch.bfloat16).view(torch.int16).cpu().numpy().view(np.uint16)
        lens = lens0.astype(np.int32).copy()
        c_oracle.decode_attn(qs[0], kc, vc, lens, cache_bf16=True)  # warm-up (pages, threads)
        n, tok, t0 = 0, 0, time.perf_counter()
        n_max = 2 if args.no_cpu_baseline else steps
        while n < n_max and (n == 0 or time.perf_counter() - t0 < args.cpu_seconds):
            for b in range(B):  # host append at lens[b]
                kc[b, lens[b]], vc[b, lens[b]] = ks[n, b], vs[n, b]
            lens += 1
            tok += B
            oracle_outs.append(c_oracle.decode_attn(qs[n], kc, vc, lens, cache_bf16=True))
            n += 1
        dt = time.perf_counter() - t0
        if not args.no_cpu_baseline:
            cpu = {"value": tok / dt, "unit": "tokens/s", "cores": c_oracle.threads(),
                   "kind": "port",
                   "sample": f"first {n} of the {steps} C5 steps (append + GQA decode attention "
                             f"over the pool gathered into a contiguous bf16 cache), "
                             f"oracle/c/kv_attn_ref.c with OpenMP, {dt:.1f} s"}
    accuracy = accuracy_record(replay(len(oracle_outs)), oracle_outs, 2e-2,
                               "oracle/c/kv_attn_ref.c on the pool gathered into a contiguous "
                               "cache (the same bf16 values, fp32 math), the first steps of the "
                               "timed run")
    return _record(
        "decode tokens/sec", active / wall, "tokens/s", steps, args.warmup, wall / steps * 1e3,
        "bf16",
        {"workload": "C5 batched ragged GQA decode: 64 seqs, 32 q heads over 8 kv heads, "
                     "head_dim 128, bf16 paged cache (16-token pages, random page table), "
                     "lognormal lengths median 1500 sigma 0.8 in [16, 8192], 128 steps of "
                     "append + decode attention",
         "batch": B, "mean_len": float(lens0.mean()), "pages": n_blocks},
        roof, cpu, max_rel_err=accuracy["max_rel_err"], accuracy=accuracy)


def run_c2(args, ctx):
    """fp32 cache [B=8, H=8, T=2048, D=64], start lengths
    U[1, 2047], 256 steps of append at pos_b + attention over [0, pos_b];
    sequences that reach 2048 retire (no append, not counted)."""
    import numpy as np
    import torch

    from simple_llm_amd.gpu import gpu

    B, H, T, Dh, steps = 8, 8, 2048, 64, 256
    lens0 = np.random.default_rng(0).integers(1, 2048, B).astype(np.int64)
    cache = gpu.kv_cache_create(ctx, gpu.KVCacheConfig(B, T, 1, H, Dh))
    layer = cache.layers[0]
    g = torch.Generator(device=ctx.device).manual_seed(0)
    layer.k_cache.buffer.copy_(torch.randn(layer.k_cache.buffer.shape, generator=g,
                                           device=ctx.device))
    layer.v_cache.buffer.copy_(torch.randn(layer.v_cache.buffer.shape, generator=g,
                                           device=ctx.device))
    wall, active, roof, (q_all, k_all, v_all), replay = _attention_workload(
        args, ctx, cache, lens0, steps, H, H, Dh, 4, 0, "c2")
    roof["note"] = "the 67 MB cache fits in the 256 MB Infinity Cache: not an HBM figure"
    cpu = None
    oracle_outs = []
    if True:  # the CPU leg: timed unless --no-cpu-baseline; its first pass checks the GPU
        from oracle import c_oracle

        kc = layer.k_cache.buffer.cpu().numpy().reshape(B, T, H, Dh).copy()
        vc = layer.v_cache.buffer.cpu().numpy().reshape(B, T, H, Dh).copy()
        qs, ks, vs = q_all.cpu().numpy(), k_all.cpu().numpy(), v_all.cpu().numpy()
        # whole passes over the 256 steps (each restarts from the start lengths and
        # re-appends the same rows) until the time budget is spent
        passes, tok, t0 = 0, 0, time.perf_counter()
        while passes == 0 or (not args.no_cpu_baseline
                              and time.perf_counter() - t0 < args.cpu_seconds):
            lens = lens0.astype(np.int32).copy()
            for n in range(steps):
                for b in range(B):
                    if lens[b] < T:
                        kc[b, lens[b]], vc[b, lens[b]] = ks[n, b], vs[n, b]
                        lens[b] += 1
                        tok += 1
                o = c_oracle.decode_attn(qs[n], kc, vc, lens, cache_bf16=False)
                if passes == 0:
                    oracle_outs.append(o)
            passes += 1
        dt = time.perf_counter() - t0
        if not args.no_cpu_baseline:
            cpu = {"value": tok / dt, "unit": "tokens/s", "cores": c_oracle.threads(),
                   "kind": "port", "sample": f"{passes} passes over the {steps} C2 steps, "
                                             f"oracle/c/kv_attn_ref.c with OpenMP, {dt:.1f} s"}
    accuracy = accuracy_record(replay(len(oracle_outs)), oracle_outs, 1e-4,
                               "oracle/c/kv_attn_ref.c on the same fp32 cache, every step of "
                               "the timed run")
    return _record(
        "decode tokens/sec", active / wall, "tokens/s", steps, args.warmup, wall / steps * 1e3,
        "fp32",
        {"workload": "C2 KV microbench fp32: cache [8, 8, 2048, 64], start lengths U[1,2047], "
                     "256 steps of append + attention, full sequences retire", "batch": B},
        roof, cpu, max_rel_err=accuracy["max_rel_err"], accuracy=accuracy)


MFMA_FP32_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix peak


def run_fb(args, ctx):
    """Training-side attention: one causal FlashAttention backward (skv_flash_bwd,
    fp32) per step at B=8, N=2048, H=16, D=64, the attention shape of the
    reference's largest power-of-two head_dim anchor (hyper.py:74: d_model 1024,
    16 heads, context 2048), 8 sequences. O, L, M come from skv_flash_fwd on
    the same random q, k, v, which is timed on its own as `forward`."""
    import numpy as np
    import torch

    from simple_llm_amd import _lib

    B_, N, H_, Dh = 8, 2048, 16, 64
    dev = ctx.device
    g = torch.Generator(device=dev).manual_seed(3)
    q, k, v, do = (torch.randn(B_ * N, H_ * Dh, generator=g, device=dev) for _ in range(4))
    sc = 1.0 / float(np.sqrt(Dh))
    L = _lib.lib()
    o = torch.empty_like(q)
    Ls, Ms = torch.empty(B_ * N * H_, device=dev), torch.empty(B_ * N * H_, device=dev)
    stream = _lib.stream_handle(dev)

    def fwd():
        _lib.check(L.skv_flash_fwd(o.data_ptr(), Ls.data_ptr(), Ms.data_ptr(), q.data_ptr(),
                                   k.data_ptr(), v.data_ptr(), B_, N, H_, Dh, sc, stream),
                   "skv_flash_fwd")

    # the forward (O, L, M for the backward), timed on its own with HIP events
    # after the same clock settle as the prefill record (back-to-back calls)
    fwd_settle_s = settle(lambda: [fwd() for _ in range(4)], lambda: None)
    fevs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            for _ in range(10)]
    for e0, e1 in fevs:
        e0.record()
        fwd()
        e1.record()
    torch.cuda.synchronize()
    fwd_s = float(np.mean([a.elapsed_time(b) for a, b in fevs])) * 1e-3
    fwd_flops = 4.0 * Dh * (N * (N + 1) / 2) * B_ * H_  # S = QK^T and O = PV, causal pairs
    forward = {"mean_us": fwd_s * 1e6, "tflops": fwd_flops / fwd_s / 1e12,
               "peak_tflops": MFMA_FP32_PEAK_TFLOPS,
               "frac": fwd_flops / fwd_s / 1e12 / MFMA_FP32_PEAK_TFLOPS, "flops": fwd_flops,
               "settle_s": round(fwd_settle_s, 3),
               "kernel": "skv_flash_fwd (k_flash_fwd), O, L, M in fp32"}
    dq, dk, dv = (torch.empty_like(q) for _ in range(3))
    # the workspace of the five-product form (the row deltas and dS)
    ws = torch.empty(L.skv_flash_bwd_fast_workspace_bytes(B_, N, H_, Dh), dtype=torch.uint8,
                     device=dev)

    def call():
        rc = L.skv_flash_bwd(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), q.data_ptr(),
                             k.data_ptr(), v.data_ptr(), o.data_ptr(), Ls.data_ptr(),
                             Ms.data_ptr(), do.data_ptr(), B_, N, H_, Dh, sc, ws.data_ptr(),
                             ws.numel(), stream)
        _lib.check(rc, "skv_flash_bwd")

    for _ in range(args.warmup):
        call()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for e0, e1 in evs:
        e0.record()
        call()
        e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    call_s = float(np.mean([a.elapsed_time(b) for a, b in evs])) * 1e-3
    # five causal products of 2*D flops per (query, key <= query) pair:
    # S = QK^T, dP = dO V^T, dV = P^T dO, dK = dS^T Q, dQ = dS K
    flops = 10.0 * Dh * (N * (N + 1) / 2) * B_ * H_
    roof = {"bound": "mfma", "achieved": flops / call_s / 1e12, "peak": MFMA_FP32_PEAK_TFLOPS,
            "unit": "TFLOP/s", "frac": flops / call_s / 1e12 / MFMA_FP32_PEAK_TFLOPS,
            "traffic": None, "kernel": "skv_flash_bwd, five-product form (k_fbwd_delta + k_fbwd_dkv + k_fbwd_dq_ds), HIP events",
            "mean_call_us": call_s * 1e6, "algorithmic_flops": flops}
    # same-run accuracy: the gradients of two (sequence, head) pairs against
    # float64 autograd on the CPU over the same q, k, v, dO (norm-wise per tensor)
    errs = []
    for b, h in ((0, 0), (B_ - 1, H_ - 1)):
        xs = [x.view(B_, N, H_, Dh)[b, :, h].double().cpu() for x in (q, k, v, do)]
        qh, kh, vh = (x.clone().requires_grad_(True) for x in xs[:3])
        mask = torch.ones(N, N, dtype=torch.bool).tril()
        oh = torch.softmax((qh @ kh.T * sc).masked_fill(~mask, float("-inf")), -1) @ vh
        want = torch.autograd.grad(oh, (qh, kh, vh), xs[3])
        for gt, wt in zip((dq, dk, dv), want):
            gh = gt.view(B_, N, H_, Dh)[b, :, h].double().cpu()
            errs.append(float((gh - wt).norm() / wt.norm()))
    accuracy = {"max_rel_err": max(errs), "tolerance": 1e-4, "pass": max(errs) <= 1e-4,
                "against": "torch float64 autograd on the CPU, (sequence, head) (0, 0) and "
                           "(7, 15) of the last timed call",
                "norm": "||gpu - oracle||_F / ||oracle||_F per gradient tensor (dq, dk, dv)"}
    cpu = None
    if not args.no_cpu_baseline:
        # the reference's CPU path differentiates attention with JAX autodiff; the
        # same backward in torch CPU fp32 autograd, one (sequence, head) at a time
        qc, kc, vc, doc = (x.view(B_, N, H_, Dh).cpu() for x in (q, k, v, do))
        maskc = torch.ones(N, N, dtype=torch.bool).tril()
        n, t0 = 0, time.perf_counter()
        while n == 0 or time.perf_counter() - t0 < args.cpu_seconds:
            b, h = divmod(n % (B_ * H_), H_)
            qh, kh, vh = (x[b, :, h].clone().requires_grad_(True) for x in (qc, kc, vc))
            s_ = (qh @ kh.T * sc).masked_fill(~maskc, float("-inf"))
            oh = torch.softmax(s_, -1) @ vh
            torch.autograd.grad(oh, (qh, kh, vh), doc[b, :, h])
            n += 1
        dt = time.perf_counter() - t0
        cpu = {"value": n * N / H_ / dt, "unit": "tokens/s", "cores": torch.get_num_threads(),
               "kind": "port",
               "sample": f"{n} (sequence, head) backward passes of N=2048, D=64 in torch CPU "
                         f"fp32 autograd, {dt:.1f} s; tokens/s = passes * N / H / time"}
    return _record(
        "attention backward tokens/sec", B_ * N * args.steps / wall, "tokens/s", args.steps,
        args.warmup, wall / args.steps * 1e3, "fp32",
        {"workload": "FB causal flash-attention backward fp32: B=8, N=2048, H=16, D=64 "
                     "(O, L, M from skv_flash_fwd)", "batch": B_},
        roof, cpu, forward=forward, max_rel_err=accuracy["max_rel_err"], accuracy=accuracy)


def run_sample(args, ctx):
    """Next-token sampling at the C3 decode shape: 16 rows of 50,304 fp32
    logits with the reference's default parameters (temperature 1, no min-p,
    top-k or top-p, no penalty: generate.py:8-18), one skv_sample call per
    step with the split-row workspace (a new seed each call); the
    one-workgroup-per-row kernel (no workspace) is timed the same way
    beside it."""
    import numpy as np
    import torch

    from simple_llm_amd import _lib

    M, V, CTX = 16, 50304, 1024
    dev = ctx.device
    g = torch.Generator(device=dev).manual_seed(5)
    logits = torch.randn((M, V), generator=g, device=dev) * 2.5
    seq = torch.randint(0, V, (M, CTX), generator=g, device=dev, dtype=torch.int32)
    lens = torch.full((M,), 512, dtype=torch.int32, device=dev)
    out = torch.zeros(M, dtype=torch.int32, device=dev)
    L = _lib.lib()
    wsb = L.skv_sample_workspace_bytes(M, V)
    ws = torch.zeros(wsb, dtype=torch.uint8, device=dev)
    stream = _lib.stream_handle(dev)

    def call(split, seed):
        _lib.check(L.skv_sample(out.data_ptr(), None, logits.data_ptr(), seq.data_ptr(), CTX,
                                lens.data_ptr(), M, V, 1.0, 0, 1.0, 0.0, 1.0, 64, seed,
                                ws.data_ptr() if split else None, wsb if split else 0, stream),
                   "skv_sample")

    def timed(split):
        for i in range(args.warmup):
            call(split, i)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record()
        for i in range(args.steps):
            call(split, i)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e-3 / args.steps, time.perf_counter() - t0

    one_s, _ = timed(False)
    call_s, wall = timed(True)
    # same-run accuracy: the last timed call's draws (seed steps - 1) against
    # the oracle's inverse-CDF draw from sample_token's distribution with the
    # same uniform; a draw whose u * total lies within 1e-5 of a step of the
    # running sum may take either neighbour
    from oracle import sample_oracle as so
    got = out.cpu().numpy()
    lgh = logits.cpu().numpy().astype(np.float64)
    seed = args.steps - 1
    equal = ambiguous = 0
    for m in range(M):
        pr = so.sample_filter(lgh[m], 1.0)
        u = so.splitmix_uniform(seed, m, 512)
        c = np.cumsum(pr)
        if int(got[m]) == so.sample_draw(pr, u):
            equal += 1
        elif np.abs(c - u * c[-1]).min() < 1e-5 * c[-1]:
            ambiguous += 1
    accuracy = {"max_rel_err": None, "draws": M, "draws_equal_oracle": equal,
                "draws_at_a_rounding_step": ambiguous, "pass": equal + ambiguous == M,
                "against": "oracle/sample_oracle.py (float64 sample_token filter + the same "
                           "uniform), the last timed call's 16 draws; a draw is a token id, "
                           "so it is checked for equality, not a relative error"}
    # the logits once, and the picked 2048-entry slice of each row again
    nbytes = M * V * 4 + M * 2048 * 4
    roof = {"bound": "launch latency", "achieved": nbytes / call_s / 1e9, "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": nbytes / call_s / 1e9 / HBM_PEAK_GBS, "traffic": None,
            "kernel": "skv_sample split path (k_sample_slices + k_sample_pick), HIP events",
            "mean_call_us": call_s * 1e6, "algorithmic_bytes": nbytes,
            "note": "two launches of ~3 MB: each at the per-kernel floor"}
    cpu = None
    if not args.no_cpu_baseline:
        # the oracle's restatement of sample_token (float64 numpy), row by row
        from oracle import sample_oracle as so
        lg = logits.cpu().numpy().astype(np.float64)
        n, t0 = 0, time.perf_counter()
        while n == 0 or time.perf_counter() - t0 < min(args.cpu_seconds, 5.0):
            m = n % M
            so.sample_draw(so.sample_filter(lg[m], 1.0), so.splitmix_uniform(n, m, 512))
            n += 1
        dt = time.perf_counter() - t0
        cpu = {"value": n / dt, "unit": "draws/s", "cores": 1, "kind": "port",
               "sample": f"{n} draws from 50,304-entry rows by oracle/sample_oracle.py "
                         f"(numpy float64 softmax + inverse-CDF draw), {dt:.1f} s"}
    return _record(
        "sampled draws/sec", M * args.steps / wall, "draws/s", args.steps, args.warmup,
        wall / args.steps * 1e3, "fp32",
        {"workload": "sampling at the C3 shape: 16 rows x 50,304 fp32 logits, temperature 1, "
                     "no min-p/top-k/top-p, no penalty (the reference's defaults)",
         "batch": M, "vocab": V},
        roof, cpu, one_workgroup_per_row={"mean_call_us": one_s * 1e6,
                                          "kernel": "k_sample, one 1024-thread workgroup a row"},
        max_rel_err=None, accuracy=accuracy)


def main():
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build runs on one GPU only (the decode path would shard over "
              "sequences, kv heads or token ranges, each GPU running the same kernels on its "
              f"share); --gpus {args.gpus} is not supported", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration()
        return
    if args.workload != "c4":
        from simple_llm_amd.gpu import gpu

        ctx = gpu.context_create()
        ctx.config.decode_chunk_tokens = args.chunk_tokens
        rec = {"c1": run_c1, "c2": run_c2, "c3": run_c3, "c5": run_c5,
               "fb": run_fb, "sample": run_sample}[args.workload](args, ctx)
        print(json.dumps(rec), flush=True)
        return
    if FILL + args.steps > T_CAP or args.steps < 1 or args.warmup < 0:
        print(f"bench.py: --steps must lie in [1, {T_CAP - FILL}]", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from simple_llm_amd.gpu import gpu

    ctx = gpu.context_create()
    ctx.config.decode_chunk_tokens = args.chunk_tokens
    dev = ctx.device
    cache = gpu.kv_cache_create(ctx, gpu.KVCacheConfig(B, T_CAP, 1, H, D, dtype=torch.bfloat16))
    layer = cache.layers[0]
    g = torch.Generator(device=dev).manual_seed(0)
    kv = layer.k_cache.buffer.view(B, T_CAP, H, D)
    vv = layer.v_cache.buffer.view(B, T_CAP, H, D)
    for b in range(B):  # fill [0, FILL) with N(0,1), one sequence at a time
        kv[b, :FILL].copy_(torch.randn((FILL, H, D), generator=g, device=dev))
        vv[b, :FILL].copy_(torch.randn((FILL, H, D), generator=g, device=dev))
    n_in = args.warmup + args.steps
    q_all = torch.randn((n_in, B, H, D), generator=g, device=dev)
    k_all = torch.randn((n_in, B, H, D), generator=g, device=dev)
    v_all = torch.randn((n_in, B, H, D), generator=g, device=dev)
    out = torch.empty((B, H, D), device=dev)
    max_len = FILL + args.steps  # split-K plan sized for the longest step

    # per-step views made once, outside the timed loop (indexing a tensor costs ~1 us of
    # host time, and each call is ~13 us of it)
    qs, ks, vs = q_all.unbind(0), k_all.unbind(0), v_all.unbind(0)

    def step(i):
        gpu.kv_cache_append_attend(ctx, cache, 0, ks[i], vs[i], qs[i], out, max_len=max_len)

    # clock settle and warm-up, then rewind the fill to FILL
    settle_s = settle(lambda: [step(i) for i in range(min(args.steps, 32))],
                      lambda: setattr(cache, "current_len", FILL))
    for i in range(args.warmup):
        step(args.steps + i)
    torch.cuda.synchronize()
    cache.current_len = FILL
    torch.cuda.synchronize()

    # one HIP event pair around the timed region, on the launch stream (per-step
    # events would add a marker and ~5 us of host time to every step)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record()
    for i in range(args.steps):
        step(i)
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0

    lens_per_step = [[FILL + i + 1] * B for i in range(args.steps)]
    bytes_per_call = float(np.mean([algorithmic_bytes(ls) for ls in lens_per_step]))
    mean_s = ev0.elapsed_time(ev1) * 1e-3 / args.steps
    achieved = bytes_per_call / mean_s / 1e9
    assert cache.layers[0].lens.cpu().tolist() == [FILL + args.steps] * B

    chunk, n_chunks = gpu.decode_plan(ctx, B, H, H, max_len, head_dim=D, dtype=cache.dtype)
    # the same K steps again with an event pair per call (outside the timed
    # region above, whose single pair carries no per-call markers): the
    # spread of the call time over the run
    cache.current_len = FILL
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(args.steps)]
    torch.cuda.synchronize()
    for i, (e0, e1) in enumerate(evs):
        e0.record()
        step(i)
        e1.record()
    torch.cuda.synchronize()
    per = np.array([a.elapsed_time(b) * 1e3 for a, b in evs])
    per_call = {"events": "one pair per call, a second pass over the same steps",
                "mean_us": float(per.mean()), "median_us": float(np.median(per)),
                "min_us": float(per.min()), "max_us": float(per.max()),
                "first5_us": [round(float(x), 1) for x in per[:5]]}
    oracle_outs = []
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(args, layer.k_cache.buffer, layer.v_cache.buffer, q_all, k_all,
                           v_all, outs=oracle_outs)
    else:  # no timing, but the same-run accuracy check still runs 2 steps of the oracle
        short = argparse.Namespace(**{**vars(args), "steps": min(args.steps, 2)})
        cpu_baseline(short, layer.k_cache.buffer, layer.v_cache.buffer, q_all, k_all, v_all,
                     outs=oracle_outs)
    gpu_outs = replay_outputs(step, len(oracle_outs), lambda: setattr(cache, "current_len", FILL),
                              out)
    accuracy = accuracy_record(gpu_outs, oracle_outs, 2e-2,
                               "oracle/c/kv_attn_ref.c on the same bf16 cache values (fp32 "
                               "math), the first steps of the timed run")
    prefill = None if args.no_prefill else time_prefill(ctx, cache, reps=20)

    traffic = measured_traffic()
    rec = {
        "metric": "decode tokens/sec",
        "value": B * args.steps / wall,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_settle_s": round(settle_s, 3),
        "ms_per_step": wall / args.steps * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "C4 long-context decode: B=4, H=16 (MHA), D=128, KV cap 32768 bf16 "
                        "storage / fp32 accumulation, filled to 32000, per step append + "
                        "decode attention",
            "batch": B, "n_heads": H, "head_dim": D, "kv_capacity": T_CAP,
            "start_fill": FILL, "kv_dtype": "bf16", "accumulate": "fp32",
            "parallelism": "single GPU",
        },
        "roofline": {
            "kernel": "append + decode attention (k_decode_partial + k_decode_merge)",
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": traffic,
            "mean_call_us": mean_s * 1e6,
            "split_k": {"chunk_tokens": chunk, "n_chunks": n_chunks},
            "algorithmic_bytes_per_call": bytes_per_call,
            "per_call": per_call,
        },
        "cpu_baseline": _with_cpu_model(cpu),
        "max_rel_err": accuracy["max_rel_err"],
        "accuracy": accuracy,
        "prefill": prefill,
    }
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
