"""Compile the HIP kernels and the C ABI into libskv.so for gfx950.

Used by __graft_entry__.build(); also runnable as a script. The library is
built in-tree (next to this file) so that it travels with the source tree.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
LIB = os.path.join(HERE, "libskv.so")

SOURCES = ["skv_api.hip", "append.hip", "decode_attn.hip", "decode_attn_generic.hip",
           "decode_attn_generic_paged.hip", "decode_gqa_mfma.hip",
           "decode_direct.hip", "prefill_attn.hip", "model_ops.hip", "gemm.hip",
           "sample.hip", "flash_fp32.hip", "flash_fp32.hip:wide_bwd", "bpe_tokenizer.cpp"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # packed fp32 (v_pk_*_f32) is kept off for all device code on this pool
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return os.path.join(rocm, "bin", "hipcc")


# Extra flags per source. The flash backward keeps its MFMA accumulators in
# ordinary VGPRs (gfx950 MFMAs take either register file); the default
# heuristic put them in AGPRs and copied them back and forth every step.
SOURCE_FLAGS = {"flash_fp32.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
                # the flash backward past a head dim of 128: the same source as its own
                # translation unit, accumulators free to live in AGPRs
                "flash_fp32.hip:wide_bwd": ["-DSKV_FLASH_WIDE_BWD=1"]}

_NOISE = "is not a recognized feature for this target"  # hipcc's host pass on -packed-fp32-ops


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    msgs = [ln for ln in (res.stdout + res.stderr).splitlines() if _NOISE not in ln]
    if res.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(msgs))
    if verbose and msgs:
        print("\n".join(msgs))


def build(verbose: bool = False) -> str:
    """Compiles every source to an object (in parallel, each with its own
    extra flags), then links libskv.so."""
    import tempfile
    from concurrent.futures import ThreadPoolExecutor

    flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    with tempfile.TemporaryDirectory(prefix="skv_build_") as tmpdir:
        jobs = []
        for src in SOURCES:  # "file" or "file:variant" (the same file, other flags)
            obj = os.path.join(tmpdir, src.replace(":", "_") + ".o")
            path = os.path.join(CSRC, src.split(":")[0])
            jobs.append((obj, [hipcc(), *flags, *SOURCE_FLAGS.get(src, []), "-I", CSRC, "-I",
                               INCLUDE, "-c", path, "-o", obj]))
        with ThreadPoolExecutor(max_workers=min(len(jobs), os.cpu_count() or 4, 8)) as pool:
            for f in [pool.submit(_run, cmd, verbose) for _, cmd in jobs]:
                f.result()
        tmp = LIB + ".tmp"
        _run([hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *[o for o, _ in jobs], "-o",
              tmp], verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
