"""bench.py's driver contract, checked without a GPU: the one-GPU guard, the
HBM traffic it reads from the committed rocprofv3 summaries into
`roofline.traffic`, and the prefill's algorithmic flops."""
import importlib.util
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", BENCH)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)  # module level defines constants and functions only
    return mod


@pytest.mark.parametrize("argv,env", [(["--gpus", "2"], {}), (["--gpus", "8"], {}),
                                      ([], {"WORLD_SIZE": "2"})])
def test_more_than_one_gpu_exits_with_a_message(argv, env):
    r = subprocess.run([sys.executable, BENCH, *argv], capture_output=True, text=True,
                       timeout=120, env={**os.environ, **env})
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout == ""  # no JSON line


def _algorithmic_decode_bytes(lens, h_kv, h_q, d, s_kv, s_q, s_o):
    """One decode call's algorithmic bytes: every filled K and V row of every
    (sequence, kv head), plus q and out."""
    return sum(2 * h_kv * (n * d * s_kv) + h_q * d * (s_q + s_o) for n in lens)


def test_c4_traffic_is_read_from_the_committed_profile(bench):
    t = bench.measured_traffic("c4")
    assert t is not None, "profiles/decode_attn_c4_pmc.md lost its traffic_bytes_per_call line"
    # the profile's run spans fills 32001..32256: bytes between the first and last call's
    lo = _algorithmic_decode_bytes([32001] * 4, 16, 16, 128, 2, 2, 2)
    hi = _algorithmic_decode_bytes([32256] * 4, 16, 16, 128, 2, 2, 2)
    assert lo <= t <= 1.05 * hi


def test_c5_traffic_is_read_from_the_committed_profile(bench):
    t = bench.measured_traffic("c5")
    assert t is not None, "profiles/decode_attn_c5_pmc.md lost its traffic_bytes_per_call line"
    # 64 sequences of mean length ~2057 over 8 kv heads x 128, bf16: ~5.4e8 algorithmic bytes
    assert 4.5e8 < t < 7.0e8


def test_missing_profile_gives_no_traffic(bench):
    assert bench.measured_traffic("no_such_workload") is None


def test_prefill_flops_match_the_sum_over_the_chunk(bench):
    start, c = 32256, bench.PREFILL_C
    # each query i of the chunk attends start + i + 1 positions; QK^T and PV are 2*D flops each
    brute = sum(4 * bench.D * bench.H * bench.B * (start + i + 1) for i in range(c))
    assert bench.prefill_flops(start) == brute
    assert abs(bench.prefill_flops(start) - 5.4547e11) / 5.4547e11 < 1e-4
