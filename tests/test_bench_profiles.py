"""The benchmark's counter figures come from the committed profiles/
summaries; these checks read them the way bench.py does, on the CPU.

- every summary the bench cites parses, with a kernel trace and the
  counter sections the bench reads;
- the headline launch's HBM traffic (stream kernel + its merge) is within a
  few percent above its algorithmic bytes, and the stack's per-step total is
  present;
- every command a summary quotes runs bench.py with a mode it accepts, so
  the figures can be regenerated from committed files;
- bench.py refuses more than one GPU before touching a device.
"""
import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402

PROFILES = os.path.join(ROOT, "profiles")
CITED = ["decode_global_d512_ctx4096.txt", "decode_ragged_b32_ctx1k-32k.txt", "decode_sliding_d256_ctx64.txt",
         "decode_e2b_stack_35_layers_ctx8192.txt", "decode_e2b_stack_35_layers_ctx8192_layer_attention.txt",
         "prefill_2048_sliding_and_global.txt",
         "q8_0_matvec_output_head_262144x1536.txt", "layer_drivers_global_decode_and_prefill_2048.txt",
         "floors_empty_kernel_and_streaming_read.txt", "hbm_counter_calibration.txt"]


@pytest.mark.parametrize("name", CITED)
def test_cited_summary_exists_and_names_its_commands(name):
    text = open(os.path.join(PROFILES, name)).read()
    commands = re.findall(r"bench\.py --only (\w+)", text)
    assert commands, name
    for mode in commands:
        assert mode in bench.ONLY, (name, mode)


def test_headline_traffic_is_the_algorithmic_bytes_plus_partials():
    algorithmic = 2041479168  # K/V rows of the 32 sequences at d=512, q and out (bench.decode_bytes)
    traffic = bench.traffic_bytes("decode_ragged_b32_ctx1k-32k.txt",
                                  ["decode_stream_kernel<512", "decode_merge_kernel<3, 512"])
    assert traffic is not None
    assert 1.0 <= traffic / algorithmic <= 1.05, traffic / algorithmic


def test_decode_summaries_carry_per_step_totals():
    for name in ("decode_global_d512_ctx4096.txt", "decode_e2b_stack_35_layers_ctx8192.txt",
                 "decode_ragged_b32_ctx1k-32k.txt", "decode_sliding_d256_ctx64.txt"):
        t = bench.traffic_bytes(name)
        assert t is not None and t > 0, name
    # the stack reads every layer's rows at least once
    assert bench.traffic_bytes("decode_e2b_stack_35_layers_ctx8192.txt") >= 264929280


def test_prefill_summary_has_trace_and_mfma_busy():
    prof = bench.profile_summary("prefill_2048_sliding_and_global.txt")
    for kernel in ("prefill_kernel<256>", "prefill_kernel<512>"):
        rows = [v for k, v in prof.items() if kernel in k]
        assert rows, kernel
        v = rows[0]
        assert v.get("avg_us", 0) > 0
        busy = v.get("mfma_busy")
        assert busy is not None and 0.0 < busy < 1.0, (kernel, busy)
    # HBM traffic of a step: MFMA-bound, so far below what the launches could stream
    t = bench.traffic_bytes("prefill_2048_sliding_and_global.txt")
    assert t is not None and 0 < t < 1e9, t


def test_counter_calibration_factors():
    text = open(os.path.join(PROFILES, "hbm_counter_calibration.txt")).read()
    factors = [float(x) for x in re.findall(r"factor ([0-9.]+)", text)]
    assert factors and all(0.5 < f < 4.0 for f in factors), factors


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode != 0
    assert "one GPU" in r.stderr or "1 GPU" in r.stderr, r.stderr
