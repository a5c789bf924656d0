"""CPU checks of bench.py's contract and byte accounting (no GPU needed)."""

from __future__ import annotations

import math
import os
import subprocess
import sys

from conftest import ROOT

sys.path.insert(0, ROOT)
import bench  # noqa: E402


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode != 0
    assert "one GPU" in r.stderr and r.stdout == ""


def test_attention_bytes_follow_the_formula():
    # per sequence: K and V of L + C keys, Q read and O written, block ids, start / id
    lens = [256, 4096, 1]
    C, Hq, Hkv, d, bs = 6, 12, 2, 128, 16
    want = sum((L + C) * 2 * Hkv * d * 2 + 2 * C * Hq * d * 2 + 4 * math.ceil((L + C) / bs) + 8 for L in lens)
    assert bench.attention_bytes(lens, C, Hq, Hkv, d, bs) == want
    # the headline workload: 87.3 MB per call
    assert abs(bench.attention_bytes(bench.workload_lens(0)[0]) - 87.33e6) < 0.01e6


def test_sample_bytes_follow_the_formula():
    B, C, G, V = 32, 6, 5, 151936
    # every row read for its statistics, then the noise row
    assert bench.sample_bytes(B, draft_stats=False) == B * ((C + G) * V * 4 + V * 4 + G * 8 + 12)
    # the draft rows' statistics from the draft sampler: target rows, noise row,
    # the raced draft row, and per position u, proposal, q at it and the statistics
    assert bench.sample_bytes(B) == B * ((C + 2) * V * 4 + G * (4 + 4 + 4 + 8) + 12)


def test_workload_lengths_are_seeded_and_in_range():
    a, _ = bench.workload_lens(0)
    b, _ = bench.workload_lens(0)
    assert a == b and len(a) == bench.B and all(256 <= L <= 4096 for L in a)


def test_replicas_are_distinct_context_draws_near_the_distribution_mean():
    rl = bench.replica_lens(0)
    assert len(rl) == bench.REPLICAS and rl[0] == bench.workload_lens(0)[0]
    assert len({tuple(r) for r in rl}) == bench.REPLICAS
    mean = sum(sum(r) for r in rl) / (bench.REPLICAS * bench.B)
    # U[256, 4096] has mean 2176; 256 draws put the sample mean within ~6%
    assert abs(mean - 2176) < 0.06 * 2176, mean
