"""The benchmark's contract on the CPU: the driver's command times config 2's whole 262,144-token
chunk, split over its --steps launches, and refuses more than one GPU."""

import os
import subprocess
import sys

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_chunk_split_covers_the_chunk():
    for steps in (1, 3, 20, 64, 1000):
        sizes = bench.split_chunk(262_144, steps)
        assert len(sizes) == steps
        assert sum(sizes) == 262_144
        assert max(sizes) - min(sizes) <= 1
    # the driver's command: --steps 20 --warmup 5
    assert bench.split_chunk(262_144, 20)[:4] == [13_108] * 4
    assert bench.split_chunk(262_144, 20)[4:] == [13_107] * 16


def test_defaults_are_the_driver_workload():
    a = bench.make_parser().parse_args(["--gpus", "1", "--steps", "20", "--warmup", "5"])
    assert a.config == "c2" and a.chunk == 262_144
    assert sum(bench.split_chunk(a.chunk, a.steps)) == 262_144
    assert set(a.legs.split(",")) == {"decode", "stress", "plumbing", "prefill", "dense"}
    # config 5's run: 65,536 greedy tokens; config 1: 256 steps
    assert a.c5_tokens == 65_536 and sum(bench.split_chunk(a.c5_tokens, a.c5_steps)) == 65_536
    d = bench.make_parser().parse_args([])
    assert (d.gpus, d.steps, d.warmup) == (1, 20, 5)


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_latency_roofline_counts_hops():
    """Two one-way hops per token for the head, three per GDN event, each half a round trip."""
    sync = {"round_trip_other_xcd_us": 1.0}
    r = bench.latency_roofline(sync, 1.0, 100.0)
    assert r["hops_per_token"] == 5.0 and r["round_trips_per_token"] == 2.5
    assert r["t_sync_us"] == 2.5 and r["frac"] == 0.025
