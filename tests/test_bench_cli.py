"""bench.py's command line on the host: the runner mode's --param parsing
(reference benchmarks/benchmark_main.cpp:61-115 takes KEY=VALUE pairs after
--param), the batch statistics of the reported value and the single-GPU
guard. CPU only: nothing here touches a GPU.
"""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import pytest

import bench

REPO = Path(__file__).resolve().parent.parent


def test_param_pairs_in_one_or_several_flags():
    a = bench.parse(["--suite", "chain_from_route_ids", "--param", "T=8", "E=4", "top_k=4",
                     "--param", "K=16", "distribution=zipf", "zipf_s=1.2"])
    p = bench.runner_params(a.param)
    assert (p["T"], p["E"], p["top_k"], p["K"], p["N"]) == (8, 4, 4, 16, 128)
    assert p["distribution"] == "zipf" and p["zipf_s"] == 1.2 and p["seed"] == 0


def test_param_defaults_are_the_headline_shape():
    p = bench.runner_params([])
    assert (p["T"], p["E"], p["K"], p["N"], p["top_k"]) == (4096, 64, 256, 128, 2)


@pytest.mark.parametrize("bad", ["T", "X=1", "=3"])
def test_param_rejects_unknown_or_malformed_pairs(bad):
    with pytest.raises(SystemExit, match="--param"):
        bench.runner_params([bad])


def test_percentile_interpolates_between_closest_ranks():
    # reference runner.cpp:42-50: linear interpolation at q (n - 1)
    assert bench.percentile([4.0, 1.0, 3.0, 2.0], 0.5) == 2.5
    assert bench.percentile([7.0], 0.95) == 7.0
    assert bench.percentile([1.0, 2.0, 3.0, 4.0, 5.0], 0.95) == pytest.approx(4.8)


def test_more_than_one_gpu_exits_with_a_message():
    proc = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"],
                          capture_output=True, text=True, timeout=300)
    assert proc.returncode != 0
    assert "measures one MI355X" in (proc.stdout + proc.stderr)
