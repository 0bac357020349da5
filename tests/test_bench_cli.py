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


@pytest.mark.parametrize("steps,expect", [(20, [10, 10]), (200, [10] * 20), (5, [5]), (1000, [50] * 20),
                                          (37, [13, 12, 12]), (1, [1])])
def test_batches_keep_at_least_ten_calls_per_timed_sample(steps, expect):
    # the per-call share of a sample's timing event must not depend on --steps
    sizes = bench.batch_sizes(steps)
    assert sizes == expect and sum(sizes) == steps


def _oracle_chain_as_device_outputs(cfg):
    import oracle
    from raggedroute_amd import workloads
    host = workloads.chain_inputs(cfg, seed=0)
    ref = oracle.chain(host["x"], host["expert_weights"], router_weights=host["router_weights"])
    dev = {key: ref[key].copy() for key in ("logits", "ids", "weights", "counts", "offsets", "route_pos", "y")}
    dev["x_permuted"] = oracle.permute_rows(host["x"], ref["route_pos"], 2)
    return host, ref, dev


def test_validation_of_the_timed_chain_accepts_oracle_outputs():
    from raggedroute_amd import workloads
    cfg = workloads.ChainConfig("v", 64, 8, 32, 16)
    host, ref, dev = _oracle_chain_as_device_outputs(cfg)
    out = bench.validate_chain(cfg, host, dev, ref)
    assert out["ok"], out["checks"]
    assert out["id_rows_differing_from_cpu_logits"] == 0


@pytest.mark.parametrize("plant", ["route_pos", "x_permuted", "y", "counts", "ids", "logits"])
def test_validation_of_the_timed_chain_catches_planted_mistakes(plant):
    from raggedroute_amd import workloads
    cfg = workloads.ChainConfig("v", 64, 8, 32, 16)
    host, ref, dev = _oracle_chain_as_device_outputs(cfg)
    if plant == "route_pos":
        dev["route_pos"][[0, 1]] = dev["route_pos"][[1, 0]]
    elif plant == "x_permuted":
        dev["x_permuted"][3, 5] = dev["x_permuted"][3, 5] + 1.0
    elif plant == "y":
        dev["y"][7, 2] += 1e-2
    elif plant == "counts":
        dev["counts"][0] += 1
    elif plant == "ids":
        dev["ids"][4] = dev["ids"][4][::-1]
    else:
        dev["logits"][9, 1] += 1e-3
    assert not bench.validate_chain(cfg, host, dev, ref)["ok"]
