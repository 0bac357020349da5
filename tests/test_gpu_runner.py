"""bench.py's runner mode on the GPU (reference benchmarks/benchmark_main.cpp:
--suite / --operator with --param shapes, --variant, --cache-mode): every
entry point and a stage operator run at small shapes, warm and cold, and each
prints the record the headline line has. Outputs are checked elsewhere
against the oracle; here the record's shape, units and values are."""
from __future__ import annotations

import math

import pytest

import bench

pytestmark = pytest.mark.gpu


def _run(*argv):
    import torch
    args = bench.parse(["--warmup", "2", "--samples", "3", "--kernel-repeats", "2", *argv])
    return bench.run_runner(torch, torch.device("cuda:0"), args)


def _common(line, workload, samples=3):
    assert line["config"]["workload"] == workload
    assert line["n_gpus"] == 1 and line["dtype"] == "fp32" and line["higher_is_better"]
    assert math.isfinite(line["value"]) and line["value"] > 0
    assert line["samples"]["samples"] == samples and line["ms_per_step"] > 0


@pytest.mark.parametrize("suite,params,unit", [
    ("chain_from_tokens", ["T=256", "E=16", "K=64", "N=32"], "tokens/s"),
    ("chain_from_logits", ["T=300", "E=8", "K=32", "N=48", "tie_fraction=0.05"], "tokens/s"),
    ("chain_from_route_ids", ["T=200", "E=16", "K=64", "N=64", "top_k=4", "distribution=zipf"], "tokens/s"),
])
def test_suites_print_one_record(suite, params, unit):
    line = _run("--suite", suite, "--param", *params)
    _common(line, suite)
    assert line["unit"] == unit and line["config"]["T"] == int(params[0][2:])


def test_operator_cold_scrub_prices_the_roofline():
    line = _run("--operator", "grouped_gemm", "--cache-mode", "cold_scrub", "--cache-scrub-bytes",
                str(64 << 20), "--param", "T=512", "E=8", "K=128", "N=96")
    _common(line, "grouped_gemm")
    assert line["config"]["cache_mode"] == "cold_scrub"
    roof = line["roofline"]
    assert line["flops"] == 2 * 1024 * 128 * 96 and line["bytes"] > 0 and 0 < roof["frac"] < 1
    # priced against the bound its arithmetic intensity selects
    mfma = line["flops"] / line["bytes"] >= bench.RIDGE
    assert (roof["bound"], roof["unit"]) == (("mfma", "TFLOP/s") if mfma else ("hbm", "GB/s"))


def test_naive_variant_and_profile_once():
    line = _run("--operator", "unpermute", "--variant", "naive", "--param", "T=128", "E=4", "K=16", "N=40")
    _common(line, "unpermute")
    assert line["config"]["variant"] == "naive" and line["roofline"]["bound"] == "hbm"
    assert _run("--suite", "chain_from_tokens", "--profile-once", "--param", "T=64", "E=8", "K=32", "N=32") is None
