"""The instrumentation build (libraggedroute_amd_stamps.so: strip.hip with
-DRR_PHASE_STAMPS) runs the headline chain and `bench.py --phase-stamps`
reads a consistent set of phase stamps from it: every workgroup of the expert
launch stamped, phases in order, a shader clock between 1 and 3 GHz, and the
strip counts of the launch summing to at least the headline's strips. The
stamps build's chain outputs equal the product library's bit for bit (same
kernels apart from the stamp stores)."""
from __future__ import annotations

import json
import os
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

REPO = Path(__file__).resolve().parents[1]
STAMPS = REPO / "raggedroute_amd" / "libraggedroute_amd_stamps.so"

CHECKSUM = r"""
import hashlib, sys, torch
sys.path.insert(0, sys.argv[1])
import bench
from raggedroute_amd import workloads
dev = torch.device("cuda:0")
cfg = workloads.HEADLINE
ch = bench.Chain(cfg, workloads.chain_inputs_device(cfg, 0, dev), dev)
for _ in range(3):
    ch.chain()
torch.cuda.synchronize()
h = hashlib.sha256()
for t in (ch.logits, ch.ids, ch.w, ch.counts, ch.offsets, ch.pos, ch.xp, ch.y):
    h.update(t.cpu().numpy().tobytes())
print(h.hexdigest())
"""


def _run(args, env, timeout=240):
    print("phase stamps:", " ".join(args), flush=True)
    return subprocess.run([sys.executable, *args], cwd=REPO, env=env, capture_output=True, text=True,
                          timeout=timeout)


def test_phase_stamps_read_back():
    assert STAMPS.exists(), "build the library first (python raggedroute_amd/build.py)"
    env = dict(os.environ, RR_LIBRARY=str(STAMPS))
    out = _run(["bench.py", "--phase-stamps"], env)
    assert out.returncode == 0, out.stderr[-2000:]
    rec = json.loads(out.stdout.strip().splitlines()[-1])
    assert rec["grid"] > 0
    assert 1.0 < rec["shader_clock_ghz_median"] < 3.0
    strips = np.array(rec["strips_per_workgroup"])
    assert (strips * np.arange(strips.size)).sum() >= 8192 // 16  # every strip of the 8192 routes
    for row in rec["prologue"]:
        assert row["wave0_median_us"] >= 0.0, row
    assert rec["workgroup_span_us"]["median"] > 0.0


def test_stamps_build_outputs_match_the_product():
    base = _run(["-c", CHECKSUM, str(REPO)], dict(os.environ))
    assert base.returncode == 0, base.stderr[-2000:]
    stamped = _run(["-c", CHECKSUM, str(REPO)], dict(os.environ, RR_LIBRARY=str(STAMPS)))
    assert stamped.returncode == 0, stamped.stderr[-2000:]
    assert base.stdout.strip().splitlines()[-1] == stamped.stdout.strip().splitlines()[-1]
