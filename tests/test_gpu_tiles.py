"""Every GEMM kernel configuration gives the same bits: the strip kernels and
each tiled configuration forced through RR_GEMM_TILE (read by the library at
every launch), and the large tile with its slices staged through registers
instead of loaded straight into LDS (RR_GEMM_STAGING=registers), accumulate
each output in the same k order (16-wide k chunks in ascending order, one MFMA
step per 4 k), so dense and grouped outputs must be bit-identical to the
default dispatch, and within the accumulation-aware bound of the float64
product. Shapes cover aligned (vector loads) and odd K / N or
offset pointers (scalar loads; for the large tile, direct loads at any
alignment with the last slice fixed up in LDS), ragged and empty segments and
the K tails of the 16-, 32- and 64-deep slices.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

import raggedroute_amd as rr
from test_gpu_ops import NATIVE, check_grouped, gemm_ok, ok, run_grouped

pytestmark = pytest.mark.gpu

# "large/registers": the large tile with register-staged slices where the
# direct LDS loads would otherwise run; "large/aligned": direct loads only for
# whole 32-deep slices and 16-byte rows (register staging for the rest, which
# the default large tile loads directly at any alignment)
TILES = ["large", "large/registers", "large/aligned", "small", "medium", "narrow", "small256",
         "medium256", "narrow256"]


@pytest.fixture()
def tile_env():
    saved = {v: os.environ.get(v) for v in ("RR_GEMM_TILE", "RR_GEMM_STAGING")}

    def put(var, value):
        if value is None:
            os.environ.pop(var, None)
        else:
            os.environ[var] = value

    def set_tile(name):
        tile, _, staging = (name or "").partition("/")
        put("RR_GEMM_TILE", tile or None)
        put("RR_GEMM_STAGING", staging or None)
    yield set_tile
    for var, value in saved.items():
        put(var, value)


GROUPED = [
    ([0, 300, 5, 1000, 0, 0, 77, 1], 256, 128, 0),  # strip-eligible default
    ([0, 300, 5, 1000, 0, 0, 77, 1], 100, 72, 0),
    ([0, 300, 5, 1000, 0, 0, 77, 1], 252, 128, 0),  # strip K tail: masked rows of the last k chunk
    ([7, 0, 12, 1, 0], 33, 17, 0),                    # scalar loads (K, N odd)
    ([40, 0, 3, 90], 96, 40, 1),                      # offset pointers
    ([200, 129, 64], 300, 136, 0),                    # K past 256, N past 128
    ([200, 129, 64, 0, 250], 320, 136, 0),            # whole 32-deep slices, N past 128
    ([150, 0, 33, 131], 32, 8, 0),                     # one slice (it reloads itself), N = 8
    ([257, 3, 128], 64, 260, 0),                       # two slices, three column tiles
    ([0, 300, 5, 1000, 0, 0, 77, 1], 128, 128, 0),  # strip K = 128 instance (8 chunks)
    ([0, 300, 5, 1000, 0, 0, 77, 1], 128, 64, 1),   # ... four-wave strips, offset pointers
    # direct loads at any alignment: the last slice's A chunk across K (3 of 4
    # floats kept) and B chunk across N in the last row of W (the last expert
    # has rows), fixed up in LDS
    ([5, 9, 70], 35, 19, 0),
    ([10, 20, 30], 32, 13, 1),                        # one slice, odd N, offset pointers
    ([33, 1, 64, 97], 4095, 21, 0),                   # long K with a 31-float last slice
    ([64, 2, 0, 191], 4001, 9, 1),                    # K % 4 == 1, offset pointers
]


@pytest.mark.parametrize("counts,k,n,offset", GROUPED)
def test_grouped_tiles_bit_identical(ctx, device, tile_env, counts, k, n, offset):
    rng = np.random.default_rng(len(counts) * 31 + k + n)
    e = len(counts)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    rows = int(offsets[-1])
    x = rng.standard_normal((rows, k)).astype(np.float32)
    w = (rng.standard_normal((e, k, n)) / np.sqrt(k)).astype(np.float32)
    tile_env(None)
    base = run_grouped(ctx, device, x, w, offsets, NATIVE, max_tokens=max(counts), offset=offset)
    check_grouped(base, x, w, offsets)
    for tile in TILES:
        tile_env(tile)
        y = run_grouped(ctx, device, x, w, offsets, NATIVE, max_tokens=max(counts), offset=offset)
        assert np.array_equal(y.view(np.uint32), base.view(np.uint32)), tile


@pytest.mark.parametrize("m,n,k", [(4096, 64, 256), (300, 128, 96), (500, 128, 244), (77, 40, 260),
                                   (129, 17, 33), (4096, 64, 128), (700, 128, 128), (300, 19, 4095),
                                   (64, 13, 35)])
def test_dense_tiles_bit_identical(ctx, device, tile_env, m, n, k):
    import torch
    from conftest import to_dev, to_host
    rng = np.random.default_rng(m + n + k)
    a_h = rng.standard_normal((m, k)).astype(np.float32)
    b_h = (rng.standard_normal((k, n)) / np.sqrt(k)).astype(np.float32)
    a, b = to_dev(a_h, device), to_dev(b_h, device)

    def run():
        c = torch.full((m, n), 7.0, device=device)
        ok(rr.dense_gemm(rr.DenseGemmArgs(a=rr.cview(a.data_ptr()), b=rr.cview(b.data_ptr()),
                                          c=rr.mview(c.data_ptr()), m=m, n=n, k=k, kernel=NATIVE), ctx))
        return to_host(c)
    tile_env(None)
    base = run()
    gemm_ok(base, a_h, b_h)
    for tile in TILES:
        tile_env(tile)
        assert np.array_equal(run().view(np.uint32), base.view(np.uint32)), tile
