"""Shared pytest configuration.

`-m "not gpu"`: oracle against the golden vectors, host-side contracts of the
C ABI (dispatch, argument and workspace checks that return before any device
call) and symbol exports. `-m gpu`: parity of the HIP library against the
oracle, called through the C ABI on a gfx950 device.
"""
from __future__ import annotations

import json
import math
import sys
from pathlib import Path

import numpy as np
import pytest
import torch  # noqa: F401  (before the library: torch's bundled HIP runtime serves the process)

REPO = Path(__file__).resolve().parent.parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

GOLDEN = REPO / "tests" / "golden" / "kat.json"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 (MI355X) device")


def _num(v):
    if isinstance(v, str):
        return {"nan": math.nan, "inf": math.inf, "-inf": -math.inf}[v]
    if isinstance(v, list):
        return [_num(x) for x in v]
    return v


@pytest.fixture(scope="session")
def kat():
    data = json.loads(GOLDEN.read_text())

    def get(name, field):
        return _num(data[name][field])

    get.raw = data
    return get


# ---------------------------------------------------------------- GPU helpers

def _gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:  # pragma: no cover
        return False


@pytest.fixture(scope="session")
def device():
    if not _gpu_available():
        pytest.skip("no ROCm GPU visible")
    import torch
    import raggedroute_amd as rr
    status, arch = rr.query_current_device_architecture()
    assert status.ok(), status.message
    if arch != rr.DeviceArchitecture.kGfx950:
        pytest.skip(f"device is not gfx950 ({arch.name})")
    return torch.device("cuda:0")


@pytest.fixture()
def ctx(device):
    """RuntimeContext on torch's current stream with the resolved architecture."""
    import torch
    import raggedroute_amd as rr
    stream = torch.cuda.current_stream(device).cuda_stream
    return rr.RuntimeContext(stream=stream, architecture=int(rr.DeviceArchitecture.kGfx950))


class Guarded:
    """Device buffer with 256-byte redzones (canary 0xA5) and a poisoned payload
    (0xCD), the scheme of reference include/raggedroute/correctness/guarded_buffer.h:38-125."""

    REDZONE = 256
    CANARY = 0xA5
    POISON = 0xCD

    def __init__(self, n: int, dtype, device, offset_elems: int = 0):
        import torch
        self.dtype = np.dtype(dtype)
        self.n = n
        self.offset = offset_elems * self.dtype.itemsize
        self.payload = n * self.dtype.itemsize
        total = self.REDZONE * 2 + self.offset + self.payload
        self.raw = torch.full((total,), self.POISON, dtype=torch.uint8, device=device)
        self.raw[: self.REDZONE] = self.CANARY
        self.raw[self.REDZONE + self.offset + self.payload:] = self.CANARY
        if self.offset:
            self.raw[self.REDZONE:self.REDZONE + self.offset] = self.CANARY

    @property
    def ptr(self) -> int:
        return self.raw.data_ptr() + self.REDZONE + self.offset

    def write(self, values) -> None:
        import torch
        arr = np.ascontiguousarray(np.asarray(values, dtype=self.dtype).reshape(-1))
        assert arr.size == self.n
        view = self.raw[self.REDZONE + self.offset: self.REDZONE + self.offset + self.payload]
        view.copy_(torch.from_numpy(arr.view(np.uint8).copy()))

    def read(self) -> np.ndarray:
        import torch
        torch.cuda.synchronize()
        view = self.raw[self.REDZONE + self.offset: self.REDZONE + self.offset + self.payload]
        return view.cpu().numpy().view(self.dtype).copy()

    def canaries_intact(self) -> bool:
        import torch
        torch.cuda.synchronize()
        host = self.raw.cpu().numpy()
        head = host[: self.REDZONE + self.offset]
        tail = host[self.REDZONE + self.offset + self.payload:]
        return bool((head == self.CANARY).all() and (tail == self.CANARY).all())


@pytest.fixture()
def guarded(device):
    def make(n, dtype, values=None, offset_elems=0):
        g = Guarded(n, dtype, device, offset_elems)
        if values is not None:
            g.write(values)
        return g
    return make


def to_dev(arr, device):
    import torch
    return torch.from_numpy(np.ascontiguousarray(arr)).to(device)


def to_host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()
