"""Build recipe for libraggedroute_amd.so (gfx950).

HIP sources (*.hip) are compiled with hipcc for gfx950 only; host-only C++
sources (*.cpp) with g++ against the HIP headers. Objects go to _build/ at the
repository root and the shared library is written in-tree next to this file so
that it travels with the repository snapshot.

    python raggedroute_amd/build.py          # full rebuild

The same build also links libraggedroute_amd_stamps.so, an instrumentation
copy whose strip.hip is compiled with -DRR_PHASE_STAMPS (phase stamps of the
chain launch, read by `bench.py --phase-stamps`); nothing loads it unless
RR_LIBRARY names it.

Run it as a script (or load it by path): importing the package loads the
library, which does not exist yet on a fresh checkout.
"""
from __future__ import annotations

import concurrent.futures
import datetime
import json
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO / "include"
BUILD = REPO / "_build"
LIB_NAME = "libraggedroute_amd.so"
LIB_PATH = PKG_DIR / LIB_NAME
STAMPS_PATH = PKG_DIR / "libraggedroute_amd_stamps.so"
# sources compiled a second time, with this define, for the instrumentation copy
STAMPED_SOURCES = ("strip.hip",)
STAMPS_DEFINE = "-DRR_PHASE_STAMPS"
# Source revision and toolchain of the last build (git-ignored like the
# library, and shipped beside it): benchmark records name what they ran.
BUILD_INFO = PKG_DIR / "build_info.json"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
ARCH = "gfx950"

HIP_FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-fPIC",
    # Packed FP32 instructions stay disabled: scalar/float2 code only.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # HIP contracts a*b+c into FMA across statements by default; the kernels
    # rely on separately rounded multiply and add where they follow the
    # reference's FP32 loops (naive GEMMs, unpermute, input fills).
    "-ffp-contract=off",
    "-Wall",
    "-Wno-unused-command-line-argument",
]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-D__HIP_PLATFORM_AMD__"]


def _hipcc() -> str:
    path = ROCM / "bin" / "hipcc"
    if not path.exists():
        raise RuntimeError(f"hipcc not found at {path}")
    return str(path)


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(
            "command failed (%d): %s\n%s%s" % (proc.returncode, " ".join(cmd), proc.stdout, proc.stderr)
        )


def _compile(src: Path, stamps: bool = False) -> Path:
    obj = BUILD / (src.name + (".stamps.o" if stamps else ".o"))
    includes = [f"-I{INCLUDE}", f"-I{CSRC}"]
    if src.suffix == ".hip":
        extra = [STAMPS_DEFINE] if stamps else []
        cmd = [_hipcc(), *HIP_FLAGS, *extra, *includes, "-c", str(src), "-o", str(obj)]
    else:
        cmd = ["g++", *CXX_FLAGS, *includes, f"-I{ROCM / 'include'}", "-c", str(src), "-o", str(obj)]
    _run(cmd)
    return obj


def _git(*args: str) -> str | None:
    try:
        proc = subprocess.run(["git", "-C", str(REPO), *args], capture_output=True, text=True, timeout=30)
    except (OSError, subprocess.SubprocessError):
        return None
    return proc.stdout.strip() if proc.returncode == 0 else None


def _build_info() -> dict:
    hipcc = subprocess.run([_hipcc(), "--version"], capture_output=True, text=True)
    version = next((line.strip() for line in hipcc.stdout.splitlines() if line.startswith("HIP version")), None)
    status = _git("status", "--porcelain", "--untracked-files=no")
    return {"git_sha": _git("rev-parse", "HEAD"), "git_dirty": None if status is None else bool(status),
            "built_utc": datetime.datetime.now(datetime.timezone.utc).strftime("%Y-%m-%dT%H:%M:%SZ"),
            "hip": version, "arch": ARCH, "hip_flags": " ".join(HIP_FLAGS)}


def _link(objects: list[Path], out: Path) -> None:
    tmp = out.with_suffix(".so.tmp")
    _run([_hipcc(), "-shared", f"--offload-arch={ARCH}", "-fPIC", "-o", str(tmp),
          *map(str, objects), f"-L{ROCM / 'lib'}", "-lamdhip64",
          f"-Wl,-rpath,{ROCM / 'lib'}"])
    shutil.move(str(tmp), str(out))


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile every source and link the shared library (and its phase-stamp
    instrumentation copy); returns the library's path."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    if not sources:
        raise RuntimeError(f"no sources under {CSRC}")
    stamped = [src for src in sources if src.name in STAMPED_SOURCES]
    jobs = jobs or min(8, os.cpu_count() or 1)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        futures = [pool.submit(_compile, src) for src in sources]
        stamp_futures = {src.name: pool.submit(_compile, src, True) for src in stamped}
        objects = [f.result() for f in futures]
        stamp_objects = {name: f.result() for name, f in stamp_futures.items()}
    _link(objects, LIB_PATH)
    _link([stamp_objects.get(src.name, obj) for src, obj in zip(sources, objects)], STAMPS_PATH)
    BUILD_INFO.write_text(json.dumps(_build_info(), indent=1) + "\n")
    if verbose:
        print(f"built {LIB_PATH} (and {STAMPS_PATH.name})")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
