"""Builds libdlhip.so (the gfx950 backend) in-tree with hipcc.

    python -m dolittle_amd.build          # or dolittle_amd.build.build()

Every translation unit is compiled with -ffp-contract=off (every FMA in this
project is explicit, matching the reference's --fmad=false build,
CMakeLists.txt:167) and without packed FP32 instructions.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIBRARY = os.path.join(HERE, "libdlhip.so")
SOURCES = ["runtime.cpp", "ops.hip", "packed.hip", "qwen3.hip", "sampler.hip", "prefill.hip", "nla.hip", "sequence.hip", "archive.cpp"]
ARCH = os.environ.get("DL_OFFLOAD_ARCH", "gfx950")


def _hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if candidate and (os.path.sep not in candidate or os.path.exists(candidate)):
            return candidate
    raise RuntimeError("hipcc not found")


def _flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall", "-Wno-unused-function", "-Wno-unused-result",
        f"-I{os.path.join(HERE, '..', 'include')}",
    ]


def _compile(source: str) -> str:
    src = os.path.join(CSRC, source)
    obj = os.path.join(BUILD, source + ".o")
    cmd = [_hipcc(), *_flags(), "-c", src, "-o", obj]
    if source.endswith(".cpp"):
        cmd = [_hipcc(), *_flags(), "-x", "hip", "-c", src, "-o", obj]
    result = subprocess.run(cmd, capture_output=True, text=True)
    noise = [l for l in result.stderr.splitlines() if "packed-fp32-ops" not in l and l.strip()]
    if result.returncode != 0:
        raise RuntimeError(f"compiling {source} failed:\n" + "\n".join(noise))
    if noise and os.environ.get("DL_BUILD_VERBOSE"):
        print("\n".join(noise), file=sys.stderr)
    return obj


def build(jobs: int | None = None) -> str:
    """Compiles every HIP source for gfx950 and links libdlhip.so; returns its path."""
    os.makedirs(BUILD, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 1)
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objects = list(pool.map(_compile, SOURCES))
    tmp = LIBRARY + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objects]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError("linking libdlhip.so failed:\n" + result.stderr)
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build())
