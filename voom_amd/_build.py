"""Compile libvoom_hip.so for gfx950 with hipcc, in-tree.

The library is built next to this file so that it travels with the source
tree; nothing is installed.  ``build()`` always recompiles.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_NAME = "libvoom_hip.so"
LIB_PATH = PKG_DIR / LIB_NAME
# bench-only probe kernels (csrc/bench), linked against LIB_NAME
CALIB_LIB_PATH = PKG_DIR / "libvoom_calibrate.so"
ARCH = "gfx950"

# Packed-fp32 instructions are disabled for every device pass (the flag is
# unknown to the host pass, which only warns).
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the ROCm toolchain is required to build libvoom_hip.so")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))


def _run(cmd: list[str]) -> str:
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{err}")
    return err


def _link(cc: str, objs: list[Path], out: Path, extra: list[str]) -> str:
    tmp = out.with_suffix(".so.tmp")
    err = _run([cc, *HIP_FLAGS, "-shared", "-o", str(tmp), *map(str, objs), *extra])
    os.replace(tmp, out)
    return err


def build(verbose: bool = False) -> Path:
    """Compile every kernel source into one shared library and return its path;
    the bench-only probes (csrc/bench) go into libvoom_calibrate.so beside it.

    Each source is compiled to an object in its own hipcc process (in
    parallel; every translation unit holds its kernels and their launchers,
    so no relocatable device code is needed), then the objects are linked."""
    cc = hipcc()
    srcs = sources()
    bench_srcs = sorted((CSRC / "bench").glob("*.hip"))
    every = srcs + bench_srcs
    jobs = max(1, min(len(every), int(os.environ.get("MAX_JOBS", "") or os.cpu_count() or 1)))
    with tempfile.TemporaryDirectory(prefix="voom_build_") as tdir:
        objs = [Path(tdir) / f"{i}_{src.name}.o" for i, src in enumerate(every)]
        cmds = [[cc, *HIP_FLAGS, "-c", "-o", str(obj), str(src)] for src, obj in zip(every, objs)]
        if verbose:
            for cmd in cmds:
                print(" ".join(cmd), flush=True)
        with ThreadPoolExecutor(max_workers=jobs) as pool:
            errs = list(pool.map(_run, cmds))
        errs.append(_link(cc, objs[:len(srcs)], LIB_PATH, []))
        errs.append(_link(cc, objs[len(srcs):], CALIB_LIB_PATH,
                          [f"-L{PKG_DIR}", "-lvoom_hip", "-Wl,-rpath,$ORIGIN"]))
    if verbose:
        for err in errs:
            if err.strip():
                print(err, file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
