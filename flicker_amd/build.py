"""Build recipe for libflicker_hip.so (hipcc, gfx950 only).

Every ``csrc/*.hip`` file is compiled to an object in parallel, then linked into
``flicker_amd/libflicker_hip.so`` next to this file, so the library travels with
the source tree.  Run ``python -m flicker_amd.build`` or ``__graft_entry__.build()``.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import pathlib
import shutil
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
BUILD = PKG / "_build"
LIB = PKG / "libflicker_hip.so"
ARCH = "gfx950"

# Packed float32 VALU ops are turned off for all device code; -O3 would otherwise form them.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", f"-I{INCLUDE}", f"-I{CSRC}",
                "-Wall", "-Wno-unused-function"]


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(exe):
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build flicker_amd")
    return exe


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = False, jobs: int | None = None) -> pathlib.Path:
    """Compile every csrc/*.hip for gfx950 and link libflicker_hip.so; returns its path."""
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    BUILD.mkdir(exist_ok=True)
    cc = hipcc()
    objects = [BUILD / (src.stem + ".o") for src in sources]
    jobs = jobs or min(len(sources), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        futures = [pool.submit(_run, [cc, *COMMON_FLAGS, *DEVICE_FLAGS, "-c", str(src), "-o", str(obj)],
                               verbose) for src, obj in zip(sources, objects)]
        for f in futures:
            f.result()
    tmp = LIB.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)], verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
