"""Build libgadeon_hip.so (the HIP kernels + C ABI) for gfx950 with hipcc.

Every translation unit in gadeon_amd/csrc is compiled to an object under
gadeon_amd/_build and linked into gadeon_amd/libgadeon_hip.so, in-tree, so
the library travels with the source tree.  Usage:

    python -m gadeon_amd.build [--force] [-j N]
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libgadeon_hip.so"
INCLUDE = PKG.parent / "include"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# Packed-FP32 instructions are disabled for all device code: hipcc -O3 would
# otherwise form v_pk_{add,mul,fma}_f32 from ordinary float code.
CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _stale(obj: Path, src: Path) -> bool:
    if not obj.exists():
        return True
    deps = [src, *CSRC.glob("*.h"), INCLUDE / "gadeon_hip.h"]
    t = obj.stat().st_mtime
    return any(d.stat().st_mtime > t for d in deps)


def _compile(src: Path, force: bool) -> Path:
    obj = BUILD / (src.stem + ".o")
    if force or _stale(obj, src):
        cmd = [HIPCC, *CFLAGS, "-I", str(INCLUDE), "-c", str(src), "-o", str(obj)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src.name}:\n{r.stdout}\n{r.stderr}")
        # hipcc's host pass does not know the device-only feature flag; that
        # warning is expected, anything else is shown.
        noise = "is not a recognized feature for this target"
        msgs = [l for l in r.stderr.splitlines() if l.strip() and noise not in l]
        if msgs:
            print("\n".join(msgs), file=sys.stderr)
    return obj


def build(force: bool = False, jobs: int | None = None) -> Path:
    """Compile every csrc/*.hip and link libgadeon_hip.so; returns its path."""
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 2)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, force), srcs))
    if force or not LIB.exists() or any(o.stat().st_mtime > LIB.stat().st_mtime for o in objs):
        tmp = LIB.with_suffix(".so.tmp")
        cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs),
               "-o", str(tmp)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
        os.replace(tmp, LIB)
    return LIB


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--force", action="store_true")
    ap.add_argument("-j", type=int, default=None)
    a = ap.parse_args()
    print(build(force=a.force, jobs=a.j))


if __name__ == "__main__":
    main()
