"""Builds libspkv2_mi355x.so (runtime + HIP kernels for gfx950) in-tree.

    python -m spinnv2_amd.build            # incremental
    python -m spinnv2_amd.build --force    # rebuild everything

Every source under spinnv2_amd/csrc is compiled by hipcc for gfx950 only and
linked into spinnv2_amd/lib/libspkv2_mi355x.so.  Packed-FP32 instruction
selection is disabled (-packed-fp32-ops) for all device code.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB_DIR = PKG / "lib"
LIB = LIB_DIR / "libspkv2_mi355x.so"
INCLUDE = ROOT / "include"
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build the MI355X backend)")


COMMON_FLAGS = [
    "-std=c++17",
    "-O3",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}",
]


def sources() -> list[Path]:
    return sorted(list(CSRC.rglob("*.cpp")) + list(CSRC.rglob("*.hip")))


def headers() -> list[Path]:
    return sorted(list(CSRC.rglob("*.hpp")) + list(INCLUDE.glob("*.h")))


def _obj_for(src: Path) -> Path:
    rel = src.relative_to(CSRC)
    return BUILD / (str(rel).replace(os.sep, "__") + ".o")


def _compile(src: Path, force: bool, newest_header: float) -> tuple[Path, str]:
    obj = _obj_for(src)
    if not force and obj.exists():
        mtime = obj.stat().st_mtime
        if mtime >= src.stat().st_mtime and mtime >= newest_header:
            return obj, ""
    cmd = [hipcc(), "-x", "hip", *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"compile failed: {src}\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    warnings = "\n".join(
        line for line in (proc.stdout + proc.stderr).splitlines()
        if "packed-fp32-ops" not in line and "target-feature" not in line and line.strip()
    )
    return obj, warnings


def build(force: bool = False, jobs: int | None = None, verbose: bool = False) -> Path:
    BUILD.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    newest_header = max((h.stat().st_mtime for h in headers()), default=0.0)
    srcs = sources()
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 16)
    objs: list[Path] = []
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        for obj, warnings in pool.map(lambda s: _compile(s, force, newest_header), srcs):
            objs.append(obj)
            if warnings and verbose:
                print(warnings, file=sys.stderr)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", str(tmp), *map(str, objs),
           "-Wl,-Bsymbolic", "-Wl,--no-undefined", "-lamdhip64"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB)
    return LIB


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--force", action="store_true")
    ap.add_argument("-j", "--jobs", type=int, default=None)
    ap.add_argument("-v", "--verbose", action="store_true")
    args = ap.parse_args()
    print(build(force=args.force, jobs=args.jobs, verbose=args.verbose))


if __name__ == "__main__":
    main()
