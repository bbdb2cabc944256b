"""Builds libullis_hip.so in-tree with hipcc for gfx950.

Every .hip source under csrc/ is compiled separately (in parallel) and linked
into ullis_amd/libullis_hip.so. Flags:
  -ffp-contract=off                 keeps SGD updates as two roundings, like the
                                    reference's Rust f32 arithmetic;
  -target-feature -packed-fp32-ops  no packed fp32 VALU instructions.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import pathlib
import shutil
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
LIB = HERE / "libullis_hip.so"
ARCH = os.environ.get("ULLIS_HIP_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
CFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def _compile(src: pathlib.Path) -> pathlib.Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [HIPCC, *CFLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        msg = "\n".join(l for l in proc.stderr.splitlines() if "packed-fp32-ops" not in l)
        raise RuntimeError(f"hipcc failed for {src.name}:\n{msg}")
    return obj


def _stale(src: pathlib.Path) -> bool:
    """An object is out of date when it is older than its source or any header."""
    obj = BUILD / (src.stem + ".o")
    if not obj.exists():
        return True
    t = obj.stat().st_mtime
    headers = list(CSRC.glob("*.hpp")) + list((HERE.parent / "include").glob("*.h"))
    return any(p.stat().st_mtime > t for p in [src, *headers])


def build(verbose: bool = True, incremental: bool = False) -> pathlib.Path:
    """Compiles every source (incremental: only sources whose object is out of
    date) and links the library."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    todo = [s for s in sources if _stale(s)] if incremental else sources
    jobs = min(max(len(todo), 1), int(os.environ.get("MAX_JOBS", "8")))
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        list(pool.map(_compile, todo))
    objs = [BUILD / (s.stem + ".o") for s in sources]
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build(incremental="--incremental" in sys.argv[1:])
