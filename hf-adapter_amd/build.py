"""Build librwkv7mi.so (gfx950) in-tree with hipcc.

Usage: python hf-adapter_amd/build.py [--jobs N]

Every *.hip / *.cpp under csrc/ is compiled to an object in _build/ and linked
into rwkv7mi/librwkv7mi.so next to the Python package that loads it.  The
build always recompiles (the driver's build check must exercise hipcc).
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OUT_DIR = HERE / "_build"
LIB = HERE / "rwkv7mi" / "librwkv7mi.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    # Packed FP32 instructions are disabled for every HIP translation unit.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def _compile(src: Path) -> Path:
    obj = OUT_DIR / (src.stem + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stdout}\n{proc.stderr}")
    return obj


def _stale(src: Path) -> bool:
    obj = OUT_DIR / (src.stem + ".o")
    if not obj.exists():
        return True
    newest = max([src.stat().st_mtime] + [h.stat().st_mtime for h in CSRC.glob("*.h")]
                 + [(HERE.parent / "include" / "rwkv7mi.h").stat().st_mtime])
    return newest > obj.stat().st_mtime


def build(jobs: int | None = None, verbose: bool = True, incremental: bool = False) -> Path:
    """Compile every source (``incremental``: only those older than their
    sources or headers) and link the library."""
    OUT_DIR.mkdir(exist_ok=True)
    sources = sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))
    if not sources:
        raise RuntimeError("no sources under csrc/")
    todo = [s for s in sources if _stale(s)] if incremental else sources
    jobs = jobs or min(max(len(todo), 1), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_compile, todo))
    objs = [OUT_DIR / (s.stem + ".o") for s in sources]
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources", flush=True)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--incremental", action="store_true", help="recompile only stale objects")
    args = ap.parse_args()
    try:
        build(args.jobs, incremental=args.incremental)
    except RuntimeError as exc:
        print(exc, file=sys.stderr)
        sys.exit(1)
