"""Build the gfx950 kernel library ``libthintensor_hip.so`` in-tree with hipcc.

The library is a plain C-ABI shared object (no torch types in any signature); the
Python host side loads it with ctypes.  Every HIP source is compiled for gfx950
only, with packed-fp32 instructions disabled and no floating-point contraction
(every fused multiply-add in the kernels is written explicitly).
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_NAME = "libthintensor_hip.so"
LIB_PATH = PKG_DIR / LIB_NAME

ARCH = "gfx950"
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the HIP kernel library cannot be built")


def _compile(src: Path, obj: Path) -> tuple[Path, str]:
    cmd = [hipcc(), *HIP_FLAGS, "-I", str(CSRC), "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr[-6000:]}")
    return obj, proc.stderr


def _stale(src: Path, obj: Path, headers_mtime: float) -> bool:
    if not obj.exists():
        return True
    t = obj.stat().st_mtime
    return src.stat().st_mtime > t or headers_mtime > t


def build(verbose: bool = False, jobs: int | None = None, incremental: bool = False) -> Path:
    """Compile every source under csrc/ and link the shared library.  With
    ``incremental`` only sources newer than their object (or older than a changed
    header) are recompiled."""
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))
    if not sources:
        raise RuntimeError("no kernel sources found")
    jobs = jobs or min(8, os.cpu_count() or 4)
    headers = list(CSRC.glob("*.h")) + list((PKG_DIR.parent / "include").glob("*.h"))
    headers_mtime = max((h.stat().st_mtime for h in headers), default=0.0)
    objs: list[Path] = []
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        futs = []
        for s in sources:
            obj = BUILD_DIR / (s.stem + ".o")
            if incremental and not _stale(s, obj, headers_mtime):
                objs.append(obj)
                continue
            futs.append(pool.submit(_compile, s, obj))
        for fut in futs:
            obj, log = fut.result()
            objs.append(obj)
            if verbose and log.strip():
                filtered = "\n".join(ln for ln in log.splitlines() if "packed-fp32-ops" not in ln)
                if filtered.strip():
                    print(filtered, file=sys.stderr)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr[-4000:]}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv, incremental="--incremental" in sys.argv)
    print(path)
