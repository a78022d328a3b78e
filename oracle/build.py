"""Build recipe for the CPU oracle (test infrastructure only).

Compiles oracle/tt_oracle.c with gcc into oracle/_build/libtt_oracle.so.  No
floating-point contraction (-ffp-contract=off) and no fast-math: the restatement
relies on IEEE binary32 semantics with explicit fmaf().
"""

from __future__ import annotations

import os
import subprocess
from pathlib import Path

ORACLE_DIR = Path(__file__).resolve().parent
BUILD_DIR = ORACLE_DIR / "_build"
LIB_PATH = BUILD_DIR / "libtt_oracle.so"
SOURCES = [ORACLE_DIR / "tt_oracle.c"]
CFLAGS = ["-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math", "-fopenmp", "-Wall"]


def build() -> Path:
    BUILD_DIR.mkdir(exist_ok=True)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = ["gcc", *CFLAGS, "-o", str(tmp), *map(str, SOURCES), "-lm"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{proc.stderr[-4000:]}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def ensure_built() -> Path:
    newest = max(s.stat().st_mtime for s in SOURCES)
    if not LIB_PATH.exists() or LIB_PATH.stat().st_mtime < newest:
        return build()
    return LIB_PATH


if __name__ == "__main__":
    print(build())
