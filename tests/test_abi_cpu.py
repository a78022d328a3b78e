"""CPU checks of the drop-in boundary: the kernel library loads without a GPU, exports
every entry point the C header declares, the ctypes table binds exactly those
entry points, and host-side rules restated in Python agree with the library's own
exports.  No kernel is launched here."""

from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from thintensor_amd import _lib
from thintensor_amd import build as hip_build

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "thintensor_hip.h"


def declared_symbols() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return set(re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\*?\s*(tt_[a-z0-9_]+)\s*\(", text, flags=re.M))


@pytest.fixture(scope="module")
def lib():
    if not _lib.library_path().exists():
        pytest.skip("kernel library not built (run __graft_entry__.build())")
    return _lib.load(build_if_missing=False)


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert len(syms) >= 30
    assert {"tt_int4_scaled_matvec", "tt_mxfp4_selected_matvec", "tt_moe_router_matvec_topk", "tt_add_rms_norm",
            "tt_matvec_argmax"} <= syms


def test_library_exports_every_declared_symbol(lib):
    missing = [s for s in sorted(declared_symbols()) if not hasattr(lib, s)]
    assert not missing, f"declared in {HEADER.name} but not exported: {missing}"


def test_dynamic_symbol_table_matches_header(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.library_path())], capture_output=True, text=True,
                         check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln and ln.split()[-1].startswith("tt_")}
    assert exported == declared_symbols()


def test_ctypes_table_covers_header():
    assert set(_lib.SIGNATURES) == declared_symbols()


def test_version_and_error_channel(lib):
    assert lib.tt_version() >= 1
    assert isinstance(lib.tt_last_error(), bytes)


def test_lanes_rule_matches_python_restatement(lib):
    from oracle.decode_ref import lanes

    for chunks in list(range(1, 300)) + [90, 160, 256, 1024]:
        for L in (1, 2, 4, 8):
            if L > 1 and chunks % L:
                continue
            assert lib.tt_gemv_lanes_per_row(chunks, L) == lanes(32 * chunks, L), (chunks, L)


def test_argument_errors_are_reported_without_a_gpu(lib):
    """Validation happens before any launch: bad shapes come back as TT_ERR_INVALID
    with a message, so the Python wrapper can raise ValueError."""
    rc = lib.tt_int4_scaled_matvec(None, 0, None, 0, 0, 0, 0, 0, None, 0, None, 0, 16, 30, 128, None)
    assert rc != 0
    assert lib.tt_last_error()


def test_build_flags_disable_packed_fp32():
    flags = " ".join(hip_build.HIP_FLAGS)
    assert "-packed-fp32-ops" in flags and "--offload-arch=gfx950" in flags
