"""The C ABI library loads and exports every symbol ``include/reelcache_hip.h`` declares (no GPU needed)."""

import re
from pathlib import Path

from reelcache_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "reelcache_hip.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rch_[a-z0-9_]+)\s*\(", text)))


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.library()
    names = declared_functions()
    assert "rch_restore" in names and len(names) >= 10
    missing = [name for name in names if not hasattr(lib, name)]
    assert not missing, missing


def test_abi_version_and_descriptor_layout():
    lib = _lib.library()
    assert lib.rch_abi_version() == _lib.ABI_VERSION
    assert lib.rch_job_size() == _lib.JOB_DTYPE.itemsize == 40 * 8
    assert lib.rch_pack_size() == _lib.PACK_DTYPE.itemsize == 12 * 8
    assert lib.rch_fragment_bytes(_lib.PRECISION_CODES["fp16x2"]) == 16
    assert lib.rch_fragment_bytes(_lib.PRECISION_CODES["fp32"]) == 32
    assert lib.rch_fit_matrix_size() == _lib.FIT_DTYPE.itemsize == 16 * 8
    assert _lib.QUANTIZE_DTYPE.itemsize == 8 * 8
