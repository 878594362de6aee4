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
    assert lib.rch_slice_entry_size() == _lib.SLICE_ENTRY_DTYPE.itemsize == 8 * 4


def test_header_struct_fields_match_the_binding():
    """Field order of the int64 / int32 descriptor structs in the header == the numpy dtypes."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    for struct, fields in (("rch_job", _lib.JOB_FIELDS), ("rch_slice_entry", _lib.SLICE_ENTRY_FIELDS)):
        body = re.search(r"typedef struct " + struct + r" \{(.*?)\}", text, flags=re.S).group(1)
        names = []
        for declaration in body.split(";"):
            declaration = re.sub(r"\[\d+\]", "", declaration).strip()
            if declaration:
                names.extend(part.strip().split()[-1] for part in declaration.split(","))
        assert len(names) == len(fields), struct
        assert [n for n in names if not n.startswith("reserved")] == [f for f in fields if not f.startswith("reserved")]
