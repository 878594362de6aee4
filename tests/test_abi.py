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


def test_header_struct_fields_match_the_binding():
    """Field order of the int64 descriptor structs in the header == the numpy dtypes."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    for struct, fields in (("rch_job", _lib.JOB_FIELDS), ("rch_pack", _lib.PACK_FIELDS)):
        body = re.search(r"typedef struct " + struct + r" \{(.*?)\}", text, flags=re.S).group(1)
        names = []
        for declaration in body.split(";"):
            declaration = re.sub(r"\[\d+\]", "", declaration).strip()
            if declaration:
                names.extend(part.strip().split()[-1] for part in declaration.split(","))
        assert len(names) == len(fields), struct
        assert [n for n in names if not n.startswith("reserved")] == [f for f in fields if not f.startswith("reserved")]


def test_header_constants_match_the_binding():
    """Status, precision, dtype, source, RoPE, job-flag and group-flag codes of the header ==
    the values the ctypes binding writes into descriptors and passes to the entry points."""
    defines = {name: int(value) for name, value in
               re.findall(r"#define (RCH_[A-Z0-9_]+) (\d+)\b", HEADER.read_text())}
    expected = {"RCH_E_CONFIG": _lib.E_CONFIG, "RCH_E_UNSUPPORTED": _lib.E_UNSUPPORTED, "RCH_E_LAUNCH": _lib.E_LAUNCH,
                "RCH_DT_F32": _lib.DT_F32, "RCH_DT_F16": _lib.DT_F16, "RCH_DT_BF16": _lib.DT_BF16,
                "RCH_DT_U8": _lib.DT_U8, "RCH_DT_F64": _lib.DT_F64,
                "RCH_SRC_FLOAT": _lib.SRC_FLOAT, "RCH_SRC_U8": _lib.SRC_U8, "RCH_SRC_PICTURE": _lib.SRC_PICTURE,
                "RCH_SRC_DENSE": _lib.SRC_DENSE,
                "RCH_ROPE_NONE": _lib.ROPE_NONE, "RCH_ROPE_SEPARABLE": _lib.ROPE_SEPARABLE,
                "RCH_ROPE_DENSE": _lib.ROPE_DENSE,
                "RCH_JF_SRC_VEC": _lib.JF_SRC_VEC, "RCH_JF_DST_VEC": _lib.JF_DST_VEC,
                "RCH_JF_ROPE_VEC": _lib.JF_ROPE_VEC, "RCH_JF_PIC_VEC4": _lib.JF_PIC_VEC4,
                "RCH_GF_FAST": _lib.GF_FAST, "RCH_GF_ROPE": _lib.GF_ROPE, "RCH_GF_HEAD_PAIRS": _lib.GF_HEAD_PAIRS,
                "RCH_GF_SPLIT_RANK": _lib.GF_SPLIT_RANK, "RCH_GF_STREAM": _lib.GF_STREAM,
                "RCH_GF_DENSE_ROPE": _lib.GF_DENSE_ROPE}
    expected.update({"RCH_PREC_" + name.upper(): code for name, code in _lib.PRECISION_CODES.items()})
    assert {name: defines.get(name) for name in expected} == expected
