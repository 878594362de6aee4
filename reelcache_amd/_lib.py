"""ctypes binding of ``libreelcache_hip.so`` (the C ABI declared in ``include/reelcache_hip.h``).

The library is built ahead of time (``reelcache_amd.csrc.build``) and loaded on
first use.  There is no fallback: when it is missing or was built for another
ABI, every GPU entry point raises :class:`UnsupportedError` with the reason.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import numpy as np

from .errors import ConfigurationError, UnsupportedError

LIBRARY = Path(__file__).resolve().with_name("libreelcache_hip.so")
ABI_VERSION = 12

# Status codes (RCH_E_*).
OK, E_CONFIG, E_UNSUPPORTED, E_LAUNCH = 0, 1, 2, 3

# Precision codes follow the reference's PRECISIONS order (reelcache/restore_kernels.py:137).
PRECISION_CODES = {"fp32": 0, "tf32": 1, "tf32x3": 2, "fp16": 3, "fp16x2": 4, "bf16": 5}
DT_F32, DT_F16, DT_BF16, DT_U8, DT_F64 = 0, 1, 2, 3, 4
SRC_FLOAT, SRC_U8, SRC_PICTURE, SRC_DENSE = 0, 1, 2, 3
ROPE_NONE, ROPE_SEPARABLE, ROPE_DENSE = 0, 1, 2
JF_SRC_VEC, JF_DST_VEC, JF_ROPE_VEC, JF_PIC_VEC4 = 1, 2, 4, 8
GF_FAST, GF_ROPE, GF_HEAD_PAIRS, GF_SPLIT_RANK, GF_STREAM, GF_DENSE_ROPE = 1, 2, 4, 8, 16, 32
STREAM_SECTION_PAIRS = 2048

# rch_job field order (40 x int64).
JOB_FIELDS = (
    "tokens", "rank", "frames", "grid_h", "grid_w",
    "src_dtype", "src_ptr", "src_row_stride", "src_col_stride",
    "scale_ptr", "offset_ptr", "coef_exp", "bound_index",
    "pack_ptr", "pack_nblocks", "basis_exp_index",
    "dst_ptr", "dst_token_stride", "dst_head_stride", "dst_dim_stride",
    "rope", "cos_ptr", "sin_ptr", "rope_row_stride",
    "row_t", "row_h", "row_w", "sec_t", "sec_h",
    "pic_slots", "pic_planes", "pic_grid_cols", "pic_plane_stride", "pic_row_stride",
    "pic_table_ptr", "flags", "pairs_ptr", "pairs_bytes", "dst_bytes", "reserved",
)
JOB_DTYPE = np.dtype([(name, "<i8") for name in JOB_FIELDS])
PACK_FIELDS = ("src_ptr", "src_dtype", "row_stride", "rank", "channels", "dst_ptr", "ksteps", "nblocks",
               "kind", "exp_ptr", "scale_ptr", "offset_ptr")
PACK_FRAGMENTS, PACK_STREAM = 0, 1


def stream_slab_bytes(ksteps: int) -> int:
    """Bytes of one (job, 32-channel block) slab of an RCH_PACK_STREAM pack."""
    return (ksteps * 2048 + 128 + 16 + 255) // 256 * 256
PACK_DTYPE = np.dtype([(name, "<i8") for name in PACK_FIELDS])
# rch_fit_matrix field order (16 x int64).
FIT_FIELDS = ("src_ptr", "src_dtype", "rows", "src_stride", "basis_ptr", "basis_stride", "rank", "coef_ptr",
              "coef_stride", "gram_ptr", "gram_stride", "absmax_ptr", "extrema_ptr", "energy_ptr", "partial_ptr",
              "resid_ptr")
FIT_DTYPE = np.dtype([(name, "<i8") for name in FIT_FIELDS])
QUANTIZE_FIELDS = ("values_ptr", "rows", "cols", "stride", "affine_ptr", "codes_ptr", "code_stride", "reserved")
QUANTIZE_DTYPE = np.dtype([(name, "<i8") for name in QUANTIZE_FIELDS])
GAUSS_FIELDS = ("dst_ptr", "rows", "cols", "stride", "seed", "reserved0", "reserved1", "reserved2")
GAUSS_DTYPE = np.dtype([(name, "<i8") for name in GAUSS_FIELDS])

_i, _i64, _p = ctypes.c_int, ctypes.c_int64, ctypes.c_void_p
_SIGNATURES = {
    "rch_abi_version": ([], _i),
    "rch_job_size": ([], _i),
    "rch_pack_size": ([], _i),
    "rch_last_error": ([], ctypes.c_char_p),
    "rch_fragment_bytes": ([_i], _i),
    "rch_basis_pack": ([_p, _i, _i64, _i64, _i, _p], _i),
    "rch_coefficient_bound": ([_p, _i, _p, _i, _i, _p, _p], _i),
    "rch_restore": ([_p, _i, _p, _i, _p, _i, _i, _i, _i, _i, _i, _i, _i, _p, _p], _i),
    "rch_restore_occupancy": ([_i, _i, _i, _i, _i, _i, ctypes.POINTER(_i)], _i),
    "rch_restore_pair": ([_p, _i, _p, _i, _i, _p, _i, _i, _i, _i, _i, _i, _i, _i, _p, _p], _i),
    "rch_restore_pair_occupancy": ([_i, _i, _i, _i, _i, _i, ctypes.POINTER(_i)], _i),
    "rch_rope_store": ([_p, _i, _p, _i, _i, _i, _i, _p], _i),
    "rch_staged_unpack": ([_p, _i, _p, _i, _p, _p, _i64, _i, _i, _i, _i, _p, _p], _i),
    "rch_staged_store": ([_p, _i, _p, _i, _p, _p, _i64, _i, _i, _i, _i, _p, _p], _i),
    "rch_restore_noalloc": ([_p, _i, _p, _i, _p, _i, _p, _i, _i, _i, _i, _i, _i, _i, _i, _p], _i),
    "rch_fit_matrix_size": ([], _i),
    "rch_fit_absmax": ([_p, _i, _i, _i64, _i, _p], _i),
    "rch_fit_gram": ([_p, _i, _i, _i, _p], _i),
    "rch_fit_project": ([_p, _i, _i, _i64, _i, _i, _p], _i),
    "rch_fit_residual": ([_p, _i, _i, _i64, _i, _p], _i),
    "rch_column_extrema": ([_p, _i64, _i, _i64, _p, _p], _i),
    "rch_quantize": ([_p, _i64, _i, _i64, _p, _p, _p, _i64, _p], _i),
    "rch_quantize_batched": ([_p, _i, _i64, _p], _i),
    "rch_cholesky_inverse": ([_p, _p, _p, _i, _i, _p], _i),
    "rch_fit_gaussian": ([_p, _i, _i64, _p], _i),
}
# Further entry points registered by other modules are bound when present.
_OPTIONAL_SIGNATURES: dict = {}

_LOCK = threading.Lock()
_STATE: dict = {}


def _load():
    if not LIBRARY.exists():
        raise UnsupportedError(
            f"the HIP kernel library {LIBRARY.name} is not built; run reelcache_amd.csrc.build (hipcc, gfx950)")
    try:
        lib = ctypes.CDLL(str(LIBRARY))
    except OSError as error:
        raise UnsupportedError(f"the HIP kernel library could not be loaded: {error}") from error
    for name, (arguments, result) in _SIGNATURES.items():
        try:
            function = getattr(lib, name)
        except AttributeError as error:
            raise UnsupportedError(f"{LIBRARY.name} does not export {name}; rebuild it") from error
        function.argtypes, function.restype = arguments, result
    for name, (arguments, result) in _OPTIONAL_SIGNATURES.items():
        function = getattr(lib, name, None)
        if function is not None:
            function.argtypes, function.restype = arguments, result
    if lib.rch_abi_version() != ABI_VERSION:
        raise UnsupportedError(f"{LIBRARY.name} has ABI {lib.rch_abi_version()}, expected {ABI_VERSION}; rebuild it")
    if (lib.rch_job_size() != JOB_DTYPE.itemsize or lib.rch_pack_size() != PACK_DTYPE.itemsize
            or lib.rch_fit_matrix_size() != FIT_DTYPE.itemsize):
        raise UnsupportedError(f"{LIBRARY.name} descriptor layout differs from this package; rebuild it")
    return lib


def library():
    """The loaded library (raises :class:`UnsupportedError` when unavailable)."""
    with _LOCK:
        if "lib" in _STATE:
            return _STATE["lib"]
        if "error" in _STATE:
            raise UnsupportedError(_STATE["error"])
        try:
            _STATE["lib"] = _load()
        except UnsupportedError as error:
            _STATE["error"] = str(error)
            raise
        return _STATE["lib"]


def unavailable_reason() -> str | None:
    """Why the kernel library cannot be used in this process, or None."""
    try:
        library()
    except UnsupportedError as error:
        return str(error)
    return None


def register(signatures: dict) -> None:
    """Declare further entry points (bound on first load, or now if already loaded)."""
    _OPTIONAL_SIGNATURES.update(signatures)
    lib = _STATE.get("lib")
    if lib is not None:
        for name, (arguments, result) in signatures.items():
            function = getattr(lib, name, None)
            if function is not None:
                function.argtypes, function.restype = arguments, result


def call(name: str, *arguments) -> None:
    """Calls an entry point; maps a nonzero status to the declared error classes."""
    lib = library()
    function = getattr(lib, name, None)
    if function is None:
        raise UnsupportedError(f"{LIBRARY.name} does not export {name}; rebuild it")
    status = function(*arguments)
    if status == OK:
        return
    message = (lib.rch_last_error() or b"").decode(errors="replace")
    if status == E_CONFIG:
        raise ConfigurationError(message)
    if status == E_UNSUPPORTED:
        raise UnsupportedError(message)
    raise RuntimeError(f"HIP launch failed: {message}")


def occupancy(precision: int, source_kind: int, max_ksteps: int, head_dim: int, out_dtype: int,
              group_flags: int) -> int:
    """Resident workgroups per CU of the restore variant for these arguments."""
    blocks = ctypes.c_int(0)
    call("rch_restore_occupancy", precision, source_kind, max_ksteps, head_dim, out_dtype, group_flags,
         ctypes.byref(blocks))
    return blocks.value


def pair_occupancy(precision: int, source_kind: int, ksteps0: int, ksteps1: int, head_dim: int,
                   out_dtype: int) -> int:
    """Resident workgroups per CU of the pair kernel for two head-pair groups (a RoPE group of
    ``ksteps0`` rank steps, then a plain one of ``ksteps1``); 0 when none is compiled for them."""
    blocks = ctypes.c_int(0)
    call("rch_restore_pair_occupancy", precision, source_kind, ksteps0, ksteps1, head_dim, out_dtype,
         ctypes.byref(blocks))
    return blocks.value


