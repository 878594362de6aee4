"""Batched, fused reconstruction of restored KV matrices into native caches (MI355X).

One :func:`reconstruct` call writes any number of restored matrices -- one
layer's K or V of one chunk each -- straight into native cache slots::

    pre-RoPE K or V = dequantize(codes) @ Q[:rank]        (per chunk)
    native slot    <- cast(RoPE(K at its original positions))   (K)
    native slot    <- cast(V)                                   (V)

The data contract is ReelCache's (reelcache/restore_kernels.py:1-37): a matrix
is ``[N, C]`` with ``N = frames * height * width`` tokens in (frame, row,
column) order and ``C = heads * head_dim``; the basis is the immutable row
matrix ``Q[R, C]`` used through its prefix ``Q[:rank]``; 8-bit codes carry an
FP32 affine per rank column, dequantized as ``float(q) * scale + offset`` with
two roundings; pictures use the ``reelcache.channel_tiles.v1`` layout; RoPE
rotates interleaved pairs ``(2j, 2j+1)``; destinations are ``BTHD``, ``THD`` or
``BHTD`` views with any strides.

Backends (same names as the reference, reelcache/restore_kernels.py:138):

* ``auto`` -- on ROCm tensors the compiled HIP kernels (``libreelcache_hip.so``,
  gfx950); on host tensors the reference backend.  If the library is missing on
  a GPU call, :class:`UnsupportedError` is raised: the reference is never run
  in its place.
* ``fused`` -- the HIP path: one basis-packing launch and one fused kernel per
  launch group (gather/dequantize -> MFMA rank-view product -> RoPE -> cast ->
  strided store).  ``two_pass`` selects the same kernels (pictures are gathered
  inside the fused kernel; there is no separate unpack pass).
* ``reference`` -- plain torch, FP64 (default) or IEEE FP32, on the jobs' device.
* ``staged`` and ``interpret`` (cuBLAS comparison and Triton interpreter in the
  reference) do not exist on this platform and raise :class:`UnsupportedError`.

Precision modes keep the reference's names and error contract
(:func:`error_bound`): ``fp32`` (FP32 matrix cores), ``fp16`` (prescaled
coefficients rounded to FP16), ``fp16x2`` (FP16 hi + lo split, two products,
near-FP32), ``bf16``.  ``tf32``/``tf32x3`` have no matrix-core form on gfx950
and raise :class:`UnsupportedError`.  A bf16 basis is accepted as well as the
canonical fp16 one (converted to fp16 with an exact power-of-two scale).

GPU work runs on a caller-provided stream (default: the current stream) after
``wait_events``; the returned :class:`RestoreHandle` records a completion event
and keeps every input, table and temporary alive until released.  The module
never changes process-wide torch settings.
"""

from __future__ import annotations

import contextlib
import math
import threading

import numpy as np
import torch

from . import _lib
from .errors import ConfigurationError, IntegrityError, StateError, UnsupportedError
from ._checks import need
from .restore_handle import RestoreHandle, _sweep_deferred, park_failed, pending_deferred
from .restore_model import (COEFFICIENT_DTYPES, LAYOUTS, OUTPUT_DTYPES, CoefficientSource, DenseSource, NativeView, PictureSource, ReconstructionJob,
                            RopePositions, RopeTable, expand_affine, wan_sections)
from .restore_reference import (_OUTPUT_FLOOR, _UNIT_ROUNDOFF, _check_compute_dtype, _check_disjoint, _gemm_gamma,
                                _native_rotation, _require_fp32_matmul, _storage_key, _validate, apply_rope_reference, dequantize,
                                error_bound, fp32_matmul_precision, reconstruct_reference, reference_coefficients,
                                reference_values, rope_cos_sin, unpack_pictures)

PRECISIONS = ("fp32", "tf32", "tf32x3", "fp16", "fp16x2", "bf16")
BACKENDS = ("auto", "reference", "fused", "two_pass", "staged", "interpret")
BASIS_DTYPES = (torch.float16, torch.bfloat16)

#: Why the compiled HIP kernels cannot be used in this process (None when they can).
HIP_IMPORT_ERROR = _lib.unavailable_reason()
HIP_AVAILABLE = HIP_IMPORT_ERROR is None
# The reference exposes the availability of its compiled kernels under these names
# (reelcache/restore_kernels.py:103-114); here they describe the HIP library.
TRITON_AVAILABLE = HIP_AVAILABLE
TRITON_IMPORT_ERROR = HIP_IMPORT_ERROR

_DEFAULT_PRECISION = "fp16x2"
_MATRIX_CORE_PRECISIONS = ("fp32", "fp16", "fp16x2", "bf16")
TILE_TOKENS = 128  # tokens per workgroup tile (4 waves x 32)
SLICE_TOKENS = 32  # tokens per tile of the channel-slice kernel (one wave's MFMA columns)
_DEFAULT_CONFIG = {"TILE_TOKENS": TILE_TOKENS, "BLOCK_N": 32, "waves": 4, "workgroups_per_cu": None,
                   "store_cost": 4.0, "fast_variant": True, "slice_variant": False, "head_pairs": True,
                   "split_rank": True, "static_scratch": False, "stream_variant": False}
# Triton tile keys the reference accepts in ``config``; they have no meaning for the HIP
# kernels and are accepted (and ignored) so that caller configurations keep working.
_REFERENCE_TILE_KEYS = {"BLOCK_M", "BLOCK_K", "num_warps", "num_stages", "N_GROUP", "PIC_T", "UNPACK_BLOCK_K",
                        "maxnreg", "_n_group"}




# ---------------------------------------------------------------------------
# HIP launch planning
# ---------------------------------------------------------------------------

_DEVICE_INFO: dict = {}


def _compute_units(device):
    if device not in _DEVICE_INFO:
        _DEVICE_INFO[device] = torch.cuda.get_device_properties(device).multi_processor_count
    return _DEVICE_INFO[device]


def device_config(device):
    """Launch configuration for a device (tile geometry of the HIP kernels)."""
    return dict(_DEFAULT_CONFIG)


def recommended_precision(device):
    """Default precision: ``fp16x2`` (FP16 hi + lo products, near-FP32 accuracy), as in the reference."""
    return _DEFAULT_PRECISION


_DTYPE_CODES = {torch.float32: _lib.DT_F32, torch.float16: _lib.DT_F16, torch.bfloat16: _lib.DT_BF16,
                torch.uint8: _lib.DT_U8}


def _source_kind(job):
    source = job.source
    if isinstance(source, PictureSource):
        return _lib.SRC_PICTURE, torch.uint8
    if isinstance(source, CoefficientSource):
        return (_lib.SRC_U8, torch.uint8) if source.quantized else (_lib.SRC_FLOAT, source.values.dtype)
    return _lib.SRC_DENSE, source.values.dtype


def _destination_address(view):
    tensor = view.tensor
    return tensor.data_ptr() + (view.element_offset() - tensor.storage_offset()) * tensor.element_size()


def _prescale_exponent(bound):
    """The FP16 modes' exact power-of-two prescale: max|coefficient| lands in (2**13, 2**14].

    Same rule as reelcache/restore_kernels.py:1386-1398 (``14 - ceil(log2(bound))``,
    clamped to [-100, 100]), evaluated exactly on the FP32 bound.
    """
    bound = float(np.float32(bound))
    if not bound > 0:
        return 0
    mantissa, exponent = math.frexp(bound)
    ceiling = exponent - 1 if mantissa == 0.5 else exponent
    return max(-100, min(100, 14 - ceiling))


def _coefficient_bound(scale, offset):
    """Upper bound of ``|pixel * scale + offset|`` over 8-bit pixels (reelcache/restore_kernels.py:1782-1785)."""
    return float(max(np.abs(offset).max(), np.abs(np.float32(255) * scale + offset).max())) * 1.0001


def _coefficient_bounds(scales, offsets, starts):
    """:func:`_coefficient_bound` of consecutive segments ``[starts[i], starts[i + 1])`` of
    concatenated fp32 affine vectors, in one vectorized pass (same fp32 arithmetic)."""
    magnitude = np.maximum(np.abs(offsets), np.abs(np.float32(255) * scales + offsets))
    return np.maximum.reduceat(magnitude, starts).astype(np.float64) * 1.0001


_STAGING_LOCK = threading.Lock()
_STAGING: dict = {}  # "slab": [pinned uint8 tensor, bytes handed out]
# Every slab that has handed out a region: captured graphs copy their descriptors from those
# regions on every replay, so a slab is never released, also after a larger one replaces it.
_RETIRED_SLABS: list = []


def reserve_capture_staging(nbytes=1 << 20):
    """Reserve pinned host memory for :func:`reconstruct` calls captured in a HIP graph.

    A captured call uploads its descriptor tables from this staging instead of a fresh pinned
    buffer (pinned allocation is not permitted while a stream captures).  Each captured call
    takes its own region, which stays owned by the capture for the life of the process (its
    graph reads it on every replay); eager calls do not use it.  Call outside capture with at
    least the bytes the captured calls need (about 10 KB per call of 14 jobs)."""
    if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
        raise ConfigurationError("reserve_capture_staging must be called before the capture")
    with _STAGING_LOCK:
        slab = _STAGING.get("slab")
        if slab is None or slab[0].numel() - slab[1] < nbytes:
            if slab is not None and slab[1] > 0:
                _RETIRED_SLABS.append(slab[0])
            _STAGING["slab"] = [_pinned_bytes(max(int(nbytes), 1 << 20)), 0]


def _pinned_bytes(nbytes):
    return torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)


def _capture_staging(nbytes):
    with _STAGING_LOCK:
        slab = _STAGING.get("slab")
        start = 0 if slab is None else (slab[1] + 255) // 256 * 256
        if slab is None or start + nbytes > slab[0].numel():
            raise ConfigurationError("a reconstruct() captured in a HIP graph needs pinned staging reserved "
                                     "beforehand: call reserve_capture_staging(nbytes) before the capture")
        slab[1] = start + nbytes
        return slab[0][start:start + nbytes]


class _Arena:
    """Host tables packed into one pinned buffer and uploaded with one copy."""

    def __init__(self):
        self._parts = []
        self._size = 0

    def add(self, array):
        """Appends a copy of ``array``; returns its byte offset (16-byte aligned)."""
        array = np.array(array, copy=True, order="C")
        offset = (self._size + 15) // 16 * 16
        self._parts.append((offset, array))
        self._size = offset + array.nbytes
        return offset

    def reserve(self, nbytes):
        """Reserves ``nbytes`` (filled later with :meth:`put`); returns the byte offset."""
        offset = (self._size + 15) // 16 * 16
        self._size = offset + nbytes
        return offset

    def put(self, offset, array):
        self._parts.append((offset, np.array(array, copy=True, order="C")))

    @property
    def size(self):
        return max(16, (self._size + 15) // 16 * 16)

    def upload(self, target):
        """Fill a pinned host buffer and copy it into ``target`` (uint8 device tensor) on the
        current stream (the caller's launch stream).  Under HIP graph capture the buffer comes
        from the staging reserved by :func:`reserve_capture_staging` (a capture cannot allocate
        pinned memory; the graph's copy node reads the buffer on every replay)."""
        if torch.cuda.is_current_stream_capturing():
            host = _capture_staging(self.size)
        else:
            host = torch.empty(self.size, dtype=torch.uint8, pin_memory=True)
        buffer = host.numpy()
        for offset, array in self._parts:
            buffer[offset:offset + array.nbytes] = array.reshape(-1).view(np.uint8)
        target[:self.size].copy_(host, non_blocking=True)
        return host


def _balanced_bounds(tile_costs, blocks_per_tile, grid):
    """int32 ``[grid + 1]`` boundaries splitting the (tile, 32-channel block) units into
    ``grid`` contiguous ranges of near-equal cost.  A tile's units share its cost, so the
    cumulative unit cost is piecewise linear over tiles: each boundary is found at tile
    granularity and placed inside its tile by linear interpolation."""
    costs = np.maximum(np.asarray(tile_costs, dtype=np.float64), 1e-9)
    tiles = len(costs)
    units = tiles * blocks_per_tile
    if units > 2 ** 31 - 1:
        raise UnsupportedError("restore launch group exceeds 2**31 work units; split the call")
    before = np.concatenate(([0.0], np.cumsum(costs * blocks_per_tile)))  # cost ahead of each tile
    targets = before[-1] * np.arange(grid + 1) / grid
    tile = np.clip(np.searchsorted(before, targets, side="right") - 1, 0, tiles - 1)
    inside = np.minimum((targets - before[tile]) / costs[tile], blocks_per_tile)
    bounds = np.rint(tile * blocks_per_tile + inside).astype(np.int64)
    bounds[0], bounds[-1] = 0, units
    return np.maximum.accumulate(bounds).astype(np.int32)


_MEMO: dict = {}


def _memo(key, build):
    """Tile tables and balanced ranges of recurring call shapes (pure functions of the key;
    callers never modify the returned arrays).  A small table, cleared when it grows."""
    value = _MEMO.get(key)
    if value is None:
        if len(_MEMO) >= 512:
            _MEMO.clear()
        value = _MEMO[key] = build()
    return value


def _config_value(config, name):
    return config.get(name, _DEFAULT_CONFIG[name])


def _tiles(job_indices, jobs, size=TILE_TOKENS):
    """int32 ``[tiles, 2]``: (job index, first token) of every ``size``-token tile of the given jobs."""
    counts = np.array([(jobs[i].tokens + size - 1) // size for i in job_indices], dtype=np.int64)
    total = int(counts.sum())
    first = np.repeat(np.cumsum(counts) - counts, counts)
    tiles = np.empty((total, 2), dtype=np.int32)
    tiles[:, 0] = np.repeat(np.asarray(job_indices, dtype=np.int32), counts)
    tiles[:, 1] = (np.arange(total, dtype=np.int64) - first) * size
    return tiles


_SLICE_BLOCKS: dict = {}


def _slice_blocks(code, max_ksteps, out_dtype, group_flags):
    """(32-channel blocks one channel-slice workgroup computes, workgroups per CU) of a variant
    ((0, 0): no slice variant)."""
    key = (code, max_ksteps, out_dtype, group_flags)
    if key not in _SLICE_BLOCKS:
        _SLICE_BLOCKS[key] = _lib.slice_blocks(code, max_ksteps, out_dtype, group_flags)
    return _SLICE_BLOCKS[key]


SLICE_JOBS = 8  # jobs whose affine one channel-slice entry stages (csrc/restore_slice.h kSliceJobs)


def _slice_heads(blocks, head_blocks):
    """Heads per slice for a slice workgroup holding ``blocks`` 32-channel blocks: pairs of heads
    (one dim block of two heads per wave), so an even count unless one head is all that fits;
    0 when not even two heads' blocks fit."""
    if head_blocks < 1 or 2 * head_blocks > blocks:
        return 0
    heads = blocks // head_blocks
    return heads - (heads & 1)


def _slice_plan(members, jobs, member_packs, pack_steps, heads, head_blocks, heads_per_slice, grid):
    """Work of one channel-slice launch (csrc/restore_slice.h): ``(tiles, entries, wg_entries)``.

    The group's jobs are ordered so that jobs sharing a basis pack are contiguous (one segment
    per pack) and cut into 32-token tiles.  The heads are split into near-equal slices of at
    most ``heads_per_slice``; a (segment, slice) pair is one tile per segment tile, every tile
    of equal cost (a workgroup computes all of its slice's blocks per tile).  The concatenated
    tiles of all pairs are split into ``grid`` near-equal ranges, each range into one entry per
    pair it touches, and entries touching more than ``SLICE_JOBS`` jobs are split further."""
    order = sorted(range(len(members)), key=lambda position: member_packs[position])
    ordered = [members[position] for position in order]
    packs = [member_packs[position] for position in order]
    tiles = _tiles(ordered, jobs, SLICE_TOKENS)
    counts = np.array([(jobs[index].tokens + SLICE_TOKENS - 1) // SLICE_TOKENS for index in ordered], np.int64)
    # Ordinal of each tile's job in the ordered list (jobs of one entry = an ordinal range).
    job_ordinal = np.repeat(np.arange(len(ordered), dtype=np.int64), counts)
    seg_tile0, seg_tiles, seg_job, seg_steps = [], [], [], []
    start = 0
    for position, index in enumerate(ordered):
        if position == 0 or packs[position] != packs[position - 1]:
            seg_tile0.append(start)
            seg_tiles.append(0)
            seg_job.append(index)
            seg_steps.append(pack_steps[packs[position]])
        seg_tiles[-1] += int(counts[position])
        start += int(counts[position])
    n_slices = -(-heads // heads_per_slice)
    sizes = np.array([heads // n_slices + (1 if s < heads % n_slices else 0) for s in range(n_slices)], np.int64)
    first_head = np.concatenate(([0], np.cumsum(sizes)[:-1]))
    segments = len(seg_tile0)
    pair_tile0 = np.repeat(np.asarray(seg_tile0, np.int64), n_slices)
    pair_units = np.repeat(np.asarray(seg_tiles, np.int64), n_slices)
    starts = np.concatenate(([0], np.cumsum(pair_units)))
    total = int(starts[-1])
    if total > 2 ** 31 - 1:
        raise UnsupportedError("restore launch group exceeds 2**31 tiles; split the call")
    bounds = np.rint(total * np.arange(grid + 1, dtype=np.float64) / grid).astype(np.int64)
    cuts = np.unique(np.concatenate((starts, bounds)))
    low, high = cuts[:-1], cuts[1:]
    pair = np.searchsorted(starts, low, side="right") - 1
    # Entries touching more than SLICE_JOBS jobs are cut at job boundaries (rare: tiny jobs).
    first_tile = pair_tile0[pair] + low - starts[pair]
    last_tile = pair_tile0[pair] + high - starts[pair] - 1
    if bool((job_ordinal[last_tile] - job_ordinal[first_tile] >= SLICE_JOBS).any()):
        extra = []
        for lo, hi, p, a, b in zip(low.tolist(), high.tolist(), pair.tolist(), first_tile.tolist(), last_tile.tolist()):
            if job_ordinal[b] - job_ordinal[a] < SLICE_JOBS:
                continue
            tile = a
            while True:
                limit = int(np.searchsorted(job_ordinal, job_ordinal[tile] + SLICE_JOBS, side="left"))
                if limit > b:
                    break
                extra.append(lo + limit - a)
                tile = limit
        cuts = np.unique(np.concatenate((cuts, np.asarray(extra, np.int64))))
        low, high = cuts[:-1], cuts[1:]
        pair = np.searchsorted(starts, low, side="right") - 1
    owner = np.searchsorted(bounds, low, side="right") - 1
    entries = np.zeros(len(low), dtype=_lib.SLICE_ENTRY_DTYPE)
    entries["tile0"] = pair_tile0[pair]
    entries["head0"] = np.tile(first_head, segments)[pair]
    entries["nh"] = np.tile(sizes, segments)[pair]
    entries["u0"] = low - starts[pair]
    entries["u1"] = high - starts[pair]
    entries["pack_job"] = np.repeat(np.asarray(seg_job, np.int64), n_slices)[pair]
    entries["pack_ksteps"] = np.repeat(np.asarray(seg_steps, np.int64), n_slices)[pair]
    wg_entries = np.searchsorted(owner, np.arange(grid + 1), side="left").astype(np.int32)
    # The kernel trusts these tables: every entry inside its pair, every tile inside the table,
    # at most SLICE_JOBS jobs per entry, slices of whole head pairs within the workgroup's blocks.
    a = entries["tile0"].astype(np.int64) + entries["u0"]
    b = entries["tile0"].astype(np.int64) + entries["u1"] - 1
    assert bool((entries["u1"] <= pair_units[pair]).all() and (entries["u0"] < entries["u1"]).all())
    assert int(b.max()) < len(tiles) and bool((job_ordinal[b] - job_ordinal[a] < SLICE_JOBS).all())
    assert int(entries["nh"].max()) <= heads_per_slice and wg_entries[-1] == len(entries)
    return tiles, entries, wg_entries


_JOB_INDEX = {name: index for index, name in enumerate(_lib.JOB_FIELDS)}
_N_FIELDS = len(_lib.JOB_FIELDS)
(_C_TOKENS, _C_RANK, _C_FRAMES, _C_GRID_H, _C_GRID_W, _C_SRC_DTYPE, _C_SRC_PTR, _C_SRC_ROW, _C_SRC_COL, _C_SCALE,
 _C_OFFSET, _C_COEF_EXP, _C_BOUND_INDEX, _C_PACK_PTR, _C_PACK_NBLOCKS, _C_EXP_INDEX, _C_DST_PTR, _C_DST_TOKEN,
 _C_DST_HEAD, _C_DST_DIM, _C_ROPE, _C_COS, _C_SIN, _C_ROPE_STRIDE, _C_ROW_T, _C_ROW_H, _C_ROW_W, _C_SEC_T, _C_SEC_H,
 _C_PIC_SLOTS, _C_PIC_PLANES, _C_PIC_COLS, _C_PIC_PLANE_STRIDE, _C_PIC_ROW_STRIDE, _C_PIC_TABLE, _C_FLAGS, _C_PAIRS,
 _C_PAIRS_BYTES, _C_DST_BYTES, _C_RESERVED) = range(40)
assert _N_FIELDS == 40 and _JOB_INDEX["pairs_ptr"] == _C_PAIRS and _JOB_INDEX["pic_table_ptr"] == _C_PIC_TABLE
_OCCUPANCY: dict = {}


def _occupancy(code, kind, max_ksteps, head_dim, out_dtype, group_flags):
    """Resident restore workgroups per CU for a variant (cached: a runtime query per variant)."""
    key = (code, kind, max_ksteps, head_dim % 32 == 0, out_dtype, group_flags)
    if key not in _OCCUPANCY:
        _OCCUPANCY[key] = _lib.occupancy(code, kind, max_ksteps, head_dim, out_dtype, group_flags)
    return _OCCUPANCY[key]


_FAST_LIMIT = 2 ** 31
# Largest ceil(rank / 16) the compiled straight-line variants cover (csrc/restore_fast.h: fast_ks);
# larger ranks run the general kernel.
_FAST_MAX_KSTEPS = {"fp16x2": 12, "fp16": 16, "bf16": 16, "fp32": 0}
_PAIRS_MAX_KSTEPS = 12
_STREAM_MAX_KSTEPS = 16  # the stream kernel keeps W (both fp16 parts) of up to 256 ranks in registers
STREAM_TOKENS = 32  # tokens per work unit of the stream kernel (csrc/restore_stream.h)
_SPLIT_MAX_KSTEPS = 32  # rank halves (RCH_GF_SPLIT_RANK): up to 512 ranks


def _fast_flags(row, job, precision):
    """``RCH_GF_*`` of one job: whether it qualifies for the straight-line restore kernel
    (csrc/restore_fast.h), and whether it rotates."""
    kind, _ = _source_kind(job)
    if isinstance(row, dict):  # a partial row by field name
        row = [row.get(name, -1 if name == "bound_index" else 0) for name in _lib.JOB_FIELDS]
    flags = row[_C_FLAGS]
    if precision == "fp32" or job.destination.head_dim % 32 or row[_C_BOUND_INDEX] >= 0:
        return 0
    if not (kind == _lib.SRC_PICTURE or (kind == _lib.SRC_U8 and flags & _lib.JF_SRC_VEC)):
        return 0
    if not flags & _lib.JF_DST_VEC or row[_C_DST_BYTES] >= _FAST_LIMIT:
        return 0
    if job.rope is None:
        return _lib.GF_FAST
    if not row[_C_PAIRS] or row[_C_PAIRS_BYTES] >= _FAST_LIMIT:
        return 0
    return _lib.GF_FAST | _lib.GF_ROPE


class _CallPlan:
    """Descriptors, basis packs and launches of one :func:`reconstruct` call on the HIP backend.

    One descriptor table and one pinned upload per call; one basis-maximum launch (non-fp16
    bases in the fp16 modes) and one packing launch for every basis of the call; then one
    fused restore launch per launch group (source kind, output dtype, head geometry and rank
    class) and one RoPE-store launch per group of dense sources.
    """

    def __init__(self, jobs, device, stream, precision, config, keepalive):
        self.jobs = jobs
        self.device = device
        self.stream = stream
        self.precision = precision
        self.code = _lib.PRECISION_CODES[precision]
        self.config = config
        self.keepalive = keepalive
        self.grids = []
        self.variants = []  # per restore launch: "pairs" / "fast" / "split" (straight-line kernel: two
        #                     heads per step, one, or rank halves), "sliced" (channel-slice kernel) or "general"

    # -- per-job descriptor fields ------------------------------------------------------------
    # Rows are plain lists indexed by the rch_job field columns (``_JOB_INDEX``); one int64
    # table is built from them at the end of the call.
    @staticmethod
    def _destination(row, job):
        view = job.destination
        address = _destination_address(view)
        strides = view.strides()
        row[_C_DST_PTR] = address
        row[_C_DST_TOKEN], row[_C_DST_HEAD], row[_C_DST_DIM] = strides
        size = view.tensor.element_size()
        row[_C_DST_BYTES] = ((job.tokens - 1) * strides[0] + (view.heads - 1) * strides[1]
                             + (view.head_dim - 1) * strides[2] + 1) * size
        per16 = 16 // size
        if (address % 16 == 0 and strides[2] == 1 and strides[0] % per16 == 0 and strides[1] % per16 == 0
                and view.head_dim % 16 == 0):
            row[_C_FLAGS] |= _lib.JF_DST_VEC

    def _rope(self, row, job, tables):
        if job.rope is None:
            return
        table = job.rope.table
        entry = tables.get(id(table))
        if entry is None:
            cos, sin = table.kernel_tables(self.device, self.stream)
            pairs = None
            if cos.stride(0) % 2 == 0 and cos.stride(1) == 1:
                pairs = table.kernel_pairs(self.device, self.stream)
                self.keepalive.append(pairs)
            vec = (cos.data_ptr() % 16 == 0 and sin.data_ptr() % 16 == 0 and cos.stride(0) % 4 == 0
                   and cos.stride(1) == 1 and sin.stride(0) == cos.stride(0))
            entry = (cos, sin, pairs, vec)
            tables[id(table)] = entry
            self.keepalive.extend((cos, sin))
        cos, sin, pairs, vec = entry
        row[_C_COS], row[_C_SIN], row[_C_ROPE_STRIDE] = cos.data_ptr(), sin.data_ptr(), cos.stride(0)
        if table.sections is None:
            row[_C_ROPE] = _lib.ROPE_DENSE
            row[_C_ROW_T] = job.rope.rows
        else:
            row[_C_ROPE] = _lib.ROPE_SEPARABLE
            row[_C_ROW_T], row[_C_ROW_H], row[_C_ROW_W] = job.rope.rows
            row[_C_SEC_T], row[_C_SEC_H] = table.sections[0], table.sections[1]
        head_dim = job.destination.head_dim
        if vec and head_dim % 16 == 0:
            row[_C_FLAGS] |= _lib.JF_ROPE_VEC
        if pairs is not None and head_dim % 32 == 0:
            row[_C_PAIRS], row[_C_PAIRS_BYTES] = pairs.data_ptr(), pairs.numel() * 4

    def run(self, stage_events=None):
        """Build the call's descriptors in four phases -- per-job fields, launch groups and their
        kernel variants, basis packs, then one device buffer and the launches -- and enqueue them."""
        jobs, precision = self.jobs, self.precision
        fp16_mode = precision in ("fp16", "fp16x2")
        arena = _Arena()
        rows = [[0] * _N_FIELDS for _ in jobs]
        arena_refs = []  # (job index, column, arena byte offset): the field becomes buffer base + offset
        affine_at = {}   # job index -> (scale, offset) arena byte offsets of its fp32 affine
        bound_jobs = self._job_fields(rows, arena_refs, affine_at, arena, fp16_mode)
        plans = self._launch_groups(rows, bound_jobs, arena)
        packs, pack_of, static = self._packs(plans, affine_at, arena)

        # Basis packs: sizes and offsets in the call buffer (or in the library's static array,
        # one group at a time, for static_scratch calls).
        fragment = 32 if precision == "fp32" else 16
        for pack in packs:
            pack["bytes"] = (pack["nblocks"] * _lib.stream_slab_bytes(pack["ksteps"]) if pack["kind"] == _lib.PACK_STREAM
                             else (pack["ksteps"] * pack["nblocks"] * 64 * fragment + 255) // 256 * 256)
        pack_total = 0
        exp_words = 0
        for pack in packs:
            pack["offset"], pack["word"] = pack_total, exp_words
            pack_total += pack["bytes"]
            if pack["kind"] == _lib.PACK_FRAGMENTS:
                exp_words += pack["nblocks"]
        if static:
            pack_total = 0
            for plan in plans:
                fragment_at, word_at = 0, 0
                for index in plan.get("packs", ()):
                    pack = packs[index]
                    pack["static_offset"], pack["static_word"] = fragment_at, word_at
                    fragment_at += pack["bytes"]
                    word_at += pack["nblocks"] if pack["kind"] == _lib.PACK_FRAGMENTS else 0
        bound_first = exp_words
        for position, index in enumerate(bound_jobs):
            rows[index][_C_BOUND_INDEX] = bound_first + position
        for index, pack_index in pack_of.items():
            pack = packs[pack_index]
            rows[index][_C_PACK_NBLOCKS] = pack["nblocks"]
            if static:
                rows[index][_C_PACK_PTR], rows[index][_C_EXP_INDEX] = pack["static_offset"], pack["static_word"]
            else:
                rows[index][_C_EXP_INDEX] = pack["word"]

        bound_tiles = _tiles(bound_jobs, jobs) if bound_jobs else None
        bound_tile_offset = arena.add(bound_tiles) if bound_jobs else None
        pack_desc = np.zeros(len(packs), dtype=_lib.PACK_DTYPE)
        packs_offset = arena.reserve(pack_desc.nbytes) if packs else None
        desc_offset = arena.reserve(len(jobs) * _N_FIELDS * 8)

        # One device buffer per call: [host tables | packed bases | scratch words].
        arena_bytes = (arena.size + 255) // 256 * 256
        scratch_words = bound_first + len(jobs)
        buffer = torch.empty(arena_bytes + pack_total + 4 * scratch_words + 256, dtype=torch.uint8, device=self.device)
        base = buffer.data_ptr()
        pack_base = base + arena_bytes
        scratch_base = pack_base + pack_total
        if bound_jobs:
            start = arena_bytes + pack_total + 4 * bound_first
            buffer[start:start + 4 * len(bound_jobs)].zero_()  # fill kernel, not a memset (graph-capture safe)
        for index, column, offset in arena_refs:
            rows[index][column] = base + offset
        for position, pack in enumerate(packs):
            entry = pack_desc[position]
            entry["src_ptr"], entry["row_stride"], entry["channels"] = pack["src"], pack["row_stride"], pack["channels"]
            entry["src_dtype"], entry["rank"], entry["kind"] = pack["dtype"], pack["rank"], pack["kind"]
            entry["ksteps"], entry["nblocks"] = pack["ksteps"], pack["nblocks"]
            entry["dst_ptr"] = pack_base + pack["offset"]
            entry["exp_ptr"] = scratch_base + 4 * pack["word"]
            if pack["kind"] == _lib.PACK_STREAM:
                entry["scale_ptr"], entry["offset_ptr"] = base + pack["scale"], base + pack["offset_table"]
        if not static:
            for index, pack_index in pack_of.items():
                rows[index][_C_PACK_PTR] = pack_base + packs[pack_index]["offset"]
        if packs:
            arena.put(packs_offset, pack_desc)
        arena.put(desc_offset, np.array(rows, dtype=np.int64))
        host = arena.upload(buffer)
        self.keepalive.extend((host, buffer))

        hip_stream = self.stream.cuda_stream
        launches = 0
        if stage_events is not None:
            stage_events.append(("start", _record(self.stream)))
        if packs and not static:
            _lib.call("rch_basis_pack", base + packs_offset, len(packs), int(max(p["nblocks"] for p in packs)),
                      int(max(p["ksteps"] for p in packs)), self.code, hip_stream)
            launches += 1
        if stage_events is not None:
            stage_events.append(("pack", _record(self.stream)))
        if bound_jobs:
            _lib.call("rch_coefficient_bound", base + desc_offset, len(jobs), base + bound_tile_offset,
                      len(bound_tiles), int(max(jobs[i].rank for i in bound_jobs)), scratch_base, hip_stream)
            launches += 1
        for plan in plans:
            variant = plan["variant"]
            if variant == "dense":
                _lib.call("rch_rope_store", base + desc_offset, len(jobs), base + plan["tiles"], plan["n_tiles"],
                          plan["channels"], plan["head_dim"], plan["out_dtype"], hip_stream)
            elif variant == "sliced":
                _lib.call("rch_restore_sliced", base + desc_offset, len(jobs), base + plan["tiles"], plan["n_tiles"],
                          base + plan["entries"], plan["n_entries"], base + plan["bounds"], plan["grid"],
                          plan["channels"], plan["head_dim"], plan["out_dtype"], self.code, plan["max_ksteps"],
                          plan["flags"], scratch_base, hip_stream)
            elif static:
                host_packs = np.ascontiguousarray(pack_desc[list(plan["packs"])])
                _lib.call("rch_restore_noalloc", host_packs.ctypes.data, len(host_packs), base + desc_offset,
                          len(jobs), base + plan["tiles"], plan["n_tiles"], base + plan["bounds"], plan["grid"],
                          plan["channels"], plan["head_dim"], plan["kind"], plan["out_dtype"], self.code,
                          plan["max_ksteps"], plan["flags"], hip_stream)
            else:
                _lib.call("rch_restore", base + desc_offset, len(jobs), base + plan["tiles"], plan["n_tiles"],
                          base + plan["bounds"], plan["grid"], plan["channels"], plan["head_dim"], plan["kind"],
                          plan["out_dtype"], self.code, plan["max_ksteps"], plan["flags"], scratch_base, hip_stream)
            launches += 1
            if stage_events is not None:
                stage_events.append((f"launch{launches}", _record(self.stream)))
        if stage_events is not None:
            stage_events.append(("fused", _record(self.stream)))
        return launches

    def _job_fields(self, rows, arena_refs, affine_at, arena, fp16_mode):
        """Phase 1: every job's own descriptor fields and the call's fp32 affine table; returns the
        float-source jobs whose fp16 prescale needs a device coefficient bound."""
        jobs = self.jobs
        tables: dict = {}
        affine_jobs, bound_jobs = [], []
        for index, job in enumerate(jobs):
            row = rows[index]
            source = job.source
            row[_C_TOKENS] = job.tokens
            row[_C_FRAMES], row[_C_GRID_H], row[_C_GRID_W] = job.grid
            row[_C_BOUND_INDEX] = -1
            self._destination(row, job)
            self._rope(row, job, tables)
            if isinstance(source, DenseSource):
                values = source.values
                row[_C_SRC_DTYPE] = _DTYPE_CODES[values.dtype]
                row[_C_SRC_PTR] = values.data_ptr()
                row[_C_SRC_ROW], row[_C_SRC_COL] = values.stride()
                continue
            basis = job.basis
            if basis.dtype not in BASIS_DTYPES or basis.stride(1) != 1:
                raise ConfigurationError("GPU kernels need a float16 (or bfloat16) basis with unit column stride")
            row[_C_RANK] = job.rank
            if isinstance(source, PictureSource):
                layout = source.layout
                pointers = [[picture.data_ptr() for picture in segment] for segment in source.pictures]
                base = min(min(segment) for segment in pointers)
                row[_C_SRC_PTR] = base
                row[_C_SRC_DTYPE] = _lib.DT_U8
                row[_C_PIC_SLOTS] = layout["channels_per_segment"]
                row[_C_PIC_PLANES] = layout["planes"]
                row[_C_PIC_COLS] = layout["grid"][0]
                row[_C_PIC_PLANE_STRIDE] = source.plane_stride
                row[_C_PIC_ROW_STRIDE] = source.row_stride
                offsets = np.array([[pointer - base for pointer in segment] for segment in pointers], dtype=np.int64)
                arena_refs.append((index, _C_PIC_TABLE, arena.add(offsets)))
                affine_jobs.append((index, source.scale, source.offset))
                continue
            values = source.values
            row[_C_SRC_PTR] = values.data_ptr()
            row[_C_SRC_DTYPE] = _DTYPE_CODES[values.dtype]
            row[_C_SRC_ROW], row[_C_SRC_COL] = values.stride()
            if source.quantized:
                affine_jobs.append((index, source.scale, source.offset))
                if values.data_ptr() % 16 == 0 and values.stride(1) == 1 and values.stride(0) % 16 == 0:
                    row[_C_FLAGS] |= _lib.JF_SRC_VEC
            elif fp16_mode:
                if source.bound is not None:
                    row[_C_COEF_EXP] = _prescale_exponent(source.bound)
                else:
                    row[_C_BOUND_INDEX] = 0  # a device bound; its scratch word is assigned with the packs
                    bound_jobs.append(index)
        if affine_jobs:
            # Every job's fp32 (scale | offset) in one host table; the fp16 modes' prescale bound
            # max(|offset|, |255 * scale + offset|) of every job in one vectorized pass.
            ranks = [jobs[index].rank for index, _, _ in affine_jobs]
            scales = np.concatenate([np.asarray(scale[:rank], dtype=np.float32)
                                     for (_, scale, _), rank in zip(affine_jobs, ranks)])
            offsets = np.concatenate([np.asarray(offset[:rank], dtype=np.float32)
                                      for (_, _, offset), rank in zip(affine_jobs, ranks)])
            starts = np.concatenate(([0], np.cumsum(ranks)[:-1])).astype(np.int64)
            table_offset = arena.add(np.concatenate((scales, offsets)))
            total = int(scales.size)
            bounds = _coefficient_bounds(scales, offsets, starts) if fp16_mode else None
            for position, (index, _, _) in enumerate(affine_jobs):
                first = int(starts[position])
                at = (table_offset + 4 * first, table_offset + 4 * (total + first))
                affine_at[index] = at
                arena_refs.append((index, _C_SCALE, at[0]))
                arena_refs.append((index, _C_OFFSET, at[1]))
                if fp16_mode:
                    rows[index][_C_COEF_EXP] = _prescale_exponent(float(bounds[position]))
        return bound_jobs

    def _launch_groups(self, rows, bound_jobs, arena):
        """Phase 2: launch groups (source kind, dtypes, head geometry, rank class, straight-line
        eligibility) and the kernel variant, grid and work tables of each."""
        jobs, precision, config = self.jobs, self.precision, self.config
        static = bool(_config_value(config, "static_scratch"))
        if static and bound_jobs:
            raise ConfigurationError("static_scratch restores hold no device coefficient bounds: float sources in "
                                     "the fp16 modes need a host bound")
        allow_fast = bool(_config_value(config, "fast_variant"))
        allow_slice = allow_fast and bool(_config_value(config, "slice_variant")) and not static
        allow_pairs = allow_fast and bool(_config_value(config, "head_pairs"))
        allow_split = bool(_config_value(config, "split_rank"))
        allow_stream = allow_fast and bool(_config_value(config, "stream_variant")) and precision == "fp16x2"
        groups: dict = {}
        for index, job in enumerate(jobs):
            flags = _fast_flags(rows[index], job, precision) if allow_fast else 0
            groups.setdefault(_group_key(job, precision) + (flags,), []).append(index)
        compute_units = _compute_units(self.device)
        passes = 2 if precision == "fp16x2" else (4 if precision == "fp32" else 1)
        store_cost = float(_config_value(config, "store_cost"))
        plans = []
        for key, members in groups.items():
            kind, group_flags = key[0], key[-1]
            first = jobs[members[0]]
            channels, head_dim = first.channels, first.destination.head_dim
            plan = {"kind": kind, "members": members, "channels": channels, "head_dim": head_dim,
                    "out_dtype": _DTYPE_CODES[first.destination.tensor.dtype]}
            plans.append(plan)
            shape = (tuple(members), tuple(jobs[i].tokens for i in members))
            if kind == _lib.SRC_DENSE:
                tiles = _memo(("tiles",) + shape, lambda: _tiles(members, jobs))
                plan.update(variant="dense", tiles=arena.add(tiles), n_tiles=len(tiles))
                continue
            job_steps = {i: (jobs[i].rank + 15) // 16 for i in members}
            max_ksteps = max(job_steps.values())
            plan["max_ksteps"] = max_ksteps
            stream = (allow_stream and group_flags & _lib.GF_FAST and kind == _lib.SRC_U8 and head_dim == 128
                      and channels % 128 == 0 and max_ksteps <= _STREAM_MAX_KSTEPS)
            stream_flags = group_flags & (_lib.GF_FAST | _lib.GF_ROPE)
            if stream and group_flags & _lib.GF_ROPE:
                if first.rope.table.sections is None:
                    stream_flags |= _lib.GF_DENSE_ROPE
                elif max(_section_pairs(jobs[i]) for i in members) > _lib.STREAM_SECTION_PAIRS:
                    stream = False  # section rows beyond the kernel's LDS table
            if stream:
                self._stream_plan(plan, stream_flags, compute_units, arena)
                continue
            if allow_slice and kind == _lib.SRC_U8 and group_flags & _lib.GF_FAST:
                head_blocks = head_dim // 32
                blocks, slice_per_cu = _slice_blocks(self.code, max_ksteps, plan["out_dtype"], group_flags)
                per_slice = _slice_heads(blocks, head_blocks)
                if per_slice >= 1 and slice_per_cu >= 1:
                    slice_grid = compute_units * slice_per_cu
                    plan["pending_slice"] = (group_flags, head_blocks, per_slice, slice_grid)
                    plan.update(variant="sliced", flags=group_flags, grid=slice_grid)
                    self.grids.append(slice_grid)
                    self.variants.append("sliced")
                    continue
            tiles = _memo(("tiles",) + shape, lambda: _tiles(members, jobs))
            if group_flags & _lib.GF_FAST and max_ksteps > _FAST_MAX_KSTEPS[precision]:
                # Beyond one wave's registers: rank halves in 8-wave workgroups (uint8 rows, up to
                # 32 rank steps), else the general kernel.
                if allow_split and kind == _lib.SRC_U8 and max_ksteps <= _SPLIT_MAX_KSTEPS:
                    group_flags = (group_flags & ~_lib.GF_HEAD_PAIRS) | _lib.GF_SPLIT_RANK
                else:
                    group_flags = 0
            if (allow_pairs and group_flags & _lib.GF_FAST and not group_flags & _lib.GF_SPLIT_RANK
                    and (channels // head_dim) % 2 == 0 and max_ksteps <= _PAIRS_MAX_KSTEPS):
                group_flags |= _lib.GF_HEAD_PAIRS  # a work unit: one dim block of two heads
            blocks_per_tile = (channels + 31) // 32 // (2 if group_flags & _lib.GF_HEAD_PAIRS else 1)
            per_cu = config.get("workgroups_per_cu") or _occupancy(self.code, kind, max_ksteps, head_dim,
                                                                   plan["out_dtype"], group_flags)
            grid = int(max(1, min(len(tiles) * blocks_per_tile, compute_units * max(1, per_cu))))

            def balanced():
                steps = np.array([job_steps[i] for i in tiles[:, 0].tolist()], dtype=np.float64)
                return _balanced_bounds(steps * passes + store_cost, blocks_per_tile, grid)
            bounds = _memo(("bounds",) + shape + (tuple(job_steps[i] for i in members), blocks_per_tile, grid, passes,
                                                  store_cost), balanced)
            plan.update(variant="general" if not group_flags & _lib.GF_FAST
                        else ("pairs" if group_flags & _lib.GF_HEAD_PAIRS
                              else ("split" if group_flags & _lib.GF_SPLIT_RANK else "fast")),
                        tiles=arena.add(tiles), n_tiles=len(tiles), bounds=arena.add(bounds), grid=grid,
                        flags=group_flags)
            self.grids.append(grid)
            self.variants.append(plan["variant"])
        return plans

    def _stream_plan(self, plan, group_flags, compute_units, arena):
        """Work tables of a stream-kernel group: units (job, head, 32-token tile) job-major, and an
        equal split of them over the resident workgroups."""
        jobs, members = self.jobs, plan["members"]
        heads = plan["channels"] // 128
        flags = group_flags | _lib.GF_STREAM
        units = [heads * ((jobs[i].tokens + STREAM_TOKENS - 1) // STREAM_TOKENS) for i in members]
        table = np.zeros((len(members) + 1, 2), dtype=np.int32)
        table[1:, 0] = np.cumsum(units)
        table[:-1, 1] = members
        total = int(table[-1, 0])
        per_cu = self.config.get("workgroups_per_cu") or _occupancy(self.code, _lib.SRC_U8, plan["max_ksteps"], 128,
                                                                    plan["out_dtype"], flags)
        grid = int(max(1, min(total, compute_units * max(1, per_cu))))
        bounds = (np.arange(grid + 1, dtype=np.int64) * total // grid).astype(np.int32)
        plan.update(variant="stream", flags=flags, tiles=arena.add(table), n_tiles=len(members),
                    bounds=arena.add(bounds), grid=grid,
                    stream_ksteps=next(size for size in (4, 8, 12, 16) if plan["max_ksteps"] <= size))
        self.grids.append(grid)
        self.variants.append("stream")

    def _packs(self, plans, affine_at, arena):
        """Phase 3: the basis packs of the call -- one per job of a stream group (its scaled slabs),
        one per distinct basis view for the other kernels (fragments of the largest rank used) --
        and the pending work tables of channel-slice groups, which index packs."""
        jobs = self.jobs
        static = bool(_config_value(self.config, "static_scratch"))
        packs: list = []
        pack_of: dict = {}
        by_basis: dict = {}
        for plan in plans:
            if plan["variant"] == "dense":
                continue
            used = []
            for index in plan["members"]:
                job = jobs[index]
                basis = job.basis
                if plan["variant"] == "stream":
                    packs.append({"kind": _lib.PACK_STREAM, "src": basis.data_ptr(), "row_stride": basis.stride(0),
                                  "channels": basis.shape[1], "dtype": _DTYPE_CODES[basis.dtype], "rank": job.rank,
                                  "ksteps": plan["stream_ksteps"], "nblocks": basis.shape[1] // 32,
                                  "scale": affine_at[index][0], "offset_table": affine_at[index][1]})
                    pack_of[index] = len(packs) - 1
                    used.append(len(packs) - 1)
                    continue
                key = (basis.data_ptr(), basis.stride(0), basis.shape[1], basis.dtype)
                position = by_basis.get(key)
                if position is None:
                    position = by_basis[key] = len(packs)
                    packs.append({"kind": _lib.PACK_FRAGMENTS, "src": key[0], "row_stride": key[1], "channels": key[2],
                                  "dtype": _DTYPE_CODES[key[3]], "rank": 0, "nblocks": 2 * ((key[2] + 63) // 64)})
                packs[position]["rank"] = max(packs[position]["rank"], job.rank)
                pack_of[index] = position
                if position not in used:
                    used.append(position)
            plan["packs"] = used
        for pack in packs:
            if pack["kind"] == _lib.PACK_FRAGMENTS:
                pack["ksteps"] = (pack["rank"] + 15) // 16
        for plan in plans:
            pending = plan.pop("pending_slice", None)
            if pending is None:
                continue
            group_flags, head_blocks, per_slice, slice_grid = pending
            members = plan["members"]
            ksteps = [pack["ksteps"] for pack in packs]
            tiles, entries, wg_entries = _slice_plan(members, jobs, [pack_of[i] for i in members], ksteps,
                                                     plan["channels"] // plan["head_dim"], head_blocks, per_slice,
                                                     slice_grid)
            plan.update(tiles=arena.add(tiles), n_tiles=len(tiles), entries=arena.add(entries),
                        n_entries=len(entries), bounds=arena.add(wg_entries))
        return packs, pack_of, static


def _record(stream):
    event = torch.cuda.Event(enable_timing=True)
    event.record(stream)
    return event


def _rank_class(precision, job):
    """The compiled variant's register-resident rank steps for this job (see ``pick_ks`` in
    csrc/restore_kernel.h); jobs of one class share a launch, so the product loop is fixed."""
    if job.rank is None:
        return 0
    steps = (job.rank + 15) // 16
    # The 16-bit modes add the rank-halves variants' classes (24, 32; fp16x2 also 16).
    classes = (4, 8) if precision == "fp32" else (2, 4, 8, 12, 16, 24, 32)
    for size in classes:
        if steps <= size:
            return size
    return -1  # chunked


def _group_key(job, precision=None):
    kind, dtype = _source_kind(job)
    rope = None if job.rope is None else job.rope.table.sections is None  # dense tables apart from separable
    return (kind, dtype, job.destination.tensor.dtype, job.destination.head_dim, job.channels,
            _rank_class(precision, job) if precision is not None else 0, rope)


def _section_pairs(job):
    """(cos, sin) pairs of a separable table that the stream kernel stages in LDS for a job: every
    row of each section the job's grid can reach."""
    sections = job.rope.table.sections
    frames, height, width = job.grid
    return frames * sections[0] + height * sections[1] + width * sections[2]


def _resolve_backend(backend, cuda):
    """``backend`` resolved for jobs on a GPU (``cuda=True``) or host tensors; never a silent fallback."""
    if backend == "reference" or (backend == "auto" and not cuda):
        return "reference"
    if backend in ("staged", "interpret"):
        raise UnsupportedError(f"the {backend!r} backend (cuBLAS comparison / Triton interpreter) does not exist on "
                               "ROCm; use 'fused' or 'reference'")
    if not cuda:
        raise UnsupportedError(f"the {backend} backend needs GPU tensors; use 'reference'")
    reason = _lib.unavailable_reason()
    if reason is not None:
        if backend == "auto":
            raise UnsupportedError(f"backend='auto' cannot run the HIP reconstruction: {reason}. The FP64 reference "
                                   "is never substituted silently; pass backend='reference' to request it explicitly.")
        raise UnsupportedError(f"the {backend} backend is unavailable: {reason}")
    return "fused"


def _resolve_precision(precision, device):
    if precision == "auto":
        precision = recommended_precision(device)
    if precision not in _MATRIX_CORE_PRECISIONS:
        raise UnsupportedError(f"precision {precision!r} has no matrix-core form on gfx950 (no TF32 MFMA); "
                               f"use one of {_MATRIX_CORE_PRECISIONS}")
    return precision


def _merged_config(config):
    merged = dict(_DEFAULT_CONFIG)
    for name, value in (config or {}).items():
        if name in _DEFAULT_CONFIG:
            merged[name] = value
        elif name not in _REFERENCE_TILE_KEYS:
            raise ConfigurationError(f"unknown restore config key {name!r}")
    if merged["workgroups_per_cu"] is not None and (type(merged["workgroups_per_cu"]) is not int
                                                    or merged["workgroups_per_cu"] < 1):
        raise ConfigurationError("workgroups_per_cu must be a positive integer")
    return merged


class _null(contextlib.nullcontext):
    """A context that does nothing (host execution has no stream to enter)."""


def _on(stream):
    return torch.cuda.stream(stream) if stream is not None else contextlib.nullcontext()


def _execution_stream(device, stream, wait_events):
    """The stream a call runs on (``None`` for host execution), after ``wait_events``."""
    if device.type != "cuda":
        need(stream is None and not wait_events, "host execution takes no GPU stream or events")
        return None
    stream = torch.cuda.current_stream(device) if stream is None else stream
    need(isinstance(stream, torch.cuda.Stream) and stream.device == device,
         "stream must be a torch.cuda.Stream on the jobs' device")
    for event in wait_events:
        stream.wait_event(event)
    return stream


def _matrix_flops(jobs):
    return sum(2 * job.tokens * job.rank * job.channels for job in jobs if job.rank)


class _FusedCall:
    """The HIP execution of one :func:`reconstruct` call: one :class:`_CallPlan` for the jobs the
    kernels rotate (or write unrotated) and, with ``native_rope``, one for the pre-RoPE K that the
    engine's callable rotates before the copy into its slot."""

    def __init__(self, device, stream, precision, config, keepalive, stage_events, stats):
        self.device, self.stream, self.precision = device, stream, precision
        self.config, self.keepalive, self.stage_events, self.stats = config, keepalive, stage_events, stats
        stats.update(grids=[], variants=[])

    def launch(self, jobs):
        plan = _CallPlan(list(jobs), self.device, self.stream, self.precision, self.config, self.keepalive)
        self.stats["launches"] += plan.run(self.stage_events)
        self.stats["grids"].extend(plan.grids)
        self.stats["variants"].extend(plan.variants)

    def rotate_natively(self, jobs, native_rope, native_rope_dtype):
        """Exact path: pre-RoPE K into THD temporaries (a dense source already in the rotation
        dtype is used as is), the engine's rotation, then a copy into each slot."""
        need(native_rope_dtype is None or native_rope_dtype in OUTPUT_DTYPES,
             "native RoPE input dtype must be bfloat16, float16 or float32")
        inputs, staged = [], []
        for job in jobs:
            view = job.destination
            shape = (job.tokens, view.heads, view.head_dim)
            dtype = native_rope_dtype or view.tensor.dtype
            if isinstance(job.source, DenseSource) and job.source.values.dtype == dtype:
                inputs.append(job.source.values.reshape(shape))
                continue
            temporary = torch.empty(shape, dtype=dtype, device=view.tensor.device)
            self.keepalive.append(temporary)
            staged.append(ReconstructionJob(job.source, NativeView(temporary, "THD"), job.grid, job.basis, job.rank,
                                            None, job.label))
            inputs.append(temporary)
        if staged:
            self.launch(staged)
        for job, values in zip(jobs, inputs):
            rotated = _native_rotation(native_rope, values, job, values.dtype)
            self.keepalive.append(rotated)
            job.destination.slot(job.tokens).copy_(rotated)


def reconstruct(jobs, *, backend="auto", precision="auto", stream=None, wait_events=(), native_rope=None,
                native_rope_dtype=None, config=None, compute_dtype=torch.float64, stage_events=None):
    """Reconstruct restored matrices into their native cache slots.

    ``jobs``: :class:`ReconstructionJob` sequence; one call should cover all
    restored chunks of a layer (K and V) so each launch group (jobs sharing
    source kind, output dtype and head geometry) is one fused launch.
    ``backend``: see the module docstring.  ``precision``: one of
    :data:`PRECISIONS` or ``"auto"`` (:func:`recommended_precision`).
    ``stream``: torch stream to run on (default: current), after ``wait_events``.
    ``native_rope``: optional ``(pre_rope[N, H, D], job) -> post_rope`` used instead
    of the built-in rotation for jobs with RoPE.  ``config``: launch overrides
    (``workgroups_per_cu``, ``store_cost``, kernel-variant switches).  ``stage_events``: optional
    list receiving ``(stage, event)`` timing events ("start", "pack", "launch<n>" after the n-th
    launch of the call, "fused", "rope_store").

    Returns a :class:`RestoreHandle`; destinations are valid after its event.
    """
    _sweep_deferred()
    jobs, device = _validate(jobs)
    need(backend in BACKENDS, f"backend must be one of {BACKENDS}")
    need(precision == "auto" or precision in PRECISIONS, f"precision must be 'auto' or one of {PRECISIONS}")
    need(native_rope is None or callable(native_rope), "native_rope must be callable")
    stats = {"jobs": len(jobs), "matrices": len(jobs), "flops": _matrix_flops(jobs), "launches": 0}
    if not jobs:
        stats.update(backend="none", precision=None)
        return RestoreHandle(event=None, stream=None, keepalive=None, stats=stats)
    resolved = _resolve_backend(backend, device.type == "cuda")
    if resolved == "reference":
        _check_compute_dtype(compute_dtype, device)
        label = str(compute_dtype)
    else:
        precision = label = _resolve_precision(precision, device)
    stream = _execution_stream(device, stream, wait_events)
    keepalive = [tensor for job in jobs for tensor in job.tensors()]
    stats.update(backend=resolved, precision=label, picture_path="fused_gather" if resolved == "fused" else resolved)
    if resolved == "reference":
        with _on(stream):
            reconstruct_reference(jobs, compute_dtype=compute_dtype, native_rope=native_rope,
                                  native_rope_dtype=native_rope_dtype)
    else:
        call = _FusedCall(device, stream, precision, _merged_config(config), keepalive, stage_events, stats)
        native = [job for job in jobs if native_rope is not None and job.rope is not None]
        fused = [job for job in jobs if native_rope is None or job.rope is None]
        try:
            with torch.cuda.stream(stream):
                if fused:
                    call.launch(fused)
                if native:
                    call.rotate_natively(native, native_rope, native_rope_dtype)
        except BaseException:
            park_failed(stream, keepalive)
            raise
    event = None
    if stream is not None:
        event = torch.cuda.Event()
        event.record(stream)
    return RestoreHandle(event=event, stream=stream, keepalive=keepalive, stats=stats)


# Warm-up: :mod:`reelcache_amd.restore_warmup` (it calls back into :func:`reconstruct`).
from .restore_warmup import WARMUP_ROPE_MODES, WARMUP_SOURCES, WarmupShape, warmup  # noqa: E402


__all__ = [
    "BACKENDS", "HIP_AVAILABLE", "HIP_IMPORT_ERROR", "LAYOUTS", "OUTPUT_DTYPES", "PRECISIONS", "TRITON_AVAILABLE",
    "TRITON_IMPORT_ERROR",
    "CoefficientSource", "DenseSource", "NativeView", "PictureSource", "ReconstructionJob",
    "RestoreHandle", "RopePositions", "RopeTable",
    "apply_rope_reference", "dequantize", "device_config", "error_bound", "expand_affine", "fp32_matmul_precision",
    "pending_deferred",
    "reconstruct",
    "reconstruct_reference", "recommended_precision", "reference_coefficients", "reference_values",
    "reserve_capture_staging", "rope_cos_sin",
    "unpack_pictures", "wan_sections",
    "WARMUP_ROPE_MODES", "WARMUP_SOURCES", "WarmupShape", "warmup",
]
