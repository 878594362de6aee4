"""HIP launch planning of :func:`reelcache_amd.restore_kernels.reconstruct`.

A call's jobs become one int64 descriptor table (``rch_job``, include/reelcache_hip.h), the work
tables of each launch group, the basis-pack descriptors and the launches that read them, all
in one device buffer uploaded with one copy from pinned memory.

Planning is split so that a call costs little host time when its geometry recurs (a restore of
many layers of one model):

* :class:`_JobDesc` -- everything a job contributes that does not change between calls, computed
  once per job object (jobs are immutable): its static descriptor row, alignment rules, the
  tensors whose addresses are read at each call, its affine arrays and devices;
* :class:`_Layout` -- the launch groups, kernel variants, grids, work tables, basis packs and
  the byte layout of the call buffer, memoized by the call's geometry (the jobs' static rows,
  alignment bits, and which jobs share a destination view, a basis or a RoPE table);
* :func:`run_call` -- per call: read the addresses, copy the layout's template bytes into
  pinned staging, write the pointer columns, affine tables and prescale exponents, upload, launch.
"""

from __future__ import annotations

import math
import threading

import numpy as np
import torch

from . import _lib
from .errors import ConfigurationError, UnsupportedError
from .restore_model import CoefficientSource, DenseSource, PictureSource, settle_table_uploads
from .restore_reference import _require_fp32_matmul

TILE_TOKENS = 128  # tokens per workgroup tile (4 waves x 32)
BASIS_DTYPES = (torch.float16, torch.bfloat16)
_DEFAULT_CONFIG = {"TILE_TOKENS": TILE_TOKENS, "BLOCK_N": 32, "waves": 4, "workgroups_per_cu": None,
                   "store_cost": None, "fast_variant": True, "head_pairs": True,
                   "split_rank": True, "static_scratch": False, "stream_variant": False,
                   "pair_launch": True}
DEFAULT_MERGED = dict(_DEFAULT_CONFIG)  # the merged configuration of calls without overrides (never modified)

_DEVICE_INFO: dict = {}

# A work unit's cost for the balanced split of a launch is store_cost + rank steps x MFMA passes.
# The constant is the unit's work besides its products (tile entry share, epilogue, stores, fetch,
# barrier) in units of one 16-rank product step, fitted on MI355X to the measured time of a
# rank-128 RoPE unit against a rank-192 plain unit (CausVid K and V: 44 / 51 us per launch in
# fp16x2, 42 / 42 us in fp16).  A pair launch mixes both, so the split must weigh them right.
_STORE_COST = {"fp16x2": 48.0, "fp16": 120.0, "bf16": 120.0, "fp32": 4.0, "tf32": 4.0, "tf32x3": 4.0}


def _compute_units(device):
    if device not in _DEVICE_INFO:
        _DEVICE_INFO[device] = torch.cuda.get_device_properties(device).multi_processor_count
    return _DEVICE_INFO[device]



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
    if torch.cuda.is_available():
        settle_table_uploads()
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
    """Byte layout of a call buffer's host tables: arrays added (copied) or regions reserved, each
    16-byte aligned."""

    def __init__(self):
        self._parts = []
        self._size = 0

    def add(self, array):
        """Appends a copy of ``array``; returns its byte offset (16-byte aligned)."""
        offset = self.reserve(np.asarray(array).nbytes)
        self._parts.append((offset, np.array(array, copy=True, order="C")))
        return offset

    def reserve(self, nbytes):
        """Reserves ``nbytes`` (written per call); returns the byte offset."""
        offset = (self._size + 15) // 16 * 16
        self._size = offset + nbytes
        return offset

    def parts(self):
        return list(self._parts)

    @property
    def size(self):
        return max(16, (self._size + 15) // 16 * 16)


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


def _fast_eligibility(kind, head_dim, rotates, row, precision):
    """``RCH_GF_*`` of one job: whether it qualifies for the straight-line restore kernel
    (csrc/restore_fast.h) -- 16-bit MFMA precision, head_dim a multiple of 32, no device bound,
    16-byte aligned code rows (or pictures) and slot, slot and RoPE table within 32-bit offsets --
    and whether it rotates (which needs the interleaved table)."""
    flags = int(row[_C_FLAGS])
    if precision == "fp32" or head_dim % 32 or row[_C_BOUND_INDEX] >= 0:
        return 0
    if not (kind == _lib.SRC_PICTURE or (kind == _lib.SRC_U8 and flags & _lib.JF_SRC_VEC)):
        return 0
    if not flags & _lib.JF_DST_VEC or row[_C_DST_BYTES] >= _FAST_LIMIT:
        return 0
    if not rotates:
        return _lib.GF_FAST
    if not row[_C_PAIRS] or row[_C_PAIRS_BYTES] >= _FAST_LIMIT:
        return 0
    return _lib.GF_FAST | _lib.GF_ROPE


def _fast_flags(row, job, precision):
    """:func:`_fast_eligibility` of a job and a descriptor row (a list by column, or a dict by
    field name with the missing fields zero and ``bound_index`` -1)."""
    if isinstance(row, dict):
        row = [row.get(name, -1 if name == "bound_index" else 0) for name in _lib.JOB_FIELDS]
    return _fast_eligibility(_source_kind(job)[0], job.destination.head_dim, job.rope is not None, row, precision)


def _record(stream):
    event = torch.cuda.Event(enable_timing=True)
    event.record(stream)
    return event


# ---------------------------------------------------------------------------
# Per-job descriptors
# ---------------------------------------------------------------------------


class _JobDesc:
    """What one job contributes to every call that includes it, computed once per job object.

    ``row`` holds every ``rch_job`` field that does not depend on addresses (a placeholder 1 in
    ``pairs_ptr`` marks a job that reads the interleaved RoPE table); ``key`` is the job's share
    of a call's geometry key.  Addresses (destination, source, basis, tables) are read from the
    referenced tensors at every call."""

    __slots__ = ("affine", "basis", "basis_key", "channels", "dst", "dst_shift", "dst_vec_rule", "dtype",
                 "exponent", "grid", "head_dim", "host_bound", "key", "key_id", "kind", "out_dtype", "pictures",
                 "rank", "rope_kind", "row", "section_pairs", "src", "src_vec_rule", "table", "tokens", "pic_vec_rule")

    def __init__(self, job):
        view, source = job.destination, job.source
        tensor = view.tensor
        row = np.zeros(_N_FIELDS, dtype=np.int64)
        self.tokens, self.grid = job.tokens, job.grid
        self.head_dim, self.channels = view.head_dim, view.channels
        row[_C_TOKENS] = self.tokens
        row[_C_FRAMES], row[_C_GRID_H], row[_C_GRID_W] = self.grid
        row[_C_BOUND_INDEX] = -1
        self._destination(row, view, tensor)
        self._rope(row, job)
        self.kind, dtype = _source_kind(job)
        self.dtype = _DTYPE_CODES[dtype]
        self.src = self.pictures = self.basis = self.basis_key = self.affine = self.host_bound = None
        self.src_vec_rule, self.rank, self.exponent = False, 0, 0
        self.pic_vec_rule = False
        if isinstance(source, DenseSource):
            self.src = source.values
            row[_C_SRC_DTYPE] = self.dtype
            row[_C_SRC_ROW], row[_C_SRC_COL] = self.src.stride()
        else:
            self._factorized(row, job, source)
        self.row = row
        pictures = None if self.pictures is None else (len(source.pictures), len(source.pictures[0]))
        self.key = (row.tobytes(), self.kind, self.dtype, self.out_dtype, self.head_dim, self.channels, self.rope_kind,
                    self.basis_key, self.host_bound is None, pictures, self.section_pairs)
        self.key_id = _KEY_IDS.setdefault(self.key, len(_KEY_IDS))

    def _destination(self, row, view, tensor):
        size = tensor.element_size()
        strides = view.strides()
        row[_C_DST_TOKEN], row[_C_DST_HEAD], row[_C_DST_DIM] = strides
        row[_C_DST_BYTES] = ((self.tokens - 1) * strides[0] + (view.heads - 1) * strides[1]
                             + (self.head_dim - 1) * strides[2] + 1) * size
        per16 = 16 // size
        # 16-byte stores also need a 16-byte aligned slot address, checked at each call.
        self.dst_vec_rule = (strides[2] == 1 and strides[0] % per16 == 0 and strides[1] % per16 == 0
                             and self.head_dim % 16 == 0)
        self.dst = tensor
        self.dst_shift = (view.element_offset() - tensor.storage_offset()) * size
        self.out_dtype = _DTYPE_CODES[tensor.dtype]

    def _rope(self, row, job):
        self.table, self.rope_kind, self.section_pairs = None, None, 0
        if job.rope is None:
            return
        table = self.table = job.rope.table
        # Device copies are one block (csrc reads row-major [rows, pairs] planes and the interleaved
        # pairs), every part 256-byte aligned: row stride = pairs.
        row[_C_ROPE_STRIDE] = table.pairs
        if table.sections is None:
            self.rope_kind = "dense"
            row[_C_ROPE], row[_C_ROW_T] = _lib.ROPE_DENSE, job.rope.rows
        else:
            self.rope_kind = "separable"
            row[_C_ROPE] = _lib.ROPE_SEPARABLE
            row[_C_ROW_T], row[_C_ROW_H], row[_C_ROW_W] = job.rope.rows
            row[_C_SEC_T], row[_C_SEC_H] = table.sections[0], table.sections[1]
            self.section_pairs = sum(extent * pairs for extent, pairs in zip(self.grid, table.sections))
        if table.pairs % 4 == 0 and self.head_dim % 16 == 0:
            row[_C_FLAGS] |= _lib.JF_ROPE_VEC
        if self.head_dim % 32 == 0:
            row[_C_PAIRS], row[_C_PAIRS_BYTES] = 1, table.rows * table.pairs * 8

    def _factorized(self, row, job, source):
        basis = job.basis
        if basis.dtype not in BASIS_DTYPES or basis.stride(1) != 1:
            raise ConfigurationError("GPU kernels need a float16 (or bfloat16) basis with unit column stride")
        self.basis, self.rank = basis, job.rank
        self.basis_key = (basis.stride(0), basis.shape[1], _DTYPE_CODES[basis.dtype])
        row[_C_RANK] = job.rank
        if isinstance(source, PictureSource):
            layout = source.layout
            self.pictures = [picture for segment in source.pictures for picture in segment]
            row[_C_SRC_DTYPE] = _lib.DT_U8
            row[_C_PIC_SLOTS], row[_C_PIC_PLANES] = layout["channels_per_segment"], layout["planes"]
            row[_C_PIC_COLS] = layout["grid"][0]
            row[_C_PIC_PLANE_STRIDE], row[_C_PIC_ROW_STRIDE] = source.plane_stride, source.row_stride
            # Word gathers (4 tokens of a cell row per 32-bit load) when the geometry keeps them aligned.
            self.pic_vec_rule = source.plane_stride % 4 == 0 and source.row_stride % 4 == 0 and job.grid[2] % 4 == 0
            self._affine(source.scale, source.offset)
            return
        values = self.src = source.values
        row[_C_SRC_DTYPE] = self.dtype
        row[_C_SRC_ROW], row[_C_SRC_COL] = values.stride()
        if source.quantized:
            self._affine(source.scale[:self.rank], source.offset[:self.rank])
            self.src_vec_rule = values.stride(1) == 1 and values.stride(0) % 16 == 0
        else:
            self.host_bound = source.bound

    def _affine(self, scale, offset):
        """The job's fp32 (scale | offset) block and the fp16 modes' prescale exponent of its
        coefficient bound max(|offset|, |255 * scale + offset|) (the affine arrays are read-only copies)."""
        self.affine = np.concatenate((scale, offset)).astype(np.float32, copy=False)
        self.exponent = _prescale_exponent(_coefficient_bound(scale, offset))

    def source_address(self):
        if self.pictures is None:
            return self.src.data_ptr()
        return min(picture.data_ptr() for picture in self.pictures)


# Distinct job geometries (descriptor keys) seen by this process, numbered for cheap call keys.
_KEY_IDS: dict = {}


def job_desc(job):
    """The job's :class:`_JobDesc` (built on first use and kept on the job)."""
    desc = job.__dict__.get("_hip_desc")
    if desc is None:
        desc = _JobDesc(job)
        object.__setattr__(job, "_hip_desc", desc)
    return desc


def _rank_steps_class(precision, rank):
    """The compiled variant's register-resident rank steps for a rank (see ``pick_ks`` in
    csrc/restore_kernel.h); jobs of one class share a launch, so the product loop is fixed."""
    if not rank:
        return 0
    steps = (rank + 15) // 16
    # The 16-bit modes add the rank-halves variants' classes (24, 32; fp16x2 also 16).
    for size in (4, 8) if precision == "fp32" else (2, 4, 8, 12, 16, 24, 32):
        if steps <= size:
            return size
    return -1  # chunked


# ---------------------------------------------------------------------------
# Call layouts
# ---------------------------------------------------------------------------

# Columns that hold an offset into the call buffer in a layout's rows; the base is added per call.
_BASE_RELATIVE_PACK = ("dst_ptr", "exp_ptr", "scale_ptr", "offset_ptr")
_PACK_COLUMN = {name: index for index, name in enumerate(_lib.PACK_FIELDS)}


class _Layout:
    """Launch groups, variants, work tables, basis packs and the call-buffer layout of one call
    geometry.  ``rows`` / ``rows_relative`` and ``packs`` / ``packs_relative`` are the
    descriptor tables with buffer offsets where the call writes ``base + offset``;
    ``template`` is the host image of the buffer's tables, static parts filled."""

    def __init__(self, descs, dynamic_flags, basis_groups, precision, config, device, staged=False):
        self.precision, self.config = precision, config
        self.code = _lib.PRECISION_CODES[precision]
        self.staged = staged
        self.static = bool(_config_value(config, "static_scratch")) and not staged
        self.fp16_mode = precision in ("fp16", "fp16x2")
        self.grids, self.variants = [], []
        rows = np.stack([desc.row for desc in descs])
        rows[:, _C_FLAGS] |= np.asarray(dynamic_flags, dtype=np.int64)
        relative = np.zeros_like(rows)
        arena = _Arena()
        self.bound_jobs = [i for i, d in enumerate(descs)
                           if self.fp16_mode and d.kind == _lib.SRC_FLOAT and d.host_bound is None]
        rows[self.bound_jobs, _C_BOUND_INDEX] = 0
        self._affine_layout(descs, rows, relative, arena)
        self.picture_tables = []
        for index, desc in enumerate(descs):
            if desc.pictures is not None:
                at = arena.reserve(8 * len(desc.pictures))
                self.picture_tables.append((index, at))
                rows[index, _C_PIC_TABLE], relative[index, _C_PIC_TABLE] = at, 1
        self.staged_rows = np.zeros(len(descs), dtype=np.int64)
        plans = self._launch_groups(descs, rows, arena, device, basis_groups)
        self.staged_rows_offset = arena.add(self.staged_rows) if staged else None
        packs, pack_of = self._packs(descs, plans, basis_groups, arena)
        self._pack_layout(descs, rows, relative, plans, packs, pack_of)
        self.bound_tiles = _tiles(self.bound_jobs, descs) if self.bound_jobs else None
        self.bound_tile_offset = arena.add(self.bound_tiles) if self.bound_jobs else None
        self.packs_offset = arena.reserve(len(packs) * _lib.PACK_DTYPE.itemsize) if packs else None
        self.desc_offset = arena.reserve(len(descs) * _N_FIELDS * 8)
        self.arena_bytes = (arena.size + 255) // 256 * 256
        if not self.static:
            for index, pack_index in pack_of.items():
                rows[index, _C_PACK_PTR] = self.arena_bytes + packs[pack_index]["offset"]
        self.template = np.zeros(arena.size, dtype=np.uint8)
        for offset, array in arena.parts():
            self.template[offset:offset + array.nbytes] = array.reshape(-1).view(np.uint8)
        self.plans, self.jobs = plans, len(descs)
        self.scratch_words = self.exp_words + len(descs)
        self.buffer_bytes = self.arena_bytes + self.pack_total + 4 * self.scratch_words + 256
        # Pack-table and pack-pointer offsets are relative to the buffer base.
        pack_rows = np.zeros((len(packs), len(_lib.PACK_FIELDS)), dtype=np.int64)
        pack_relative = np.zeros_like(pack_rows)
        self.pack_sources = []
        for position, pack in enumerate(packs):
            entry = pack_rows[position]
            for name in ("src_dtype", "row_stride", "channels", "rank", "kind", "ksteps", "nblocks"):
                entry[_PACK_COLUMN[name]] = pack[name]
            entry[_PACK_COLUMN["dst_ptr"]] = self.arena_bytes + pack["offset"]
            entry[_PACK_COLUMN["exp_ptr"]] = self.arena_bytes + self.pack_total + 4 * pack["word"]
            columns = ["dst_ptr", "exp_ptr"]
            if pack["kind"] == _lib.PACK_STREAM:
                entry[_PACK_COLUMN["scale_ptr"]], entry[_PACK_COLUMN["offset_ptr"]] = pack["scale"], pack["offset_table"]
                columns += ["scale_ptr", "offset_ptr"]
            pack_relative[position, [_PACK_COLUMN[name] for name in columns]] = 1
            self.pack_sources.append(pack["member"])
        self.pack_rows, self.pack_relative = pack_rows, pack_relative
        self.rows, self.rows_relative = rows, relative
        self.table_jobs = [i for i, d in enumerate(descs) if d.table is not None]
        self.host_bound_jobs = [i for i, d in enumerate(descs) if self.fp16_mode and d.host_bound is not None]

    def _affine_layout(self, descs, rows, relative, arena):
        """One fp32 table of every job's (scale | offset) block, in job order; the rows' pointers."""
        self.affine_jobs = [i for i, d in enumerate(descs) if d.affine is not None]
        sizes = [descs[i].affine.size for i in self.affine_jobs]
        self.affine_total = int(sum(sizes))
        self.affine_offset = arena.reserve(4 * self.affine_total) if sizes else None
        self.affine_at = {}
        first = 0
        for index, size in zip(self.affine_jobs, sizes):
            at = (self.affine_offset + 4 * first, self.affine_offset + 4 * (first + size // 2))
            self.affine_at[index] = at
            rows[index, _C_SCALE], rows[index, _C_OFFSET] = at
            relative[index, _C_SCALE] = relative[index, _C_OFFSET] = 1
            first += size

    def _launch_groups(self, descs, rows, arena, device, basis_groups):
        """Launch groups (source kind, dtypes, head geometry, rank class, straight-line eligibility)
        and the kernel variant, grid and work tables of each."""
        precision, config = self.precision, self.config
        if self.static and self.bound_jobs:
            raise ConfigurationError("static_scratch restores hold no device coefficient bounds: float sources in "
                                     "the fp16 modes need a host bound")
        allow_fast = bool(_config_value(config, "fast_variant"))
        allow_pairs = allow_fast and bool(_config_value(config, "head_pairs"))
        allow_split = bool(_config_value(config, "split_rank"))
        allow_stream = allow_fast and bool(_config_value(config, "stream_variant")) and precision == "fp16x2"
        groups: dict = {}
        for index, desc in enumerate(descs):
            flags = (_fast_eligibility(desc.kind, desc.head_dim, desc.table is not None, rows[index], precision)
                     if allow_fast else 0)
            key = (desc.kind, desc.dtype, desc.out_dtype, desc.head_dim, desc.channels,
                   _rank_steps_class(precision, desc.rank), None if desc.table is None else desc.rope_kind == "dense",
                   flags)
            groups.setdefault(key, []).append(index)
        compute_units = _compute_units(device)
        passes = 2 if precision == "fp16x2" else (4 if precision == "fp32" else 1)
        store_cost = _config_value(config, "store_cost")
        store_cost = float(_STORE_COST[precision] if store_cost is None else store_cost)
        plans = []
        for key, members in groups.items():
            kind, group_flags = key[0], key[-1]
            first = descs[members[0]]
            channels, head_dim = first.channels, first.head_dim
            plan = {"kind": kind, "members": members, "channels": channels, "head_dim": head_dim,
                    "out_dtype": first.out_dtype}
            plans.append(plan)
            if kind == _lib.SRC_DENSE:
                tiles = _tiles(members, descs)
                plan.update(variant="dense", tiles=arena.add(tiles), n_tiles=len(tiles))
                continue
            if self.staged:
                self._staged_plan(descs, plan, basis_groups, arena)
                continue
            job_steps = {i: (descs[i].rank + 15) // 16 for i in members}
            max_ksteps = plan["max_ksteps"] = max(job_steps.values())
            stream = (allow_stream and group_flags & _lib.GF_FAST and kind == _lib.SRC_U8 and head_dim == 128
                      and channels % 128 == 0 and max_ksteps <= _STREAM_MAX_KSTEPS)
            stream_flags = group_flags & (_lib.GF_FAST | _lib.GF_ROPE)
            if stream and group_flags & _lib.GF_ROPE:
                if first.rope_kind == "dense":
                    stream_flags |= _lib.GF_DENSE_ROPE
                elif max(descs[i].section_pairs for i in members) > _lib.STREAM_SECTION_PAIRS:
                    stream = False  # section rows beyond the kernel's LDS table
            if stream:
                self._stream_plan(descs, plan, stream_flags, compute_units, arena)
                continue
            tiles = _tiles(members, descs)
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
            steps = np.array([job_steps[i] for i in tiles[:, 0].tolist()], dtype=np.float64)
            plan.update(variant="general" if not group_flags & _lib.GF_FAST
                        else ("pairs" if group_flags & _lib.GF_HEAD_PAIRS
                              else ("split" if group_flags & _lib.GF_SPLIT_RANK else "fast")),
                        flags=group_flags, tile_rows=tiles, tile_costs=steps * passes + store_cost,
                        blocks_per_tile=blocks_per_tile)
        if not self.static and bool(_config_value(config, "pair_launch")):
            plans = self._pair_groups(plans)
        for plan in plans:
            tiles = plan.pop("tile_rows", None)
            if tiles is None:
                continue
            costs, blocks_per_tile = plan.pop("tile_costs"), plan.pop("blocks_per_tile")
            if plan["variant"] == "pair":
                per_cu = config.get("workgroups_per_cu") or _lib.pair_occupancy(
                    self.code, plan["kind"], plan["ksteps0"], plan["ksteps1"], plan["head_dim"], plan["out_dtype"])
            else:
                per_cu = config.get("workgroups_per_cu") or _occupancy(self.code, plan["kind"], plan["max_ksteps"],
                                                                       plan["head_dim"], plan["out_dtype"],
                                                                       plan["flags"])
            grid = int(max(1, min(len(tiles) * blocks_per_tile, compute_units * max(1, per_cu))))
            bounds = _balanced_bounds(costs, blocks_per_tile, grid)
            plan.update(tiles=arena.add(tiles), n_tiles=len(tiles), bounds=arena.add(bounds), grid=grid)
            self.grids.append(grid)
            self.variants.append(plan["variant"])
        return plans

    def _pair_groups(self, plans):
        """Merges a RoPE head-pair group with a plain head-pair group of the same geometry (a call's
        K and V) into one ``pair`` launch when a pair kernel covers them (``rch_restore_pair``):
        the concatenated units get one cost-balanced split, so the persistent grid fills and drains
        once per call instead of once per group."""
        candidates = [plan for plan in plans if plan.get("variant") == "pairs"]
        for first in candidates:
            if not first["flags"] & _lib.GF_ROPE or first.get("paired"):
                continue
            for second in candidates:
                if second["flags"] & _lib.GF_ROPE or second.get("paired"):
                    continue
                if any(first[name] != second[name] for name in ("channels", "head_dim", "out_dtype")):
                    continue
                # The straight-line kernel reads uint8 rows or pictures per job, so either kind pairs.
                kinds = {first["kind"], second["kind"]}
                if not kinds <= {_lib.SRC_U8, _lib.SRC_PICTURE}:
                    continue
                kind = _lib.SRC_PICTURE if _lib.SRC_PICTURE in kinds else _lib.SRC_U8
                if _lib.pair_occupancy(self.code, kind, first["max_ksteps"], second["max_ksteps"],
                                       first["head_dim"], first["out_dtype"]) <= 0:
                    continue
                first["paired"] = second["paired"] = True
                merged = {"kind": kind, "members": first["members"] + second["members"],
                          "channels": first["channels"], "head_dim": first["head_dim"],
                          "out_dtype": first["out_dtype"], "variant": "pair",
                          "max_ksteps": max(first["max_ksteps"], second["max_ksteps"]),
                          "ksteps0": first["max_ksteps"], "ksteps1": second["max_ksteps"],
                          "flags": _lib.GF_FAST | _lib.GF_HEAD_PAIRS, "n_tiles0": len(first["tile_rows"]),
                          "n_tiles1": len(second["tile_rows"]),
                          "tile_rows": np.concatenate([first["tile_rows"], second["tile_rows"]]),
                          "tile_costs": np.concatenate([first["tile_costs"], second["tile_costs"]]),
                          "blocks_per_tile": first["blocks_per_tile"]}
                plans = [merged if plan is first else plan for plan in plans if plan is not second]
                break
        for plan in plans:
            plan.pop("paired", None)
        return plans

    def _staged_plan(self, descs, plan, basis_groups, arena):
        """GEMM groups of a staged launch group: jobs sharing a basis view and rank stack their
        coefficient rows into one work matrix (job order), so each group is one library GEMM
        (reelcache/restore_kernels.py:2198-2213)."""
        gemms: dict = {}
        for index in plan["members"]:
            gemms.setdefault((basis_groups[index], descs[index].rank), []).append(index)
        plan["gemms"] = []
        for (_, rank), members in gemms.items():
            first = 0
            for index in members:
                self.staged_rows[index] = first
                first += descs[index].tokens
            tiles = _tiles(members, descs)
            plan["gemms"].append({"members": members, "rank": rank, "rows": first, "tiles": arena.add(tiles),
                                  "n_tiles": len(tiles)})
        plan.update(variant="staged", grid=0)
        self.variants.append("staged")

    def _stream_plan(self, descs, plan, group_flags, compute_units, arena):
        """Work tables of a stream-kernel group: units (job, head, 32-token tile) job-major, and an
        equal split of them over the resident workgroups."""
        members = plan["members"]
        heads = plan["channels"] // 128
        flags = group_flags | _lib.GF_STREAM
        units = [heads * ((descs[i].tokens + STREAM_TOKENS - 1) // STREAM_TOKENS) for i in members]
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

    def _packs(self, descs, plans, basis_groups, arena):
        """The basis packs: one per job of a stream group (its scaled slabs), one per distinct basis
        view for the other kernels (fragments of the largest rank used)."""
        packs: list = []
        pack_of: dict = {}
        by_basis: dict = {}
        for plan in plans:
            if plan["variant"] in ("dense", "staged"):
                continue
            used = []
            for index in plan["members"]:
                desc = descs[index]
                stride, channels, dtype = desc.basis_key
                if plan["variant"] == "stream":
                    packs.append({"kind": _lib.PACK_STREAM, "member": index, "row_stride": stride, "channels": channels,
                                  "src_dtype": dtype, "rank": desc.rank, "ksteps": plan["stream_ksteps"],
                                  "nblocks": channels // 32, "scale": self.affine_at[index][0],
                                  "offset_table": self.affine_at[index][1]})
                    pack_of[index] = len(packs) - 1
                    used.append(len(packs) - 1)
                    continue
                position = by_basis.get(basis_groups[index])
                if position is None:
                    position = by_basis[basis_groups[index]] = len(packs)
                    packs.append({"kind": _lib.PACK_FRAGMENTS, "member": index, "row_stride": stride,
                                  "channels": channels, "src_dtype": dtype, "rank": 0,
                                  "nblocks": 2 * ((channels + 63) // 64)})
                packs[position]["rank"] = max(packs[position]["rank"], desc.rank)
                pack_of[index] = position
                if position not in used:
                    used.append(position)
            plan["packs"] = used
        for pack in packs:
            if pack["kind"] == _lib.PACK_FRAGMENTS:
                pack["ksteps"] = (pack["rank"] + 15) // 16
        return packs, pack_of

    def _pack_layout(self, descs, rows, relative, plans, packs, pack_of):
        """Pack sizes and offsets (in the call buffer, or per launch group in the library's static
        array), the exponent and bound scratch words, and the pack fields of the rows."""
        fragment = 32 if self.precision == "fp32" else 16
        total, words = 0, 0
        for pack in packs:
            pack["bytes"] = (pack["nblocks"] * _lib.stream_slab_bytes(pack["ksteps"]) if pack["kind"] == _lib.PACK_STREAM
                             else (pack["ksteps"] * pack["nblocks"] * 64 * fragment + 255) // 256 * 256)
            pack["offset"], pack["word"] = total, words
            total += pack["bytes"]
            words += pack["nblocks"] if pack["kind"] == _lib.PACK_FRAGMENTS else 0
        self.exp_words = words
        # Static scratch: each launch group packs its own bases at the start of the library's array,
        # in the order of ``plan["packs"]``, so a pack's position is a property of the (group, pack)
        # pair: one basis can sit at different positions in two groups (ranks in two rank classes).
        static_at = {}
        if self.static:
            total = 0
            for plan in plans:
                fragment_at, word_at = 0, 0
                for pack_index in plan.get("packs", ()):
                    pack = packs[pack_index]
                    for member in plan["members"]:
                        if pack_of.get(member) == pack_index:
                            static_at[member] = (fragment_at, word_at)
                    fragment_at += pack["bytes"]
                    word_at += pack["nblocks"] if pack["kind"] == _lib.PACK_FRAGMENTS else 0
        self.pack_total = total
        for position, index in enumerate(self.bound_jobs):
            rows[index, _C_BOUND_INDEX] = words + position
        for index, pack_index in pack_of.items():
            pack = packs[pack_index]
            rows[index, _C_PACK_NBLOCKS] = pack["nblocks"]
            if self.static:
                rows[index, _C_PACK_PTR], rows[index, _C_EXP_INDEX] = static_at[index]
            else:
                rows[index, _C_EXP_INDEX] = pack["word"]
                relative[index, _C_PACK_PTR] = 1  # the buffer offset is known once the arena is complete


    def enqueue(self, descs, dst, src, bases, device, stream, keepalive, stage_events):
        """Write this call's addresses and affine tables into the layout's tables, upload them with
        one copy, and launch."""
        buffer = torch.empty(self.buffer_bytes, dtype=torch.uint8, device=device)
        base = buffer.data_ptr()
        rows = self.rows + self.rows_relative * base
        rows[:, _C_DST_PTR] = dst
        rows[:, _C_SRC_PTR] = src
        tables: dict = {}
        for index in self.table_jobs:
            table = descs[index].table
            entry = tables.get(id(table))
            if entry is None:
                block = table._kernel_block(device, stream)
                entry = tables[id(table)] = (block.cos.data_ptr(), block.sin.data_ptr(), block.pairs.data_ptr())
                keepalive.append(block.block)
            rows[index, _C_COS], rows[index, _C_SIN] = entry[0], entry[1]
            if rows[index, _C_PAIRS]:
                rows[index, _C_PAIRS] = entry[2]
        host = _pinned_host(self.template.size)
        image = host.numpy()
        image[:] = self.template
        if self.affine_jobs:
            image[self.affine_offset:self.affine_offset + 4 * self.affine_total].view(np.float32)[:] = \
                np.concatenate([descs[index].affine for index in self.affine_jobs])
            if self.fp16_mode:
                rows[self.affine_jobs, _C_COEF_EXP] = [descs[index].exponent for index in self.affine_jobs]
        for index in self.host_bound_jobs:
            rows[index, _C_COEF_EXP] = _prescale_exponent(descs[index].host_bound)
        for index, at in self.picture_tables:
            pictures = descs[index].pictures
            offsets = np.fromiter((picture.data_ptr() for picture in pictures), dtype=np.int64, count=len(pictures))
            image[at:at + 8 * len(pictures)].view(np.int64)[:] = offsets - src[index]
        packs = None
        if len(self.pack_rows):
            packs = self.pack_rows + self.pack_relative * base
            packs[:, _PACK_COLUMN["src_ptr"]] = [bases[member] for member in self.pack_sources]
            image[self.packs_offset:self.packs_offset + packs.nbytes] = packs.view(np.uint8).reshape(-1)
        image[self.desc_offset:self.desc_offset + rows.nbytes] = rows.view(np.uint8).reshape(-1)
        scratch_base = base + self.arena_bytes + self.pack_total
        if self.bound_jobs:
            start = self.arena_bytes + self.pack_total + 4 * self.exp_words
            buffer[start:start + 4 * len(self.bound_jobs)].zero_()  # fill kernel, not a memset (graph-capture safe)
        buffer[:image.size].copy_(host, non_blocking=True)
        keepalive.extend((host, buffer))
        return self._launch(base, scratch_base, packs, stream, stage_events, descs, keepalive)


    def _launch(self, base, scratch_base, packs, stream, stage_events, descs, keepalive):
        hip_stream = stream.cuda_stream
        jobs, table = self.jobs, base + self.desc_offset
        launches = 0
        if stage_events is not None:
            stage_events.append(("start", _record(stream)))
        if packs is not None and not self.static:
            _lib.call("rch_basis_pack", base + self.packs_offset, len(packs), int(packs[:, _PACK_COLUMN["nblocks"]].max()),
                      int(packs[:, _PACK_COLUMN["ksteps"]].max()), self.code, hip_stream)
            launches += 1
        if stage_events is not None:
            stage_events.append(("pack", _record(stream)))
        if self.bound_jobs:
            _lib.call("rch_coefficient_bound", table, jobs, base + self.bound_tile_offset, len(self.bound_tiles),
                      int(max(self.rows[i, _C_RANK] for i in self.bound_jobs)), scratch_base, hip_stream)
            launches += 1
        for plan in self.plans:
            variant = plan["variant"]
            if variant == "staged":
                launches += self._launch_staged(plan, base, scratch_base, stream, stage_events, descs, keepalive)
                continue
            if variant == "dense":
                _lib.call("rch_rope_store", table, jobs, base + plan["tiles"], plan["n_tiles"], plan["channels"],
                          plan["head_dim"], plan["out_dtype"], hip_stream)
            elif variant == "pair":
                _lib.call("rch_restore_pair", table, jobs, base + plan["tiles"], plan["n_tiles0"], plan["n_tiles1"],
                          base + plan["bounds"], plan["grid"], plan["channels"], plan["head_dim"], plan["kind"],
                          plan["out_dtype"], self.code, plan["ksteps0"], plan["ksteps1"], scratch_base, hip_stream)
            elif self.static:
                group = np.ascontiguousarray(packs[plan["packs"]])
                _lib.call("rch_restore_noalloc", group.ctypes.data, len(group), table, jobs, base + plan["tiles"],
                          plan["n_tiles"], base + plan["bounds"], plan["grid"], plan["channels"], plan["head_dim"],
                          plan["kind"], plan["out_dtype"], self.code, plan["max_ksteps"], plan["flags"], hip_stream)
            else:
                _lib.call("rch_restore", table, jobs, base + plan["tiles"], plan["n_tiles"], base + plan["bounds"],
                          plan["grid"], plan["channels"], plan["head_dim"], plan["kind"], plan["out_dtype"], self.code,
                          plan["max_ksteps"], plan["flags"], scratch_base, hip_stream)
            launches += 1
            if stage_events is not None:
                stage_events.append((f"launch{launches}", _record(stream)))
        if stage_events is not None:
            stage_events.append(("fused", _record(stream)))
        return launches

    def _launch_staged(self, plan, base, scratch_base, stream, stage_events, descs, keepalive):
        """The staged comparison path of one launch group: every GEMM group's unpack, then the
        library GEMMs (FP32 output), then the RoPE / cast / store launches, with the reference's
        stage events ("unpack", "gemm", "rope_store")."""
        hip_stream = stream.cuda_stream
        table, jobs, rows = base + self.desc_offset, self.jobs, base + self.staged_rows_offset
        work_dtype = _STAGED_WORK[self.precision]
        launches, products = 0, []
        for gemm in plan["gemms"]:
            work = torch.empty((gemm["rows"], gemm["rank"]), dtype=work_dtype, device=descs[0].dst.device)
            keepalive.append(work)
            _lib.call("rch_staged_unpack", table, jobs, base + gemm["tiles"], gemm["n_tiles"], rows, work.data_ptr(),
                      work.stride(0), gemm["rank"], plan["kind"], _DTYPE_CODES[work_dtype], self.code, scratch_base,
                      hip_stream)
            launches += 1
            products.append(work)
        if stage_events is not None:
            stage_events.append(("unpack", _record(stream)))
        for position, gemm in enumerate(plan["gemms"]):
            basis = descs[gemm["members"][0]].basis[:gemm["rank"]]
            products[position] = staged_gemm(products[position], basis, self.precision)
            keepalive.append(products[position])
            launches += 1
        if stage_events is not None:
            stage_events.append(("gemm", _record(stream)))
        for gemm, product in zip(plan["gemms"], products):
            _lib.call("rch_staged_store", table, jobs, base + gemm["tiles"], gemm["n_tiles"], rows, product.data_ptr(),
                      product.stride(0), plan["channels"], plan["head_dim"], plan["out_dtype"], self.code, scratch_base,
                      hip_stream)
            launches += 1
        if stage_events is not None:
            stage_events.append(("rope_store", _record(stream)))
        return launches


# Work (coefficient) dtype of the staged path's GEMM per precision.
_STAGED_WORK = {"fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}
STAGED_PRECISIONS = ("fp32", "tf32", "fp16", "bf16")


def check_staged_precision(precision):
    """The staged GEMM's precision follows process-wide torch settings: check them, never change
    them (reelcache/restore_kernels.py:2153-2164).  gfx950 has no TF32 matrix cores, so ``tf32``
    is refused as in the fused path."""
    if precision not in STAGED_PRECISIONS:
        raise UnsupportedError("the staged backend supports fp32, tf32, fp16 and bf16")
    if precision == "tf32":
        raise UnsupportedError("the staged tf32 GEMM has no matrix-core form on gfx950 (no TF32 MFMA); use fp32, "
                               "fp16 or bf16")
    if precision == "fp32":
        _require_fp32_matmul("cuda", ("ieee",), "the staged fp32 GEMM (rocBLAS)")
    elif precision == "fp16" and getattr(torch.backends.cuda.matmul, "allow_fp16_accumulation", False):
        raise UnsupportedError(
            "the staged fp16 GEMM needs FP32 accumulation, but this process allows FP16 accumulation in the BLAS "
            "library (torch.backends.cuda.matmul.allow_fp16_accumulation=True). That setting is process-wide, so "
            "restore_kernels never changes it: use the fused backend or change the setting in your own code.")


def staged_gemm(coefficients, basis, precision):
    """Rank-view product with FP32 accumulation and FP32 output on the GPU BLAS library
    (reelcache/restore_kernels.py:2167-2189): ``torch.mm`` on FP32 operands for fp32; FP16 / BF16
    operands through ``torch.mm(..., out_dtype=torch.float32)``.  A Torch that rejects that
    overload raises :class:`UnsupportedError` (no retry with a 16-bit output, which would round and
    could overflow the prescaled products); every other error propagates unchanged."""
    if precision == "fp32":
        return torch.mm(coefficients, basis.float())
    operand = basis.to(_STAGED_WORK[precision])
    try:
        return torch.mm(coefficients, operand, out_dtype=torch.float32)
    except (TypeError, NotImplementedError) as error:
        raise UnsupportedError(
            f"the staged {precision} GEMM needs torch.mm(..., out_dtype=torch.float32) (FP32 output); "
            f"Torch {torch.__version__} rejected it: {type(error).__name__}: {error}") from error


_LAYOUTS: dict = {}
_LAYOUT_LIMIT = 256


def _config_key(config):
    """Hashable form of a merged launch configuration."""
    if config is DEFAULT_MERGED:
        return _DEFAULT_KEY
    return tuple(sorted((name, repr(item)) for name, item in config.items()))


_DEFAULT_KEY = _config_key(dict(_DEFAULT_CONFIG))


def _pinned_host(nbytes):
    """Pinned staging for a call's tables: fresh pinned memory, or under HIP-graph capture a
    region of the staging reserved beforehand (the graph's copy node reads it on every replay)."""
    if torch.cuda.is_current_stream_capturing():
        return _capture_staging(nbytes)
    return torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)


def run_call(descs, device, stream, precision, config, keepalive, stage_events=None, staged=False):
    """Plan (or reuse the layout of) one HIP call and enqueue it on ``stream``; returns
    ``(launches, grids, variants)``.  ``staged``: the staged comparison path (unpack, library
    GEMM, store) for the factorized jobs instead of the fused kernels."""
    dst = [desc.dst.data_ptr() + desc.dst_shift for desc in descs]
    src = [desc.source_address() for desc in descs]
    dynamic = [(_lib.JF_DST_VEC if desc.dst_vec_rule and not d & 15 else 0)
               | (_lib.JF_SRC_VEC if desc.src_vec_rule and not s & 15 else 0)
               | (_lib.JF_PIC_VEC4 if desc.pic_vec_rule and all(not p.data_ptr() & 3 for p in desc.pictures) else 0)
               for desc, d, s in zip(descs, dst, src)]
    bases, groups, first_of = [0] * len(descs), [None] * len(descs), {}
    for index, desc in enumerate(descs):
        if desc.basis is not None:
            bases[index] = address = desc.basis.data_ptr()
            groups[index] = first_of.setdefault((address, desc.basis_key), index)
    key = (precision, _config_key(config), tuple(desc.key_id for desc in descs), tuple(dynamic), tuple(groups),
           staged)
    layout = _LAYOUTS.get(key)
    if layout is None:
        layout = _Layout(descs, dynamic, groups, precision, config, device, staged)
        if len(_LAYOUTS) >= _LAYOUT_LIMIT:
            _LAYOUTS.clear()
        _LAYOUTS[key] = layout
    launches = layout.enqueue(descs, dst, src, bases, device, stream, keepalive, stage_events)
    return launches, list(layout.grids), list(layout.variants)
