"""The restore job model: destinations, RoPE tables and positions, sources, jobs.

These are the reference's public contract types (reelcache/restore_kernels.py:235-868): same
class names, fields, defaults, properties and accepted inputs, re-exported by
:mod:`reelcache_amd.restore_kernels`.  The implementation is this package's own:

* layouts are described by one table of tensor axes (batch, token, head, dim), from which every
  property of :class:`NativeView` is derived;
* validation is a list of rules built from :mod:`reelcache_amd._checks`;
* separable RoPE tables of several axes are assembled by one helper that pads with NaN;
* each :class:`RopeTable` caches one set of FP32 device copies per device (``cos``, ``sin`` and
  the interleaved ``(cos, sin)`` pairs the straight-line kernels read), ordered for every
  consumer stream by the event that completes them.
"""

from __future__ import annotations

import math
import threading
import weakref
from collections.abc import Mapping
from dataclasses import dataclass, field
from typing import Any

import numpy as np
import torch

from ._checks import bound as _bound, count, host_floats, matrix, need, one_of, strided
from .errors import ConfigurationError

LAYOUTS = ("BTHD", "THD", "BHTD")
OUTPUT_DTYPES = (torch.bfloat16, torch.float16, torch.float32)
COEFFICIENT_DTYPES = (torch.float32, torch.float16, torch.bfloat16)

# Tensor axes of (batch, token, head, dim) per layout; THD has no batch axis.
_AXES = {"BTHD": (0, 1, 2, 3), "THD": (None, 0, 1, 2), "BHTD": (0, 2, 1, 3)}


# ---------------------------------------------------------------------------
# Destinations
# ---------------------------------------------------------------------------


@dataclass(frozen=True, eq=False)
class NativeView:
    """A native cache tensor, its layout and the first destination token.

    ``"BTHD"``: Wan/SGLang ``[B, T, H, D]``; ``"THD"``: RAVEN packed ``[T, H, D]``;
    ``"BHTD"``: LongCat ``[B, H, T, D]``.  Any strides are accepted.
    """

    tensor: torch.Tensor
    layout: str = "BTHD"
    token_offset: int = 0
    batch_index: int = 0

    def __post_init__(self):
        tensor = strided(self.tensor, "destination tensor")
        one_of(self.layout, LAYOUTS, "destination layout")
        batch_axis = _AXES[self.layout][0]
        need(tensor.ndim == (3 if batch_axis is None else 4), f"{self.layout} destination has the wrong number of dimensions")
        need(tensor.dtype in OUTPUT_DTYPES, "destination dtype must be bfloat16, float16 or float32")
        count(self.token_offset, "token_offset")
        count(self.batch_index, "batch_index")
        if batch_axis is None:
            need(self.batch_index == 0, "a packed THD destination has no batch dimension")
        else:
            need(self.batch_index < tensor.shape[batch_axis], "batch_index is outside the destination")
        need(self.head_dim % 2 == 0, "head_dim must be even")
        need(all(stride != 0 or size <= 1 for size, stride in zip(tensor.shape, tensor.stride())),
             "destination views with broadcast (zero) strides alias")

    def _size(self, role):
        return self.tensor.shape[_AXES[self.layout][role]]

    @property
    def heads(self):
        return self._size(2)

    @property
    def head_dim(self):
        return self._size(3)

    @property
    def channels(self):
        return self.heads * self.head_dim

    @property
    def capacity(self):
        return self._size(1)

    def strides(self):
        """Element strides of (token, head, dim)."""
        return tuple(self.tensor.stride(axis) for axis in _AXES[self.layout][1:])

    def element_offset(self):
        """Element offset (in the storage) of (batch_index, token_offset, head 0, dim 0)."""
        batch_axis = _AXES[self.layout][0]
        batch = 0 if batch_axis is None else self.batch_index * self.tensor.stride(batch_axis)
        return self.tensor.storage_offset() + batch + self.token_offset * self.strides()[0]

    def slot(self, tokens):
        """A ``[tokens, H, D]`` view of the destination slot."""
        batch_axis, *rest = _AXES[self.layout]
        canonical = (self.tensor.permute(*rest) if batch_axis is None
                     else self.tensor.permute(batch_axis, *rest)[self.batch_index])
        return canonical[self.token_offset:self.token_offset + tokens]


# ---------------------------------------------------------------------------
# RoPE tables
# ---------------------------------------------------------------------------


def wan_sections(pairs):
    """Wan/LongCat 3-D split of ``pairs = head_dim // 2`` into (t, h, w) pair counts: h and w
    take a third each (rounded down), t the rest."""
    count(pairs, "pairs", minimum=1)
    spatial = pairs // 3
    return (pairs - 2 * spatial, spatial, spatial)


def _assemble_sections(parts, dtype, device):
    """(cos, sin, sections, section_rows) of a separable table from per-axis ``(cos, sin)``
    blocks ``[positions, pairs]``; cells an axis does not reach stay NaN."""
    rows = max(cos.shape[0] for cos, _ in parts)
    pairs = sum(cos.shape[1] for cos, _ in parts)
    tables = [torch.full((rows, pairs), float("nan"), dtype=dtype, device=device) for _ in range(2)]
    column = 0
    for block in parts:
        positions, width = block[0].shape
        for table, values in zip(tables, block):
            table[:positions, column:column + width] = values
        column += width
    return (*tables, tuple(cos.shape[1] for cos, _ in parts), tuple(cos.shape[0] for cos, _ in parts))


def _complex_parts(freqs, dtype):
    real = torch.view_as_real(freqs.resolve_conj()).to(dtype)
    return real[..., 0], real[..., 1]


_UPLOAD_STREAMS: dict = {}
_UPLOAD_LOCK = threading.Lock()
_PLANE_ALIGN = 64  # floats: every part of a device table block starts on a 256-byte boundary


def _upload_stream(device):
    """Private per-device stream for RoPE-table uploads (default priority)."""
    with _UPLOAD_LOCK:
        if device not in _UPLOAD_STREAMS:
            _UPLOAD_STREAMS[device] = torch.cuda.Stream(device)
        return _UPLOAD_STREAMS[device]


def _carve(block, rows, width):
    """(cos, sin, pairs) views of a table block: two ``[rows, width]`` planes, then the
    interleaved ``[rows, width, 2]`` pairs."""
    plane = block.numel() // 4
    cos = block[:rows * width].view(rows, width)
    sin = block[plane:plane + rows * width].view(rows, width)
    pairs = block[2 * plane:2 * plane + 2 * rows * width].view(rows, width, 2)
    return cos, sin, pairs


def _fill(views, cos, sin):
    """Round the table into the planes (one float32 rounding) and interleave them."""
    plane_cos, plane_sin, pairs = views
    plane_cos.copy_(cos)
    plane_sin.copy_(sin)
    pairs[..., 0].copy_(plane_cos)
    pairs[..., 1].copy_(plane_sin)


class _DeviceTable:
    """FP32 copies of one :class:`RopeTable` on one device in a single block: the planes ``cos``
    and ``sin`` ``[rows, pairs]`` and the interleaved ``pairs`` ``[rows, pairs, 2]`` that the
    straight-line kernels read.

    A host table is laid out in pinned memory right away and sent with one copy on a private
    stream; a device table is converted on the caller's stream, after the work already enqueued
    there.  ``ready`` is the event that completes the block (``None`` on the host, and once it
    has been observed complete, when the pinned source is dropped as well).  ``stamp`` is the
    table state the block was made from."""

    __slots__ = ("__weakref__", "block", "cos", "pairs", "pinned", "ready", "sin", "stamp")

    def __init__(self, cos, sin, device, stream, stamp):
        rows, width = cos.shape
        size = 4 * (-(-rows * width // _PLANE_ALIGN) * _PLANE_ALIGN)
        self.stamp, self.ready, self.pinned = stamp, None, None
        with torch.inference_mode(False), torch.no_grad():
            if device.type != "cuda":
                self.block = torch.empty(size, dtype=torch.float32, device=device)
                self.cos, self.sin, self.pairs = views = _carve(self.block, rows, width)
                _fill(views, cos, sin)
                return
            if torch.cuda.is_current_stream_capturing():
                # Work enqueued now would only run when the graph replays, and eager calls
                # before the first replay would read unwritten tables.
                raise ConfigurationError("a RoPE table's device copy cannot be built during HIP-graph capture: "
                                         "run one call with the table (or warmup) before capturing")
            if cos.device.type == "cpu":
                self.pinned = torch.empty(size, dtype=torch.float32, pin_memory=True)
                _fill(_carve(self.pinned, rows, width), cos, sin)
                work = _upload_stream(device)
            else:
                work = torch.cuda.current_stream(device) if stream is None else stream
            with torch.cuda.stream(work):
                self.block = torch.empty(size, dtype=torch.float32, device=device)
                self.cos, self.sin, self.pairs = views = _carve(self.block, rows, width)
                if self.pinned is not None:
                    self.block.copy_(self.pinned, non_blocking=True)
                else:
                    _fill(views, cos, sin)
                self.ready = torch.cuda.Event()
                self.ready.record(work)
            _PENDING_TABLES.add(self)

    def fence(self, device, stream):
        """Order ``stream`` (default: the current one) after the block's writes."""
        if self.ready is None:
            return
        if torch.cuda.is_current_stream_capturing():
            # A capture can neither query the upload's event nor wait on work outside the graph.
            raise ConfigurationError("a RoPE table's device copy was still pending when the capture began: call "
                                     "reserve_capture_staging() after the table's first use and before capturing")
        if self.ready.query():
            self.settle()
            return
        (torch.cuda.current_stream(device) if stream is None else stream).wait_event(self.ready)

    def settle(self):
        """Wait (host) for the block's writes; afterwards no consumer needs to wait for them."""
        if self.ready is not None:
            self.ready.synchronize()
        self.ready = self.pinned = None
        _PENDING_TABLES.discard(self)


# Device tables whose upload has not been observed complete (settled before HIP-graph captures).
_PENDING_TABLES: weakref.WeakSet = weakref.WeakSet()


def settle_table_uploads():
    """Wait for every pending RoPE-table upload, so that calls captured afterwards need no
    ordering against them (a capture cannot query or wait on work outside its graph)."""
    for table in list(_PENDING_TABLES):
        table.settle()


def _table_device(device):
    device = torch.device(device)
    if device.type == "cuda" and device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    return device


@dataclass(frozen=True, eq=False)
class RopeTable:
    """cos/sin rotation tables ``[R, head_dim // 2]`` for interleaved pairs.

    ``sections=None``: dense -- token ``t`` uses row ``positions.rows + t``.
    ``sections=(t, h, w)``: separable 3-D RoPE -- the first ``t`` pairs use the
    frame row, the next ``h`` the height row, the last ``w`` the width row.
    ``section_rows`` bounds the rows each section may use (default: all).
    """

    cos: torch.Tensor
    sin: torch.Tensor
    sections: tuple | None = None
    section_rows: tuple | None = None
    _device_cache: dict = field(default_factory=dict, init=False, repr=False, compare=False)
    _inference: bool = field(default=False, init=False, repr=False, compare=False)

    def __post_init__(self):
        cos, sin = strided(self.cos, "RoPE cos"), strided(self.sin, "RoPE sin")
        need(cos.ndim == 2 and cos.shape == sin.shape and cos.dtype == sin.dtype and cos.device == sin.device
             and cos.dtype in (torch.float32, torch.float64) and min(cos.shape) >= 1,
             "RoPE cos/sin must be matching float32/float64 [rows, head_dim // 2] tensors")
        object.__setattr__(self, "_inference", cos.is_inference() or sin.is_inference())
        if self.sections is None:
            need(self.section_rows is None, "section_rows requires separable sections")
            return
        sections = tuple(self.sections)
        need(len(sections) == 3 and all(type(v) is int and v >= 0 for v in sections) and sum(sections) == self.pairs,
             "RoPE sections must be three nonnegative pair counts summing to head_dim // 2")
        limits = (self.rows,) * 3 if self.section_rows is None else tuple(self.section_rows)
        need(len(limits) == 3 and all(type(v) is int and 0 <= v <= self.rows for v in limits),
             "section_rows must be three row counts within the table")
        object.__setattr__(self, "sections", sections)
        object.__setattr__(self, "section_rows", limits)

    @property
    def rows(self):
        return self.cos.shape[0]

    @property
    def pairs(self):
        return self.cos.shape[1]

    @property
    def head_dim(self):
        return 2 * self.pairs

    @classmethod
    def from_complex(cls, freqs, sections="wan"):
        """From complex ``freqs[rows, head_dim // 2]`` (the Wan ``rope_params`` concatenation)."""
        freqs = strided(freqs, "freqs")
        need(freqs.is_complex() and freqs.ndim == 2, "freqs must be a complex [rows, head_dim // 2] tensor")
        dtype = torch.float64 if freqs.dtype == torch.complex128 else torch.float32
        cos, sin = _complex_parts(freqs, dtype)
        return cls(cos.contiguous(), sin.contiguous(), wan_sections(freqs.shape[1]) if sections == "wan" else sections)

    @classmethod
    def from_axes(cls, temporal, height, width):
        """Separable table from per-axis complex tensors ``[positions, pairs]`` (unused cells NaN),
        e.g. non-integer temporal positions of multi-shot generation."""
        axes = [strided(value, "axis freqs") for value in (temporal, height, width)]
        need(all(value.is_complex() and value.ndim == 2 for value in axes),
             "axis frequencies must be complex [positions, pairs] tensors")
        need(len({value.device for value in axes}) == 1, "axis frequencies must share a device")
        dtype = torch.float64 if all(value.dtype == torch.complex128 for value in axes) else torch.float32
        cos, sin, sections, rows = _assemble_sections([_complex_parts(value, dtype) for value in axes], dtype,
                                                      axes[0].device)
        return cls(cos, sin, sections, rows)

    @classmethod
    def from_cos_sin(cls, cos, sin, sections=None):
        """From real tables, e.g. SGLang's dense ``freqs_cis = (cos, sin)``."""
        return cls(cos, sin, sections)

    @classmethod
    def longcat(cls, head_dim, num_frames, height, width, *, base=10000.0, device="cpu"):
        """LongCat-Video ``rope_3d`` tables in float32: per-axis inverse frequencies
        ``base ** -(2j / dim)``, grid positions and their products in float32, then cos / sin of
        the float32 angles.  LongCat caches hold pre-RoPE K (the engine rotates when attending), so
        restored LongCat caches are written without rotation; the table serves the engine."""
        count(head_dim, "head_dim", minimum=8)
        need(head_dim % 8 == 0, "LongCat 3D RoPE requires head_dim divisible by 8")
        extents = (num_frames, height, width)
        for value, name in zip(extents, ("num_frames", "height", "width")):
            count(value, name, minimum=1)
        spatial = 2 * (head_dim // 6)
        parts = []
        for dim, extent in zip((head_dim - 2 * spatial, spatial, spatial), extents):
            inverse = 1.0 / (base ** (torch.arange(0, dim, 2)[: dim // 2].float() / dim))
            positions = torch.from_numpy(np.arange(extent, dtype=np.float32))
            angles = positions[:, None] * inverse[None, :]
            parts.append((angles.cos(), angles.sin()))
        cos, sin, sections, rows = _assemble_sections(parts, torch.float32, torch.device("cpu"))
        return cls(cos.to(device), sin.to(device), sections, rows)

    def _stamp(self):
        """What the cached copies depend on: version counters, or (inference tensors, which track
        none) the storages."""
        if self._inference:
            return (self.cos.data_ptr(), self.sin.data_ptr())
        return (self.cos._version, self.sin._version)

    def invalidate(self):
        """Drop the cached device copies (after updating inference-tensor tables in place)."""
        self._device_cache.clear()

    def _kernel_block(self, device, stream):
        """The table's :class:`_DeviceTable` on ``device``, ordered before work enqueued next on ``stream``."""
        device = _table_device(device)
        stamp = self._stamp()
        entry = self._device_cache.get(device)
        if entry is None or entry.stamp != stamp:
            entry = self._device_cache[device] = _DeviceTable(self.cos, self.sin, device, stream, stamp)
        entry.fence(device, stream)
        return entry

    def kernel_tables(self, device, stream=None):
        """Contiguous float32 ``(cos, sin)`` on ``device``, valid for work enqueued next on ``stream``."""
        entry = self._kernel_block(device, stream)
        return entry.cos, entry.sin

    def kernel_pairs(self, device, stream=None):
        """Interleaved float32 ``[rows, pairs, 2]`` (cos, sin) on ``device``, valid for work enqueued
        next on ``stream`` (built with :meth:`kernel_tables`' copies and ordered by the same event)."""
        return self._kernel_block(device, stream).pairs


@dataclass(frozen=True, eq=False)
class RopePositions:
    """Original positions of one chunk in a :class:`RopeTable`.

    Separable tables take ``rows=(t_row, h_row, w_row)`` (an int means
    ``(t_row, 0, 0)``); dense tables take ``rows=first_row``.
    """

    table: RopeTable
    rows: Any = 0

    def __post_init__(self):
        need(isinstance(self.table, RopeTable), "RoPE positions require a RopeTable")
        if self.table.sections is None:
            count(self.rows, "dense RoPE row")
            return
        rows = (self.rows, 0, 0) if type(self.rows) is int else tuple(self.rows)
        need(len(rows) == 3, "separable RoPE positions are (t_row, h_row, w_row)")
        for value in rows:
            count(value, "RoPE row")
        object.__setattr__(self, "rows", rows)


# ---------------------------------------------------------------------------
# Sources
# ---------------------------------------------------------------------------


def _affine_pair(scale, offset, columns):
    scale, offset = host_floats(scale, columns, "scale"), host_floats(offset, columns, "offset")
    need(not np.any(scale < 0), "affine scales must be nonnegative")
    return scale, offset


@dataclass(frozen=True, eq=False)
class CoefficientSource:
    """Coefficients ``[N, >= rank]`` already unpacked from their pictures.

    Float values are used as is; ``uint8`` values are quantized pixels with the
    per-column FP32 affine ``scale``/``offset`` as host arrays.  ``bound``
    optionally bounds ``|values|`` for the FP16 modes' power-of-two prescale.
    """

    values: torch.Tensor
    scale: Any = None
    offset: Any = None
    bound: float | None = None

    def __post_init__(self):
        values = strided(self.values, "coefficients")
        need(values.ndim == 2, "coefficients must be a [tokens, rank] matrix")
        _bound(self.bound, "bound")
        if values.dtype == torch.uint8:
            need(self.scale is not None and self.offset is not None,
                 "quantized coefficients require their affine scale and offset")
            scale, offset = _affine_pair(self.scale, self.offset, values.shape[1])
            object.__setattr__(self, "scale", scale)
            object.__setattr__(self, "offset", offset)
            return
        need(values.dtype in COEFFICIENT_DTYPES,
             "coefficients must be uint8 pixels or float32/float16/bfloat16 values")
        need(self.scale is None and self.offset is None, "dequantized coefficients take no affine")

    @property
    def quantized(self):
        return self.values.dtype == torch.uint8


_LAYOUT_COUNTS = ("frames", "height", "width", "rank", "planes", "channels_per_segment", "segments")


@dataclass(frozen=True, eq=False)
class PictureSource:
    """Quantized coefficients read in place from decoded pictures.

    ``pictures[segment][frame]`` is a uint8 view ``[planes, rows, columns]``
    whose origin is this matrix's rectangle; all views share plane and row
    strides and have unit column stride.  ``layout`` is the matrix's
    ``reelcache.channel_tiles.v1`` layout, ``scale``/``offset`` its expanded affine.
    """

    pictures: Any
    layout: Mapping
    scale: Any
    offset: Any

    def __post_init__(self):
        layout = self.layout
        need(isinstance(layout, Mapping) and all(name in layout for name in _LAYOUT_COUNTS + ("grid",)),
             "picture layout must be a reelcache.channel_tiles.v1 layout")
        for name in _LAYOUT_COUNTS:
            count(layout[name], f"layout {name}", minimum=1)
        columns, rows = layout["grid"]
        count(columns, "grid columns", minimum=1)
        count(rows, "grid rows", minimum=1)
        slots = layout["channels_per_segment"]
        need(slots == columns * rows * layout["planes"] and layout["segments"] == math.ceil(layout["rank"] / slots),
             "picture layout slot/segment counts are inconsistent")
        pictures = tuple(tuple(segment) for segment in self.pictures)
        need(len(pictures) == layout["segments"] and all(len(segment) == layout["frames"] for segment in pictures),
             "pictures must be indexed [segment][frame] for every segment and frame")
        extent = (layout["planes"], rows * layout["height"], columns * layout["width"])
        shared = set()
        for picture in (picture for segment in pictures for picture in segment):
            strided(picture, "picture")
            need(picture.dtype == torch.uint8 and picture.ndim == 3, "pictures must be uint8 [planes, rows, columns] views")
            need(all(have >= want for have, want in zip(picture.shape, extent)),
                 "picture view does not cover the matrix rectangle")
            need(picture.stride(2) == 1, "picture rows must be contiguous (unit column stride)")
            shared.add((picture.stride(0), picture.stride(1), picture.device))
        need(len(shared) == 1, "pictures of one matrix must share plane/row strides and device")
        scale, offset = _affine_pair(self.scale, self.offset, layout["rank"])
        object.__setattr__(self, "pictures", pictures)
        object.__setattr__(self, "scale", scale)
        object.__setattr__(self, "offset", offset)

    @property
    def device(self):
        return self.pictures[0][0].device

    @property
    def rank(self):
        return self.layout["rank"]

    @property
    def plane_stride(self):
        return self.pictures[0][0].stride(0)

    @property
    def row_stride(self):
        return self.pictures[0][0].stride(1)

    @classmethod
    def from_canvases(cls, canvases, layout, picture_indices, origins, scale, offset):
        """Views on decoded canvases ``[pictures, planes, height, width]``.

        ``picture_indices[segment][frame]`` selects the canvas picture; ``origins`` is
        one ``(y, x)`` for the matrix or a ``[segment][frame]`` table of origins.
        """
        canvases = strided(canvases, "canvases")
        need(canvases.ndim == 4 and canvases.dtype == torch.uint8, "canvases must be uint8 [pictures, planes, height, width]")
        one_origin = len(origins) == 2 and all(type(value) is int for value in origins)

        def view(segment, frame, picture):
            y, x = origins if one_origin else origins[segment][frame]
            count(picture, "picture index")
            count(y, "rectangle y")
            count(x, "rectangle x")
            need(picture < canvases.shape[0], "picture index is outside the canvases")
            return canvases[picture, :, y:, x:]

        pictures = tuple(tuple(view(segment, frame, picture) for frame, picture in enumerate(row))
                         for segment, row in enumerate(picture_indices))
        return cls(pictures, layout, scale, offset)


@dataclass(frozen=True, eq=False)
class DenseSource:
    """An uncompressed canonical ``[N, C]`` matrix (RAW archive, exact path)."""

    values: torch.Tensor

    def __post_init__(self):
        matrix(self.values, "dense values", COEFFICIENT_DTYPES, "a float32/float16/bfloat16 [tokens, channels] matrix")


# ---------------------------------------------------------------------------
# Jobs
# ---------------------------------------------------------------------------


@dataclass(frozen=True, eq=False)
class ReconstructionJob:
    """Reconstruct one restored matrix into one native destination slot.

    ``grid=(frames, height, width)`` is the chunk's token geometry.  Factorized
    sources need ``basis`` (rows ``[R, C]``) and use the prefix view
    ``basis[:rank]`` (``rank`` defaults to the source's coefficient columns).
    ``rope=None`` writes without rotation (V, or pre-RoPE K caches such as LongCat's).
    """

    source: Any
    destination: NativeView
    grid: tuple
    basis: torch.Tensor | None = None
    rank: int | None = None
    rope: RopePositions | None = None
    label: str | None = None

    def __post_init__(self):
        need(isinstance(self.source, (CoefficientSource, PictureSource, DenseSource)),
             "source must be a CoefficientSource, PictureSource or DenseSource")
        need(isinstance(self.destination, NativeView), "destination must be a NativeView")
        grid = tuple(self.grid)
        need(len(grid) == 3, "grid must be (frames, height, width)")
        for value in grid:
            count(value, "grid size", minimum=1)
        object.__setattr__(self, "grid", grid)
        need(self.destination.token_offset + self.tokens <= self.destination.capacity,
             "destination slot exceeds the native cache capacity")
        if isinstance(self.source, DenseSource):
            self._check_dense()
        else:
            object.__setattr__(self, "rank", self._check_factorized())
        if self.rope is not None:
            self._check_rope()

    def _check_dense(self):
        need(self.basis is None and self.rank is None, "dense sources take no basis or rank")
        need(tuple(self.source.values.shape) == (self.tokens, self.channels),
             "dense values must be [tokens, heads * head_dim]")

    def _check_factorized(self):
        basis = strided(self.basis, "basis")
        need(basis.ndim == 2 and basis.shape[1] == self.channels, "basis must be [rows, heads * head_dim] of the destination")
        need(basis.dtype in (torch.float16, torch.bfloat16, torch.float32),
             "basis must be float16 rows (bfloat16 accepted; float32 for reference use)")
        source = self.source
        if isinstance(source, PictureSource):
            geometry = tuple(source.layout[name] for name in ("frames", "height", "width"))
            need(geometry == self.grid, "picture layout geometry differs from the job grid")
            columns = source.layout["rank"]
        else:
            need(source.values.shape[0] == self.tokens, "coefficient rows differ from the job token count")
            columns = source.values.shape[1]
        rank = columns if self.rank is None else self.rank
        count(rank, "rank", minimum=1)
        need(rank <= basis.shape[0], "rank view exceeds the basis rows")
        need(rank <= columns and not (isinstance(source, PictureSource) and rank != columns),
             "rank view exceeds the available coefficient columns")
        return rank

    def _check_rope(self):
        need(isinstance(self.rope, RopePositions), "rope must be RopePositions")
        table = self.rope.table
        need(table.head_dim == self.destination.head_dim, "RoPE table pairs differ from head_dim // 2")
        if table.sections is None:
            need(self.rope.rows + self.tokens <= table.rows, "dense RoPE rows exceed the table")
            return
        reach = [row + extent for row, extent in zip(self.rope.rows, self.grid)]
        need(all(end <= limit or pairs == 0 for end, limit, pairs in zip(reach, table.section_rows, table.sections)),
             "separable RoPE rows exceed the table")

    @property
    def tokens(self):
        return math.prod(self.grid)

    @property
    def channels(self):
        return self.destination.channels

    def tensors(self):
        """Every tensor this job reads or writes (for lifetime tracking)."""
        source = self.source
        inputs = ([picture for segment in source.pictures for picture in segment] if isinstance(source, PictureSource)
                  else [source.values])
        extra = [] if self.basis is None else [self.basis]
        tables = [] if self.rope is None else [self.rope.table.cos, self.rope.table.sin]
        return [self.destination.tensor, *inputs, *extra, *tables]


def expand_affine(affine, normalization, rank):
    """Per-column ``(scale, offset)`` from a packet affine payload ``[2, records]``.

    ``per_channel``: one record per column.  ``global`` / ``leading_columns``:
    record 0 is shared by the unprotected columns and records ``1..count`` belong
    to the leading ``protected_count`` columns (reelcache/restore_kernels.py:204-227,
    reelcache/_hevc.py:475-483).
    """
    affine = np.asarray(affine)
    need(affine.dtype == np.dtype("<f4") and affine.ndim == 2 and affine.shape[0] == 2,
         "affine must be a little-endian float32 [2, records] array")
    need(isinstance(normalization, Mapping) and "mode" in normalization,
         "normalization must be the packet normalization layout")
    count(rank, "rank", minimum=1)
    if normalization["mode"] == "per_channel":
        need(affine.shape[1] == rank, "per-channel affine must have one record per rank column")
        return affine[0].copy(), affine[1].copy()
    protected = normalization["protected_count"]
    need(type(protected) is int and 0 <= protected <= rank and affine.shape[1] == protected + 1,
         "affine record count differs from the protected columns")
    # Record index of every column: its own record for the protected leading columns, 0 otherwise.
    record = np.zeros(rank, dtype=np.int64)
    record[:protected] = np.arange(1, protected + 1)
    return affine[0, record].astype(np.float32), affine[1, record].astype(np.float32)
