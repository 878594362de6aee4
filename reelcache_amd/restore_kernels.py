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

import math
import threading
import time
from collections.abc import Mapping, Sequence
from dataclasses import dataclass, field
from typing import Any

import numpy as np
import torch

from . import _lib
from .errors import ConfigurationError, IntegrityError, StateError, UnsupportedError

LAYOUTS = ("BTHD", "THD", "BHTD")
PRECISIONS = ("fp32", "tf32", "tf32x3", "fp16", "fp16x2", "bf16")
BACKENDS = ("auto", "reference", "fused", "two_pass", "staged", "interpret")
OUTPUT_DTYPES = (torch.bfloat16, torch.float16, torch.float32)
COEFFICIENT_DTYPES = (torch.float32, torch.float16, torch.bfloat16)
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


def _int(value, name, *, minimum=0):
    if type(value) is not int or value < minimum:
        raise ConfigurationError(f"{name} must be an integer >= {minimum}")
    return value


def _require_tensor(value, name):
    if not isinstance(value, torch.Tensor) or value.layout != torch.strided:
        raise ConfigurationError(f"{name} must be a strided torch.Tensor")
    if value.device.type == "meta":
        raise ConfigurationError(f"{name} cannot be a meta tensor")
    return value


def _host_vector(value, length, name):
    """FP32 host copy of a per-rank-column affine vector."""
    if isinstance(value, torch.Tensor):
        if value.device.type != "cpu":
            raise ConfigurationError(f"{name} must be a host array; pass the packet affine payload")
        value = value.detach().numpy()
    array = np.asarray(value)
    if array.dtype != np.float32 or array.shape != (length,):
        raise ConfigurationError(f"{name} must be a float32 vector with one entry per rank column")
    if not np.isfinite(array).all():
        raise ConfigurationError(f"{name} must be finite")
    return np.ascontiguousarray(array)


def expand_affine(affine, normalization, rank):
    """Per-column ``(scale, offset)`` from a packet affine payload ``[2, records]``.

    ``per_channel``: one record per column.  ``global`` / ``leading_columns``:
    record 0 is shared by the unprotected columns and records ``1..count`` belong
    to the leading ``protected_count`` columns (reelcache/restore_kernels.py:204-227,
    reelcache/_hevc.py:475-483).
    """
    affine = np.asarray(affine)
    if affine.dtype != np.dtype("<f4") or affine.ndim != 2 or affine.shape[0] != 2:
        raise ConfigurationError("affine must be a little-endian float32 [2, records] array")
    if not isinstance(normalization, Mapping) or "mode" not in normalization:
        raise ConfigurationError("normalization must be the packet normalization layout")
    _int(rank, "rank", minimum=1)
    if normalization["mode"] == "per_channel":
        if affine.shape[1] != rank:
            raise ConfigurationError("per-channel affine must have one record per rank column")
        return affine[0].copy(), affine[1].copy()
    count = normalization["protected_count"]
    if type(count) is not int or not 0 <= count <= rank or affine.shape[1] != count + 1:
        raise ConfigurationError("affine record count differs from the protected columns")
    scale = np.full(rank, affine[0, 0], dtype=np.float32)
    offset = np.full(rank, affine[1, 0], dtype=np.float32)
    scale[:count] = affine[0, 1:]
    offset[:count] = affine[1, 1:]
    return scale, offset


# ---------------------------------------------------------------------------
# Destinations, RoPE tables and sources
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
        tensor = _require_tensor(self.tensor, "destination tensor")
        if self.layout not in LAYOUTS:
            raise ConfigurationError(f"destination layout must be one of {LAYOUTS}")
        if tensor.ndim != (3 if self.layout == "THD" else 4):
            raise ConfigurationError(f"{self.layout} destination has the wrong number of dimensions")
        if tensor.dtype not in OUTPUT_DTYPES:
            raise ConfigurationError("destination dtype must be bfloat16, float16 or float32")
        _int(self.token_offset, "token_offset")
        _int(self.batch_index, "batch_index")
        if self.layout == "THD" and self.batch_index:
            raise ConfigurationError("a packed THD destination has no batch dimension")
        if self.layout != "THD" and self.batch_index >= tensor.shape[0]:
            raise ConfigurationError("batch_index is outside the destination")
        if self.head_dim % 2:
            raise ConfigurationError("head_dim must be even")
        if any(size > 1 and stride == 0 for size, stride in zip(tensor.shape, tensor.stride())):
            raise ConfigurationError("destination views with broadcast (zero) strides alias")

    @property
    def heads(self):
        return self.tensor.shape[1] if self.layout == "BHTD" else self.tensor.shape[-2]

    @property
    def head_dim(self):
        return self.tensor.shape[-1]

    @property
    def channels(self):
        return self.heads * self.head_dim

    @property
    def capacity(self):
        return self.tensor.shape[2] if self.layout == "BHTD" else self.tensor.shape[-3]

    def strides(self):
        """Element strides of (token, head, dim)."""
        stride = self.tensor.stride()
        if self.layout == "BHTD":
            return stride[2], stride[1], stride[3]
        return stride[-3], stride[-2], stride[-1]

    def element_offset(self):
        """Element offset (in the storage) of (batch_index, token_offset, head 0, dim 0)."""
        base = self.tensor.storage_offset()
        if self.layout != "THD":
            base += self.batch_index * self.tensor.stride(0)
        return base + self.token_offset * self.strides()[0]

    def slot(self, tokens):
        """A ``[tokens, H, D]`` view of the destination slot."""
        stop = self.token_offset + tokens
        if self.layout == "THD":
            return self.tensor[self.token_offset:stop]
        if self.layout == "BTHD":
            return self.tensor[self.batch_index, self.token_offset:stop]
        return self.tensor[self.batch_index, :, self.token_offset:stop].transpose(0, 1)


def wan_sections(pairs):
    """Wan/LongCat 3-D split of ``pairs = head_dim // 2`` into (t, h, w) pair counts."""
    _int(pairs, "pairs", minimum=1)
    third = pairs // 3
    return (pairs - 2 * third, third, third)


_UPLOAD_STREAMS: dict = {}
_UPLOAD_LOCK = threading.Lock()


def _upload_stream(device):
    """Private per-device stream for RoPE-table uploads (default priority)."""
    with _UPLOAD_LOCK:
        stream = _UPLOAD_STREAMS.get(device)
        if stream is None:
            stream = _UPLOAD_STREAMS[device] = torch.cuda.Stream(device)
        return stream


class _KernelTables:
    """FP32 device copies of one table -- ``cos``, ``sin`` and the interleaved ``pairs``
    ``[rows, pairs, 2]`` the straight-line kernels read -- and the event that completes all three.

    Every consumer stream waits on the event (``order_before``) until it has completed, so a
    call on any stream that finds the cached entry cannot read a table before it is written."""

    __slots__ = ("cos", "event", "pairs", "sin", "staging", "stamp")

    def __init__(self, cos, sin, pairs, stamp, event=None, staging=None):
        self.cos, self.sin, self.pairs, self.stamp, self.event, self.staging = cos, sin, pairs, stamp, event, staging

    @classmethod
    def make(cls, cos, sin, device, stream, stamp):
        on_device = device.type == "cuda"
        with torch.inference_mode(False), torch.no_grad():
            if not on_device:
                cos32, sin32 = (t.to(device=device, dtype=torch.float32).contiguous() for t in (cos, sin))
                return cls(cos32, sin32, torch.stack((cos32, sin32), dim=-1).contiguous(), stamp)
            if torch.cuda.is_current_stream_capturing():
                # Work enqueued now would only run when the graph replays, and eager calls
                # before the first replay would read unwritten tables.
                raise ConfigurationError("a RoPE table's device copy cannot be built during HIP-graph capture: "
                                         "run one call with the table (or warmup) before capturing")
            staging = None
            if cos.device.type == "cpu":
                # Read the host tables now into private pinned memory; upload on a private stream.
                staging = tuple(torch.empty(t.shape, dtype=torch.float32, pin_memory=True).copy_(t) for t in (cos, sin))
                work = _upload_stream(device)
            else:
                work = torch.cuda.current_stream(device) if stream is None else stream
            with torch.cuda.stream(work):
                if staging is not None:
                    cos32, sin32 = (torch.empty(t.shape, dtype=torch.float32, device=device) for t in staging)
                    cos32.copy_(staging[0], non_blocking=True)
                    sin32.copy_(staging[1], non_blocking=True)
                else:
                    # A contiguous float32 device table is used in place; other dtypes / layouts
                    # are converted after the work already enqueued on the caller's stream.
                    cos32, sin32 = (t.to(device=device, dtype=torch.float32).contiguous() for t in (cos, sin))
                pairs = torch.stack((cos32, sin32), dim=-1).contiguous()
                event = torch.cuda.Event()
                event.record(work)
            return cls(cos32, sin32, pairs, stamp, event, staging)

    def order_before(self, device, stream):
        """Make ``stream`` (default: current) wait for the copies; no-op once complete."""
        event = self.event
        if event is None:
            return
        if event.query():
            self.event = None
            self.staging = None
            return
        (torch.cuda.current_stream(device) if stream is None else stream).wait_event(event)


@dataclass(frozen=True, eq=False)
class RopeTable:
    """cos/sin rotation tables ``[R, head_dim // 2]`` for interleaved pairs.

    ``sections=(t, h, w)`` makes the table separable: pair ``j`` of a token at
    (frame f, row y, column x) uses row ``t_row + f`` when ``j < t``, row
    ``h_row + y`` when ``j < t + h`` and row ``w_row + x`` otherwise.
    ``sections=None`` is a dense per-token table (row ``row + n`` for token ``n``).
    Tables are float64 or float32; the GPU kernels use float32 device copies
    (:meth:`kernel_tables`), the reference backend the table's own precision.
    """

    cos: torch.Tensor
    sin: torch.Tensor
    sections: tuple | None = None
    section_rows: tuple | None = None
    _device_cache: dict = field(default_factory=dict, init=False, repr=False, compare=False)
    _inference: bool = field(default=False, init=False, repr=False, compare=False)

    def __post_init__(self):
        cos, sin = _require_tensor(self.cos, "RoPE cos"), _require_tensor(self.sin, "RoPE sin")
        if (cos.ndim != 2 or cos.shape != sin.shape or cos.dtype != sin.dtype
                or cos.dtype not in (torch.float32, torch.float64) or cos.device != sin.device or min(cos.shape) < 1):
            raise ConfigurationError("RoPE cos/sin must be matching float32/float64 [rows, head_dim // 2] tensors")
        object.__setattr__(self, "_inference", cos.is_inference() or sin.is_inference())
        rows, pairs = cos.shape
        if self.sections is not None:
            sections = tuple(self.sections)
            if len(sections) != 3 or any(type(v) is not int or v < 0 for v in sections) or sum(sections) != pairs:
                raise ConfigurationError("RoPE sections must be three nonnegative pair counts summing to head_dim // 2")
            object.__setattr__(self, "sections", sections)
            limits = (rows, rows, rows) if self.section_rows is None else tuple(self.section_rows)
            if len(limits) != 3 or any(type(v) is not int or not 0 <= v <= rows for v in limits):
                raise ConfigurationError("section_rows must be three row counts within the table")
            object.__setattr__(self, "section_rows", limits)
        elif self.section_rows is not None:
            raise ConfigurationError("section_rows requires separable sections")

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
        freqs = _require_tensor(freqs, "freqs")
        if not freqs.is_complex() or freqs.ndim != 2:
            raise ConfigurationError("freqs must be a complex [rows, head_dim // 2] tensor")
        real = torch.view_as_real(freqs.resolve_conj())
        dtype = torch.float64 if freqs.dtype == torch.complex128 else torch.float32
        if sections == "wan":
            sections = wan_sections(freqs.shape[1])
        return cls(real[..., 0].to(dtype).contiguous(), real[..., 1].to(dtype).contiguous(), sections)

    @classmethod
    def from_axes(cls, temporal, height, width):
        """Separable table from per-axis complex tensors ``[positions, pairs]`` (unused cells NaN)."""
        axes = [_require_tensor(value, "axis freqs") for value in (temporal, height, width)]
        if any(not value.is_complex() or value.ndim != 2 for value in axes):
            raise ConfigurationError("axis frequencies must be complex [positions, pairs] tensors")
        if len({value.device for value in axes}) != 1:
            raise ConfigurationError("axis frequencies must share a device")
        dtype = torch.float64 if all(value.dtype == torch.complex128 for value in axes) else torch.float32
        rows = max(value.shape[0] for value in axes)
        pairs = sum(value.shape[1] for value in axes)
        cos = torch.full((rows, pairs), float("nan"), dtype=dtype, device=axes[0].device)
        sin = torch.full_like(cos, float("nan"))
        column = 0
        for value in axes:
            real = torch.view_as_real(value.resolve_conj()).to(dtype)
            cos[:value.shape[0], column:column + value.shape[1]] = real[..., 0]
            sin[:value.shape[0], column:column + value.shape[1]] = real[..., 1]
            column += value.shape[1]
        return cls(cos, sin, tuple(value.shape[1] for value in axes), tuple(value.shape[0] for value in axes))

    @classmethod
    def from_cos_sin(cls, cos, sin, sections=None):
        """From real tables, e.g. SGLang's dense ``freqs_cis = (cos, sin)``."""
        return cls(cos, sin, sections)

    @classmethod
    def longcat(cls, head_dim, num_frames, height, width, *, base=10000.0, device="cpu"):
        """LongCat-Video ``rope_3d`` tables in float32 (angles and cos/sin of float32 angles).

        LongCat's KV cache stores pre-RoPE K, so restored LongCat caches are written
        without rotation; the table serves the engine's own RoPE.
        """
        _int(head_dim, "head_dim", minimum=8)
        if head_dim % 8:
            raise ConfigurationError("LongCat 3D RoPE requires head_dim divisible by 8")
        for value, name in ((num_frames, "num_frames"), (height, "height"), (width, "width")):
            _int(value, name, minimum=1)
        sixth = head_dim // 6
        dims = (head_dim - 4 * sixth, 2 * sixth, 2 * sixth)
        tables = []
        for dim, count in zip(dims, (num_frames, height, width)):
            inverse = 1.0 / (base ** (torch.arange(0, dim, 2)[: dim // 2].float() / dim))
            grid = torch.from_numpy(np.linspace(0, count, count, endpoint=False, dtype=np.float32)).float()
            tables.append(grid[:, None] * inverse[None, :])
        rows = max(table.shape[0] for table in tables)
        pairs = sum(table.shape[1] for table in tables)
        cos = torch.full((rows, pairs), float("nan"), dtype=torch.float32)
        sin = torch.full_like(cos, float("nan"))
        column = 0
        for table in tables:
            cos[:table.shape[0], column:column + table.shape[1]] = table.cos()
            sin[:table.shape[0], column:column + table.shape[1]] = table.sin()
            column += table.shape[1]
        return cls(cos.to(device), sin.to(device), tuple(t.shape[1] for t in tables), tuple(t.shape[0] for t in tables))

    def _stamp(self):
        if self._inference:
            return (self.cos.data_ptr(), self.sin.data_ptr())
        return (self.cos._version, self.sin._version)

    def invalidate(self):
        """Drop the cached device copies (after updating inference-tensor tables in place)."""
        self._device_cache.clear()

    def kernel_tables(self, device, stream=None):
        """Contiguous float32 ``(cos, sin)`` on ``device``, valid for work enqueued next on ``stream``."""
        device = torch.device(device)
        if device.type == "cuda" and device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        stamp = self._stamp()
        entry = self._device_cache.get(device)
        if entry is None or entry.stamp != stamp:
            entry = _KernelTables.make(self.cos, self.sin, device, stream, stamp)
            self._device_cache[device] = entry
        if entry.event is not None:
            entry.order_before(device, stream)
        return entry.cos, entry.sin

    def kernel_pairs(self, device, stream=None):
        """Interleaved float32 ``[rows, pairs, 2]`` (cos, sin) on ``device``, valid for work enqueued
        next on ``stream`` (built with :meth:`kernel_tables`' copies and ordered by the same event)."""
        cos, _ = self.kernel_tables(device, stream)
        return self._device_cache[cos.device].pairs


@dataclass(frozen=True, eq=False)
class RopePositions:
    """Original positions of one chunk in a :class:`RopeTable`.

    Separable tables take ``rows=(t_row, h_row, w_row)`` (an int means
    ``(t_row, 0, 0)``); dense tables take ``rows=first_row``.
    """

    table: RopeTable
    rows: Any = 0

    def __post_init__(self):
        if not isinstance(self.table, RopeTable):
            raise ConfigurationError("RoPE positions require a RopeTable")
        if self.table.sections is None:
            _int(self.rows, "dense RoPE row")
            return
        rows = (self.rows, 0, 0) if type(self.rows) is int else tuple(self.rows)
        if len(rows) != 3:
            raise ConfigurationError("separable RoPE positions are (t_row, h_row, w_row)")
        for value in rows:
            _int(value, "RoPE row")
        object.__setattr__(self, "rows", rows)


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
        values = _require_tensor(self.values, "coefficients")
        if values.ndim != 2:
            raise ConfigurationError("coefficients must be a [tokens, rank] matrix")
        if self.bound is not None and (isinstance(self.bound, bool) or not isinstance(self.bound, (int, float))
                                       or not math.isfinite(self.bound) or self.bound < 0):
            raise ConfigurationError("bound must be a finite nonnegative upper bound on |coefficients|")
        if values.dtype == torch.uint8:
            if self.scale is None or self.offset is None:
                raise ConfigurationError("quantized coefficients require their affine scale and offset")
            object.__setattr__(self, "scale", _host_vector(self.scale, values.shape[1], "scale"))
            object.__setattr__(self, "offset", _host_vector(self.offset, values.shape[1], "offset"))
            if np.any(self.scale < 0):
                raise ConfigurationError("affine scales must be nonnegative")
        elif values.dtype in COEFFICIENT_DTYPES:
            if self.scale is not None or self.offset is not None:
                raise ConfigurationError("dequantized coefficients take no affine")
        else:
            raise ConfigurationError("coefficients must be uint8 pixels or float32/float16/bfloat16 values")

    @property
    def quantized(self):
        return self.values.dtype == torch.uint8


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
        required = ("frames", "height", "width", "rank", "planes", "grid", "channels_per_segment", "segments")
        if not isinstance(layout, Mapping) or any(name not in layout for name in required):
            raise ConfigurationError("picture layout must be a reelcache.channel_tiles.v1 layout")
        frames, height, width, rank = (layout[name] for name in ("frames", "height", "width", "rank"))
        planes, slots, segments = layout["planes"], layout["channels_per_segment"], layout["segments"]
        for value, name in ((frames, "frames"), (height, "height"), (width, "width"), (rank, "rank"),
                            (planes, "planes"), (slots, "channels_per_segment"), (segments, "segments")):
            _int(value, f"layout {name}", minimum=1)
        columns, rows = layout["grid"]
        _int(columns, "grid columns", minimum=1)
        _int(rows, "grid rows", minimum=1)
        if slots != columns * rows * planes or segments != math.ceil(rank / slots):
            raise ConfigurationError("picture layout slot/segment counts are inconsistent")
        pictures = tuple(tuple(segment) for segment in self.pictures)
        if len(pictures) != segments or any(len(segment) != frames for segment in pictures):
            raise ConfigurationError("pictures must be indexed [segment][frame] for every segment and frame")
        strides = device = None
        for segment in pictures:
            for picture in segment:
                _require_tensor(picture, "picture")
                if picture.dtype != torch.uint8 or picture.ndim != 3:
                    raise ConfigurationError("pictures must be uint8 [planes, rows, columns] views")
                if picture.shape[0] < planes or picture.shape[1] < rows * height or picture.shape[2] < columns * width:
                    raise ConfigurationError("picture view does not cover the matrix rectangle")
                if picture.stride(2) != 1:
                    raise ConfigurationError("picture rows must be contiguous (unit column stride)")
                current = (picture.stride(0), picture.stride(1))
                if strides is None:
                    strides, device = current, picture.device
                elif current != strides or picture.device != device:
                    raise ConfigurationError("pictures of one matrix must share plane/row strides and device")
        object.__setattr__(self, "pictures", pictures)
        object.__setattr__(self, "scale", _host_vector(self.scale, rank, "scale"))
        object.__setattr__(self, "offset", _host_vector(self.offset, rank, "offset"))
        if np.any(self.scale < 0):
            raise ConfigurationError("affine scales must be nonnegative")

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
        canvases = _require_tensor(canvases, "canvases")
        if canvases.ndim != 4 or canvases.dtype != torch.uint8:
            raise ConfigurationError("canvases must be uint8 [pictures, planes, height, width]")
        single = len(origins) == 2 and all(type(value) is int for value in origins)
        pictures = []
        for segment_index, segment in enumerate(picture_indices):
            row = []
            for frame_index, picture in enumerate(segment):
                y, x = origins if single else origins[segment_index][frame_index]
                _int(picture, "picture index")
                _int(y, "rectangle y")
                _int(x, "rectangle x")
                if picture >= canvases.shape[0]:
                    raise ConfigurationError("picture index is outside the canvases")
                row.append(canvases[picture, :, y:, x:])
            pictures.append(tuple(row))
        return cls(tuple(pictures), layout, scale, offset)


@dataclass(frozen=True, eq=False)
class DenseSource:
    """An uncompressed canonical ``[N, C]`` matrix (RAW archive, exact path)."""

    values: torch.Tensor

    def __post_init__(self):
        values = _require_tensor(self.values, "dense values")
        if values.ndim != 2 or values.dtype not in COEFFICIENT_DTYPES:
            raise ConfigurationError("dense values must be a float32/float16/bfloat16 [tokens, channels] matrix")


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
        if not isinstance(self.source, (CoefficientSource, PictureSource, DenseSource)):
            raise ConfigurationError("source must be a CoefficientSource, PictureSource or DenseSource")
        if not isinstance(self.destination, NativeView):
            raise ConfigurationError("destination must be a NativeView")
        grid = tuple(self.grid)
        if len(grid) != 3:
            raise ConfigurationError("grid must be (frames, height, width)")
        for value in grid:
            _int(value, "grid size", minimum=1)
        object.__setattr__(self, "grid", grid)
        tokens, channels = self.tokens, self.destination.channels
        if self.destination.token_offset + tokens > self.destination.capacity:
            raise ConfigurationError("destination slot exceeds the native cache capacity")
        if isinstance(self.source, DenseSource):
            if self.basis is not None or self.rank is not None:
                raise ConfigurationError("dense sources take no basis or rank")
            if tuple(self.source.values.shape) != (tokens, channels):
                raise ConfigurationError("dense values must be [tokens, heads * head_dim]")
        else:
            basis = _require_tensor(self.basis, "basis")
            if basis.ndim != 2 or basis.shape[1] != channels:
                raise ConfigurationError("basis must be [rows, heads * head_dim] of the destination")
            if basis.dtype not in (torch.float16, torch.bfloat16, torch.float32):
                raise ConfigurationError("basis must be float16 rows (bfloat16 accepted; float32 for reference use)")
            if isinstance(self.source, PictureSource):
                layout = self.source.layout
                if (layout["frames"], layout["height"], layout["width"]) != grid:
                    raise ConfigurationError("picture layout geometry differs from the job grid")
                columns = layout["rank"]
            else:
                if self.source.values.shape[0] != tokens:
                    raise ConfigurationError("coefficient rows differ from the job token count")
                columns = self.source.values.shape[1]
            rank = columns if self.rank is None else self.rank
            _int(rank, "rank", minimum=1)
            if rank > basis.shape[0]:
                raise ConfigurationError("rank view exceeds the basis rows")
            if rank > columns or (isinstance(self.source, PictureSource) and rank != columns):
                raise ConfigurationError("rank view exceeds the available coefficient columns")
            object.__setattr__(self, "rank", rank)
        if self.rope is not None:
            if not isinstance(self.rope, RopePositions):
                raise ConfigurationError("rope must be RopePositions")
            table = self.rope.table
            if table.head_dim != self.destination.head_dim:
                raise ConfigurationError("RoPE table pairs differ from head_dim // 2")
            if table.sections is None:
                if self.rope.rows + tokens > table.rows:
                    raise ConfigurationError("dense RoPE rows exceed the table")
            else:
                needed = tuple(row + size for row, size in zip(self.rope.rows, grid))
                if any(need > limit for need, limit, pairs in zip(needed, table.section_rows, table.sections) if pairs):
                    raise ConfigurationError("separable RoPE rows exceed the table")

    @property
    def tokens(self):
        frames, height, width = self.grid
        return frames * height * width

    @property
    def channels(self):
        return self.destination.channels

    def tensors(self):
        """Every tensor this job reads or writes (for lifetime tracking)."""
        result = [self.destination.tensor]
        source = self.source
        if isinstance(source, PictureSource):
            result.extend(picture for segment in source.pictures for picture in segment)
        else:
            result.append(source.values)
        if self.basis is not None:
            result.append(self.basis)
        if self.rope is not None:
            result.extend((self.rope.table.cos, self.rope.table.sin))
        return result


# ---------------------------------------------------------------------------
# Completion handle
# ---------------------------------------------------------------------------

_DEFERRED: list = []
_DEFERRED_LOCK = threading.RLock()


def _sweep_deferred():
    """Drop references of collected-but-unreleased handles whose GPU work has finished."""
    with _DEFERRED_LOCK:
        if _DEFERRED:
            _DEFERRED[:] = [(event, refs) for event, refs in _DEFERRED if not event.query()]


def pending_deferred():
    """Number of collected handles whose inputs are still held until their event completes."""
    with _DEFERRED_LOCK:
        return len(_DEFERRED)


class RestoreHandle:
    """Completion of one :func:`reconstruct` call.

    ``event`` is recorded on the execution stream after the last write (None for
    host execution).  The handle keeps all inputs, tables and temporaries alive
    until :meth:`release`; a handle collected before release parks them until its
    event completes.
    """

    def __init__(self, *, event, stream, keepalive, stats):
        self._event = event
        self._stream = stream
        self._keepalive = keepalive
        self._released = False
        self.stats = stats

    @property
    def event(self):
        return self._event

    @property
    def stream(self):
        return self._stream

    @property
    def released(self):
        return self._released

    def query(self):
        return self._event is None or self._event.query()

    def synchronize(self):
        if self._event is not None:
            self._event.synchronize()

    def wait(self, stream=None):
        """Make ``stream`` (default: current) wait for completion without blocking the host."""
        if self._event is None:
            return
        (torch.cuda.current_stream(self._stream.device) if stream is None else stream).wait_event(self._event)

    def release(self):
        """Wait for completion, then drop every retained input and temporary."""
        if self._released:
            return
        self.synchronize()
        self._keepalive = None
        self._released = True
        _sweep_deferred()

    def __del__(self):
        try:
            if not self._released and self._event is not None and self._keepalive is not None:
                if not self._event.query():
                    with _DEFERRED_LOCK:
                        _DEFERRED.append((self._event, self._keepalive))
        except Exception:  # noqa: BLE001 - interpreter shutdown
            pass


# ---------------------------------------------------------------------------
# Validation and the reference backend
# ---------------------------------------------------------------------------


def _storage_key(tensor):
    try:
        return tensor.untyped_storage().data_ptr(), tensor.device
    except (RuntimeError, NotImplementedError):
        return tensor.data_ptr(), tensor.device


def _check_disjoint(jobs):
    """Reject jobs whose slots in the same destination view overlap (concurrent writes would race)."""
    spans: dict = {}
    for index, job in enumerate(jobs):
        view = job.destination
        tensor = view.tensor
        key = (*_storage_key(tensor), tensor.storage_offset(), tuple(tensor.shape), tensor.stride(),
               view.layout, view.batch_index)
        spans.setdefault(key, []).append((view.token_offset, view.token_offset + job.tokens, index))
    for intervals in spans.values():
        intervals.sort()
        for (_, stop, first), (start, _, second) in zip(intervals, intervals[1:]):
            if start < stop:
                raise ConfigurationError(f"jobs {first} and {second} write overlapping destination tokens")


def _validate(jobs):
    if isinstance(jobs, ReconstructionJob):
        jobs = (jobs,)
    if not isinstance(jobs, Sequence) or isinstance(jobs, (str, bytes)):
        raise ConfigurationError("jobs must be a sequence of ReconstructionJob")
    jobs = tuple(jobs)
    if any(not isinstance(job, ReconstructionJob) for job in jobs):
        raise ConfigurationError("jobs must be ReconstructionJob instances")
    devices = set()
    for job in jobs:
        devices.add(job.destination.tensor.device)
        source = job.source
        devices.add(source.device if isinstance(source, PictureSource) else source.values.device)
        if job.basis is not None:
            devices.add(job.basis.device)
    if len(devices) > 1:
        raise ConfigurationError("all job tensors (except RoPE tables) must share one device")
    _check_disjoint(jobs)
    return jobs, (devices.pop() if devices else None)


def unpack_pictures(source):
    """Quantized coefficient pixels ``[N, rank]`` of a :class:`PictureSource` (channel_tiles.v1)."""
    layout = source.layout
    frames, height, width, rank = layout["frames"], layout["height"], layout["width"], layout["rank"]
    columns, rows = layout["grid"]
    planes, slots = layout["planes"], layout["channels_per_segment"]
    values = torch.empty((frames, height, width, rank), dtype=torch.uint8, device=source.device)
    for segment, pictures in enumerate(source.pictures):
        first = segment * slots
        count = min(slots, rank - first)
        for frame, picture in enumerate(pictures):
            # [planes, rows*height, columns*width] -> cells ordered (row, column, plane) per token.
            cells = picture[:planes, :rows * height, :columns * width].reshape(planes, rows, height, columns, width)
            values[frame, :, :, first:first + count] = cells.permute(2, 4, 1, 3, 0).reshape(height, width, -1)[..., :count]
    return values.reshape(-1, rank)


def dequantize(pixels, scale, offset):
    """``float(pixel) * scale + offset`` with the eager rounding (mul, then add)."""
    scale = torch.from_numpy(np.ascontiguousarray(scale)).to(pixels.device)
    offset = torch.from_numpy(np.ascontiguousarray(offset)).to(pixels.device)
    return pixels.float().mul_(scale).add_(offset)


def reference_coefficients(job):
    """The FP32 coefficient matrix ``[N, rank]`` a job reconstructs from."""
    source = job.source
    if isinstance(source, PictureSource):
        return dequantize(unpack_pictures(source), source.scale, source.offset)
    if isinstance(source, CoefficientSource):
        if source.quantized:
            return dequantize(source.values[:, :job.rank], source.scale[:job.rank], source.offset[:job.rank])
        return source.values[:, :job.rank].float()
    raise ConfigurationError("dense sources have no coefficients")


def rope_cos_sin(positions, grid, *, dtype=torch.float64, device=None):
    """Per-token ``(cos, sin)`` ``[N, head_dim // 2]`` for a job's positions."""
    table = positions.table
    device = table.cos.device if device is None else device
    cos = table.cos.to(device=device, dtype=dtype)
    sin = table.sin.to(device=device, dtype=dtype)
    frames, height, width = grid
    tokens = frames * height * width
    if table.sections is None:
        first = positions.rows
        return cos[first:first + tokens], sin[first:first + tokens]
    index = torch.arange(tokens, device=device)
    plane = height * width
    axes = (index // plane, (index % plane) // width, index % width)
    out_cos = torch.empty((tokens, table.pairs), dtype=dtype, device=device)
    out_sin = torch.empty_like(out_cos)
    column = 0
    for axis, pairs in enumerate(table.sections):
        rows = positions.rows[axis] + axes[axis]
        out_cos[:, column:column + pairs] = cos[rows, column:column + pairs]
        out_sin[:, column:column + pairs] = sin[rows, column:column + pairs]
        column += pairs
    return out_cos, out_sin


def apply_rope_reference(values, positions, grid, *, dtype=torch.float64):
    """Rotate interleaved pairs of ``values[N, H, D]`` in ``dtype`` (Wan complex product)."""
    cos, sin = rope_cos_sin(positions, grid, dtype=dtype, device=values.device)
    x = values.to(dtype)
    even, odd = x[..., 0::2], x[..., 1::2]
    cos, sin = cos[:, None, :], sin[:, None, :]
    out = torch.empty_like(x)
    out[..., 0::2] = even * cos - odd * sin
    out[..., 1::2] = even * sin + odd * cos
    return out


def _pre_rope(job, compute):
    if isinstance(job.source, DenseSource):
        return job.source.values
    coefficients = reference_coefficients(job)
    basis = job.basis[:job.rank]
    return coefficients.to(compute) @ basis.to(device=coefficients.device, dtype=compute)


def fp32_matmul_precision(device_type):
    """Precision this process lets FP32 torch matmuls on ``"cuda"`` or ``"cpu"`` use (read only)."""
    holder = torch.backends.cuda.matmul if device_type == "cuda" else getattr(
        getattr(torch.backends, "mkldnn", None), "matmul", None)
    precision = getattr(holder, "fp32_precision", None)
    if isinstance(precision, str):
        return "ieee" if precision in ("ieee", "none") else precision
    legacy = torch.get_float32_matmul_precision()
    return "ieee" if legacy == "highest" else legacy


def _require_fp32_matmul(device_type, accepted, what):
    actual = fp32_matmul_precision(device_type)
    if actual not in accepted:
        raise UnsupportedError(
            f"{what} needs {device_type} FP32 matmuls at {' / '.join(accepted)} precision, but this process set "
            f"{actual!r}; that setting is process-wide, so restore_kernels never changes it")


def _reference_job(job, compute, native_rope, native_rope_dtype):
    heads, head_dim, tokens = job.destination.heads, job.destination.head_dim, job.tokens
    slot = job.destination.slot(tokens)
    values = _pre_rope(job, compute)
    if native_rope is not None and job.rope is not None:
        dtype = slot.dtype if native_rope_dtype is None else native_rope_dtype
        result = native_rope(values.to(dtype).reshape(tokens, heads, head_dim), job)
        if not isinstance(result, torch.Tensor) or result.numel() != tokens * heads * head_dim:
            raise IntegrityError("native RoPE callable returned a tensor of the wrong size")
        slot.copy_(result.reshape(tokens, heads, head_dim))
        return
    values = values.reshape(tokens, heads, head_dim)
    if job.rope is not None:
        values = apply_rope_reference(values, job.rope, job.grid, dtype=compute)
    slot.copy_(values)


def reconstruct_reference(jobs, *, compute_dtype=torch.float64, native_rope=None, native_rope_dtype=None):
    """Plain-torch reference: FP64 (default) or IEEE FP32 math, then one cast (runs on the jobs' device)."""
    jobs, device = _validate(jobs)
    if compute_dtype not in (torch.float32, torch.float64):
        raise ConfigurationError("reference compute dtype must be float32 or float64")
    if compute_dtype == torch.float32 and device is not None:
        _require_fp32_matmul(device.type, ("ieee",), "the FP32 reference (compute_dtype=torch.float32)")
    with torch.no_grad():
        for job in jobs:
            _reference_job(job, compute_dtype, native_rope, native_rope_dtype)


_UNIT_ROUNDOFF = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11, torch.float32: 2.0 ** -24}
# Smallest-magnitude rounding floor of each output format (half its subnormal spacing).
_OUTPUT_FLOOR = {torch.bfloat16: 2.0 ** -134, torch.float16: 2.0 ** -25, torch.float32: 2.0 ** -150}


def _gemm_gamma(precision, rank):
    """Relative product error per unit of ``sum_k |a_k| |q_k|`` for each precision mode
    (reelcache/restore_kernels.py:1176-1187)."""
    accumulate = (rank + 1) * 2.0 ** -24
    return {
        "fp32": accumulate,
        "tf32": 2.0 ** -10 + accumulate,
        "tf32x3": 2.0 ** -20 + 3 * accumulate,
        "fp16": 2.0 ** -11 + accumulate,
        "fp16x2": 2.0 ** -21 + 2 * accumulate,
        "bf16": 2.0 ** -7 + 2.0 ** -16 + accumulate,
        "reference32": accumulate,
    }[precision]


def reference_values(job):
    """FP64 values ``y*[N, C]`` a job writes before the final cast, and ``sum_k |p_k| |q_k|``."""
    tokens, heads, head_dim = job.tokens, job.destination.heads, job.destination.head_dim
    if isinstance(job.source, DenseSource):
        values = job.source.values.double()
        magnitude = torch.zeros_like(values)
    else:
        coefficients = reference_coefficients(job).double()
        basis = job.basis[:job.rank].to(device=coefficients.device, dtype=torch.float64)
        values = coefficients @ basis
        magnitude = coefficients.abs() @ basis.abs()
    if job.rope is not None:
        values = apply_rope_reference(values.reshape(tokens, heads, head_dim), job.rope, job.grid).reshape(tokens, -1)
        pairs = magnitude.reshape(tokens, -1, 2)
        magnitude = (pairs[..., 0] + pairs[..., 1]).repeat_interleave(2, dim=-1)
    return values, magnitude


def error_bound(job, precision, out_dtype=None):
    """Elementwise bound on ``|written - y*|`` for a precision mode (first-order analysis).

    ``|y_hat - y*| <= u_out |y*| + (1 + u_out) E + floor`` with
    ``E = gamma(precision, rank) * S + 2**-21 (|y_e| + |y_o|)`` (the last term only
    with RoPE), ``S = sum_k |p_k| |q_k|`` summed over each rotated pair
    (reelcache/restore_kernels.py:1208-1227).  Returns ``(y*, bound)`` in FP64.
    """
    values, magnitude = reference_values(job)
    out_dtype = job.destination.tensor.dtype if out_dtype is None else out_dtype
    unit = _UNIT_ROUNDOFF[out_dtype]
    error = _gemm_gamma(precision, job.rank or 0) * magnitude
    if job.rope is not None:
        pairs = values.reshape(job.tokens, -1, 2).abs()
        error = error + 2.0 ** -21 * (pairs[..., 0] + pairs[..., 1]).repeat_interleave(2, dim=-1)
    return values, unit * values.abs() + (1 + unit) * error + _OUTPUT_FLOOR[out_dtype]


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


def _run_hip(jobs, *, precision, config, stream, device, keepalive, stage_events):
    plan = _CallPlan(list(jobs), device, stream, precision, config, keepalive)
    launches = plan.run(stage_events)
    return launches, plan.grids, plan.variants


class _null:
    def __enter__(self):
        return self

    def __exit__(self, *_):
        return False


def _native_rope_jobs(jobs, native_rope, native_rope_dtype, run, stream, keepalive):
    """Exact path: reconstruct pre-RoPE K into temporaries, call the engine's RoPE, copy into the slot."""
    staged, prepared = [], []
    for job in jobs:
        heads, head_dim, tokens = job.destination.heads, job.destination.head_dim, job.tokens
        dtype = job.destination.tensor.dtype if native_rope_dtype is None else native_rope_dtype
        if isinstance(job.source, DenseSource) and job.source.values.dtype == dtype:
            prepared.append((job, job.source.values.reshape(tokens, heads, head_dim)))
            continue
        if dtype not in OUTPUT_DTYPES:
            raise ConfigurationError("native RoPE input dtype must be bfloat16, float16 or float32")
        with torch.cuda.stream(stream) if stream is not None else _null():
            temporary = torch.empty((tokens, heads, head_dim), dtype=dtype, device=job.destination.tensor.device)
        keepalive.append(temporary)
        staged.append(ReconstructionJob(job.source, NativeView(temporary, "THD"), job.grid, job.basis, job.rank, None,
                                        job.label))
        prepared.append((job, temporary))
    launches = run(staged) if staged else 0
    with torch.cuda.stream(stream) if stream is not None else _null():
        for job, values in prepared:
            result = native_rope(values, job)
            heads, head_dim, tokens = job.destination.heads, job.destination.head_dim, job.tokens
            if not isinstance(result, torch.Tensor) or result.numel() != tokens * heads * head_dim:
                raise IntegrityError("native RoPE callable returned a tensor of the wrong size")
            keepalive.append(result)
            job.destination.slot(tokens).copy_(result.reshape(tokens, heads, head_dim))
    return launches


def _matrix_flops(jobs):
    return sum(2 * job.tokens * job.rank * job.channels for job in jobs if job.rank)


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
    (``workgroups_per_cu``, ``store_cost``).  ``stage_events``: optional list
    receiving ``(stage, event)`` timing events ("start", "pack", "launch<n>" after the n-th launch of the
    call, "fused", "rope_store").

    Returns a :class:`RestoreHandle`; destinations are valid after its event.
    """
    _sweep_deferred()
    jobs, device = _validate(jobs)
    if backend not in BACKENDS:
        raise ConfigurationError(f"backend must be one of {BACKENDS}")
    if precision != "auto" and precision not in PRECISIONS:
        raise ConfigurationError(f"precision must be 'auto' or one of {PRECISIONS}")
    if native_rope is not None and not callable(native_rope):
        raise ConfigurationError("native_rope must be callable")
    stats = {"jobs": len(jobs), "matrices": len(jobs), "flops": _matrix_flops(jobs), "launches": 0}
    if not jobs:
        stats.update(backend="none", precision=None)
        return RestoreHandle(event=None, stream=None, keepalive=None, stats=stats)
    cuda = device.type == "cuda"
    resolved = _resolve_backend(backend, cuda)
    if resolved == "reference":
        if compute_dtype not in (torch.float32, torch.float64):
            raise ConfigurationError("reference compute dtype must be float32 or float64")
        if compute_dtype == torch.float32:
            _require_fp32_matmul(device.type, ("ieee",), "the FP32 reference (compute_dtype=torch.float32)")
    else:
        precision = _resolve_precision(precision, device)
    if cuda:
        stream = torch.cuda.current_stream(device) if stream is None else stream
        if not isinstance(stream, torch.cuda.Stream) or stream.device != device:
            raise ConfigurationError("stream must be a torch.cuda.Stream on the jobs' device")
    elif stream is not None or wait_events:
        raise ConfigurationError("host execution takes no GPU stream or events")
    keepalive = [tensor for job in jobs for tensor in job.tensors()]
    stats.update(backend=resolved, precision=precision if resolved != "reference" else str(compute_dtype),
                 picture_path="fused_gather" if resolved == "fused" else resolved)
    if cuda:
        for event in wait_events:
            stream.wait_event(event)
    if resolved == "reference":
        with torch.cuda.stream(stream) if cuda else _null():
            reconstruct_reference(jobs, compute_dtype=compute_dtype, native_rope=native_rope,
                                  native_rope_dtype=native_rope_dtype)
    else:
        merged = _merged_config(config)
        grids, variants = [], []

        def run(selected):
            launches, group_grids, group_variants = _run_hip(selected, precision=precision, config=merged,
                                                             stream=stream, device=device, keepalive=keepalive,
                                                             stage_events=stage_events)
            grids.extend(group_grids)
            variants.extend(group_variants)
            return launches

        exact = [job for job in jobs if native_rope is not None and job.rope is not None]
        ordinary = [job for job in jobs if not (native_rope is not None and job.rope is not None)]
        try:
            with torch.cuda.stream(stream):
                if ordinary:
                    stats["launches"] += run(ordinary)
                if exact:
                    stats["launches"] += _native_rope_jobs(exact, native_rope, native_rope_dtype, run, stream,
                                                           keepalive)
        except BaseException:
            failed = torch.cuda.Event()
            failed.record(stream)
            with _DEFERRED_LOCK:
                _DEFERRED.append((failed, keepalive))
            raise
        stats["grids"] = grids
        stats["variants"] = variants
    event = None
    if cuda:
        event = torch.cuda.Event()
        event.record(stream)
    return RestoreHandle(event=event, stream=stream, keepalive=keepalive, stats=stats)


# ---------------------------------------------------------------------------
# Warm-up
# ---------------------------------------------------------------------------

WARMUP_SOURCES = ("pictures", "uint8", "float", "dense")
WARMUP_ROPE_MODES = ("none", "fused", "native")
_WARMUP_GRID = (1, 4, 8)
_WARMUP_MAX_RANK = 65536
_WARMUP_LOCK = threading.Lock()
_WARMED: set = set()


@dataclass(frozen=True)
class WarmupShape:
    """One kind of launch group of the restore path (see :func:`warmup`)."""

    heads: int
    head_dim: int
    dtype: torch.dtype = torch.bfloat16
    layout: str = "BTHD"
    source: str = "pictures"
    rope: str = "fused"
    ranks: tuple = (1, 1024)
    source_dtype: torch.dtype | None = None
    native_rope_dtype: torch.dtype | None = None

    def __post_init__(self):
        _int(self.heads, "heads", minimum=1)
        _int(self.head_dim, "head_dim", minimum=1)
        if self.dtype not in OUTPUT_DTYPES:
            raise ConfigurationError(f"warm-up cache dtype must be one of {OUTPUT_DTYPES}")
        if self.layout not in LAYOUTS:
            raise ConfigurationError(f"warm-up layout must be one of {LAYOUTS}")
        if self.source not in WARMUP_SOURCES:
            raise ConfigurationError(f"warm-up source must be one of {WARMUP_SOURCES}")
        if self.rope not in WARMUP_ROPE_MODES:
            raise ConfigurationError(f"warm-up rope must be one of {WARMUP_ROPE_MODES}")
        if self.rope != "none" and self.head_dim % 2:
            raise ConfigurationError("RoPE needs an even head_dim")
        ranks = tuple(self.ranks) if isinstance(self.ranks, Sequence) and not isinstance(self.ranks, str) else ()
        if len(ranks) != 2:
            raise ConfigurationError("ranks must be (minimum, maximum)")
        low = _int(ranks[0], "minimum rank", minimum=1)
        high = _int(ranks[1], "maximum rank", minimum=low)
        if high > _WARMUP_MAX_RANK:
            raise ConfigurationError(f"warm-up ranks above {_WARMUP_MAX_RANK} are not supported")
        object.__setattr__(self, "ranks", (low, high))
        if self.source in ("float", "dense"):
            if self.source_dtype is not None and self.source_dtype not in COEFFICIENT_DTYPES:
                raise ConfigurationError(f"source_dtype must be one of {COEFFICIENT_DTYPES}")
        elif self.source_dtype is not None:
            raise ConfigurationError("source_dtype applies to float and dense sources only")
        if self.native_rope_dtype is not None:
            if self.rope != "native":
                raise ConfigurationError("native_rope_dtype applies to rope='native' only")
            if self.native_rope_dtype not in OUTPUT_DTYPES:
                raise ConfigurationError(f"native_rope_dtype must be one of {OUTPUT_DTYPES}")

    def describe(self):
        return {"heads": self.heads, "head_dim": self.head_dim, "dtype": str(self.dtype), "layout": self.layout,
                "source": self.source, "rope": self.rope, "ranks": list(self.ranks),
                "source_dtype": None if self.source_dtype is None else str(self.source_dtype),
                "native_rope_dtype": None if self.native_rope_dtype is None else str(self.native_rope_dtype)}


# Register-resident rank steps of the compiled variants (their code objects load on first launch):
# the one-wave classes, the rank-halves classes and the chunked general kernel beyond them.
_VARIANT_STEPS = (2, 4, 8, 12, 16, 24, 32, 33)


def _warmup_ranks(ranks):
    """One rank per compiled variant class reachable within ``ranks``."""
    low, high = ranks
    chosen = []
    for steps in _VARIANT_STEPS:
        rank = min(high, 16 * steps)
        if rank >= low and rank not in chosen:
            chosen.append(rank)
        if 16 * steps >= high:
            break
    return chosen or [high]


def _warmup_jobs(shape, rank, device):
    from .quantize import video_layout

    tokens = math.prod(_WARMUP_GRID)
    targets = ("K", "V") if shape.rope != "none" else ("V",)
    sizes = {"BTHD": (1, tokens * len(targets), shape.heads, shape.head_dim),
             "THD": (tokens * len(targets), shape.heads, shape.head_dim),
             "BHTD": (1, shape.heads, tokens * len(targets), shape.head_dim)}[shape.layout]
    destination = torch.zeros(sizes, dtype=shape.dtype, device=device)
    channels = shape.heads * shape.head_dim
    basis = None if shape.source == "dense" else torch.zeros((rank, channels), dtype=torch.float16, device=device)
    table = None
    if shape.rope != "none":
        cos = torch.ones((tokens, shape.head_dim // 2), dtype=torch.float32, device=device)
        table = RopeTable.from_cos_sin(cos, torch.zeros_like(cos))
    jobs = []
    for position, target in enumerate(targets):
        view = NativeView(destination, shape.layout, token_offset=position * tokens)
        scale, offset = np.full(rank, 1 / 255, dtype=np.float32), np.zeros(rank, dtype=np.float32)
        if shape.source == "dense":
            source = DenseSource(torch.zeros((tokens, channels), dtype=shape.source_dtype or shape.dtype,
                                             device=device))
        elif shape.source == "float":
            source = CoefficientSource(torch.zeros((tokens, rank), dtype=shape.source_dtype or torch.float32,
                                                   device=device))
        elif shape.source == "uint8":
            source = CoefficientSource(torch.zeros((tokens, rank), dtype=torch.uint8, device=device), scale, offset)
        else:
            layout = video_layout(*_WARMUP_GRID, rank, "yuv444p")
            frames = layout["frames"]
            canvases = torch.zeros((layout["segments"] * frames, layout["planes"], layout["image_height"],
                                    layout["image_width"]), dtype=torch.uint8, device=device)
            indices = [[segment * frames + frame for frame in range(frames)] for segment in range(layout["segments"])]
            source = PictureSource.from_canvases(canvases, layout, indices, (0, 0), scale, offset)
        jobs.append(ReconstructionJob(source, view, _WARMUP_GRID, basis=basis,
                                      rank=None if shape.source == "dense" else rank,
                                      rope=RopePositions(table, 0) if target == "K" else None,
                                      label=f"warmup:{target}:{rank}"))
    return jobs


def _identity_rope(values, job):
    """Stands in for the engine's ``native_rope`` callable during :func:`warmup`."""
    return values


def warmup(device, shapes, *, backend="auto", precision="auto", config=None, stream=None):
    """Load every kernel variant :func:`reconstruct` launches for ``shapes`` before the first restore.

    The HIP kernels are compiled ahead of time, so warming up loads their code
    objects and runs one tiny synthetic call per reachable variant (rank class x
    precision) through the real launch path.  Serialized by a lock; repeat calls
    for a warmed (device, shape, backend, precision, config) do no work.
    Returns a report (``seconds``, ``calls``, ``launches``, per-shape entries).
    """
    started = time.perf_counter()
    if isinstance(shapes, (WarmupShape, Mapping)):
        shapes = [shapes]
    shapes = [shape if isinstance(shape, WarmupShape) else WarmupShape(**shape) for shape in shapes]
    if not shapes:
        raise ConfigurationError("warmup needs at least one WarmupShape")
    if backend not in BACKENDS:
        raise ConfigurationError(f"backend must be one of {BACKENDS}")
    device = torch.device(device)
    cuda = device.type == "cuda"
    resolved = _resolve_backend(backend, cuda)
    if cuda and device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    names = [precision] if isinstance(precision, str) else list(precision)
    if not names:
        raise ConfigurationError("warmup needs at least one precision")
    report = {"device": str(device), "backend": backend, "resolved_backend": resolved, "precisions": [],
              "repeat": False, "warmed": 0, "skipped": 0, "calls": 0, "launches": 0, "shapes": []}
    if resolved == "reference":
        report.update(seconds=time.perf_counter() - started, note="the reference backend compiles no kernels")
        return report
    precisions = []
    for name in names:
        if name != "auto" and name not in PRECISIONS:
            raise ConfigurationError(f"precision must be 'auto' or one of {PRECISIONS}")
        name = _resolve_precision(name, device)
        if name not in precisions:
            precisions.append(name)
    report["precisions"] = precisions
    merged = _merged_config(config)
    config_key = tuple(sorted((name, repr(value)) for name, value in merged.items()))
    with _WARMUP_LOCK, torch.cuda.device(device), (torch.cuda.stream(stream) if stream is not None else _null()):
        for shape in shapes:
            for name in precisions:
                key = (str(device), backend, name, shape, config_key)
                ranks = [None] if shape.source == "dense" else _warmup_ranks(shape.ranks)
                entry = {"shape": shape.describe(), "precision": name, "ranks": ranks, "calls": 0, "launches": 0,
                         "seconds": 0.0, "repeat": key in _WARMED}
                if entry["repeat"]:
                    report["skipped"] += 1
                    report["shapes"].append(entry)
                    continue
                shape_started = time.perf_counter()
                for rank in ranks:
                    jobs = _warmup_jobs(shape, rank or 1, device)
                    handle = reconstruct(jobs, backend=backend, precision=name, stream=stream, config=config,
                                         native_rope=_identity_rope if shape.rope == "native" else None,
                                         native_rope_dtype=shape.native_rope_dtype)
                    handle.release()
                    entry["calls"] += 1
                    entry["launches"] += handle.stats["launches"]
                entry["seconds"] = time.perf_counter() - shape_started
                _WARMED.add(key)
                report["warmed"] += 1
                report["calls"] += entry["calls"]
                report["launches"] += entry["launches"]
                report["shapes"].append(entry)
    report["repeat"] = report["warmed"] == 0
    report["seconds"] = time.perf_counter() - started
    return report


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
