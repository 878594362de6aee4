"""Ahead-of-first-restore loading of the kernel variants a deployment will launch.

Contract of reelcache/restore_kernels.py:2449-2763 (``WarmupShape``, ``warmup``, the report
keys), re-exported by :mod:`reelcache_amd.restore_kernels`.  The HIP kernels are compiled ahead of
time, so warming up here means loading each reachable code object (first launch of a variant)
and running one tiny synthetic call per variant class through the real launch path: the compiled
variants are keyed by rank step (16 ranks) classes, so one call per class within ``ranks`` reaches
all of them.

A shape is validated by an ordered rule list (:func:`_shape_rules`); the work of one
:func:`warmup` call is a list of :class:`_Item` (shape x precision), each run once per process
and remembered in :data:`_WARMED`.
"""

from __future__ import annotations

import math
import threading
import time
from collections.abc import Mapping, Sequence
from dataclasses import dataclass

import numpy as np
import torch

from ._checks import need
from .errors import ConfigurationError
from .restore_model import (COEFFICIENT_DTYPES, LAYOUTS, OUTPUT_DTYPES, CoefficientSource, DenseSource, NativeView,
                            PictureSource, ReconstructionJob, RopePositions, RopeTable)

WARMUP_SOURCES = ("pictures", "uint8", "float", "dense")
WARMUP_ROPE_MODES = ("none", "fused", "native")
_WARMUP_GRID = (1, 4, 8)
_WARMUP_MAX_RANK = 65536
_WARMUP_LOCK = threading.Lock()
_WARMED: set = set()

# Register-resident rank steps of the compiled variant classes (their code objects load on first
# launch): the one-wave classes, the rank-halves classes and the chunked general kernel beyond them.
_VARIANT_STEPS = (2, 4, 8, 12, 16, 24, 32, 33)


def _positive(value, minimum=1):
    return type(value) is int and value >= minimum


def _pair(value):
    return tuple(value) if isinstance(value, Sequence) and not isinstance(value, str) else ()


def _shape_rules(shape):
    """``(holds, message)`` rules of a :class:`WarmupShape`, in order; later rules may assume the
    earlier ones hold (the generator is consumed until the first failure)."""
    yield _positive(shape.heads), "heads must be an integer >= 1"
    yield _positive(shape.head_dim), "head_dim must be an integer >= 1"
    yield shape.dtype in OUTPUT_DTYPES, f"warm-up cache dtype must be one of {OUTPUT_DTYPES}"
    yield shape.layout in LAYOUTS, f"warm-up layout must be one of {LAYOUTS}"
    yield shape.source in WARMUP_SOURCES, f"warm-up source must be one of {WARMUP_SOURCES}"
    yield shape.rope in WARMUP_ROPE_MODES, f"warm-up rope must be one of {WARMUP_ROPE_MODES}"
    yield shape.rope == "none" or shape.head_dim % 2 == 0, "RoPE needs an even head_dim"
    ranks = _pair(shape.ranks)
    yield len(ranks) == 2, "ranks must be (minimum, maximum)"
    yield _positive(ranks[0]), "minimum rank must be an integer >= 1"
    yield _positive(ranks[1], ranks[0]), f"maximum rank must be an integer >= {ranks[0]}"
    yield ranks[1] <= _WARMUP_MAX_RANK, f"warm-up ranks above {_WARMUP_MAX_RANK} are not supported"
    if shape.source_dtype is not None:
        yield shape.source in ("float", "dense"), "source_dtype applies to float and dense sources only"
        yield shape.source_dtype in COEFFICIENT_DTYPES, f"source_dtype must be one of {COEFFICIENT_DTYPES}"
    if shape.native_rope_dtype is not None:
        yield shape.rope == "native", "native_rope_dtype applies to rope='native' only"
        yield shape.native_rope_dtype in OUTPUT_DTYPES, f"native_rope_dtype must be one of {OUTPUT_DTYPES}"


@dataclass(frozen=True)
class WarmupShape:
    """One kind of launch group of the restore path (see :func:`warmup`).

    ``heads``/``head_dim``/``dtype``/``layout`` describe the native cache the jobs write;
    ``source`` the coefficient form (decoded ``"pictures"``, ``"uint8"`` or ``"float"``
    matrices, ``"dense"`` RAW rows); ``rope`` whether the calls rotate K in the kernel
    (``"fused"``), through the engine's callable (``"native"``, in ``native_rope_dtype``) or
    not at all (``"none"``); ``ranks=(min, max)`` the rank range of one call's factorized
    matrices; ``source_dtype`` the float/dense source dtype.
    """

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
        for holds, message in _shape_rules(self):
            need(holds, message)
        object.__setattr__(self, "ranks", _pair(self.ranks))

    def describe(self):
        """JSON-friendly description (dtypes as strings, ranks as a list)."""
        fields = {name: getattr(self, name) for name in self.__dataclass_fields__}
        fields["ranks"] = list(self.ranks)
        for name in ("dtype", "source_dtype", "native_rope_dtype"):
            fields[name] = None if fields[name] is None else str(fields[name])
        return fields


def _warmup_ranks(ranks):
    """One rank per compiled variant class reachable within ``ranks``: the class's largest rank,
    clipped to the range's maximum."""
    low, high = ranks
    picks = []
    for steps in _VARIANT_STEPS:
        rank = min(high, 16 * steps)
        if rank >= low and rank not in picks:
            picks.append(rank)
        if 16 * steps >= high:
            break
    return picks or [high]


def _synthetic_source(shape, rank, tokens, channels, device):
    """A zero-valued source of the shape's kind (affine 1/255, 0 for quantized ones)."""
    scale, offset = np.full(rank, 1 / 255, dtype=np.float32), np.zeros(rank, dtype=np.float32)
    if shape.source == "dense":
        return DenseSource(torch.zeros((tokens, channels), dtype=shape.source_dtype or shape.dtype, device=device))
    if shape.source == "float":
        return CoefficientSource(torch.zeros((tokens, rank), dtype=shape.source_dtype or torch.float32,
                                             device=device))
    if shape.source == "uint8":
        return CoefficientSource(torch.zeros((tokens, rank), dtype=torch.uint8, device=device), scale, offset)
    from .quantize import video_layout

    layout = video_layout(*_WARMUP_GRID, rank, "yuv444p")
    frames, segments = layout["frames"], layout["segments"]
    canvases = torch.zeros((segments * frames, layout["planes"], layout["image_height"], layout["image_width"]),
                           dtype=torch.uint8, device=device)
    picture = np.arange(segments * frames).reshape(segments, frames).tolist()
    return PictureSource.from_canvases(canvases, layout, picture, (0, 0), scale, offset)


def _warmup_jobs(shape, rank, device):
    """K (when the shape rotates) and V jobs of one synthetic call into one scratch cache."""
    tokens = math.prod(_WARMUP_GRID)
    targets = ("K", "V") if shape.rope != "none" else ("V",)
    span = tokens * len(targets)
    extent = {"BTHD": (1, span, shape.heads, shape.head_dim), "THD": (span, shape.heads, shape.head_dim),
              "BHTD": (1, shape.heads, span, shape.head_dim)}[shape.layout]
    cache = torch.zeros(extent, dtype=shape.dtype, device=device)
    channels = shape.heads * shape.head_dim
    factorized = shape.source != "dense"
    basis = torch.zeros((rank, channels), dtype=torch.float16, device=device) if factorized else None
    rope = None
    if shape.rope != "none":
        ones = torch.ones((tokens, shape.head_dim // 2), dtype=torch.float32, device=device)
        rope = RopePositions(RopeTable.from_cos_sin(ones, torch.zeros_like(ones)), 0)
    return [ReconstructionJob(_synthetic_source(shape, rank, tokens, channels, device),
                              NativeView(cache, shape.layout, token_offset=position * tokens), _WARMUP_GRID,
                              basis=basis, rank=rank if factorized else None,
                              rope=rope if target == "K" else None, label=f"warmup:{target}:{rank}")
            for position, target in enumerate(targets)]


def _identity_rope(values, job):
    """Stands in for the engine's ``native_rope`` callable during :func:`warmup`."""
    return values


@dataclass
class _Item:
    """One (shape, precision) of a warm-up call and its report entry."""

    shape: WarmupShape
    precision: str
    key: tuple

    def entry(self, repeat):
        ranks = [None] if self.shape.source == "dense" else _warmup_ranks(self.shape.ranks)
        return {"shape": self.shape.describe(), "precision": self.precision, "ranks": ranks, "calls": 0,
                "launches": 0, "seconds": 0.0, "repeat": repeat}


def _shapes(shapes):
    listed = [shapes] if isinstance(shapes, (WarmupShape, Mapping)) else list(shapes)
    need(listed, "warmup needs at least one WarmupShape")
    return [shape if isinstance(shape, WarmupShape) else WarmupShape(**shape) for shape in listed]


def warmup(device, shapes, *, backend="auto", precision="auto", config=None, stream=None):
    """Load every kernel variant :func:`reconstruct` launches for ``shapes`` before the first restore.

    Runs one tiny synthetic call per reachable variant class (rank class x precision) through
    the real launch path, on ``stream`` (default: the current one), into scratch caches.
    Serialized by a lock; repeat calls for a warmed (device, shape, backend, precision, config)
    do no work (``report["repeat"]``).  Returns a report: ``seconds``, ``calls``, ``launches``,
    ``warmed``/``skipped`` counts and per-shape entries.  On host tensors the reference backend
    compiles nothing and the report says so.
    """
    from . import restore_kernels as rk

    started = time.perf_counter()
    shapes = _shapes(shapes)
    need(backend in rk.BACKENDS, f"backend must be one of {rk.BACKENDS}")
    device = torch.device(device)
    cuda = device.type == "cuda"
    resolved = rk._resolve_backend(backend, cuda)
    if cuda and device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    requested = [precision] if isinstance(precision, str) else list(precision)
    need(requested, "warmup needs at least one precision")
    report = {"device": str(device), "backend": backend, "resolved_backend": resolved, "precisions": [],
              "repeat": False, "warmed": 0, "skipped": 0, "calls": 0, "launches": 0, "shapes": []}
    if resolved == "reference":
        report.update(seconds=time.perf_counter() - started, note="the reference backend compiles no kernels")
        return report
    for name in requested:
        need(name == "auto" or name in rk.PRECISIONS, f"precision must be 'auto' or one of {rk.PRECISIONS}")
    precisions = list(dict.fromkeys(rk._resolve_precision(name, device) for name in requested))
    report["precisions"] = precisions
    merged = rk._merged_config(config)
    config_key = tuple(sorted((name, repr(value)) for name, value in merged.items()))
    items = [_Item(shape, name, (str(device), backend, name, shape, config_key))
             for shape in shapes for name in precisions]
    streamed = torch.cuda.stream(stream) if stream is not None else rk._null()
    with _WARMUP_LOCK, torch.cuda.device(device), streamed:
        for item in items:
            entry = item.entry(item.key in _WARMED)
            report["shapes"].append(entry)
            if entry["repeat"]:
                continue
            clock = time.perf_counter()
            for rank in entry["ranks"]:
                handle = rk.reconstruct(_warmup_jobs(item.shape, rank or 1, device), backend=backend,
                                        precision=item.precision, stream=stream, config=config,
                                        native_rope=_identity_rope if item.shape.rope == "native" else None,
                                        native_rope_dtype=item.shape.native_rope_dtype)
                handle.release()
                entry["calls"] += 1
                entry["launches"] += handle.stats["launches"]
            entry["seconds"] = time.perf_counter() - clock
            _WARMED.add(item.key)
    done = [entry for entry in report["shapes"] if not entry["repeat"]]
    report.update(warmed=len(done), skipped=len(report["shapes"]) - len(done),
                  calls=sum(entry["calls"] for entry in done), launches=sum(entry["launches"] for entry in done))
    report["repeat"] = not done
    report["seconds"] = time.perf_counter() - started
    return report


__all__ = ["WARMUP_ROPE_MODES", "WARMUP_SOURCES", "WarmupShape", "warmup"]
