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
* ``staged`` -- the comparison path of the reference's ``_staged_group``: a HIP
  unpack of each GEMM group's coefficients into a dense work matrix, the GPU BLAS
  library's product with FP32 output (``torch.mm``), then a HIP RoPE / cast /
  store pass.  Precisions ``fp32``, ``fp16`` and ``bf16``; it follows the
  process-wide torch matmul settings and refuses what they forbid.
* ``reference`` -- plain torch, FP64 (default) or IEEE FP32, on the jobs' device.
* ``interpret`` (the Triton interpreter in the reference) has no counterpart and
  raises :class:`UnsupportedError`.

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

import torch

from . import _lib
from ._checks import need
from .errors import ConfigurationError, UnsupportedError
from .restore_handle import RestoreHandle, _sweep_deferred, park_failed, pending_deferred
from .restore_model import (COEFFICIENT_DTYPES, LAYOUTS, OUTPUT_DTYPES, CoefficientSource, DenseSource, NativeView,
                            PictureSource, ReconstructionJob, RopePositions, RopeTable, expand_affine, wan_sections)
from .restore_plan import (DEFAULT_MERGED, _DEFAULT_CONFIG, _RETIRED_SLABS, _STAGING, BASIS_DTYPES,  # noqa: F401
                           STAGED_PRECISIONS, STREAM_TOKENS, TILE_TOKENS, _balanced_bounds,
                           _capture_staging, check_staged_precision, staged_gemm,
                           _coefficient_bound, _fast_flags, _pinned_bytes, _prescale_exponent,
                           _tiles, job_desc, reserve_capture_staging, run_call)
from .restore_reference import (_OUTPUT_FLOOR, _UNIT_ROUNDOFF, _check_compute_dtype,  # noqa: F401
                                _check_disjoint, _facts, _gemm_gamma, _native_rotation, _require_fp32_matmul, _storage_key,
                                _validate, apply_rope_reference, dequantize, error_bound, fp32_matmul_precision,
                                reconstruct_reference, reference_coefficients, reference_values, rope_cos_sin,
                                unpack_pictures)

PRECISIONS = ("fp32", "tf32", "tf32x3", "fp16", "fp16x2", "bf16")
BACKENDS = ("auto", "reference", "fused", "two_pass", "staged", "interpret")

#: Why the compiled HIP kernels cannot be used in this process (None when they can).
HIP_IMPORT_ERROR = _lib.unavailable_reason()
HIP_AVAILABLE = HIP_IMPORT_ERROR is None
# The reference exposes the availability of its compiled kernels under these names
# (reelcache/restore_kernels.py:103-114); here they describe the HIP library.
TRITON_AVAILABLE = HIP_AVAILABLE
TRITON_IMPORT_ERROR = HIP_IMPORT_ERROR

_DEFAULT_PRECISION = "fp16x2"
_MATRIX_CORE_PRECISIONS = ("fp32", "fp16", "fp16x2", "bf16")
# Triton tile keys the reference accepts in ``config``; they have no meaning for the HIP
# kernels and are accepted (and ignored) so that caller configurations keep working.
_REFERENCE_TILE_KEYS = {"BLOCK_M", "BLOCK_K", "num_warps", "num_stages", "N_GROUP", "PIC_T", "UNPACK_BLOCK_K",
                        "maxnreg", "_n_group"}


# The reference's names for the staged GEMM and its settings check (restore_kernels.py:2153-2189).
_staged_gemm = staged_gemm
_check_staged_precision = check_staged_precision


def device_config(device):
    """Launch configuration for a device (tile geometry of the HIP kernels)."""
    return dict(_DEFAULT_CONFIG)


def recommended_precision(device):
    """Default precision: ``fp16x2`` (FP16 hi + lo products, near-FP32 accuracy), as in the reference."""
    return _DEFAULT_PRECISION


def _resolve_backend(backend, cuda):
    """``backend`` resolved for jobs on a GPU (``cuda=True``) or host tensors; never a silent fallback."""
    if backend == "reference" or (backend == "auto" and not cuda):
        return "reference"
    if backend == "interpret":
        raise UnsupportedError("the 'interpret' backend (the Triton interpreter) does not exist on ROCm; use "
                               "'fused', 'staged' or 'reference'")
    if not cuda:
        raise UnsupportedError(f"the {backend} backend needs GPU tensors; use 'reference'")
    reason = _lib.unavailable_reason()
    if reason is not None:
        if backend == "auto":
            raise UnsupportedError(f"backend='auto' cannot run the HIP reconstruction: {reason}. The FP64 reference "
                                   "is never substituted silently; pass backend='reference' to request it explicitly.")
        raise UnsupportedError(f"the {backend} backend is unavailable: {reason}")
    return "staged" if backend == "staged" else "fused"


def _resolve_precision(precision, device):
    if precision == "auto":
        precision = recommended_precision(device)
    if precision not in _MATRIX_CORE_PRECISIONS:
        raise UnsupportedError(f"precision {precision!r} has no matrix-core form on gfx950 (no TF32 MFMA); "
                               f"use one of {_MATRIX_CORE_PRECISIONS}")
    return precision


def _merged_config(config):
    if not config:
        return DEFAULT_MERGED
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
    return sum(_facts(job).flops for job in jobs)


class _FusedCall:
    """The HIP execution of one :func:`reconstruct` call: one planned launch sequence
    (:func:`reelcache_amd.restore_plan.run_call`) for the jobs the kernels rotate (or write
    unrotated) and, with ``native_rope``, one for the pre-RoPE K that the engine's callable
    rotates before the copy into its slot."""

    def __init__(self, device, stream, precision, config, keepalive, stage_events, stats, staged=False):
        self.device, self.stream, self.precision = device, stream, precision
        self.config, self.keepalive, self.stage_events, self.stats = config, keepalive, stage_events, stats
        self.staged = staged
        stats.update(grids=[], variants=[])

    def launch(self, jobs):
        launches, grids, variants = run_call([job_desc(job) for job in jobs], self.device, self.stream,
                                             self.precision, self.config, self.keepalive, self.stage_events,
                                             staged=self.staged)
        self.stats["launches"] += launches
        self.stats["grids"].extend(grids)
        self.stats["variants"].extend(variants)

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
    launch of the call, "fused"; the staged backend adds "unpack", "gemm" and "rope_store").

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
    elif resolved == "staged":
        # The staged GEMM follows process-wide torch settings: refuse before any work is enqueued.
        precision = label = recommended_precision(device) if precision == "auto" else precision
        check_staged_precision(precision)
    else:
        precision = label = _resolve_precision(precision, device)
    stream = _execution_stream(device, stream, wait_events)
    keepalive = list(jobs)  # the jobs reference every input tensor and table
    stats.update(backend=resolved, precision=label, picture_path="fused_gather" if resolved == "fused" else resolved)
    if resolved == "reference":
        with _on(stream):
            reconstruct_reference(jobs, compute_dtype=compute_dtype, native_rope=native_rope,
                                  native_rope_dtype=native_rope_dtype)
    else:
        call = _FusedCall(device, stream, precision, _merged_config(config), keepalive, stage_events, stats,
                          staged=resolved == "staged")
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
