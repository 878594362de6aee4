"""Job-list validation, the plain-torch reference backend and the elementwise error bound.

Public contract of reelcache/restore_kernels.py:957-1227 (``unpack_pictures``, ``dequantize``,
``reference_coefficients``, ``rope_cos_sin``, ``apply_rope_reference``, ``fp32_matmul_precision``,
``reconstruct_reference``, ``reference_values``, ``error_bound``), re-exported by
:mod:`reelcache_amd.restore_kernels`.  The bodies are this package's own:

* pictures are unpacked with one gather per picture, through per-layout index vectors of the
  ``reelcache.channel_tiles.v1`` slot order (plane fastest, then grid column, then grid row);
* separable RoPE rows are read with one index matrix ``[tokens, pairs]`` per table;
* the precision modes' product error is a table of (leading term, passes) pairs.

The arithmetic that the parity tests pin is unchanged: dequantize rounds twice (multiply, then
add), the rotation computes ``e*c - o*s`` and ``e*s + o*c`` in the compute dtype, and the reference
product is one matmul in FP64 (or IEEE FP32) followed by one cast.
"""

from __future__ import annotations

import functools
from collections.abc import Sequence

import numpy as np
import torch

from ._checks import need
from .errors import ConfigurationError, IntegrityError, UnsupportedError
from .restore_model import CoefficientSource, DenseSource, PictureSource, ReconstructionJob

# ---------------------------------------------------------------------------
# Job-list validation
# ---------------------------------------------------------------------------


def _storage_key(tensor):
    """(storage address, device) of a tensor; the data address for tensors without a storage."""
    try:
        address = tensor.untyped_storage().data_ptr()
    except (RuntimeError, NotImplementedError):
        address = tensor.data_ptr()
    return address, tensor.device


class _Facts:
    """What call validation needs of a job, computed once per job object (jobs are immutable):
    the devices of its tensors, its destination view's geometry, its token span and its
    matrix-product flops."""

    __slots__ = ("devices", "dst", "flops", "shift", "span", "view")

    def __init__(self, job):
        view, source = job.destination, job.source
        tensor = self.dst = view.tensor
        devices = {tensor.device, source.device if isinstance(source, PictureSource) else source.values.device}
        if job.basis is not None:
            devices.add(job.basis.device)
        self.devices = devices
        self.shift = tensor.storage_offset() * tensor.element_size()
        self.view = (tensor.storage_offset(), tuple(tensor.shape), tensor.stride(), view.layout, view.batch_index,
                     tensor.device)
        self.span = (view.token_offset, view.token_offset + job.tokens)
        self.flops = 2 * job.tokens * job.rank * view.channels if job.rank else 0


def _facts(job):
    facts = job.__dict__.get("_facts")
    if facts is None:
        facts = _Facts(job)
        object.__setattr__(job, "_facts", facts)
    return facts


def _check_disjoint(jobs, facts=None):
    """Reject jobs whose slots in the same destination view overlap (concurrent writes would race)."""
    facts = [_facts(job) for job in jobs] if facts is None else facts
    views: dict = {}
    for index, fact in enumerate(facts):
        # Views of one storage share its base address (data address less the view's offset).
        views.setdefault((fact.dst.data_ptr() - fact.shift, fact.view), []).append(index)
    for members in views.values():
        if len(members) < 2:
            continue
        # Sweep the slots in start order, keeping the one that reaches furthest so far.
        ordered = sorted(members, key=lambda index: facts[index].span)
        reach, holder = facts[ordered[0]].span[1], ordered[0]
        for index in ordered[1:]:
            start, stop = facts[index].span
            if start < reach:
                first, second = sorted((holder, index))
                raise ConfigurationError(f"jobs {first} and {second} write overlapping destination tokens")
            if stop > reach:
                reach, holder = stop, index


def _validate(jobs):
    """``(jobs tuple, device or None)`` of a job list; raises on mixed devices or overlapping slots."""
    if isinstance(jobs, ReconstructionJob):
        jobs = (jobs,)
    need(isinstance(jobs, Sequence) and not isinstance(jobs, (str, bytes)),
         "jobs must be a sequence of ReconstructionJob")
    jobs = tuple(jobs)
    need(all(isinstance(job, ReconstructionJob) for job in jobs), "jobs must be ReconstructionJob instances")
    facts = [_facts(job) for job in jobs]
    devices = set().union(*(fact.devices for fact in facts)) if facts else set()
    need(len(devices) <= 1, "all job tensors (except RoPE tables) must share one device")
    _check_disjoint(jobs, facts)
    return jobs, next(iter(devices), None)


# ---------------------------------------------------------------------------
# Coefficients
# ---------------------------------------------------------------------------


@functools.lru_cache(maxsize=256)
def _slot_coordinates(planes, columns, count):
    """(plane, grid column, grid row) of the first ``count`` slots of a segment in
    channel_tiles.v1 order: the plane varies fastest, then the grid column, then the grid row."""
    slot = np.arange(count)
    return slot % planes, (slot // planes) % columns, slot // (planes * columns)


def unpack_pictures(source):
    """Quantized coefficient pixels ``[N, rank]`` of a :class:`PictureSource` (channel_tiles.v1)."""
    layout = source.layout
    frames, height, width, rank = (layout[name] for name in ("frames", "height", "width", "rank"))
    columns, _ = layout["grid"]
    slots = layout["channels_per_segment"]
    device = source.device
    out = torch.empty((frames, height, width, rank), dtype=torch.uint8, device=device)
    y = torch.arange(height, device=device)[:, None, None]
    x = torch.arange(width, device=device)[None, :, None]
    for segment, pictures in enumerate(source.pictures):
        first = segment * slots
        count = min(slots, rank - first)
        plane, column, row = (torch.from_numpy(v).to(device) for v in _slot_coordinates(layout["planes"], columns,
                                                                                             count))
        # Pixel of slot k for token (y, x): plane p_k, picture row r_k * height + y, column c_k * width + x.
        rows_index = row[None, None, :] * height + y
        columns_index = column[None, None, :] * width + x
        for frame, picture in enumerate(pictures):
            out[frame, :, :, first:first + count] = picture[plane[None, None, :], rows_index, columns_index]
    return out.reshape(-1, rank)


def dequantize(pixels, scale, offset):
    """``float(pixel) * scale + offset`` rounded twice: the product, then the sum (no fused
    multiply-add), as the eager reference computes it."""
    scale_t, offset_t = (torch.tensor(np.asarray(v, dtype=np.float32), device=pixels.device) for v in (scale, offset))
    product = pixels.to(torch.float32) * scale_t
    return product + offset_t


def reference_coefficients(job):
    """The FP32 coefficient matrix ``[N, rank]`` a job reconstructs from."""
    source = job.source
    if isinstance(source, DenseSource):
        raise ConfigurationError("dense sources have no coefficients")
    if isinstance(source, PictureSource):
        return dequantize(unpack_pictures(source), source.scale, source.offset)
    assert isinstance(source, CoefficientSource)
    columns = source.values[:, :job.rank]
    if not source.quantized:
        return columns.float()
    return dequantize(columns, source.scale[:job.rank], source.offset[:job.rank])


# ---------------------------------------------------------------------------
# RoPE
# ---------------------------------------------------------------------------


def _section_rows(positions, grid, device):
    """Row index ``[tokens, pairs]`` of a separable table: pair j of token (f, y, x) reads the row of
    the axis its section belongs to, offset by the chunk's first row on that axis."""
    table = positions.table
    frames, height, width = grid
    token = torch.arange(frames * height * width, device=device)
    coordinate = torch.stack((token // (height * width), (token // width) % height, token % width))  # [3, N]
    axis = torch.repeat_interleave(torch.arange(3, device=device), torch.tensor(table.sections, device=device))
    first = torch.tensor(positions.rows, device=device)
    return (coordinate + first[:, None])[axis].T  # [N, pairs]


def rope_cos_sin(positions, grid, *, dtype=torch.float64, device=None):
    """Per-token ``(cos, sin)`` ``[N, head_dim // 2]`` for a job's positions."""
    table = positions.table
    device = table.cos.device if device is None else torch.device(device)
    cos, sin = (t.to(device=device, dtype=dtype) for t in (table.cos, table.sin))
    tokens = grid[0] * grid[1] * grid[2]
    if table.sections is None:
        rows = slice(positions.rows, positions.rows + tokens)
        return cos[rows], sin[rows]
    rows = _section_rows(positions, grid, device)
    pair = torch.arange(table.pairs, device=device).expand_as(rows)
    return cos[rows, pair], sin[rows, pair]


def apply_rope_reference(values, positions, grid, *, dtype=torch.float64):
    """Rotate interleaved pairs of ``values[N, H, D]`` in ``dtype`` (Wan complex product)."""
    cos, sin = rope_cos_sin(positions, grid, dtype=dtype, device=values.device)
    cos, sin = cos[:, None, :], sin[:, None, :]
    pairs = values.to(dtype).unflatten(-1, (-1, 2))
    even, odd = pairs[..., 0], pairs[..., 1]
    rotated = torch.stack((even * cos - odd * sin, even * sin + odd * cos), dim=-1)
    return rotated.flatten(-2)


# ---------------------------------------------------------------------------
# Reference backend
# ---------------------------------------------------------------------------


def fp32_matmul_precision(device_type):
    """Precision this process lets FP32 torch matmuls on ``"cuda"`` or ``"cpu"`` use (read only):
    ``"ieee"`` or a reduced mode name.  Torch >= 2.9 keeps it per backend (``fp32_precision``);
    older Torch has one process-wide ``float32_matmul_precision``."""
    if device_type == "cuda":
        backend = torch.backends.cuda.matmul
    else:
        backend = getattr(getattr(torch.backends, "mkldnn", None), "matmul", None)
    setting = getattr(backend, "fp32_precision", None)
    if not isinstance(setting, str):
        setting = {"highest": "ieee"}.get(torch.get_float32_matmul_precision(), torch.get_float32_matmul_precision())
    return "ieee" if setting == "none" else setting


def _require_fp32_matmul(device_type, accepted, what):
    actual = fp32_matmul_precision(device_type)
    if actual not in accepted:
        raise UnsupportedError(f"{what} needs {device_type} FP32 matmuls at {' / '.join(accepted)} precision, but "
                               f"this process set {actual!r}; the setting is process-wide and this module never "
                               "changes it")


def _pre_rope(job, compute):
    """Values ``[N, C]`` before RoPE: the dense matrix as given, or the rank-view product in
    ``compute``."""
    if isinstance(job.source, DenseSource):
        return job.source.values
    coefficients = reference_coefficients(job).to(compute)
    return coefficients @ job.basis[:job.rank].to(device=coefficients.device, dtype=compute)


def _native_rotation(native_rope, values, job, dtype):
    result = native_rope(values.to(dtype), job)
    if not isinstance(result, torch.Tensor) or result.numel() != values.numel():
        raise IntegrityError("native RoPE callable returned a tensor of the wrong size")
    return result.reshape(values.shape)


def _reference_job(job, compute, native_rope, native_rope_dtype):
    view = job.destination
    shape = (job.tokens, view.heads, view.head_dim)
    slot = view.slot(job.tokens)
    values = _pre_rope(job, compute).reshape(shape)
    if job.rope is None:
        slot.copy_(values)
    elif native_rope is not None:
        slot.copy_(_native_rotation(native_rope, values, job, native_rope_dtype or slot.dtype))
    else:
        slot.copy_(apply_rope_reference(values, job.rope, job.grid, dtype=compute))


def _check_compute_dtype(compute_dtype, device):
    need(compute_dtype in (torch.float32, torch.float64), "reference compute dtype must be float32 or float64")
    if compute_dtype == torch.float32 and device is not None:
        _require_fp32_matmul(device.type, ("ieee",), "the FP32 reference (compute_dtype=torch.float32)")


def reconstruct_reference(jobs, *, compute_dtype=torch.float64, native_rope=None, native_rope_dtype=None):
    """Plain-torch reference: FP64 (default) or IEEE FP32 math, then one cast (runs on the jobs' device)."""
    jobs, device = _validate(jobs)
    _check_compute_dtype(compute_dtype, device)
    with torch.no_grad():
        for job in jobs:
            _reference_job(job, compute_dtype, native_rope, native_rope_dtype)


# ---------------------------------------------------------------------------
# Error bound
# ---------------------------------------------------------------------------

_UNIT_ROUNDOFF = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11, torch.float32: 2.0 ** -24}
# Half the smallest subnormal spacing of each output format: the absolute rounding floor.
_OUTPUT_FLOOR = {torch.bfloat16: 2.0 ** -134, torch.float16: 2.0 ** -25, torch.float32: 2.0 ** -150}

# (leading relative error of the operand rounding, FP32-accumulated products) per precision mode
# (reelcache/restore_kernels.py:1176-1187): fp16x2 splits each coefficient into hi + lo (two
# products, 2^-21 from the lo part's rounding); bf16 rounds operands to 8 bits (2^-7 + 2^-16).
_PRODUCT_ERROR = {
    "fp32": (0.0, 1),
    "reference32": (0.0, 1),
    "tf32": (2.0 ** -10, 1),
    "tf32x3": (2.0 ** -20, 3),
    "fp16": (2.0 ** -11, 1),
    "fp16x2": (2.0 ** -21, 2),
    "bf16": (2.0 ** -7 + 2.0 ** -16, 1),
}


def _gemm_gamma(precision, rank):
    """Relative product error per unit of ``sum_k |a_k| |q_k|``: the mode's operand rounding plus
    ``passes`` FP32 accumulations of ``rank + 1`` roundings each."""
    lead, passes = _PRODUCT_ERROR[precision]
    return lead + passes * (rank + 1) * 2.0 ** -24


def _pair_sums(matrix, tokens):
    """``|a_e| + |a_o|`` of every interleaved pair, repeated on both members."""
    pairs = matrix.reshape(tokens, -1, 2)
    return pairs.sum(dim=-1).repeat_interleave(2, dim=-1)


def reference_values(job):
    """FP64 values ``y*[N, C]`` a job writes before the final cast, and ``sum_k |p_k| |q_k|``."""
    if isinstance(job.source, DenseSource):
        values = job.source.values.double()
        magnitude = torch.zeros_like(values)
    else:
        coefficients = reference_coefficients(job).double()
        basis = job.basis[:job.rank].to(device=coefficients.device, dtype=torch.float64)
        values, magnitude = coefficients @ basis, coefficients.abs() @ basis.abs()
    if job.rope is None:
        return values, magnitude
    view = job.destination
    rotated = apply_rope_reference(values.reshape(job.tokens, view.heads, view.head_dim), job.rope, job.grid)
    # A rotated element mixes both members of its pair, so it inherits both magnitudes.
    return rotated.reshape(job.tokens, -1), _pair_sums(magnitude, job.tokens)


def error_bound(job, precision, out_dtype=None):
    """Elementwise bound on ``|written - y*|`` for a precision mode (first-order analysis).

    ``|y_hat - y*| <= u_out |y*| + (1 + u_out) E + floor`` with
    ``E = gamma(precision, rank) * S + 2**-21 (|y_e| + |y_o|)`` (the last term only
    with RoPE: FP32 cos/sin tables and the rotation's own roundings),
    ``S = sum_k |p_k| |q_k|`` summed over each rotated pair
    (reelcache/restore_kernels.py:1208-1227).  Returns ``(y*, bound)`` in FP64.
    """
    values, magnitude = reference_values(job)
    out_dtype = job.destination.tensor.dtype if out_dtype is None else out_dtype
    unit = _UNIT_ROUNDOFF[out_dtype]
    product = _gemm_gamma(precision, job.rank or 0) * magnitude
    if job.rope is not None:
        product = product + 2.0 ** -21 * _pair_sums(values.abs(), job.tokens)
    return values, unit * values.abs() + (1 + unit) * product + _OUTPUT_FLOOR[out_dtype]
