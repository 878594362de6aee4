"""Oracle (numpy) for the restore half: dequantize -> P @ Q[:rank] -> RoPE -> one cast.

Test infrastructure only (see ``oracle/__init__.py``).  Follows
reelcache/restore_kernels.py:
  dequantize                 :1034-1038  float32(q) * scale, then + offset (two roundings)
  unpack_pictures            :1013-1031  channel_tiles.v1 cells (reelcache/_hevc.py:543-548)
  wan_sections               :308-311
  rope_cos_sin               :1053-1075  separable (t, h, w) rows or dense rows
  apply_rope_reference       :1078-1087  interleaved-pair rotation
  reconstruct_reference      :1090-1168  FP64 (or FP32) product, rotation, one cast
  gemm_gamma / error_bound   :1171-1227
Wan tables follow the native rope_params restated in tests/test_restore_kernels.py:68-80.
"""

from __future__ import annotations

import math

import numpy as np

LAYOUTS = ("BTHD", "THD", "BHTD")


# ---------------------------------------------------------------------------
# Number formats
# ---------------------------------------------------------------------------


def f32_to_bf16_bits(x):
    """Round float32 values to bfloat16 (round to nearest even); returns uint16 bit patterns."""
    bits = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    rounded = (bits + 0x7FFF + ((bits >> 16) & 1)) >> 16
    out = rounded.astype(np.uint16)
    out[nan] = 0x7FC0
    return out


def bf16_bits_to_f32(bits):
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)


def cast(values, dtype):
    """The destination cast of a float64 value as torch performs it: float64 -> float32
    (one rounding), then -> bfloat16 / float16 (a second rounding).  Returns float64."""
    single = np.asarray(values, dtype=np.float64).astype(np.float32)
    if dtype == "float32":
        return single.astype(np.float64)
    if dtype == "float16":
        return single.astype(np.float16).astype(np.float64)
    if dtype == "bfloat16":
        return bf16_bits_to_f32(f32_to_bf16_bits(single)).astype(np.float64)
    raise ValueError(dtype)


UNIT_ROUNDOFF = {"bfloat16": 2.0 ** -8, "float16": 2.0 ** -11, "float32": 2.0 ** -24}
OUTPUT_FLOOR = {"bfloat16": 2.0 ** -134, "float16": 2.0 ** -25, "float32": 2.0 ** -150}


# ---------------------------------------------------------------------------
# Coefficients
# ---------------------------------------------------------------------------


def dequantize(codes, scale, offset):
    """``float32(q) * scale + offset`` with two float32 roundings (no fused multiply-add)."""
    product = np.asarray(codes).astype(np.float32) * np.asarray(scale, dtype=np.float32)
    return (product + np.asarray(offset, dtype=np.float32)).astype(np.float32)


def cells(layout, count):
    """(slot index, plane, y, x) of the first ``count`` cells of a segment (reelcache/_hevc.py:543-548)."""
    columns = layout["grid"][0]
    for index in range(count):
        plane = index % layout["planes"]
        row, column = divmod(index // layout["planes"], columns)
        yield index, plane, row * layout["height"], column * layout["width"]


def unpack_pictures(pictures, layout):
    """uint8 ``[N, rank]`` from ``pictures[segment][frame]`` views ``[planes, rows, cols]`` (numpy)."""
    frames, height, width, rank = layout["frames"], layout["height"], layout["width"], layout["rank"]
    slots = layout["channels_per_segment"]
    out = np.zeros((frames, height, width, rank), dtype=np.uint8)
    for segment, row in enumerate(pictures):
        first = segment * slots
        count = min(slots, rank - first)
        for frame, picture in enumerate(row):
            for index, plane, y, x in cells(layout, count):
                out[frame, :, :, first + index] = picture[plane, y:y + height, x:x + width]
    return out.reshape(-1, rank)


def pack_pictures(codes, layout, origin=(0, 0), pad=(3, 5), fill=7):
    """Canvases ``[segments * frames, planes, H, W]`` holding ``codes`` [N, rank] in the
    channel_tiles.v1 layout at ``origin`` (the inverse of :func:`unpack_pictures`)."""
    frames, height, width, rank = layout["frames"], layout["height"], layout["width"], layout["rank"]
    columns, rows = layout["grid"]
    slots, segments = layout["channels_per_segment"], layout["segments"]
    values = np.asarray(codes).reshape(frames, height, width, rank)
    y0, x0 = origin
    shape = (segments * frames, layout["planes"], rows * height + y0 + pad[0], columns * width + x0 + pad[1])
    canvas = np.full(shape, fill, dtype=np.uint8)
    indices = []
    for segment in range(segments):
        first = segment * slots
        count = min(slots, rank - first)
        for frame in range(frames):
            for index, plane, y, x in cells(layout, count):
                canvas[segment * frames + frame, plane, y0 + y:y0 + y + height, x0 + x:x0 + x + width] = \
                    values[frame, :, :, first + index]
        indices.append([segment * frames + frame for frame in range(frames)])
    return canvas, indices


# ---------------------------------------------------------------------------
# RoPE
# ---------------------------------------------------------------------------


def wan_sections(pairs):
    """(t, h, w) pair counts: t = pairs - 2 * (pairs // 3), h = w = pairs // 3."""
    third = pairs // 3
    return (pairs - 2 * third, third, third)


def wan_rope_params(rows, dim, theta=10000.0):
    """Complex128 ``[rows, dim // 2]``: exp(i * n / theta ** (2j / dim)) (Wan rope_params)."""
    exponents = np.arange(0, dim, 2, dtype=np.float64) / dim
    angles = np.outer(np.arange(rows, dtype=np.float64), 1.0 / np.power(theta, exponents))
    return np.cos(angles) + 1j * np.sin(angles)


def wan_freqs(head_dim, rows, theta=10000.0):
    """Wan 3-D table: t/h/w parts of dims d - 4(d//6), 2(d//6), 2(d//6) concatenated."""
    sixth = head_dim // 6
    return np.concatenate([wan_rope_params(rows, head_dim - 4 * sixth, theta),
                           wan_rope_params(rows, 2 * sixth, theta),
                           wan_rope_params(rows, 2 * sixth, theta)], axis=1)


def token_coordinates(grid):
    frames, height, width = grid
    index = np.arange(frames * height * width)
    plane = height * width
    return index // plane, (index % plane) // width, index % width


def rope_cos_sin(cos, sin, sections, rows, grid):
    """Per-token ``(cos, sin)`` ``[N, pairs]`` from a table: separable (``sections`` (t, h, w),
    ``rows`` (t_row, h_row, w_row)) or dense (``sections=None``, ``rows`` = first row)."""
    cos = np.asarray(cos, dtype=np.float64)
    sin = np.asarray(sin, dtype=np.float64)
    tokens = int(np.prod(grid))
    if sections is None:
        return cos[rows:rows + tokens], sin[rows:rows + tokens]
    axes = token_coordinates(grid)
    out_cos = np.empty((tokens, cos.shape[1]))
    out_sin = np.empty_like(out_cos)
    column = 0
    for axis, pairs in enumerate(sections):
        index = rows[axis] + axes[axis]
        out_cos[:, column:column + pairs] = cos[index, column:column + pairs]
        out_sin[:, column:column + pairs] = sin[index, column:column + pairs]
        column += pairs
    return out_cos, out_sin


def apply_rope(values, cos, sin):
    """Rotate interleaved pairs of ``values[N, H, D]``: (e, o) -> (e c - o s, e s + o c)."""
    x = np.asarray(values, dtype=np.float64)
    even, odd = x[..., 0::2], x[..., 1::2]
    c, s = cos[:, None, :], sin[:, None, :]
    out = np.empty_like(x)
    out[..., 0::2] = even * c - odd * s
    out[..., 1::2] = even * s + odd * c
    return out


# ---------------------------------------------------------------------------
# Reconstruction
# ---------------------------------------------------------------------------


def reconstruct(coefficients, basis, heads, rope=None, *, compute=np.float64):
    """Pre-cast values ``[N, C]``: ``coefficients[N, r] @ basis[r, C]`` in ``compute``, then the
    rotation (``rope=(cos, sin)`` per token) in ``compute``."""
    p = np.asarray(coefficients, dtype=compute)
    q = np.asarray(basis, dtype=compute)
    values = p @ q
    if rope is not None:
        tokens, channels = values.shape
        values = apply_rope(values.reshape(tokens, heads, channels // heads), *rope).reshape(tokens, channels)
        values = values.astype(compute)
    return values


def gemm_gamma(precision, rank):
    """Relative product error per unit of sum_k |p_k||q_k| (reelcache/restore_kernels.py:1176-1187)."""
    accumulate = (rank + 1) * 2.0 ** -24
    return {"fp32": accumulate, "tf32": 2.0 ** -10 + accumulate, "tf32x3": 2.0 ** -20 + 3 * accumulate,
            "fp16": 2.0 ** -11 + accumulate, "fp16x2": 2.0 ** -21 + 2 * accumulate,
            "bf16": 2.0 ** -7 + 2.0 ** -16 + accumulate}[precision]


def error_bound(coefficients, basis, heads, rope, precision, out_dtype):
    """``(y*, bound)``: FP64 exact values and the elementwise bound
    ``u_out |y*| + (1 + u_out) E + floor``, ``E = gamma S (+ 2**-21 (|y_e| + |y_o|) with RoPE)``,
    ``S = sum_k |p_k| |q_k|`` summed over each rotated pair (reelcache/restore_kernels.py:1190-1227)."""
    p = np.asarray(coefficients, dtype=np.float64)
    q = np.asarray(basis, dtype=np.float64)
    values = p @ q
    magnitude = np.abs(p) @ np.abs(q)
    tokens, channels = values.shape
    rank = p.shape[1]
    if rope is not None:
        values = apply_rope(values.reshape(tokens, heads, channels // heads), *rope).reshape(tokens, channels)
        pairs = magnitude.reshape(tokens, -1, 2)
        magnitude = np.repeat(pairs[..., 0] + pairs[..., 1], 2, axis=-1)
    error = gemm_gamma(precision, rank) * magnitude
    if rope is not None:
        pairs = np.abs(values).reshape(tokens, -1, 2)
        error = error + 2.0 ** -21 * np.repeat(pairs[..., 0] + pairs[..., 1], 2, axis=-1)
    unit = UNIT_ROUNDOFF[out_dtype]
    return values, unit * np.abs(values) + (1 + unit) * error + OUTPUT_FLOOR[out_dtype]


def coefficient_bound(scale, offset):
    """Upper bound of |q * scale + offset| over 8-bit q (reelcache/restore_kernels.py:1782-1785)."""
    scale = np.asarray(scale, dtype=np.float32)
    offset = np.asarray(offset, dtype=np.float32)
    return float(max(np.abs(offset).max(), np.abs(np.float32(255) * scale + offset).max())) * 1.0001


def prescale_exponent(bound):
    """14 - ceil(log2(bound)), clamped to [-100, 100], 0 for a zero bound
    (reelcache/restore_kernels.py:1386-1398), on the float32 bound."""
    bound = float(np.float32(bound))
    if not bound > 0:
        return 0
    return int(max(-100, min(100, 14 - math.ceil(math.log2(bound)))))


def relative_frobenius(actual, expected):
    expected = np.asarray(expected, dtype=np.float64)
    return float(np.linalg.norm(np.asarray(actual, dtype=np.float64) - expected) / np.linalg.norm(expected))
