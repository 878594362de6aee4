"""Oracle (numpy) for 8-bit coefficient quantization and the channel-tile layout.

Test infrastructure only (see ``oracle/__init__.py``).  Follows reelcache/_hevc.py
(_covering_affine :400-422, normalization_layout :425-447, quantize_coefficients
:450-472, _expanded_affine :475-483, dequantize_coefficients :505-515, video_layout
:517-540, _cells/_mosaic :543-612) and reelcache/node_packets.py (affine_from_extrema
:140-152, quantize_device :155-173, mosaic_device :176-187).
"""

from __future__ import annotations

import math

import numpy as np

MAX_DIMENSION = 8192


def covering_affine(lo, hi):
    """Per column: offset = float32(lo); scale = float32(span / 255) raised by one float32
    ulp while float64(scale) * 255 < span, and once more while float64(255 * scale + offset)
    (evaluated in float32) < hi.  Returns float32 [2, n] (scale; offset)."""
    lo = np.atleast_1d(np.asarray(lo, dtype=np.float64))
    hi = np.atleast_1d(np.asarray(hi, dtype=np.float64))
    scale = np.empty(lo.shape, dtype=np.float32)
    offset = lo.astype(np.float32)
    for i in range(lo.size):
        span = hi[i] - lo[i]
        s = np.float32(span / 255.0)
        if float(s) * 255.0 < span:
            s = np.nextafter(s, np.float32(np.inf))
        top = np.float32(np.float32(255) * s) + offset[i]
        if float(top) < hi[i]:
            s = np.nextafter(s, np.float32(np.inf))
            top = np.float32(np.float32(255) * s) + offset[i]
        if not (np.isfinite(s) and np.isfinite(top)) or float(top) < hi[i]:
            raise ValueError("no finite covering FP32 affine")
        scale[i] = s
    return np.stack((scale, offset)).astype("<f4")


def normalization_layout(rank, normalization, protected_fraction=1.0):
    if normalization == "per_channel":
        count, records = rank, rank
    elif normalization == "global":
        count, records = 0, 1
    elif normalization == "leading_columns":
        count = int(math.ceil(rank * protected_fraction))
        records = count + 1
    else:
        raise ValueError(normalization)
    return {"mode": normalization, "protected_count": count, "affine_shape": [2, records],
            "affine_order": ["scale", "offset"], "protected_columns": "leading"}


def expanded_affine(affine, layout, rank):
    if layout["mode"] == "per_channel":
        return np.asarray(affine[0], dtype=np.float32), np.asarray(affine[1], dtype=np.float32)
    count = layout["protected_count"]
    scale = np.full(rank, affine[0][0], dtype=np.float32)
    offset = np.full(rank, affine[1][0], dtype=np.float32)
    for column in range(count):
        scale[column] = affine[0][column + 1]
        offset[column] = affine[1][column + 1]
    return scale, offset


def affine_from_extrema(lo, hi, layout):
    lo = np.asarray(lo, dtype=np.float32)
    hi = np.asarray(hi, dtype=np.float32)
    if layout["mode"] == "per_channel":
        return covering_affine(lo, hi)
    count = layout["protected_count"]
    affine = np.zeros(layout["affine_shape"], dtype="<f4")
    if count < lo.shape[0]:
        affine[:, 0] = covering_affine(lo[count:].min(), hi[count:].max())[:, 0]
    if count:
        affine[:, 1:] = covering_affine(lo[:count], hi[:count])
    return affine


def quantize_with_affine(values, scale, offset):
    """Codes: rint((float64(v) - float64(offset)) / float64(scale)) clipped to [0, 255];
    0 where the scale is 0 (round half to even)."""
    v = np.asarray(values, dtype=np.float32).astype(np.float64)
    s = np.asarray(scale, dtype=np.float32).astype(np.float64)
    o = np.asarray(offset, dtype=np.float32).astype(np.float64)
    ratios = np.zeros(v.shape)
    positive = np.broadcast_to(s > 0, v.shape)
    quotient = (v - o) / np.where(s > 0, s, 1.0)
    ratios[positive] = quotient[positive]
    return np.clip(np.rint(ratios), 0, 255).astype(np.uint8)


def quantize(values, normalization="per_channel", protected_fraction=1.0):
    """(codes, affine, layout) of a float32 [N, r] matrix."""
    values = np.asarray(values, dtype=np.float32)
    layout = normalization_layout(values.shape[1], normalization, protected_fraction)
    affine = affine_from_extrema(values.min(0), values.max(0), layout)
    scale, offset = expanded_affine(affine, layout, values.shape[1])
    return quantize_with_affine(values, scale, offset), affine, layout


def dequantize(codes, affine, layout):
    scale, offset = expanded_affine(affine, layout, np.asarray(codes).shape[1])
    return (np.asarray(codes).astype(np.float32) * scale + offset).astype(np.float32)


def video_layout(frames, height, width, rank, pix_fmt="yuv444p"):
    planes = 3 if pix_fmt == "yuv444p" else 1
    columns = min(MAX_DIMENSION // width, max(1, math.ceil(math.sqrt(rank / planes))))
    rows = min(MAX_DIMENSION // height, max(1, math.ceil(rank / (planes * columns))))
    image_width, image_height = max(16, columns * width), max(16, rows * height)
    if pix_fmt == "yuv420p":
        image_width += image_width % 2
        image_height += image_height % 2
    slots = columns * rows * planes
    return {"schema": "reelcache.channel_tiles.v1", "frames": frames, "height": height, "width": width,
            "rank": rank, "pix_fmt": pix_fmt, "grid": [columns, rows], "planes": planes,
            "image_height": image_height, "image_width": image_width, "channels_per_segment": slots,
            "segments": math.ceil(rank / slots),
            "frame_padding": [image_height - rows * height, image_width - columns * width]}
