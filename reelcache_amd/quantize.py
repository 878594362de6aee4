"""8-bit coefficient quantization and the channel-tile picture layout (host side).

The device half is :func:`reelcache_amd.gpu_fitting.quantize_device` (HIP
extrema and quantize kernels); this module holds the host arithmetic that the
reference runs in numpy and that the device path must match bit for bit:

* :func:`covering_affine` -- FP32 ``(scale, offset)`` per column whose 255 steps
  provably cover ``[lo, hi]`` (reelcache/_hevc.py:400-422);
* :func:`normalization_layout` / :func:`expanded_affine` / :func:`affine_from_extrema`
  -- ``per_channel``, ``global`` and ``leading_columns`` records
  (reelcache/_hevc.py:425-483, reelcache/node_packets.py:140-152);
* :func:`quantize_coefficients` / :func:`dequantize_coefficients` -- the CPU codec
  path (reelcache/_hevc.py:450-515): codes ``clip(rint((v - offset) / scale), 0, 255)``
  in float64, 0 where the scale is 0;
* :func:`video_layout` -- ``reelcache.channel_tiles.v1`` geometry (reelcache/_hevc.py:517-540).
"""

from __future__ import annotations

import math

import numpy as np

from .errors import ConfigurationError, IntegrityError, UnsupportedError

MAX_DIMENSION = 8192
PIXEL_FORMATS = ("yuv444p", "yuv420p")
NORMALIZATIONS = ("per_channel", "global", "leading_columns")


def covering_affine(lo, hi):
    """``float32[2, n]`` (scale, offset) with ``offset = f32(lo)`` and the smallest FP32 scale,
    up to two ``nextafter`` steps above ``f32((hi - lo) / 255)``, such that both
    ``f32(scale) * 255 >= hi - lo`` and ``f32(255 * scale + offset) >= hi`` hold in float64."""
    lo = np.asarray(lo, dtype=np.float64)
    hi = np.asarray(hi, dtype=np.float64)
    span = hi - lo
    up = np.float32(np.inf)
    with np.errstate(over="ignore", invalid="ignore", under="ignore"):
        scale = (span / 255.0).astype(np.float32)
        scale = np.where(scale.astype(np.float64) * 255.0 < span, np.nextafter(scale, up), scale)
        offset = lo.astype(np.float32)
        top = np.float32(255) * scale + offset
        scale = np.where(top.astype(np.float64) < hi, np.nextafter(scale, up), scale)
        top = np.float32(255) * scale + offset
    if not np.isfinite(scale).all() or not np.isfinite(top).all() or np.any(top.astype(np.float64) < hi):
        raise ConfigurationError("coefficient range cannot use a finite covering FP32 affine")
    return np.stack((scale, offset)).astype("<f4", copy=False)


def normalization_layout(rank, normalization, protected_fraction=1.0):
    """Record layout of the affine payload for a normalization mode."""
    if type(rank) is not int or rank < 1:
        raise ConfigurationError("coefficient rank must be a positive integer")
    if normalization not in NORMALIZATIONS:
        raise UnsupportedError("normalization must be per_channel, global, or leading_columns")
    if (isinstance(protected_fraction, bool) or not isinstance(protected_fraction, (int, float))
            or not math.isfinite(protected_fraction) or not 0 <= protected_fraction <= 1):
        raise ConfigurationError("protected_fraction must be in [0, 1]")
    if normalization == "per_channel":
        count, records = rank, rank
    elif normalization == "global":
        count, records = 0, 1
    else:
        count = int(math.ceil(rank * protected_fraction))
        records = count + 1
    return {"mode": normalization, "protected_count": count, "affine_shape": [2, records],
            "affine_order": ["scale", "offset"], "protected_columns": "leading"}


def expanded_affine(affine, layout, rank):
    """Per-column FP32 ``(scale, offset)`` vectors of an affine payload."""
    if layout["mode"] == "per_channel":
        return affine[0], affine[1]
    count = layout["protected_count"]
    scale = np.full(rank, affine[0, 0], dtype=np.float32)
    offset = np.full(rank, affine[1, 0], dtype=np.float32)
    if count:
        scale[:count] = affine[0, 1:]
        offset[:count] = affine[1, 1:]
    return scale, offset


def affine_from_extrema(lo, hi, layout):
    """The covering affine payload from per-column FP32 extrema."""
    lo = np.asarray(lo, dtype=np.float32)
    hi = np.asarray(hi, dtype=np.float32)
    if layout["mode"] == "per_channel":
        return covering_affine(lo, hi)
    count = layout["protected_count"]
    affine = np.zeros(layout["affine_shape"], dtype="<f4")
    if count < lo.shape[0]:
        affine[:, 0] = covering_affine(lo[count:].min(), hi[count:].max())
    if count:
        affine[:, 1:] = covering_affine(lo[:count], hi[:count])
    return affine


def quantize_coefficients(values, normalization, protected_fraction=1.0):
    """Host quantizer: ``(uint8 codes [N, r], affine [2, records], layout)``."""
    values = np.asarray(values, dtype=np.float32)
    if values.ndim != 2 or min(values.shape) < 1 or not np.isfinite(values).all():
        raise ConfigurationError("coefficients must be a nonempty finite FP32 matrix")
    layout = normalization_layout(values.shape[1], normalization, protected_fraction)
    affine = affine_from_extrema(values.min(0), values.max(0), layout)
    scale, offset = expanded_affine(affine, layout, values.shape[1])
    ratios = np.zeros(values.shape, dtype=np.float64)
    np.divide(values.astype(np.float64) - offset.astype(np.float64), scale.astype(np.float64), out=ratios,
              where=scale > 0)
    return np.clip(np.rint(ratios), 0, 255).astype(np.uint8), affine, layout


def validate_affine(affine, layout, rank):
    affine = np.asarray(affine)
    if (affine.dtype != np.dtype("<f4") or list(affine.shape) != layout["affine_shape"]
            or not np.isfinite(affine).all() or np.any(affine[0] < 0)):
        raise IntegrityError("invalid coefficient affine payload")
    if layout["mode"] == "leading_columns" and layout["protected_count"] == rank and np.any(affine[:, 0] != 0):
        raise IntegrityError("unused global affine must be zero when all columns are protected")
    with np.errstate(over="ignore", invalid="ignore"):
        top = np.float32(255) * affine[0] + affine[1]
    if not np.isfinite(top).all():
        raise IntegrityError("coefficient affine endpoints are nonfinite")
    return affine


def dequantize_coefficients(pixels, affine, layout):
    """Host dequantization ``float32(q) * scale + offset`` (two roundings)."""
    pixels = np.asarray(pixels)
    if pixels.dtype != np.uint8 or pixels.ndim != 2 or min(pixels.shape) < 1:
        raise IntegrityError("decoded coefficient pixels must be a nonempty uint8 matrix")
    affine = validate_affine(affine, layout, pixels.shape[1])
    scale, offset = expanded_affine(affine, layout, pixels.shape[1])
    result = pixels.astype(np.float32) * scale + offset
    if not np.isfinite(result).all():
        raise IntegrityError("decoded coefficients are nonfinite")
    return np.ascontiguousarray(result)


def video_layout(frames, height, width, rank, pix_fmt):
    """``reelcache.channel_tiles.v1`` geometry: a grid of ``height x width`` cells per plane,
    ``columns x rows x planes`` rank columns per segment (picture), one picture per
    (segment, frame)."""
    if pix_fmt not in PIXEL_FORMATS:
        raise UnsupportedError(f"picture layouts support exactly {PIXEL_FORMATS}, not {pix_fmt!r}")
    if any(type(v) is not int or v < 1 for v in (frames, height, width, rank)):
        raise ConfigurationError("picture dimensions must be positive integers")
    if height > MAX_DIMENSION or width > MAX_DIMENSION:
        raise UnsupportedError(f"coefficient tiles cannot exceed {MAX_DIMENSION}x{MAX_DIMENSION}")
    planes = 3 if pix_fmt == "yuv444p" else 1
    columns = min(MAX_DIMENSION // width, max(1, math.ceil(math.sqrt(rank / planes))))
    rows = min(MAX_DIMENSION // height, max(1, math.ceil(rank / (planes * columns))))
    image_width, image_height = max(16, columns * width), max(16, rows * height)
    if pix_fmt == "yuv420p":
        image_width += image_width % 2
        image_height += image_height % 2
    if image_width > MAX_DIMENSION or image_height > MAX_DIMENSION:
        raise UnsupportedError("padded picture dimensions exceed provider support")
    slots = columns * rows * planes
    return {"schema": "reelcache.channel_tiles.v1", "frames": frames, "height": height, "width": width,
            "rank": rank, "pix_fmt": pix_fmt, "grid": [columns, rows], "planes": planes,
            "image_height": image_height, "image_width": image_width, "channels_per_segment": slots,
            "segments": math.ceil(rank / slots),
            "frame_padding": [image_height - rows * height, image_width - columns * width]}


__all__ = ["MAX_DIMENSION", "NORMALIZATIONS", "PIXEL_FORMATS", "affine_from_extrema", "covering_affine",
           "dequantize_coefficients", "expanded_affine", "normalization_layout", "quantize_coefficients",
           "validate_affine", "video_layout"]
