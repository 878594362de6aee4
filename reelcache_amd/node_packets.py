"""Device quantization of fitted coefficients and the channel-tile canvas of a packet tile.

Mirrors ``reelcache/node_packets.py``: affine_from_extrema (:140-152), quantize_device
(:155-173, exactly ``_hevc.quantize_coefficients`` on the device) and mosaic_device (:176-187).

MI355X execution: the per-column extrema come from the extrema kernel (or from the projection
kernel, which computes them while writing the coefficients: :func:`quantize_with_extrema`),
the covering affine is computed on the host from those fp32 extrema exactly as the reference
does, and the codes come from the FP64 quantizer kernel (round half to even, clamp), which
reproduces numpy's ``clip(rint((v - offset) / scale), 0, 255)`` bit for bit.
"""

from __future__ import annotations

import numpy as np
import torch

from . import fit_kernels
from .errors import ConfigurationError
from .quantize import affine_from_extrema, expanded_affine, normalization_layout, video_layout

__all__ = ["affine_from_extrema", "mosaic_device", "quantize_device", "quantize_many", "quantize_with_extrema",
           "video_layout"]


def _check(coefficients) -> None:
    if (not isinstance(coefficients, torch.Tensor) or coefficients.dtype != torch.float32
            or coefficients.ndim != 2 or min(coefficients.shape) < 1):
        raise ConfigurationError("coefficients must be a nonempty FP32 matrix")


def _codes(coefficients: torch.Tensor, low: np.ndarray, high: np.ndarray, spec):
    if not (np.isfinite(low).all() and np.isfinite(high).all()):
        raise ConfigurationError("coefficients must be finite")
    rank = int(coefficients.shape[1])
    layout = normalization_layout(rank, spec.normalization, spec.protected_fraction)
    affine = affine_from_extrema(low, high, layout)
    scale, offset = expanded_affine(affine, layout, rank)
    device = coefficients.device
    scale64 = torch.from_numpy(np.ascontiguousarray(scale, dtype=np.float64)).to(device)
    offset64 = torch.from_numpy(np.ascontiguousarray(offset, dtype=np.float64)).to(device)
    values = coefficients if coefficients.stride(1) == 1 else coefficients.contiguous()
    pixels = fit_kernels.quantize(values, scale64, offset64)
    return pixels, affine.astype("<f4", copy=False), layout


@torch.no_grad()
def quantize_device(coefficients: torch.Tensor, spec) -> tuple[torch.Tensor, np.ndarray, dict]:
    """``_hevc.quantize_coefficients`` on the coefficients' device: (uint8 pixels, affine, layout)."""
    _check(coefficients)
    values = coefficients if coefficients.stride(1) == 1 else coefficients.contiguous()
    keys = fit_kernels.column_extrema(values).cpu().numpy()
    low, high = fit_kernels.split_keys(keys, int(values.shape[1]))
    return _codes(values, low, high, spec)


@torch.no_grad()
def quantize_with_extrema(coefficients: torch.Tensor, keys_row, spec) -> tuple[torch.Tensor, np.ndarray, dict]:
    """:func:`quantize_device` with the column extrema the projection kernel already produced
    (one row of ``fit_kernels.project(..., extrema=True)`` keys, on the host)."""
    _check(coefficients)
    low, high = fit_kernels.split_keys(np.asarray(keys_row), int(coefficients.shape[1]))
    return _codes(coefficients, low, high, spec)


@torch.no_grad()
def quantize_many(coefficients, keys, specs):
    """:func:`quantize_with_extrema` of many matrices (e.g. a chunk's) with one quantizer launch:
    ``keys`` are the host extrema rows of ``fit_kernels.project(..., extrema=True)``.
    Returns ``[(pixels, affine, layout)]``."""
    affines, layouts, outputs, values = [], [], [], []
    for p, row, spec in zip(coefficients, keys, specs):
        _check(p)
        rank = int(p.shape[1])
        low, high = fit_kernels.split_keys(np.asarray(row), rank)
        if not (np.isfinite(low).all() and np.isfinite(high).all()):
            raise ConfigurationError("coefficients must be finite")
        layout = normalization_layout(rank, spec.normalization, spec.protected_fraction)
        affine = affine_from_extrema(low, high, layout)
        scale, offset = expanded_affine(affine, layout, rank)
        affines.append(np.stack((np.asarray(scale, np.float64), np.asarray(offset, np.float64))))
        layouts.append((affine.astype("<f4", copy=False), layout))
        values.append(p if p.stride(1) == 1 else p.contiguous())
    codes = fit_kernels.quantize_batched(values, affines)
    for pixels, (affine, layout) in zip(codes, layouts):
        outputs.append((pixels, affine, layout))
    return outputs


def _cell_columns(video) -> np.ndarray:
    """Rank column held by each (segment, plane, grid row, grid column) picture cell, or ``rank``
    (a zero column) for unused cells: cell i of segment s is column s * slots + i, and cell i
    sits on plane i % planes at grid position divmod(i // planes, columns)."""
    columns, rows = video["grid"]
    planes, segments, slots, rank = video["planes"], video["segments"], video["channels_per_segment"], video["rank"]
    table = np.full((segments, planes, rows, columns), rank, dtype=np.int64)
    for segment in range(segments):
        for cell in range(min(slots, rank - segment * slots)):
            row, column = divmod(cell // planes, columns)
            table[segment, cell % planes, row, column] = segment * slots + cell
    return table


def mosaic_device(pixels: torch.Tensor, video) -> torch.Tensor:
    """``[frames * segments, planes, rows * height, columns * width]`` channel-tile pictures
    (reelcache.channel_tiles.v1) of a tile's codes ``[frames * height * width, rank]``, gathered
    through the cell table of :func:`_cell_columns`; unused cells are 0."""
    frames, height, width, rank = video["frames"], video["height"], video["width"], video["rank"]
    columns, rows = video["grid"]
    planes, segments = video["planes"], video["segments"]
    if pixels.dtype != torch.uint8 or tuple(pixels.shape) != (frames * height * width, rank):
        raise ConfigurationError("mosaic needs the tile's uint8 codes [frames * height * width, rank]")
    table = torch.from_numpy(_cell_columns(video)).to(pixels.device)
    padded = torch.cat((pixels, torch.zeros((pixels.shape[0], 1), dtype=torch.uint8, device=pixels.device)), 1)
    cells = padded[:, table.reshape(-1)].reshape(frames, height, width, segments, planes, rows, columns)
    # -> [segment, frame, plane, grid row, y, grid column, x]
    pictures = cells.permute(3, 0, 4, 5, 1, 6, 2)
    return pictures.reshape(segments * frames, planes, rows * height, columns * width)
