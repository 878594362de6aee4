"""Node packs: canonical canvases, device quantization of fitted coefficients, tile canvases and
the external-basis wire functions.

Mirrors ``reelcache/node_packets.py``: the canvas ladder ``_tile_dims`` / ``canvas_ladder`` /
``canonical_canvas`` (:63-114), affine_from_extrema (:140-152), quantize_device (:155-173, exactly
``_hevc.quantize_coefficients`` on the device), mosaic_device (:176-187) and
``detach_pack_bases`` / ``attach_pack_bases`` / ``pack_tile_index`` (:771-825).

Canvas ladder: decoders cannot change picture size within a session, so a node's canvas comes from
a fixed ladder per (frames, height, width, pixel format): the canvas of the smallest ladder step
at or above the node's widest tile rank, where a step's canvas covers every rank up to it.  Here
the channel_tiles.v1 picture size of every rank up to the largest step is computed in one
vectorized pass and the ladder is its running maximum at the steps.

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
import hashlib
from typing import Any, Mapping, Sequence

from ._checks import need
from .errors import ConfigurationError, IntegrityError, UnsupportedError
from .quantize import (MAX_DIMENSION, PIXEL_FORMATS, affine_from_extrema, covering_affine, expanded_affine,
                       normalization_layout, video_layout)
from .types import EncodedTensor, MatrixKey, TensorContext, json_copy

__all__ = ["CANVAS_ALIGNMENT", "CANVAS_RANK_LADDER", "FACTOR_PACK_SCHEMA", "MIN_CANVAS", "PACK_SCHEMA",
           "affine_from_extrema", "attach_pack_bases", "canonical_canvas", "canonical_canvas_shapes", "canvas_ladder",
           "detach_pack_bases",
           "mosaic_device", "pack_tile_index", "quantize_device", "quantize_many", "quantize_with_extrema",
           "video_layout"]

#: Rank steps of the canonical canvas ladder (per frames/height/width/pix_fmt geometry).
CANVAS_RANK_LADDER = (32, 64, 96, 128, 160, 192, 256, 320, 384, 512, 640, 768, 1024, 1280, 1536, 2048,
                      3072, 4096, 6144, 8192)
#: Packed canvases hold whole 32 x 32 coding tree units.
CANVAS_ALIGNMENT = 32
#: Smallest picture a hardware HEVC decoder accepts; canvases are at least this, in whole CTUs.
NVDEC_MIN_DIMENSION = 144
MIN_CANVAS = -(-NVDEC_MIN_DIMENSION // CANVAS_ALIGNMENT) * CANVAS_ALIGNMENT
PACK_SCHEMA = "reelcache.tensor_pack.v2"
FACTOR_PACK_SCHEMA = "reelcache.factor_pack.v1"
_LADDERS: dict = {}


def _align(values):
    return -(-values // CANVAS_ALIGNMENT) * CANVAS_ALIGNMENT


def _tile_sizes(frames: int, height: int, width: int, ranks, pix_fmt: str):
    """CTU-aligned (width, height) int64 arrays of the channel_tiles.v1 picture of every rank in
    ``ranks``: the vectorized form of :func:`reelcache_amd.quantize.video_layout`'s grid rule
    (columns = min(8192 // width, max(1, ceil(sqrt(rank / planes)))), rows likewise from the
    columns; at least 16 pixels; even sizes for yuv420p)."""
    need(pix_fmt in PIXEL_FORMATS, f"picture layouts support exactly {PIXEL_FORMATS}, not {pix_fmt!r}",
         UnsupportedError)
    need(height <= MAX_DIMENSION and width <= MAX_DIMENSION,
         f"coefficient tiles cannot exceed {MAX_DIMENSION}x{MAX_DIMENSION}", UnsupportedError)
    planes = 3 if pix_fmt == "yuv444p" else 1
    rank = np.asarray(ranks, dtype=np.float64)
    columns = np.minimum(MAX_DIMENSION // width, np.maximum(1, np.ceil(np.sqrt(rank / planes)))).astype(np.int64)
    rows = np.minimum(MAX_DIMENSION // height, np.maximum(1, np.ceil(rank / (planes * columns)))).astype(np.int64)
    image_width, image_height = np.maximum(16, columns * width), np.maximum(16, rows * height)
    if pix_fmt == "yuv420p":
        image_width, image_height = image_width + image_width % 2, image_height + image_height % 2
    need(int(image_width.max()) <= MAX_DIMENSION and int(image_height.max()) <= MAX_DIMENSION,
         "padded picture dimensions exceed provider support", UnsupportedError)
    return _align(image_width), _align(image_height)


def _tile_dims(frames: int, height: int, width: int, rank: int, pix_fmt: str) -> tuple[int, int]:
    """CTU-aligned (width, height) of one rank's channel_tiles.v1 picture."""
    widths, heights = _tile_sizes(frames, height, width, [rank], pix_fmt)
    return int(widths[0]), int(heights[0])


def canvas_ladder(frames: int, height: int, width: int, pix_fmt: str, *, max_rank: int,
                  ladder: Sequence[int] = CANVAS_RANK_LADDER) -> tuple[tuple[int, int, int], ...]:
    """``(rank_step, width, height)`` canvases, each covering every rank up to its step (cached);
    the steps are the ladder's below ``max_rank`` and ``max_rank`` itself."""
    for value in (frames, height, width, max_rank):
        need(type(value) is int and value >= 1, "canvas ladder geometry and rank must be positive integers")
    steps = tuple(ladder)
    need(steps and all(type(step) is int and step >= 1 for step in steps)
         and all(a < b for a, b in zip(steps, steps[1:])),
         "canvas rank ladder must be strictly increasing positive integers")
    key = (frames, height, width, pix_fmt, max_rank, steps)
    if key not in _LADDERS:
        widths, heights = _tile_sizes(frames, height, width, np.arange(1, max_rank + 1), pix_fmt)
        widest = np.maximum.accumulate(np.maximum(widths, MIN_CANVAS))
        tallest = np.maximum.accumulate(np.maximum(heights, MIN_CANVAS))
        targets = [step for step in steps if step < max_rank] + [max_rank]
        _LADDERS[key] = tuple((step, int(widest[step - 1]), int(tallest[step - 1])) for step in targets)
    return _LADDERS[key]


def canonical_canvas(frames: int, height: int, width: int, pix_fmt: str, node_max_rank: int, *, channels: int,
                     ladder: Sequence[int] | None = CANVAS_RANK_LADDER) -> dict[str, Any]:
    """The canvas of a node whose widest tile has ``node_max_rank`` coefficient columns: the first
    ladder step at or above it (``policy="canonical_rank_ladder"``), or with ``ladder=None`` the
    node's own smallest canvas (``policy="own_size"``)."""
    need(type(node_max_rank) is int and 1 <= node_max_rank <= channels,
         "node rank must be a positive integer within the channel count")
    if ladder is None:
        tile_width, tile_height = _tile_dims(frames, height, width, node_max_rank, pix_fmt)
        return {"width": max(tile_width, MIN_CANVAS), "height": max(tile_height, MIN_CANVAS), "rank_step": None,
                "policy": "own_size"}
    for step, canvas_width, canvas_height in canvas_ladder(frames, height, width, pix_fmt, max_rank=channels,
                                                           ladder=ladder):
        if step >= node_max_rank:
            need(canvas_width <= MAX_DIMENSION and canvas_height <= MAX_DIMENSION,
                 "canonical canvas exceeds the HEVC provider's maximum picture dimension", UnsupportedError)
            return {"width": canvas_width, "height": canvas_height, "rank_step": step,
                    "policy": "canonical_rank_ladder"}
    raise ConfigurationError("canvas ladder does not cover the node rank")


def canonical_canvas_shapes(frames: int, height: int, width: int, pix_fmt: str, *, channels: int,
                            max_rank: int | None = None,
                            ladder: Sequence[int] | None = None) -> list[tuple[int, int, str]]:
    """``(width, height, pix_fmt)`` of every canonical node canvas of one tile geometry, smallest
    first (reelcache/packed_decode.py:115-139): the distinct canvases of :func:`canvas_ladder` over
    all ``channels`` ranks, up to the first step covering ``max_rank`` (default: every rank), without
    those beyond the maximum picture dimension (no pack can use them).  These are the pictures a
    decoder must be ready for to restore any node pack of the geometry."""
    need(type(channels) is int and channels >= 1, "channels must be a positive integer")
    limit = channels if max_rank is None else max_rank
    need(type(limit) is int and 1 <= limit <= channels, "max_rank must be an integer in [1, channels]")
    need(pix_fmt in PIXEL_FORMATS, f"HEVC supports exactly {PIXEL_FORMATS}, not {pix_fmt!r}", UnsupportedError)
    shapes: list[tuple[int, int, str]] = []
    for step, canvas_width, canvas_height in canvas_ladder(frames, height, width, pix_fmt, max_rank=channels,
                                                           ladder=CANVAS_RANK_LADDER if ladder is None else ladder):
        shape = (canvas_width, canvas_height, pix_fmt)
        if max(canvas_width, canvas_height) <= MAX_DIMENSION and shape not in shapes:
            shapes.append(shape)
        if step >= limit:
            break
    return shapes


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
    ``keys`` are the host extrema rows of ``fit_kernels.project(..., extrema=True)`` (decoded
    together; per-channel covering affines of equal rank computed together).
    Returns ``[(pixels, affine, layout)]``."""
    ranks = []
    for p in coefficients:
        _check(p)
        ranks.append(int(p.shape[1]))
    rows = [np.asarray(row) for row in keys]
    width = max((len(row) for row in rows), default=0)
    if rows and all(len(row) == width for row in rows):
        block = np.stack(rows).astype(np.int64)  # rows of one key block (the common case)
    else:
        block = np.zeros((len(ranks), width), dtype=np.int64)
        for index, row in enumerate(rows):
            block[index, :len(row)] = row
    lows, highs, finite = fit_kernels.split_keys_many(block, ranks)
    if not all(finite):
        raise ConfigurationError("coefficients must be finite")
    layouts = [normalization_layout(rank, spec.normalization, spec.protected_fraction)
               for rank, spec in zip(ranks, specs)]
    payloads: list = [None] * len(ranks)
    per_channel: dict = {}
    for index, layout in enumerate(layouts):
        if layout["mode"] == "per_channel":
            per_channel.setdefault(ranks[index], []).append(index)
        else:
            payloads[index] = affine_from_extrema(lows[index], highs[index], layout)
    for members in per_channel.values():
        # Elementwise covering affine of every per-channel matrix of one rank in one call.
        covered = covering_affine(np.stack([lows[i] for i in members]), np.stack([highs[i] for i in members]))
        for position, index in enumerate(members):
            payloads[index] = np.ascontiguousarray(covered[:, position])
    affines, outputs, values = [], [], []
    for p, rank, layout, affine in zip(coefficients, ranks, layouts, payloads):
        if layout["mode"] == "per_channel":  # the payload is the per-column (scale; offset) itself
            affines.append(affine.astype(np.float64))
        else:
            scale, offset = expanded_affine(affine, layout, rank)
            affines.append(np.stack((np.asarray(scale, np.float64), np.asarray(offset, np.float64))))
        values.append(p if p.stride(1) == 1 else p.contiguous())
    layouts = [(affine.astype("<f4", copy=False), layout) for affine, layout in zip(payloads, layouts)]
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


# ---------------------------------------------------------------------------
# External tile bases of node packs
# ---------------------------------------------------------------------------


def _basis_matches(raw: bytes, descriptor: Mapping[str, Any], check_digest: bool = True) -> bool:
    return (isinstance(raw, (bytes, bytearray)) and len(raw) == descriptor.get("bytes")
            and (not check_digest or hashlib.sha256(raw).hexdigest() == descriptor.get("sha256")))


def detach_pack_bases(encoded: EncodedTensor) -> tuple[dict[str, Any], dict[str, bytes], list[bytes]]:
    """Split a node pack into (metadata, the payloads without the tile bases, each tile's basis
    bytes in tile order), after checking every basis against its payload descriptor."""
    metadata = json_copy(encoded.metadata)
    need(metadata.get("schema") in (PACK_SCHEMA, FACTOR_PACK_SCHEMA) and encoded.basis is None,
         "only tensor_pack.v2 node packs detach per-tile bases")
    payloads = dict(encoded.payloads)
    bases = []
    for tile in metadata["tiles"]:
        name = tile["basis"]["payload"]
        need(name in payloads, "node pack lacks a tile basis payload", IntegrityError)
        raw = payloads.pop(name)
        need(_basis_matches(raw, metadata["payloads"][name]), "node pack tile basis differs from its descriptor",
             IntegrityError)
        bases.append(raw)
    return metadata, payloads, bases


def attach_pack_bases(metadata: Mapping[str, Any], payloads: Mapping[str, bytes], bases: Sequence[bytes], *,
                      check_digests: bool = True) -> EncodedTensor:
    """Re-insert assembled basis prefixes, one per tile in tile order, each checked against its tile's
    descriptor: FP16 ``[view_rank, channels]`` of the tile's context, its length and (unless
    ``check_digests`` is False, for prefixes assembled from hash-checked blocks) its SHA-256."""
    tiles = metadata["tiles"]
    need(len(bases) == len(tiles), "one assembled basis prefix is required per pack tile", IntegrityError)
    combined = dict(payloads)
    for tile, raw in zip(tiles, bases):
        name = tile["basis"]["payload"]
        descriptor = metadata["payloads"].get(name)
        need(name not in combined and isinstance(descriptor, Mapping),
             "stored node pack embeds a basis or lacks its descriptor", IntegrityError)
        channels = TensorContext.from_dict(tile["context"]).channels
        need(descriptor.get("shape") == [tile["basis"]["view_rank"], channels] and descriptor.get("dtype") == "float16",
             "node pack basis descriptor is not the tile's rank-view prefix", IntegrityError)
        need(_basis_matches(raw, descriptor, check_digests),
             "assembled basis version prefix differs from the packed tile descriptor", IntegrityError)
        combined[name] = bytes(raw)
    return EncodedTensor(metadata, combined, None, {})


def pack_tile_index(metadata: Mapping[str, Any]) -> dict[Any, int]:
    """Tile index of every ``MatrixKey`` (or ``(MatrixKey, stream)``) entry of a pack."""
    index = {}
    for position, tile in enumerate(metadata["tiles"]):
        key = MatrixKey.from_dict(tile["key"])
        index[key if tile["stream"] is None else (key, tile["stream"])] = position
    return index


# Final measurement and node canvases live in :mod:`reelcache_amd.finalize` (they use the functions
# above); the reference's module exports them from here.
from .finalize import (FinalizeItem, FinalTile, NodeCanvas, assemble_canvas, finalize_tile,  # noqa: E402
                       finalize_tiles, pack_codec)

__all__ += ["FinalTile", "FinalizeItem", "NodeCanvas", "assemble_canvas", "finalize_tile", "finalize_tiles",
            "pack_codec"]
