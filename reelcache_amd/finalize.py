"""Final stored measurement, exact quantization and node canvases of fitted tiles (device).

Contract of reelcache/node_packets.py:189-448 (``FinalTile``, ``NodeCanvas``, ``FinalizeItem``,
``finalize_tile``, ``finalize_tiles``, ``assemble_canvas``) with the ideal energy of
reelcache/deferred_reads.py:682-714 (``span_energy_routine``), re-exported by
:mod:`reelcache_amd.node_packets`.

What a finalized tile records, per matrix ``X`` and its FP16 rank-view rows ``Q``:

* ``P = X Q^T`` rounded once to fp32 (the projection kernel: exact products summed in FP64);
* the stored energy ``1 - ||X - P Q||^2 / ||X||^2`` (FP64 residual kernel), which must reach the
  matrix's target unless the tile is a diagnostic one (IntegrityError otherwise);
* the ideal energy of the span of ``Q``: ``||L^-1 P^T||_F^2 / ||X||^2`` with ``L L^T = Q Q^T``;
* the fast condition bound of ``Q`` and the 8-bit codes with their covering affine.

MI355X design: a batch of tiles (a whole chunk: 60 CausVid matrices) is one launch each of the
absmax, projection (with per-column extrema) and residual-energy kernels, per channel count.
The span energy uses the identity ``||L^-1 P^T||_F^2 = trace(G^-1 C)`` with ``G = Q Q^T`` and
``C = P^T P`` (FP64): per group of tiles of one rank, one batched product ``C``, one batched
Cholesky factorization of ``G`` and one batched solve, instead of an ``N x r`` triangular solve
per tile.  The fast condition bound's Gram is one batched fp32
product.  Every scalar the host needs (scales, extrema, energies, traces, factorization status,
condition terms) crosses in one transfer; the quantizer is one launch for the batch.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, replace
from typing import Any, Mapping, Sequence

import numpy as np
import torch

from . import fit_kernels
from ._checks import need
from .errors import IntegrityError
from .factorization import basis_condition_bound
from .quantize import video_layout
from .types import CodecSpec, MatrixKey, TensorContext

_UNIT = 2.0 ** -24


def entry_parts(entry) -> tuple[MatrixKey, str | None]:
    """(key, stream) of a pack entry: a ``MatrixKey`` or a ``(MatrixKey, stream)`` pair."""
    if isinstance(entry, MatrixKey):
        return entry, None
    need(isinstance(entry, tuple) and len(entry) == 2 and isinstance(entry[0], MatrixKey)
         and isinstance(entry[1], str), "a pack entry is a MatrixKey or (MatrixKey, stream)")
    return entry


def entry_order(entry) -> tuple:
    key, stream = entry_parts(entry)
    return key.layer, key.target, "" if stream is None else stream


@dataclass(frozen=True)
class FinalizeItem:
    """One matrix to finalize: device source and FP16 rank-view rows (``host_rows``: the same rows on the host)."""

    matrix: torch.Tensor
    rows16: torch.Tensor
    context: TensorContext
    spec: CodecSpec
    entry: Any
    target: float
    diagnostic: bool
    host_rows: torch.Tensor | None = None


@dataclass(frozen=True)
class FinalTile:
    """One finalized tile: placement, affine, basis prefix bytes and measured energies."""

    entry: Any
    context: TensorContext
    spec: CodecSpec
    video: Mapping[str, Any]
    normalization: Mapping[str, Any]
    affine: bytes
    basis: bytes
    rank: int
    pictures: tuple[int, int]
    stored_energy: float
    relative_residual: float
    condition_bound: float
    ideal_energy: float
    source_energy: float
    zero_input: bool
    coefficients: np.ndarray | None = None
    gram: np.ndarray | None = None

    @property
    def key(self) -> MatrixKey:
        return entry_parts(self.entry)[0]

    @property
    def stream(self) -> str | None:
        return entry_parts(self.entry)[1]


def pack_codec(spec: CodecSpec) -> dict[str, Any]:
    """The pack codec record of an all-intra svd_hevc specification (pixel format, QP, preset)."""
    need(isinstance(spec, CodecSpec) and spec.kind == "svd_hevc", "node packs carry only svd_hevc coefficient tiles")
    return {"kind": "svd_hevc", "pix_fmt": spec.pix_fmt, "qp": spec.qp, "preset": spec.preset,
            "inter_prediction": False}


@dataclass
class NodeCanvas:
    """A node's finalized device canvas, its tiles and (after :meth:`to_host`) host pictures."""

    node_id: str
    contexts: Mapping[Any, TensorContext]
    codec: Mapping[str, Any]
    canvas: Mapping[str, Any]
    tiles: list
    device_pictures: torch.Tensor | None
    host_pictures: np.ndarray | None = None
    event: Any = None
    finalize_seconds: float = 0.0

    @property
    def pictures(self) -> int:
        return int(self.canvas["pictures"])

    @property
    def nbytes(self) -> int:
        return self.pictures * self.canvas["planes"] * self.canvas["width"] * self.canvas["height"]

    def to_host(self, *, buffer: torch.Tensor | None = None, stream: Any = None) -> None:
        """Start the copy of the canvas into ``buffer`` (contiguous host uint8 staging, pinned for an
        asynchronous copy) or a new host array; :meth:`wait` before reading ``host_pictures``."""
        source = self.device_pictures
        need(source is not None, "node canvas has no device pictures")
        if buffer is None:
            host = torch.empty(source.shape, dtype=torch.uint8)
        else:
            need(isinstance(buffer, torch.Tensor) and buffer.dtype == torch.uint8 and buffer.device.type == "cpu"
                 and buffer.is_contiguous() and buffer.numel() >= source.numel(),
                 "canvas staging must be a contiguous host uint8 buffer large enough")
            host = buffer.reshape(-1)[:source.numel()].view(source.shape)
        host.copy_(source, non_blocking=buffer is not None and buffer.is_pinned())
        self.event = torch.cuda.Event()
        self.event.record(torch.cuda.current_stream(source.device) if stream is None else stream)
        self.host_pictures = host.numpy()
        self._host = host

    def wait(self) -> None:
        """Host-wait for the copy; the device pictures are released."""
        if self.event is not None:
            self.event.synchronize()
            self.event = None
        self.device_pictures = None


def _check_item(item: FinalizeItem) -> int:
    rows = item.rows16
    need(isinstance(item, FinalizeItem), "finalization takes FinalizeItem records")
    need(isinstance(rows, torch.Tensor) and rows.dtype == torch.float16 and rows.ndim == 2
         and int(rows.shape[0]) == item.spec.rank,
         "finalization needs the exact FP16 rank-view rows of the resolved spec")
    need(isinstance(item.matrix, torch.Tensor) and item.matrix.ndim == 2
         and int(item.matrix.shape[1]) == int(rows.shape[1]), "finalization rows do not match the matrix channels")
    return int(rows.shape[0])


def _rank_terms(coefficients, rows):
    """Per tile of one rank: FP64 span trace ``trace(G^-1 C)`` (``G = Q Q^T``, ``C = P^T P``), the
    Cholesky status of ``G``, and the fast condition terms (``eta = ||Q Q^T - I||_inf`` of the fp32
    Gram -- fp16 products are exact in fp32 -- and its largest diagonal entry): a handful of
    batched launches for the whole group."""
    q = torch.stack(rows)
    # Tiles of one token count: one stack and one widening for the group.
    p = torch.stack(coefficients).double() if len({c.shape[0] for c in coefficients}) == 1 else None
    if p is not None:
        products = torch.bmm(p.mT, p)
    else:  # tiles of different token counts: one product each
        products = torch.stack([c.double().T @ c.double() for c in coefficients])
    q64 = q.double()
    gram = torch.bmm(q64, q64.mT)
    if gram.shape[1] <= fit_kernels.CHOLESKY_MAX_K and gram.device.type == "cuda":
        # G = R^T R, X = R^-1 (one launch for the group): trace(G^-1 C) = trace(X^T C X) = sum X * (C X).
        inverse, info = fit_kernels.cholesky_inverse(gram)
        traces = (inverse * torch.bmm(products, inverse)).sum((1, 2))
    else:
        factor, info = torch.linalg.cholesky_ex(gram)
        traces = torch.cholesky_solve(products, factor).diagonal(dim1=1, dim2=2).sum(-1)
    q32 = q.float()
    gram32 = torch.bmm(q32, q32.mT)
    largest = gram32.diagonal(dim1=1, dim2=2).abs().amax(-1)
    gram32.diagonal(dim1=1, dim2=2).sub_(1.0)
    eta = gram32.abs().sum(-1).amax(-1)
    return traces, info.double(), eta.double(), largest.double()


def _launch_group(items, ranks):
    """Device measurements of tiles sharing a channel count and dtype, launched: (coefficients,
    the device scalars that :func:`_read_group` transfers)."""
    sources = [item.matrix for item in items]
    rows = [item.rows16 for item in items]
    keys = fit_kernels.absmax(sources)
    coefficients, extrema = fit_kernels.project(sources, rows, ranks, extrema=True)
    totals = fit_kernels.energies(sources, keys, bases=rows, ranks=ranks, coefficients=coefficients)
    n = len(items)
    terms = torch.zeros((4, n), dtype=torch.float64, device=sources[0].device)
    by_rank: dict = {}
    for index, rank in enumerate(ranks):
        by_rank.setdefault(rank, []).append(index)
    for members in by_rank.values():
        values = _rank_terms([coefficients[i] for i in members], [rows[i] for i in members])
        # Consecutive members (one rank: the usual case) take a slice; others an index tensor
        # copied from pinned memory without a host wait (a pageable copy would drain the stream).
        if members == list(range(members[0], members[0] + len(members))):
            index = slice(members[0], members[0] + len(members))
        else:
            index = torch.tensor(members, dtype=torch.long).pin_memory().to(terms.device, non_blocking=True)
        terms[:, index] = torch.stack(values)
    return coefficients, torch.cat((keys.double(), totals.reshape(-1), terms.reshape(-1), extrema.double().reshape(-1)))


def _read_group(launched):
    """(coefficients, per-item host scalar dicts) of a :func:`_launch_group`; one host transfer."""
    coefficients, scalars = launched
    n = len(coefficients)
    scalars = scalars.cpu().numpy()
    fields = {"bits": scalars[:n], "totals": scalars[n:3 * n].reshape(n, 2), "traces": scalars[3 * n:4 * n],
              "info": scalars[4 * n:5 * n], "eta": scalars[5 * n:6 * n], "largest": scalars[6 * n:7 * n],
              "extrema": scalars[7 * n:].reshape(n, -1).astype(np.int64).astype(np.int32)}
    return coefficients, [{name: value[index] for name, value in fields.items()} for index in range(n)]


class _Raised:
    """An exception kept to be raised later."""

    def __init__(self, error: BaseException):
        self.error = error


def _attempt(function, *args):
    try:
        return function(*args)
    except Exception as error:  # raised again by _result, in the item's turn
        return _Raised(error)


def _result(value):
    if isinstance(value, _Raised):
        raise value.error
    return value


def _condition(eta: float, largest: float, rank: int, channels: int, rows16: torch.Tensor) -> float:
    """(1 + eta) / (1 - eta) with eta widened by the fp32 summation slack; the exact FP64 bound when
    eta >= 1/3 (see ``factorization.fast_condition_bound``)."""
    gamma = channels * _UNIT / (1 - channels * _UNIT)
    eta = eta + rank * gamma * largest + rank * _UNIT
    if not math.isfinite(eta) or eta >= 1 / 3:
        return basis_condition_bound(rows16)
    return (1 + eta) / (1 - eta)


@torch.no_grad()
def finalize_tiles(items: Sequence[FinalizeItem], *, tile_rows: int, keep_coefficients: bool = False,
                   products: str = "fp32", workspace=None) -> list[tuple[FinalTile, torch.Tensor]]:
    """:func:`finalize_tile` of many matrices with batched launches and one host transfer per
    channel-count group; errors follow the order of the items.  ``products`` and ``workspace``
    are accepted for the reference's signature (the measurement products are exact products
    summed in FP64 on the device; no host temporaries are pooled)."""
    from . import node_packets as npk
    from .basis_versions import rows_to_bytes

    need(type(tile_rows) is int and tile_rows >= 1, "tile_rows must be a positive integer")
    need(products in ("fp32", "fp32_verified_fp64", "fp64"), "measurement products must be fp32 or fp64")
    items = list(items)
    ranks = [_check_item(item) for item in items]
    groups: dict = {}
    for index, item in enumerate(items):
        groups.setdefault((int(item.matrix.shape[1]), item.matrix.dtype, item.matrix.device), []).append(index)
    coefficients: list = [None] * len(items)
    measured: list = [None] * len(items)
    launched = [(members, _launch_group([items[i] for i in members], [ranks[i] for i in members]))
                for members in groups.values()]
    # Host-only records of every item while the device measures: the picture layout and the
    # stored rows as bytes (from the host copy when there is one).  An error raised here is
    # raised again where the item's record is made, so errors keep the order of the items.
    layouts: list = []
    stored_rows: list = []
    for item, rank in zip(items, ranks):
        context, spec = item.context, item.spec
        layouts.append(_attempt(video_layout, context.frames, context.height, context.width, rank, spec.pix_fmt))
        stored_rows.append(None if item.host_rows is None else _attempt(rows_to_bytes, item.host_rows))
    for members, pending in launched:
        values, scalars = _read_group(pending)
        for position, index in enumerate(members):
            coefficients[index], measured[index] = values[position], scalars[position]
    _, _, finite = fit_kernels.split_keys_many(np.stack([m["extrema"] for m in measured]), ranks)
    tiles = []
    for index, (item, rank, m) in enumerate(zip(items, ranks, measured)):
        need(m["bits"] < fit_kernels.NONFINITE_BITS, "projection requires a nonempty finite FP32-compatible matrix")
        scale = float(np.array([m["bits"]], dtype=np.int64).astype(np.int32).view(np.float32)[0])
        scaled_source, scaled_error = float(m["totals"][0]), float(m["totals"][1])
        zero = scale == 0.0
        residual = 0.0 if zero else math.sqrt(scaled_error / scaled_source)
        stored = 1.0 if zero else 1.0 - residual ** 2
        if not item.diagnostic and not zero and stored < item.target:
            raise IntegrityError(f"{item.entry}: finalized stored representation measures {stored:.9f}, "
                                 f"below {item.target}")
        source_energy = (scale * math.sqrt(scaled_source)) ** 2
        if zero:
            ideal = 1.0
        else:
            need(m["info"] == 0, "stored basis rows are singular", IntegrityError)
            ideal = min(1.0, float(m["traces"]) / source_energy)
        need(finite[index], "coefficients must be finite")
        condition = _condition(float(m["eta"]), float(m["largest"]), rank, int(item.rows16.shape[1]), item.rows16)
        tiles.append((stored, residual, condition, ideal, source_energy, zero))
    codes = npk.quantize_many(coefficients, [m["extrema"] for m in measured], [item.spec for item in items])
    results = []
    for index, (item, rank, measures) in enumerate(zip(items, ranks, tiles)):
        pixels, affine, layout = codes[index]
        context, spec = item.context, item.spec
        video = _result(layouts[index])
        gram = host_coefficients = None
        if keep_coefficients:
            rows64 = item.rows16.double()
            gram = (rows64 @ rows64.T).cpu().numpy()
            host_coefficients = coefficients[index].cpu().numpy()
        basis = rows_to_bytes(item.rows16) if stored_rows[index] is None else _result(stored_rows[index])
        tile = FinalTile(item.entry, context, spec, video, layout, affine.astype("<f4", copy=False).tobytes(), basis,
                         rank, (0, 0), *measures[:2], measures[2], measures[3], measures[4], measures[5],
                         host_coefficients, gram)
        results.append((tile, pixels))
    return results


def finalize_tile(matrix: torch.Tensor, rows16: torch.Tensor, context: TensorContext, spec: CodecSpec, *,
                  entry: Any, target: float, diagnostic: bool, tile_rows: int, keep_coefficients: bool = False,
                  decision_band: float = 0.0, host_rows: torch.Tensor | None = None,
                  products: str = "fp32") -> tuple[FinalTile, torch.Tensor]:
    """Final stored measurement and exact quantization of one matrix on its device: the tile
    (picture range unset) and its device uint8 pixels ``[N, rank]``; IntegrityError when the
    stored representation misses its target."""
    item = FinalizeItem(matrix, rows16, context, spec, entry, target, diagnostic, host_rows)
    return finalize_tiles([item], tile_rows=tile_rows, keep_coefficients=keep_coefficients, products=products)[0]


def assemble_canvas(node_id: str, tiles: Sequence[tuple[FinalTile, torch.Tensor]], *, codec: Mapping[str, Any],
                    ladder: Sequence[int] | None, channels: int) -> NodeCanvas:
    """Lay finalized tiles (in layer, target, stream order) into one temporal canonical canvas: each
    tile's pictures (segments x frames, channel_tiles.v1) at the top-left of consecutive canvas
    pictures, zero elsewhere."""
    from . import node_packets as npk

    need(len(tiles) > 0, "a node pack needs at least one tile")
    ordered = sorted(tiles, key=lambda pair: entry_order(pair[0].entry))
    first = ordered[0][0].context
    for tile, _ in ordered:
        context = tile.context
        need(context.model == first.model and context.token_start == first.token_start
             and (context.frames, context.height, context.width) == (first.frames, first.height, first.width),
             "a node pack cannot span two nodes: matrices differ in token range or geometry")
        need(pack_codec(tile.spec) == dict(codec), "one node pack requires one pixel format, QP and preset")
    node_rank = max(tile.rank for tile, _ in ordered)
    choice = npk.canonical_canvas(first.frames, first.height, first.width, codec["pix_fmt"], node_rank,
                                  channels=channels, ladder=ladder)
    width, height = choice["width"], choice["height"]
    planes = 3 if codec["pix_fmt"] == "yuv444p" else 1
    for tile, _ in ordered:
        need(tile.video["image_width"] <= width and tile.video["image_height"] <= height,
             "a tile exceeds its canonical canvas", IntegrityError)
    counts = [tile.video["frames"] * tile.video["segments"] for tile, _ in ordered]
    canvas = torch.zeros((sum(counts), planes, height, width), dtype=torch.uint8, device=ordered[0][1].device)
    placed, cursor = [], 0
    for (tile, pixels), count in zip(ordered, counts):
        images = npk.mosaic_device(pixels, tile.video)
        canvas[cursor:cursor + count, :, :images.shape[2], :images.shape[3]] = images
        placed.append(replace(tile, pictures=(cursor, count)))
        cursor += count
    record = {"width": width, "height": height, "alignment": npk.CANVAS_ALIGNMENT, "pictures": cursor,
              "planes": planes, "pix_fmt": codec["pix_fmt"], "fill": 0, "rank_step": choice["rank_step"],
              "policy": choice["policy"], "node_max_rank": node_rank}
    return NodeCanvas(node_id, {tile.entry: tile.context for tile in placed}, dict(codec), record, placed, canvas)


__all__ = ["FinalTile", "FinalizeItem", "NodeCanvas", "assemble_canvas", "entry_order", "entry_parts",
           "finalize_tile", "finalize_tiles", "pack_codec"]
