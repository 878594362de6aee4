"""GPU parity of the final measurement of a fitted chunk (reelcache/node_packets.py:290-448,
reelcache/deferred_reads.py:682-714) at the BASELINE configs[2] shape: 60 matrices
``[4680, 1536]`` bf16 finalized in one batched call.

Against the oracle (each tile's own fp32 coefficients, read back with ``keep_coefficients``):
codes and affine bit for bit (``oracle.quantize``), FP64 stored energy and source energy within
1e-12, the ideal (span) energy within 1e-12 of ``oracle.fit.span_energy`` (the reference's
triangular-solve form; the product computes ``trace(G^-1 C)``), the condition bound at or above
the exact FP64 bound and below 1.5 for these near-orthonormal rows, basis bytes equal to the
FP16 rows.  The coefficients themselves are the projection kernel's (tested against the oracle's
exactly rounded product in test_fit_gpu.py).  Also: a missed target is an IntegrityError unless
the tile is diagnostic, a zero matrix is measured as zero input, and a node canvas places every
tile's channel_tiles.v1 pictures at the top-left of its canonical canvas pictures.
"""

import numpy as np
import pytest
import torch

from oracle import fit as of
from oracle import quantize as oq
from reelcache_amd import node_packets as npk
from reelcache_amd.basis_versions import rows_to_bytes
from reelcache_amd.errors import IntegrityError
from reelcache_amd.factorization import basis_condition_bound
from reelcache_amd.types import CodecSpec, MatrixKey, ModelIdentity, TensorContext

pytestmark = pytest.mark.gpu

TOKENS, CHANNELS, GRID = 4680, 1536, (3, 30, 52)
MODEL = ModelIdentity("finalize-test", "e" * 64, 30, CHANNELS, "THD", "bfloat16")


def _context(key, token_start=0):
    return TensorContext(MODEL, key, token_start, *GRID, "pre_rope" if key.target == "K" else "none")


def _item(rng, generator, device, index, rank, target=0.9, diagnostic=False, normalization="per_channel"):
    """X = C Q + noise with Q the FP16 rank-view rows (orthonormal columns of a host QR, rounded)."""
    key = MatrixKey(index // 2, "KV"[index % 2])
    q, _ = np.linalg.qr(rng.standard_normal((CHANNELS, rank)))
    rows16 = torch.from_numpy(q.T.copy()).to(torch.float16)
    weights = torch.linspace(3.0, 0.2, rank, device=device)
    coefficients = torch.randn(TOKENS, rank, device=device, generator=generator) * weights
    noise = torch.randn(TOKENS, CHANNELS, device=device, generator=generator) * 0.01
    x = (coefficients @ rows16.to(device).float() + noise).to(torch.bfloat16)
    spec = CodecSpec("svd_hevc", rank, normalization=normalization,
                     protected_fraction=0.25 if normalization == "leading_columns" else 1.0)
    return npk.FinalizeItem(x, rows16.to(device), _context(key), spec, key, target, diagnostic, rows16)


def test_finalize_chunk_matches_oracle(device):
    rng = np.random.default_rng(90)
    generator = torch.Generator(device=device).manual_seed(90)
    normalizations = ["per_channel", "global", "leading_columns"]
    items = [_item(rng, generator, device, index, int(rng.choice([16, 32, 48, 64, 96])),
                   normalization=normalizations[index % 3]) for index in range(60)]
    results = npk.finalize_tiles(items, tile_rows=1024, keep_coefficients=True)
    assert len(results) == 60
    for item, (tile, pixels) in zip(items, results):
        rows = item.host_rows.numpy()
        host = item.matrix.float().cpu().numpy()
        p = tile.coefficients
        assert p.dtype == np.float32 and p.shape == (TOKENS, tile.rank)
        scale, source, error = of.energies(host, rows, p)
        assert abs(tile.stored_energy - (1.0 - error / source)) <= 1e-12
        assert abs(tile.relative_residual - np.sqrt(error / source)) <= 1e-12
        source_energy = source * scale ** 2
        assert abs(tile.source_energy - source_energy) <= 1e-12 * source_energy
        assert abs(tile.ideal_energy - min(1.0, of.span_energy(p, rows, source_energy))) <= 1e-12
        assert tile.stored_energy <= tile.ideal_energy + 1e-12  # the span holds at least the stored energy
        codes, affine, layout = oq.quantize(p, item.spec.normalization, item.spec.protected_fraction)
        np.testing.assert_array_equal(pixels.cpu().numpy(), codes)
        assert tile.affine == affine.astype("<f4").tobytes()
        assert tile.normalization["protected_count"] == layout["protected_count"]
        assert tile.basis == rows_to_bytes(item.host_rows)
        assert basis_condition_bound(item.rows16) <= tile.condition_bound < 1.5
        assert tile.video["rank"] == tile.rank and not tile.zero_input
        np.testing.assert_array_equal(tile.gram, rows.astype(np.float64) @ rows.astype(np.float64).T)


def test_finalize_targets_zero_input_and_canvas(device):
    rng = np.random.default_rng(91)
    generator = torch.Generator(device=device).manual_seed(91)
    low = _item(rng, generator, device, 0, 8, target=0.9)
    # Only 4 of the 8 rows: about 3/4 of the energy is outside their span.
    short = npk.FinalizeItem(low.matrix, low.rows16[:4].contiguous(), low.context, CodecSpec("svd_hevc", 4),
                             low.entry, 0.999, False)
    with pytest.raises(IntegrityError):
        npk.finalize_tiles([short], tile_rows=1024)
    diagnostic = npk.FinalizeItem(short.matrix, short.rows16, short.context, short.spec, short.entry, 0.999, True)
    (tile, _), = npk.finalize_tiles([diagnostic], tile_rows=1024)
    assert tile.stored_energy < 0.999 and tile.ideal_energy < 1.0
    zero = npk.FinalizeItem(torch.zeros(TOKENS, CHANNELS, dtype=torch.bfloat16, device=device), low.rows16,
                            low.context, low.spec, low.entry, 0.98, False)
    (tile, pixels), = npk.finalize_tiles([zero], tile_rows=1024)
    assert tile.zero_input and tile.stored_energy == 1.0 and tile.ideal_energy == 1.0
    assert int(pixels.max()) == 0
    # A node canvas: K and V of one layer and a streamed entry, in (layer, target, stream) order.
    node = [_item(rng, generator, device, index, rank) for index, rank in ((1, 40), (0, 96))]
    streamed = _item(rng, generator, device, 2, 24)
    node.append(npk.FinalizeItem(streamed.matrix, streamed.rows16, _context(MatrixKey(0, "K")), streamed.spec,
                                 (MatrixKey(0, "K"), "s1"), 0.9, False))
    tiles = npk.finalize_tiles(node, tile_rows=1024)
    codec = npk.pack_codec(node[0].spec)
    canvas = npk.assemble_canvas("n0", tiles, codec=codec, ladder=npk.CANVAS_RANK_LADDER, channels=CHANNELS)
    choice = npk.canonical_canvas(*GRID, "yuv444p", 96, channels=CHANNELS)
    assert (canvas.canvas["width"], canvas.canvas["height"]) == (choice["width"], choice["height"])
    order = [tile.entry for tile in canvas.tiles]
    assert order == [MatrixKey(0, "K"), (MatrixKey(0, "K"), "s1"), MatrixKey(0, "V")]
    pictures = canvas.device_pictures.cpu().numpy()
    covered = np.zeros(pictures.shape, dtype=bool)
    by_entry = {tile.entry: pixels for tile, pixels in tiles}
    for tile in canvas.tiles:
        first, count = tile.pictures
        images = npk.mosaic_device(by_entry[tile.entry], tile.video).cpu().numpy()
        region = (slice(first, first + count), slice(None), slice(0, images.shape[2]), slice(0, images.shape[3]))
        np.testing.assert_array_equal(pictures[region], images)
        covered[region] = True
    assert not pictures[~covered].any()  # zero fill outside the tiles
    assert canvas.pictures == sum(tile.pictures[1] for tile in canvas.tiles)
