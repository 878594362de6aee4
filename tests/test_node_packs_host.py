"""CPU tests of the node-pack geometry and wire functions (reelcache/node_packets.py:63-114,
:771-825).

Canvas ladder: the reference's own invariants (tests/test_step6_node_packets.py:45-70 -- ladder
monotone and cached, every rank covered by its canvas with whole CTUs and at least the decoder's
minimum size, ranks 257..320 of the CausVid geometry sharing one canvas, own-size policy, ranks
beyond the channels refused), a brute-force pass over every rank against the per-rank
channel_tiles.v1 layout (itself pinned to the oracle's layout), and hand-computed sizes.

External tile bases: a pack with three tiles (K, V and a streamed entry) detaches its tile
bases and attaches them back byte for byte; substituted, missing, short and mis-shaped bases
are integrity errors; the tile index maps every entry.
"""

import hashlib

import numpy as np
import pytest
import torch

from reelcache_amd import node_packets as npk
from reelcache_amd import quantize as pq
from reelcache_amd.errors import ConfigurationError, IntegrityError, UnsupportedError
from reelcache_amd.types import EncodedTensor, MatrixKey, ModelIdentity, TensorContext


def test_ladder_invariants_of_the_reference():
    ladder = npk.canvas_ladder(3, 30, 52, "yuv444p", max_rank=1536)
    assert ladder is npk.canvas_ladder(3, 30, 52, "yuv444p", max_rank=1536)  # cached
    widths, heights = [row[1] for row in ladder], [row[2] for row in ladder]
    assert widths == sorted(widths) and heights == sorted(heights)
    for rank in (1, 31, 32, 33, 200, 262, 288, 500, 1536):
        canvas = npk.canonical_canvas(3, 30, 52, "yuv444p", rank, channels=1536)
        layout = pq.video_layout(3, 30, 52, rank, "yuv444p")
        assert canvas["width"] >= layout["image_width"] and canvas["height"] >= layout["image_height"]
        assert min(canvas["width"], canvas["height"]) >= npk.MIN_CANVAS == 160
        assert canvas["width"] % npk.CANVAS_ALIGNMENT == 0 and canvas["height"] % npk.CANVAS_ALIGNMENT == 0
        assert canvas["rank_step"] >= rank and canvas["policy"] == "canonical_rank_ladder"
    sizes = {(c["width"], c["height"]) for c in (npk.canonical_canvas(3, 30, 52, "yuv444p", rank, channels=1536)
                                                 for rank in range(257, 321))}
    assert len(sizes) == 1
    own = npk.canonical_canvas(3, 30, 52, "yuv444p", 262, channels=1536, ladder=None)
    assert own["policy"] == "own_size" and own["rank_step"] is None
    with pytest.raises(ConfigurationError):
        npk.canonical_canvas(3, 30, 52, "yuv444p", 2000, channels=1536)
    with pytest.raises(ConfigurationError):
        npk.canvas_ladder(3, 30, 52, "yuv444p", max_rank=64, ladder=(64, 32))


@pytest.mark.parametrize("geometry,fmt", [((3, 30, 52), "yuv444p"), ((1, 60, 104), "yuv420p"), ((2, 9, 13), "yuv444p"),
                                          ((4, 4, 4), "yuv420p")])
def test_ladder_is_the_running_maximum_of_every_rank(geometry, fmt):
    """Brute force: each step's canvas is the largest CTU-aligned picture of ranks 1..step (and at
    least MIN_CANVAS), from the per-rank layout."""
    channels = 700
    ladder = dict((step, (w, h)) for step, w, h in npk.canvas_ladder(*geometry, fmt, max_rank=channels))
    widest = tallest = npk.MIN_CANVAS
    for rank in range(1, channels + 1):
        layout = pq.video_layout(*geometry, rank, fmt)
        widest = max(widest, -(-layout["image_width"] // 32) * 32)
        tallest = max(tallest, -(-layout["image_height"] // 32) * 32)
        if rank in ladder:
            assert ladder[rank] == (widest, tallest), (rank, ladder[rank], widest, tallest)
    assert max(ladder) == channels


def test_hand_computed_canvases():
    # Rank 262 of 3 x 30 x 52 in yuv444p: ceil(sqrt(262 / 3)) = 10 grid columns, ceil(262 / 30) = 9
    # rows -> a 520 x 270 picture -> 544 x 288 in whole 32-pixel CTUs.
    own = npk.canonical_canvas(3, 30, 52, "yuv444p", 262, channels=1536, ladder=None)
    assert (own["width"], own["height"]) == (544, 288)
    # Ranks 1..32: rank 32 is the widest (4 columns, 3 rows: 208 x 90 -> 224 x 96), height raised to
    # the 160-pixel minimum.
    assert npk.canvas_ladder(3, 30, 52, "yuv444p", max_rank=1536)[0] == (32, 224, 160)


def _context(layer, target):
    model = ModelIdentity("pack-test", "b" * 64, 4, 64, "THD", "bfloat16")
    return TensorContext(model, MatrixKey(layer, target), 0, 1, 4, 6, "pre_rope" if target == "K" else "none")


def _pack(rng):
    tiles, payloads, descriptors, bases = [], {}, {}, []
    for index, (layer, target, stream, rank) in enumerate([(0, "K", None, 5), (0, "V", None, 3), (1, "K", 2, 7)]):
        rows = torch.from_numpy(rng.standard_normal((rank, 64))).to(torch.float16)
        raw = rows.numpy().tobytes()
        name = f"basis.{index:03d}.f16"
        payloads[name] = raw
        descriptors[name] = {"bytes": len(raw), "sha256": hashlib.sha256(raw).hexdigest(), "dtype": "float16",
                             "shape": [rank, 64]}
        coefficients = rng.integers(0, 256, size=24 * rank, dtype=np.uint8).tobytes()
        payloads[f"coefficients.{index:03d}"] = coefficients
        descriptors[f"coefficients.{index:03d}"] = {"bytes": len(coefficients), "dtype": "uint8"}
        tiles.append({"key": MatrixKey(layer, target).to_dict(), "stream": stream,
                      "context": _context(layer, target).to_dict(), "basis": {"payload": name, "view_rank": rank}})
        bases.append(raw)
    metadata = {"schema": npk.PACK_SCHEMA, "tiles": tiles, "payloads": descriptors}
    return EncodedTensor(metadata, payloads), bases


def test_canonical_canvas_shapes_known_answers():
    """The reference's known answers (tests/test_packed_nvdec.py:1404-1424): the shapes are the
    ladder's canvases in order; every rank's canonical canvas is one of them and is the last shape
    when ``max_rank`` is that rank; the CausVid geometry has 15 canonical canvases, 9 up to rank
    384; bad ranks and pixel formats are refused."""
    for frames, height, width, channels in ((3, 30, 52, 1536), (8, 22, 40, 3072), (4, 44, 82, 4096)):
        shapes = npk.canonical_canvas_shapes(frames, height, width, "yuv444p", channels=channels)
        ladder = npk.canvas_ladder(frames, height, width, "yuv444p", max_rank=channels)
        assert shapes == [(w, h, "yuv444p") for _, w, h in ladder]
        for rank in range(1, channels + 1, 7):
            canvas = npk.canonical_canvas(frames, height, width, "yuv444p", rank, channels=channels)
            assert (canvas["width"], canvas["height"], "yuv444p") in shapes
            bounded = npk.canonical_canvas_shapes(frames, height, width, "yuv444p", channels=channels, max_rank=rank)
            assert bounded[-1] == (canvas["width"], canvas["height"], "yuv444p")
    assert len(npk.canonical_canvas_shapes(3, 30, 52, "yuv444p", channels=1536)) == 15  # CausVid
    assert len(npk.canonical_canvas_shapes(3, 30, 52, "yuv444p", channels=1536, max_rank=384)) == 9
    for bad in (0, 1537, 2.0):
        with pytest.raises(ConfigurationError):
            npk.canonical_canvas_shapes(3, 30, 52, "yuv444p", channels=1536, max_rank=bad)
    with pytest.raises(UnsupportedError):
        npk.canonical_canvas_shapes(3, 30, 52, "rgb24", channels=1536)


def test_pack_bases_detach_and_attach_byte_exact():
    encoded, bases = _pack(np.random.default_rng(5))
    metadata, payloads, detached = npk.detach_pack_bases(encoded)
    assert detached == bases and not any(name.startswith("basis.") for name in payloads)
    restored = npk.attach_pack_bases(metadata, payloads, detached)
    assert dict(restored.payloads) == dict(encoded.payloads) and restored.metadata == encoded.metadata
    assert npk.pack_tile_index(metadata) == {MatrixKey(0, "K"): 0, MatrixKey(0, "V"): 1, (MatrixKey(1, "K"), 2): 2}


def test_pack_bases_refuse_substitutes():
    encoded, bases = _pack(np.random.default_rng(6))
    metadata, payloads, detached = npk.detach_pack_bases(encoded)
    forged = list(detached)
    forged[1] = bytes(len(forged[1]))  # same length, other bytes
    with pytest.raises(IntegrityError):
        npk.attach_pack_bases(metadata, payloads, forged)
    npk.attach_pack_bases(metadata, payloads, forged, check_digests=False)  # only the digest is skipped
    with pytest.raises(IntegrityError):
        npk.attach_pack_bases(metadata, payloads, forged[:1] + [forged[1][:-2]] + forged[2:], check_digests=False)
    with pytest.raises(IntegrityError):
        npk.attach_pack_bases(metadata, payloads, detached[:-1])
    with pytest.raises(IntegrityError):
        npk.attach_pack_bases(metadata, dict(encoded.payloads), detached)  # bases embedded already
    bad = dict(metadata, payloads=dict(metadata["payloads"]))
    bad["payloads"]["basis.000.f16"] = dict(bad["payloads"]["basis.000.f16"], shape=[4, 64])
    with pytest.raises(IntegrityError):
        npk.attach_pack_bases(bad, payloads, detached)
    tampered = dict(encoded.payloads)
    tampered["basis.002.f16"] = bytes(len(tampered["basis.002.f16"]))
    with pytest.raises(IntegrityError):
        npk.detach_pack_bases(EncodedTensor(encoded.metadata, tampered))
    with pytest.raises(ConfigurationError):
        npk.detach_pack_bases(EncodedTensor(dict(encoded.metadata, schema="reelcache.tensor.v1"), encoded.payloads))
