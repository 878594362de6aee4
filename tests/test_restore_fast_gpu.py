"""GPU parity of the straight-line restore kernels (csrc/restore_fast.h).

Launch groups whose jobs all qualify (uint8 codes in 16-byte aligned rows or pictures,
head_dim % 32 == 0, unit-stride aligned destinations) run the straight-line kernel (two heads
per step when the head count is even, one with ``config={"head_pairs": False}``); every case
here runs the same inputs through the straight-line and general kernels
(``config={"fast_variant": False}``) and requires equal values, then checks them against the
oracle's elementwise error bound (reelcache/restore_kernels.py:1208-1227).
"""

import zlib

import numpy as np
import pytest
import torch

from oracle import quantize as oq
from oracle import restore as orc
from reelcache_amd import restore_kernels as rk

from restore_cases import destination, expected, make_case, written

pytestmark = pytest.mark.gpu

# (layout, heads, head_dim, rank, rope, grid, token_offset, code_pitch)
SHAPES = [
    ("BTHD", 3, 128, 128, "separable", (3, 7, 11), 5, None),   # ragged last tile (231 tokens)
    ("THD", 2, 64, 33, "dense", (2, 9, 13), 0, 48),             # rank tail inside a 16-byte group
    ("BHTD", 4, 64, 150, "none", (1, 16, 8), 2, 160),            # exactly one tile
    ("BTHD", 12, 128, 192, "none", (1, 20, 26), 0, None),        # V-shaped, 5 tiles
    ("BTHD", 1, 96, 7, "separable", (2, 3, 5), 1, 16),           # tiny rank, 30 tokens
]


VARIANTS = {"pairs": {}, "fast": {"head_pairs": False}, "general": {"fast_variant": False}}


def _copies(seed, precision, out_dtype, shape, device, count=len(VARIANTS)):
    layout, heads, head_dim, rank, rope, grid, token_offset, pitch = shape
    cases = []
    for _ in range(count):
        rng = np.random.default_rng(seed)
        cases.append(make_case(rng, grid=grid, heads=heads, head_dim=head_dim, rank=rank, source="uint8",
                               rope=rope, layout=layout, out_dtype=out_dtype, device=device,
                               token_offset=token_offset, code_pitch=pitch))
    return cases


def _run(case, precision, variant):
    handle = rk.reconstruct([case.job], precision=precision, config=VARIANTS[variant])
    handle.release()
    return handle.stats["variants"]


def _check_bound(case, precision):
    values, bound = expected(case, precision)
    excess = np.abs(written(case) - values) - bound
    assert float(excess.max()) <= 0, f"{int((excess > 0).sum())} elements exceed the error bound"


@pytest.mark.parametrize("precision", ["fp16x2", "fp16", "bf16"])
@pytest.mark.parametrize("out_dtype", ["bfloat16", "float16", "float32"])
def test_fast_matches_general_and_oracle(device, precision, out_dtype):
    for index, shape in enumerate(SHAPES):
        seed = zlib.crc32(f"{precision}/{out_dtype}/{index}".encode())
        cases = dict(zip(VARIANTS, _copies(seed, precision, out_dtype, shape, device)))
        for variant, case in cases.items():
            label = "fast" if variant == "pairs" and shape[1] % 2 else variant  # odd heads: one per step
            assert _run(case, precision, variant) == [label], shape
        out_general = written(cases["general"])
        for variant in ("pairs", "fast"):
            assert np.array_equal(written(cases[variant]), out_general), f"{shape}: {variant} and general kernels differ"
        _check_bound(cases["pairs"], precision)
        # Tokens outside the slot are untouched.
        layout, token_offset = shape[0], shape[6]
        tensor = cases["pairs"].job.destination.tensor
        canonical = (tensor.transpose(1, 2) if layout == "BHTD" else tensor).reshape(-1, shape[1] * shape[2])
        tokens = int(np.prod(shape[5]))
        assert bool((canonical[:token_offset] == -123.0).all())
        assert bool((canonical[token_offset + tokens:] == -123.0).all())


def test_fast_pictures_and_mixed_groups(device):
    """Pictures and uint8 sources, K (RoPE) and V (none) jobs in one call: the (source kind, RoPE)
    groups (two heads per step: the head count is even) run as one pair launch, bit-identical to
    one straight-line launch per group; with the channel-slice variant enabled, the uint8 rows
    take it and the pictures stay on the straight-line kernel."""
    rng = np.random.default_rng(31)
    table = rk.RopeTable.from_complex(torch.from_numpy(orc.wan_freqs(64, 64)))
    heads, head_dim, grid, tokens = 4, 64, (2, 12, 14), 336
    cache_k = destination("BTHD", 2 * tokens, heads, head_dim, "bfloat16", device)
    cache_v = destination("BTHD", 2 * tokens, heads, head_dim, "bfloat16", device)
    cases = []
    for chunk in range(2):
        cases.append(make_case(rng, grid=grid, heads=heads, head_dim=head_dim, rank=96, source="pictures",
                               view=rk.NativeView(cache_k, token_offset=chunk * tokens), table=table,
                               rope_rows=(2 * chunk, 0, 0), out_dtype="bfloat16", device=device))
        cases.append(make_case(rng, grid=grid, heads=heads, head_dim=head_dim, rank=160, source="uint8",
                               view=rk.NativeView(cache_v, token_offset=chunk * tokens), rope="none",
                               out_dtype="bfloat16", device=device))
    handle = rk.reconstruct([case.job for case in cases])
    handle.release()
    assert handle.stats["variants"] == ["pair"]  # the K (pictures, RoPE) and V groups in one launch
    for case in cases:
        _check_bound(case, "fp16x2")
    paired = [case.job.destination.slot(case.job.tokens).clone() for case in cases]
    handle = rk.reconstruct([case.job for case in cases], config={"pair_launch": False})
    handle.release()
    assert sorted(handle.stats["variants"]) == ["pairs", "pairs"]
    for case, want in zip(cases, paired):
        assert torch.equal(case.job.destination.slot(case.job.tokens), want)  # same bits, one launch per group


def test_unaligned_jobs_use_the_general_kernel(device):
    rng = np.random.default_rng(37)
    case = make_case(rng, grid=(1, 5, 7), heads=2, head_dim=64, rank=33, source="uint8", device=device)
    handle = rk.reconstruct([case.job])
    handle.release()
    assert handle.stats["variants"] == ["general"]  # rows of 33 bytes are not 16-byte aligned
    _check_bound(case, "fp16x2")


@pytest.mark.parametrize("grid,rank,heads,rope", [((2, 12, 16), 96, 4, "none"),        # one segment, 4-aligned
                                                  ((3, 30, 52), 192, 2, "separable")])  # CausVid cells, rank 192
def test_fast_picture_word_gather(device, grid, rank, heads, rope):
    """Pictures whose geometry is 4-byte aligned (origin x and grid_w multiples of 4, aligned
    strides) take the word gather (4 tokens x 4 ranks per set of 32-bit loads, transposed in
    registers); the same codes at an unaligned origin take the byte gather.  Both equal the
    general kernel bit for bit and stay within the oracle's bound."""
    from reelcache_amd.restore_plan import job_desc

    cases = []
    for origin, pad in (((0, 0), (3, 4)), ((0, 0), (3, 4)), ((2, 3), (3, 5))):
        rng = np.random.default_rng(59)
        cases.append(make_case(rng, grid=grid, heads=heads, head_dim=128 if rank == 192 else 32, rank=rank,
                               source="pictures", rope=rope, out_dtype="bfloat16", device=device, picture_origin=origin,
                               picture_pad=pad))
    assert job_desc(cases[0].job).pic_vec_rule and all(p.data_ptr() % 4 == 0 for p in job_desc(cases[0].job).pictures)
    assert _run(cases[0], "fp16x2", "pairs") == ["pairs"]
    assert _run(cases[1], "fp16x2", "general") == ["general"]
    assert _run(cases[2], "fp16x2", "pairs") == ["pairs"]
    assert np.array_equal(written(cases[0]), written(cases[1]))
    assert np.array_equal(written(cases[2]), written(cases[1]))
    _check_bound(cases[0], "fp16x2")


# (heads, head_dim, rank, rope, grid): ranks beyond one wave's registers (rank halves)
SPLIT_SHAPES = [
    (4, 128, 200, "separable", (2, 9, 13)),   # fp16x2: 13 steps -> halves of 8
    (6, 64, 300, "none", (1, 16, 9)),         # 19 steps -> halves of 12, one partial tile
    (5, 128, 500, "dense", (3, 7, 11)),       # 32 steps -> halves of 16, ragged last tile
]


@pytest.mark.parametrize("precision", ["fp16x2", "fp16", "bf16"])
@pytest.mark.parametrize("out_dtype", ["bfloat16", "float32"])
def test_rank_halves_match_general_and_oracle(device, precision, out_dtype):
    """Ranks beyond one wave's registers run the rank-halves kernel (8-wave workgroups, the high
    half's fp32 partial sums added through LDS): within the oracle's bound like the general
    kernel, and equal to it except where the different fp32 summation order moves a final
    rounding (a small fraction of elements)."""
    limit = 12 if precision == "fp16x2" else 16
    for index, (heads, head_dim, rank, rope, grid) in enumerate(SPLIT_SHAPES):
        seed = zlib.crc32(f"split/{precision}/{out_dtype}/{index}".encode())
        cases = []
        for _ in range(2):
            rng = np.random.default_rng(seed)
            cases.append(make_case(rng, grid=grid, heads=heads, head_dim=head_dim, rank=rank, source="uint8",
                                   rope=rope, out_dtype=out_dtype, device=device, token_offset=3,
                                   code_pitch=-(-rank // 16) * 16))  # 16-byte aligned code rows
        handle = rk.reconstruct([cases[0].job], precision=precision)
        handle.release()
        steps = (rank + 15) // 16
        want = ["split"] if steps > limit else ["fast" if heads % 2 or steps > 12 else "pairs"]
        assert handle.stats["variants"] == want, (rank, handle.stats["variants"])
        assert _run(cases[1], precision, "general") == ["general"]
        _check_bound(cases[0], precision)
        _check_bound(cases[1], precision)
        ours, general = written(cases[0]), written(cases[1])
        if out_dtype != "float32":  # fp32 outputs keep the summation order's last bits
            differ = float((ours != general).mean())
            assert differ <= 0.02, f"rank {rank}: {differ:.4f} of elements differ from the general kernel"


@pytest.mark.parametrize("grid,rank,heads", [((2, 12, 14), 96, 4),     # one segment (the coalesced gather)
                                             ((1, 2100, 100), 40, 2)])  # two segments (cells of 2100 x 100)
def test_fast_picture_segments(device, grid, rank, heads):
    """Picture sources in the straight-line kernel: layouts of one segment take the coalesced
    gather (cell offsets tabulated per tile), others the per-token gather; both equal the
    general kernel bit for bit and stay within the oracle's bound."""
    assert oq.video_layout(*grid, rank, "yuv444p")["segments"] == (1 if rank == 96 else 2)
    cases = []
    for _ in range(2):
        rng = np.random.default_rng(53)
        cases.append(make_case(rng, grid=grid, heads=heads, head_dim=32, rank=rank, source="pictures", rope="none",
                               out_dtype="bfloat16", device=device))
    assert _run(cases[0], "fp16x2", "fast") == ["fast"]
    assert _run(cases[1], "fp16x2", "general") == ["general"]
    assert np.array_equal(written(cases[0]), written(cases[1]))
    _check_bound(cases[0], "fp16x2")
