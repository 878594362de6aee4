"""CPU tests of the product's host logic (``reelcache_amd``) against the oracle.

Covers the parts of the restore path that run on the host: the 8-bit quantizer and its
layouts (reelcache/_hevc.py:400-540), RoPE tables and positions (reelcache/restore_kernels.py
:308-607), the CPU reference backend (:1090-1168), input validation and error classes
(:770-868, errors.py), backend / precision resolution (never a silent fallback), and the
launch planner's tile table, cost-balanced ranges and straight-line eligibility.
"""

import numpy as np
import pytest
import torch

from oracle import quantize as oq
from oracle import restore as orc
from reelcache_amd import _lib, quantize as pq
from reelcache_amd import restore_kernels as rk
from reelcache_amd import restore_plan as rp
from reelcache_amd.errors import ConfigurationError, IntegrityError, UnsupportedError

from restore_cases import make_case, written


# ---------------------------------------------------------------------------
# Quantizer: product == oracle, bit for bit
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("normalization,fraction", [("per_channel", 1.0), ("global", 1.0),
                                                    ("leading_columns", 0.25), ("leading_columns", 0.5)])
def test_quantizer_matches_oracle(normalization, fraction):
    rng = np.random.default_rng(21)
    values = (rng.standard_normal((700, 40)) * rng.lognormal(0, 2, size=40)).astype(np.float32)
    values[:, 3] = 1.25  # a constant column
    codes, affine, layout = pq.quantize_coefficients(values, normalization, fraction)
    o_codes, o_affine, o_layout = oq.quantize(values, normalization, fraction)
    np.testing.assert_array_equal(codes, o_codes)
    np.testing.assert_array_equal(affine, o_affine)
    assert layout["protected_count"] == o_layout["protected_count"]
    assert list(layout["affine_shape"]) == list(o_layout["affine_shape"])
    np.testing.assert_array_equal(pq.dequantize_coefficients(codes, affine, layout),
                                  oq.dequantize(o_codes, o_affine, o_layout))


def test_covering_affine_and_layout_match_oracle():
    rng = np.random.default_rng(22)
    lo = rng.uniform(-8, 0, size=500).astype(np.float32)
    hi = (lo + rng.uniform(0, 9, size=500)).astype(np.float32)
    np.testing.assert_array_equal(pq.covering_affine(lo, hi), oq.covering_affine(lo, hi))
    for shape in ((3, 30, 52, 192), (3, 30, 52, 128), (1, 4, 4, 100), (16, 60, 104, 512), (2, 3000, 3000, 50)):
        for fmt in ("yuv444p", "yuv420p"):
            ours, theirs = pq.video_layout(*shape, fmt), oq.video_layout(*shape, fmt)
            for key in theirs:
                assert list(np.atleast_1d(ours[key])) == list(np.atleast_1d(theirs[key])), (shape, fmt, key)


def test_invalid_affine_is_an_integrity_error():
    values = np.arange(24, dtype=np.float32).reshape(6, 4)
    codes, affine, layout = pq.quantize_coefficients(values, "per_channel")
    for bad in (-1.0, float("nan"), float("inf")):
        corrupt = affine.copy()
        corrupt[0, 0] = bad
        with pytest.raises(IntegrityError):
            pq.dequantize_coefficients(codes, corrupt, layout)
    with pytest.raises(ConfigurationError):
        pq.quantize_coefficients(values, "leading_columns", float("nan"))
    huge = np.array([[-np.finfo(np.float32).max], [np.finfo(np.float32).max]])
    with pytest.raises(ConfigurationError):
        pq.quantize_coefficients(huge, "global")


# ---------------------------------------------------------------------------
# RoPE tables
# ---------------------------------------------------------------------------


def test_rope_table_from_wan_freqs_matches_oracle():
    freqs = orc.wan_freqs(128, 30)
    table = rk.RopeTable.from_complex(torch.from_numpy(freqs))
    assert table.sections == (22, 21, 21)
    np.testing.assert_array_equal(table.cos.numpy(), freqs.real)
    np.testing.assert_array_equal(table.sin.numpy(), freqs.imag)
    positions = rk.RopePositions(table, (6, 2, 1))
    cos, sin = rk.rope_cos_sin(positions, (3, 5, 7))
    o_cos, o_sin = orc.rope_cos_sin(freqs.real, freqs.imag, (22, 21, 21), (6, 2, 1), (3, 5, 7))
    np.testing.assert_array_equal(cos.numpy(), o_cos)
    np.testing.assert_array_equal(sin.numpy(), o_sin)


def test_kernel_pairs_interleave_the_fp32_tables():
    table = rk.RopeTable.from_complex(torch.from_numpy(orc.wan_freqs(64, 12)))
    pairs = table.kernel_pairs("cpu")
    cos, sin = table.kernel_tables("cpu")
    assert pairs.shape == (12, 32, 2) and pairs.dtype == torch.float32 and pairs.is_contiguous()
    assert torch.equal(pairs[..., 0], cos) and torch.equal(pairs[..., 1], sin)


# ---------------------------------------------------------------------------
# CPU reference backend == oracle
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("source,rope,layout", [("uint8", "separable", "BTHD"), ("pictures", "dense", "THD"),
                                                ("float", "none", "BHTD")])
def test_reference_backend_matches_oracle(source, rope, layout):
    rng = np.random.default_rng(23)
    case = make_case(rng, grid=(2, 4, 6), heads=2, head_dim=16, rank=9, source=source, rope=rope, layout=layout,
                     out_dtype="float32")
    handle = rk.reconstruct([case.job])  # CPU tensors: backend "auto" resolves to the FP64 reference
    assert handle.stats["backend"] == "reference"
    exact = orc.reconstruct(case.coefficients, case.basis, case.heads, case.rope)
    np.testing.assert_allclose(written(case), orc.cast(exact, "float32"), rtol=0, atol=1e-6)


# ---------------------------------------------------------------------------
# Validation, backends, precisions
# ---------------------------------------------------------------------------


def test_validation_errors():
    rng = np.random.default_rng(24)
    case = make_case(rng, grid=(1, 4, 8), heads=2, head_dim=16, rank=8)
    job = case.job
    with pytest.raises(ConfigurationError):
        rk.ReconstructionJob(job.source, job.destination, job.grid, job.basis, 9, None)  # rank > basis rows
    with pytest.raises(ConfigurationError):
        rk.ReconstructionJob(job.source, job.destination, (1, 4, 9), job.basis, 8, None)  # tokens != source rows
    with pytest.raises(ConfigurationError):
        rk.reconstruct([job, job])  # overlapping destination slots
    with pytest.raises(ConfigurationError):
        rk.reconstruct("not jobs")
    with pytest.raises(ConfigurationError):
        rk.reconstruct([job], backend="cuda-graphs")
    with pytest.raises(ConfigurationError):
        rk.reconstruct([job], precision="fp8")


def test_no_silent_fallback_on_host_tensors():
    rng = np.random.default_rng(25)
    case = make_case(rng, grid=(1, 4, 8), heads=2, head_dim=16, rank=8)
    for backend in ("fused", "two_pass"):
        with pytest.raises(UnsupportedError):
            rk.reconstruct([case.job], backend=backend)
    for backend in ("staged", "interpret"):
        with pytest.raises(UnsupportedError):
            rk.reconstruct([case.job], backend=backend)
    assert rk.PRECISIONS == ("fp32", "tf32", "tf32x3", "fp16", "fp16x2", "bf16")
    assert rk.recommended_precision("cpu") == "fp16x2"


# ---------------------------------------------------------------------------
# Planner helpers
# ---------------------------------------------------------------------------


class _Job:
    def __init__(self, tokens):
        self.tokens = tokens


def test_tile_table_covers_every_token_once():
    jobs = [_Job(300), _Job(128), _Job(1), _Job(257)]
    tiles = rk._tiles([0, 2, 3], jobs)
    assert tiles.dtype == np.int32 and tiles.shape == (3 + 1 + 3, 2)
    assert tiles[:, 0].tolist() == [0, 0, 0, 2, 3, 3, 3]
    assert tiles[:, 1].tolist() == [0, 128, 256, 0, 0, 128, 256]


@pytest.mark.parametrize("grid", [1, 7, 512, 5000])
def test_balanced_bounds_partition_the_units(grid):
    rng = np.random.default_rng(26)
    costs = rng.choice([4.0, 8.0, 12.0, 24.0], size=300)
    blocks = 48
    bounds = rk._balanced_bounds(costs, blocks, grid)
    units = len(costs) * blocks
    assert bounds.dtype == np.int32 and bounds.shape == (grid + 1,)
    assert bounds[0] == 0 and bounds[-1] == units and np.all(np.diff(bounds) >= 0)
    unit_cost = np.repeat(costs, blocks)
    per_range = np.add.reduceat(np.append(unit_cost, 0), bounds[:-1])[np.diff(bounds) > 0]
    if grid <= units:
        # Every range is within one unit's cost of the ideal share.
        assert per_range.max() <= unit_cost.sum() / grid + unit_cost.max() + 1e-9


def test_fast_eligibility_rules():
    rng = np.random.default_rng(27)
    case = make_case(rng, grid=(1, 4, 8), heads=2, head_dim=64, rank=32, rope="none")
    row = {"flags": _lib.JF_SRC_VEC | _lib.JF_DST_VEC, "dst_bytes": 4096, "bound_index": -1}
    assert rk._fast_flags(row, case.job, "fp16x2") == _lib.GF_FAST
    assert rk._fast_flags(row, case.job, "fp32") == 0
    assert rk._fast_flags(dict(row, flags=_lib.JF_DST_VEC), case.job, "fp16x2") == 0  # unaligned code rows
    assert rk._fast_flags(dict(row, dst_bytes=2 ** 31), case.job, "bf16") == 0  # slot beyond 32-bit offsets
    roped = make_case(rng, grid=(1, 4, 8), heads=2, head_dim=64, rank=32).job
    assert rk._fast_flags(row, roped, "fp16") == 0  # no pairs table
    assert rk._fast_flags(dict(row, pairs_ptr=256, pairs_bytes=1024), roped, "fp16") == _lib.GF_FAST | _lib.GF_ROPE
    odd = make_case(rng, grid=(1, 4, 8), heads=2, head_dim=48, rank=32, rope="none").job
    assert rk._fast_flags(row, odd, "fp16x2") == 0  # head_dim % 32 != 0


def test_captured_calls_need_reserved_staging(monkeypatch):
    monkeypatch.setattr(rp, "_STAGING", {})
    with pytest.raises(ConfigurationError, match="reserve_capture_staging"):
        rp._capture_staging(4096)
    slab = torch.zeros(1 << 12, dtype=torch.uint8)
    monkeypatch.setattr(rp, "_STAGING", {"slab": [slab, 0]})
    first = rp._capture_staging(1000)
    second = rp._capture_staging(1000)
    assert first.numel() == second.numel() == 1000
    assert second.data_ptr() - slab.data_ptr() == 1024  # regions start 256-byte aligned
    with pytest.raises(ConfigurationError):
        rp._capture_staging(3000)  # 2048 + 3000 exceeds the 4096-byte slab


def test_replaced_staging_slab_stays_alive(monkeypatch):
    """A slab that handed out regions to captured calls is kept when a larger one replaces it
    (captured graphs copy from those regions on every replay)."""
    monkeypatch.setattr(rp, "_STAGING", {})
    monkeypatch.setattr(rp, "_RETIRED_SLABS", [])
    monkeypatch.setattr(rp, "_pinned_bytes", lambda n: torch.zeros(n, dtype=torch.uint8))
    monkeypatch.setattr(rp.torch.cuda, "is_available", lambda: False)
    rp.reserve_capture_staging(1 << 20)
    first_slab = rp._STAGING["slab"][0]
    region = rp._capture_staging(1 << 19)
    rp.reserve_capture_staging(1 << 20)  # does not fit the rest of the first slab: a new slab
    assert rp._STAGING["slab"][0] is not first_slab
    assert any(kept is first_slab for kept in rp._RETIRED_SLABS)
    assert region.data_ptr() == first_slab.data_ptr()
    # An unused slab is simply replaced (nothing captured reads it).
    unused = rp._STAGING["slab"][0]
    rp.reserve_capture_staging(1 << 21)
    assert not any(kept is unused for kept in rp._RETIRED_SLABS)
