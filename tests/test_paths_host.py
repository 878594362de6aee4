"""CPU pins of host-side pieces the GPU tests build on.

* ``RopeTable.from_axes`` / ``RopeTable.longcat`` against closed-form tables
  (reelcache/restore_kernels.py:467-576);
* ``fast_condition_bound`` as the reference's tests state it: an upper bound of the exact
  FP64 condition bound, below 1.5 for rounded orthonormal bases, and the exact bound for a
  basis that is not near orthonormal (tests/test_gpu_fitting_batched.py:64-77);
* the oracle's ``coefficient_bound`` (reelcache/restore_kernels.py:1782-1785) against a
  brute-force maximum over all 256 codes, and the product's per-job bound against it.
"""

import math

import numpy as np
import pytest
import torch

from oracle import restore as orc
from reelcache_amd import restore_kernels as rk
from reelcache_amd.errors import ConfigurationError
from reelcache_amd.factorization import basis_condition_bound, fast_condition_bound
from reelcache_amd.restore_plan import job_desc
from restore_cases import make_case, orthonormal_basis


# ---------------------------------------------------------------------------
# RoPE tables
# ---------------------------------------------------------------------------


def _axis(rows, pairs, rng, dtype=torch.complex128):
    angles = rng.uniform(-math.pi, math.pi, size=(rows, pairs))
    return torch.from_numpy(np.cos(angles) + 1j * np.sin(angles)).to(dtype)


def test_from_axes_places_each_axis_in_its_columns():
    rng = np.random.default_rng(5)
    temporal, height, width = _axis(7, 6, rng), _axis(4, 5, rng), _axis(9, 5, rng)
    table = rk.RopeTable.from_axes(temporal, height, width)
    assert table.sections == (6, 5, 5) and table.section_rows == (7, 4, 9)
    assert table.cos.dtype == torch.float64 and tuple(table.cos.shape) == (9, 16)
    column = 0
    for axis in (temporal, height, width):
        rows, pairs = axis.shape
        block = slice(column, column + pairs)
        assert torch.equal(table.cos[:rows, block], axis.real)
        assert torch.equal(table.sin[:rows, block], axis.imag)
        # Rows an axis does not have stay NaN, so an out-of-range row cannot pass silently.
        assert bool(torch.isnan(table.cos[rows:, block]).all()) and bool(torch.isnan(table.sin[rows:, block]).all())
        column += pairs
    # complex64 axes give a float32 table.
    assert rk.RopeTable.from_axes(*(a.to(torch.complex64) for a in (temporal, height, width))).cos.dtype == torch.float32


def test_from_axes_rows_follow_the_oracle_selection():
    """Per-token (cos, sin) of a from_axes table equal the axes' values at (t, y, x) + (t_row, h_row, w_row)."""
    rng = np.random.default_rng(6)
    temporal, height, width = _axis(6, 4, rng), _axis(5, 2, rng), _axis(7, 2, rng)
    table = rk.RopeTable.from_axes(temporal, height, width)
    grid, rows = (2, 3, 4), (3, 1, 2)
    cos, sin = rk.rope_cos_sin(rk.RopePositions(table, rows), grid)
    frames, ys, xs = orc.token_coordinates(grid)
    expected = np.concatenate([temporal.numpy()[frames + rows[0]], height.numpy()[ys + rows[1]],
                               width.numpy()[xs + rows[2]]], axis=1)
    np.testing.assert_array_equal(cos.numpy(), expected.real)
    np.testing.assert_array_equal(sin.numpy(), expected.imag)
    # A position past an axis' rows is refused (the t axis has 6 rows: 3 + 2 frames fits, 5 + 2 does not).
    with pytest.raises(ConfigurationError):
        rk.ReconstructionJob(rk.DenseSource(torch.zeros(24, 16)), rk.NativeView(torch.zeros(1, 24, 2, 8)), grid,
                             rope=rk.RopePositions(table, (5, 0, 0)))


def test_from_axes_validation():
    rng = np.random.default_rng(7)
    good = _axis(3, 2, rng)
    with pytest.raises(ConfigurationError):
        rk.RopeTable.from_axes(good.real, good, good)
    with pytest.raises(ConfigurationError):
        rk.RopeTable.from_axes(good[0], good, good)


@pytest.mark.parametrize("head_dim,grid", [(128, (3, 30, 52)), (32, (3, 4, 5)), (48, (16, 6, 2))])
def test_longcat_tables_match_the_closed_form(head_dim, grid):
    """LongCat rope_3d: axis dims (d - 4(d//6), 2(d//6), 2(d//6)); angle p * base^(-2j/dim) in float32,
    cos / sin of the float32 angle.  Checked against float64 evaluation of the same formula: angles
    within one float32 rounding of each step, cos / sin within 2 ulps of float64 cos / sin of the
    float32 angle."""
    table = rk.RopeTable.longcat(head_dim, *grid)
    sixth = head_dim // 6
    dims = (head_dim - 4 * sixth, 2 * sixth, 2 * sixth)
    assert table.sections == tuple(d // 2 for d in dims)
    assert table.section_rows == grid
    assert table.cos.dtype == torch.float32 and tuple(table.cos.shape) == (max(grid), head_dim // 2)
    column = 0
    for dim, count in zip(dims, grid):
        pairs = dim // 2
        exponent = np.arange(0, dim, 2, dtype=np.float64)[:pairs] / dim
        inverse64 = 10000.0 ** -exponent
        angles64 = np.arange(count, dtype=np.float64)[:, None] * inverse64[None, :]
        cos = table.cos[:count, column:column + pairs].double().numpy()
        sin = table.sin[:count, column:column + pairs].double().numpy()
        # Recover the float32 angles the table used from the exact float64 formula: each of the
        # three float32 roundings (exponent ratio, power / reciprocal, product) perturbs the angle
        # by a few units of 2**-24 relative.
        slack = 8 * 2.0 ** -24 * np.abs(angles64) + 1e-30
        assert np.all(np.abs(np.cos(angles64) - cos) <= slack + 2 * 2.0 ** -24)
        assert np.all(np.abs(np.sin(angles64) - sin) <= slack + 2 * 2.0 ** -24)
        # Position 0 is the identity rotation exactly.
        assert np.all(cos[0] == 1.0) and np.all(sin[0] == 0.0)
        assert bool(torch.isnan(table.cos[count:, column:column + pairs]).all())
        column += pairs
    with pytest.raises(ConfigurationError):
        rk.RopeTable.longcat(36 + 2, *grid)


# ---------------------------------------------------------------------------
# fast_condition_bound (reelcache/factorization.py:295-314)
# ---------------------------------------------------------------------------


def test_fast_condition_bound_upper_bounds_exact_for_rounded_orthonormal_bases():
    generator = torch.Generator().manual_seed(11)
    for rank, channels in ((4, 16), (32, 96), (64, 128), (128, 1536)):
        q = torch.linalg.qr(torch.randn(channels, rank, generator=generator, dtype=torch.float64))[0]
        basis = q.T.contiguous().half()
        exact, fast = basis_condition_bound(basis), fast_condition_bound(basis)
        assert fast >= exact
        assert fast < 1.5


def test_fast_condition_bound_falls_back_to_exact_off_orthonormal():
    basis = torch.tensor([[1.0, 0.0], [0.9, 0.1]], dtype=torch.float16)
    assert fast_condition_bound(basis) == basis_condition_bound(basis)


def test_exact_condition_bound_closed_form():
    """basis_condition_bound of a diagonal basis diag(d) is max(d)^2 / min(d)^2 (the condition
    number of B B^T), and 1 for a coordinate basis."""
    assert basis_condition_bound(torch.eye(5, 9, dtype=torch.float16)) == pytest.approx(1.0, abs=1e-12)
    d = torch.tensor([1.0, 0.5, 2.0, 0.25], dtype=torch.float64)
    basis = torch.zeros(4, 6, dtype=torch.float64)
    basis[range(4), range(4)] = d
    assert basis_condition_bound(basis) == pytest.approx(float((d.max() / d.min()) ** 2), rel=1e-12)


# ---------------------------------------------------------------------------
# The 8-bit coefficient bound (oracle and product)
# ---------------------------------------------------------------------------


def test_coefficient_bound_is_the_maximum_over_all_codes():
    """oracle.coefficient_bound == 1.0001 * max over q in 0..255 of |fl(fl(q s) + o)|: the reference's
    closed form takes the two endpoints q = 0 and q = 255, which is the maximum because q s + o is
    monotone in q and the two float32 roundings are monotone too."""
    rng = np.random.default_rng(31)
    for trial in range(40):
        rank = int(rng.integers(1, 40))
        scale = (rng.lognormal(-4, 3, size=rank) * (rng.random(rank) > 0.1)).astype(np.float32)
        offset = (rng.standard_normal(rank) * rng.lognormal(0, 3, size=rank)).astype(np.float32)
        codes = np.arange(256, dtype=np.uint8)[:, None].repeat(rank, axis=1)
        brute = float(np.abs(orc.dequantize(codes, scale, offset)).max())
        bound = orc.coefficient_bound(scale, offset)
        assert bound == pytest.approx(brute * 1.0001, rel=1e-12)
        assert orc.prescale_exponent(bound) == rk._prescale_exponent(bound)


def test_product_coefficient_bounds_match_the_oracle():
    rng = np.random.default_rng(32)
    ranks = [3, 17, 1, 64]
    scales = [rng.lognormal(-3, 2, size=r).astype(np.float32) for r in ranks]
    offsets = [rng.standard_normal(r).astype(np.float32) * 5 for r in ranks]
    for s, o in zip(scales, offsets):
        assert rk._coefficient_bound(s, o) == orc.coefficient_bound(s, o)


@pytest.mark.parametrize("origin,pad,grid,aligned", [((0, 0), (3, 4), (3, 30, 52), True),
                                                     ((2, 4), (3, 4), (3, 30, 52), True),
                                                     ((2, 3), (3, 5), (3, 30, 52), False),   # odd origin and stride
                                                     ((0, 0), (3, 4), (2, 12, 14), False)])  # cell width 14
def test_picture_word_gather_rule(origin, pad, grid, aligned):
    """A picture matrix takes the 32-bit word gather only when every cell-row start is
    4-byte aligned: plane and row strides and the cell width multiples of 4 (the job rule),
    and every picture view's address a multiple of 4 (checked per call)."""
    case = make_case(np.random.default_rng(3), grid=grid, heads=4, head_dim=32, rank=96, source="pictures",
                     rope="none", out_dtype="bfloat16", device="cpu", picture_origin=origin, picture_pad=pad)
    desc = job_desc(case.job)
    assert (desc.pic_vec_rule and all(p.data_ptr() % 4 == 0 for p in desc.pictures)) == aligned


def _noalloc_placement(group_packs, fragment_bytes):
    """Where rch_restore_noalloc puts a launch group's packs (csrc/restore.hip): pack i's fragments
    at byte sum_{j<i} round_up(ksteps_j * nblocks_j * 64 * fragment, 256) of the fragment region, its
    block exponents at word sum_{j<i} nblocks_j (fragment packs)."""
    places, at, word = [], 0, 0
    for pack in group_packs:
        places.append((at, word))
        at += (int(pack["ksteps"]) * int(pack["nblocks"]) * 64 * fragment_bytes + 255) // 256 * 256
        word += int(pack["nblocks"])
    return places


def test_static_scratch_rows_point_at_their_own_group_packs(monkeypatch):
    """One basis used by two launch groups at different positions (two rank classes): every job's
    pack pointer and exponent word must name where its own group's no-allocation call packs it."""
    from reelcache_amd import restore_plan as rp

    monkeypatch.setattr(rp, "_compute_units", lambda device: 256)
    monkeypatch.setattr(rp, "_occupancy", lambda *args: 2)
    rng = np.random.default_rng(5)
    heads = 2
    basis_x = orthonormal_basis(128, heads * 128, rng)
    basis_y = orthonormal_basis(192, heads * 128, rng)
    # Group 1 (8 rank steps): A on X, B on Y -> packs [X, Y].  Group 2 (4 steps): C on Y -> [Y].
    cases = [make_case(rng, grid=(1, 4, 8), heads=heads, head_dim=128, rank=rank, rope="none", basis=basis)
             for rank, basis in ((128, basis_x), (120, basis_y), (40, basis_y))]
    descs = [job_desc(case.job) for case in cases]
    dynamic = [rp._lib.JF_DST_VEC | rp._lib.JF_SRC_VEC] * len(descs)
    groups = [0, 1, 1]
    config = {**rp.DEFAULT_MERGED, "static_scratch": True}
    layout = rp._Layout(descs, dynamic, groups, "fp16x2", config, "cpu")
    assert len(layout.plans) == 2
    pack_group = {}  # job -> index of its basis pack in the layout's pack table
    for position, member in enumerate(layout.pack_sources):
        for job, group in enumerate(groups):
            if group == groups[member]:
                pack_group[job] = position
    checked = 0
    for plan in layout.plans:
        group_packs = layout.pack_rows[plan["packs"]]
        fields = {name: group_packs[:, rp._PACK_COLUMN[name]] for name in ("ksteps", "nblocks")}
        places = _noalloc_placement([{k: v[i] for k, v in fields.items()} for i in range(len(group_packs))], 16)
        for job in plan["members"]:
            where = plan["packs"].index(pack_group[job])
            assert (layout.rows[job, rp._C_PACK_PTR], layout.rows[job, rp._C_EXP_INDEX]) == places[where]
            checked += 1
    assert checked == 3
    # Job C (group 2) reads basis Y at the start of the array; job B (group 1) after X's fragments.
    assert layout.rows[2, rp._C_PACK_PTR] == 0 and layout.rows[1, rp._C_PACK_PTR] > 0
