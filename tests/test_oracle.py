"""Pins of the oracle (``oracle/``) on the CPU.

The oracle restates the reference's arithmetic; these tests check it against what fixes
that arithmetic independently of the restatement:
  * the reference's own known answers (tests/test_codecs.py:383-436, NormalizationTests), held
    as data in tests/golden/quantizer_known_answers.json;
  * library routines that implement the same rounding (torch casts and float32 arithmetic);
  * closed forms and brute force (complex multiplication for RoPE, nearest code by search,
    explicit loops for the product and the picture cells);
  * invariants (covering of the affine range, round trips, the error bound holding for
    emulated precision modes).
"""

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import quantize as oq
from oracle import restore as orc


# ---------------------------------------------------------------------------
# Quantizer: reference known answers (tests/test_codecs.py:383-436)
# ---------------------------------------------------------------------------


GOLDEN = json.loads((Path(__file__).resolve().parent / "golden" / "quantizer_known_answers.json").read_text())


def test_leading_columns_known_answers():
    case = GOLDEN["leading_columns"]
    expect = case["expect"]
    coefficients = np.array(case["coefficients"], dtype=np.float32)
    codes, affine, layout = oq.quantize(coefficients, "leading_columns", case["fraction"])
    assert layout["protected_count"] == expect["protected_count"]
    assert layout["affine_shape"] == expect["affine_shape"]
    assert float(affine[1, 0]) == expect["offset_first_protected"]
    assert abs(float(affine[0, 0]) - expect["scale_first_protected"]) < expect["scale_tolerance"]
    reconstructed = oq.dequantize(codes, affine, layout)
    assert np.abs(reconstructed[:, 2:] - coefficients[:, 2:]).max() < expect["max_abs_error_unprotected"]
    _, global_affine, _ = oq.quantize(coefficients, "global")
    assert global_affine[0, 0] > affine[0, 0] * expect["global_scale_ratio_min"]


def test_protection_endpoints():
    case = GOLDEN["protection_endpoints"]
    coefficients = np.arange(int(np.prod(case["coefficients_arange"])), dtype=np.float32).reshape(case["coefficients_arange"])
    q_all, a_all, l_all = oq.quantize(coefficients, "leading_columns", 1)
    q_pc, a_pc, l_pc = oq.quantize(coefficients, case["expect"]["fraction_1_equals"])
    np.testing.assert_array_equal(a_all[:, 0], case["expect"]["fraction_1_first_affine"])
    np.testing.assert_array_equal(q_all, q_pc)
    np.testing.assert_array_equal(a_all[:, 1:], a_pc)
    q_none, a_none, _ = oq.quantize(coefficients, "leading_columns", 0)
    q_global, a_global, _ = oq.quantize(coefficients, case["expect"]["fraction_0_equals"])
    np.testing.assert_array_equal(q_none, q_global)
    np.testing.assert_array_equal(a_none, a_global)
    np.testing.assert_array_equal(oq.dequantize(q_all, a_all, l_all), oq.dequantize(q_pc, a_pc, l_pc))


def test_constant_channels():
    case = GOLDEN["constant_channels"]
    coefficients = np.tile(np.array(case["row"], dtype=np.float32), (case["rows"], 1))
    for normalization, fraction in case["cases"]:
        codes, affine, layout = oq.quantize(coefficients, normalization, fraction)
        assert np.all(affine[0] == 0)
        np.testing.assert_array_equal(oq.dequantize(np.full_like(codes, 255), affine, layout), coefficients)
    uniform = np.full(case["uniform_shape"], case["uniform_value"], dtype=np.float32)
    codes, affine, layout = oq.quantize(uniform, "global")
    assert affine[0, 0] == 0
    np.testing.assert_array_equal(oq.dequantize(codes + case["uniform_code_shift"], affine, layout), uniform)


# ---------------------------------------------------------------------------
# Quantizer: invariants and brute force
# ---------------------------------------------------------------------------


def test_covering_affine_covers_and_is_tight():
    rng = np.random.default_rng(5)
    lo = rng.uniform(-50, 50, size=4000).astype(np.float32)
    hi = (lo.astype(np.float64) + rng.lognormal(0, 3, size=4000)).astype(np.float32)
    scale, offset = oq.covering_affine(lo, hi)
    top = (np.float32(255) * scale).astype(np.float32) + offset  # float32 arithmetic, as the decoder
    assert np.all(top.astype(np.float64) >= hi.astype(np.float64))
    assert np.all(offset == lo)
    span = hi.astype(np.float64) - lo.astype(np.float64)
    assert np.all(scale.astype(np.float64) * 255 >= span)
    # At most two float32 steps above float32(span / 255).
    start = (span / 255).astype(np.float32)
    steps = (scale.view(np.int32) - start.view(np.int32))
    assert steps.min() >= 0 and steps.max() <= 2


def test_codes_are_the_nearest_level():
    """rint((v - o) / s) clipped is the code whose level o + q s is nearest to v (brute force
    over all 256 levels in float64; exact ties excluded)."""
    rng = np.random.default_rng(9)
    values = rng.normal(0, 3, size=(300, 6)).astype(np.float32)
    codes, affine, layout = oq.quantize(values, "per_channel")
    scale, offset = oq.expanded_affine(affine, layout, values.shape[1])
    levels = offset.astype(np.float64)[None, :] + np.arange(256)[:, None] * scale.astype(np.float64)[None, :]
    distance = np.abs(values.astype(np.float64)[:, None, :] - levels[None])
    best = distance.argmin(axis=1)
    ordered = np.sort(distance, axis=1)
    tie = np.isclose(ordered[:, 0], ordered[:, 1], rtol=0, atol=1e-12)
    np.testing.assert_array_equal(codes[~tie], best[~tie])


def test_quantize_round_trip_within_half_a_step():
    rng = np.random.default_rng(11)
    values = (rng.standard_normal((500, 8)) * rng.uniform(0.01, 100, size=8)).astype(np.float32)
    codes, affine, layout = oq.quantize(values, "per_channel")
    restored = oq.dequantize(codes, affine, layout)
    scale = affine[0].astype(np.float64)
    assert np.all(np.abs(restored - values) <= scale / 2 * (1 + 1e-5) + 1e-6 * np.abs(values))


def test_video_layout_known_geometry():
    # CausVid chunk (3 x 30 x 52), r = 192: 8 x 8 cells of 3 planes, one segment.
    layout = oq.video_layout(3, 30, 52, 192, "yuv444p")
    assert layout["grid"] == [8, 8] and layout["channels_per_segment"] == 192 and layout["segments"] == 1
    assert (layout["image_width"], layout["image_height"]) == (416, 240)
    # Rank beyond one segment; small frames are padded to 16 pixels.
    layout = oq.video_layout(1, 4, 4, 100, "yuv420p")
    assert layout["planes"] == 1 and layout["grid"] == [10, 10] and layout["segments"] == 1
    assert (layout["image_width"], layout["image_height"]) == (40, 40)
    layout = oq.video_layout(2, 3000, 3000, 50, "yuv444p")
    assert layout["grid"] == [2, 2] and layout["channels_per_segment"] == 12 and layout["segments"] == 5


# ---------------------------------------------------------------------------
# Number formats
# ---------------------------------------------------------------------------


def test_dequantize_matches_torch_float32_arithmetic():
    rng = np.random.default_rng(3)
    codes = rng.integers(0, 256, size=(64, 33), dtype=np.uint8)
    scale = rng.uniform(1e-3, 0.1, size=33).astype(np.float32)
    offset = rng.uniform(-5, 5, size=33).astype(np.float32)
    expected = torch.from_numpy(codes).float() * torch.from_numpy(scale)
    expected = expected + torch.from_numpy(offset)
    np.testing.assert_array_equal(orc.dequantize(codes, scale, offset), expected.numpy())


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(4)
    values = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(1e3),
        np.array([0.0, -0.0, np.inf, -np.inf, 1e-40, -3e-39, 3.4e38, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8],
                 dtype=np.float32),
        (np.arange(1 << 16, dtype=np.uint32) << 16 | 0x8000).view(np.float32)[:4000],  # exact ties
    ])
    values = values[np.isfinite(values) | np.isinf(values)]
    ours = orc.f32_to_bf16_bits(values)
    theirs = torch.from_numpy(values).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    finite = ~np.isnan(values)
    np.testing.assert_array_equal(ours[finite], theirs[finite])


def test_cast_matches_torch_double_to_half_formats():
    rng = np.random.default_rng(6)
    values = rng.standard_normal(5000) * 100
    for name, dtype in (("bfloat16", torch.bfloat16), ("float16", torch.float16), ("float32", torch.float32)):
        expected = torch.from_numpy(values).to(torch.float32).to(dtype).double().numpy()
        np.testing.assert_array_equal(orc.cast(values, name), expected)


def test_prescale_exponent_agrees_with_frexp_rule():
    from reelcache_amd.restore_kernels import _prescale_exponent

    samples = [0.0, 1.0, 2.0 ** 14, 2.0 ** 14 * (1 + 2 ** -23), 2.0 ** 13 * (1 - 2 ** -24), 3.0e-30, 7.5e20,
               np.float32(255) * np.float32(0.1)]
    rng = np.random.default_rng(8)
    samples += list(np.exp(rng.uniform(-80, 80, size=2000)))
    for value in samples:
        exponent = orc.prescale_exponent(value)
        assert exponent == _prescale_exponent(value)
        bound = float(np.float32(value))
        if bound > 0 and -100 < exponent < 100:
            scaled = bound * 2.0 ** exponent
            assert 2.0 ** 13 < scaled <= 2.0 ** 14


# ---------------------------------------------------------------------------
# RoPE
# ---------------------------------------------------------------------------


def test_wan_sections_and_table():
    assert orc.wan_sections(64) == (22, 21, 21)  # 44 / 42 / 42 dims of head_dim 128
    assert orc.wan_sections(16) == (6, 5, 5)
    freqs = orc.wan_freqs(128, 21)
    assert freqs.shape == (21, 64)
    # Row n, pair j of the t part: exp(i n theta**(-2j / 44)); h / w parts restart at j = 0.
    for n, j, dim, column in ((5, 3, 44, 3), (20, 0, 42, 22), (7, 20, 42, 63)):
        local = j if column < 22 else column - (22 if column < 43 else 43)
        angle = n * 10000.0 ** (-2.0 * local / dim)
        assert abs(freqs[n, column] - complex(math.cos(angle), math.sin(angle))) < 1e-15


def test_separable_rows_select_by_section():
    cos = np.arange(40 * 8, dtype=np.float64).reshape(40, 8)
    sin = -cos
    sections, rows, grid = (4, 2, 2), (6, 1, 3), (3, 4, 5)
    c, s = orc.rope_cos_sin(cos, sin, sections, rows, grid)
    token = 2 * 20 + 3 * 5 + 4  # frame 2, row 3, column 4
    expected = [cos[6 + 2, j] for j in range(4)] + [cos[1 + 3, j] for j in (4, 5)] + [cos[3 + 4, j] for j in (6, 7)]
    np.testing.assert_array_equal(c[token], expected)
    np.testing.assert_array_equal(s[token], -np.asarray(expected))
    dense_c, _ = orc.rope_cos_sin(cos, sin, None, 5, grid)
    np.testing.assert_array_equal(dense_c, cos[5:5 + 60])


def test_rotation_is_complex_multiplication():
    rng = np.random.default_rng(12)
    values = rng.standard_normal((10, 3, 16))
    angles = rng.uniform(0, 2 * np.pi, size=(10, 8))
    rotated = orc.apply_rope(values, np.cos(angles), np.sin(angles))
    complex_values = values[..., 0::2] + 1j * values[..., 1::2]
    expected = complex_values * np.exp(1j * angles)[:, None, :]
    np.testing.assert_allclose(rotated[..., 0::2], expected.real, rtol=0, atol=1e-12)
    np.testing.assert_allclose(rotated[..., 1::2], expected.imag, rtol=0, atol=1e-12)


# ---------------------------------------------------------------------------
# Product, error bound, pictures
# ---------------------------------------------------------------------------


def test_reconstruct_matches_explicit_loops():
    """The reference test's independent form (tests/test_restore_kernels.py:305-314): dequantize,
    project, rotate with complex math; here as explicit loops on a tiny case."""
    rng = np.random.default_rng(13)
    tokens, rank, heads, head_dim = 5, 3, 2, 4
    p = rng.standard_normal((tokens, rank))
    q = rng.standard_normal((rank, heads * head_dim))
    angles = rng.uniform(0, 6, size=(tokens, head_dim // 2))
    out = orc.reconstruct(p, q, heads, (np.cos(angles), np.sin(angles)))
    for n in range(tokens):
        for head in range(heads):
            for pair in range(head_dim // 2):
                c = head * head_dim + 2 * pair
                e = sum(p[n, k] * q[k, c] for k in range(rank))
                o = sum(p[n, k] * q[k, c + 1] for k in range(rank))
                z = complex(e, o) * complex(math.cos(angles[n, pair]), math.sin(angles[n, pair]))
                assert abs(out[n, c] - z.real) < 1e-12 and abs(out[n, c + 1] - z.imag) < 1e-12


def _emulate(precision, p, q):
    """The product as the precision mode forms it: operands rounded as the mode rounds them
    (prescaled fp16 split for fp16x2), products exact, float32 accumulation in rank order."""
    p32 = p.astype(np.float32)
    if precision == "fp32":
        parts = [p32.astype(np.float64)]
    elif precision in ("fp16", "fp16x2"):
        e = orc.prescale_exponent(np.abs(p32).max())
        scaled = p32.astype(np.float64) * 2.0 ** e
        hi = scaled.astype(np.float16).astype(np.float64)
        parts = [hi * 2.0 ** -e]
        if precision == "fp16x2":
            lo = (scaled - hi).astype(np.float32).astype(np.float16).astype(np.float64)
            parts.append(lo * 2.0 ** -e)
    else:  # bf16 operands
        parts = [orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(p32)).astype(np.float64)]
    acc = np.zeros((p.shape[0], q.shape[1]), dtype=np.float32)
    for part in parts:
        for k in range(p.shape[1]):
            acc = (acc + (part[:, k:k + 1] * q[k:k + 1, :]).astype(np.float32)).astype(np.float32)
    return acc.astype(np.float64)


@pytest.mark.parametrize("precision", ["fp32", "fp16", "fp16x2", "bf16"])
def test_error_bound_holds_for_emulated_modes(precision):
    """gamma(precision, rank) * S bounds the error of the emulated product, so a gamma that is
    too small for the mode's operand rounding fails here."""
    rng = np.random.default_rng(14)
    codes = rng.integers(0, 256, size=(64, 48), dtype=np.uint8)
    scale = rng.uniform(0.005, 0.03, size=48).astype(np.float32)
    offset = rng.uniform(-4, 0, size=48).astype(np.float32)
    p = orc.dequantize(codes, scale, offset).astype(np.float64)
    q = np.linalg.qr(rng.standard_normal((96, 48)))[0].T
    q = orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(q.astype(np.float32))).astype(np.float64)  # bf16 basis
    exact, bound = orc.error_bound(p, q, 2, None, precision, "float32")
    emulated = _emulate(precision, p, q)
    assert np.all(np.abs(emulated - exact) <= bound)
    # The bound is not vacuous: the mode's own error reaches a fair part of it.
    assert np.abs(emulated - exact).max() > 0.01 * (bound - 2.0 ** -24 * np.abs(exact)).max()


def test_error_bound_covers_the_final_cast():
    rng = np.random.default_rng(15)
    p = rng.standard_normal((40, 16))
    q = rng.standard_normal((16, 32))
    for dtype in ("bfloat16", "float16", "float32"):
        exact, bound = orc.error_bound(p, q, 2, None, "fp32", dtype)
        assert np.all(np.abs(orc.cast(exact, dtype) - exact) <= bound)


def test_picture_cells_and_round_trip():
    layout = {"frames": 2, "height": 3, "width": 4, "rank": 11, "grid": [2, 1], "planes": 3,
              "channels_per_segment": 6, "segments": 2}
    cells = list(orc.cells(layout, 6))
    # Cell i: plane i % 3, grid cell divmod(i // 3, columns) (reelcache/_hevc.py:543-548).
    assert cells == [(0, 0, 0, 0), (1, 1, 0, 0), (2, 2, 0, 0), (3, 0, 0, 4), (4, 1, 0, 4), (5, 2, 0, 4)]
    rng = np.random.default_rng(16)
    codes = rng.integers(0, 256, size=(24, 11), dtype=np.uint8)
    canvas, indices = orc.pack_pictures(codes, layout, origin=(2, 3))
    assert canvas.shape == (4, 3, 3 + 2 + 3, 8 + 3 + 5)
    # Column 7 = segment 1, cell 1: plane 1 of pictures 2 (frame 0) and 3 (frame 1) at (2, 3).
    frame0 = codes[:12, 7].reshape(3, 4)
    np.testing.assert_array_equal(canvas[2, 1, 2:5, 3:7], frame0)
    pictures = [[canvas[i, :, 2:, 3:] for i in row] for row in indices]
    np.testing.assert_array_equal(orc.unpack_pictures(pictures, layout), codes)
