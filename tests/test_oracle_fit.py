"""Pins of the fit oracle (``oracle/fit.py``) on the CPU.

Each check is independent of the formula it checks: brute-force Python sums, numpy's SVD,
exact rational arithmetic, closed forms of coordinate bases and hand-counted crossings, chosen
so that a dropped term, a transposed operand, a wrong sign rule or an off-by-one crossing fails.
"""

import math
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import fit as of


def test_gram_matches_brute_force_sums():
    rng = np.random.default_rng(1)
    x = rng.integers(-7, 8, size=(5, 4)).astype(np.float32)
    g = of.gram(x)
    for i in range(4):
        for j in range(4):
            assert g[i, j] == sum(float(x[r, i]) * float(x[r, j]) for r in range(5))


def test_gram_bases_span_the_svd_subspace():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((60, 12)) @ np.diag(np.linspace(3, 0.1, 12))
    values, rows = of.gram_bases(x, 4)
    _, sigma, vt = np.linalg.svd(x, full_matrices=False)
    np.testing.assert_allclose(values, sigma ** 2, rtol=1e-12)
    assert np.all(np.diff(values) <= 0)
    projector = rows.T @ rows
    np.testing.assert_allclose(projector, vt[:4].T @ vt[:4], atol=1e-10)
    np.testing.assert_allclose(rows @ rows.T, np.eye(4), atol=1e-12)


def test_canonical_signs_rule():
    basis = np.array([[1.0, -1.0, 0.5], [-1.0, 1.0, 0.0], [0.1, -0.3, 0.3], [0.0, 0.0, 0.0]])
    signed = of.canonical_signs(basis)
    # First entry of largest magnitude becomes positive; ties go to the first index.
    np.testing.assert_array_equal(signed[0], [1.0, -1.0, 0.5])
    np.testing.assert_array_equal(signed[1], [1.0, -1.0, 0.0])
    np.testing.assert_array_equal(signed[2], [-0.1, 0.3, -0.3])
    np.testing.assert_array_equal(signed[3], [0.0, 0.0, 0.0])
    np.testing.assert_array_equal(of.canonical_signs(-basis[:3]), signed[:3])
    np.testing.assert_array_equal(of.canonical_signs(signed), signed)


def test_projection_is_the_rounded_exact_dot_product():
    rng = np.random.default_rng(3)
    x = of.to_bfloat16_values(rng.standard_normal((3, 8)).astype(np.float32))
    q = rng.standard_normal((2, 8)).astype(np.float16)
    p = of.project(x, q)
    for t in range(3):
        for k in range(2):
            exact = sum(Fraction(float(x[t, c])) * Fraction(float(q[k, c])) for c in range(8))
            # 8 products of 8-bit x 11-bit significands with nearby exponents are exact in float64,
            # so float32(float64) is the single rounding of the exact value.
            assert Fraction(float(exact)) == exact
            assert p[t, k] == np.float32(float(exact))


def test_energies_of_a_coordinate_basis():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((40, 16)).astype(np.float32)
    q = np.eye(16, dtype=np.float16)[:5]
    p = of.project(x, q)
    np.testing.assert_array_equal(p, x[:, :5])
    scale, source, error = of.energies(x, q, p)
    assert scale == float(np.abs(x).max())
    assert source == pytest.approx(float((x.astype(np.float64) ** 2).sum()) / scale ** 2, rel=1e-14)
    assert error == pytest.approx(float((x[:, 5:].astype(np.float64) ** 2).sum()) / scale ** 2, rel=1e-14)
    assert of.energies(np.zeros((3, 4), np.float32)) == (0.0, 0.0, 0.0)


def test_crossing_counts_by_hand():
    energies = [4.0, 3.0, 2.0, 1.0]
    assert of.crossing(energies, 10.0, 0.7) == 2
    assert of.crossing(energies, 10.0, 0.71) == 3
    assert of.crossing(energies, 10.0, 1.0) == 4
    assert of.crossing(energies, 20.0, 0.9) is None
    assert of.crossing(energies, 0.0, 0.9) == 0


def test_bucket_grid():
    assert of.bucket(10, 32, 1536) == 32
    assert of.bucket(32, 32, 1536) == 32
    assert of.bucket(33, 32, 1536) == 64
    assert of.bucket(0.2, 32, 1536) == 32
    assert of.bucket(math.inf, 32, 1536) == 1536
    assert of.bucket(1530, 32, 1536) == 1536
    assert of.bucket(5, 32, 20) == 20


def test_decaying_spectrum_crossings():
    # sigma_i = i ** -1.2 over 1536 directions: K at 98 % needs 10, V at 95 % needs 5 (counted).
    assert of.closed_form_crossing(1536, 0.98) == 10
    assert of.closed_form_crossing(1536, 0.95) == 5
    rng = np.random.default_rng(5)
    x = of.decaying_spectrum(rng, 400, 64, noise=0.0, dtype=np.float64)
    values, _ = of.gram_bases(x, 1)
    assert of.crossing(values, values.sum(), 0.98) == of.closed_form_crossing(64, 0.98)
    assert of.crossing(values, values.sum(), 0.95) == of.closed_form_crossing(64, 0.95)


def test_bfloat16_rounding_matches_torch():
    rng = np.random.default_rng(6)
    x = (rng.standard_normal(4096) * np.exp(rng.uniform(-30, 30, 4096))).astype(np.float32)
    x[:4] = [1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -(1.0 + 2 ** -8), 0.0]  # ties to even
    expected = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(of.to_bfloat16_values(x), expected)


def test_span_energy_closed_forms():
    """Coordinate rows e_i: the span energy is the energy of those columns of X (P = X[:, idx]).
    Any invertible mix A of the same rows spans the same subspace, so the value does not change
    (a dropped Gram inverse fails this); an orthonormal complement adds the rest (total 1)."""
    rng = np.random.default_rng(41)
    x = rng.integers(-8, 9, size=(50, 8)).astype(np.float64)  # small integers: every P below is exact in fp32
    total = float(np.square(x).sum())
    idx = [1, 4, 6]
    coordinate = np.eye(8)[idx].astype(np.float16)
    p = of.project(x, coordinate)
    expected = float(np.square(x[:, idx]).sum()) / total
    assert abs(of.span_energy(p, coordinate, total) - expected) <= 1e-12
    mix = np.array([[2.0, 0.0, 0.0], [0.5, 1.0, 0.0], [-1.0, 0.25, 4.0]])  # exact in fp16 products
    mixed = (mix @ coordinate.astype(np.float64)).astype(np.float16)
    assert abs(of.span_energy(of.project(x, mixed), mixed, total) - expected) <= 1e-12
    everything = np.eye(8).astype(np.float16)
    assert abs(of.span_energy(of.project(x, everything), everything, total) - 1.0) <= 1e-12
    assert of.span_energy(np.zeros((50, 3)), coordinate, 0.0) == 1.0
