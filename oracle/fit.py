"""Oracle (numpy, FP64) for the fit path -- TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Restates, in float64 numpy, what the reference computes on its fitting path:

* :func:`gram` -- ``mm(x.T, x)`` symmetrized (reelcache/gpu_fitting.py:288-289,
  reelcache/rank_method.py:634-638), here in FP64 on the exact source values;
* :func:`gram_bases` -- eigh of the Gram, the top ``rank`` eigenvectors as rows in descending
  energy (reelcache/gpu_fitting.py:290-295);
* :func:`canonical_signs` -- reelcache/factorization.py:437-441;
* :func:`stored_basis` -- canonical signs then FP16 rounding (reelcache/gpu_fitting.py:392-393);
* :func:`project` -- ``P = X.float() @ Q.float().T`` (reelcache/factorization.py:384-392) as the
  fp32 rounding of the FP64 dot product of the exact operands;
* :func:`energies` -- the FP64 source and direct residual energies scaled by max|X|
  (reelcache/factorization.py:398-419, :692-724);
* :func:`span_energy` -- the ideal energy of the stored rows' span, ``||L^-1 P^T||_F^2 / ||X||^2``
  with ``L L^T = Q Q^T`` in FP64 (reelcache/deferred_reads.py:682-714, the value
  ``reelcache/node_packets.py:370-371`` records as a tile's ideal energy);
* :func:`crossing` / :func:`bucket` -- DirectionSet.crossing (reelcache/rank_method.py:411-417)
  and _bucket (:487-490);
* :func:`decaying_spectrum` -- the synthetic fit workload (sigma_i = i ** -1.2 plus noise);
* :func:`closed_form_crossing` -- the crossing of a known spectrum, by direct summation.

How each is pinned (tests/test_oracle_fit.py): brute-force Python sums on tiny inputs, SVD
subspaces, exact rational arithmetic for the projection, closed forms for the energies of
coordinate bases (and, for the span energy, of any invertible mix of coordinate rows: the span
is unchanged), and hand-counted crossings.
"""

from __future__ import annotations

import math

import numpy as np


def as_float(x) -> np.ndarray:
    """Exact float64 values of a float16 / bfloat16-as-float32 / float32 array."""
    return np.asarray(x, dtype=np.float64)


def gram(x) -> np.ndarray:
    """FP64 X^T X of the exact source values (symmetric by construction)."""
    x = as_float(x)
    g = x.T @ x
    return (g + g.T) * 0.5


def gram_bases(x, rank: int) -> tuple[np.ndarray, np.ndarray]:
    """(descending eigenvalues, [rank, n] eigenvector rows) of the FP64 Gram."""
    values, columns = np.linalg.eigh(gram(x))
    return values[::-1].copy(), columns[:, ::-1][:, :rank].T.copy()


def canonical_signs(basis) -> np.ndarray:
    """Each row times the sign of its first entry of largest magnitude (+1 for zero)."""
    basis = np.asarray(basis)
    pivot = basis[np.arange(basis.shape[0]), np.abs(basis).argmax(axis=1)]
    return basis * np.where(pivot < 0, -1.0, 1.0).astype(basis.dtype)[:, None]


def stored_basis(rows) -> np.ndarray:
    """FP16 stored basis of FP32 directions: canonical signs, then one rounding to FP16."""
    return canonical_signs(np.asarray(rows, dtype=np.float32)).astype(np.float16)


def project(x, basis16, rank: int | None = None) -> np.ndarray:
    """fp32 coefficients: the FP64 product of the exact operands rounded once to fp32."""
    q = np.asarray(basis16, dtype=np.float16)
    rank = q.shape[0] if rank is None else rank
    return (as_float(x) @ q[:rank].astype(np.float64).T).astype(np.float32)


def energies(x, basis16=None, coefficients=None, rank: int | None = None) -> tuple[float, float, float]:
    """(scale, sum (X/s)^2, sum ((X - P Q)/s)^2) in FP64; no scaling when s == 0."""
    x = as_float(x)
    scale = float(np.abs(x).max())
    error = x.copy()
    if basis16 is not None:
        q = np.asarray(basis16, dtype=np.float16).astype(np.float64)
        rank = q.shape[0] if rank is None else rank
        error = x - np.asarray(coefficients, dtype=np.float64) @ q[:rank]
    if scale:
        x, error = x / scale, error / scale
    return scale, float(np.square(x).sum()), float(np.square(error).sum())


def span_energy(coefficients, basis16, source_energy: float) -> float:
    """Share of the source energy in the span of the stored rows: ``||L^-1 P^T||_F^2 / E`` where
    ``L`` is the Cholesky factor of the FP64 Gram ``Q Q^T`` of the FP16 rows and ``P`` the fp32
    coefficients (1 for a zero source; ValueError for singular rows)."""
    if source_energy <= 0:
        return 1.0
    q = np.asarray(basis16, dtype=np.float16).astype(np.float64)
    factor = np.linalg.cholesky(q @ q.T)
    solved = np.linalg.solve(factor, as_float(coefficients).T)  # lower-triangular system
    return float(np.square(solved).sum() / source_energy)


def crossing(energies_desc, total: float, fraction: float) -> int | None:
    """Smallest rank whose cumulative energy reaches ``fraction * total`` (0 when total <= 0,
    None when the directions never reach it)."""
    if total <= 0:
        return 0
    cumulative = np.cumsum(np.asarray(energies_desc, dtype=np.float64))
    hits = np.nonzero(cumulative >= fraction * total)[0]
    return None if hits.size == 0 else int(hits[0]) + 1


def bucket(rank: float, width: int, full: int) -> int:
    """``rank`` rounded up to the ``width`` grid, at least one bucket, at most ``full``."""
    if not math.isfinite(rank):
        return full
    return int(min(full, max(width, math.ceil(max(rank, 1.0) / width) * width)))


def decaying_spectrum(rng, rows: int, channels: int, *, exponent: float = 1.2, noise: float = 1e-3,
                      dtype=np.float32) -> np.ndarray:
    """X = U diag(sigma) V^T + eta with orthonormal U [rows, channels], V [channels, channels]
    (QR of Gaussians), sigma_i = i ** -exponent and eta ~ N(0, (noise * sigma_1)^2 / rows)."""
    u, _ = np.linalg.qr(rng.standard_normal((rows, channels)))
    v, _ = np.linalg.qr(rng.standard_normal((channels, channels)))
    sigma = np.arange(1, channels + 1, dtype=np.float64) ** -exponent
    x = (u * sigma) @ v.T
    if noise:
        x += rng.standard_normal((rows, channels)) * (noise * sigma[0] / math.sqrt(rows))
    return x.astype(dtype)


def closed_form_crossing(channels: int, fraction: float, exponent: float = 1.2) -> int:
    """Crossing of the noise-free spectrum sigma_i = i ** -exponent by direct summation."""
    energy = [i ** (-2.0 * exponent) for i in range(1, channels + 1)]
    total = math.fsum(energy)
    running = 0.0
    for rank, value in enumerate(energy, start=1):
        running += value
        if running >= fraction * total:
            return rank
    return channels


def to_bfloat16_values(x) -> np.ndarray:
    """float32 values of the bfloat16 rounding (nearest even) of ``x``."""
    bits = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16) << 16
    return rounded.astype(np.uint32).view(np.float32)
